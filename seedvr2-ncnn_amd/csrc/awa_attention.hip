// Window attention kernels for gfx950 (CDNA4).
//
// One workgroup = 4 waves = 128 query rows of one (window, head). Each wave
// owns 32 query rows and computes the transposed score tile S^T = K Q^T with
// 32x32 MFMAs, so that a lane holds one query column: the online-softmax
// statistics of a query live in two lanes (lane and lane^32), and the
// rescale of the output accumulator O^T = V^T P^T is lane-local.
//
// K and V tiles of 32 keys are staged through LDS (K row-major, V transposed
// so that the PV operand reads are contiguous in the key index). Keys are
// read out of the K tile in an order (bits 2 and 3 of the row swapped) that
// makes every lane's 16 probabilities cover two runs of 8 consecutive keys,
// which is exactly the K-slot layout of the B operand of the PV MFMA.
//
// In fused mode the kernel gathers rows straight from the video / text QKV
// blobs using the window geometry (the reference's Pack), applies the 3-axis
// interleaved RoPE while staging Q and K (MMRoPE), and writes video rows to
// their grid position (Unpack); text rows go to per-window partials that a
// second kernel averages in window order. Packed mode reads a packed
// [S][3H][d] blob and writes [S][H][d], for the staged WindowAttention layer.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "awa_kernels.h"

namespace awa
{
namespace
{

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKeyTile = 32;
constexpr int kRopePairs = kRopeDim / 6; // 21 pairs per axis
static_assert(kMaxRopeCoords * kRopePairs * 2 * 4 <= 24 * 1024, "RoPE table must stay small in LDS");

// LDS pitches (elements). Rows stay 16-byte aligned for ds_read_b128.
constexpr int kKPitchBf = kHeadDim + 8;   // 272 B
constexpr int kVPitchBf = kKeyTile + 8;   // 80 B
constexpr int kKPitchF = kHeadDim + 4;    // 528 B
constexpr int kVPitchF = kKeyTile + 4;    // 144 B

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16)
{
    return __uint_as_float(bits16 << 16);
}

// Round to nearest even (the reference's bit formula, src/dit/shader/dit_rmsnorm.comp:47-51).
__device__ __forceinline__ uint32_t float_to_bf16_bits(float f)
{
    const uint32_t bits = __float_as_uint(f);
    return (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    return float_to_bf16_bits(lo) | (float_to_bf16_bits(hi) << 16);
}

// Loads 8 consecutive elements as floats (16-byte aligned source).
__device__ __forceinline__ void load8(const float* p, float v[8])
{
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void load8(const uint16_t* p, float v[8])
{
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++)
    {
        v[2 * i] = bf16_bits_to_float(w[i] & 0xffffu);
        v[2 * i + 1] = bf16_bits_to_float(w[i] >> 16);
    }
}

// Interleaved-pair rotation of 8 features starting at feature f0 (even):
// even' = x_even*cos - x_odd*sin, odd' = x_odd*cos + x_even*sin, for features
// below kRopeDim; the axis of pair p is p / 21. No contraction, so the result
// is bit-identical to the reference's CPU rotation.
__device__ __forceinline__ void rope8(float v[8], int f0, int ct, int ch, int cw, const float* table)
{
#pragma clang fp contract(off)
#pragma unroll
    for (int q = 0; q < 4; q++)
    {
        const int f = f0 + 2 * q;
        if (f < kRopeDim)
        {
            const int pair = f >> 1;
            const int axis = pair / kRopePairs;
            const int pp = pair - axis * kRopePairs;
            const int coord = axis == 0 ? ct : (axis == 1 ? ch : cw);
            const float c = table[(coord * kRopePairs + pp) * 2];
            const float s = table[(coord * kRopePairs + pp) * 2 + 1];
            const float x0 = v[2 * q];
            const float x1 = v[2 * q + 1];
            v[2 * q] = x0 * c - x1 * s;
            v[2 * q + 1] = x1 * c + x0 * s;
        }
    }
}

struct Row
{
    bool video;
    int t, h, w; // absolute grid position (video)
    int k;       // text index
    int ct, ch, cw;
};

// Window-local row i -> grid position / text index and RoPE coordinates
// (video coordinates are (T_x + t - t0, h - h0, w - w0), text (k, k, k)).
__device__ __forceinline__ Row locate_row(const WindowDesc& win, int i, int text_tokens)
{
    Row r;
    if (i < win.video_tokens)
    {
        const int area = win.eh * win.ew;
        const int lt = i / area;
        const int rem = i - lt * area;
        const int lh = rem / win.ew;
        const int lw = rem - lh * win.ew;
        r.video = true;
        r.t = win.t0 + lt;
        r.h = win.h0 + lh;
        r.w = win.w0 + lw;
        r.k = 0;
        r.ct = text_tokens + lt;
        r.ch = lh;
        r.cw = lw;
    }
    else
    {
        const int k = i - win.video_tokens;
        r.video = false;
        r.t = r.h = r.w = 0;
        r.k = k;
        r.ct = r.ch = r.cw = k;
    }
    return r;
}

template <typename TIn>
__device__ __forceinline__ const TIn* fused_row_ptr(const AttentionLaunch& p, const Row& r, int qkv, int head)
{
    if (r.video)
    {
        const long long token = (static_cast<long long>(r.t) * p.source_h + r.h) * p.source_w + r.w;
        return static_cast<const TIn*>(p.video.data) + token * p.video.token_stride + qkv * p.video.qkv_stride +
               head * kHeadDim;
    }
    return static_cast<const TIn*>(p.text.data) + r.k * p.text.token_stride + qkv * p.text.qkv_stride +
           head * kHeadDim;
}

template <typename TIn>
__device__ __forceinline__ const TIn* packed_row_ptr(const AttentionLaunch& p, int row, int qkv, int head)
{
    return static_cast<const TIn*>(p.packed_in) + row * p.packed_in_row + (qkv * p.heads + head) * kHeadDim;
}

// Row order of the K tile as read by the S^T MFMA: swap bits 2 and 3.
__device__ __forceinline__ int key_permute(int m)
{
    return (m & ~0xC) | ((m & 4) << 1) | ((m & 8) >> 1);
}

__device__ __forceinline__ void store4(float* dst, const float v[4])
{
    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void store4(uint16_t* dst, const float v[4])
{
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

template <typename TIn, typename TOut, bool BF16, bool FUSED>
__global__ __launch_bounds__(kThreads, 2) void window_attention_kernel(const AttentionLaunch p)
{
    // LDS: K tile, transposed V tile, RoPE table.
    constexpr int kKBytes = BF16 ? kKeyTile * kKPitchBf * 2 : kKeyTile * kKPitchF * 4;
    constexpr int kVBytes = BF16 ? kHeadDim * kVPitchBf * 2 : kHeadDim * kVPitchF * 4;
    __shared__ __attribute__((aligned(16))) unsigned char k_lds[kKBytes];
    __shared__ __attribute__((aligned(16))) unsigned char v_lds[kVBytes];
    __shared__ float rope_lds[FUSED ? kMaxRopeCoords * kRopePairs * 2 : 1];

    const WorkItem item = p.work[blockIdx.x];
    if (item.window < 0)
        return;
    const WindowDesc win = p.windows[item.window];
    const int head = item.head_qblock >> 16;
    const int qblock = item.head_qblock & 0xffff;
    const int L = win.video_tokens + p.text_tokens;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;

    if constexpr (FUSED)
    {
        for (int e = tid; e < p.rope_coords * kRopePairs * 2; e += kThreads)
            rope_lds[e] = p.rope_cs[e];
        __syncthreads();
    }

    const int wave_row0 = qblock * kQueryRows + wave * 32;
    const bool wave_active = wave_row0 < L;
    const int qi = wave_row0 + col;
    const bool q_valid = qi < L;

    // ---- Q into registers (B operand of S^T = K Q^T) ----
    // bf16: lane holds features 16c + 8*half + [0,8) for c = 0..7.
    // fp32: lane holds features 64*half + [0,64).
    bf16x8 qb[BF16 ? 8 : 1];
    float qf[BF16 ? 1 : 64];
    {
        const TIn* src = nullptr;
        Row r{};
        if (q_valid)
        {
            if constexpr (FUSED)
            {
                r = locate_row(win, qi, p.text_tokens);
                src = fused_row_ptr<TIn>(p, r, 0, head);
            }
            else
            {
                src = packed_row_ptr<TIn>(p, win.seq_start + qi, 0, head);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; c++)
        {
            const int f0 = BF16 ? 16 * c + 8 * half : 64 * half + 8 * c;
            float v[8];
            if (q_valid)
            {
                load8(src + f0, v);
                if constexpr (FUSED)
                    rope8(v, f0, r.ct, r.ch, r.cw, rope_lds);
            }
            else
            {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    v[e] = 0.f;
            }
            if constexpr (BF16)
            {
                bf16x8 x;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    x[e] = static_cast<__bf16>(v[e]);
                qb[c] = x;
            }
            else
            {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    qf[8 * c + e] = v[e];
            }
        }
    }

    // ---- staging assignment ----
    // K: thread -> (row kr, 16 features from 16*kc); V: thread -> (keys 2*vp, 2*vp+1; features 8*vj..).
    const int kr = tid >> 3;
    const int kc = tid & 7;
    const int vp = tid & 15;
    const int vj = tid >> 4;
    float kreg[16];
    float vreg[16];

    auto load_tile = [&](int tile) {
        const int key = tile * kKeyTile + kr;
        if (key < L)
        {
            const TIn* src;
            if constexpr (FUSED)
            {
                const Row r = locate_row(win, key, p.text_tokens);
                src = fused_row_ptr<TIn>(p, r, 1, head);
                load8(src + 16 * kc, kreg);
                load8(src + 16 * kc + 8, kreg + 8);
                rope8(kreg, 16 * kc, r.ct, r.ch, r.cw, rope_lds);
                rope8(kreg + 8, 16 * kc + 8, r.ct, r.ch, r.cw, rope_lds);
            }
            else
            {
                src = packed_row_ptr<TIn>(p, win.seq_start + key, 1, head);
                load8(src + 16 * kc, kreg);
                load8(src + 16 * kc + 8, kreg + 8);
            }
        }
        else
        {
#pragma unroll
            for (int e = 0; e < 16; e++)
                kreg[e] = 0.f;
        }
#pragma unroll
        for (int s = 0; s < 2; s++)
        {
            const int vkey = tile * kKeyTile + 2 * vp + s;
            if (vkey < L)
            {
                const TIn* src;
                if constexpr (FUSED)
                    src = fused_row_ptr<TIn>(p, locate_row(win, vkey, p.text_tokens), 2, head);
                else
                    src = packed_row_ptr<TIn>(p, win.seq_start + vkey, 2, head);
                load8(src + 8 * vj, vreg + 8 * s);
            }
            else
            {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    vreg[8 * s + e] = 0.f;
            }
        }
    };

    auto store_tile = [&]() {
        if constexpr (BF16)
        {
            uint16_t* ks = reinterpret_cast<uint16_t*>(k_lds);
            uint16_t* vt = reinterpret_cast<uint16_t*>(v_lds);
            uint4 a, b;
            a.x = pack_bf16x2(kreg[0], kreg[1]);
            a.y = pack_bf16x2(kreg[2], kreg[3]);
            a.z = pack_bf16x2(kreg[4], kreg[5]);
            a.w = pack_bf16x2(kreg[6], kreg[7]);
            b.x = pack_bf16x2(kreg[8], kreg[9]);
            b.y = pack_bf16x2(kreg[10], kreg[11]);
            b.z = pack_bf16x2(kreg[12], kreg[13]);
            b.w = pack_bf16x2(kreg[14], kreg[15]);
            *reinterpret_cast<uint4*>(ks + kr * kKPitchBf + 16 * kc) = a;
            *reinterpret_cast<uint4*>(ks + kr * kKPitchBf + 16 * kc + 8) = b;
#pragma unroll
            for (int e = 0; e < 8; e++)
                *reinterpret_cast<uint32_t*>(vt + (8 * vj + e) * kVPitchBf + 2 * vp) =
                    pack_bf16x2(vreg[e], vreg[8 + e]);
        }
        else
        {
            float* ks = reinterpret_cast<float*>(k_lds);
            float* vt = reinterpret_cast<float*>(v_lds);
#pragma unroll
            for (int q = 0; q < 4; q++)
                *reinterpret_cast<float4*>(ks + kr * kKPitchF + 16 * kc + 4 * q) =
                    make_float4(kreg[4 * q], kreg[4 * q + 1], kreg[4 * q + 2], kreg[4 * q + 3]);
#pragma unroll
            for (int e = 0; e < 8; e++)
                *reinterpret_cast<float2*>(vt + (8 * vj + e) * kVPitchF + 2 * vp) = make_float2(vreg[e], vreg[8 + e]);
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[db][i] = 0.f;
    float row_max = -INFINITY; // log2 domain
    float row_sum = 0.f;       // partial over this lane's keys

    const int tiles = (L + kKeyTile - 1) / kKeyTile;
    load_tile(0);
    for (int tile = 0; tile < tiles; tile++)
    {
        store_tile();
        __syncthreads();
        if (tile + 1 < tiles)
            load_tile(tile + 1);

        if (wave_active)
        {
            // ---- S^T = K Q^T (32 keys x 32 queries) ----
            f32x16 s;
#pragma unroll
            for (int i = 0; i < 16; i++)
                s[i] = 0.f;
            const int krow = key_permute(col);
            if constexpr (BF16)
            {
                const uint16_t* ks = reinterpret_cast<const uint16_t*>(k_lds) + krow * kKPitchBf + 8 * half;
#pragma unroll
                for (int c = 0; c < 8; c++)
                {
                    const bf16x8 ka = *reinterpret_cast<const bf16x8*>(ks + 16 * c);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qb[c], s, 0, 0, 0);
                }
            }
            else
            {
                const float* ks = reinterpret_cast<const float*>(k_lds) + krow * kKPitchF + 64 * half;
#pragma unroll
                for (int c4 = 0; c4 < 16; c4++)
                {
                    const float4 ka = *reinterpret_cast<const float4*>(ks + 4 * c4);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.x, qf[4 * c4 + 0], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.y, qf[4 * c4 + 1], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.z, qf[4 * c4 + 2], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.w, qf[4 * c4 + 3], s, 0, 0, 0);
                }
            }

            // ---- online softmax: register i holds key 16*(i/8) + 8*half + i%8 ----
            const int key0 = tile * kKeyTile + 8 * half;
            float tile_max = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; i++)
            {
                const int key = key0 + 16 * (i >> 3) + (i & 7);
                const float v = key < L ? s[i] * p.scale_log2 : -INFINITY;
                s[i] = v;
                tile_max = fmaxf(tile_max, v);
            }
            tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
            const float new_max = fmaxf(row_max, tile_max);
            const float alpha = exp2f(row_max - new_max);
            row_max = new_max;
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++)
            {
                s[i] = exp2f(s[i] - new_max);
                psum += s[i];
            }
            row_sum = row_sum * alpha + psum;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    o[db][i] *= alpha;

            // ---- O^T += V^T P^T ----
            if constexpr (BF16)
            {
                bf16x8 pb0, pb1;
#pragma unroll
                for (int e = 0; e < 8; e++)
                {
                    pb0[e] = static_cast<__bf16>(s[e]);
                    pb1[e] = static_cast<__bf16>(s[8 + e]);
                }
                const uint16_t* vt = reinterpret_cast<const uint16_t*>(v_lds);
#pragma unroll
                for (int db = 0; db < 4; db++)
                {
                    const uint16_t* vrow = vt + (db * 32 + col) * kVPitchBf + 8 * half;
                    const bf16x8 va0 = *reinterpret_cast<const bf16x8*>(vrow);
                    const bf16x8 va1 = *reinterpret_cast<const bf16x8*>(vrow + 16);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va0, pb0, o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va1, pb1, o[db], 0, 0, 0);
                }
            }
            else
            {
                const float* vt = reinterpret_cast<const float*>(v_lds);
#pragma unroll
                for (int db = 0; db < 4; db++)
                {
                    const float* vrow = vt + (db * 32 + col) * kVPitchF + 8 * half;
#pragma unroll
                    for (int g = 0; g < 4; g++)
                    {
                        const float4 va = *reinterpret_cast<const float4*>(vrow + 16 * (g >> 1) + 4 * (g & 1));
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.x, s[4 * g + 0], o[db], 0, 0, 0);
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.y, s[4 * g + 1], o[db], 0, 0, 0);
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.z, s[4 * g + 2], o[db], 0, 0, 0);
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va.w, s[4 * g + 3], o[db], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }

    if (!q_valid)
        return;
    const float total = row_sum + __shfl_xor(row_sum, 32);
    const float inv = 1.f / total;

    // ---- store: lane holds features db*32 + 8*g + 4*half + [0,4) ----
    if constexpr (FUSED)
    {
        const Row r = locate_row(win, qi, p.text_tokens);
        if (r.video)
        {
            TOut* dst = static_cast<TOut*>(p.video_out.data) + r.t * p.video_out.ts + r.h * p.video_out.hs +
                        r.w * p.video_out.ws + head * kHeadDim;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                {
                    const float v[4] = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                        o[db][4 * g + 3] * inv};
                    store4(dst + db * 32 + 8 * g + 4 * half, v);
                }
        }
        else
        {
            float* dst = p.text_partials +
                         ((static_cast<long long>(item.window) * p.text_tokens + r.k) * p.heads + head) * kHeadDim;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                {
                    const float v[4] = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                        o[db][4 * g + 3] * inv};
                    store4(dst + db * 32 + 8 * g + 4 * half, v);
                }
        }
    }
    else
    {
        float* dst = p.packed_out + (win.seq_start + qi) * p.packed_out_row + head * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int g = 0; g < 4; g++)
            {
                const float v[4] = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                    o[db][4 * g + 3] * inv};
                store4(dst + db * 32 + 8 * g + 4 * half, v);
            }
    }
}

} // namespace

template <typename TIn, typename TOut, bool BF16, bool FUSED>
static hipError_t launch_one(const AttentionLaunch& p, hipStream_t stream)
{
    hipLaunchKernelGGL((window_attention_kernel<TIn, TOut, BF16, FUSED>), dim3(p.work_count), dim3(kThreads), 0,
                       stream, p);
    return hipGetLastError();
}

template <bool BF16, bool FUSED>
static hipError_t launch_typed(const AttentionLaunch& p, hipStream_t stream)
{
    const int in_size = FUSED ? p.video.elemsize : p.packed_in_elemsize;
    const int out_size = FUSED ? p.video_out.elemsize : 4;
    if (in_size == 4 && out_size == 4)
        return launch_one<float, float, BF16, FUSED>(p, stream);
    if (in_size == 2 && out_size == 4)
        return launch_one<uint16_t, float, BF16, FUSED>(p, stream);
    if constexpr (FUSED)
    {
        if (in_size == 4 && out_size == 2)
            return launch_one<float, uint16_t, BF16, FUSED>(p, stream);
        if (in_size == 2 && out_size == 2)
            return launch_one<uint16_t, uint16_t, BF16, FUSED>(p, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_attention(const AttentionLaunch& p, hipStream_t stream)
{
    if (p.work_count <= 0)
        return hipSuccess;
    if (p.fused)
        return p.bf16_mfma ? launch_typed<true, true>(p, stream) : launch_typed<false, true>(p, stream);
    return p.bf16_mfma ? launch_typed<true, false>(p, stream) : launch_typed<false, false>(p, stream);
}

} // namespace awa
