// fp32 window attention on exact integer and bf16 matrix cores (gfx950).
//
// The fp32 layer (AWA_COMPUTE_F32) takes fp32 Q, K and V and must land within
// 1e-4 of the reference's fp32 arithmetic, whose shaders use Kahan sums
// because real-model Q/K make the scores large and cancelling. This kernel
// computes the scores nearly exactly and rounds them once, on int8 MFMA:
//
// - Every Q row and K row is written as x = 2^(e-6) (d1 + d2 2^-8 + d3 2^-16
//   + d4 2^-24) with e the row's exponent (max |x| < 2^e), d1 in [-64, 64] and
//   d2..d4 in [-128, 127] (balanced base-256 digits, int8 slices). The
//   representation error is below 2^-30 of the row maximum.
// - q.k = 2^(eq+ek-12) (C2 + C3 2^-8 + C4 2^-16 + C5 2^-24), where C_w sums
//   the slice products d_s(q) d_t(k) with s + t = w over the 128 features.
//   v_mfma_i32_32x32x32_i8 accumulates them in int32 exactly (each C_w stays
//   below 2^23, so its conversion to fp32 is exact too), the dropped classes
//   w > 5 weigh below 2^-30, and the classes are combined from the smallest
//   up (C4 2^8 + C5 exactly in int32, then C3 and C2 in fp32), so a score
//   carries one fp32 rounding, like a correctly rounded dot product.
// - P V runs on bf16 MFMA with P = p1 + p2 + p3 and V = v1 + v2 + v3, three
//   bf16 pieces each (all 24 bits of the fp32 value), products p1 (v1 + v2 +
//   v3) + p2 (v1 + v2) + p3 v1 (the dropped ones weigh below 2^-24), fp32
//   accumulation; the row sum adds the fp32 probabilities. Two pieces of P
//   would not do: a peaked softmax returns about one V row, so P's relative
//   error (2^-16 with two pieces) would reach the output times |v|.
//
// Structure: 32-key tiles staged through LDS as four K slices (int8,
// row-major, rows key-permuted as in the other attention kernel so that the
// score accumulator layout is the PV operand layout) and three V slices (bf16,
// row-major, natural key order, read transposed with ds_read_b64_tr_b16); a
// per-key scale 2^(ek-6) beside them. Each wave owns 32 query rows (S^T = K
// Q^T, one query per lane column), the online softmax runs in the log2 domain
// relative to a running maximum that is only moved when a tile exceeds it by
// more than 2^8, and the window gather, RoPE, optional q/k RMSNorm, scatter
// and text partials are those of the fused bf16 kernel.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "awa_device.h"
#include "awa_kernels.h"

namespace awa
{
namespace
{

using namespace dev;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kXKeys = 32;       // keys per tile
constexpr int kXKPitch = 144;    // bytes per key row of one int8 K slice (128 + 16: conflict-free row reads)
constexpr int kXKSlice = kXKeys * kXKPitch;
constexpr int kXVPitch = 160;    // bf16 elements per key row of one V slice (conflict-free transposed reads)
constexpr int kXVSlice = kXKeys * kXVPitch * 2;
// One wave's output stage: 8 fp32 rows of 512 bytes and their 8 destinations.
constexpr int kXOutStageWaveBytes = 8 * 512 + 64;

// x ~= 2^(e-6) (d1 + d2 2^-8 + d3 2^-16 + d4 2^-24) for |x| < 2^e: X = x *
// 2^(30-e) truncated (|X| < 2^30) plus 128 (1 + 2^8 + 2^16), so that its top
// byte (arithmetic) is d1 and each lower byte b is a digit b - 128, the int8
// b ^ 0x80.
__device__ __forceinline__ uint32_t digit_word(float x, int e)
{
    return static_cast<uint32_t>(static_cast<int>(ldexpf(x, 30 - e))) + 0x808080u;
}

// The digits of four values as four int8 slices (w0 = d1 ... w3 = d4, byte i
// from value i): a 4 x 4 byte transpose in eight v_perm_b32.
__device__ __forceinline__ void transpose_digits(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                                 uint32_t& w0, uint32_t& w1, uint32_t& w2, uint32_t& w3)
{
    const uint32_t a = __builtin_amdgcn_perm(x1, x0, 0x06020400u); // x0.b0 x1.b0 x0.b2 x1.b2
    const uint32_t b = __builtin_amdgcn_perm(x1, x0, 0x07030501u); // x0.b1 x1.b1 x0.b3 x1.b3
    const uint32_t c = __builtin_amdgcn_perm(x3, x2, 0x06020400u);
    const uint32_t d = __builtin_amdgcn_perm(x3, x2, 0x07030501u);
    w0 = __builtin_amdgcn_perm(d, b, 0x07060302u);
    w1 = __builtin_amdgcn_perm(c, a, 0x07060302u) ^ 0x80808080u;
    w2 = __builtin_amdgcn_perm(d, b, 0x05040100u) ^ 0x80808080u;
    w3 = __builtin_amdgcn_perm(c, a, 0x05040100u) ^ 0x80808080u;
}

// Eight consecutive values of one row as four int8 slices (two words each).
__device__ __forceinline__ void split8(const float* v, int e, uint32_t (&w)[4][2])
{
    uint32_t x[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        x[i] = digit_word(v[i], e);
    transpose_digits(x[0], x[1], x[2], x[3], w[0][0], w[1][0], w[2][0], w[3][0]);
    transpose_digits(x[4], x[5], x[6], x[7], w[0][1], w[1][1], w[2][1], w[3][1]);
}

// Three bf16 pieces of v (v1 = rne(v), v2 = rne(v - v1), v3 = rne(v - v1 - v2)),
// two elements per word.
__device__ __forceinline__ void split_bf16x3(float a, float b, uint32_t& w1, uint32_t& w2, uint32_t& w3)
{
    w1 = cvt_pk_bf16(a, b);
    const float a1 = a - bf16_lo(w1);
    const float b1 = b - bf16_hi(w1);
    w2 = cvt_pk_bf16(a1, b1);
    w3 = cvt_pk_bf16(a1 - bf16_lo(w2), b1 - bf16_hi(w2));
}

template <typename TIn, typename TOut, bool FUSED, bool WIDE, bool NORM>
__global__ __launch_bounds__(WIDE ? 512 : 256, WIDE ? 1 : 2) void window_attention_x_kernel(const AttentionLaunch p)
{
    static_assert(!NORM || FUSED, "the q/k RMSNorm is fused into the gather");
    constexpr int kThreads = WIDE ? 512 : 256;
    static_assert(kThreads / 2 == (WIDE ? awa::kWideQueryRows : awa::kQueryRows), "work items match the variant");
    constexpr int KT = kXKeys;
    constexpr int kRW = kRawWords8<TIn>;

    // The 8-wave form double-buffers its tiles (one barrier per tile); the
    // 4-wave form keeps one buffer so that two workgroups share a CU.
    constexpr int kBufs = WIDE ? 2 : 1;
    constexpr int kKBuf = 4 * kXKSlice;
    constexpr int kVBuf = 3 * kXVSlice;
    __shared__ __attribute__((aligned(16))) unsigned char k_lds[kBufs * kKBuf];
    __shared__ __attribute__((aligned(16))) unsigned char v_lds[kBufs * kVBuf];
    __shared__ __attribute__((aligned(16))) float kscale_lds[kBufs * KT];
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn_lds[];
    float* const norm_lds = reinterpret_cast<float*>(dyn_lds);
    float* const rope_lds = reinterpret_cast<float*>(dyn_lds + kNormLdsBytes<NORM>);
    unsigned char* const row_dyn = dyn_lds + kNormLdsBytes<NORM> + rope_table_bytes(FUSED, p.rope_coords);

    // RoPE table: its loads are issued first, before the work item is read
    // (they do not depend on it), unconditionally (indices past the table
    // are clamped to its last entry and their values dropped), and land in
    // LDS after the Q and first-tile loads are in flight.
    constexpr int kRopePerThread = (kMaxRopeCoords * kRopeRow + kThreads - 1) / kThreads;
    float rope_reg[FUSED ? kRopePerThread : 1];
    if constexpr (FUSED)
    {
        const int n = p.rope_coords * kRopeRow;
#pragma unroll
        for (int j = 0; j < kRopePerThread; j++)
            rope_reg[j] = p.rope_cs[min(static_cast<int>(threadIdx.x) + j * kThreads, n - 1)];
    }

    const WorkItem item = p.work[blockIdx.x];
    if (item.window < 0)
        return;
    const WindowDesc win = item.win;
    const int head = item.head;
    const int L = win.video_tokens + p.text_tokens;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int head_off = head * kHeadDim;
    const int tiles = (L + KT - 1) / KT;
    // Key tiles of this item: all of them, or one segment of a split layer.
    const int t_begin = item.key0 / KT;
    const int t_end = min(tiles, (item.key1 + KT - 1) / KT);
    const int table_rows = (p.max_window_tokens + 63) & ~63;

    const TIn* const video_base = static_cast<const TIn*>(p.video.data);
    const TIn* const text_base = static_cast<const TIn*>(p.text.data);
    const long long v_tok = p.video.token_stride;
    const long long v_qkv = p.video.qkv_stride;
    const long long t_tok = p.text.token_stride;
    const long long t_qkv = p.text.qkv_stride;
    const TIn* const packed_base = static_cast<const TIn*>(p.packed_in);
    const long long packed_row = p.packed_in_row;
    const long long packed_qkv = static_cast<long long>(p.heads) * kHeadDim;

    const RowDivisors divisors = row_divisors(win);
    auto decode = [&](int i) { return window_row(win, divisors, i, p.text_tokens, p.source_h, p.source_w); };
    auto source_ptr = [&](const RowRef& r, int qkv) -> const TIn* {
        return r.text ? text_base + r.k * t_tok + qkv * t_qkv + head_off
                      : video_base + static_cast<long long>(r.token) * v_tok + qkv * v_qkv + head_off;
    };
    auto row_ptr = [&](int i, int qkv) -> const TIn* {
        if constexpr (FUSED)
            return source_ptr(decode(i), qkv);
        else
            return packed_base + (win.seq_start + i) * packed_row + qkv * packed_qkv + head_off;
    };

    const int wave_row0 = item.row0 + wave * 32;
    const bool wave_active = wave * 32 < item.rows && wave_row0 < L;
    const int qi = wave_row0 + col;
    const bool q_valid = wave_active && qi < L;
    const int q_row = min(qi, L - 1);

    // Q: lane holds features 32c + 16*half + [0,16) for c = 0..3 (the B
    // operand of the int8 score MFMA).
    uint32_t qraw[8 * kRW];
    {
        const TIn* q_src = row_ptr(q_row, 0);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int x = 0; x < 2; x++)
                load_raw8(q_src + 32 * c + 16 * half + 8 * x, qraw + (2 * c + x) * kRW);
    }

    // Row table: byte offsets of each row's K and V, RoPE coordinates (see
    // the bf16 kernel), padded to whole 64-row blocks with the last row.
    const unsigned char* const load_base =
        reinterpret_cast<const unsigned char*>(FUSED ? static_cast<const void*>(video_base)
                                                     : static_cast<const void*>(packed_base));
    long long* row_k = reinterpret_cast<long long*>(row_dyn);
    long long* row_v = row_k + table_rows;
    uint32_t* row_code = reinterpret_cast<uint32_t*>(row_v + table_rows);
    for (int i = tid; i < tiles * KT; i += kThreads)
    {
        const int src = min(i, L - 1);
        if constexpr (FUSED)
        {
            const RowRef r = decode(src);
            const TIn* const k_ptr = source_ptr(r, 1);
            row_k[i] = reinterpret_cast<const unsigned char*>(k_ptr) - load_base;
            row_v[i] = reinterpret_cast<const unsigned char*>(k_ptr + (r.text ? t_qkv : v_qkv)) - load_base;
            row_code[i] = static_cast<uint32_t>(r.ct) | (static_cast<uint32_t>(r.ch) << 8) |
                          (static_cast<uint32_t>(r.cw) << 16) | (static_cast<uint32_t>(p.rope_coords) << 24);
        }
        else
        {
            row_k[i] = reinterpret_cast<const unsigned char*>(row_ptr(src, 1)) - load_base;
            row_v[i] = reinterpret_cast<const unsigned char*>(row_ptr(src, 2)) - load_base;
        }
    }
    __syncthreads();

    // Staging: 16 consecutive threads own the 16 chunks of 8 features of one
    // key row (K and V); a pass covers kThreads / 16 rows.
    constexpr int kRowsPerPass = kThreads / 16;
    constexpr int kRows = KT / kRowsPerPass;
    static_assert(kRows * kRowsPerPass == KT, "staging split");
    const int kc = tid & 15;
    const int kr0 = tid >> 4;
    int rope_shift[4], rope_col[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
    {
        const int pair = 4 * kc + q;
        const int axis = 2 * pair < kRopeDim ? pair / kRopePairs : 3;
        rope_shift[q] = 8 * axis;
        rope_col[q] = axis < 3 ? 2 * (pair - axis * kRopePairs) : 0;
    }
    uint32_t st_k[kRows * kRW], st_v[kRows * kRW];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int j = 0; j < kRows; j++)
        {
            const int r = tile * KT + kr0 + kRowsPerPass * j;
            load_raw8(reinterpret_cast<const TIn*>(load_base + row_k[r]) + 8 * kc, st_k + j * kRW);
            load_raw8(reinterpret_cast<const TIn*>(load_base + row_v[r]) + 8 * kc, st_v + j * kRW);
        }
    };
    auto store_k = [&](int tile, int buf) {
#pragma unroll
        for (int j = 0; j < kRows; j++)
        {
            const int row = kr0 + kRowsPerPass * j;
            float kv[8];
            raw_to_float8<TIn>(st_k + j * kRW, kv);
            if constexpr (FUSED)
            {
                if constexpr (NORM)
                {
                    // DitRMSNorm of the K row, bit for bit (its 16 chunks sit
                    // in 16 consecutive lanes).
                    const float coef = rms_coef_row16(kv, p.norm_eps);
                    const bool text = tile * KT + row >= win.video_tokens;
                    const float* const g = norm_lds + (text ? kHeadDim : 0) + 8 * kc;
                    const float4 g0 = *reinterpret_cast<const float4*>(g);
                    const float4 g1 = *reinterpret_cast<const float4*>(g + 4);
                    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        kv[e] = (kv[e] * coef) * gv[e];
                }
                const uint32_t code = row_code[tile * KT + row];
#pragma unroll
                for (int q = 0; q < 4; q++)
                {
                    const uint32_t coord = (code >> rope_shift[q]) & 255u;
                    const float2 t = *reinterpret_cast<const float2*>(rope_lds + coord * kRopeRow + rope_col[q]);
                    rope_pair_cs(kv[2 * q], kv[2 * q + 1], t.x, t.y);
                }
            }
            // Row exponent over the 16 lanes of the row, then the int8 slices.
            float m = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++)
                m = fmaxf(m, fabsf(kv[e]));
            const int ek = __builtin_amdgcn_frexp_expf(max16(m));
            uint32_t w[4][2];
            split8(kv, ek, w);
            unsigned char* const krow = k_lds + buf * kKBuf + key_permute(row) * kXKPitch + 8 * kc;
#pragma unroll
            for (int s = 0; s < 4; s++)
                *reinterpret_cast<uint2*>(krow + s * kXKSlice) = make_uint2(w[s][0], w[s][1]);
            if (kc == 0)
                kscale_lds[buf * KT + row] = ldexpf(1.f, ek - 6);
        }
    };
    auto store_v = [&](int buf) {
        // V: three bf16 pieces, row-major.
#pragma unroll
        for (int j = 0; j < kRows; j++)
        {
            const int row = kr0 + kRowsPerPass * j;
            float vv[8];
            raw_to_float8<TIn>(st_v + j * kRW, vv);
            uint32_t v1[4], v2[4], v3[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                split_bf16x3(vv[2 * i], vv[2 * i + 1], v1[i], v2[i], v3[i]);
            unsigned char* const vrow = v_lds + buf * kVBuf + row * kXVPitch * 2 + 16 * kc;
            *reinterpret_cast<uint4*>(vrow) = make_uint4(v1[0], v1[1], v1[2], v1[3]);
            *reinterpret_cast<uint4*>(vrow + kXVSlice) = make_uint4(v2[0], v2[1], v2[2], v2[3]);
            *reinterpret_cast<uint4*>(vrow + 2 * kXVSlice) = make_uint4(v3[0], v3[1], v3[2], v3[3]);
        }
    };

    // ---- prologue: tile 0's loads (8-wave form), the RoPE table (plus an
    // identity row) and the K gammas into LDS ----
    if constexpr (WIDE)
        load_tile(t_begin);
    uint32_t q_code = 0;
    if constexpr (FUSED)
    {
        q_code = row_code[q_row];
        const int n = p.rope_coords * kRopeRow;
#pragma unroll
        for (int j = 0; j < kRopePerThread; j++)
        {
            const int e = tid + j * kThreads;
            if (e < n)
                rope_lds[e] = rope_reg[j];
        }
        if (tid < kRopeRow)
            rope_lds[n + tid] = (tid & 1) ? 0.f : 1.f;
        if constexpr (NORM)
            for (int i = tid; i < 2 * kHeadDim; i += kThreads)
                norm_lds[i] = i < kHeadDim ? p.norm_gamma[1][i] : p.norm_gamma[3][i - kHeadDim];
        __syncthreads();
    }

    // Q: optional RMSNorm, RoPE, then the row exponent (lane and lane ^ 32
    // hold the row's halves) and the four int8 slices in registers.
    float qv[64];
#pragma unroll
    for (int c = 0; c < 8; c++)
        raw_to_float8<TIn>(qraw + c * kRW, qv + 8 * c);
    if constexpr (NORM)
    {
        // DitRMSNorm of the Q row, bit for bit (rms_coef_row16's tree): qv[16c
        // + i] holds feature 32c + 16*half + i, so strides 64 and 32 pair
        // values of the lane, stride 16 the lane and its partner lane ^ 32,
        // strides 8 to 1 values of the lane again.
        float coef;
        {
#pragma clang fp contract(off)
            float a[32];
#pragma unroll
            for (int i = 0; i < 32; i++)
                a[i] = qv[i] * qv[i] + qv[32 + i] * qv[32 + i];
#pragma unroll
            for (int i = 0; i < 16; i++)
                a[i] = sum_xor32(a[i] + a[16 + i]);
#pragma unroll
            for (int w = 8; w > 0; w /= 2)
#pragma unroll
                for (int i = 0; i < w; i++)
                    a[i] = a[i] + a[i + w];
            coef = rms_coef(a[0], p.norm_eps);
        }
        const float* const gamma = q_row >= win.video_tokens ? p.norm_gamma[2] : p.norm_gamma[0];
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int x = 0; x < 4; x++)
            {
                const float4 g = *reinterpret_cast<const float4*>(gamma + 32 * c + 16 * half + 4 * x);
                qv[16 * c + 4 * x + 0] = (qv[16 * c + 4 * x + 0] * coef) * g.x;
                qv[16 * c + 4 * x + 1] = (qv[16 * c + 4 * x + 1] * coef) * g.y;
                qv[16 * c + 4 * x + 2] = (qv[16 * c + 4 * x + 2] * coef) * g.z;
                qv[16 * c + 4 * x + 3] = (qv[16 * c + 4 * x + 3] * coef) * g.w;
            }
    }
    if constexpr (FUSED)
    {
        // Pair 16c + 8*half + q of this lane: its axis and table column are
        // compile-time for either half; one select picks the lane's.
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int q = 0; q < 8; q++)
            {
                const int p0 = 16 * c + q;
                const int p1 = 16 * c + 8 + q;
                const int ax0 = 2 * p0 < kRopeDim ? p0 / kRopePairs : 3;
                const int ax1 = 2 * p1 < kRopeDim ? p1 / kRopePairs : 3;
                const int col0 = ax0 < 3 ? 2 * (p0 - ax0 * kRopePairs) : 0;
                const int col1 = ax1 < 3 ? 2 * (p1 - ax1 * kRopePairs) : 0;
                const uint32_t coord = (q_code >> (half ? 8 * ax1 : 8 * ax0)) & 255u;
                const float2 t = *reinterpret_cast<const float2*>(rope_lds + coord * kRopeRow + (half ? col1 : col0));
                rope_pair_cs(qv[16 * c + 2 * q], qv[16 * c + 2 * q + 1], t.x, t.y);
            }
    }
    float qmax = 0.f;
#pragma unroll
    for (int e = 0; e < 64; e++)
        qmax = fmaxf(qmax, fabsf(qv[e]));
    const int eq = __builtin_amdgcn_frexp_expf(max_xor32(qmax));
    // log2-domain score = sum * 2^(eq-6) * 2^(ek-6) * log2(e) / sqrt(d)
    const float qscale = ldexpf(p.scale_log2, eq - 6);
    i32x4 qs[4][4]; // [slice][feature chunk c]
#pragma unroll
    for (int c = 0; c < 4; c++)
    {
        uint32_t w0[4][2], w1[4][2];
        split8(qv + 16 * c, eq, w0);
        split8(qv + 16 * c + 8, eq, w1);
#pragma unroll
        for (int s = 0; s < 4; s++)
            qs[s][c] = i32x4{static_cast<int>(w0[s][0]), static_cast<int>(w0[s][1]), static_cast<int>(w1[s][0]),
                             static_cast<int>(w1[s][1])};
    }

    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[db][i] = 0.f;
    float row_max = 0.f; // running maximum (log2 domain), possibly stale by < 2^8
    float row_sum = 0.f; // this lane's share of the row's probability sum

    const i32x16 izero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    // Transposed V reads: lane (group g = lane / 16, j = lane % 16) addresses
    // key row 8*half + j/4 (+4 for the second read) and features 16*(g & 1) +
    // 4*(j & 3) of a 32-feature block; the hardware hands lane j the column
    // j of the 4 x 16 block its group read.
    const int vt_lane = (8 * half + ((lane & 15) >> 2)) * kXVPitch + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // Per-wave work on the tile in buffer buf: (a) the score classes 5 and 4,
    // (b) classes 3 and 2: f = C3 + C4 / 2^8 + C5 / 2^16 (fp32, from the
    // smallest up) and c2 = C2 (exact in fp32); (c) softmax, P and PV.
    auto scores_hi = [&](int buf, f32x16& f) {
        const unsigned char* const kb = k_lds + buf * kKBuf + col * kXKPitch + 16 * half;
        // ---- scores: S^T = K Q^T, four exact int32 classes ----
        {
            i32x16 c5 = izero, c4 = izero;
#pragma unroll
            for (int c = 0; c < 4; c++)
            {
                i32x4 k[4];
#pragma unroll
                for (int s = 0; s < 4; s++)
                    k[s] = *reinterpret_cast<const i32x4*>(kb + s * kXKSlice + 32 * c);
                c5 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[3], qs[0][c], c5, 0, 0, 0);
                c4 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[2], qs[0][c], c4, 0, 0, 0);
                c5 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[2], qs[1][c], c5, 0, 0, 0);
                c4 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[1], qs[1][c], c4, 0, 0, 0);
                c5 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[1], qs[2][c], c5, 0, 0, 0);
                c4 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[0], qs[2][c], c4, 0, 0, 0);
                c5 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k[0], qs[3][c], c5, 0, 0, 0);
            }
            // C4 2^8 + C5 is exact in int32 (|C4| <= 2^22, |C5| < 2^23), so
            // its conversion is the one rounding of C4 + C5 / 2^8 (scaled by
            // 2^8, which the next step folds into its factor).
#pragma unroll
            for (int i = 0; i < 16; i++)
                f[i] = static_cast<float>(
                    static_cast<int>((static_cast<uint32_t>(c4[i]) << 8) + static_cast<uint32_t>(c5[i])));
        }
    };
    auto scores_lo = [&](int buf, f32x16& f, f32x16& c2f) {
        const unsigned char* const kb = k_lds + buf * kKBuf + col * kXKPitch + 16 * half;
        {
            i32x16 c3 = izero, c2 = izero;
#pragma unroll
            for (int c = 0; c < 4; c++)
            {
                const i32x4 k0 = *reinterpret_cast<const i32x4*>(kb + 32 * c);
                const i32x4 k1 = *reinterpret_cast<const i32x4*>(kb + kXKSlice + 32 * c);
                c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k1, qs[0][c], c3, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k0, qs[0][c], c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(k0, qs[1][c], c3, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; i++)
            {
                f[i] = fmaf(f[i], 1.f / 65536.f, static_cast<float>(c3[i]));
                c2f[i] = static_cast<float>(c2[i]);
            }
        }
    };
    auto softmax_pv = [&](int tile, int buf, const f32x16& f, const f32x16& c2f, bool last) {
        // Register i holds key 16*(i/8) + 8*half + i%8 (key-permuted K rows).
        float kq[16];
        {
            const float4* const ks = reinterpret_cast<const float4*>(kscale_lds + buf * KT + 8 * half);
            const float4 a = ks[0], b = ks[1], c = ks[4], d = ks[5];
            const float kv[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
            for (int i = 0; i < 16; i++)
                kq[i] = kv[i] * qscale;
        }
        // Log2-domain score relative to the running maximum: (C2 + f / 2^8) kq
        // - row_max as C2 kq - row_max (one rounding, near zero for the keys
        // that matter) plus f kq / 2^8. Rounding the whole score first would
        // cost an error of 2^-24 |score| (1e-4 of a probability at scores of
        // ~1000, large shared Q/K directions) before the maximum cancels.
        auto relative_scores = [&](float (&s)[16]) {
#pragma unroll
            for (int i = 0; i < 16; i++)
                s[i] = fmaf(f[i], kq[i] * (1.f / 256.f), fmaf(c2f[i], kq[i], -row_max));
        };
        float s[16];
        relative_scores(s);
        // ---- online softmax, relative to the running maximum (keys past the
        // window in a ragged last tile repeat its last key, so they leave the
        // maximum unchanged and are masked below) ----
        float tile_max = s[0];
#pragma unroll
        for (int i = 1; i < 16; i++)
            tile_max = fmaxf(tile_max, s[i]);
        tile_max = max_xor32(tile_max);
        if (tile == t_begin || __any(tile_max > kRescaleThreshold))
        {
            // New maximum; the old terms are rescaled by 2^(old - new), the
            // exact difference of the two maxima, and the scores recomputed
            // relative to the new one (not shifted, which would round them at
            // their full magnitude).
            const float new_max = row_max + (tile == t_begin ? tile_max : fmaxf(tile_max, 0.f));
            if (tile != t_begin)
            {
                const float alpha = __builtin_amdgcn_exp2f(row_max - new_max);
                row_sum *= alpha;
#pragma unroll
                for (int db = 0; db < 4; db++)
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        o[db][i] *= alpha;
            }
            row_max = new_max;
            relative_scores(s);
        }
        if (last && (L % KT))
        {
            const int key0 = tile * KT + 8 * half;
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (key0 + 16 * (i >> 3) + (i & 7) >= L)
                    s[i] = -INFINITY;
        }
        // ---- P = p1 + p2 + p3 as bf16 operands (p1, p2 truncations, p3 the
        // rounded rest: all of p's 24 bits); the row sum adds the fp32 P ----
        bf16x8 p1[2], p2[2], p3[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 8; e += 2)
            {
                const float pa = __builtin_amdgcn_exp2f(s[8 * j + e]);
                const float pb = __builtin_amdgcn_exp2f(s[8 * j + e + 1]);
                const uint32_t ua = __float_as_uint(pa), ub = __float_as_uint(pb);
                const float ra = pa - __uint_as_float(ua & 0xffff0000u);
                const float rb = pb - __uint_as_float(ub & 0xffff0000u);
                const uint32_t rua = __float_as_uint(ra), rub = __float_as_uint(rb);
                const bf16x2 h1 = __builtin_bit_cast(bf16x2, __builtin_amdgcn_perm(ub, ua, 0x07060302u));
                const bf16x2 h2 = __builtin_bit_cast(bf16x2, __builtin_amdgcn_perm(rub, rua, 0x07060302u));
                const bf16x2 h3 = __builtin_bit_cast(bf16x2, cvt_pk_bf16(ra - __uint_as_float(rua & 0xffff0000u),
                                                                         rb - __uint_as_float(rub & 0xffff0000u)));
                p1[j][e] = h1[0];
                p1[j][e + 1] = h1[1];
                p2[j][e] = h2[0];
                p2[j][e + 1] = h2[1];
                p3[j][e] = h3[0];
                p3[j][e + 1] = h3[1];
                row_sum += pa;
                row_sum += pb;
            }
        // ---- O^T += V^T P^T: V pieces read transposed; the products
        // p1 (v1 + v2 + v3) + p2 (v1 + v2) + p3 v1 (weights down to 2^-16) ----
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int sl = 0; sl < 3; sl++)
            {
                bf16x8 va[4];
#pragma unroll
                for (int db = 0; db < 4; db++)
                {
                    const uint16_t* base = reinterpret_cast<const uint16_t*>(v_lds + buf * kVBuf + sl * kXVSlice) +
                                           vt_lane + 16 * j * kXVPitch + 32 * db;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 4 * kXVPitch));
                    const i16x4 lohi[2] = {lo, hi};
                    va[db] = __builtin_bit_cast(bf16x8, lohi);
                }
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[db], p1[j], o[db], 0, 0, 0);
                if (sl < 2)
#pragma unroll
                    for (int db = 0; db < 4; db++)
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[db], p2[j], o[db], 0, 0, 0);
                if (sl == 0)
#pragma unroll
                    for (int db = 0; db < 4; db++)
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[db], p3[j], o[db], 0, 0, 0);
            }
    };

    if constexpr (WIDE)
    {
        // Step t: the scores, softmax and PV of tile t, the staging of tile
        // t+1 (K and V into the other buffer), the loads of tile t+2, one
        // barrier. A buffer is rewritten only after the barrier that ends the
        // step reading it. Waves 0-3 compute first and stage last, waves 4-7
        // (the second wave on each SIMD) stage first, so that one wave's VALU
        // staging runs while the other's MFMAs hold the matrix core.
        const bool stage_first = wave >= 4;
        store_k(t_begin, 0);
        store_v(0);
        if (t_begin + 1 < t_end)
            load_tile(t_begin + 1);
        __syncthreads();
        for (int tile = t_begin; tile < t_end; tile++)
        {
            const int buf = (tile - t_begin) & 1;
            const bool next = tile + 1 < t_end;
            auto stage = [&]() {
                if (next)
                {
                    store_k(tile + 1, buf ^ 1);
                    store_v(buf ^ 1);
                    if (tile + 2 < t_end)
                        load_tile(tile + 2);
                }
            };
            if (stage_first)
                stage();
            if (wave_active)
            {
                f32x16 f;
                f32x16 c2f;
                scores_hi(buf, f);
                scores_lo(buf, f, c2f);
                softmax_pv(tile, buf, f, c2f, tile == tiles - 1);
            }
            if (!stage_first)
                stage();
            __syncthreads();
        }
    }
    else
    {
        // Step t: load, stage, barrier, compute, barrier (the other workgroup
        // on the CU covers the load latency).
        for (int tile = t_begin; tile < t_end; tile++)
        {
            load_tile(tile);
            store_k(tile, 0);
            store_v(0);
            __syncthreads();
            if (wave_active)
            {
                f32x16 f;
                f32x16 c2f;
                scores_hi(0, f);
                scores_lo(0, f, c2f);
                softmax_pv(tile, 0, f, c2f, tile == tiles - 1);
            }
            __syncthreads();
        }
    }

    if (p.split > 1)
    {
        // One key segment of a split layer: the unnormalised row (relative to
        // the running maximum) and (maximum, probability sum), for
        // launch_split_merge.
        const float l = sum_xor32(row_sum);
        if (!q_valid)
            return;
        const long long slot =
            (static_cast<long long>(win.seq_start + qi) * p.heads + head) * p.split + item.seg;
        store_row(p.split_o + slot * kHeadDim, o, 1.f, half);
        if (half == 0)
            p.split_ml[slot] = make_float2(row_max, l);
        return;
    }
    if constexpr (FUSED && WIDE && sizeof(TOut) == 4)
        if (p.text_partial_elemsize == 4)
        {
            // ---- 8-wave form: fp32 rows through LDS, 8 rows per pass (the V
            // tiles' space, free after the loop's last barrier): the lane
            // pair (col, half) holds row col's 16-byte chunks 8 db + 2 g +
            // half, written at position chunk ^ (2 row) of the row
            // (conflict-free), read back 16 bytes a lane, 32 lanes a row, and
            // stored as whole 512-byte rows with nontemporal stores (dirty
            // lines left in L2 lengthen the kernel's end; the text mean then
            // reads its rows from beyond L2, which costs it less than the
            // attention kernel gains). The 4-wave form measured slower this
            // way and stores its rows directly. ----
            if (!wave_active)
                return;
            const float inv = 1.f / sum_xor32(row_sum);
            float* dst = nullptr;
            if (q_valid)
            {
                const RowRef r = decode(qi);
                dst = !r.text ? static_cast<float*>(p.video_out.data) + r.t * p.video_out.ts + r.h * p.video_out.hs +
                                    r.w * p.video_out.ws + head_off
                              : static_cast<float*>(p.text_partials) +
                                    ((static_cast<long long>(item.window) * p.text_tokens + r.k) * p.heads + head) *
                                        kHeadDim;
            }
            unsigned char* const region = v_lds + wave * kXOutStageWaveBytes;
            float* const rows_lds = reinterpret_cast<float*>(region);
            unsigned long long* const dst_lds = reinterpret_cast<unsigned long long*>(region + 8 * 512);
            const int c = lane & 31;
#pragma unroll
            for (int pass = 0; pass < 4; pass++)
            {
                const int rl = col - 8 * pass;
                if (rl >= 0 && rl < 8)
                {
#pragma unroll
                    for (int db = 0; db < 4; db++)
#pragma unroll
                        for (int g = 0; g < 4; g++)
                        {
                            const int pos = (8 * db + 2 * g + half) ^ (2 * rl);
                            *reinterpret_cast<f32x4*>(rows_lds + rl * kHeadDim + 4 * pos) =
                                f32x4{o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                                      o[db][4 * g + 3] * inv};
                        }
                    if (half == 0)
                        dst_lds[rl] = reinterpret_cast<unsigned long long>(dst);
                }
                // The wave reads what its own lanes wrote.
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int i = 0; i < 4; i++)
                {
                    const int row = 2 * i + (lane >> 5);
                    const f32x4 v = *reinterpret_cast<const f32x4*>(rows_lds + row * kHeadDim + 4 * (c ^ (2 * row)));
                    float* const d = reinterpret_cast<float*>(dst_lds[row]);
                    if (d)
                        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(d + 4 * c));
                }
                // The next pass rewrites the region only after these reads.
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            return;
        }
    if (!q_valid)
        return;
    const float inv = 1.f / sum_xor32(row_sum);
    if constexpr (FUSED)
    {
        const RowRef r = decode(qi);
        if (!r.text)
        {
            TOut* dst = static_cast<TOut*>(p.video_out.data) + r.t * p.video_out.ts + r.h * p.video_out.hs +
                        r.w * p.video_out.ws + head_off;
            store_row(dst, o, inv, half);
        }
        else
        {
            const long long off =
                ((static_cast<long long>(item.window) * p.text_tokens + r.k) * p.heads + head) * kHeadDim;
            if (p.text_partial_elemsize == 2)
                store_row(static_cast<uint16_t*>(p.text_partials) + off, o, inv, half);
            else
                store_row(static_cast<float*>(p.text_partials) + off, o, inv, half);
        }
    }
    else
    {
        float* dst = p.packed_out + (win.seq_start + qi) * p.packed_out_row + head_off;
        store_row(dst, o, inv, half);
    }
}

} // namespace

template <typename TIn, typename TOut, bool FUSED, bool WIDE, bool NORM>
static hipError_t launch_x_one(const AttentionLaunch& p, hipStream_t stream)
{
    const size_t dynamic_lds = attention_x_dynamic_lds(p, NORM);
    hipLaunchKernelGGL((window_attention_x_kernel<TIn, TOut, FUSED, WIDE, NORM>), dim3(p.work_count),
                       dim3(WIDE ? 512 : 256), dynamic_lds, stream, p);
    return hipGetLastError();
}

template <bool FUSED, bool WIDE, bool NORM = false>
static hipError_t launch_x_typed(const AttentionLaunch& p, hipStream_t stream)
{
    const int in_size = FUSED ? p.video.elemsize : p.packed_in_elemsize;
    const int out_size = FUSED ? p.video_out.elemsize : 4;
    if (in_size == 4 && out_size == 4)
        return launch_x_one<float, float, FUSED, WIDE, NORM>(p, stream);
    if (in_size == 2 && out_size == 4)
        return launch_x_one<uint16_t, float, FUSED, WIDE, NORM>(p, stream);
    if constexpr (FUSED)
    {
        if (in_size == 4 && out_size == 2)
            return launch_x_one<float, uint16_t, FUSED, WIDE, NORM>(p, stream);
        if (in_size == 2 && out_size == 2)
            return launch_x_one<uint16_t, uint16_t, FUSED, WIDE, NORM>(p, stream);
    }
    return hipErrorInvalidValue;
}

size_t attention_x_dynamic_lds(const AttentionLaunch& p, bool norm)
{
    const size_t row_table = static_cast<size_t>((p.max_window_tokens + 63) & ~63) * (2 * sizeof(long long) + 4);
    return (norm ? 2 * kHeadDim * 4 : 0) + dev::rope_table_bytes(p.fused, p.rope_coords) + row_table;
}

static_assert(4 * kXOutStageWaveBytes <= 3 * kXVSlice && 8 * kXOutStageWaveBytes <= 2 * 3 * kXVSlice,
              "the output stage fits the V tiles");

size_t attention_x_static_lds(bool wide)
{
    return (wide ? 2 : 1) * (4 * kXKSlice + 3 * kXVSlice + kXKeys * sizeof(float));
}

hipError_t launch_attention_x(const AttentionLaunch& p, hipStream_t stream)
{
    if (p.work_count <= 0)
        return hipSuccess;
    if (p.qk_norm && !p.fused)
        return hipErrorInvalidValue;
    const bool wide = p.variant == kVariantWide;
    if (!wide && p.variant != kVariantNarrow)
        return hipErrorInvalidValue;
    if (!p.fused)
        return wide ? launch_x_typed<false, true>(p, stream) : launch_x_typed<false, false>(p, stream);
    if (p.qk_norm)
        return wide ? launch_x_typed<true, true, true>(p, stream) : launch_x_typed<true, false, true>(p, stream);
    return wide ? launch_x_typed<true, true>(p, stream) : launch_x_typed<true, false>(p, stream);
}

} // namespace awa
