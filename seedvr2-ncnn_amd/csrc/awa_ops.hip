// Data-movement kernels of the AWA path (gfx950): the staged Pack, MMRoPE and
// Unpack layers, the ordered text mean of the fused path, a generic-head_dim
// window attention for the staged layer, casts, fills.
//
// All of these are HBM-bound byte movers: each thread moves 4 consecutive
// elements (16 B of fp32 / 8 B of bf16) so that a wave touches contiguous
// 256-1024 B runs of a row.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "awa_kernels.h"

namespace awa
{
namespace
{

constexpr int kBlock = 256;

__device__ __forceinline__ float bf16_to_f32(uint16_t b)
{
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    const uint32_t bits = __float_as_uint(f);
    return static_cast<uint16_t>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float load_elem(const void* base, long long index, int elemsize)
{
    return elemsize == 4 ? static_cast<const float*>(base)[index]
                         : bf16_to_f32(static_cast<const uint16_t*>(base)[index]);
}

__device__ __forceinline__ void store_elem(void* base, long long index, int elemsize, float v)
{
    if (elemsize == 4)
        static_cast<float*>(base)[index] = v;
    else
        static_cast<uint16_t*>(base)[index] = f32_to_bf16(v);
}

// ---- Pack: packed[p][qkv][head][f] = source row (src/awa/awa_layers.cpp:440-454) ----
__global__ void pack_kernel(const RowInfo* rows, int sequence_tokens, int source_tokens, QkvSource video,
                            QkvSource text, int heads, int head_dim, float* packed, long long packed_row)
{
    const int row_elems = 3 * heads * head_dim;
    const long long total = static_cast<long long>(sequence_tokens) * row_elems;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int position = static_cast<int>(idx / row_elems);
    const int e = static_cast<int>(idx - static_cast<long long>(position) * row_elems);
    const int qkv = e / (heads * head_dim);
    const int rest = e - qkv * heads * head_dim;
    const int source = rows[position].source;
    const bool is_video = source < source_tokens;
    const QkvSource& src = is_video ? video : text;
    const long long token = is_video ? source : source - source_tokens;
    packed[position * packed_row + e] =
        load_elem(src.data, token * src.token_stride + qkv * src.qkv_stride + rest, src.elemsize);
}

__global__ void cu_seqlens_kernel(const int* cu, int count, float* out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count)
        out[i] = static_cast<float>(cu[i]);
}

// ---- MMRoPE on a packed blob (src/awa/awa_layers.cpp:930-951): one thread per feature pair ----
__global__ void mmrope_kernel(const RowInfo* rows, int sequence_tokens, const void* in, long long in_row,
                              int in_elemsize, float* out, long long out_row, int heads, int head_dim, int rope_dim,
                              int rope_pairs, const float* rope_cs)
{
#pragma clang fp contract(off)
    const int pairs_per_row = 3 * heads * head_dim / 2;
    const long long total = static_cast<long long>(sequence_tokens) * pairs_per_row;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int position = static_cast<int>(idx / pairs_per_row);
    const int pair_in_row = static_cast<int>(idx - static_cast<long long>(position) * pairs_per_row);
    const int e = 2 * pair_in_row; // even element index within the row
    const int qkv_head = e / head_dim;
    const int feature = e - qkv_head * head_dim;
    const long long src = position * in_row + e;
    const long long dst = position * out_row + e;
    float x0 = load_elem(in, src, in_elemsize);
    float x1;
    if (feature + 1 < head_dim)
        x1 = load_elem(in, src + 1, in_elemsize);
    else
        x1 = 0.f;
    if (qkv_head < 2 * heads && feature < rope_dim)
    {
        // rope_dim is even, so feature+1 < rope_dim too.
        const RowInfo r = rows[position];
        const int pair = feature >> 1;
        const int axis = pair / rope_pairs;
        const int pp = pair - axis * rope_pairs;
        const int coord = axis == 0 ? r.ct : (axis == 1 ? r.ch : r.cw);
        const float c = rope_cs[(coord * rope_pairs + pp) * 2];
        const float s = rope_cs[(coord * rope_pairs + pp) * 2 + 1];
        const float y0 = x0 * c - x1 * s;
        const float y1 = x1 * c + x0 * s;
        x0 = y0;
        x1 = y1;
    }
    out[dst] = x0;
    if (feature + 1 < head_dim)
        out[dst + 1] = x1;
}

// ---- Unpack video: video[t][h][w][head][f] = packed[video_positions[token]] (awa_layers.cpp:659-676) ----
__global__ void unpack_video_kernel(const int* video_positions, int source_t, int source_h, int source_w,
                                    const void* packed, long long packed_row, int packed_elemsize, VideoSink out,
                                    int row_elems)
{
    const long long total = static_cast<long long>(source_t) * source_h * source_w * row_elems;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int token = static_cast<int>(idx / row_elems);
    const int e = static_cast<int>(idx - static_cast<long long>(token) * row_elems);
    const int t = token / (source_h * source_w);
    const int spatial = token - t * source_h * source_w;
    const int h = spatial / source_w;
    const int w = spatial - h * source_w;
    const float v = load_elem(packed, video_positions[token] * packed_row + e, packed_elemsize);
    store_elem(out.data, t * out.ts + h * out.hs + w * out.ws + e, out.elemsize, v);
}

// ---- Unpack text: (sum over windows in window order) / nwin (src/awa/shader/awa_unpack.comp:47-58) ----
__global__ void unpack_text_kernel(const int* text_positions, int window_count, int text_tokens, const void* packed,
                                   long long packed_row, int packed_elemsize, void* out, long long out_row,
                                   int out_elemsize, int row_elems)
{
    const long long total = static_cast<long long>(text_tokens) * row_elems;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int k = static_cast<int>(idx / row_elems);
    const int e = static_cast<int>(idx - static_cast<long long>(k) * row_elems);
    float sum = 0.f;
    for (int w = 0; w < window_count; w++)
        sum += load_elem(packed, text_positions[w * text_tokens + k] * packed_row + e, packed_elemsize);
    store_elem(out, k * out_row + e, out_elemsize, sum / static_cast<float>(window_count));
}

// ---- Fused-path text mean over the per-window partials [nwin][T_x][H][d]
// (fp32 or bf16, the layer's output type) ----
// One thread per output element pair. Windows are read in batches of 16
// unconditional loads (indices past the last window are clamped to it and
// their values replaced by zero), so that a layer of up to 16 windows waits
// for one memory latency; the sum keeps window order (adding +0 leaves every
// partial sum unchanged).
template <typename TPart>
__global__ void text_mean_kernel(const TPart* partials, int window_count, int text_tokens, int row_elems,
                                 void* out, long long out_row, int out_elemsize)
{
    constexpr int kBatch = 16;
    const int pairs = row_elems / 2;
    const long long total = static_cast<long long>(text_tokens) * pairs;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int k = static_cast<int>(idx / pairs);
    const int e = 2 * static_cast<int>(idx - static_cast<long long>(k) * pairs);
    const long long window_stride = static_cast<long long>(text_tokens) * row_elems;
    const TPart* src = partials + static_cast<long long>(k) * row_elems + e;
    // Element pair (x, y) of window w's partial row.
    auto load_pair = [&](long long w) -> float2 {
        if constexpr (sizeof(TPart) == 4)
            return *reinterpret_cast<const float2*>(src + w * window_stride);
        else
        {
            const uint32_t b = *reinterpret_cast<const uint32_t*>(src + w * window_stride);
            return make_float2(__uint_as_float(b << 16), __uint_as_float(b & 0xffff0000u));
        }
    };
    float sx = 0.f, sy = 0.f;
    const int last = window_count - 1;
    for (int w = 0; w < window_count; w += kBatch)
    {
        float2 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++)
            v[j] = load_pair(min(w + j, last));
#pragma unroll
        for (int j = 0; j < kBatch; j++)
        {
            const bool valid = w + j < window_count;
            sx += valid ? v[j].x : 0.f;
            sy += valid ? v[j].y : 0.f;
        }
    }
    const float n = static_cast<float>(window_count);
    const long long o = k * out_row + e;
    if (out_elemsize == 4)
        *reinterpret_cast<float2*>(static_cast<float*>(out) + o) = make_float2(sx / n, sy / n);
    else
        *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + o) =
            f32_to_bf16(sx / n) | (static_cast<uint32_t>(f32_to_bf16(sy / n)) << 16);
}

// ---- Split layers: the key segments of each row combined. Segment s of a
// row holds O_s (unnormalised, relative to its running maximum m_s, in log2
// units) and its probability sum l_s; with M = max m_s and w_s = 2^(m_s - M),
// the row is (sum_s w_s O_s) * (1 / sum_s w_s l_s), the form the unsplit
// kernels use (O * (1 / l)). ----
template <int NB>
__device__ __forceinline__ void merge_segments(const SplitMerge& m, const long long (&p)[NB], int head, int f0,
                                               float (&r)[NB][8])
{
    // Rows p[0..NB) at once: every (max, sum) load, then every row load,
    // issued before any is used (kMaxSegments unrolled, predicated by split).
    constexpr int kMaxSegments = 8;
    float2 ml[NB][kMaxSegments];
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int s = 0; s < kMaxSegments; s++)
            if (s < m.split)
                ml[j][s] = m.ml[(p[j] * m.heads + head) * m.split + s];
#pragma unroll
    for (int j = 0; j < NB; j++)
    {
        const long long base = (p[j] * m.heads + head) * m.split;
        float4 o[kMaxSegments][2];
#pragma unroll
        for (int s = 0; s < kMaxSegments; s++)
            if (s < m.split)
            {
                const float4* src = reinterpret_cast<const float4*>(m.o + (base + s) * 128 + f0);
                o[s][0] = src[0];
                o[s][1] = src[1];
            }
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < kMaxSegments; s++)
            if (s < m.split)
                mx = fmaxf(mx, ml[j][s].x);
        float l = 0.f;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kMaxSegments; s++)
            if (s < m.split)
            {
                const float w = __builtin_amdgcn_exp2f(ml[j][s].x - mx);
                l = fmaf(w, ml[j][s].y, l);
                const float v[8] = {o[s][0].x, o[s][0].y, o[s][0].z, o[s][0].w,
                                    o[s][1].x, o[s][1].y, o[s][1].z, o[s][1].w};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    acc[i] = fmaf(w, v[i], acc[i]);
            }
        const float inv = 1.f / l;
#pragma unroll
        for (int i = 0; i < 8; i++)
            r[j][i] = acc[i] * inv;
    }
}

__device__ __forceinline__ void store8(void* dst, int elemsize, const float (&r)[8])
{
    if (elemsize == 4)
    {
        float4* d = static_cast<float4*>(dst);
        d[0] = make_float4(r[0], r[1], r[2], r[3]);
        d[1] = make_float4(r[4], r[5], r[6], r[7]);
    }
    else
    {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            w[i] = f32_to_bf16(r[2 * i]) | (static_cast<uint32_t>(f32_to_bf16(r[2 * i + 1])) << 16);
        *static_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// One thread per 8 features of one (row, head): fused mode covers the video
// tokens, then the text rows (each a window-order mean); packed mode every
// packed row.
__global__ __launch_bounds__(kBlock) void split_merge_kernel(const SplitMerge m)
{
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int f0 = 8 * static_cast<int>(idx & 15);
    const long long row_head = idx >> 4;
    const int head = static_cast<int>(row_head % m.heads);
    const long long row = row_head / m.heads;
    if (!m.fused)
    {
        if (row >= m.sequence_tokens)
            return;
        float r[1][8];
        merge_segments<1>(m, {row}, head, f0, r);
        store8(m.packed_out + row * m.packed_row + head * 128 + f0, 4, r[0]);
        return;
    }
    if (row < m.video_tokens)
    {
        const int v = static_cast<int>(row);
        float r[1][8];
        merge_segments<1>(m, {static_cast<long long>(m.video_positions[v])}, head, f0, r);
        const int area = m.source_h * m.source_w;
        const int t = v / area;
        const int h = (v - t * area) / m.source_w;
        const int w = v - t * area - h * m.source_w;
        const long long off = t * m.video_out.ts + h * m.video_out.hs + w * m.video_out.ws + head * 128 + f0;
        store8(static_cast<unsigned char*>(m.video_out.data) + off * m.video_out.elemsize, m.video_out.elemsize,
               r[0]);
        return;
    }
    const int k = static_cast<int>(row - m.video_tokens);
    if (k >= m.text_tokens)
        return;
    // Window-order sum of the windows' rows (rounded to bf16 first when the
    // unsplit path would store bf16 partials), then the division by nwin;
    // kBatch windows' loads at a time (indices past the last window are
    // clamped to it and their rows not added).
    constexpr int kBatch = 4;
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int w0 = 0; w0 < m.window_count; w0 += kBatch)
    {
        long long pos[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++)
        {
            const WindowDesc win = m.windows[min(w0 + j, m.window_count - 1)];
            pos[j] = win.seq_start + win.video_tokens + k;
        }
        float r[kBatch][8];
        merge_segments<kBatch>(m, pos, head, f0, r);
#pragma unroll
        for (int j = 0; j < kBatch; j++)
            if (w0 + j < m.window_count)
#pragma unroll
                for (int i = 0; i < 8; i++)
                    sum[i] += m.text_round_bf16 ? bf16_to_f32(f32_to_bf16(r[j][i])) : r[j][i];
    }
    const float n = static_cast<float>(m.window_count);
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        r[i] = sum[i] / n;
    store8(static_cast<unsigned char*>(m.text_out) + (k * m.text_row + head * 128 + f0) * m.text_elemsize,
           m.text_elemsize, r);
}

// ---- DitRMSNorm (src/dit/dit_precision.cpp:63-86, src/dit/shader/dit_rmsnorm.comp):
// one 128-thread workgroup per (row, channel). Lane l sums x[i]^2 over i = l,
// l + 128, ... (products and sums rounded separately, as the shader's
// `precise` asks: no contraction here), the 128 partial sums are added
// pairwise (stride 64, 32,
// ..., 1), coefficient = 1 / sqrt(sum / width + eps); out = x * coefficient,
// times gamma[i] when gamma is given. ----
__global__ __launch_bounds__(128) void rmsnorm_kernel(const void* in, int in_elemsize, long long in_cstep, void* out,
                                                      int out_elemsize, long long out_cstep, int width,
                                                      const float* gamma, float eps)
{
#pragma clang fp contract(off)
    __shared__ float sums[128];
    const int lane = threadIdx.x;
    const long long src = static_cast<long long>(blockIdx.y) * in_cstep + static_cast<long long>(blockIdx.x) * width;
    const long long dst = static_cast<long long>(blockIdx.y) * out_cstep + static_cast<long long>(blockIdx.x) * width;
    float sum = 0.f;
    for (int i = lane; i < width; i += 128)
    {
        const float v = load_elem(in, src + i, in_elemsize);
        sum += v * v;
    }
    sums[lane] = sum;
    __syncthreads();
    for (int stride = 64; stride > 0; stride /= 2)
    {
        if (lane < stride)
            sums[lane] += sums[lane + stride];
        __syncthreads();
    }
    const float coefficient = 1.f / sqrtf(sums[0] / static_cast<float>(width) + eps);
    for (int i = lane; i < width; i += 128)
    {
        float v = load_elem(in, src + i, in_elemsize) * coefficient;
        if (gamma)
            v *= gamma[i];
        store_elem(out, dst + i, out_elemsize, v);
    }
}

// ---- Generic window attention, any head_dim: one wave per (window-row, head) ----
// Lanes stride over features; online softmax over keys with wave reductions.
__global__ void attention_generic_kernel(const void* packed_in, long long in_row, int in_elemsize, float* out,
                                         long long out_row, const int* cu_seqlens, int window_count, int heads,
                                         int head_dim, int sequence_tokens, float scale)
{
    const int wave_global = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int row = wave_global / heads;
    const int head = wave_global - row * heads;
    if (row >= sequence_tokens)
        return;
    int lo = 0, hi = window_count;
    while (hi - lo > 1)
    {
        const int mid = (lo + hi) >> 1;
        if (cu_seqlens[mid] <= row)
            lo = mid;
        else
            hi = mid;
    }
    const int start = cu_seqlens[lo];
    const int end = cu_seqlens[lo + 1];
    constexpr int kMaxPerLane = 16; // head_dim <= 1024
    float q[kMaxPerLane], acc[kMaxPerLane];
    for (int j = 0; j < kMaxPerLane; j++)
    {
        const int f = lane + 64 * j;
        q[j] = f < head_dim ? load_elem(packed_in, row * in_row + head * head_dim + f, in_elemsize) : 0.f;
        acc[j] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int key = start; key < end; key++)
    {
        float dot = 0.f;
        for (int j = 0; j < kMaxPerLane; j++)
        {
            const int f = lane + 64 * j;
            if (f < head_dim)
                dot += q[j] * load_elem(packed_in, key * in_row + (heads + head) * head_dim + f, in_elemsize);
        }
        for (int off = 32; off > 0; off >>= 1)
            dot += __shfl_xor(dot, off);
        const float s = dot * scale;
        const float m_new = fmaxf(m, s);
        const float alpha = __expf(m - m_new);
        const float pk = __expf(s - m_new);
        l = l * alpha + pk;
        for (int j = 0; j < kMaxPerLane; j++)
        {
            const int f = lane + 64 * j;
            const float v =
                f < head_dim ? load_elem(packed_in, key * in_row + (2 * heads + head) * head_dim + f, in_elemsize) : 0.f;
            acc[j] = acc[j] * alpha + pk * v;
        }
        m = m_new;
    }
    for (int j = 0; j < kMaxPerLane; j++)
    {
        const int f = lane + 64 * j;
        if (f < head_dim)
            out[row * out_row + head * head_dim + f] = acc[j] / l;
    }
}

// ---- Strided cast (src/awa/shader/cast_bf16_f32.comp / cast_f32_bf16.comp semantics) ----
__global__ void cast_kernel(const void* in, int in_elemsize, void* out, int out_elemsize, CastShape s)
{
    const long long total = static_cast<long long>(s.w) * s.h * s.d * s.c * s.n;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const long long plane = static_cast<long long>(s.w) * s.h * s.d;
    const long long channel_index = idx / plane;
    const long long inner = idx - channel_index * plane;
    const long long b = channel_index / s.c;
    const long long c = channel_index - b * s.c;
    const float v = load_elem(in, b * s.in_nstep + c * s.in_cstep + inner, in_elemsize);
    store_elem(out, b * s.out_nstep + c * s.out_cstep + inner, out_elemsize, v);
}

// ---- DitQKVConcat: out[token][y][x] = q / k / v[token][y % heads][x] for y in
// [0, heads) / [heads, 2 heads) / [2 heads, 3 heads); v fp32 or bf16 (exact
// promotion), out fp32. One thread per 4 consecutive x when every row is
// 16-byte aligned, else per element. ----
__global__ void qkv_concat_kernel(const float* q, long long q_cstep, const float* k, long long k_cstep,
                                  const void* v, int v_elemsize, long long v_cstep, float* out, long long out_cstep,
                                  int width, int heads, int tokens, int vec)
{
    const int groups = width / vec;
    const long long per_token = 3ll * heads * groups;
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= per_token * tokens)
        return;
    const long long token = idx / per_token;
    const int rem = static_cast<int>(idx - token * per_token);
    const int y = rem / groups;
    const int x = (rem - y * groups) * vec;
    const int head = y % heads;
    const long long i = static_cast<long long>(head) * width + x;
    float* dst = out + token * out_cstep + static_cast<long long>(y) * width + x;
    if (vec == 4)
    {
        float4 val;
        if (y < heads)
            val = *reinterpret_cast<const float4*>(q + token * q_cstep + i);
        else if (y < 2 * heads)
            val = *reinterpret_cast<const float4*>(k + token * k_cstep + i);
        else if (v_elemsize == 4)
            val = *reinterpret_cast<const float4*>(static_cast<const float*>(v) + token * v_cstep + i);
        else
        {
            const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(v) + token * v_cstep + i);
            val = make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                              __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
        }
        *reinterpret_cast<float4*>(dst) = val;
        return;
    }
    if (y < heads)
        *dst = q[token * q_cstep + i];
    else if (y < 2 * heads)
        *dst = k[token * k_cstep + i];
    else
        *dst = load_elem(v, token * v_cstep + i, v_elemsize);
}

// ---- Seeded N(0,1): splitmix64 counter hash -> two 32-bit uniforms -> Box-Muller ----
__device__ __forceinline__ uint64_t splitmix64(uint64_t x)
{
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

__global__ void fill_normal_kernel(void* dst, size_t count, int elemsize, unsigned long long seed, float stddev)
{
    const size_t pair = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t i0 = 2 * pair;
    if (i0 >= count)
        return;
    const uint64_t r = splitmix64(seed * 0x100000001b3ull + pair);
    const float u1 = (static_cast<float>(static_cast<uint32_t>(r >> 32)) + 0.5f) * 2.3283064365386963e-10f;
    const float u2 = (static_cast<float>(static_cast<uint32_t>(r)) + 0.5f) * 2.3283064365386963e-10f;
    const float radius = sqrtf(-2.f * logf(u1));
    float sn, cs;
    sincosf(6.283185307179586f * u2, &sn, &cs);
    store_elem(dst, static_cast<long long>(i0), elemsize, stddev * (radius * cs));
    if (i0 + 1 < count)
        store_elem(dst, static_cast<long long>(i0 + 1), elemsize, stddev * (radius * sn));
}

__global__ void zero_kernel(uint32_t* dst, size_t words, unsigned char* tail, size_t tail_bytes)
{
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < words)
        dst[i] = 0u;
    if (i < tail_bytes)
        tail[i] = 0;
}

unsigned grid_for(long long total)
{
    return static_cast<unsigned>((total + kBlock - 1) / kBlock);
}

} // namespace

hipError_t launch_text_mean(const void* partials, int partial_elemsize, int window_count, int text_tokens, int heads, int head_dim,
                            void* text_out, long long text_token_stride, int out_elemsize, hipStream_t stream)
{
    const int row_elems = heads * head_dim;
    const long long total = static_cast<long long>(text_tokens) * (row_elems / 2);
    if (partial_elemsize == 4)
        hipLaunchKernelGGL(text_mean_kernel<float>, dim3(grid_for(total)), dim3(kBlock), 0, stream,
                           static_cast<const float*>(partials), window_count, text_tokens, row_elems, text_out,
                           text_token_stride, out_elemsize);
    else if (partial_elemsize == 2)
        hipLaunchKernelGGL(text_mean_kernel<uint16_t>, dim3(grid_for(total)), dim3(kBlock), 0, stream,
                           static_cast<const uint16_t*>(partials), window_count, text_tokens, row_elems, text_out,
                           text_token_stride, out_elemsize);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_split_merge(const SplitMerge& m, hipStream_t stream)
{
    if (m.split < 2 || m.heads <= 0)
        return hipErrorInvalidValue;
    const long long rows = m.fused ? static_cast<long long>(m.video_tokens) + m.text_tokens : m.sequence_tokens;
    const long long total = rows * m.heads * 16;
    hipLaunchKernelGGL(split_merge_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, m);
    return hipGetLastError();
}

hipError_t launch_attention_generic(const void* packed_in, long long in_row, int in_elemsize, float* out,
                                    long long out_row, const int* cu_seqlens_dev, int window_count, int heads,
                                    int head_dim, int sequence_tokens, hipStream_t stream)
{
    if (head_dim > 1024)
        return hipErrorInvalidValue;
    const long long waves = static_cast<long long>(sequence_tokens) * heads;
    const float scale = 1.f / sqrtf(static_cast<float>(head_dim));
    hipLaunchKernelGGL(attention_generic_kernel, dim3(grid_for(waves * 64)), dim3(kBlock), 0, stream, packed_in,
                       in_row, in_elemsize, out, out_row, cu_seqlens_dev, window_count, heads, head_dim,
                       sequence_tokens, scale);
    return hipGetLastError();
}

hipError_t launch_pack(const RowInfo* rows, int sequence_tokens, int source_tokens, const QkvSource& video,
                       const QkvSource& text, int heads, int head_dim, float* packed, long long packed_row,
                       hipStream_t stream)
{
    const long long total = static_cast<long long>(sequence_tokens) * 3 * heads * head_dim;
    hipLaunchKernelGGL(pack_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, rows, sequence_tokens,
                       source_tokens, video, text, heads, head_dim, packed, packed_row);
    return hipGetLastError();
}

hipError_t launch_cu_seqlens(const int* cu_dev, int count, float* out, hipStream_t stream)
{
    hipLaunchKernelGGL(cu_seqlens_kernel, dim3(grid_for(count)), dim3(kBlock), 0, stream, cu_dev, count, out);
    return hipGetLastError();
}

hipError_t launch_mmrope(const RowInfo* rows, int sequence_tokens, const void* in, long long in_row,
                         int in_elemsize, float* out, long long out_row, int heads, int head_dim, int rope_dim,
                         int rope_pairs, const float* rope_cs, hipStream_t stream)
{
    const long long total = static_cast<long long>(sequence_tokens) * (3 * heads * head_dim / 2);
    hipLaunchKernelGGL(mmrope_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, rows, sequence_tokens, in,
                       in_row, in_elemsize, out, out_row, heads, head_dim, rope_dim, rope_pairs, rope_cs);
    return hipGetLastError();
}

hipError_t launch_unpack_video(const int* video_positions, int source_t, int source_h, int source_w,
                               const void* packed, long long packed_row, int packed_elemsize, const VideoSink& out,
                               int heads, int head_dim, hipStream_t stream)
{
    const int row_elems = heads * head_dim;
    const long long total = static_cast<long long>(source_t) * source_h * source_w * row_elems;
    hipLaunchKernelGGL(unpack_video_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, video_positions,
                       source_t, source_h, source_w, packed, packed_row, packed_elemsize, out, row_elems);
    return hipGetLastError();
}

hipError_t launch_unpack_text(const int* text_positions, int window_count, int text_tokens, const void* packed,
                              long long packed_row, int packed_elemsize, void* out, long long out_row,
                              int out_elemsize, int heads, int head_dim, hipStream_t stream)
{
    const int row_elems = heads * head_dim;
    const long long total = static_cast<long long>(text_tokens) * row_elems;
    hipLaunchKernelGGL(unpack_text_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, text_positions,
                       window_count, text_tokens, packed, packed_row, packed_elemsize, out, out_row, out_elemsize,
                       row_elems);
    return hipGetLastError();
}

hipError_t launch_cast(const void* in, int in_elemsize, void* out, int out_elemsize, const CastShape& s,
                       hipStream_t stream)
{
    const long long total = static_cast<long long>(s.w) * s.h * s.d * s.c * s.n;
    hipLaunchKernelGGL(cast_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, in, in_elemsize, out,
                       out_elemsize, s);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const void* in, int in_elemsize, long long in_cstep, void* out, int out_elemsize,
                          long long out_cstep, int width, int rows, int channels, const float* gamma, float eps,
                          hipStream_t stream)
{
    if (rows <= 0 || channels <= 0 || width <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows, channels), dim3(128), 0, stream, in, in_elemsize, in_cstep, out,
                       out_elemsize, out_cstep, width, gamma, eps);
    return hipGetLastError();
}

hipError_t launch_qkv_concat(const float* q, long long q_cstep, const float* k, long long k_cstep, const void* v,
                             int v_elemsize, long long v_cstep, float* out, long long out_cstep, int width, int heads,
                             int tokens, hipStream_t stream)
{
    if (width <= 0 || heads <= 0 || tokens <= 0)
        return hipSuccess;
    const bool aligned = width % 4 == 0 && q_cstep % 4 == 0 && k_cstep % 4 == 0 && v_cstep % 4 == 0 &&
                         out_cstep % 4 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v) % (4 * v_elemsize) == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const int vec = aligned ? 4 : 1;
    const long long total = 3ll * heads * (width / vec) * tokens;
    hipLaunchKernelGGL(qkv_concat_kernel, dim3(grid_for(total)), dim3(kBlock), 0, stream, q, q_cstep, k, k_cstep, v,
                       v_elemsize, v_cstep, out, out_cstep, width, heads, tokens, vec);
    return hipGetLastError();
}

hipError_t launch_fill_normal(void* dst, size_t count, int elemsize, unsigned long long seed, float stddev,
                              hipStream_t stream)
{
    const long long pairs = static_cast<long long>((count + 1) / 2);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(pairs)), dim3(kBlock), 0, stream, dst, count, elemsize,
                       seed, stddev);
    return hipGetLastError();
}

hipError_t launch_zero(void* dst, size_t bytes, hipStream_t stream)
{
    const size_t words = bytes / 4;
    const size_t tail = bytes - words * 4;
    const long long threads = static_cast<long long>(words > tail ? words : tail);
    if (threads == 0)
        return hipSuccess;
    hipLaunchKernelGGL(zero_kernel, dim3(grid_for(threads)), dim3(kBlock), 0, stream, static_cast<uint32_t*>(dst),
                       words, static_cast<unsigned char*>(dst) + words * 4, tail);
    return hipGetLastError();
}

} // namespace awa
