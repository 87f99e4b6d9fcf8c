// Launch interface of the AWA HIP kernels (gfx950). All pointers are device
// pointers; strides are in elements.
#pragma once

#include <hip/hip_runtime.h>

#include "awa_plan.h"

namespace awa
{

constexpr int kHeadDim = 128;   // head_dim of the MFMA attention kernels
constexpr int kRopeDim = 126;   // rope_dim of the fused kernel
constexpr int kQueryRows = 128;     // query rows per workgroup (4 waves of 32)
constexpr int kWideQueryRows = 256; // query rows per workgroup of the wide variant (8 waves)

// Attention kernel variants.
constexpr int kVariantNarrow = 0;   // 4 waves, single-buffered tiles
constexpr int kVariantWidePipe = 1; // 8 waves, double-buffered, software-pipelined
constexpr int kVariantWide = 2;     // 8 waves, single-buffered tiles (the narrow loop on 256 rows)
constexpr int kMaxRopeCoords = 128; // RoPE coordinates the fused kernel holds in LDS
// Windows the attention kernels accept: fewer rows than this (the float
// reciprocal row decode is exact below it), and LDS tiles + tables within a
// workgroup's share of a CU's LDS.
constexpr int kMaxWindowRows = 1 << 14;
constexpr size_t kWorkgroupLds = 160 * 1024;

// One QKV source: row of (token, qkv, head) starts at
// token * token_stride + qkv * qkv_stride + head * head_dim.
struct QkvSource
{
    const void* data;
    long long token_stride;
    long long qkv_stride;
    int elemsize;
};

// Video output addressing: token (t, h, w) starts at t*ts + h*hs + w*ws.
struct VideoSink
{
    void* data;
    long long ts, hs, ws;
    int elemsize;
};

struct AttentionLaunch
{
    bool fused;      // gather + RoPE from video/text sources, scatter to video/text
    bool bf16_mfma;  // AWA_COMPUTE_BF16
    int variant;     // kVariant*: kVariantWidePipe takes work items of kWideQueryRows rows
    // fused inputs / outputs
    QkvSource video, text;
    VideoSink video_out;
    void* text_partials;  // [nwin][T_x][H][d], fp32 or bf16 (text_partial_elemsize)
    int text_partial_elemsize;
    // fused q/k RMSNorm over head_dim: gammas q video, k video, q text, k text
    bool qk_norm;
    const float* norm_gamma[4];
    float norm_eps;
    // packed inputs / outputs (fused == false)
    const void* packed_in;
    long long packed_in_row;
    int packed_in_elemsize;
    float* packed_out;
    long long packed_out_row;
    // geometry
    const WindowDesc* windows;
    const WorkItem* work;
    int work_count;
    const float* rope_cs;
    int rope_coords;
    int max_window_tokens; // rows of the largest window (fused-mode LDS row table)
    int heads;
    int text_tokens;
    int source_h, source_w;
    float scale_log2; // (1/sqrt(head_dim)) * log2(e)
    // split > 1: every row's keys are split into `split` segments (the work
    // items' key ranges); the kernel writes each segment's unnormalised row
    // split_o[((p * heads + head) * split + seg) * head_dim + f] (p the packed
    // row: window seq_start + window row) and its (running maximum in log2
    // units, probability sum) to split_ml[same index / head_dim], and
    // launch_split_merge combines them.
    int split;
    float* split_o;
    float2* split_ml;
};

// Combines the key segments of a split layer (AttentionLaunch::split): per
// row and head, M = max m_s, out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
// Fused mode writes video rows to their grid position and the text rows'
// window-order mean (each window's row rounded to bf16 first when
// text_round_bf16, as the unsplit path's partials are); packed mode writes
// every packed row to packed_out.
struct SplitMerge
{
    const float* o;
    const float2* ml;
    int split, heads;
    bool fused;
    // fused: video
    int video_tokens;
    const int* video_positions; // token -> packed row
    int source_h, source_w;
    VideoSink video_out;
    // fused: text
    int text_tokens, window_count;
    const WindowDesc* windows;
    void* text_out;
    long long text_row;
    int text_elemsize;
    bool text_round_bf16;
    // packed
    int sequence_tokens;
    float* packed_out;
    long long packed_row;
};
hipError_t launch_split_merge(const SplitMerge& m, hipStream_t stream);

hipError_t launch_attention(const AttentionLaunch& p, hipStream_t stream);
// LDS of one workgroup of that kernel: the static K/V tiles of the variant
// (bf16 or fp32 MFMA) and the dynamic norm / RoPE / row tables of a launch.
size_t attention_static_lds(bool bf16_mfma, int variant);
size_t attention_dynamic_lds(const AttentionLaunch& p);

// fp32 window attention with nearly exact scores: Q/K as int8 digit slices
// on int8 MFMA (exact int32 sums), P V as bf16 pieces on bf16 MFMA
// (AWA_COMPUTE_F32). Variants kVariantNarrow / kVariantWide.
hipError_t launch_attention_x(const AttentionLaunch& p, hipStream_t stream);
// LDS of one workgroup of that kernel: static tiles (double-buffered in the
// 8-wave form), and the dynamic RoPE / row tables for a launch.
size_t attention_x_static_lds(bool wide);
size_t attention_x_dynamic_lds(const AttentionLaunch& p, bool norm);

// text_out[k][head][:] = (sum_w partials[w][k][head][:]) / nwin, window order.
hipError_t launch_text_mean(const void* partials, int partial_elemsize, int window_count, int text_tokens, int heads, int head_dim,
                            void* text_out, long long text_token_stride, int out_elemsize, hipStream_t stream);

// Generic (head_dim <= 1024) window attention over a packed [S][3H][d] blob;
// used by the staged entry point when head_dim != 128.
hipError_t launch_attention_generic(const void* packed_in, long long in_row, int in_elemsize, float* out,
                                    long long out_row, const int* cu_seqlens_dev, int window_count, int heads,
                                    int head_dim, int sequence_tokens, hipStream_t stream);

hipError_t launch_pack(const RowInfo* rows, int sequence_tokens, int source_tokens, const QkvSource& video,
                       const QkvSource& text, int heads, int head_dim, float* packed, long long packed_row,
                       hipStream_t stream);

hipError_t launch_cu_seqlens(const int* cu_dev, int count, float* out, hipStream_t stream);

hipError_t launch_mmrope(const RowInfo* rows, int sequence_tokens, const void* in, long long in_row,
                         int in_elemsize, float* out, long long out_row, int heads, int head_dim, int rope_dim,
                         int rope_pairs, const float* rope_cs, hipStream_t stream);

hipError_t launch_unpack_video(const int* video_positions, int source_t, int source_h, int source_w,
                               const void* packed, long long packed_row, int packed_elemsize, const VideoSink& out,
                               int heads, int head_dim, hipStream_t stream);

hipError_t launch_unpack_text(const int* text_positions, int window_count, int text_tokens, const void* packed,
                              long long packed_row, int packed_elemsize, void* out, long long out_row,
                              int out_elemsize, int heads, int head_dim, hipStream_t stream);

// Strided element cast between fp32 and bf16 (or same-type copy): element
// (x, y, z, c, b) at b*nstep + c*cstep + (z*h + y)*w + x on both sides.
struct CastShape
{
    int w, h, d, c, n;
    long long in_cstep, in_nstep, out_cstep, out_nstep;
};
hipError_t launch_rmsnorm(const void* in, int in_elemsize, long long in_cstep, void* out, int out_elemsize,
                          long long out_cstep, int width, int rows, int channels, const float* gamma, float eps,
                          hipStream_t stream);
hipError_t launch_cast(const void* in, int in_elemsize, void* out, int out_elemsize, const CastShape& s,
                       hipStream_t stream);

// DitQKVConcat: out[token][3 heads][width] (fp32) from q, k (fp32) and v
// (fp32 or bf16), each [token][heads][width] with its own token step.
hipError_t launch_qkv_concat(const float* q, long long q_cstep, const float* k, long long k_cstep, const void* v,
                             int v_elemsize, long long v_cstep, float* out, long long out_cstep, int width, int heads,
                             int tokens, hipStream_t stream);

hipError_t launch_fill_normal(void* dst, size_t count, int elemsize, unsigned long long seed, float stddev,
                              hipStream_t stream);
hipError_t launch_zero(void* dst, size_t bytes, hipStream_t stream);

} // namespace awa
