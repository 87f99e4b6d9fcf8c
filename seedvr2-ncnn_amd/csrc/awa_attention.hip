// Window attention kernels for gfx950 (CDNA4).
//
// Each wave owns 32 query rows of one (window, head) and computes the
// transposed score tile S^T = K Q^T with 32x32 MFMAs, so that a lane holds one
// query column: the online-softmax statistics of a query live in two lanes
// (lane and lane^32), and the rescale of the output accumulator O^T = V^T P^T
// is lane-local. A workgroup is 4 waves (128 query rows; bf16 MFMA) or 8
// waves (256 query rows; bf16 MFMA single-buffered, or the fp32 MFMA
// pipeline), see the variants below.
//
// K and V tiles (64 keys for bf16, 32 for fp32) are staged through LDS (K
// row-major, V transposed so that the PV operand reads are contiguous in the
// key index). Keys are read out of the K tile in an order (bits 2 and 3 of the
// row swapped) that makes every lane's 16 probabilities of a 32-key block
// cover two runs of 8 consecutive keys, which is exactly the K-slot layout of
// the B operand of the PV MFMA. bf16 tiles hold two 32-key blocks whose
// score MFMA chains are interleaved.
//
// In fused mode the kernel gathers rows straight from the video / text QKV
// blobs using the window geometry (the reference's Pack), applies the 3-axis
// interleaved RoPE while staging Q and K (MMRoPE), and writes video rows to
// their grid position (Unpack); text rows go to per-window partials that a
// second kernel averages in window order. Packed mode reads a packed
// [S][3H][d] blob and writes [S][H][d], for the staged WindowAttention layer.
//
// Per-tile VALU work is kept small: the window's row -> (source offset, RoPE
// coordinates) table is built once per workgroup in LDS (padded to whole
// tiles, so staging loads need no bounds checks), the softmax scale is folded
// into Q, masking only runs on a ragged last tile, and (bf16) the output
// accumulator is only rescaled when a row maximum grows by more than 2^8
// (exact: numerator and denominator share the stale maximum). The next
// tile's global loads are in flight while the current tile is computed.
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

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Bytes of one wave's output stage: 32 rows of 128 bf16 features and 32 row
// pointers.
constexpr int kOutStageWaveBytes = 32 * kHeadDim * 2 + 32 * 8;

// Static LDS of a kernel instance: the K tile (keys x padded head_dim) and the
// V tile (bf16: keys x padded head_dim; fp32: head_dim x padded keys), 64
// bf16 keys or 32 fp32 keys, double-buffered in the fp32 pipeline; the bf16
// kernels' output stage reuses the space and may need more.
constexpr int static_lds_bytes(bool bf16, int variant)
{
    const int tiles = bf16 ? 64 * (kHeadDim + 8) * 2 + 64 * (kHeadDim + 32) * 2
                           : 32 * (kHeadDim + 4) * 4 + kHeadDim * (32 + 4) * 4;
    const int buffered = (variant == kVariantWidePipe ? 2 : 1) * tiles;
    const int waves = variant == kVariantNarrow ? 4 : 8;
    return bf16 && buffered < waves * kOutStageWaveBytes ? waves * kOutStageWaveBytes : buffered;
}

// Variants (AttentionLaunch::variant):
//   kVariantNarrow: 4 waves (128 query rows), single-buffered K/V tiles of 64
//     (bf16) or 32 (fp32) keys, two barriers per tile; the LDS footprint stays
//     under half a CU's, so that two workgroups share a CU.
//   kVariantWide: the same loop on 8 waves (256 query rows): a unit of up to
//     256 rows stages and rotates its K/V tiles once.
//   kVariantWidePipe: 8 waves (256 query rows), double-buffered tiles and a
//     software pipeline with one barrier per tile: the scores of tile t+1 and
//     the PV of tile t are issued next to the softmax of tile t and the
//     staging of the next tiles.
// NORM (fused mode): the DiT block's q/k RMSNorm over head_dim is applied to
// Q and K rows as they are gathered, before RoPE.
template <typename TIn, typename TOut, bool BF16, bool FUSED, int VARIANT, bool NORM>
__global__ __launch_bounds__(VARIANT != kVariantNarrow ? 512 : 256,
                             VARIANT != kVariantNarrow ? 1 : 2) void window_attention_kernel(const AttentionLaunch p)
{
    static_assert(!NORM || FUSED, "the q/k RMSNorm is fused into the gather");
    constexpr bool WIDE = VARIANT != kVariantNarrow;
    constexpr bool PIPE = VARIANT == kVariantWidePipe;
    constexpr int kThreads = WIDE ? 512 : 256;
    constexpr int kQueryRows = kThreads / 2; // 32 rows per wave
    static_assert(kQueryRows == (WIDE ? awa::kWideQueryRows : awa::kQueryRows), "work items match the variant");
    constexpr int kBufs = PIPE ? 2 : 1;
    // Key tile and LDS layout (pitches in elements; rows stay 16-byte aligned).
    // 64-key tiles (two 32-key score blocks) on bf16 MFMA, 32 on fp32 MFMA.
    constexpr int KT = BF16 ? 64 : 32;
    constexpr int kKPitch = BF16 ? kHeadDim + 8 : kHeadDim + 4;
    // bf16: V row-major [key][feature] (pitch 160 elements: the transposed
    // operand reads below hit distinct banks); fp32: V^T [feature][key].
    constexpr int kVPitch = BF16 ? kHeadDim + 32 : KT + 4;
    constexpr int kElem = BF16 ? 2 : 4;
    constexpr int kRW = kRawWords8<TIn>;
    constexpr int kKBytes = KT * kKPitch * kElem;
    constexpr int kVBytes = (BF16 ? KT : kHeadDim) * kVPitch * kElem;
    constexpr int kBlocks = KT / 32; // 32-key score blocks per tile

    // bf16 fused kernels stage each wave's output rows through LDS after the
    // loop (see the store below): 32 rows of 256 bytes plus 32 row pointers
    // per wave, in the tile buffers' space.
    constexpr bool kStageOut = BF16 && FUSED;
    constexpr int kStaticBytes = static_lds_bytes(BF16, VARIANT);
    static_assert(kStaticBytes >= kBufs * (kKBytes + kVBytes), "tiles fit the static LDS");
    static_assert(!kStageOut || kStaticBytes >= (kThreads / 64) * kOutStageWaveBytes, "output stage fits");
    // With the output stage, one array holds the K tiles, then the V tiles.
    __shared__ __attribute__((aligned(16))) unsigned char k_lds[kStageOut ? kStaticBytes : kBufs * kKBytes];
    __shared__ __attribute__((aligned(16))) unsigned char v_lds_own[kStageOut ? 16 : kBufs * kVBytes];
    unsigned char* const v_lds = kStageOut ? k_lds + kBufs * kKBytes : v_lds_own;
    unsigned char* const tile_lds = k_lds;
    // Dynamic LDS: the RoPE table (fused mode; its coordinates plus an
    // identity row), then the row table.
    extern __shared__ __attribute__((aligned(16))) unsigned char dyn_lds[];
    float* const norm_lds = reinterpret_cast<float*>(dyn_lds); // NORM: K gammas, video then text
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
    // Key tiles of this item: all of them, or one segment of a split layer
    // (its key range starts at a multiple of 64 keys; the pipelined fp32
    // variant is never split).
    const int t_begin = PIPE ? 0 : item.key0 / KT;
    const int t_end = PIPE ? tiles : min(tiles, (item.key1 + KT - 1) / KT);
    const int table_rows = (p.max_window_tokens + 63) & ~63;

    // Wave-uniform scalars read once from the kernel arguments (plain values,
    // so that per-lane selects never turn into indexed struct accesses).
    const TIn* const video_base = static_cast<const TIn*>(p.video.data);
    const TIn* const text_base = static_cast<const TIn*>(p.text.data);
    const long long v_tok = p.video.token_stride;
    const long long v_qkv = p.video.qkv_stride;
    const long long t_tok = p.text.token_stride;
    const long long t_qkv = p.text.qkv_stride;
    const TIn* const packed_base = static_cast<const TIn*>(p.packed_in);
    const long long packed_row = p.packed_in_row;
    const long long packed_qkv = static_cast<long long>(p.heads) * kHeadDim;
    const float scale_log2 = p.scale_log2;

    const RowDivisors divisors = row_divisors(win);
    auto decode = [&](int i) { return window_row(win, divisors, i, p.text_tokens, p.source_h, p.source_w); };
    // Element pointer of (decoded window row, qkv, head) in its source blob.
    auto source_ptr = [&](const RowRef& r, int qkv) -> const TIn* {
        return r.text ? text_base + r.k * t_tok + qkv * t_qkv + head_off
                      : video_base + static_cast<long long>(r.token) * v_tok + qkv * v_qkv + head_off;
    };
    // Element pointer of (window row i < L, qkv, head).
    auto row_ptr = [&](int i, int qkv) -> const TIn* {
        if constexpr (FUSED)
            return source_ptr(decode(i), qkv);
        else
            return packed_base + (win.seq_start + i) * packed_row + qkv * packed_qkv + head_off;
    };

    const int wave_row0 = item.row0 + wave * 32;
    // Waves past the item's rows only stage; their rows (if any) belong to
    // another work item and are neither computed nor stored here.
    const bool wave_active = wave * 32 < item.rows && wave_row0 < L;
    const int qi = wave_row0 + col;
    const bool q_valid = wave_active && qi < L;
    const int q_row = min(qi, L - 1);

    // Q rows go straight to registers; their addresses do not need the table.
    uint32_t qraw[8 * kRW];
    {
        const TIn* q_src = row_ptr(q_row, 0);
#pragma unroll
        for (int c = 0; c < 8; c++)
            load_raw8(q_src + (BF16 ? 16 * c + 8 * half : 64 * half + 8 * c), qraw + c * kRW);
    }

    // Row table (LDS), padded to whole tiles with copies of the last row so
    // that every staging load is unconditional and in bounds (padded keys are
    // masked, padded values weighted by zero): the byte offsets of each row's
    // K and V from a kernel-argument base pointer (so that the loads stay
    // global-memory loads, which the LDS counters do not wait on) and, in
    // fused mode, its RoPE coordinates ct | ch << 8 | cw << 16 (all below 128)
    // with byte 3 naming the table's identity row.
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
            // One decode per row: V sits one qkv step after K.
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

    // ---- staging assignment ----
    // Loads are coalesced: 16 consecutive threads read the 16 chunks of 8
    // features of one row, so each load instruction covers 4 whole rows.
    // Thread tid owns chunk kc = tid % 16 of K rows kr0 + 16 j and of V key
    // groups g = kr0 + 16 j: keys 2g, 2g + 1 for bf16 MFMA (one 32-bit word
    // of the transposed tile), key g for fp32 MFMA.
    constexpr int kRowsPerPass = kThreads / 16;     // rows one load instruction set covers
    constexpr int kKRows = KT / kRowsPerPass;       // K rows per thread
    constexpr int kVKeys = BF16 ? 2 : 1;            // keys per V word group
    constexpr int kVGroups = KT / kVKeys / kRowsPerPass; // V key groups per thread
    static_assert(kKRows >= 1 && kVGroups >= 1 && kKRows * kRowsPerPass == KT &&
                      kVGroups * kRowsPerPass * kVKeys == KT,
                  "staging split");
    const int kc = tid & 15;
    const int kr0 = tid >> 4;
    // RoPE of this thread's feature pairs 4kc .. 4kc+3: the coordinate of pair
    // q is byte rope_shift[q] / 8 of the row's coordinate word (byte 3 names
    // the identity row: unrotated features 126, 127), and rope_col[q] is its
    // column in the table.
    int rope_shift[4], rope_col[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
    {
        const int pair = 4 * kc + q;
        const int axis = 2 * pair < kRopeDim ? pair / kRopePairs : 3;
        rope_shift[q] = 8 * axis;
        rope_col[q] = axis < 3 ? 2 * (pair - axis * kRopePairs) : 0;
    }

    // One register stage: tile t+1's loads are in flight while tile t is
    // computed.
    struct Stage
    {
        uint32_t k[kKRows * kRW];
        uint32_t v[kVGroups * kVKeys * kRW];
    };
    Stage st;

    auto load_k_to = [&](int tile, uint32_t* dst) {
#pragma unroll
        for (int j = 0; j < kKRows; j++)
            load_raw8(reinterpret_cast<const TIn*>(load_base + row_k[tile * KT + kr0 + kRowsPerPass * j]) + 8 * kc,
                      dst + j * kRW);
    };
    auto load_k = [&](int tile) { load_k_to(tile, st.k); };
    auto load_v = [&](int tile) {
#pragma unroll
        for (int j = 0; j < kVGroups; j++)
#pragma unroll
            for (int i = 0; i < kVKeys; i++)
                load_raw8(reinterpret_cast<const TIn*>(
                              load_base + row_v[tile * KT + kVKeys * (kr0 + kRowsPerPass * j) + i]) +
                              8 * kc,
                          st.v + (j * kVKeys + i) * kRW);
    };
    auto load_tile = [&](int tile) {
        load_k(tile);
        load_v(tile);
    };

    auto store_k_from = [&](int tile, int buf, const uint32_t* src) {
        unsigned char* const kb = k_lds + buf * kKBytes;
        // The (cos, sin) of every pair of this thread's K rows are read before
        // any is used, so that their LDS latency is paid once per tile rather
        // than once per row and pair (in the bf16 kernels a scheduling
        // barrier keeps the compiler from interleaving them back).
        float2 cs[FUSED ? kKRows : 1][4];
        if constexpr (FUSED)
        {
            uint32_t code[kKRows];
#pragma unroll
            for (int j = 0; j < kKRows; j++)
                code[j] = row_code[tile * KT + kr0 + kRowsPerPass * j];
#pragma unroll
            for (int j = 0; j < kKRows; j++)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    cs[j][q] = *reinterpret_cast<const float2*>(rope_lds + ((code[j] >> rope_shift[q]) & 255u) * kRopeRow +
                                                                rope_col[q]);
            if constexpr (BF16)
                __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < kKRows; j++)
        {
            const int row = kr0 + kRowsPerPass * j;
            const int lds_row = (row & ~31) | key_permute(row & 31);
            float kv[8];
            raw_to_float8<TIn>(src + j * kRW, kv);
            if constexpr (FUSED)
            {
                if constexpr (NORM)
                {
                    // RMSNorm of the K row over head_dim (its 16 chunks sit
                    // in 16 consecutive lanes), then the video or text gamma.
                    float ss = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        ss = fmaf(kv[e], kv[e], ss);
                    const float coef = __builtin_amdgcn_rsqf(sum16(ss) * (1.f / kHeadDim) + p.norm_eps);
                    const bool text = tile * KT + row >= win.video_tokens;
                    const float* const g = norm_lds + (text ? kHeadDim : 0) + 8 * kc;
                    const float4 g0 = *reinterpret_cast<const float4*>(g);
                    const float4 g1 = *reinterpret_cast<const float4*>(g + 4);
                    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        kv[e] = (kv[e] * coef) * gv[e];
                }
#pragma unroll
                for (int q = 0; q < 4; q++)
                {
                    if constexpr (BF16)
                        rope_pair_fma(kv[2 * q], kv[2 * q + 1], cs[j][q].x, cs[j][q].y);
                    else
                        rope_pair_cs(kv[2 * q], kv[2 * q + 1], cs[j][q].x, cs[j][q].y);
                }
            }
            if constexpr (BF16)
            {
                uint16_t* ks = reinterpret_cast<uint16_t*>(kb) + lds_row * kKPitch + 8 * kc;
                *reinterpret_cast<uint4*>(ks) = make_uint4(cvt_pk_bf16(kv[0], kv[1]), cvt_pk_bf16(kv[2], kv[3]),
                                                           cvt_pk_bf16(kv[4], kv[5]), cvt_pk_bf16(kv[6], kv[7]));
            }
            else
            {
                float* ks = reinterpret_cast<float*>(kb) + lds_row * kKPitch + 8 * kc;
                *reinterpret_cast<float4*>(ks) = make_float4(kv[0], kv[1], kv[2], kv[3]);
                *reinterpret_cast<float4*>(ks + 4) = make_float4(kv[4], kv[5], kv[6], kv[7]);
            }
        }
    };
    auto store_k = [&](int tile, int buf) { store_k_from(tile, buf, st.k); };
    auto store_v = [&](int buf) {
        unsigned char* const vb = v_lds + buf * kVBytes;
        if constexpr (BF16)
        {
            // Row-major: each thread's 8 features of a key, one 16-byte store.
#pragma unroll
            for (int j = 0; j < kVGroups; j++)
#pragma unroll
                for (int i = 0; i < kVKeys; i++)
                {
                    const int key = kVKeys * (kr0 + kRowsPerPass * j) + i;
                    const uint32_t* const sv = st.v + (j * kVKeys + i) * kRW;
                    uint4 w;
                    if constexpr (sizeof(TIn) == 2)
                        w = make_uint4(sv[0], sv[1], sv[2], sv[3]);
                    else
                        w = make_uint4(cvt_pk_bf16(__uint_as_float(sv[0]), __uint_as_float(sv[1])),
                                       cvt_pk_bf16(__uint_as_float(sv[2]), __uint_as_float(sv[3])),
                                       cvt_pk_bf16(__uint_as_float(sv[4]), __uint_as_float(sv[5])),
                                       cvt_pk_bf16(__uint_as_float(sv[6]), __uint_as_float(sv[7])));
                    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(vb) + key * kVPitch + 8 * kc) = w;
                }
        }
        else
        {
            // V transposed: Vt[d][key], keys swizzled in groups of 8 per feature chunk.
#pragma unroll
            for (int j = 0; j < kVGroups; j++)
            {
                const int key = (kVKeys * (kr0 + kRowsPerPass * j)) ^ (8 * vt_swizzle<KT>(8 * kc));
                const uint32_t* const sv = st.v + j * kVKeys * kRW;
#pragma unroll
                for (int e = 0; e < 8; e++)
                {
                    float v;
                    if constexpr (sizeof(TIn) == 2)
                        v = (e & 1) ? bf16_hi(sv[e >> 1]) : bf16_lo(sv[e >> 1]);
                    else
                        v = __uint_as_float(sv[e]);
                    reinterpret_cast<float*>(vb)[(8 * kc + e) * kVPitch + key] = v;
                }
            }
        }
    };
    auto store_tile = [&](int tile, int buf) {
        store_k(tile, buf);
        store_v(buf);
    };

    // ---- prologue: tile 0's loads, the RoPE table into LDS (plus an
    // identity row after the last coordinate), Q rotated and scaled in
    // registers ----
    load_tile(t_begin);
    // The pipeline also stages K(1) before its first step.
    uint32_t k1[PIPE ? kKRows * kRW : 1];
    if constexpr (PIPE)
        load_k_to(min(1, tiles - 1), k1);
    uint32_t q_code = 0; // RoPE coordinate word of this lane's query row
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

    // Q into registers (B operand of S^T = K Q^T), scaled by log2(e)/sqrt(d).
    // bf16: lane holds features 16c + 8*half + [0,8) for c = 0..7.
    // fp32: lane holds features 64*half + [0,64).
    bf16x8 qb[BF16 ? 8 : 1];
    float qf[BF16 ? 1 : 64];
    // Optional q RMSNorm over head_dim (the lane and its partner lane ^ 32
    // hold the row's two halves): coefficient and the row's gamma.
    float q_coef = 1.f;
    const float* q_gamma = nullptr;
    if constexpr (NORM)
    {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < 8; c++)
        {
            float v[8];
            raw_to_float8<TIn>(qraw + c * kRW, v);
#pragma unroll
            for (int e = 0; e < 8; e++)
                ss = fmaf(v[e], v[e], ss);
        }
        q_coef = __builtin_amdgcn_rsqf(sum_xor32(ss) * (1.f / kHeadDim) + p.norm_eps);
        q_gamma = q_row >= win.video_tokens ? p.norm_gamma[2] : p.norm_gamma[0];
    }
#pragma unroll
    for (int c = 0; c < 8; c++)
    {
        float v[8];
        raw_to_float8<TIn>(qraw + c * kRW, v);
        if constexpr (NORM)
        {
            const int f0 = BF16 ? 16 * c + 8 * half : 64 * half + 8 * c;
            const float4 g0 = *reinterpret_cast<const float4*>(q_gamma + f0);
            const float4 g1 = *reinterpret_cast<const float4*>(q_gamma + f0 + 4);
            const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                v[e] = (v[e] * q_coef) * g[e];
        }
        if constexpr (FUSED)
        {
            // 4 pairs from pair 8c + 4*half (bf16) or 32*half + 4c (fp32):
            // their axes and table columns are compile-time for either half,
            // one select picks the lane's.
#pragma unroll
            for (int q = 0; q < 4; q++)
            {
                const int p0 = (BF16 ? 8 * c : 4 * c) + q;
                const int p1 = (BF16 ? 8 * c + 4 : 32 + 4 * c) + q;
                const int ax0 = 2 * p0 < kRopeDim ? p0 / kRopePairs : 3;
                const int ax1 = 2 * p1 < kRopeDim ? p1 / kRopePairs : 3;
                const int col0 = ax0 < 3 ? 2 * (p0 - ax0 * kRopePairs) : 0;
                const int col1 = ax1 < 3 ? 2 * (p1 - ax1 * kRopePairs) : 0;
                const uint32_t coord = (q_code >> (half ? 8 * ax1 : 8 * ax0)) & 255u;
                const float2 t =
                    *reinterpret_cast<const float2*>(rope_lds + coord * kRopeRow + (half ? col1 : col0));
                if constexpr (BF16)
                    rope_pair_fma(v[2 * q], v[2 * q + 1], t.x, t.y);
                else
                    rope_pair_cs(v[2 * q], v[2 * q + 1], t.x, t.y);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++)
            v[e] *= scale_log2;
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


    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[db][i] = 0.f;
    // The bf16 kernel keeps its scores relative to the running maximum: the
    // score MFMA chains start from -row_max (negm), so that exp2 needs no
    // subtraction. Before the first tile row_max is 0 and the first tile
    // always sets it.
    constexpr bool kRel = BF16 && !PIPE;
    float row_max = kRel ? 0.f : -INFINITY; // running maximum (log2 domain), possibly stale by < 2^8
    float row_sum = 0.f;                    // partial sum over this lane's keys
    f32x16 negm;
#pragma unroll
    for (int i = 0; i < 16; i++)
        negm[i] = 0.f;

    const int krow = col; // K rows are stored key-permuted

    // S^T = K Q^T of one tile: one 32x32 block per 32 keys; chains interleaved.
    // nb: 32-key blocks of the tile that hold keys of the window (1 on a
    // last tile of at most 32 keys, whose second block would be all masked).
    auto scores = [&](f32x16 (&s)[kBlocks], int buf, auto nb) {
        constexpr int NB = decltype(nb)::value;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                s[b][i] = 0.f;
        if constexpr (BF16)
        {
            // The chains start from -row_max in the relative form (the first
            // MFMA's C operand), from zero otherwise.
            f32x16 c0;
#pragma unroll
            for (int i = 0; i < 16; i++)
                c0[i] = 0.f;
            if constexpr (kRel)
                c0 = negm;
            const uint16_t* ks =
                reinterpret_cast<const uint16_t*>(k_lds + buf * kKBytes) + krow * kKPitch + 8 * half;
            // The K operand reads run kAhead feature steps ahead of the MFMAs
            // that use them. The scheduling barriers pin that order: left to
            // itself the compiler sinks each read next to its MFMA, behind a
            // wait for that read alone, and every MFMA then waits a full LDS
            // latency. (The narrow kernels on fp32 input keep one read ahead:
            // their register stages leave no room for more.)
            constexpr int kAhead = WIDE || sizeof(TIn) == 2 ? 3 : 1;
            bf16x8 ka[kBlocks][8];
#pragma unroll
            for (int c = 0; c < kAhead; c++)
#pragma unroll
                for (int b = 0; b < NB; b++)
                    ka[b][c] = *reinterpret_cast<const bf16x8*>(ks + b * 32 * kKPitch + 16 * c);
#pragma unroll
            for (int c = 0; c < 8; c++)
            {
                if (c + kAhead < 8)
#pragma unroll
                    for (int b = 0; b < NB; b++)
                        ka[b][c + kAhead] = *reinterpret_cast<const bf16x8*>(ks + b * 32 * kKPitch + 16 * (c + kAhead));
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[b][c], qb[c], c == 0 ? c0 : s[b], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        else
        {
            // Two interleaved chains over this lane's 64 features (32x32x2
            // f32 MFMAs), so that consecutive MFMAs are independent.
            const float* ks = reinterpret_cast<const float*>(k_lds + buf * kKBytes) + krow * kKPitch + 64 * half;
            f32x16 s1;
#pragma unroll
            for (int i = 0; i < 16; i++)
                s1[i] = 0.f;
#pragma unroll
            for (int c4 = 0; c4 < 16; c4++)
            {
                const float4 ka = *reinterpret_cast<const float4*>(ks + 4 * c4);
                s[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.x, qf[4 * c4 + 0], s[0], 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.y, qf[4 * c4 + 1], s1, 0, 0, 0);
                s[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.z, qf[4 * c4 + 2], s[0], 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ka.w, qf[4 * c4 + 3], s1, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; i++)
                s[0][i] += s1[i];
        }
    };

    // Online softmax of one tile's scores; the probabilities replace them.
    // Register i of score block b holds key 32b + 16*(i/8) + 8*half + i%8.
    // lazy: O is rescaled only when a row maximum grows by more than 2^8 (a
    // wave-uniform branch); otherwise every tile rescales, without a branch,
    // so that the code can be interleaved with independent MFMA work.
    // may_mask: the tile can be the ragged last one.
    auto softmax = [&](f32x16 (&s)[kBlocks], int tile, auto lazy, auto may_mask, auto nb) {
        constexpr int NB = decltype(nb)::value;
        if (decltype(may_mask)::value && tile == tiles - 1 && (L % KT))
        {
            const int key0 = tile * KT + 8 * half;
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    if (key0 + 32 * b + 16 * (i >> 3) + (i & 7) >= L)
                        s[b][i] = -INFINITY;
        }
        float tile_max = s[0][0];
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                tile_max = fmaxf(tile_max, s[b][i]);
        tile_max = max_xor32(tile_max);
        if constexpr (kRel)
        {
            // tile_max is relative to row_max.
            if (tile == t_begin || __any(tile_max > kRescaleThreshold))
            {
                const float delta = tile == t_begin ? tile_max : fmaxf(tile_max, 0.f);
                if (tile != t_begin)
                {
                    const float alpha = __builtin_amdgcn_exp2f(-delta);
                    row_sum *= alpha;
#pragma unroll
                    for (int db = 0; db < 4; db++)
#pragma unroll
                        for (int i = 0; i < 16; i++)
                            o[db][i] *= alpha;
                }
                row_max += delta;
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        s[b][i] -= delta;
#pragma unroll
                for (int i = 0; i < 16; i++)
                    negm[i] = -row_max;
            }
            // The row sum is taken in pv(), over the bf16 probabilities.
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    s[b][i] = __builtin_amdgcn_exp2f(s[b][i]);
            return;
        }
        if (!decltype(lazy)::value || __any(tile_max > row_max + kRescaleThreshold))
        {
            const float new_max = fmaxf(row_max, tile_max);
            const float alpha = __builtin_amdgcn_exp2f(row_max - new_max);
            row_max = new_max;
            row_sum *= alpha;
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    o[db][i] *= alpha;
        }
        float psum = 0.f;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
            {
                s[b][i] = __builtin_amdgcn_exp2f(s[b][i] - row_max);
                psum += s[b][i];
            }
        row_sum += psum;
    };

    // O^T += V^T P^T of one tile.
    auto pv = [&](const f32x16 (&s)[kBlocks], int buf, auto nb) {
        constexpr int NB = decltype(nb)::value;
        if constexpr (BF16)
        {
            bf16x8 pb[2 * kBlocks];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                {
                    pb[2 * b][e] = static_cast<__bf16>(s[b][e]);
                    pb[2 * b + 1][e] = static_cast<__bf16>(s[b][8 + e]);
                }
            if constexpr (kRel)
            {
                // Row sum over the probabilities as the MFMA sees them (bf16):
                // one dot product with (1, 1) per pair, so that numerator and
                // denominator share the rounding.
                const bf16x2 ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
#pragma unroll
                for (int j = 0; j < 2 * NB; j++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                    {
                        const bf16x2 pair = {pb[j][2 * q], pb[j][2 * q + 1]};
                        row_sum = __builtin_amdgcn_fdot2_f32_bf16(pair, ones, row_sum, false);
                    }
            }
            // V^T operands read transposed from the row-major tile
            // (ds_read_b64_tr_b16): within each group of 16 lanes, lane j
            // addresses key row 8*half + j/4 (+4 for the second read) and
            // features 16*(group & 1) + 4*(j & 3) of a 32-feature block, and
            // receives column j of the 4 x 16 block its group read: keys
            // 16 step + 8 half + [0, 8) of feature 32 db + col. The four
            // output chains are interleaved: consecutive MFMAs are independent.
            const uint16_t* vt = reinterpret_cast<const uint16_t*>(v_lds + buf * kVBytes) +
                                 (8 * half + ((lane & 15) >> 2)) * kVPitch + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
            for (int j = 0; j < 2 * NB; j++)
            {
                bf16x8 va[4];
#pragma unroll
                for (int db = 0; db < 4; db++)
                {
                    const uint16_t* const base = vt + 16 * j * kVPitch + 32 * db;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 4 * kVPitch));
                    const i16x4 lohi[2] = {lo, hi};
                    va[db] = __builtin_bit_cast(bf16x8, lohi);
                }
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[db], pb[j], o[db], 0, 0, 0);
            }
        }
        else
        {
            // The four output chains are interleaved: consecutive MFMAs are
            // independent.
            const float* vt = reinterpret_cast<const float*>(v_lds + buf * kVBytes);
#pragma unroll
            for (int g = 0; g < 4; g++)
            {
                float4 va[4];
#pragma unroll
                for (int db = 0; db < 4; db++)
                {
                    const int d = db * 32 + col;
                    va[db] = *reinterpret_cast<const float4*>(
                        vt + d * kVPitch + ((16 * (g >> 1) + 8 * half + 4 * (g & 1)) ^ (8 * vt_swizzle<KT>(d))));
                }
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[db].x, s[0][4 * g + 0], o[db], 0, 0, 0);
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[db].y, s[0][4 * g + 1], o[db], 0, 0, 0);
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[db].z, s[0][4 * g + 2], o[db], 0, 0, 0);
#pragma unroll
                for (int db = 0; db < 4; db++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[db].w, s[0][4 * g + 3], o[db], 0, 0, 0);
            }
        }
    };

    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;
    using AllBlocks = std::integral_constant<int, kBlocks>;
    using OneBlock = std::integral_constant<int, 1>;
    if constexpr (PIPE)
    {
        // Software pipeline, one barrier per tile, K and V double-buffered
        // (buffer t & 1 holds tile t). Step t:
        //   1. S(t+1) = K(t+1) Q^T (MFMA) with the softmax of S(t) (VALU; fp32
        //      rescales every tile, without a branch) and V(t+1) into its
        //      buffer;
        //   2. O += V(t) P(t) (MFMA) with K(t+2) into buffer t & 1.
        // Buffer writes never meet reads of the same step: V(t+1)'s buffer
        // was last read by step t-1's PV and K(t+2)'s by step t-1's scores.
        // Register stages: V(t+1) and K(t+2) are loaded one step before they
        // are stored; loads past the last tile are clamped to it (in bounds,
        // never used).
        const int last = tiles - 1;
        store_tile(0, 0);
        store_k_from(min(1, last), 1, k1);
        load_v(min(1, last));
        load_k(min(2, last));
        __syncthreads();
        f32x16 s[kBlocks];
        if (wave_active)
            scores(s, 0, AllBlocks());
        __syncthreads(); // K buffer 0 is rewritten in step 0
        for (int tile = 0; tile < last; tile++)
        {
            const int buf = tile & 1;
            if (wave_active)
            {
                f32x16 sn[kBlocks];
                scores(sn, buf ^ 1, AllBlocks());
                softmax(s, tile, std::integral_constant<bool, BF16>(), No(), AllBlocks());
                store_v(buf ^ 1);
                load_v(min(tile + 2, last));
                pv(s, buf, AllBlocks());
                store_k(min(tile + 2, last), buf);
                load_k(min(tile + 3, last));
#pragma unroll
                for (int b = 0; b < kBlocks; b++)
                    s[b] = sn[b];
            }
            else
            {
                store_v(buf ^ 1);
                load_v(min(tile + 2, last));
                store_k(min(tile + 2, last), buf);
                load_k(min(tile + 3, last));
            }
            __syncthreads();
        }
        if (wave_active)
        {
            softmax(s, last, std::integral_constant<bool, BF16>(), Yes(), AllBlocks());
            pv(s, last & 1, AllBlocks());
        }
    }
    else
    {
        // Step t: stage tile t into LDS, refill the registers with tile t+1's
        // loads, then scores, softmax and PV of tile t. A last tile of at
        // most 32 keys runs its first score block only (the second would be
        // masked whole: probabilities 0, the same bits); it is peeled off the
        // loop so that the loop body keeps one form. (Kernels on fp32 inputs,
        // whose register stages leave no room for the second form, keep the
        // loop whole.)
        auto step = [&](int tile, auto nb) {
            store_tile(tile, 0);
            __syncthreads();
            if (tile + 1 < t_end)
                load_tile(tile + 1);
            if (wave_active)
            {
                f32x16 s[kBlocks];
                scores(s, 0, nb);
                softmax(s, tile, Yes(), Yes(), nb);
                pv(s, 0, nb);
            }
            __syncthreads();
        };
        const bool short_last = kBlocks > 1 && sizeof(TIn) == 2 && L - (t_end - 1) * KT <= 32;
        const int full_end = short_last ? t_end - 1 : t_end;
        for (int tile = t_begin; tile < full_end; tile++)
            step(tile, AllBlocks());
        if constexpr (kBlocks > 1 && sizeof(TIn) == 2)
            if (short_last)
                step(t_end - 1, OneBlock());
    }

    if (p.split > 1)
    {
        // ---- one key segment of a split layer: the unnormalised row (relative
        // to the running maximum) and (maximum, probability sum), for
        // launch_split_merge ----
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
    if constexpr (kStageOut)
    {
        // ---- store through LDS: the lane pair (col, half) holds row col's
        // features db*32 + 8*g + 4*half + [0,4); the wave writes its rows as
        // bf16 into its own LDS region (16-byte chunk c of row i at position
        // c ^ (i & 15): conflict-free both ways), then reads them back 16
        // bytes a lane, 16 lanes a row, and writes whole 256-byte rows. Rows
        // with an fp32 destination (fp32 outputs or text rows) are stored
        // directly; rows past the window are not stored. The row stores are
        // nontemporal: dirty lines left in L2 lengthen the kernel's end (the
        // text mean then reads its rows from beyond L2, which costs it less
        // than the attention kernel gains). ----
        if (!wave_active)
            return;
        const float inv = 1.f / sum_xor32(row_sum);
        unsigned char* const region = tile_lds + wave * kOutStageWaveBytes;
        uint16_t* const rows_lds = reinterpret_cast<uint16_t*>(region);
        unsigned long long* const dst_lds = reinterpret_cast<unsigned long long*>(region + 32 * 256);
        uint16_t* dst16 = nullptr;
        if (q_valid)
        {
            const RowRef r = decode(qi);
            if (!r.text)
            {
                TOut* dst = static_cast<TOut*>(p.video_out.data) + r.t * p.video_out.ts + r.h * p.video_out.hs +
                            r.w * p.video_out.ws + head_off;
                if constexpr (sizeof(TOut) == 2)
                    dst16 = dst;
                else
                    store_row(dst, o, inv, half);
            }
            else
            {
                // Text partials in the text output's type (bf16 rows are
                // rounded before the mean, as in the reference's bf16 layer).
                const long long off =
                    ((static_cast<long long>(item.window) * p.text_tokens + r.k) * p.heads + head) * kHeadDim;
                if (p.text_partial_elemsize == 2)
                    dst16 = static_cast<uint16_t*>(p.text_partials) + off;
                else
                    store_row(static_cast<float*>(p.text_partials) + off, o, inv, half);
            }
        }
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int g = 0; g < 4; g++)
            {
                const int chunk = (4 * db + g) ^ (col & 15);
                *reinterpret_cast<uint2*>(rows_lds + col * kHeadDim + 8 * chunk + 4 * half) =
                    make_uint2(cvt_pk_bf16(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                               cvt_pk_bf16(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv));
            }
        if (half == 0)
            dst_lds[col] = reinterpret_cast<unsigned long long>(dst16);
        // The wave reads what its own lanes wrote.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int chunk = lane & 15;
#pragma unroll
        for (int j = 0; j < 8; j++)
        {
            const int row = 4 * j + (lane >> 4);
            const u32x4 v = *reinterpret_cast<const u32x4*>(rows_lds + row * kHeadDim + 8 * (chunk ^ (row & 15)));
            uint16_t* const d = reinterpret_cast<uint16_t*>(dst_lds[row]);
            if (d)
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(d + 8 * chunk));
        }
        return;
    }
    if (!q_valid)
        return;
    const float inv = 1.f / sum_xor32(row_sum);

    // ---- store: lane holds features db*32 + 8*g + 4*half + [0,4) ----
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
            // Text partials are stored in the text output's type: with a bf16
            // text output the per-window rows are rounded to bf16 before they
            // are averaged, as the packed attention output is in a bf16 layer.
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

size_t attention_static_lds(bool bf16_mfma, int variant)
{
    return static_lds_bytes(bf16_mfma, variant);
}

size_t attention_dynamic_lds(const AttentionLaunch& p)
{
    // Norm gammas, RoPE table, then the row table: K and V row offsets and one
    // coordinate word per row, padded to whole 64-row tiles.
    const size_t row_table = static_cast<size_t>((p.max_window_tokens + 63) & ~63) * (2 * sizeof(long long) + 4);
    return (p.qk_norm ? 2 * kHeadDim * 4 : 0) + rope_table_bytes(p.fused, p.rope_coords) + row_table;
}

template <typename TIn, typename TOut, bool BF16, bool FUSED, int VARIANT, bool NORM>
static hipError_t launch_one(const AttentionLaunch& p, hipStream_t stream)
{
    const size_t dynamic_lds = attention_dynamic_lds(p);
    hipLaunchKernelGGL((window_attention_kernel<TIn, TOut, BF16, FUSED, VARIANT, NORM>), dim3(p.work_count),
                       dim3(VARIANT != kVariantNarrow ? 512 : 256), dynamic_lds, stream, p);
    return hipGetLastError();
}

template <bool BF16, bool FUSED, int VARIANT, bool NORM = false>
static hipError_t launch_typed(const AttentionLaunch& p, hipStream_t stream)
{
    const int in_size = FUSED ? p.video.elemsize : p.packed_in_elemsize;
    const int out_size = FUSED ? p.video_out.elemsize : 4;
    if (in_size == 4 && out_size == 4)
        return launch_one<float, float, BF16, FUSED, VARIANT, NORM>(p, stream);
    if (in_size == 2 && out_size == 4)
        return launch_one<uint16_t, float, BF16, FUSED, VARIANT, NORM>(p, stream);
    if constexpr (FUSED)
    {
        if (in_size == 4 && out_size == 2)
            return launch_one<float, uint16_t, BF16, FUSED, VARIANT, NORM>(p, stream);
        if (in_size == 2 && out_size == 2)
            return launch_one<uint16_t, uint16_t, BF16, FUSED, VARIANT, NORM>(p, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_attention(const AttentionLaunch& p, hipStream_t stream)
{
    if (p.work_count <= 0)
        return hipSuccess;
    // Instantiated: bf16 MFMA in the narrow and the 8-wave single-buffered
    // variants, fp32 MFMA in the 8-wave pipelined one; the fused q/k RMSNorm
    // in fused mode only.
    if (p.qk_norm && !p.fused)
        return hipErrorInvalidValue;
    if (p.bf16_mfma)
    {
        if (p.variant == kVariantWide)
        {
            if (!p.fused)
                return launch_typed<true, false, kVariantWide>(p, stream);
            return p.qk_norm ? launch_typed<true, true, kVariantWide, true>(p, stream)
                             : launch_typed<true, true, kVariantWide>(p, stream);
        }
        if (p.variant != kVariantNarrow)
            return hipErrorInvalidValue;
        if (!p.fused)
            return launch_typed<true, false, kVariantNarrow>(p, stream);
        return p.qk_norm ? launch_typed<true, true, kVariantNarrow, true>(p, stream)
                         : launch_typed<true, true, kVariantNarrow>(p, stream);
    }
    if (p.variant != kVariantWidePipe)
        return hipErrorInvalidValue;
    if (!p.fused)
        return launch_typed<false, false, kVariantWidePipe>(p, stream);
    return p.qk_norm ? launch_typed<false, true, kVariantWidePipe, true>(p, stream)
                     : launch_typed<false, true, kVariantWidePipe>(p, stream);
}

} // namespace awa
