/*
 * seedvr2_awa.h — C ABI of the MI355X (gfx950) adaptive-window-attention path.
 *
 * This is the boundary a host (C, C++, ctypes, ...) binds to replace the
 * reference's AWA operator chain
 *   SeedVR2AWAPack -> SeedVR2MMRoPE -> SeedVR2WindowAttention -> SeedVR2AWAUnpack
 * (src/awa/awa_layers.h:47-220, src/awa/awa_layers.cpp:363-1291) and the
 * Vulkan memory/sync helpers it relies on (src/vulkan/transient_staging_allocator.h:10-23,
 * src/inference/vulkan_benchmark.h:22-31). Every entry point uses plain
 * pointers, sizes and the descriptor structs below; no C++ or framework types.
 *
 * Conventions
 *  - Return codes follow the reference layers: 0 success, -1 invalid argument,
 *    shape or state (src/awa/awa_layers.cpp:423-434, :506-525), -100 allocation
 *    failure (:438-439). AWA_ERR_DEVICE (-2) reports a HIP runtime error, which
 *    has no reference counterpart. awa_last_error() returns the diagnostic of
 *    the calling thread's last failure.
 *  - Device work is enqueued on the given stream (NULL = the default stream)
 *    and is asynchronous; the caller synchronises (awa_stream_synchronize
 *    replaces the reference's submit_and_wait_profiled).
 *  - Plans are immutable after awa_plan_upload except for their device
 *    workspace (work list, text rows). A forward holds the plan's lock from
 *    its workspace check until its kernels are enqueued, so calls from several
 *    threads never launch on a freed work list; but a call with another head
 *    count replaces the workspace while kernels of an earlier call on another
 *    stream may still read it. Use one plan per stream.
 */
#ifndef SEEDVR2_AWA_H
#define SEEDVR2_AWA_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AWA_OK 0
#define AWA_ERR_INVALID (-1)
#define AWA_ERR_DEVICE (-2)
#define AWA_ERR_ALLOC (-100)

/* Arithmetic of the attention contractions. AWA_COMPUTE_F32 (the reference's
 * AWA arithmetic, which is fp32 in every block: src/awa/awa_layers.cpp:203-213)
 * takes fp32 or bf16 Q, K, V. It computes each score q.k as a correctly
 * rounded fp32 dot product, the accuracy the reference's Kahan-sum shaders
 * aim for. Q and K rows are written as four balanced base-256 digit slices
 * under a per-row power of two and multiplied on int8 matrix cores with exact
 * int32 sums. P V uses P and V as three bf16 pieces each (all 24 bits of the
 * fp32 values) on bf16 matrix cores with fp32 accumulation. AWA_COMPUTE_BF16
 * rounds Q, K, V and P to bf16 and accumulates in fp32 on bf16 MFMA; this is
 * the bf16-MFMA arithmetic of the BF16 blocks. AWA_COMPUTE_F32_MFMA runs QK^T
 * and PV on fp32 MFMA with plain fp32 accumulation. It is slower, and less
 * accurate when scores are large or cancel; it is kept for comparison.
 * Softmax statistics are fp32 in all three. */
#define AWA_COMPUTE_F32 0
#define AWA_COMPUTE_BF16 1
#define AWA_COMPUTE_F32_MFMA 2

/* A device blob described the way an ncnn Mat is (elempack 1):
 * dims 1..4 with extents w (fastest), h, d, c; n batches (NCNN_BATCH, 1 when
 * unused); cstep / nstep in elements; elemsize 4 (fp32) or 2 (bf16). */
typedef struct awa_blob {
    void* data;
    int dims;
    int w, h, d, c;
    int n;
    int elemsize;
    long long cstep;
    long long nstep;
} awa_blob;

/* Layer parameters, with the reference's param ids (src/awa/awa_layers.cpp:90-114, :872):
 * 0/1/2 source_t/h/w (-1,-1,-1 = take them from the runtime spec, as the
 * dynamic model package does), 3/4/5 window COUNTS along t/h/w over the grid
 * rescaled to area 45x80, 6 text tokens, 7 shifted, 8 rope_dim (a positive
 * multiple of 6; the reference's layer defaults an absent param 8 to 126).
 * runtime_* is the AwaRuntimeSpec (src/awa/awa_layers.h:31-39); set
 * runtime_tokens = 0 when there is none. heads (no reference counterpart:
 * the layers learn it from the input blob) is optional: when positive,
 * awa_plan_upload also builds the attention work list for that head count,
 * which awa_forward_noalloc needs; 0 leaves it to the first forward. */
typedef struct awa_plan_desc {
    int source_t, source_h, source_w;
    int windows_t, windows_h, windows_w;
    int text_tokens;
    int shifted;
    int rope_dim;
    int runtime_t, runtime_h, runtime_w, runtime_tokens;
    int heads;
} awa_plan_desc;

typedef struct awa_plan_info {
    int source_t, source_h, source_w;
    int source_tokens;     /* N = t*h*w */
    int text_tokens;       /* T_x */
    int window_count;      /* nwin */
    int sequence_tokens;   /* S = N + nwin*T_x (packed rows) */
    int window_t, window_h, window_w; /* unclipped window extents */
    int max_window_tokens; /* max L over windows */
    int rope_dim;
    int shifted;
} awa_plan_info;

typedef struct awa_plan awa_plan;

/* ---- runtime: device, memory, streams, events (replaces src/vulkan for this path) ---- */

const char* awa_last_error(void);
int awa_device_count(int* count);
/* Selects the device for the calling thread and sets up the device's static
 * scratch buffer of awa_forward_noalloc (its memory is reserved then, once per
 * device, and held until the process ends). */
int awa_runtime_init(int device);
int awa_malloc(void** ptr, size_t bytes);
int awa_free(void* ptr);
/* Pinned host memory for staging (allocated, never registered). */
int awa_host_alloc(void** ptr, size_t bytes);
int awa_host_free(void* ptr);
int awa_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int awa_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int awa_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Fills bytes with zero using a kernel (safe inside captured graphs). */
int awa_zero(void* dst, size_t bytes, void* stream);
int awa_stream_create(void** stream);
int awa_stream_destroy(void* stream);
int awa_stream_synchronize(void* stream);
int awa_event_create(void** event);
int awa_event_destroy(void* event);
int awa_event_record(void* event, void* stream);
int awa_event_synchronize(void* event);
int awa_event_elapsed_ms(void* start, void* stop, float* ms);
/* Seeded N(0,1) synthetic data on the device (counter-based, Box-Muller);
 * elemsize 4 or 2 (bf16, rounded to nearest even). Used to build benchmark
 * inputs; parity tests use the host generator of the reference instead. */
int awa_fill_normal(void* dst, size_t count, int elemsize, unsigned long long seed, void* stream);
/* The same numbers times stddev (random-init weights, e.g. N(0, 0.02)). */
int awa_fill_normal_scaled(void* dst, size_t count, int elemsize, unsigned long long seed, float stddev,
                           void* stream);

/* ---- plan: windows, index maps, RoPE tables (the layers' load_param/upload_model) ---- */

/* Builds the window partition and every map on the host
 * (src/awa/awa_layers.cpp:53-88, :382-417, :599-636, :867-911, :1046-1060). */
int awa_plan_create(const awa_plan_desc* desc, awa_plan** plan);
void awa_plan_destroy(awa_plan* plan);
int awa_plan_info_get(const awa_plan* plan, awa_plan_info* info);
/* Host copies of the plan's tables, all int32 unless stated:
 * windows: 6 ints (t0,t1,h0,h1,w0,w1) per window, w-outer/h/t-inner order;
 * sequence_index[S]: source row of each packed row (video index, or N + text k);
 * cu_seqlens[nwin+1]; video_positions[N]: packed row of each video token;
 * text_positions[nwin*T_x]; rope_table: float [S][2*rope_dim] = cos | sin rows
 * exactly as the reference's rotation Mat. */
int awa_plan_windows(const awa_plan* plan, int* out);
int awa_plan_sequence_index(const awa_plan* plan, int* out);
int awa_plan_cu_seqlens(const awa_plan* plan, int* out);
int awa_plan_video_positions(const awa_plan* plan, int* out);
int awa_plan_text_positions(const awa_plan* plan, int* out);
int awa_plan_rope_table(const awa_plan* plan, float* out);
/* Copies the plan's device tables to the current device (upload_model). */
int awa_plan_upload(awa_plan* plan, void* stream);
/* No counterpart in the reference. The number of key segments the fused and
 * staged attention of this plan use for `heads` heads in `compute` mode: 1, or
 * S > 1 (AWA_COMPUTE_F32 only) when the layer's (window, head) units are long
 * but too few to fill the device, so that each unit's keys are split over S
 * workgroups and a second kernel combines the segments (in place of the
 * text-mean kernel). Builds the plan's work
 * lists for that head count if they are missing (as awa_plan_upload does with
 * awa_plan_desc.heads); SEEDVR2_AWA_SPLIT=0 in the environment when they are
 * built turns splitting off. For workspace sizing and tests. */
int awa_plan_attention_split(const awa_plan* plan, int heads, int compute, int* split);

/* ---- forward entry points ---- */

/* Heads and head_dim of a QKV blob over `tokens` tokens in one of the four
 * accepted layouts (describe_qkv_layout, src/awa/awa_layers.cpp:116-182);
 * -1 when the blob matches none. Host-only: reads the descriptor, not data. */
int awa_qkv_shape(const awa_blob* qkv, int tokens, int* heads, int* head_dim);

/* Fused layer: gather + MMRoPE + window attention + scatter + text mean in one
 * pass, equivalent to Pack -> MMRoPE -> WindowAttention -> Unpack.
 * video_qkv: the four QKV layouts of describe_qkv_layout (src/awa/awa_layers.cpp:116-170)
 *   over N tokens; text_qkv: the same over T_x tokens; fp32 or bf16.
 * video_out: Mat(d, H, N) (dims 3) or the NCNN_BATCH Mat(d, H, w, h; n = t)
 *   (dims 4); text_out: Mat(d, H, T_x); fp32 or bf16 (bf16 rounds to nearest even).
 * Requires head_dim 128 and rope_dim 126; other shapes use the staged entry points. */
int awa_forward(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_blob* video_out,
                const awa_blob* text_out, int compute, void* stream);

/* awa_forward that allocates no device memory. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The
 * per-window text rows, which awa_forward keeps in a workspace the plan
 * allocates on first use, go to a static device buffer of
 * AWA_NOALLOC_SCRATCH_BYTES per GPU instead. Limits: nwin * T_x * H * d *
 * text_out.elemsize must not exceed the buffer (else AWA_ERR_INVALID), and the
 * plan must already hold the work list for the blobs' head count (built by
 * awa_plan_upload when awa_plan_desc.heads names it, or by an earlier
 * awa_forward with that head count; else AWA_ERR_INVALID). Every call on a
 * GPU uses that GPU's one buffer, which keeps the last call's contents:
 * calls that overlap on one GPU (other streams or threads) race. The buffer
 * is set up by awa_runtime_init for its device (else by the first call on a
 * device), after which a call reserves no device memory. Same blobs, compute
 * modes and results as awa_forward. */
#define AWA_NOALLOC_SCRATCH_BYTES (32u << 20)
int awa_forward_noalloc(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv,
                        const awa_blob* video_out, const awa_blob* text_out, int compute, void* stream);

/* The DiT block's q/k RMSNorm (affine, fp32 arithmetic and output): for every
 * token and head, x * (1 / sqrt(mean(x^2 over head_dim) + eps)) * gamma, with
 * separate gammas for video and text tokens (DitRMSNorm,
 * src/dit/dit_precision.cpp:22-91 and src/dit/shader/dit_rmsnorm.comp;
 * norm_q / norm_k of tools/reference/dit_block.py:258-263, :285-288).
 * Gammas are device pointers to head_dim floats, 16-byte aligned. */
typedef struct awa_qk_norm
{
    const float* q_video;
    const float* k_video;
    const float* q_text;
    const float* k_text;
    float eps; /* 1e-5 in the DiT */
} awa_qk_norm;

/* awa_forward with the DiT block's QKV prologue fused into the gather: the
 * q/k RMSNorm above is applied to the Q and K rows as they are read, before
 * MMRoPE, so video_qkv / text_qkv are the raw QKV projection outputs (fp32 or
 * bf16). Replaces DitRMSNorm x 4 + DitQKVConcat (src/dit/dit_precision.cpp:95-142)
 * + the AWA chain, which round-trip an fp32 [N][3H][d] QKV through memory
 * (src/dit/dit_precision.cpp:314-315). Same blob rules as awa_forward. */
int awa_forward_qknorm(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv,
                       const awa_qk_norm* norm, const awa_blob* video_out, const awa_blob* text_out, int compute,
                       void* stream);

/* DitRMSNorm::forward (src/dit/dit_precision.cpp:63-86, dit_rmsnorm.comp): every
 * row of width w = input.w of a dims-2/3 Mat (fp32 or bf16) normalised over w,
 * times gamma[w] (device, fp32) when gamma is not null; output fp32 of the same
 * shape. The sum of squares follows the shader's order (128 partial sums, then
 * a pairwise tree), so results match the CPU oracle bit for bit. */
int awa_rmsnorm(const awa_blob* input, const float* gamma, float eps, const awa_blob* output, void* stream);

/* DitQKVConcat::forward (src/dit/dit_precision.cpp:95-137, dit_qkv_concat.comp):
 * q, k (fp32) and v (fp32 or bf16), each a dims-3 Mat(d, H, N), into one fp32
 * Mat(d, 3H, N) = [token][q heads, k heads, v heads][d]; v is promoted exactly.
 * The AWA input of a BF16 block (fp32 Q/K from the q/k RMSNorm, bf16 V). */
int awa_qkv_concat(const awa_blob* q, const awa_blob* k, const awa_blob* v, const awa_blob* output, void* stream);

/* SeedVR2AWAPack (src/awa/awa_layers.cpp:419-458, :501-578): packed = Mat(d, 3H, S)
 * fp32, cu_seqlens = Mat(nwin+1) fp32. */
int awa_pack(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_blob* packed,
             const awa_blob* cu_seqlens, void* stream);
/* SeedVR2MMRoPE (:913-953, :985-1025): Mat(d, 3H, S) fp32/bf16 -> fp32. */
int awa_mmrope(const awa_plan* plan, const awa_blob* input, const awa_blob* output, void* stream);
/* SeedVR2WindowAttention (:1062-1120, :1152-1234): Mat(d, 3H, S) -> Mat(d, H, S). */
int awa_window_attention(const awa_plan* plan, const awa_blob* input, const awa_blob* output, int compute,
                         void* stream);
/* SeedVR2AWAUnpack (:638-689, :743-846): Mat(d, H, S) -> video, text as in awa_forward;
 * text = (sum over windows in window order) / nwin. */
int awa_unpack(const awa_plan* plan, const awa_blob* packed, const awa_blob* video_out, const awa_blob* text_out,
               void* stream);
/* Element cast fp32 <-> bf16 honouring cstep/nstep (record_awa_cast, :301-332;
 * the block-9 precision switch convert_precision_gpu, src/dit/dit_stack.cpp:329-357). */
int awa_cast(const awa_blob* input, const awa_blob* output, void* stream);

/* ---- DiT attention stack: the AWA layer of every block with the precision dispatch ---- */

/* Mirrors DitStackSession's block loop (src/dit/dit_stack.cpp:497-565, :931-982):
 * blocks [0, fp32_prefix_blocks) compute in fp32 (fp32 QKV in and out), the
 * rest in bf16; even blocks use unshifted windows, odd blocks shifted
 * (tools/reference/dit_stack.py:75-79); one stream. */
typedef struct awa_stack_desc {
    int source_t, source_h, source_w;    /* session token grid (AwaRuntimeSpec) */
    int windows_t, windows_h, windows_w; /* window counts (params 3/4/5) */
    int text_tokens;
    int blocks;             /* 32 */
    int fp32_prefix_blocks; /* 9 (src/dit/dit_stack.cpp:519) */
    int heads, head_dim;    /* 20, 128 */
} awa_stack_desc;

typedef struct awa_stack awa_stack;

int awa_stack_create(const awa_stack_desc* desc, awa_stack** stack);
void awa_stack_destroy(awa_stack* stack);
/* Per-block device pointers, dense token-major: video_qkv[b] [N][3][H][d],
 * text_qkv[b] [T_x][3][H][d], video_out[b] [N][H][d], text_out[b] [T_x][H][d];
 * fp32 for blocks below fp32_prefix_blocks, bf16 from there on. At the first
 * bf16 block the previous block's outputs are converted to bf16 into the
 * stack's carry buffers, as convert_precision_gpu does at block 9
 * (src/dit/dit_stack.cpp:934-950). */
int awa_stack_run(awa_stack* stack, void* const* video_qkv, void* const* text_qkv, void* const* video_out,
                  void* const* text_out, void* stream);
/* Optional per-block timing (the reference's --profile surface): when enabled
 * each run records events around every block's attention kernel (and runs
 * eagerly). */
int awa_stack_set_profiling(awa_stack* stack, int enabled);
/* Step replay through a HIP graph (default on; no reference counterpart, the
 * reference submits one command buffer per block): the first run with a new
 * set of block pointers runs eagerly and records the step, later runs with
 * the same pointers replay it with one launch. Runs on the null stream are
 * always eager. */
int awa_stack_set_graph(awa_stack* stack, int enabled);
/* After a profiled run has completed: milliseconds of each block's attention
 * kernel and of the block's layer (attention kernel + text mean). */
int awa_stack_block_times(const awa_stack* stack, float* attention_ms, float* block_ms);
/* Algorithmic FLOPs of each block: sum over windows of 4 * L^2 * head_dim * heads. */
int awa_stack_block_flops(const awa_stack* stack, double* flops);

/* ---- DiT block: the layers around the AWA chain ---- */

/* One DiT block as the reference runs it per block (the ncnn graph exported
 * from FixedDitBlock, tools/reference/dit_block.py:302-378, run through
 * Extractor in0/in1/in2 -> out0/out1 by DitStackSession::run,
 * src/dit/dit_stack.cpp:951-963): RMSNorm + Ada "in", the QKV projection, the
 * AWA layer with the q/k RMSNorm fused (awa_forward_qknorm), the output
 * projection + bias, Ada gate + residual, RMSNorm + Ada "in" (mlp), the SwiGLU
 * MLP (tools/reference/dit_block.py:193-207) and Ada gate + residual, for the
 * video and the text branch. A last block (is_last_layer) modulates and runs
 * the MLP on video only and returns 2 * (text after attention + text).
 * precision AWA_COMPUTE_F32: fp32 activations, GEMM weights and GEMMs (the
 * FP32 prefix blocks); AWA_COMPUTE_BF16: bf16 activations and GEMM weights,
 * fp32 accumulation and arithmetic (the BF16 blocks, dit_stack.cpp:519,
 * :550). The GEMMs are library GEMMs (hipBLASLt). A block or stack object is
 * used by one thread at a time (it caches GEMM descriptors on first use). The
 * first GEMM of each shape in the process times hipBLASLt's candidate
 * algorithms on the caller's operands and stream, waiting for the stream once
 * (not under graph capture, where the heuristic's first is taken for that
 * call); its choice then holds for every block and stack object of the
 * process, so equal shapes give equal bits within a process. Timing noise can
 * still pick a different algorithm in another process, and results then differ
 * in the last bits (the fp32 and bf16 tolerances hold either way). With the
 * environment variable SEEDVR2_GEMM_HEURISTIC=1 the heuristic's first
 * algorithm is taken for every shape, without timing: the same choice in every
 * process on the same device and library version. */
typedef struct awa_dit_block_desc {
    int source_t, source_h, source_w;    /* token grid */
    int windows_t, windows_h, windows_w; /* window counts (params 3/4/5) */
    int text_tokens;
    int shifted;
    int heads, head_dim;  /* 20, 128 (head_dim must be 128) */
    int hidden;           /* vid_dim = txt_dim, 2560 */
    int mlp_hidden;       /* SwiGLU hidden width, 6912 for hidden 2560 */
    int last_layer;
    int precision;        /* AWA_COMPUTE_F32 or AWA_COMPUTE_BF16 */
    float norm_eps;       /* 1e-5 */
} awa_dit_block_desc;

/* Device weights of one branch (video or text). GEMM weights are row-major
 * [out][in] (torch Linear layout) in the block's precision; the rest is fp32.
 * ada holds AdaSingle's learned vectors (dit_block.py:166-172) as 6 rows of
 * hidden: attn shift, scale, gate, then mlp shift, scale, gate. The last
 * block's text branch only needs qkv, proj_out, proj_out_bias, norm_q, norm_k. */
typedef struct awa_dit_branch_weights {
    const void* qkv;            /* [3*heads*head_dim][hidden] */
    const void* proj_out;       /* [hidden][heads*head_dim] */
    const float* proj_out_bias; /* [hidden], 16-byte aligned */
    const void* mlp_gate;       /* [mlp_hidden][hidden] (proj_in_gate) */
    const void* mlp_in;         /* [mlp_hidden][hidden] (proj_in); stored right after mlp_gate, the two
                                   run as one GEMM of width 2 * mlp_hidden */
    const void* mlp_out;        /* [hidden][mlp_hidden] (proj_out) */
    const float* norm_q;        /* [head_dim], 16-byte aligned */
    const float* norm_k;        /* [head_dim], 16-byte aligned */
    const float* ada;           /* [6][hidden] */
} awa_dit_branch_weights;

typedef struct awa_dit_block awa_dit_block;

int awa_dit_block_create(const awa_dit_block_desc* desc, awa_dit_block** block);
void awa_dit_block_destroy(awa_dit_block* block);
/* video [N][hidden], text [T_x][hidden] and the block embedding emb
 * [hidden*6] (read as [hidden][2][3]: attn/mlp x shift/scale/gate) are dense
 * device arrays in the block's precision, as are video_out and text_out
 * (which must not alias the inputs). Asynchronous on stream. */
int awa_dit_block_forward(awa_dit_block* block, const awa_dit_branch_weights* video_weights,
                          const awa_dit_branch_weights* text_weights, const void* video, const void* text,
                          const void* emb, void* video_out, void* text_out, void* stream);

/* The block loop of a DiT step: DitStackSession::run (src/dit/dit_stack.cpp:931-982)
 * over full blocks. Blocks [0, fp32_prefix_blocks) run fp32, the rest bf16;
 * at the first bf16 block the carried video and text and the embedding are
 * cast to bf16 once (:934-950). Even blocks use unshifted windows, odd
 * blocks shifted (tools/reference/dit_stack.py:75-79); the last block is the
 * is_last_layer variant (tools/reference/dit_stack.py, dit_block.py:324). */
typedef struct awa_dit_stack_desc {
    int source_t, source_h, source_w;
    int windows_t, windows_h, windows_w;
    int text_tokens;
    int blocks;             /* 32 */
    int fp32_prefix_blocks; /* 9 */
    int heads, head_dim;    /* 20, 128 */
    int hidden, mlp_hidden; /* 2560, 6912 */
    float norm_eps;         /* 1e-5 */
} awa_dit_stack_desc;

typedef struct awa_dit_stack awa_dit_stack;

int awa_dit_stack_create(const awa_dit_stack_desc* desc, awa_dit_stack** stack);
void awa_dit_stack_destroy(awa_dit_stack* stack);
/* video_weights / text_weights: one struct per block, in each block's
 * precision (awa_dit_branch_weights). video [N][hidden], text [T_x][hidden]
 * and emb [hidden*6] are fp32 (the inputs of block 0, which is fp32 unless
 * fp32_prefix_blocks is 0); video_out / text_out take the last block's
 * outputs in its precision. Asynchronous on stream. */
int awa_dit_stack_run(awa_dit_stack* stack, const awa_dit_branch_weights* video_weights,
                      const awa_dit_branch_weights* text_weights, const void* video, const void* text,
                      const void* emb, void* video_out, void* text_out, void* stream);
/* Per-block timing (the reference's --profile surface): when enabled each run
 * records an event before every block and after the last. */
int awa_dit_stack_set_profiling(awa_dit_stack* stack, int enabled);
/* After a profiled run has completed: milliseconds of each block. */
int awa_dit_stack_block_times(const awa_dit_stack* stack, float* block_ms);

#ifdef __cplusplus
}
#endif

#endif /* SEEDVR2_AWA_H */
