// One DiT block around the AWA layer (tools/reference/dit_block.py:344-378,
// FixedDitBlock.forward; exported to the ncnn graph the reference runs per
// block, src/dit/dit_stack.cpp:951-963):
//
//   x_a   = rmsnorm(x) * (1 + ...) Ada "in" (attn)        rmsnorm_modulate kernel
//   qkv   = x_a W_qkv^T                                    GEMM (hipBLASLt)
//   att   = AWA(q/k RMSNorm(qkv))                          awa_forward_qknorm
//   y     = (att W_out^T + b) * gate_attn + x              GEMM + gate_residual kernel
//   x_m   = rmsnorm(y) Ada "in" (mlp)                      rmsnorm_modulate kernel
//   h     = silu(x_m W_gate^T) * (x_m W_in^T)              2 GEMMs into one buffer + swiglu kernel
//   out   = (h W_mlp^T) * gate_mlp + y                     GEMM + gate_residual kernel
//
// for the video and the text branch; the last block modulates and runs the
// MLP on video only and returns text as 2 * y_text. Precision follows the
// block: fp32 blocks keep fp32 activations, weights and GEMMs; bf16 blocks
// store activations and GEMM weights in bf16 (round to nearest even) and
// accumulate in fp32. Parameter vectors (biases, gammas, Ada) are fp32.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "awa_internal.h"
#include "dit_kernels.h"
#include "seedvr2_awa.h"

// One GEMM shape's hipBLASLt descriptors and its algorithm: the fastest of
// the heuristic's candidates, timed on first use.
struct GemmShape
{
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

struct awa_dit_block
{
    awa_dit_block_desc desc{};
    awa_plan* plan = nullptr;
    hipblasLtHandle_t lt = nullptr;
    void* lt_workspace = nullptr;
    std::map<std::tuple<int, int, int, long long, long long>, GemmShape> shapes;
    int es = 4; // activation / GEMM element size
    int tokens[2] = {0, 0};
    // Workspace per branch: normalised input, QKV, attention output, GEMM
    // output, post-attention residual, MLP hidden pair, SwiGLU output; and
    // the branch's Ada vectors [6][hidden] fp32.
    void* ws[2][7] = {};
    float* ada[2] = {nullptr, nullptr};
};

namespace
{

enum Buf
{
    kNorm = 0,
    kQkv,
    kAtt,
    kGemm,
    kResid,
    kPair,
    kHidden
};

int fail(int code, const std::string& message)
{
    awa::set_error(message);
    return code;
}

int fail_hip(hipError_t e, const char* what)
{
    awa::set_error(std::string(what) + ": " + hipGetErrorString(e));
    return AWA_ERR_DEVICE;
}

#define DIT_HIP(expr, what)                 \
    do                                      \
    {                                       \
        const hipError_t e_ = (expr);       \
        if (e_ != hipSuccess)               \
            return fail_hip(e_, what);      \
    } while (0)

void release(awa_dit_block* b)
{
    for (auto& branch : b->ws)
        for (void*& p : branch)
        {
            if (p)
                (void)hipFree(p);
            p = nullptr;
        }
    for (float*& p : b->ada)
    {
        if (p)
            (void)hipFree(p);
        p = nullptr;
    }
    for (auto& kv : b->shapes)
    {
        GemmShape& g = kv.second;
        for (hipblasLtMatrixLayout_t l : {g.a, g.b, g.c})
            if (l)
                hipblasLtMatrixLayoutDestroy(l);
        if (g.desc)
            hipblasLtMatmulDescDestroy(g.desc);
    }
    b->shapes.clear();
    if (b->lt_workspace)
        (void)hipFree(b->lt_workspace);
    b->lt_workspace = nullptr;
    if (b->lt)
        hipblasLtDestroy(b->lt);
    b->lt = nullptr;
    if (b->plan)
        awa_plan_destroy(b->plan);
    b->plan = nullptr;
}

awa_blob dense3(void* data, int w, int h, int c, int elemsize)
{
    awa_blob m{};
    m.data = data;
    m.dims = 3;
    m.w = w;
    m.h = h;
    m.d = 1;
    m.c = c;
    m.n = 1;
    m.elemsize = elemsize;
    m.cstep = static_cast<long long>(w) * h;
    m.nstep = m.cstep * c;
    return m;
}

constexpr size_t kGemmWorkspace = 64u << 20;
constexpr int kGemmCandidates = 16;
constexpr int kGemmTimedRuns = 3;

// The algorithm chosen for a GEMM shape, shared by every block object of the
// process: (device, element size, M, N, K, ldx, ldy) -> algorithm. The first
// object to meet a shape chooses; every later one, shifted or not, runs the
// same algorithm, so equal shapes give equal bits within a process.
std::mutex g_algo_mutex;
std::map<std::tuple<int, int, int, int, int, long long, long long>, hipblasLtMatmulAlgo_t> g_algos;

// SEEDVR2_GEMM_HEURISTIC=1: take the heuristic's first algorithm instead of
// timing the candidates, so that the choice (and the output bits) do not
// depend on timing noise from one process to the next.
bool heuristic_first()
{
    const char* v = std::getenv("SEEDVR2_GEMM_HEURISTIC");
    return v && v[0] == '1';
}

// Y[M][N] (row stride ldy) = X[M][K] (row stride ldx) W[N][K]^T, fp32
// accumulation. Column-major view: Y^T (N x M, ld ldy) = op(A) B with A = W
// stored K x N (ld K) and transposed, B = X^T (K x M, ld ldx). The
// descriptors are built once per shape and block object; the algorithm once
// per shape and process (g_algos): up to kGemmCandidates of the heuristic's
// algorithms each run once to warm up and kGemmTimedRuns times under HIP
// events on the call's own operands (y is rewritten by the call that
// follows), and the fastest is kept. The heuristic's first is taken instead
// under SEEDVR2_GEMM_HEURISTIC=1 and on a stream under graph capture (not
// stored, so that a later eager call still chooses for the process).
int gemm(awa_dit_block* b, const void* x, long long ldx, const void* w, void* y, long long ldy, int M, int N, int K,
         hipStream_t stream)
{
    if (M <= 0)
        return AWA_OK;
    const auto key = std::make_tuple(M, N, K, ldx, ldy);
    auto it = b->shapes.find(key);
    if (it == b->shapes.end())
    {
        GemmShape g;
        const hipDataType t = b->es == 2 ? HIP_R_16BF : HIP_R_32F;
        const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
        bool ok = hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) ==
                      HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) ==
                      HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&g.a, t, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&g.b, t, K, M, ldx) == HIPBLAS_STATUS_SUCCESS &&
                  hipblasLtMatrixLayoutCreate(&g.c, t, N, M, ldy) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulPreference_t pref = nullptr;
        hipblasLtMatmulHeuristicResult_t results[kGemmCandidates] = {};
        int found = 0;
        if (ok)
        {
            const uint64_t ws = kGemmWorkspace;
            ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                       sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatmulAlgoGetHeuristic(b->lt, g.desc, g.a, g.b, g.c, g.c, pref, kGemmCandidates, results,
                                                 &found) == HIPBLAS_STATUS_SUCCESS &&
                 found > 0 && results[0].workspaceSize <= kGemmWorkspace;
        }
        if (pref)
            hipblasLtMatmulPreferenceDestroy(pref);
        int device = 0;
        (void)hipGetDevice(&device);
        const auto algo_key = std::make_tuple(device, b->es, M, N, K, ldx, ldy);
        bool cached = false;
        if (ok)
        {
            std::lock_guard<std::mutex> lock(g_algo_mutex);
            const auto hit = g_algos.find(algo_key);
            if (hit != g_algos.end())
            {
                g.algo = hit->second;
                cached = true;
            }
        }
        if (ok && !cached)
        {
            g.algo = results[0].algo;
            hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
            (void)hipStreamIsCapturing(stream, &capture);
            const bool timed = found > 1 && !heuristic_first() && capture == hipStreamCaptureStatusNone;
            if (timed)
            {
                hipEvent_t start = nullptr, stop = nullptr;
                DIT_HIP(hipEventCreate(&start), "hipEventCreate");
                if (hipEventCreate(&stop) != hipSuccess)
                {
                    (void)hipEventDestroy(start);
                    return fail(AWA_ERR_DEVICE, "hipEventCreate failed");
                }
                const float one = 1.f, zero = 0.f;
                float best = -1.f;
                for (int i = 0; i < found; i++)
                {
                    if (results[i].workspaceSize > kGemmWorkspace)
                        continue;
                    auto run = [&]() {
                        return hipblasLtMatmul(b->lt, g.desc, &one, w, g.a, x, g.b, &zero, y, g.c, y, g.c,
                                               &results[i].algo, b->lt_workspace, kGemmWorkspace, stream);
                    };
                    if (run() != HIPBLAS_STATUS_SUCCESS)
                        continue;
                    bool ran = hipEventRecord(start, stream) == hipSuccess;
                    for (int r = 0; r < kGemmTimedRuns && ran; r++)
                        ran = run() == HIPBLAS_STATUS_SUCCESS;
                    float ms = 0.f;
                    if (!ran || hipEventRecord(stop, stream) != hipSuccess || hipEventSynchronize(stop) != hipSuccess ||
                        hipEventElapsedTime(&ms, start, stop) != hipSuccess)
                        continue;
                    if (best < 0.f || ms < best)
                    {
                        best = ms;
                        g.algo = results[i].algo;
                    }
                }
                (void)hipEventDestroy(start);
                (void)hipEventDestroy(stop);
                (void)hipGetLastError();
            }
            if (timed || heuristic_first())
            {
                // The first choice for a shape stands for the process.
                std::lock_guard<std::mutex> lock(g_algo_mutex);
                g.algo = g_algos.emplace(algo_key, g.algo).first->second;
            }
        }
        if (!ok)
        {
            for (hipblasLtMatrixLayout_t l : {g.a, g.b, g.c})
                if (l)
                    hipblasLtMatrixLayoutDestroy(l);
            if (g.desc)
                hipblasLtMatmulDescDestroy(g.desc);
            return fail(AWA_ERR_DEVICE, "hipBLASLt has no algorithm for a GEMM of the block");
        }
        it = b->shapes.emplace(key, g).first;
    }
    const float alpha = 1.f, beta = 0.f;
    const GemmShape& g = it->second;
    const hipblasStatus_t st = hipblasLtMatmul(b->lt, g.desc, &alpha, w, g.a, x, g.b, &beta, y, g.c, y, g.c, &g.algo,
                                               b->lt_workspace, kGemmWorkspace, stream);
    if (st != HIPBLAS_STATUS_SUCCESS)
        return fail(AWA_ERR_DEVICE, "hipblasLtMatmul failed");
    return AWA_OK;
}

bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

bool branch_weights_valid(const awa_dit_branch_weights* w, bool full)
{
    if (!w || !w->qkv || !w->proj_out || !w->proj_out_bias || !w->norm_q || !w->norm_k)
        return false;
    if (!aligned16(w->proj_out_bias) || !aligned16(w->norm_q) || !aligned16(w->norm_k))
        return false;
    if (full && (!w->mlp_gate || !w->mlp_in || !w->mlp_out || !w->ada))
        return false;
    return true;
}

} // namespace

extern "C" {

int awa_dit_block_create(const awa_dit_block_desc* desc, awa_dit_block** out)
{
    if (!desc || !out)
        return fail(AWA_ERR_INVALID, "null argument");
    *out = nullptr;
    if (desc->heads <= 0 || desc->head_dim != 128 || desc->hidden <= 0 || desc->mlp_hidden <= 0 ||
        (desc->precision != AWA_COMPUTE_F32 && desc->precision != AWA_COMPUTE_BF16) || !(desc->norm_eps >= 0.f) ||
        desc->hidden % 8 || desc->mlp_hidden % 8 || desc->hidden > 8192)
        return fail(AWA_ERR_INVALID,
                    "invalid DiT block description (head_dim must be 128, widths multiples of 8, hidden <= 8192)");
    awa_dit_block* b = new (std::nothrow) awa_dit_block;
    if (!b)
        return fail(AWA_ERR_ALLOC, "block allocation failed");
    b->desc = *desc;
    b->es = desc->precision == AWA_COMPUTE_BF16 ? 2 : 4;
    awa_plan_desc pd{};
    pd.source_t = desc->source_t;
    pd.source_h = desc->source_h;
    pd.source_w = desc->source_w;
    pd.windows_t = desc->windows_t;
    pd.windows_h = desc->windows_h;
    pd.windows_w = desc->windows_w;
    pd.text_tokens = desc->text_tokens;
    pd.shifted = desc->shifted;
    pd.rope_dim = 126;
    pd.heads = desc->heads;
    int rc = awa_plan_create(&pd, &b->plan);
    if (rc != AWA_OK || (rc = awa_plan_upload(b->plan, nullptr)) != AWA_OK)
    {
        release(b);
        delete b;
        return rc;
    }
    if (hipblasLtCreate(&b->lt) != HIPBLAS_STATUS_SUCCESS || hipMalloc(&b->lt_workspace, kGemmWorkspace) != hipSuccess)
    {
        release(b);
        delete b;
        return fail(AWA_ERR_DEVICE, "hipBLASLt handle or workspace creation failed");
    }
    b->tokens[0] = desc->source_t * desc->source_h * desc->source_w;
    b->tokens[1] = desc->text_tokens;
    const long long hd = static_cast<long long>(desc->heads) * desc->head_dim;
    for (int br = 0; br < 2; br++)
    {
        const long long M = b->tokens[br];
        const long long widths[7] = {desc->hidden, 3 * hd, hd, desc->hidden, desc->hidden, 2LL * desc->mlp_hidden,
                                     desc->mlp_hidden};
        bool ok = hipMalloc(&b->ada[br], static_cast<size_t>(6) * desc->hidden * sizeof(float)) == hipSuccess;
        for (int k = 0; k < 7 && ok; k++)
            ok = hipMalloc(&b->ws[br][k], static_cast<size_t>(M * widths[k] * b->es)) == hipSuccess;
        if (!ok)
        {
            release(b);
            delete b;
            return fail(AWA_ERR_ALLOC, "DiT block workspace allocation failed");
        }
    }
    *out = b;
    return AWA_OK;
}

void awa_dit_block_destroy(awa_dit_block* b)
{
    if (!b)
        return;
    release(b);
    delete b;
}

int awa_dit_block_forward(awa_dit_block* b, const awa_dit_branch_weights* video_w,
                          const awa_dit_branch_weights* text_w, const void* video, const void* text, const void* emb,
                          void* video_out, void* text_out, void* stream_ptr)
{
    if (!b || !video || !text || !emb || !video_out || !text_out)
        return fail(AWA_ERR_INVALID, "null argument");
    const awa_dit_block_desc& d = b->desc;
    const bool last = d.last_layer != 0;
    if (!branch_weights_valid(video_w, true) || !branch_weights_valid(text_w, !last))
        return fail(AWA_ERR_INVALID, "missing DiT block weights (or bias / gammas not 16-byte aligned)");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const int es = b->es;
    const int hidden = d.hidden;
    const int hd = d.heads * d.head_dim;
    const int mh = d.mlp_hidden;
    const awa_dit_branch_weights* W[2] = {video_w, text_w};
    const void* in[2] = {video, text};
    void* out[2] = {video_out, text_out};
    int rc;

    // Attention half: Ada vectors, norm + Ada in, QKV projection.
    for (int br = 0; br < 2; br++)
    {
        const int M = b->tokens[br];
        const bool modulate = br == 0 || !last;
        if (modulate)
            DIT_HIP(awa::launch_ada_prepare(emb, es, W[br]->ada, b->ada[br], hidden, stream), "ada_prepare launch");
        awa::RowNormModulate nm{};
        nm.in = in[br];
        nm.in_elemsize = es;
        nm.in_stride = hidden;
        nm.out = b->ws[br][kNorm];
        nm.out_elemsize = es;
        nm.out_stride = hidden;
        nm.rows = M;
        nm.width = hidden;
        nm.eps = d.norm_eps;
        nm.shift = modulate ? b->ada[br] + 0 * hidden : nullptr;
        nm.scale = modulate ? b->ada[br] + 1 * hidden : nullptr;
        DIT_HIP(awa::launch_rmsnorm_modulate(nm, stream), "rmsnorm_modulate launch");
        if ((rc = gemm(b, b->ws[br][kNorm], hidden, W[br]->qkv, b->ws[br][kQkv], 3LL * hd, M, 3 * hd, hidden,
                       stream)) != AWA_OK)
            return rc;
    }
    // AWA with the q/k RMSNorm fused into its gather.
    {
        const awa_blob vq = dense3(b->ws[0][kQkv], d.head_dim, 3 * d.heads, b->tokens[0], es);
        const awa_blob tq = dense3(b->ws[1][kQkv], d.head_dim, 3 * d.heads, b->tokens[1], es);
        const awa_blob vo = dense3(b->ws[0][kAtt], d.head_dim, d.heads, b->tokens[0], es);
        const awa_blob to = dense3(b->ws[1][kAtt], d.head_dim, d.heads, b->tokens[1], es);
        awa_qk_norm norm{video_w->norm_q, video_w->norm_k, text_w->norm_q, text_w->norm_k, d.norm_eps};
        if ((rc = awa::forward_fused(b->plan, &vq, &tq, &norm, &vo, &to, d.precision, stream, nullptr)) != AWA_OK)
            return rc;
    }
    for (int br = 0; br < 2; br++)
    {
        const int M = b->tokens[br];
        const bool full = br == 0 || !last;
        // Output projection, then bias, Ada gate (attn) and the residual.
        if ((rc = gemm(b, b->ws[br][kAtt], hd, W[br]->proj_out, b->ws[br][kGemm], hidden, M, hidden, hd, stream)) !=
            AWA_OK)
            return rc;
        awa::GateResidual gr{};
        gr.h = b->ws[br][kGemm];
        gr.h_elemsize = es;
        gr.h_stride = hidden;
        gr.bias = W[br]->proj_out_bias;
        gr.residual = in[br];
        gr.residual_elemsize = es;
        gr.residual_stride = hidden;
        gr.out = full ? b->ws[br][kResid] : out[br];
        gr.out_elemsize = es;
        gr.out_stride = hidden;
        gr.rows = M;
        gr.width = hidden;
        gr.gate = full ? b->ada[br] + 2 * hidden : nullptr;
        DIT_HIP(awa::launch_gate_residual(gr, stream), "gate_residual launch");
        if (!full)
        {
            // Last block, text: out = 2 * (attention output + text).
            DIT_HIP(awa::launch_double(out[br], es, hidden, out[br], es, hidden, M, hidden, stream), "double launch");
            continue;
        }
        // MLP half: norm + Ada in (mlp), SwiGLU, output projection, gate + residual.
        awa::RowNormModulate nm{};
        nm.in = b->ws[br][kResid];
        nm.in_elemsize = es;
        nm.in_stride = hidden;
        nm.out = b->ws[br][kNorm];
        nm.out_elemsize = es;
        nm.out_stride = hidden;
        nm.rows = M;
        nm.width = hidden;
        nm.eps = d.norm_eps;
        nm.shift = b->ada[br] + 3 * hidden;
        nm.scale = b->ada[br] + 4 * hidden;
        DIT_HIP(awa::launch_rmsnorm_modulate(nm, stream), "rmsnorm_modulate launch");
        char* pair = static_cast<char*>(b->ws[br][kPair]);
        // The two input projections fill the halves of one [M][2 mh] buffer.
        // Weights stored back to back ([mh][hidden] gate, then in) are one
        // [2 mh][hidden] matrix: one GEMM of twice the width.
        const bool adjacent = static_cast<const char*>(W[br]->mlp_in) ==
                              static_cast<const char*>(W[br]->mlp_gate) + static_cast<size_t>(mh) * hidden * es;
        if (adjacent)
        {
            if ((rc = gemm(b, b->ws[br][kNorm], hidden, W[br]->mlp_gate, pair, 2LL * mh, M, 2 * mh, hidden,
                           stream)) != AWA_OK)
                return rc;
        }
        else if ((rc = gemm(b, b->ws[br][kNorm], hidden, W[br]->mlp_gate, pair, 2LL * mh, M, mh, hidden, stream)) !=
                     AWA_OK ||
                 (rc = gemm(b, b->ws[br][kNorm], hidden, W[br]->mlp_in, pair + static_cast<size_t>(mh) * es, 2LL * mh,
                            M, mh, hidden, stream)) != AWA_OK)
            return rc;
        awa::SwiGlu sg{};
        sg.in = pair;
        sg.in_elemsize = es;
        sg.in_stride = 2LL * mh;
        sg.out = b->ws[br][kHidden];
        sg.out_elemsize = es;
        sg.out_stride = mh;
        sg.rows = M;
        sg.width = mh;
        DIT_HIP(awa::launch_swiglu(sg, stream), "swiglu launch");
        if ((rc = gemm(b, b->ws[br][kHidden], mh, W[br]->mlp_out, b->ws[br][kGemm], hidden, M, hidden, mh,
                       stream)) != AWA_OK)
            return rc;
        awa::GateResidual go{};
        go.h = b->ws[br][kGemm];
        go.h_elemsize = es;
        go.h_stride = hidden;
        go.bias = nullptr;
        go.residual = b->ws[br][kResid];
        go.residual_elemsize = es;
        go.residual_stride = hidden;
        go.out = out[br];
        go.out_elemsize = es;
        go.out_stride = hidden;
        go.rows = M;
        go.width = hidden;
        go.gate = b->ada[br] + 5 * hidden;
        DIT_HIP(awa::launch_gate_residual(go, stream), "gate_residual launch");
    }
    return AWA_OK;
}

} // extern "C"

// ---- The block loop: DitStackSession::run (src/dit/dit_stack.cpp:931-982) ----
//
// Blocks [0, fp32_prefix_blocks) run fp32, the rest bf16; at the first bf16
// block the carried video, text and the embedding are cast to bf16 once
// (convert_precision_gpu, :934-950). Even blocks use unshifted windows, odd
// blocks shifted (tools/reference/dit_stack.py:75-79); the last block is the
// is_last_layer variant. Activations ping-pong between two buffers per
// precision; one block object (plan, GEMM handle, workspace) serves every
// block of its (precision, shift) and the last block has its own.
struct awa_dit_stack
{
    awa_dit_stack_desc desc{};
    awa_dit_block* blocks[2][2] = {}; // [bf16][shifted]
    awa_dit_block* last = nullptr;
    void* act[2][2][2] = {};          // [bf16][ping][video, text]
    void* emb_bf16 = nullptr;
    int tokens[2] = {0, 0};
    bool profiling = false;
    std::vector<hipEvent_t> events; // blocks + 1
};

namespace
{

void release_stack(awa_dit_stack* s)
{
    for (auto& p : s->blocks)
        for (awa_dit_block*& b : p)
        {
            awa_dit_block_destroy(b);
            b = nullptr;
        }
    awa_dit_block_destroy(s->last);
    s->last = nullptr;
    for (auto& prec : s->act)
        for (auto& ping : prec)
            for (void*& p : ping)
            {
                if (p)
                    (void)hipFree(p);
                p = nullptr;
            }
    if (s->emb_bf16)
        (void)hipFree(s->emb_bf16);
    s->emb_bf16 = nullptr;
    for (hipEvent_t e : s->events)
        (void)hipEventDestroy(e);
    s->events.clear();
}

int cast_rows(const void* in, int in_es, void* out, int out_es, int rows, int width, hipStream_t stream)
{
    awa_blob a = dense3(const_cast<void*>(in), width, rows, 1, in_es);
    awa_blob b = dense3(out, width, rows, 1, out_es);
    a.dims = b.dims = 2;
    return awa_cast(&a, &b, stream);
}

} // namespace

extern "C" {

int awa_dit_stack_create(const awa_dit_stack_desc* desc, awa_dit_stack** out)
{
    if (!desc || !out)
        return fail(AWA_ERR_INVALID, "null argument");
    *out = nullptr;
    if (desc->blocks <= 0 || desc->fp32_prefix_blocks < 0 || desc->fp32_prefix_blocks > desc->blocks)
        return fail(AWA_ERR_INVALID, "invalid block counts");
    awa_dit_stack* s = new (std::nothrow) awa_dit_stack;
    if (!s)
        return fail(AWA_ERR_ALLOC, "stack allocation failed");
    s->desc = *desc;
    s->tokens[0] = desc->source_t * desc->source_h * desc->source_w;
    s->tokens[1] = desc->text_tokens;
    auto block_desc = [&](bool bf16, bool shifted, bool last) {
        awa_dit_block_desc b{};
        b.source_t = desc->source_t;
        b.source_h = desc->source_h;
        b.source_w = desc->source_w;
        b.windows_t = desc->windows_t;
        b.windows_h = desc->windows_h;
        b.windows_w = desc->windows_w;
        b.text_tokens = desc->text_tokens;
        b.shifted = shifted;
        b.heads = desc->heads;
        b.head_dim = desc->head_dim;
        b.hidden = desc->hidden;
        b.mlp_hidden = desc->mlp_hidden;
        b.last_layer = last;
        b.precision = bf16 ? AWA_COMPUTE_BF16 : AWA_COMPUTE_F32;
        b.norm_eps = desc->norm_eps;
        return b;
    };
    int rc = AWA_OK;
    for (int bf = 0; bf < 2 && rc == AWA_OK; bf++)
    {
        // Only the precisions the loop uses.
        const bool used = bf ? desc->fp32_prefix_blocks < desc->blocks - 1 : desc->fp32_prefix_blocks > 0;
        for (int sh = 0; sh < 2 && rc == AWA_OK && used; sh++)
        {
            const awa_dit_block_desc bd = block_desc(bf, sh, false);
            rc = awa_dit_block_create(&bd, &s->blocks[bf][sh]);
        }
    }
    const int lb = desc->blocks - 1;
    if (rc == AWA_OK)
    {
        const awa_dit_block_desc bd = block_desc(lb >= desc->fp32_prefix_blocks, lb % 2, true);
        rc = awa_dit_block_create(&bd, &s->last);
    }
    for (int bf = 0; bf < 2 && rc == AWA_OK; bf++)
        for (int ping = 0; ping < 2 && rc == AWA_OK; ping++)
            for (int br = 0; br < 2; br++)
                if (hipMalloc(&s->act[bf][ping][br],
                              static_cast<size_t>(s->tokens[br]) * desc->hidden * (bf ? 2 : 4)) != hipSuccess)
                {
                    rc = fail(AWA_ERR_ALLOC, "stack activation allocation failed");
                    break;
                }
    if (rc == AWA_OK && hipMalloc(&s->emb_bf16, static_cast<size_t>(desc->hidden) * 6 * 2) != hipSuccess)
        rc = fail(AWA_ERR_ALLOC, "stack embedding allocation failed");
    if (rc != AWA_OK)
    {
        release_stack(s);
        delete s;
        return rc;
    }
    *out = s;
    return AWA_OK;
}

void awa_dit_stack_destroy(awa_dit_stack* s)
{
    if (!s)
        return;
    release_stack(s);
    delete s;
}

int awa_dit_stack_set_profiling(awa_dit_stack* s, int enabled)
{
    if (!s)
        return fail(AWA_ERR_INVALID, "null stack");
    s->profiling = enabled != 0;
    if (s->profiling && s->events.empty())
    {
        s->events.resize(s->desc.blocks + 1, nullptr);
        for (hipEvent_t& e : s->events)
            DIT_HIP(hipEventCreate(&e), "hipEventCreate");
    }
    return AWA_OK;
}

int awa_dit_stack_run(awa_dit_stack* s, const awa_dit_branch_weights* video_weights,
                      const awa_dit_branch_weights* text_weights, const void* video, const void* text,
                      const void* emb, void* video_out, void* text_out, void* stream_ptr)
{
    if (!s || !video_weights || !text_weights || !video || !text || !emb || !video_out || !text_out)
        return fail(AWA_ERR_INVALID, "null argument");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const awa_dit_stack_desc& d = s->desc;
    const void* cur[2] = {video, text};
    const void* cur_emb = emb;
    int ping = 0;
    int rc;
    for (int b = 0; b < d.blocks; b++)
    {
        const bool bf16 = b >= d.fp32_prefix_blocks;
        if (bf16 && b == d.fp32_prefix_blocks)
        {
            // Precision switch: carried activations and the embedding to bf16.
            for (int br = 0; br < 2; br++)
            {
                void* dst = s->act[1][ping][br];
                if ((rc = cast_rows(cur[br], 4, dst, 2, s->tokens[br], d.hidden, stream)) != AWA_OK)
                    return rc;
                cur[br] = dst;
            }
            if ((rc = cast_rows(emb, 4, s->emb_bf16, 2, 1, d.hidden * 6, stream)) != AWA_OK)
                return rc;
            cur_emb = s->emb_bf16;
            ping ^= 1;
        }
        if (s->profiling)
            DIT_HIP(hipEventRecord(s->events[b], stream), "hipEventRecord");
        const bool last = b == d.blocks - 1;
        awa_dit_block* blk = last ? s->last : s->blocks[bf16][b % 2];
        void* nv = last ? video_out : s->act[bf16][ping][0];
        void* nt = last ? text_out : s->act[bf16][ping][1];
        if ((rc = awa_dit_block_forward(blk, &video_weights[b], &text_weights[b], cur[0], cur[1], cur_emb, nv, nt,
                                        stream)) != AWA_OK)
            return rc;
        cur[0] = nv;
        cur[1] = nt;
        ping ^= 1;
    }
    if (s->profiling)
        DIT_HIP(hipEventRecord(s->events[d.blocks], stream), "hipEventRecord");
    return AWA_OK;
}

int awa_dit_stack_block_times(const awa_dit_stack* s, float* block_ms)
{
    if (!s || !block_ms || !s->profiling)
        return fail(AWA_ERR_INVALID, "profiling is not enabled");
    for (int b = 0; b < s->desc.blocks; b++)
        DIT_HIP(hipEventElapsedTime(&block_ms[b], s->events[b], s->events[b + 1]), "hipEventElapsedTime");
    return AWA_OK;
}

} // extern "C"
