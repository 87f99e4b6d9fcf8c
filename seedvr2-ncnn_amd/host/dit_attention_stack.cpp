// The DiT attention stack: every block's AWA layer with the reference's
// mixed-precision dispatch (src/dit/dit_stack.cpp:497-565 open, :931-982 run).
//
// Blocks below fp32_prefix_blocks compute in fp32, the rest in bf16; the
// window partition alternates unshifted / shifted by block parity, so the
// stack holds two plans. At the first bf16 block the previous block's outputs
// are converted to bf16 once (the reference's convert_precision_gpu calls).
//
// A step is 32 layers of 2 kernels each on one stream. With graphs enabled
// (the default) the step is captured once per set of block pointers and
// replayed with a single graph launch; the capture only holds kernel nodes.
#include <hip/hip_runtime.h>

#include <new>
#include <vector>

#include "awa_internal.h"
#include "seedvr2_awa.h"

struct awa_stack
{
    awa_stack_desc desc{};
    awa_plan* plans[2] = {nullptr, nullptr}; // [shifted]
    void* video_carry = nullptr;             // bf16 [N][H][d]
    void* text_carry = nullptr;              // bf16 [T_x][H][d]
    bool profiling = false;
    std::vector<hipEvent_t> events; // 3 per block: start, after attention, end
    std::vector<double> flops;
    // Captured step: valid for the block pointers it was recorded with.
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
    std::vector<void*> graph_key;
};

namespace
{

int fail(int code, const char* message)
{
    awa::set_error(message);
    return code;
}

awa_blob dense_mat3(void* data, int w, int h, int c, int elemsize)
{
    awa_blob b{};
    b.data = data;
    b.dims = 3;
    b.w = w;
    b.h = h;
    b.d = 1;
    b.c = c;
    b.n = 1;
    b.elemsize = elemsize;
    b.cstep = static_cast<long long>(w) * h; // dense: w*h*elemsize is a multiple of 16 at these shapes
    b.nstep = b.cstep * c;
    return b;
}

void release(awa_stack* s)
{
    for (awa_plan*& p : s->plans)
    {
        awa_plan_destroy(p);
        p = nullptr;
    }
    if (s->video_carry)
        (void)hipFree(s->video_carry);
    if (s->text_carry)
        (void)hipFree(s->text_carry);
    for (hipEvent_t e : s->events)
        (void)hipEventDestroy(e);
    s->events.clear();
    if (s->graph)
        (void)hipGraphExecDestroy(s->graph);
    s->graph = nullptr;
    s->graph_key.clear();
}

} // namespace

extern "C" {

int awa_stack_create(const awa_stack_desc* desc, awa_stack** stack)
{
    if (!desc || !stack)
        return fail(AWA_ERR_INVALID, "null argument");
    *stack = nullptr;
    if (desc->blocks <= 0 || desc->fp32_prefix_blocks < 0 || desc->fp32_prefix_blocks > desc->blocks ||
        desc->heads <= 0 || desc->head_dim != 128 || (desc->heads * desc->head_dim) % 8 != 0)
        return fail(AWA_ERR_INVALID, "invalid stack description (head_dim must be 128)");
    awa_stack* s = new (std::nothrow) awa_stack();
    if (!s)
        return fail(AWA_ERR_ALLOC, "stack allocation failed");
    s->desc = *desc;
    for (int shifted = 0; shifted < 2; shifted++)
    {
        awa_plan_desc pd{};
        pd.source_t = desc->source_t;
        pd.source_h = desc->source_h;
        pd.source_w = desc->source_w;
        pd.windows_t = desc->windows_t;
        pd.windows_h = desc->windows_h;
        pd.windows_w = desc->windows_w;
        pd.text_tokens = desc->text_tokens;
        pd.shifted = shifted;
        pd.rope_dim = 126;
        pd.heads = desc->heads;
        int rc = awa_plan_create(&pd, &s->plans[shifted]);
        if (rc == AWA_OK)
            rc = awa_plan_upload(s->plans[shifted], nullptr);
        if (rc != AWA_OK)
        {
            release(s);
            delete s;
            return rc;
        }
    }
    awa_plan_info info{};
    awa_plan_info_get(s->plans[0], &info);
    const size_t row = static_cast<size_t>(desc->heads) * desc->head_dim;
    if (hipMalloc(&s->video_carry, static_cast<size_t>(info.source_tokens) * row * 2) != hipSuccess ||
        hipMalloc(&s->text_carry, static_cast<size_t>(info.text_tokens) * row * 2) != hipSuccess)
    {
        release(s);
        delete s;
        return fail(AWA_ERR_ALLOC, "carry buffer allocation failed");
    }
    // Algorithmic FLOPs per block: sum_w 4 L_w^2 d H.
    for (int b = 0; b < desc->blocks; b++)
    {
        awa_plan_info pi{};
        awa_plan_info_get(s->plans[b & 1], &pi);
        std::vector<int> cu(pi.window_count + 1);
        awa_plan_cu_seqlens(s->plans[b & 1], cu.data());
        double f = 0.0;
        for (int w = 0; w < pi.window_count; w++)
        {
            const double L = cu[w + 1] - cu[w];
            f += 4.0 * L * L * desc->head_dim * desc->heads;
        }
        s->flops.push_back(f);
    }
    *stack = s;
    return AWA_OK;
}

void awa_stack_destroy(awa_stack* stack)
{
    if (!stack)
        return;
    release(stack);
    delete stack;
}

int awa_stack_set_profiling(awa_stack* stack, int enabled)
{
    if (!stack)
        return fail(AWA_ERR_INVALID, "null stack");
    if (enabled && stack->events.empty())
    {
        stack->events.resize(3 * stack->desc.blocks, nullptr);
        for (hipEvent_t& e : stack->events)
            if (hipEventCreate(&e) != hipSuccess)
                return fail(AWA_ERR_DEVICE, "hipEventCreate failed");
    }
    stack->profiling = enabled != 0;
    return AWA_OK;
}

namespace
{

// Enqueues one step on s (eager, or into a capture).
int enqueue_step(awa_stack* stack, void* const* video_qkv, void* const* text_qkv, void* const* video_out,
                 void* const* text_out, hipStream_t s)
{
    const awa_stack_desc& d = stack->desc;
    awa_plan_info info{};
    awa_plan_info_get(stack->plans[0], &info);
    const int H = d.heads, D = d.head_dim;
    for (int b = 0; b < d.blocks; b++)
    {
        const bool fp32 = b < d.fp32_prefix_blocks;
        const int elem = fp32 ? 4 : 2;
        hipEvent_t* ev = stack->profiling ? &stack->events[3 * b] : nullptr;
        if (b > 0 && b == d.fp32_prefix_blocks)
        {
            // Precision switch: previous (fp32) outputs -> bf16 carry.
            const awa_blob vin = dense_mat3(video_out[b - 1], D, H, info.source_tokens, 4);
            const awa_blob vout = dense_mat3(stack->video_carry, D, H, info.source_tokens, 2);
            const awa_blob tin = dense_mat3(text_out[b - 1], D, H, info.text_tokens, 4);
            const awa_blob tout = dense_mat3(stack->text_carry, D, H, info.text_tokens, 2);
            int rc = awa_cast(&vin, &vout, s);
            if (rc == AWA_OK)
                rc = awa_cast(&tin, &tout, s);
            if (rc != AWA_OK)
                return rc;
        }
        if (ev && hipEventRecord(ev[0], s) != hipSuccess)
            return fail(AWA_ERR_DEVICE, "hipEventRecord failed");
        const awa_blob vq = dense_mat3(video_qkv[b], D, 3 * H, info.source_tokens, elem);
        const awa_blob tq = dense_mat3(text_qkv[b], D, 3 * H, info.text_tokens, elem);
        const awa_blob vo = dense_mat3(video_out[b], D, H, info.source_tokens, elem);
        const awa_blob to = dense_mat3(text_out[b], D, H, info.text_tokens, elem);
        const int rc = awa::forward_fused(stack->plans[b & 1], &vq, &tq, nullptr, &vo, &to,
                                          fp32 ? AWA_COMPUTE_F32 : AWA_COMPUTE_BF16, s, ev ? ev[1] : nullptr);
        if (rc != AWA_OK)
            return rc;
        if (ev && hipEventRecord(ev[2], s) != hipSuccess)
            return fail(AWA_ERR_DEVICE, "hipEventRecord failed");
    }
    return AWA_OK;
}

} // namespace

int awa_stack_run(awa_stack* stack, void* const* video_qkv, void* const* text_qkv, void* const* video_out,
                  void* const* text_out, void* stream)
{
    if (!stack || !video_qkv || !text_qkv || !video_out || !text_out)
        return fail(AWA_ERR_INVALID, "null argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Eager when profiling (per-block events), on the null stream (which
    // cannot be captured) or with graphs disabled.
    if (stack->profiling || !stack->use_graph || !s)
        return enqueue_step(stack, video_qkv, text_qkv, video_out, text_out, s);
    const int n = stack->desc.blocks;
    std::vector<void*> key;
    key.reserve(4 * static_cast<size_t>(n));
    for (void* const* arr : {video_qkv, text_qkv, video_out, text_out})
        key.insert(key.end(), arr, arr + n);
    if (stack->graph && key == stack->graph_key)
        return hipGraphLaunch(stack->graph, s) == hipSuccess ? AWA_OK : fail(AWA_ERR_DEVICE, "hipGraphLaunch failed");
    // New pointers: run eagerly (which also creates the plans' device
    // workspaces outside any capture), then record the step for next time.
    int rc = enqueue_step(stack, video_qkv, text_qkv, video_out, text_out, s);
    if (rc != AWA_OK)
        return rc;
    if (stack->graph)
    {
        (void)hipGraphExecDestroy(stack->graph);
        stack->graph = nullptr;
        stack->graph_key.clear();
    }
    hipGraph_t g = nullptr;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess)
        return fail(AWA_ERR_DEVICE, "hipStreamBeginCapture failed");
    rc = enqueue_step(stack, video_qkv, text_qkv, video_out, text_out, s);
    const hipError_t end = hipStreamEndCapture(s, &g);
    if (rc != AWA_OK || end != hipSuccess)
    {
        if (g)
            (void)hipGraphDestroy(g);
        return rc != AWA_OK ? rc : fail(AWA_ERR_DEVICE, "hipStreamEndCapture failed");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (inst != hipSuccess)
        return fail(AWA_ERR_DEVICE, "hipGraphInstantiate failed");
    stack->graph = exec;
    stack->graph_key = std::move(key);
    return AWA_OK;
}

int awa_stack_set_graph(awa_stack* stack, int enabled)
{
    if (!stack)
        return fail(AWA_ERR_INVALID, "null stack");
    stack->use_graph = enabled != 0;
    return AWA_OK;
}

int awa_stack_block_times(const awa_stack* stack, float* attention_ms, float* block_ms)
{
    if (!stack || !attention_ms || !block_ms)
        return fail(AWA_ERR_INVALID, "null argument");
    if (stack->events.empty())
        return fail(AWA_ERR_INVALID, "profiling was never enabled");
    for (int b = 0; b < stack->desc.blocks; b++)
    {
        const hipEvent_t* ev = &stack->events[3 * b];
        // ev[0] follows any precision-switch cast, so ev[0]..ev[1] spans the
        // attention kernel alone and ev[0]..ev[2] adds the text mean.
        if (hipEventSynchronize(ev[2]) != hipSuccess ||
            hipEventElapsedTime(&attention_ms[b], ev[0], ev[1]) != hipSuccess ||
            hipEventElapsedTime(&block_ms[b], ev[0], ev[2]) != hipSuccess)
            return fail(AWA_ERR_DEVICE, "event timing failed");
    }
    return AWA_OK;
}

int awa_stack_block_flops(const awa_stack* stack, double* flops)
{
    if (!stack || !flops)
        return fail(AWA_ERR_INVALID, "null argument");
    for (size_t b = 0; b < stack->flops.size(); b++)
        flops[b] = stack->flops[b];
    return AWA_OK;
}

} // extern "C"
