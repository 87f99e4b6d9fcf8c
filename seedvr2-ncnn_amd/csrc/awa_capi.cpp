// C ABI of the AWA path: runtime (memory, streams, events), plans and the
// forward entry points. Validates every descriptor on the host and turns
// shape errors into the reference's return codes before any kernel runs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "awa_internal.h"
#include "awa_kernels.h"
#include "awa_plan.h"
#include "seedvr2_awa.h"

namespace
{

thread_local std::string g_last_error;

int fail(int code, const std::string& message)
{
    g_last_error = message;
    return code;
}

int fail_hip(hipError_t e, const char* what)
{
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return AWA_ERR_DEVICE;
}

#define HIP_TRY(expr, what)                     \
    do                                          \
    {                                           \
        const hipError_t e_ = (expr);           \
        if (e_ != hipSuccess)                   \
            return fail_hip(e_, what);          \
    } while (0)

hipStream_t as_stream(void* s)
{
    return static_cast<hipStream_t>(s);
}

// Shape trace of the layer blobs when SEEDVR2_TRACE_OPS is set, in the
// reference's line format (trace_awa_type, src/awa/awa_layers.cpp:189-201).
void trace_blob(const char* op, const awa_blob* b)
{
    static const bool enabled = std::getenv("SEEDVR2_TRACE_OPS") != nullptr;
    if (enabled && b)
        std::fprintf(stderr, "awa-trace op=%s dims=%d w=%d h=%d d=%d c=%d elemsize=%d pack=1\n", op, b->dims, b->w,
                     b->h, b->d, b->c, b->elemsize);
}

// ---- descriptor helpers (ncnn Mat semantics, elempack 1) ----

struct QkvLayout
{
    int heads = 0;
    int head_dim = 0;
    long long token_stride = 0;
    long long qkv_stride = 0;
};

// The four QKV layouts accepted by the reference (src/awa/awa_layers.cpp:124-170),
// tried in the reference's order.
bool describe_qkv(const awa_blob& b, int tokens, QkvLayout& out)
{
    if (!b.data || b.w <= 0 || b.h <= 0 || (b.elemsize != 2 && b.elemsize != 4))
        return false;
    out.head_dim = b.w;
    if (b.dims == 3)
    {
        if (b.h % 3 == 0 && b.c == tokens)
        {
            out.heads = b.h / 3;
            out.token_stride = b.cstep;
            out.qkv_stride = static_cast<long long>(out.heads) * out.head_dim;
        }
        else if (b.c == tokens * 3)
        {
            out.heads = b.h;
            out.token_stride = b.cstep;
            out.qkv_stride = static_cast<long long>(tokens) * b.cstep;
        }
        else if (b.c == 3 && b.n == tokens)
        {
            out.heads = b.h;
            out.token_stride = b.nstep;
            out.qkv_stride = b.cstep;
        }
        else
            return false;
    }
    else if (b.dims == 4)
    {
        if (b.d != 3 || b.c != tokens)
            return false;
        out.heads = b.h;
        out.token_stride = b.cstep;
        out.qkv_stride = static_cast<long long>(out.heads) * out.head_dim;
    }
    else
        return false;
    return out.heads > 0;
}

// Video output: Mat(d, H, N) (dims 3) or NCNN_BATCH Mat(d, H, w, h; n = t) (dims 4).
bool describe_video_out(const awa_blob& b, const awa_plan& plan, int heads, int head_dim, awa::VideoSink& out)
{
    if (!b.data || (b.elemsize != 2 && b.elemsize != 4) || b.w != head_dim || b.h != heads)
        return false;
    out.data = b.data;
    out.elemsize = b.elemsize;
    if (b.dims == 3 && b.c == plan.source_tokens && b.cstep >= static_cast<long long>(heads) * head_dim)
    {
        out.ws = b.cstep;
        out.hs = b.cstep * plan.source_w;
        out.ts = b.cstep * plan.source_w * plan.source_h;
        return true;
    }
    if (b.dims == 4 && b.d == plan.source_w && b.c == plan.source_h && b.n == plan.source_t)
    {
        out.ws = static_cast<long long>(heads) * head_dim;
        out.hs = b.cstep;
        out.ts = b.nstep;
        return b.cstep >= out.ws * plan.source_w && (plan.source_t == 1 || b.nstep >= b.cstep * plan.source_h);
    }
    return false;
}

bool is_mat3(const awa_blob& b, int w, int h, int c)
{
    return b.data && b.dims == 3 && b.w == w && b.h == h && b.c == c && b.cstep >= static_cast<long long>(w) * h &&
           (b.elemsize == 2 || b.elemsize == 4);
}

bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int check_plan_uploaded(const awa_plan* plan)
{
    if (!plan)
        return fail(AWA_ERR_INVALID, "null plan");
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess)
        return fail(AWA_ERR_DEVICE, "no HIP device");
    if (plan->dev.device < 0)
        return fail(AWA_ERR_INVALID, "plan has not been uploaded (awa_plan_upload)");
    if (plan->dev.device != device)
        return fail(AWA_ERR_INVALID, "plan was uploaded to another device");
    return AWA_OK;
}

// Work list of the attention kernel for `heads` heads: every (window, head)
// unit is split into query blocks of rows_per_block rows; units are placed on the 8
// XCDs by longest-processing-time first, and each XCD's items are laid out
// at blockIdx = xcd + 8*j, since workgroups are dispatched round-robin over
// the XCDs. All query blocks of one unit therefore share one XCD's L2 for
// their K/V reads.
constexpr int kXcds = 8;

// Attention kernel variant per arithmetic and geometry. AWA_COMPUTE_F32_MFMA
// takes the 8-wave fp32-MFMA pipeline (one workgroup per unit of up to 256
// rows). The bf16 and the exact-score fp32 kernels take their 8-wave form when
// its 256-row query blocks leave no more waves idle than 128-row blocks would
// (each unit's K/V tiles are then staged once instead of once per 128-row
// block), else the 4-wave form with two workgroups per CU.
int attention_variant(int compute, const awa_plan& plan)
{
    if (compute == AWA_COMPUTE_F32_MFMA)
        return awa::kVariantWidePipe;
    long long idle_wide = 0, idle_narrow = 0;
    for (const awa::WindowDesc& w : plan.window_descs)
    {
        const int L = w.video_tokens + plan.text_tokens;
        const int waves = (L + 31) / 32;
        idle_wide += (L + awa::kWideQueryRows - 1) / awa::kWideQueryRows * (awa::kWideQueryRows / 32) - waves;
        idle_narrow += (L + awa::kQueryRows - 1) / awa::kQueryRows * (awa::kQueryRows / 32) - waves;
    }
    return idle_wide <= idle_narrow ? awa::kVariantWide : awa::kVariantNarrow;
}

// The variant to launch: attention_variant's choice, or the 4-wave form
// (single-buffered, two workgroups per CU) when the double-buffered 8-wave
// form's tiles and tables exceed a workgroup's LDS.
// Returns -1 with the reason set when no variant fits the window.
int launch_variant(int compute, const awa_plan& plan, awa::AttentionLaunch& p)
{
    if (plan.max_window_tokens >= awa::kMaxWindowRows)
        return fail(AWA_ERR_INVALID, "window of " + std::to_string(plan.max_window_tokens) +
                                         " rows exceeds the attention kernels' " +
                                         std::to_string(awa::kMaxWindowRows - 1) + "-row limit");
    p.variant = attention_variant(compute, plan);
    auto lds = [&](int variant, const awa::AttentionLaunch& q) {
        if (compute == AWA_COMPUTE_F32)
            return awa::attention_x_static_lds(variant == awa::kVariantWide) +
                   awa::attention_x_dynamic_lds(q, q.qk_norm);
        return awa::attention_static_lds(compute == AWA_COMPUTE_BF16, variant) + awa::attention_dynamic_lds(q);
    };
    // The 8-wave fallback is decided on the fused layer's tables (RoPE table
    // and norm gammas included), so that the staged and fused layers of one
    // plan take the same variant and give the same bits.
    awa::AttentionLaunch fused = p;
    fused.fused = true;
    fused.qk_norm = true;
    fused.rope_coords = plan.rope_coords;
    if (p.variant == awa::kVariantWide && lds(p.variant, fused) > awa::kWorkgroupLds)
        p.variant = awa::kVariantNarrow;
    if (lds(p.variant, p) > awa::kWorkgroupLds)
        return fail(AWA_ERR_INVALID, "window of " + std::to_string(plan.max_window_tokens) +
                                         " rows needs " + std::to_string(lds(p.variant, p)) +
                                         " bytes of LDS per workgroup, more than " +
                                         std::to_string(awa::kWorkgroupLds));
    // Split layers: the key-segment lists, for the exact-score fp32 kernel.
    const bool wide = p.variant != awa::kVariantNarrow;
    const int split = compute != AWA_COMPUTE_F32 ? 1 : (wide ? plan.split_wide : plan.split);
    p.split = split;
    if (split > 1)
    {
        p.work = wide ? plan.work_wide_split : plan.work_split;
        p.work_count = wide ? plan.work_wide_split_count : plan.work_split_count;
    }
    else
    {
        p.work = wide ? plan.work_wide : plan.work;
        p.work_count = wide ? plan.work_wide_count : plan.work_count;
    }
    return AWA_OK;
}

bool valid_compute(int compute)
{
    return compute == AWA_COMPUTE_F32 || compute == AWA_COMPUTE_BF16 || compute == AWA_COMPUTE_F32_MFMA;
}

// The attention kernel for the compute mode.
hipError_t launch_attention_for(int compute, const awa::AttentionLaunch& p, hipStream_t stream)
{
    return compute == AWA_COMPUTE_F32 ? awa::launch_attention_x(p, stream) : awa::launch_attention(p, stream);
}

// Query rows of a (window, head) unit of L rows as work items of at most
// rows_per_block rows (multiples of 32): (first row, rows).
std::vector<std::pair<int, int>> split_rows(int L, int rows_per_block)
{
    std::vector<std::pair<int, int>> items;
    for (int r = 0; r < L; r += rows_per_block)
        items.push_back({r, std::min(rows_per_block, (L - r + 31) / 32 * 32)});
    return items;
}

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus()
{
    static std::mutex m;
    static int cus[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64)
        return 256;
    std::lock_guard<std::mutex> lock(m);
    if (!cus[device])
    {
        hipDeviceProp_t prop{};
        cus[device] = hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0
                          ? prop.multiProcessorCount
                          : 256;
    }
    return cus[device];
}

// Key segments per unit of the exact-score fp32 kernel for query blocks of
// rows_per_block rows: 1 (no split), or, when the layer's work items fill
// fewer than half of the device's concurrent workgroup slots (two 4-wave or
// one 8-wave workgroup per CU) and every unit has at least kMinSplitTiles
// 64-key tiles, the most segments (at most 8) that still fit those slots with
// at least one tile per segment in every unit. The production 256x256 layer
// (20 units of 320 rows) then uses the whole device (41 -> 31 us), and the
// unshifted 2x16x16 clip (80 units of 192 rows) splits in three (37.5 -> 32.8
// us). Units of 128 rows (the 1x16x16 image: 24.5 -> 25.6 us at two
// segments), and the bf16 kernel, whose items are dominated by their start-up
// and whose text mean reads half the bytes of the combining kernel (13.2 ->
// 20.0 us on the bf16 image), lose more to the segment rows and the combining
// kernel than they gain. The environment variable SEEDVR2_AWA_SPLIT=0, read
// when a plan builds its work lists, turns splitting off.
constexpr int kMaxSplit = 8;
constexpr int kMinSplitTiles = 3;
int split_factor(const awa_plan& plan, int heads, int rows_per_block)
{
    const char* env = std::getenv("SEEDVR2_AWA_SPLIT");
    if (env && std::string(env) == "0")
        return 1;
    long long items = 0;
    int min_tiles = 1 << 30;
    for (const awa::WindowDesc& w : plan.window_descs)
    {
        const int L = w.video_tokens + plan.text_tokens;
        items += (L + rows_per_block - 1) / rows_per_block;
        min_tiles = std::min(min_tiles, (L + 63) / 64);
    }
    items *= heads;
    const long long slots = (rows_per_block == awa::kQueryRows ? 2LL : 1LL) * device_cus();
    if (items <= 0 || 2 * items > slots || min_tiles < kMinSplitTiles)
        return 1;
    const long long s = std::min<long long>({kMaxSplit, min_tiles, slots / items});
    return s >= 2 ? static_cast<int>(s) : 1;
}

std::vector<awa::WorkItem> build_work(const awa_plan& plan, int heads, int rows_per_block, int split)
{
    struct Unit
    {
        long long cost;
        int window, head;
        std::vector<std::pair<int, int>> items;
    };
    std::vector<Unit> units;
    for (size_t w = 0; w < plan.window_descs.size(); w++)
    {
        const int L = plan.window_descs[w].video_tokens + plan.text_tokens;
        const auto items = split_rows(L, rows_per_block);
        for (int h = 0; h < heads; h++)
            units.push_back({static_cast<long long>(L) * L, static_cast<int>(w), h, items});
    }
    std::stable_sort(units.begin(), units.end(), [](const Unit& a, const Unit& b) { return a.cost > b.cost; });
    std::vector<std::vector<awa::WorkItem>> lists(kXcds);
    std::vector<long long> load(kXcds, 0);
    for (const Unit& u : units)
    {
        const int x = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
        load[x] += u.cost;
        // Segment s of a unit: its 64-key tiles [s T / split, (s + 1) T / split).
        const int L = plan.window_descs[u.window].video_tokens + plan.text_tokens;
        const int T = (L + 63) / 64;
        for (const auto& it : u.items)
            for (int s = 0; s < split; s++)
                lists[x].push_back({plan.window_descs[u.window], u.window, u.head, it.first, it.second,
                                    64 * (s * T / split), std::min(L, 64 * ((s + 1) * T / split)), s, 0});
    }
    size_t longest = 0;
    for (const auto& l : lists)
        longest = std::max(longest, l.size());
    std::vector<awa::WorkItem> work(longest * kXcds, awa::WorkItem{awa::WindowDesc{}, -1, 0, 0, 0, 0, 0, 0, 0});
    for (int x = 0; x < kXcds; x++)
        for (size_t j = 0; j < lists[x].size(); j++)
            work[j * kXcds + x] = lists[x][j];
    // Drop trailing padding.
    while (!work.empty() && work.back().window < 0)
        work.pop_back();
    return work;
}

// Ensures the plan's work lists for `heads` exist on the device: query
// blocks of 128 and of 256 rows, each also split into key segments when
// split_factor says so. The caller holds plan.mutex, and keeps holding it
// until the kernels that read the lists are enqueued, so that no other call
// replaces them in between.
int ensure_work_locked(const awa_plan& plan, int heads)
{
    if (plan.work_heads == heads && plan.work)
        return AWA_OK;
    for (const bool wide : {false, true})
        for (const bool split : {false, true})
        {
            awa::WorkItem*& dst = wide ? (split ? plan.work_wide_split : plan.work_wide)
                                       : (split ? plan.work_split : plan.work);
            int& count = wide ? (split ? plan.work_wide_split_count : plan.work_wide_count)
                              : (split ? plan.work_split_count : plan.work_count);
            const int rows = wide ? awa::kWideQueryRows : awa::kQueryRows;
            const int factor = split ? split_factor(plan, heads, rows) : 1;
            if (split)
                (wide ? plan.split_wide : plan.split) = factor;
            if (dst)
            {
                (void)hipFree(dst);
                dst = nullptr;
            }
            count = 0;
            if (split && factor == 1)
                continue;
            const std::vector<awa::WorkItem> work = build_work(plan, heads, rows, factor);
            if (hipMalloc(&dst, std::max<size_t>(work.size(), 1) * sizeof(awa::WorkItem)) != hipSuccess)
                return fail(AWA_ERR_ALLOC, "work list allocation failed");
            HIP_TRY(hipMemcpy(dst, work.data(), work.size() * sizeof(awa::WorkItem), hipMemcpyHostToDevice),
                    "work list upload");
            count = static_cast<int>(work.size());
        }
    plan.work_heads = heads;
    return AWA_OK;
}

// Ensures the plan's workspace (text rows of an unsplit layer, or the key
// segments of a split one) holds at least `bytes`. Caller holds plan.mutex.
int ensure_partials_locked(const awa_plan& plan, size_t bytes)
{
    if (bytes <= plan.text_partials_bytes)
        return AWA_OK;
    if (plan.text_partials)
    {
        (void)hipFree(plan.text_partials);
        plan.text_partials = nullptr;
        plan.text_partials_bytes = 0;
    }
    if (hipMalloc(&plan.text_partials, bytes) != hipSuccess)
        return fail(AWA_ERR_ALLOC, "attention workspace allocation failed");
    plan.text_partials_bytes = bytes;
    return AWA_OK;
}

// Bytes of a split layer's segments: per packed row, head and segment the
// unnormalised row (head_dim fp32) and its (maximum, sum), the rows first.
size_t split_o_bytes(const awa_plan& plan, int heads, int split)
{
    return static_cast<size_t>(plan.sequence_tokens) * heads * split * awa::kHeadDim * sizeof(float);
}

size_t split_bytes(const awa_plan& plan, int heads, int split)
{
    return split_o_bytes(plan, heads, split) + static_cast<size_t>(plan.sequence_tokens) * heads * split * 8;
}

template <typename T>
int upload_vector(T*& dst, const std::vector<T>& src, hipStream_t stream)
{
    if (dst)
    {
        (void)hipFree(dst);
        dst = nullptr;
    }
    const size_t bytes = std::max<size_t>(src.size(), 1) * sizeof(T);
    if (hipMalloc(&dst, bytes) != hipSuccess)
        return fail(AWA_ERR_ALLOC, "plan table allocation failed");
    if (!src.empty())
        HIP_TRY(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, stream), "plan upload");
    return AWA_OK;
}

void free_device(awa_plan& plan)
{
    auto release = [](auto*& p) {
        if (p)
            (void)hipFree(p);
        p = nullptr;
    };
    release(plan.dev.windows);
    release(plan.dev.rows);
    release(plan.dev.video_positions);
    release(plan.dev.text_positions);
    release(plan.dev.cu_seqlens);
    release(plan.dev.rope_cs);
    release(plan.work);
    release(plan.work_wide);
    release(plan.work_split);
    release(plan.work_wide_split);
    plan.work_wide_count = 0;
    plan.work_split_count = 0;
    plan.work_wide_split_count = 0;
    plan.split = plan.split_wide = 1;
    release(plan.text_partials);
    plan.text_partials_bytes = 0;
    plan.work_heads = 0;
    plan.work_count = 0;
    plan.dev.device = -1;
}

} // namespace

extern "C" {

const char* awa_last_error(void)
{
    return g_last_error.c_str();
}

int awa_device_count(int* count)
{
    if (!count)
        return fail(AWA_ERR_INVALID, "null count");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    *count = e == hipSuccess ? n : 0;
    return AWA_OK;
}

int awa_runtime_init(int device)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(AWA_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= n)
        return fail(AWA_ERR_INVALID, "device index out of range");
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    // The no-alloc entry point's static scratch array is set up here, once
    // per device, so that its first call reserves nothing.
    return awa::noalloc_setup();
}

int awa_malloc(void** ptr, size_t bytes)
{
    if (!ptr)
        return fail(AWA_ERR_INVALID, "null pointer");
    *ptr = nullptr;
    if (bytes == 0)
        return AWA_OK;
    if (hipMalloc(ptr, bytes) != hipSuccess)
    {
        *ptr = nullptr;
        return fail(AWA_ERR_ALLOC, "device allocation failed");
    }
    return AWA_OK;
}

int awa_free(void* ptr)
{
    if (ptr)
        HIP_TRY(hipFree(ptr), "hipFree");
    return AWA_OK;
}

int awa_host_alloc(void** ptr, size_t bytes)
{
    if (!ptr)
        return fail(AWA_ERR_INVALID, "null pointer");
    *ptr = nullptr;
    if (bytes == 0)
        return AWA_OK;
    if (hipHostMalloc(ptr, bytes, hipHostMallocDefault) != hipSuccess)
    {
        *ptr = nullptr;
        return fail(AWA_ERR_ALLOC, "pinned host allocation failed");
    }
    return AWA_OK;
}

int awa_host_free(void* ptr)
{
    if (ptr)
        HIP_TRY(hipHostFree(ptr), "hipHostFree");
    return AWA_OK;
}

int awa_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream)
{
    if (bytes && (!dst || !src))
        return fail(AWA_ERR_INVALID, "null pointer");
    if (bytes)
        HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "copy to device");
    return AWA_OK;
}

int awa_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream)
{
    if (bytes && (!dst || !src))
        return fail(AWA_ERR_INVALID, "null pointer");
    if (bytes)
        HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "copy to host");
    return AWA_OK;
}

int awa_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream)
{
    if (bytes && (!dst || !src))
        return fail(AWA_ERR_INVALID, "null pointer");
    if (bytes)
        HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "device copy");
    return AWA_OK;
}

int awa_zero(void* dst, size_t bytes, void* stream)
{
    if (bytes && !dst)
        return fail(AWA_ERR_INVALID, "null pointer");
    HIP_TRY(awa::launch_zero(dst, bytes, as_stream(stream)), "zero kernel");
    return AWA_OK;
}

int awa_stream_create(void** stream)
{
    if (!stream)
        return fail(AWA_ERR_INVALID, "null pointer");
    hipStream_t s = nullptr;
    HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return AWA_OK;
}

int awa_stream_destroy(void* stream)
{
    if (stream)
        HIP_TRY(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    return AWA_OK;
}

int awa_stream_synchronize(void* stream)
{
    HIP_TRY(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    return AWA_OK;
}

int awa_event_create(void** event)
{
    if (!event)
        return fail(AWA_ERR_INVALID, "null pointer");
    hipEvent_t e = nullptr;
    HIP_TRY(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return AWA_OK;
}

int awa_event_destroy(void* event)
{
    if (event)
        HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
    return AWA_OK;
}

int awa_event_record(void* event, void* stream)
{
    if (!event)
        return fail(AWA_ERR_INVALID, "null event");
    HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "hipEventRecord");
    return AWA_OK;
}

int awa_event_synchronize(void* event)
{
    if (!event)
        return fail(AWA_ERR_INVALID, "null event");
    HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
    return AWA_OK;
}

int awa_event_elapsed_ms(void* start, void* stop, float* ms)
{
    if (!start || !stop || !ms)
        return fail(AWA_ERR_INVALID, "null argument");
    HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
            "hipEventElapsedTime");
    return AWA_OK;
}

int awa_fill_normal(void* dst, size_t count, int elemsize, unsigned long long seed, void* stream)
{
    return awa_fill_normal_scaled(dst, count, elemsize, seed, 1.f, stream);
}

int awa_fill_normal_scaled(void* dst, size_t count, int elemsize, unsigned long long seed, float stddev,
                           void* stream)
{
    if ((count && !dst) || (elemsize != 2 && elemsize != 4) || !std::isfinite(stddev))
        return fail(AWA_ERR_INVALID, "invalid fill arguments");
    if (count)
        HIP_TRY(awa::launch_fill_normal(dst, count, elemsize, seed, stddev, as_stream(stream)), "fill kernel");
    return AWA_OK;
}

// ---- plans ----

int awa_plan_create(const awa_plan_desc* desc, awa_plan** plan)
{
    if (!desc || !plan)
        return fail(AWA_ERR_INVALID, "null argument");
    *plan = nullptr;
    awa_plan* p = new (std::nothrow) awa_plan();
    if (!p)
        return fail(AWA_ERR_ALLOC, "plan allocation failed");
    std::string error;
    const int rc = awa::build_plan(*desc, *p, error);
    if (rc != AWA_OK)
    {
        delete p;
        return fail(rc, error);
    }
    *plan = p;
    return AWA_OK;
}

void awa_plan_destroy(awa_plan* plan)
{
    if (!plan)
        return;
    if (plan->dev.device >= 0)
    {
        int current = -1;
        (void)hipGetDevice(&current);
        (void)hipSetDevice(plan->dev.device);
        free_device(*plan);
        if (current >= 0)
            (void)hipSetDevice(current);
    }
    delete plan;
}

int awa_plan_info_get(const awa_plan* plan, awa_plan_info* info)
{
    if (!plan || !info)
        return fail(AWA_ERR_INVALID, "null argument");
    info->source_t = plan->source_t;
    info->source_h = plan->source_h;
    info->source_w = plan->source_w;
    info->source_tokens = plan->source_tokens;
    info->text_tokens = plan->text_tokens;
    info->window_count = static_cast<int>(plan->windows.size());
    info->sequence_tokens = plan->sequence_tokens;
    info->window_t = plan->window_t;
    info->window_h = plan->window_h;
    info->window_w = plan->window_w;
    info->max_window_tokens = plan->max_window_tokens;
    info->rope_dim = plan->rope_dim;
    info->shifted = plan->shifted ? 1 : 0;
    return AWA_OK;
}

int awa_plan_windows(const awa_plan* plan, int* out)
{
    if (!plan || !out)
        return fail(AWA_ERR_INVALID, "null argument");
    for (size_t i = 0; i < plan->windows.size(); i++)
    {
        const awa::Box& b = plan->windows[i];
        const int v[6] = {b.t0, b.t1, b.h0, b.h1, b.w0, b.w1};
        std::memcpy(out + 6 * i, v, sizeof(v));
    }
    return AWA_OK;
}

#define COPY_TABLE(fn, field)                                                        \
    int fn(const awa_plan* plan, int* out)                                           \
    {                                                                                \
        if (!plan || !out)                                                           \
            return fail(AWA_ERR_INVALID, "null argument");                           \
        std::memcpy(out, plan->field.data(), plan->field.size() * sizeof(int));      \
        return AWA_OK;                                                               \
    }

COPY_TABLE(awa_plan_sequence_index, sequence_index)
COPY_TABLE(awa_plan_cu_seqlens, cu_seqlens)
COPY_TABLE(awa_plan_video_positions, video_positions)
COPY_TABLE(awa_plan_text_positions, text_positions)

int awa_plan_rope_table(const awa_plan* plan, float* out)
{
    if (!plan || !out)
        return fail(AWA_ERR_INVALID, "null argument");
    for (int p = 0; p < plan->sequence_tokens; p++)
        awa::rope_row(*plan, p, out + static_cast<size_t>(p) * 2 * plan->rope_dim);
    return AWA_OK;
}

static int awa_plan_upload_tables(awa_plan* plan, void* stream)
{
    if (!plan)
        return fail(AWA_ERR_INVALID, "null plan");
    int device = -1;
    HIP_TRY(hipGetDevice(&device), "hipGetDevice");
    std::lock_guard<std::mutex> lock(plan->mutex);
    if (plan->dev.device >= 0 && plan->dev.device != device)
        return fail(AWA_ERR_INVALID, "plan already uploaded to another device");
    hipStream_t s = as_stream(stream);
    int rc;
    if ((rc = upload_vector(plan->dev.windows, plan->window_descs, s)) != AWA_OK ||
        (rc = upload_vector(plan->dev.rows, plan->rows, s)) != AWA_OK ||
        (rc = upload_vector(plan->dev.video_positions, plan->video_positions, s)) != AWA_OK ||
        (rc = upload_vector(plan->dev.text_positions, plan->text_positions, s)) != AWA_OK ||
        (rc = upload_vector(plan->dev.cu_seqlens, plan->cu_seqlens, s)) != AWA_OK ||
        (rc = upload_vector(plan->dev.rope_cs, plan->rope_cs, s)) != AWA_OK)
        return rc;
    HIP_TRY(hipStreamSynchronize(s), "plan upload sync");
    plan->dev.device = device;
    return AWA_OK;
}

} // extern "C"

namespace
{

// The plan's device tables, then its attention work list when the plan
// desc named the head count.
int upload_plan(awa_plan* plan, void* stream)
{
    const int rc = awa_plan_upload_tables(plan, stream);
    if (rc != AWA_OK || plan->heads_hint <= 0)
        return rc;
    std::lock_guard<std::mutex> lock(plan->mutex);
    return ensure_work_locked(*plan, plan->heads_hint);
}

} // namespace

extern "C" {

int awa_plan_upload(awa_plan* plan, void* stream)
{
    return upload_plan(plan, stream);
}

int awa_plan_attention_split(const awa_plan* plan, int heads, int compute, int* split)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!split || heads <= 0 || !valid_compute(compute))
        return fail(AWA_ERR_INVALID, "invalid argument");
    std::lock_guard<std::mutex> lock(plan->mutex);
    if ((rc = ensure_work_locked(*plan, heads)) != AWA_OK)
        return rc;
    awa::AttentionLaunch p{};
    p.fused = true;
    p.bf16_mfma = compute == AWA_COMPUTE_BF16;
    p.rope_coords = plan->rope_coords;
    p.max_window_tokens = plan->max_window_tokens;
    if ((rc = launch_variant(compute, *plan, p)) != AWA_OK)
        return rc;
    *split = p.split;
    return AWA_OK;
}

// ---- forward ----

int awa_forward(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_blob* video_out,
                const awa_blob* text_out, int compute, void* stream)
{
    return awa::forward_fused(plan, video_qkv, text_qkv, nullptr, video_out, text_out, compute, as_stream(stream),
                              nullptr);
}

int awa_forward_qknorm(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv,
                       const awa_qk_norm* norm, const awa_blob* video_out, const awa_blob* text_out, int compute,
                       void* stream)
{
    if (!norm)
        return fail(AWA_ERR_INVALID, "null norm parameters");
    return awa::forward_fused(plan, video_qkv, text_qkv, norm, video_out, text_out, compute, as_stream(stream),
                              nullptr);
}

} // extern "C"

namespace awa
{

void set_error(const std::string& message)
{
    g_last_error = message;
}

int forward_fused(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_qk_norm* norm,
                  const awa_blob* video_out, const awa_blob* text_out, int compute, hipStream_t stream,
                  hipEvent_t after_attention, const Scratch* scratch)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!video_qkv || !text_qkv || !video_out || !text_out)
        return fail(AWA_ERR_INVALID, "null blob");
    if (!valid_compute(compute))
        return fail(AWA_ERR_INVALID, "unknown compute mode");
    trace_blob("forward.video.in", video_qkv);
    trace_blob("forward.text.in", text_qkv);
    trace_blob("forward.video.out", video_out);
    trace_blob("forward.text.out", text_out);
    QkvLayout vl, tl;
    if (!describe_qkv(*video_qkv, plan->source_tokens, vl) || !describe_qkv(*text_qkv, plan->text_tokens, tl) ||
        vl.heads != tl.heads || vl.head_dim != tl.head_dim || video_qkv->elemsize != text_qkv->elemsize)
        return fail(AWA_ERR_INVALID, "invalid QKV input blobs");
    if (vl.head_dim != awa::kHeadDim || plan->rope_dim != awa::kRopeDim)
        return fail(AWA_ERR_INVALID, "fused path needs head_dim 128 and rope_dim 126; use the staged entry points");
    // The kernel appends an identity row after the last coordinate, and its
    // row table packs each row's three coordinates into 8-bit fields (below
    // kMaxRopeCoords = 128).
    if (plan->rope_coords + 1 > awa::kMaxRopeCoords)
        return fail(AWA_ERR_INVALID, "RoPE coordinate range exceeds the fused kernel's table");
    const int elem = video_qkv->elemsize;
    const int align_elems = 16 / elem;
    if (!aligned16(video_qkv->data) || !aligned16(text_qkv->data) || vl.token_stride % align_elems ||
        vl.qkv_stride % align_elems || tl.token_stride % align_elems || tl.qkv_stride % align_elems)
        return fail(AWA_ERR_INVALID, "QKV blobs must be 16-byte aligned with 16-byte aligned strides");
    awa::VideoSink sink{};
    if (!describe_video_out(*video_out, *plan, vl.heads, vl.head_dim, sink))
        return fail(AWA_ERR_INVALID, "invalid video output blob");
    if (!is_mat3(*text_out, vl.head_dim, vl.heads, plan->text_tokens))
        return fail(AWA_ERR_INVALID, "invalid text output blob");
    const int out_align = 16 / video_out->elemsize;
    if (!aligned16(video_out->data) || sink.ts % out_align || sink.hs % out_align || sink.ws % out_align ||
        !aligned16(text_out->data) || text_out->cstep % (16 / text_out->elemsize))
        return fail(AWA_ERR_INVALID, "output blobs must be 16-byte aligned with 16-byte aligned strides");

    if (norm)
    {
        for (const float* g : {norm->q_video, norm->k_video, norm->q_text, norm->k_text})
            if (!g || !aligned16(g))
                return fail(AWA_ERR_INVALID, "norm gammas must be non-null and 16-byte aligned");
        if (!(norm->eps >= 0.f) || !std::isfinite(norm->eps))
            return fail(AWA_ERR_INVALID, "norm eps must be finite and non-negative");
    }

    // Held until both kernels are enqueued: they read the plan's work list
    // and workspace, which a call with another head count replaces.
    std::lock_guard<std::mutex> lock(plan->mutex);
    if (scratch)
    {
        // No allocation: the work list must already be on the device.
        if (plan->work_heads != vl.heads || !plan->work)
            return fail(AWA_ERR_INVALID, "plan has no work list for " + std::to_string(vl.heads) +
                                             " heads: create it with awa_plan_desc.heads set, or run awa_forward once");
    }
    else if ((rc = ensure_work_locked(*plan, vl.heads)) != AWA_OK)
        return rc;

    awa::AttentionLaunch p{};
    p.fused = true;
    p.bf16_mfma = compute == AWA_COMPUTE_BF16;
    p.video = {video_qkv->data, vl.token_stride, vl.qkv_stride, elem};
    p.text = {text_qkv->data, tl.token_stride, tl.qkv_stride, elem};
    p.video_out = sink;
    p.text_partial_elemsize = static_cast<int>(text_out->elemsize);
    if (norm)
    {
        p.qk_norm = true;
        p.norm_gamma[0] = norm->q_video;
        p.norm_gamma[1] = norm->k_video;
        p.norm_gamma[2] = norm->q_text;
        p.norm_gamma[3] = norm->k_text;
        p.norm_eps = norm->eps;
    }
    p.windows = plan->dev.windows;
    p.rope_cs = plan->dev.rope_cs;
    p.rope_coords = plan->rope_coords;
    p.max_window_tokens = plan->max_window_tokens;
    if ((rc = launch_variant(compute, *plan, p)) != AWA_OK)
        return rc;
    // A single window's text rows are the text output itself (the mean of one
    // row is that row): with a dense text output they are written there and
    // the text-mean kernel is skipped.
    const bool text_direct = p.split == 1 && plan->windows.size() == 1 &&
                             text_out->cstep == static_cast<long long>(vl.heads) * vl.head_dim;
    // Workspace: the per-window text rows, or a split layer's key segments;
    // in the caller's scratch buffer (no allocation) or the plan's.
    const size_t need = text_direct ? 0
                        : p.split > 1 ? split_bytes(*plan, vl.heads, p.split)
                                      : plan->windows.size() * static_cast<size_t>(plan->text_tokens) * vl.heads *
                                            vl.head_dim * static_cast<size_t>(text_out->elemsize);
    void* workspace = nullptr;
    if (text_direct)
        workspace = text_out->data;
    else if (scratch)
    {
        if (need > scratch->bytes)
            return fail(AWA_ERR_INVALID, std::string(p.split > 1 ? "key segments" : "text rows") +
                                             " of this layer need " + std::to_string(need) +
                                             " bytes, more than the no-alloc scratch buffer's " +
                                             std::to_string(scratch->bytes));
        workspace = scratch->ptr;
    }
    else
    {
        if ((rc = ensure_partials_locked(*plan, need)) != AWA_OK)
            return rc;
        workspace = plan->text_partials;
    }
    if (p.split > 1)
    {
        p.split_o = static_cast<float*>(workspace);
        p.split_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + split_o_bytes(*plan, vl.heads, p.split));
    }
    else
        p.text_partials = workspace;
    p.heads = vl.heads;
    p.text_tokens = plan->text_tokens;
    p.source_h = plan->source_h;
    p.source_w = plan->source_w;
    p.scale_log2 = (1.f / std::sqrt(static_cast<float>(vl.head_dim))) * 1.4426950408889634f;
    HIP_TRY(launch_attention_for(compute, p, stream), "attention kernel launch");
    if (after_attention)
        HIP_TRY(hipEventRecord(after_attention, stream), "hipEventRecord");
    if (p.split > 1)
    {
        awa::SplitMerge m{};
        m.o = p.split_o;
        m.ml = p.split_ml;
        m.split = p.split;
        m.heads = vl.heads;
        m.fused = true;
        m.video_tokens = plan->source_tokens;
        m.video_positions = plan->dev.video_positions;
        m.source_h = plan->source_h;
        m.source_w = plan->source_w;
        m.video_out = sink;
        m.text_tokens = plan->text_tokens;
        m.window_count = static_cast<int>(plan->windows.size());
        m.windows = plan->dev.windows;
        m.text_out = text_out->data;
        m.text_row = text_out->cstep;
        m.text_elemsize = static_cast<int>(text_out->elemsize);
        m.text_round_bf16 = text_out->elemsize == 2;
        HIP_TRY(awa::launch_split_merge(m, stream), "split merge kernel launch");
        return AWA_OK;
    }
    if (text_direct)
        return AWA_OK;
    HIP_TRY(awa::launch_text_mean(workspace, p.text_partial_elemsize, static_cast<int>(plan->windows.size()),
                                  plan->text_tokens,
                                  vl.heads, vl.head_dim, text_out->data, text_out->cstep, text_out->elemsize, stream),
            "text mean kernel launch");
    return AWA_OK;
}

} // namespace awa

extern "C" {

int awa_qkv_shape(const awa_blob* qkv, int tokens, int* heads, int* head_dim)
{
    if (!qkv || !heads || !head_dim || tokens <= 0)
        return fail(AWA_ERR_INVALID, "null argument");
    QkvLayout l;
    if (!describe_qkv(*qkv, tokens, l))
        return fail(AWA_ERR_INVALID, "blob matches none of the QKV layouts");
    *heads = l.heads;
    *head_dim = l.head_dim;
    return AWA_OK;
}

int awa_pack(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv, const awa_blob* packed,
             const awa_blob* cu_seqlens, void* stream)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!video_qkv || !text_qkv || !packed || !cu_seqlens)
        return fail(AWA_ERR_INVALID, "null blob");
    trace_blob("pack.video.in", video_qkv);
    trace_blob("pack.text.in", text_qkv);
    trace_blob("pack.out", packed);
    QkvLayout vl, tl;
    if (!describe_qkv(*video_qkv, plan->source_tokens, vl) || !describe_qkv(*text_qkv, plan->text_tokens, tl) ||
        vl.heads != tl.heads || vl.head_dim != tl.head_dim)
        return fail(AWA_ERR_INVALID, "invalid QKV input blobs");
    if (!is_mat3(*packed, vl.head_dim, 3 * vl.heads, plan->sequence_tokens) || packed->elemsize != 4)
        return fail(AWA_ERR_INVALID, "packed output must be fp32 Mat(d, 3H, S)");
    const int cu_count = static_cast<int>(plan->cu_seqlens.size());
    if (!cu_seqlens->data || cu_seqlens->dims != 1 || cu_seqlens->w != cu_count || cu_seqlens->elemsize != 4)
        return fail(AWA_ERR_INVALID, "cu_seqlens output must be fp32 Mat(nwin+1)");
    hipStream_t s = as_stream(stream);
    const awa::QkvSource vs{video_qkv->data, vl.token_stride, vl.qkv_stride, video_qkv->elemsize};
    const awa::QkvSource ts{text_qkv->data, tl.token_stride, tl.qkv_stride, text_qkv->elemsize};
    HIP_TRY(awa::launch_pack(plan->dev.rows, plan->sequence_tokens, plan->source_tokens, vs, ts, vl.heads,
                             vl.head_dim, static_cast<float*>(packed->data), packed->cstep, s),
            "pack kernel launch");
    HIP_TRY(awa::launch_cu_seqlens(plan->dev.cu_seqlens, cu_count, static_cast<float*>(cu_seqlens->data), s),
            "cu_seqlens kernel launch");
    return AWA_OK;
}

int awa_mmrope(const awa_plan* plan, const awa_blob* input, const awa_blob* output, void* stream)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!input || !output)
        return fail(AWA_ERR_INVALID, "null blob");
    trace_blob("rope.in", input);
    // src/awa/awa_layers.cpp:997-1004: w >= rope_dim, h % 3 == 0, c == S.
    if (!input->data || input->dims != 3 || input->w < plan->rope_dim || input->h <= 0 || input->h % 3 != 0 ||
        input->c != plan->sequence_tokens || (input->elemsize != 2 && input->elemsize != 4))
        return fail(AWA_ERR_INVALID, "invalid MMRoPE input");
    if (!is_mat3(*output, input->w, input->h, input->c) || output->elemsize != 4)
        return fail(AWA_ERR_INVALID, "MMRoPE output must be fp32 with the input's shape");
    const int heads = input->h / 3;
    HIP_TRY(awa::launch_mmrope(plan->dev.rows, plan->sequence_tokens, input->data, input->cstep, input->elemsize,
                               static_cast<float*>(output->data), output->cstep, heads, input->w, plan->rope_dim,
                               plan->rope_pairs, plan->dev.rope_cs, as_stream(stream)),
            "MMRoPE kernel launch");
    return AWA_OK;
}

int awa_window_attention(const awa_plan* plan, const awa_blob* input, const awa_blob* output, int compute,
                         void* stream)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!input || !output)
        return fail(AWA_ERR_INVALID, "null blob");
    if (!valid_compute(compute))
        return fail(AWA_ERR_INVALID, "unknown compute mode");
    trace_blob("attention.in", input);
    if (!input->data || input->dims != 3 || input->w <= 0 || input->h <= 0 || input->h % 3 != 0 ||
        input->c != plan->sequence_tokens || (input->elemsize != 2 && input->elemsize != 4))
        return fail(AWA_ERR_INVALID, "invalid WindowAttention input");
    const int heads = input->h / 3;
    const int head_dim = input->w;
    if (!is_mat3(*output, head_dim, heads, plan->sequence_tokens) || output->elemsize != 4)
        return fail(AWA_ERR_INVALID, "WindowAttention output must be fp32 Mat(d, H, S)");
    hipStream_t s = as_stream(stream);
    if (head_dim != awa::kHeadDim)
    {
        if (head_dim > 1024)
            return fail(AWA_ERR_INVALID, "head_dim above 1024 is not supported");
        HIP_TRY(awa::launch_attention_generic(input->data, input->cstep, input->elemsize,
                                              static_cast<float*>(output->data), output->cstep, plan->dev.cu_seqlens,
                                              static_cast<int>(plan->windows.size()), heads, head_dim,
                                              plan->sequence_tokens, s),
                "generic attention kernel launch");
        return AWA_OK;
    }
    const int align_elems = 16 / input->elemsize;
    if (!aligned16(input->data) || input->cstep % align_elems || !aligned16(output->data) || output->cstep % 4)
        return fail(AWA_ERR_INVALID, "packed blobs must be 16-byte aligned with 16-byte aligned strides");
    std::lock_guard<std::mutex> lock(plan->mutex); // until the launches read the work list
    if ((rc = ensure_work_locked(*plan, heads)) != AWA_OK)
        return rc;
    awa::AttentionLaunch p{};
    p.fused = false;
    p.bf16_mfma = compute == AWA_COMPUTE_BF16;
    p.packed_in = input->data;
    p.packed_in_row = input->cstep;
    p.packed_in_elemsize = input->elemsize;
    p.packed_out = static_cast<float*>(output->data);
    p.packed_out_row = output->cstep;
    p.windows = plan->dev.windows;
    p.max_window_tokens = plan->max_window_tokens;
    // Same variant choice as the fused layer, so that both give the same bits
    // (the packed layer's tables are smaller, so it fits wherever that does).
    if ((rc = launch_variant(compute, *plan, p)) != AWA_OK)
        return rc;
    p.heads = heads;
    p.text_tokens = plan->text_tokens;
    p.source_h = plan->source_h;
    p.source_w = plan->source_w;
    p.scale_log2 = (1.f / std::sqrt(static_cast<float>(head_dim))) * 1.4426950408889634f;
    if (p.split > 1)
    {
        // Key segments in the plan's workspace, combined into the packed rows.
        if ((rc = ensure_partials_locked(*plan, split_bytes(*plan, heads, p.split))) != AWA_OK)
            return rc;
        p.split_o = plan->text_partials;
        p.split_ml = reinterpret_cast<float2*>(reinterpret_cast<char*>(plan->text_partials) +
                                               split_o_bytes(*plan, heads, p.split));
    }
    HIP_TRY(launch_attention_for(compute, p, s), "attention kernel launch");
    if (p.split > 1)
    {
        awa::SplitMerge m{};
        m.o = p.split_o;
        m.ml = p.split_ml;
        m.split = p.split;
        m.heads = heads;
        m.fused = false;
        m.sequence_tokens = plan->sequence_tokens;
        m.packed_out = p.packed_out;
        m.packed_row = p.packed_out_row;
        HIP_TRY(awa::launch_split_merge(m, s), "split merge kernel launch");
    }
    return AWA_OK;
}

int awa_unpack(const awa_plan* plan, const awa_blob* packed, const awa_blob* video_out, const awa_blob* text_out,
               void* stream)
{
    int rc = check_plan_uploaded(plan);
    if (rc != AWA_OK)
        return rc;
    if (!packed || !video_out || !text_out)
        return fail(AWA_ERR_INVALID, "null blob");
    trace_blob("unpack.in", packed);
    trace_blob("unpack.video.out", video_out);
    trace_blob("unpack.text.out", text_out);
    // src/awa/awa_layers.cpp:755-762
    if (!packed->data || packed->dims != 3 || packed->w <= 0 || packed->h <= 0 ||
        packed->c != plan->sequence_tokens || (packed->elemsize != 2 && packed->elemsize != 4))
        return fail(AWA_ERR_INVALID, "invalid packed input");
    const int heads = packed->h;
    const int head_dim = packed->w;
    awa::VideoSink sink{};
    if (!describe_video_out(*video_out, *plan, heads, head_dim, sink))
        return fail(AWA_ERR_INVALID, "invalid video output blob");
    if (!is_mat3(*text_out, head_dim, heads, plan->text_tokens))
        return fail(AWA_ERR_INVALID, "invalid text output blob");
    hipStream_t s = as_stream(stream);
    HIP_TRY(awa::launch_unpack_video(plan->dev.video_positions, plan->source_t, plan->source_h, plan->source_w,
                                     packed->data, packed->cstep, packed->elemsize, sink, heads, head_dim, s),
            "unpack video kernel launch");
    HIP_TRY(awa::launch_unpack_text(plan->dev.text_positions, static_cast<int>(plan->windows.size()),
                                    plan->text_tokens, packed->data, packed->cstep, packed->elemsize, text_out->data,
                                    text_out->cstep, text_out->elemsize, heads, head_dim, s),
            "unpack text kernel launch");
    return AWA_OK;
}

int awa_rmsnorm(const awa_blob* input, const float* gamma, float eps, const awa_blob* output, void* stream)
{
    // DitRMSNorm::forward (src/dit/dit_precision.cpp:63-86): dims 2 or 3,
    // elempack 1, no batch; the output keeps the shape, fp32 when affine,
    // else the input's type.
    if (!input || !output || !input->data || !output->data)
        return fail(AWA_ERR_INVALID, "null blob");
    if ((input->dims != 2 && input->dims != 3) || input->n != 1 || input->w <= 0 || input->h <= 0 ||
        (input->dims == 3 && input->c <= 0) || (input->elemsize != 2 && input->elemsize != 4))
        return fail(AWA_ERR_INVALID, "rmsnorm input must be a dims-2/3 fp32 or bf16 Mat");
    if (output->dims != input->dims || output->w != input->w || output->h != input->h ||
        (input->dims == 3 && output->c != input->c) || output->n != 1)
        return fail(AWA_ERR_INVALID, "rmsnorm output must have the input's shape");
    if (output->elemsize != (gamma ? 4 : input->elemsize))
        return fail(AWA_ERR_INVALID, "rmsnorm output is fp32 with gamma, else the input's type");
    if (!(eps >= 0.f) || !std::isfinite(eps))
        return fail(AWA_ERR_INVALID, "eps must be finite and non-negative");
    const int channels = input->dims == 3 ? input->c : 1;
    const long long plane = static_cast<long long>(input->w) * input->h;
    const long long in_cstep = input->dims == 3 ? input->cstep : plane;
    const long long out_cstep = output->dims == 3 ? output->cstep : plane;
    if (in_cstep < plane || out_cstep < plane)
        return fail(AWA_ERR_INVALID, "channel step smaller than a channel");
    HIP_TRY(awa::launch_rmsnorm(input->data, input->elemsize, in_cstep, output->data, output->elemsize, out_cstep,
                                input->w, input->h, channels, gamma, eps, as_stream(stream)),
            "rmsnorm kernel launch");
    return AWA_OK;
}

int awa_qkv_concat(const awa_blob* q, const awa_blob* k, const awa_blob* v, const awa_blob* output, void* stream)
{
    // DitQKVConcat::forward (src/dit/dit_precision.cpp:114-137): three dims-3
    // Mats of one shape (w = head_dim, h = heads, c = tokens), q and k fp32, v
    // fp32 or bf16; output Mat(w, 3h, c) fp32.
    if (!q || !k || !v || !output || !q->data || !k->data || !v->data || !output->data)
        return fail(AWA_ERR_INVALID, "null blob");
    for (const awa_blob* b : {q, k, v})
        if (b->dims != 3 || b->n != 1 || b->w != q->w || b->h != q->h || b->c != q->c || b->w <= 0 || b->h <= 0 ||
            b->c <= 0 || b->cstep < static_cast<long long>(b->w) * b->h)
            return fail(AWA_ERR_INVALID, "qkv concat inputs must be dims-3 Mats of one shape");
    if (q->elemsize != 4 || k->elemsize != 4 || (v->elemsize != 2 && v->elemsize != 4))
        return fail(AWA_ERR_INVALID, "qkv concat takes fp32 q and k, fp32 or bf16 v");
    if (output->dims != 3 || output->n != 1 || output->w != q->w || output->h != 3 * q->h || output->c != q->c ||
        output->elemsize != 4 || output->cstep < 3ll * q->w * q->h)
        return fail(AWA_ERR_INVALID, "qkv concat output must be an fp32 Mat(w, 3h, c)");
    HIP_TRY(awa::launch_qkv_concat(static_cast<const float*>(q->data), q->cstep, static_cast<const float*>(k->data),
                                   k->cstep, v->data, v->elemsize, v->cstep, static_cast<float*>(output->data),
                                   output->cstep, q->w, q->h, q->c, as_stream(stream)),
            "qkv concat kernel launch");
    return AWA_OK;
}

int awa_cast(const awa_blob* input, const awa_blob* output, void* stream)
{
    if (!input || !output || !input->data || !output->data)
        return fail(AWA_ERR_INVALID, "null blob");
    if ((input->elemsize != 2 && input->elemsize != 4) || (output->elemsize != 2 && output->elemsize != 4))
        return fail(AWA_ERR_INVALID, "cast supports fp32 and bf16");
    if (input->dims != output->dims || input->w != output->w || input->h != output->h || input->d != output->d ||
        input->c != output->c || input->n != output->n || input->dims < 1 || input->dims > 4 || input->n < 1)
        return fail(AWA_ERR_INVALID, "cast needs blobs of one shape");
    awa::CastShape s{};
    s.w = input->w;
    s.h = input->dims >= 2 ? input->h : 1;
    s.d = input->dims == 4 ? input->d : 1;
    s.c = input->dims >= 3 ? input->c : 1;
    s.n = input->n;
    // Elements of one channel are dense; channels and batches are strided.
    const long long plane = static_cast<long long>(s.w) * s.h * s.d;
    s.in_cstep = input->dims >= 3 ? input->cstep : plane;
    s.out_cstep = output->dims >= 3 ? output->cstep : plane;
    s.in_nstep = input->n > 1 ? input->nstep : s.in_cstep * s.c;
    s.out_nstep = output->n > 1 ? output->nstep : s.out_cstep * s.c;
    HIP_TRY(awa::launch_cast(input->data, input->elemsize, output->data, output->elemsize, s, as_stream(stream)),
            "cast kernel launch");
    return AWA_OK;
}

} // extern "C"
