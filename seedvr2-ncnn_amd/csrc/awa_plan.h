// Host-side plan of one AWA layer: window partition, index maps and RoPE
// tables, plus the device copies the kernels read.
#pragma once

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "seedvr2_awa.h"

namespace awa
{

// Half-open window box [t0,t1) x [h0,h1) x [w0,w1) (src/awa/awa_layers.h:20-28).
struct Box
{
    int t0, t1, h0, h1, w0, w1;
};

// Per-window record the kernels read: origin, extents, video token count and
// the first packed row (cu_seqlens entry). 32 bytes.
struct alignas(16) WindowDesc
{
    int t0, h0, w0;
    int et, eh, ew;
    int video_tokens;
    int seq_start;
};

// One workgroup's share of the fused / packed attention: the window (its
// descriptor is embedded so that a workgroup needs a single dependent load to
// start), the head, the query rows [row0, row0 + rows) of the window (rows a
// multiple of 32 and at most the variant's rows per workgroup) and the keys
// [key0, key1) of the window it attends to (key0 a multiple of 64): all L
// keys, or, when a layer's units are split over several workgroups, segment
// seg of them. window < 0 marks padding.
struct alignas(16) WorkItem
{
    WindowDesc win;
    int window;
    int head;
    int row0;
    int rows;
    int key0, key1;
    int seg;
    int pad;
};

// Packed-row descriptor for the staged kernels: source row (video index, or
// N + text index) and the three RoPE coordinates.
struct alignas(16) RowInfo
{
    int source;
    int ct, ch, cw;
};

struct DeviceTables
{
    int device = -1;
    WindowDesc* windows = nullptr;
    RowInfo* rows = nullptr;
    int* video_positions = nullptr;
    int* text_positions = nullptr;
    int* cu_seqlens = nullptr;
    float* rope_cs = nullptr; // [coords][pairs][2]
};

} // namespace awa

struct awa_plan
{
    // parameters after runtime-spec resolution
    int source_t = 0, source_h = 0, source_w = 0;
    int windows_t = 0, windows_h = 0, windows_w = 0;
    int text_tokens = 0;
    bool shifted = false;
    int rope_dim = 126;
    int heads_hint = 0; // awa_plan_desc.heads: work list built at upload when positive
    int window_t = 0, window_h = 0, window_w = 0;

    std::vector<awa::Box> windows;
    std::vector<int> sequence_index;  // [S]
    std::vector<int> cu_seqlens;      // [nwin+1]
    std::vector<int> video_positions; // [N]
    std::vector<int> text_positions;  // [nwin*T_x]
    std::vector<awa::RowInfo> rows;   // [S]
    std::vector<awa::WindowDesc> window_descs;
    int source_tokens = 0;
    int sequence_tokens = 0;
    int max_window_tokens = 0;

    // Compact MMRoPE table: the rotation of every packed row only depends on
    // (axis coordinate, pair), and all three axes share one frequency set, so
    // the reference's [S][2*rope_dim] table collapses to [coords][pairs][cos,sin].
    int rope_pairs = 21;
    int rope_coords = 0;
    std::vector<float> rope_cs;

    awa::DeviceTables dev;

    // Lazily built per head count; guarded by mutex.
    mutable std::mutex mutex;
    mutable int work_heads = 0;
    mutable awa::WorkItem* work = nullptr;      // query blocks of kQueryRows rows
    mutable int work_count = 0;
    mutable awa::WorkItem* work_wide = nullptr; // query blocks of kWideQueryRows rows
    mutable int work_wide_count = 0;
    // The same query blocks with their keys split into segments (split_factor
    // > 1; null otherwise), for layers whose units cannot fill the device.
    mutable int split = 1, split_wide = 1;
    mutable awa::WorkItem* work_split = nullptr;
    mutable int work_split_count = 0;
    mutable awa::WorkItem* work_wide_split = nullptr;
    mutable int work_wide_split_count = 0;
    mutable float* text_partials = nullptr;
    mutable size_t text_partials_bytes = 0;
};

namespace awa
{

// Builds every host table; returns AWA_OK or AWA_ERR_INVALID with a message.
int build_plan(const awa_plan_desc& desc, awa_plan& plan, std::string& error);

// Host RoPE row in the reference's [2*rope_dim] format for packed row p.
void rope_row(const awa_plan& plan, int position, float* out);

} // namespace awa
