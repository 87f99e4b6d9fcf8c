// Window partition, index maps and RoPE tables of one AWA layer.
//
// Semantics follow the reference's load_param of the four layers
// (src/awa/awa_layers.cpp:53-88 windows, :90-114 params, :382-417 pack maps,
// :599-636 unpack maps, :867-911 RoPE table, :1046-1060 window offsets). The
// partition is built per axis: a window is kept exactly when its t, h and w
// intervals are all non-empty, so the reference's triple loop equals the
// Cartesian product of the non-empty per-axis intervals, taken w-outer,
// h, t-inner.
#include "awa_plan.h"

#include <algorithm>
#include <cfenv>
#include <climits>
#include <cmath>

namespace awa
{
namespace
{

struct Interval
{
    int begin, end;
};

// Non-empty intervals of one axis of length `size` cut into windows of
// `window` cells, shifted by half a window when requested and the window is
// smaller than the axis.
std::vector<Interval> axis_intervals(int size, int window, bool shifted)
{
    const double shift = (shifted && window < size) ? 0.5 : 0.0;
    const int count = static_cast<int>(std::ceil((size - shift) / window)) + (shift > 0.0 ? 1 : 0);
    std::vector<Interval> out;
    for (int i = 0; i < count; i++)
    {
        // Truncation toward zero of the shifted bounds, then clipping.
        const int begin = std::max(static_cast<int>((i - shift) * window), 0);
        const int end = std::min(static_cast<int>((i - shift + 1.0) * window), size);
        if (end > begin)
            out.push_back({begin, end});
    }
    return out;
}

// Python round() of a positive value: nearest integer, ties to even. The
// default floating-point environment rounds nearbyint ties to even.
int round_half_even(double value)
{
    return static_cast<int>(std::nearbyint(value));
}

} // namespace

int build_plan(const awa_plan_desc& desc, awa_plan& plan, std::string& error)
{
    int st = desc.source_t, sh = desc.source_h, sw = desc.source_w;
    if (st == -1 && sh == -1 && sw == -1)
    {
        // Dynamic package: take the grid from the runtime spec (AwaRuntimeSpec::valid, :340-345).
        const long long tokens = static_cast<long long>(desc.runtime_t) * desc.runtime_h * desc.runtime_w;
        if (!(desc.runtime_t > 0 && desc.runtime_h > 0 && desc.runtime_w > 0 && desc.runtime_tokens > 0 &&
              tokens == desc.runtime_tokens && tokens <= INT_MAX))
        {
            error = "source grid is -1,-1,-1 but the runtime spec is missing or invalid";
            return AWA_ERR_INVALID;
        }
        st = desc.runtime_t;
        sh = desc.runtime_h;
        sw = desc.runtime_w;
    }
    const long long source_tokens = static_cast<long long>(st) * sh * sw;
    if (!(st > 0 && sh > 0 && sw > 0 && desc.windows_t > 0 && desc.windows_h > 0 && desc.windows_w > 0 &&
          desc.text_tokens > 0 && source_tokens <= INT_MAX))
    {
        error = "invalid layer params: grid, window counts and text tokens must be positive";
        return AWA_ERR_INVALID;
    }
    // src/awa/awa_layers.cpp:872-874: rope_dim must be positive and a multiple of 6.
    const int rope_dim = desc.rope_dim;
    if (rope_dim <= 0 || rope_dim % 6 != 0)
    {
        error = "rope_dim must be a positive multiple of 6";
        return AWA_ERR_INVALID;
    }
    if (desc.heads < 0)
    {
        error = "heads must be 0 (unknown) or positive";
        return AWA_ERR_INVALID;
    }
    plan.heads_hint = desc.heads;

    plan.source_t = st;
    plan.source_h = sh;
    plan.source_w = sw;
    plan.windows_t = desc.windows_t;
    plan.windows_h = desc.windows_h;
    plan.windows_w = desc.windows_w;
    plan.text_tokens = desc.text_tokens;
    plan.shifted = desc.shifted != 0;
    plan.rope_dim = rope_dim;
    plan.source_tokens = static_cast<int>(source_tokens);

    // Window extents over the grid rescaled to area 45x80 = 3600 cells.
    const double scale = std::sqrt(3600.0 / (sh * sw));
    const int resized_h = round_half_even(sh * scale);
    const int resized_w = round_half_even(sw * scale);
    plan.window_h = (resized_h + desc.windows_h - 1) / desc.windows_h;
    plan.window_w = (resized_w + desc.windows_w - 1) / desc.windows_w;
    plan.window_t = (std::min(st, 30) + desc.windows_t - 1) / desc.windows_t;
    if (plan.window_h <= 0 || plan.window_w <= 0)
    {
        error = "window extent collapsed to zero";
        return AWA_ERR_INVALID;
    }

    const std::vector<Interval> it = axis_intervals(st, plan.window_t, plan.shifted);
    const std::vector<Interval> ih = axis_intervals(sh, plan.window_h, plan.shifted);
    const std::vector<Interval> iw = axis_intervals(sw, plan.window_w, plan.shifted);

    plan.windows.clear();
    for (const Interval& w : iw)
        for (const Interval& h : ih)
            for (const Interval& t : it)
                plan.windows.push_back({t.begin, t.end, h.begin, h.end, w.begin, w.end});
    if (plan.windows.empty())
    {
        error = "window partition is empty";
        return AWA_ERR_INVALID;
    }

    const int N = plan.source_tokens;
    const int T = plan.text_tokens;
    const long long S = static_cast<long long>(N) + static_cast<long long>(plan.windows.size()) * T;
    if (S > INT_MAX / 4)
    {
        error = "packed sequence too long";
        return AWA_ERR_INVALID;
    }
    plan.sequence_tokens = static_cast<int>(S);
    plan.sequence_index.assign(S, 0);
    plan.rows.assign(S, RowInfo{0, 0, 0, 0});
    plan.video_positions.assign(N, -1);
    plan.text_positions.assign(plan.windows.size() * T, 0);
    plan.cu_seqlens.assign(plan.windows.size() + 1, 0);
    plan.window_descs.clear();
    plan.max_window_tokens = 0;

    int cursor = 0;
    int max_coord = T; // text coordinates run to T-1, video t coordinates to T+et-1
    for (size_t wi = 0; wi < plan.windows.size(); wi++)
    {
        const Box& b = plan.windows[wi];
        const int et = b.t1 - b.t0, eh = b.h1 - b.h0, ew = b.w1 - b.w0;
        plan.window_descs.push_back({b.t0, b.h0, b.w0, et, eh, ew, et * eh * ew, cursor});
        for (int t = 0; t < et; t++)
            for (int h = 0; h < eh; h++)
                for (int w = 0; w < ew; w++)
                {
                    const int source = ((b.t0 + t) * sh + (b.h0 + h)) * sw + (b.w0 + w);
                    plan.sequence_index[cursor] = source;
                    plan.rows[cursor] = {source, T + t, h, w};
                    plan.video_positions[source] = cursor;
                    cursor++;
                }
        for (int k = 0; k < T; k++)
        {
            plan.sequence_index[cursor] = N + k;
            plan.rows[cursor] = {N + k, k, k, k};
            plan.text_positions[wi * T + k] = cursor;
            cursor++;
        }
        plan.cu_seqlens[wi + 1] = cursor;
        plan.max_window_tokens = std::max(plan.max_window_tokens, et * eh * ew + T);
        max_coord = std::max(max_coord, std::max(T + et, std::max(eh, ew)));
    }
    // Every video token must be covered exactly once (src/awa/awa_layers.cpp:635).
    for (int p : plan.video_positions)
        if (p < 0)
        {
            error = "windows do not cover the token grid";
            return AWA_ERR_INVALID;
        }

    // RoPE: frequency of pair p of an axis of axis_dim = rope_dim/3 features is
    // 10000^(-2p/axis_dim) in float, angle = coordinate * frequency in float.
    const int axis_dim = rope_dim / 3;
    plan.rope_pairs = axis_dim / 2;
    plan.rope_coords = max_coord;
    plan.rope_cs.assign(static_cast<size_t>(max_coord) * plan.rope_pairs * 2, 0.f);
    for (int pair = 0; pair < plan.rope_pairs; pair++)
    {
        const float frequency = std::pow(10000.f, -static_cast<float>(2 * pair) / axis_dim);
        for (int c = 0; c < max_coord; c++)
        {
            const float angle = c * frequency;
            float* cs = &plan.rope_cs[(static_cast<size_t>(c) * plan.rope_pairs + pair) * 2];
            cs[0] = std::cos(angle);
            cs[1] = std::sin(angle);
        }
    }
    return AWA_OK;
}

void rope_row(const awa_plan& plan, int position, float* out)
{
    const RowInfo& r = plan.rows[position];
    const int coords[3] = {r.ct, r.ch, r.cw};
    const int axis_dim = plan.rope_dim / 3;
    for (int axis = 0; axis < 3; axis++)
        for (int pair = 0; pair < plan.rope_pairs; pair++)
        {
            const float* cs = &plan.rope_cs[(static_cast<size_t>(coords[axis]) * plan.rope_pairs + pair) * 2];
            const int feature = axis * axis_dim + 2 * pair;
            out[feature] = out[feature + 1] = cs[0];
            out[plan.rope_dim + feature] = out[plan.rope_dim + feature + 1] = cs[1];
        }
}

} // namespace awa
