// CPU oracle for the SeedVR2 adaptive-window-attention (AWA) path.
//
// TEST INFRASTRUCTURE ONLY. This file restates the reference's CPU semantics
// so that tests, the smoke check and the CPU-baseline leg of the benchmark can
// check the HIP implementation against it. The product library never links,
// loads or calls anything built from this directory.
//
// Each function names the reference code it restates (paths relative to the
// reference repository root). Functions follow the reference's loop order and
// arithmetic exactly; the attention has two variants because the reference has
// two arithmetic orders (plain CPU loop and the Kahan-compensated shaders).
//
// Build: g++ -O3 -fopenmp -ffp-contract=off -shared -fPIC (no fast-math, no
// -march): no FMA contraction, as in a default x86-64 Release build of the
// reference.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace
{

struct Box
{
    int t0, t1, h0, h1, w0, w1;
};

// src/awa/awa_layers.cpp:36-39
int ceil_div(int numerator, int denominator)
{
    return (numerator + denominator - 1) / denominator;
}

// src/awa/awa_layers.cpp:41-51 (Python round(): ties to even)
int python_round_positive(double value)
{
    const double lower = std::floor(value);
    const double fraction = value - lower;
    if (fraction < 0.5)
        return static_cast<int>(lower);
    if (fraction > 0.5)
        return static_cast<int>(lower + 1.0);
    const int lower_int = static_cast<int>(lower);
    return lower_int % 2 == 0 ? lower_int : lower_int + 1;
}

// src/awa/awa_layers.cpp:53-88 — literal triple loop, w outer, h, t inner.
std::vector<Box> make_windows(int source_t, int source_h, int source_w, int num_t, int num_h, int num_w,
                              bool shifted)
{
    const double scale = std::sqrt(3600.0 / (source_h * source_w));
    const int resized_h = python_round_positive(source_h * scale);
    const int resized_w = python_round_positive(source_w * scale);
    const int window_h = ceil_div(resized_h, num_h);
    const int window_w = ceil_div(resized_w, num_w);
    const int window_t = ceil_div(std::min(source_t, 30), num_t);
    const double shift_t = shifted && window_t < source_t ? 0.5 : 0.0;
    const double shift_h = shifted && window_h < source_h ? 0.5 : 0.0;
    const double shift_w = shifted && window_w < source_w ? 0.5 : 0.0;
    const int count_t = static_cast<int>(std::ceil((source_t - shift_t) / window_t)) + (shift_t > 0 ? 1 : 0);
    const int count_h = static_cast<int>(std::ceil((source_h - shift_h) / window_h)) + (shift_h > 0 ? 1 : 0);
    const int count_w = static_cast<int>(std::ceil((source_w - shift_w) / window_w)) + (shift_w > 0 ? 1 : 0);
    std::vector<Box> windows;
    for (int iw = 0; iw < count_w; iw++)
        for (int ih = 0; ih < count_h; ih++)
            for (int it = 0; it < count_t; it++)
            {
                const int t0 = std::max(static_cast<int>((it - shift_t) * window_t), 0);
                const int h0 = std::max(static_cast<int>((ih - shift_h) * window_h), 0);
                const int w0 = std::max(static_cast<int>((iw - shift_w) * window_w), 0);
                const int t1 = std::min(static_cast<int>((it - shift_t + 1.0) * window_t), source_t);
                const int h1 = std::min(static_cast<int>((ih - shift_h + 1.0) * window_h), source_h);
                const int w1 = std::min(static_cast<int>((iw - shift_w + 1.0) * window_w), source_w);
                if (t1 > t0 && h1 > h0 && w1 > w0)
                    windows.push_back({t0, t1, h0, h1, w0, w1});
            }
    return windows;
}

// Pack/unpack index maps: src/awa/awa_layers.cpp:388-407 (sequence_index,
// cu_seqlens) and :605-626 (video_positions, text_positions).
struct Maps
{
    std::vector<int> sequence_index;
    std::vector<int> cu_seqlens;
    std::vector<int> video_positions;
    std::vector<int> text_positions;
    std::vector<int> target;
    int window_count = 0;
};

Maps build_maps(int st, int sh, int sw, int nt, int nh, int nw, int text_tokens, bool shifted)
{
    Maps m;
    const int source_tokens = st * sh * sw;
    m.video_positions.assign(source_tokens, -1);
    m.cu_seqlens.push_back(0);
    const std::vector<Box> windows = make_windows(st, sh, sw, nt, nh, nw, shifted);
    int cursor = 0;
    for (const Box& b : windows)
    {
        for (int t = b.t0; t < b.t1; t++)
            for (int h = b.h0; h < b.h1; h++)
                for (int w = b.w0; w < b.w1; w++)
                {
                    const int source_index = (t * sh + h) * sw + w;
                    m.sequence_index.push_back(source_index);
                    m.target.push_back(source_index);
                    m.video_positions[source_index] = cursor++;
                }
        for (int token = 0; token < text_tokens; token++)
        {
            m.sequence_index.push_back(source_tokens + token);
            m.text_positions.push_back(cursor + token);
        }
        cursor += text_tokens;
        m.cu_seqlens.push_back(cursor);
    }
    m.window_count = static_cast<int>(windows.size());
    return m;
}

// Kahan step as written in src/awa/shader/awa_attention_score.comp:40-44.
// Correct only without reassociation: this file is built without fast-math and
// with -ffp-contract=off.
float kahan_add(float sum, float term_in, float& correction)
{
    const float term = term_in - correction;
    const float next = sum + term;
    correction = (next - sum) - term;
    return next;
}

} // namespace

extern "C" {

// Thread count of the (window, head)-parallel loops; 1 reproduces the
// reference's single-threaded CPU layers.
int orc_set_num_threads(int threads)
{
    if (threads < 1)
        return -1;
#ifdef _OPENMP
    omp_set_num_threads(threads);
#endif
    return 0;
}

int orc_python_round_positive(double value)
{
    return python_round_positive(value);
}

// Writes 6 ints per window (t0,t1,h0,h1,w0,w1); returns the window count, or
// -1 for non-positive arguments (src/awa/awa_layers.cpp:347-359 semantics) or
// when the output capacity is too small.
int orc_make_windows(int st, int sh, int sw, int nt, int nh, int nw, int shifted, int* out, int capacity)
{
    if (st <= 0 || sh <= 0 || sw <= 0 || nt <= 0 || nh <= 0 || nw <= 0)
        return -1;
    const std::vector<Box> windows = make_windows(st, sh, sw, nt, nh, nw, shifted != 0);
    if (static_cast<int>(windows.size()) > capacity)
        return -1;
    for (size_t i = 0; i < windows.size(); i++)
    {
        const Box& b = windows[i];
        const int v[6] = {b.t0, b.t1, b.h0, b.h1, b.w0, b.w1};
        std::memcpy(out + 6 * i, v, sizeof(v));
    }
    return static_cast<int>(windows.size());
}

// Sizes of the maps for one layer: out[0] = S (packed tokens), out[1] = nwin.
int orc_map_sizes(int st, int sh, int sw, int nt, int nh, int nw, int text_tokens, int shifted, int* out)
{
    const Maps m = build_maps(st, sh, sw, nt, nh, nw, text_tokens, shifted != 0);
    out[0] = static_cast<int>(m.sequence_index.size());
    out[1] = m.window_count;
    return 0;
}

// Fills every map; buffers sized from orc_map_sizes: sequence_index[S],
// cu_seqlens[nwin+1], video_positions[N], text_positions[nwin*T_x],
// target[N]. Returns 0, or -1 when the windows do not cover the grid exactly
// (the check of src/awa/awa_layers.cpp:635).
int orc_build_maps(int st, int sh, int sw, int nt, int nh, int nw, int text_tokens, int shifted,
                   int* sequence_index, int* cu_seqlens, int* video_positions, int* text_positions, int* target)
{
    const Maps m = build_maps(st, sh, sw, nt, nh, nw, text_tokens, shifted != 0);
    std::memcpy(sequence_index, m.sequence_index.data(), m.sequence_index.size() * sizeof(int));
    std::memcpy(cu_seqlens, m.cu_seqlens.data(), m.cu_seqlens.size() * sizeof(int));
    std::memcpy(video_positions, m.video_positions.data(), m.video_positions.size() * sizeof(int));
    std::memcpy(text_positions, m.text_positions.data(), m.text_positions.size() * sizeof(int));
    std::memcpy(target, m.target.data(), m.target.size() * sizeof(int));
    return (m.window_count > 0 && m.target.size() == static_cast<size_t>(st * sh * sw)) ? 0 : -1;
}

// MMRoPE rotation table Mat(2*rope_dim, S): row = [cos(rope_dim) | sin(rope_dim)].
// src/awa/awa_layers.cpp:867-911.
int orc_rope_table(int st, int sh, int sw, int nt, int nh, int nw, int text_tokens, int shifted, int rope_dim,
                   float* table)
{
    if (rope_dim <= 0 || rope_dim % 6 != 0)
        return -1;
    const int axis_dim = rope_dim / 3;
    const std::vector<Box> windows = make_windows(st, sh, sw, nt, nh, nw, shifted != 0);
    auto write_rotation = [&](int position, int ct, int ch, int cw) {
        float* data = table + static_cast<size_t>(position) * 2 * rope_dim;
        const int coordinates[] = {ct, ch, cw};
        for (int axis = 0; axis < 3; axis++)
            for (int pair = 0; pair < axis_dim / 2; pair++)
            {
                const float frequency = std::pow(10000.f, -static_cast<float>(2 * pair) / axis_dim);
                const float angle = coordinates[axis] * frequency;
                const int feature = axis * axis_dim + 2 * pair;
                data[feature] = std::cos(angle);
                data[feature + 1] = data[feature];
                data[rope_dim + feature] = std::sin(angle);
                data[rope_dim + feature + 1] = data[rope_dim + feature];
            }
    };
    int cursor = 0;
    for (const Box& b : windows)
    {
        for (int t = b.t0; t < b.t1; t++)
            for (int h = b.h0; h < b.h1; h++)
                for (int w = b.w0; w < b.w1; w++)
                    write_rotation(cursor++, text_tokens + (t - b.t0), h - b.h0, w - b.w0);
        for (int token = 0; token < text_tokens; token++)
            write_rotation(cursor++, token, token, token);
    }
    return cursor;
}

// Pack forward (src/awa/awa_layers.cpp:419-458) on fp32 inputs addressed by
// (token_stride, qkv_stride) in elements, as derived by describe_qkv_layout
// (:116-170). Output packed[S][3][H][d] dense fp32 and cu_seqlens as float.
int orc_pack_forward(const float* video, long long video_token_stride, long long video_qkv_stride,
                     const float* text, long long text_token_stride, long long text_qkv_stride,
                     const int* sequence_index, int sequence_tokens, const int* cu_seqlens, int window_count,
                     int source_tokens, int heads, int head_dim, float* packed, float* cu_out)
{
    const size_t qkv_size = static_cast<size_t>(heads) * head_dim;
    for (int position = 0; position < sequence_tokens; position++)
    {
        const int source_index = sequence_index[position];
        const bool is_video = source_index < source_tokens;
        const int token = is_video ? source_index : source_index - source_tokens;
        const float* src = is_video ? video + token * video_token_stride : text + token * text_token_stride;
        const long long qkv_stride = is_video ? video_qkv_stride : text_qkv_stride;
        float* dst = packed + static_cast<size_t>(position) * 3 * qkv_size;
        for (int qkv = 0; qkv < 3; qkv++)
            std::memcpy(dst + qkv * qkv_size, src + qkv * qkv_stride, qkv_size * sizeof(float));
    }
    for (int i = 0; i <= window_count; i++)
        cu_out[i] = static_cast<float>(cu_seqlens[i]);
    return 0;
}

// MMRoPE forward (src/awa/awa_layers.cpp:913-953) on dense [S][3H][d] fp32.
int orc_mmrope_forward(const float* input, const float* table, int sequence_tokens, int heads, int head_dim,
                       int rope_dim, float* output)
{
    const int rows = 3 * heads;
    for (int token = 0; token < sequence_tokens; token++)
    {
        const float* source = input + static_cast<size_t>(token) * rows * head_dim;
        float* out = output + static_cast<size_t>(token) * rows * head_dim;
        const float* rotation = table + static_cast<size_t>(token) * 2 * rope_dim;
        for (int qkv_head = 0; qkv_head < rows; qkv_head++)
            for (int feature = 0; feature < head_dim; feature++)
            {
                const int offset = qkv_head * head_dim + feature;
                if (qkv_head >= 2 * heads || feature >= rope_dim)
                {
                    out[offset] = source[offset];
                    continue;
                }
                const int paired_feature = feature % 2 == 0 ? feature + 1 : feature - 1;
                const float paired = source[qkv_head * head_dim + paired_feature];
                out[offset] = feature % 2 == 0
                                  ? source[offset] * rotation[feature] - paired * rotation[rope_dim + feature]
                                  : source[offset] * rotation[feature] + paired * rotation[rope_dim + feature];
            }
    }
    return 0;
}

// WindowAttention CPU forward (src/awa/awa_layers.cpp:1062-1120): plain fp32
// sums, std::exp, p/normalizer applied inside the value loop. Input packed
// [S][3H][d], output [S][H][d]. Parallel over (window, head); each (window,
// head) keeps the reference's sequential order, so the result does not depend
// on the thread count.
int orc_attention_cpu(const float* input, const int* cu_seqlens, int window_count, int heads, int head_dim,
                      float* output)
{
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    const size_t in_row = static_cast<size_t>(3) * heads * head_dim;
    const size_t out_row = static_cast<size_t>(heads) * head_dim;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int window_index = 0; window_index < window_count; window_index++)
        for (int head = 0; head < heads; head++)
        {
            const int window_start = cu_seqlens[window_index];
            const int window_length = cu_seqlens[window_index + 1] - window_start;
            std::vector<float> scores(static_cast<size_t>(window_length));
            for (int query = 0; query < window_length; query++)
            {
                float max_score = -INFINITY;
                const float* query_data = input + (window_start + query) * in_row + head * head_dim;
                for (int key = 0; key < window_length; key++)
                {
                    const float* key_data = input + (window_start + key) * in_row + (heads + head) * head_dim;
                    float dot = 0.f;
                    for (int feature = 0; feature < head_dim; feature++)
                        dot += query_data[feature] * key_data[feature];
                    scores[key] = dot * scale;
                    max_score = std::max(max_score, scores[key]);
                }
                float normalizer = 0.f;
                for (int key = 0; key < window_length; key++)
                {
                    scores[key] = std::exp(scores[key] - max_score);
                    normalizer += scores[key];
                }
                float* out = output + (window_start + query) * out_row + head * head_dim;
                for (int feature = 0; feature < head_dim; feature++)
                {
                    float value = 0.f;
                    for (int key = 0; key < window_length; key++)
                    {
                        const float* value_data =
                            input + (window_start + key) * in_row + (2 * heads + head) * head_dim;
                        value += scores[key] / normalizer * value_data[feature];
                    }
                    out[feature] = value;
                }
            }
        }
    return 0;
}

// WindowAttention in the arithmetic order of the shaders the reference runs
// on its GPU path: Kahan dot then *scale (awa_attention_score.comp:27-47);
// sequential max, exp, Kahan sum, in-place divide (awa_attention_softmax.comp:
// 21-56); Kahan P*V (awa_attention_value.comp:27-54).
int orc_attention_kahan(const float* input, const int* cu_seqlens, int window_count, int heads, int head_dim,
                        float* output)
{
    const float scale = 1.f / std::sqrt(static_cast<float>(head_dim));
    const size_t in_row = static_cast<size_t>(3) * heads * head_dim;
    const size_t out_row = static_cast<size_t>(heads) * head_dim;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int window_index = 0; window_index < window_count; window_index++)
        for (int head = 0; head < heads; head++)
        {
            const int window_start = cu_seqlens[window_index];
            const int window_length = cu_seqlens[window_index + 1] - window_start;
            std::vector<float> scores(static_cast<size_t>(window_length));
            for (int query = 0; query < window_length; query++)
            {
                const float* query_data = input + (window_start + query) * in_row + head * head_dim;
                for (int key = 0; key < window_length; key++)
                {
                    const float* key_data = input + (window_start + key) * in_row + (heads + head) * head_dim;
                    float dot = 0.f;
                    float correction = 0.f;
                    for (int feature = 0; feature < head_dim; feature++)
                    {
                        const float product = query_data[feature] * key_data[feature];
                        dot = kahan_add(dot, product, correction);
                    }
                    scores[key] = dot * scale;
                }
                float maximum = scores[0];
                for (int key = 1; key < window_length; key++)
                    maximum = std::max(maximum, scores[key]);
                float normalizer = 0.f;
                float correction = 0.f;
                for (int key = 0; key < window_length; key++)
                {
                    const float value = std::exp(scores[key] - maximum);
                    scores[key] = value;
                    normalizer = kahan_add(normalizer, value, correction);
                }
                for (int key = 0; key < window_length; key++)
                    scores[key] /= normalizer;
                float* out = output + (window_start + query) * out_row + head * head_dim;
                for (int feature = 0; feature < head_dim; feature++)
                {
                    float value = 0.f;
                    float corr = 0.f;
                    for (int key = 0; key < window_length; key++)
                    {
                        const float* value_data =
                            input + (window_start + key) * in_row + (2 * heads + head) * head_dim;
                        const float product = scores[key] * value_data[feature];
                        value = kahan_add(value, product, corr);
                    }
                    out[feature] = value;
                }
            }
        }
    return 0;
}

// Unpack forward on packed [S][H][d] fp32. Video scatter to dense [N][H][d]
// (the NCNN_BATCH [t][h][w][H][d] layout has the same order when dense).
// text_order 0: CPU order, text += x / nwin per window (awa_layers.cpp:677-687).
// text_order 1: shader order, (sum over windows in window order) / nwin
// (src/awa/shader/awa_unpack.comp:47-58).
int orc_unpack_forward(const float* packed, const int* video_positions, int source_tokens,
                       const int* text_positions, int text_tokens, int window_count, int heads, int head_dim,
                       int text_order, float* video, float* text)
{
    const size_t row = static_cast<size_t>(heads) * head_dim;
    for (int source_index = 0; source_index < source_tokens; source_index++)
        std::memcpy(video + source_index * row, packed + static_cast<size_t>(video_positions[source_index]) * row,
                    row * sizeof(float));
    for (int token = 0; token < text_tokens; token++)
    {
        float* out = text + token * row;
        for (size_t value = 0; value < row; value++)
        {
            float sum = 0.f;
            for (int window = 0; window < window_count; window++)
            {
                const float x = packed[static_cast<size_t>(text_positions[window * text_tokens + token]) * row + value];
                if (text_order == 0)
                    sum += x / window_count;
                else
                    sum += x;
            }
            out[value] = text_order == 0 ? sum : sum / static_cast<float>(window_count);
        }
    }
    return 0;
}

// fill_gaussian_noise (src/sampler/sampler.cpp:37-61): mt19937 seeded by
// seed_seq{seed, stream_lo, stream_hi}, Box-Muller in double with midpoint
// uniforms, cast to float; an odd count drops the last sine.
// DitRMSNorm (src/dit/dit_precision.cpp:63-86) as its shader computes it
// (src/dit/shader/dit_rmsnorm.comp:16-45): for each of `rows` rows of `width`
// values, 128 partial sums (lane l adds x[i]^2 for i = l, l + 128, ...), a
// pairwise reduction with stride 64, 32, ..., 1, coefficient =
// inversesqrt(sum / width + eps), restated as 1 / sqrt(...) with correctly
// rounded operations (the shader's inversesqrt is driver-defined to 2 ulp);
// out = x * coefficient, then * gamma[i] when gamma is not null (affine).
int orc_rmsnorm(const float* input, long long rows, int width, const float* gamma, float eps, float* output)
{
    if (rows < 0 || width <= 0)
        return -1;
    for (long long r = 0; r < rows; r++)
    {
        const float* x = input + r * width;
        float sums[128];
        for (int lane = 0; lane < 128; lane++)
        {
            float sum = 0.f;
            for (int i = lane; i < width; i += 128)
            {
                const float square = x[i] * x[i];
                sum = sum + square;
            }
            sums[lane] = sum;
        }
        for (int stride = 64; stride > 0; stride /= 2)
            for (int lane = 0; lane < stride; lane++)
                sums[lane] = sums[lane] + sums[lane + stride];
        const float coefficient = 1.f / std::sqrt(sums[0] / static_cast<float>(width) + eps);
        for (int i = 0; i < width; i++)
        {
            const float value = x[i] * coefficient;
            output[r * width + i] = gamma ? value * gamma[i] : value;
        }
    }
    return 0;
}

int orc_fill_gaussian(float* output, long long count, unsigned int seed, unsigned long long stream)
{
    if (!output || count <= 0)
        return -1;
    std::seed_seq sequence{seed, static_cast<std::uint32_t>(stream), static_cast<std::uint32_t>(stream >> 32)};
    std::mt19937 generator(sequence);
    const double inverse_range = 1.0 / 4294967296.0;
    const double two_pi = 6.283185307179586476925286766559;
    for (long long index = 0; index < count; index += 2)
    {
        const double radial_uniform = (static_cast<double>(generator()) + 0.5) * inverse_range;
        const double angle_uniform = (static_cast<double>(generator()) + 0.5) * inverse_range;
        const double radius = std::sqrt(-2.0 * std::log(radial_uniform));
        const double angle = two_pi * angle_uniform;
        output[index] = static_cast<float>(radius * std::cos(angle));
        if (index + 1 < count)
            output[index + 1] = static_cast<float>(radius * std::sin(angle));
    }
    return 0;
}

// The seed_seq words that initialise the generator above, for checking the
// restatement against an independent Mersenne Twister (624 words).
int orc_seed_seq_words(unsigned int seed, unsigned long long stream, unsigned int* words)
{
    std::seed_seq sequence{seed, static_cast<std::uint32_t>(stream), static_cast<std::uint32_t>(stream >> 32)};
    sequence.generate(words, words + 624);
    return 0;
}

// Round-to-nearest-even fp32 -> bf16 as written in src/dit/shader/dit_rmsnorm.comp:47-51;
// returns the bf16 bit patterns.
int orc_round_bf16(const float* input, unsigned short* output, long long count)
{
    for (long long i = 0; i < count; i++)
    {
        std::uint32_t bits;
        std::memcpy(&bits, &input[i], 4);
        bits = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
        output[i] = static_cast<unsigned short>(bits >> 16);
    }
    return 0;
}

// The whole AWA layer chain Pack -> MMRoPE -> WindowAttention -> Unpack on
// fp32 inputs in the canonical token-major [N][3][H][d] / [T_x][3][H][d]
// layout. attention_order 0 = CPU loop order, 1 = Kahan shader order;
// text_order as in orc_unpack_forward. Outputs video [N][H][d], text [T_x][H][d].
int orc_awa_layer(const float* video_qkv, const float* text_qkv, int st, int sh, int sw, int nt, int nh, int nw,
                  int text_tokens, int shifted, int rope_dim, int heads, int head_dim, int attention_order,
                  int text_order, float* video_out, float* text_out)
{
    const Maps m = build_maps(st, sh, sw, nt, nh, nw, text_tokens, shifted != 0);
    if (m.window_count <= 0)
        return -1;
    const int S = static_cast<int>(m.sequence_index.size());
    const int N = st * sh * sw;
    const size_t qkv_row = static_cast<size_t>(3) * heads * head_dim;
    std::vector<float> packed(S * qkv_row), roped(S * qkv_row), cu(m.window_count + 1);
    std::vector<float> table(static_cast<size_t>(S) * 2 * rope_dim);
    std::vector<float> attended(static_cast<size_t>(S) * heads * head_dim);
    orc_pack_forward(video_qkv, qkv_row, static_cast<long long>(heads) * head_dim, text_qkv, qkv_row,
                     static_cast<long long>(heads) * head_dim, m.sequence_index.data(), S, m.cu_seqlens.data(),
                     m.window_count, N, heads, head_dim, packed.data(), cu.data());
    if (orc_rope_table(st, sh, sw, nt, nh, nw, text_tokens, shifted, rope_dim, table.data()) != S)
        return -1;
    orc_mmrope_forward(packed.data(), table.data(), S, heads, head_dim, rope_dim, roped.data());
    if (attention_order == 0)
        orc_attention_cpu(roped.data(), m.cu_seqlens.data(), m.window_count, heads, head_dim, attended.data());
    else
        orc_attention_kahan(roped.data(), m.cu_seqlens.data(), m.window_count, heads, head_dim, attended.data());
    orc_unpack_forward(attended.data(), m.video_positions.data(), N, m.text_positions.data(), text_tokens,
                       m.window_count, heads, head_dim, text_order, video_out, text_out);
    return 0;
}

} // extern "C"
