// Device helpers shared by the attention kernels (gfx950): bf16 packing,
// raw 16-byte loads, the interleaved RoPE rotation, window-row decoding, the
// key order of staged K tiles, output row stores and cross-lane reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "awa_kernels.h"

namespace awa
{
namespace dev
{

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRopePairs = kRopeDim / 6; // 21 pairs per axis
constexpr int kRopeRow = 2 * kRopePairs; // floats per coordinate in the table
constexpr float kRescaleThreshold = 8.f; // log2 units
static_assert(kMaxRopeCoords * kRopeRow * 4 <= 24 * 1024, "RoPE table must stay small in LDS");

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi)
{
    const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w)
{
    return __uint_as_float(w << 16);
}

__device__ __forceinline__ float bf16_hi(uint32_t w)
{
    return __uint_as_float(w & 0xffff0000u);
}

// Raw 8-element loads (16-byte aligned): bf16 -> 4 words, fp32 -> 8 words.
__device__ __forceinline__ void load_raw8(const uint16_t* p, uint32_t* w)
{
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    w[0] = a.x;
    w[1] = a.y;
    w[2] = a.z;
    w[3] = a.w;
}

__device__ __forceinline__ void load_raw8(const float* p, uint32_t* w)
{
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x;
    w[1] = a.y;
    w[2] = a.z;
    w[3] = a.w;
    w[4] = b.x;
    w[5] = b.y;
    w[6] = b.z;
    w[7] = b.w;
}

template <typename TIn>
constexpr int kRawWords8 = sizeof(TIn) == 2 ? 4 : 8; // words per 8 elements

template <typename TIn>
__device__ __forceinline__ void raw_to_float8(const uint32_t* w, float* v)
{
    if constexpr (sizeof(TIn) == 2)
    {
#pragma unroll
        for (int i = 0; i < 4; i++)
        {
            v[2 * i] = bf16_lo(w[i]);
            v[2 * i + 1] = bf16_hi(w[i]);
        }
    }
    else
    {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = __uint_as_float(w[i]);
    }
}

// One interleaved RoPE pair: even' = x0*cos - x1*sin, odd' = x1*cos + x0*sin.
// No contraction, so the result is bit-identical to the reference's CPU rotation.
__device__ __forceinline__ void rope_pair_cs(float& x0, float& x1, float c, float s)
{
#pragma clang fp contract(off)
    const float a = x0;
    const float b = x1;
    x0 = a * c - b * s;
    x1 = b * c + a * s;
}

// The same rotation with fused multiply-adds, for operands that are rounded
// to bf16 right after (the two forms differ by at most an fp32 ulp).
__device__ __forceinline__ void rope_pair_fma(float& x0, float& x1, float c, float s)
{
    const float a = x0;
    const float b = x1;
    x0 = fmaf(a, c, -(b * s));
    x1 = fmaf(b, c, a * s);
}

// Window-local row i of a window, decoded: video rows (i < video_tokens)
// are in (t, h, w) order inside the window box, text rows follow. Both
// interpretations are computed and selected, so rows of a wave that mix
// video and text take no divergent branch.
struct RowRef
{
    bool text;
    int k;          // text index
    int t, h, w;    // grid position (video)
    int ct, ch, cw; // RoPE coordinates
    uint32_t token; // video token index (meaningful for video rows)
};

// Reciprocals of the window's h*w and w extents, for quotients of row
// indices: floor(i / d) = int((i + 0.5) * fl(1 / d)) exactly, since the
// relative error of the product (a few fp32 ulps) times i / d stays below
// the distance 0.5 / d of (i + 0.5) / d from an integer for any i < 2^20.
struct RowDivisors
{
    float inv_area, inv_ew;
    int area, ew;
};

__device__ __forceinline__ RowDivisors row_divisors(const WindowDesc& win)
{
    RowDivisors d;
    d.area = win.eh * win.ew;
    d.ew = win.ew;
    d.inv_area = 1.f / static_cast<float>(d.area);
    d.inv_ew = 1.f / static_cast<float>(d.ew);
    return d;
}

__device__ __forceinline__ RowRef window_row(const WindowDesc& win, const RowDivisors& dv, int i, int text_tokens,
                                             int source_h, int source_w)
{
    RowRef r;
    const int lt = static_cast<int>((static_cast<float>(i) + 0.5f) * dv.inv_area);
    const int rem = i - lt * dv.area;
    const int lh = static_cast<int>((static_cast<float>(rem) + 0.5f) * dv.inv_ew);
    const int lw = rem - lh * dv.ew;
    const int k = i - win.video_tokens;
    r.text = k >= 0;
    r.k = k;
    r.t = win.t0 + lt;
    r.h = win.h0 + lh;
    r.w = win.w0 + lw;
    // Unsigned arithmetic: for text rows the video fields are meaningless
    // (and may wrap), the value is then never used.
    r.token = (static_cast<uint32_t>(r.t) * static_cast<uint32_t>(source_h) + static_cast<uint32_t>(r.h)) *
                  static_cast<uint32_t>(source_w) +
              static_cast<uint32_t>(r.w);
    r.ct = r.text ? k : text_tokens + lt;
    r.ch = r.text ? k : lh;
    r.cw = r.text ? k : lw;
    return r;
}

// Key order of a 32-key block in the K tile: key m is stored at row
// key_permute(m) (bits 2 and 3 swapped), so that the S^T MFMA, reading rows
// in lane order (conflict-free), sees the keys in the order the PV operand
// layout needs.
__device__ __forceinline__ int key_permute(int m)
{
    return (m & ~0xC) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Key swizzle of the transposed V tile: row d of Vt stores key k at column
// k ^ (8 * vt_swizzle(d)). Groups of 8 keys stay contiguous (one 16-byte MFMA
// operand read); the PV reads of 16 consecutive rows cover every LDS bank
// once, with 32 or 64 banks.
template <int KT>
__device__ __forceinline__ int vt_swizzle(int d)
{
    return (d >> 4) & (KT / 8 - 1);
}

__device__ __forceinline__ void store4(float* dst, float a, float b, float c, float d)
{
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
}

__device__ __forceinline__ void store4(uint16_t* dst, float a, float b, float c, float d)
{
    *reinterpret_cast<uint2*>(dst) = make_uint2(cvt_pk_bf16(a, b), cvt_pk_bf16(c, d));
}

template <typename TOut>
__device__ __forceinline__ void store_row(TOut* dst, const f32x16 (&o)[4], float inv, int half)
{
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            store4(dst + db * 32 + 8 * g + 4 * half, o[db][4 * g] * inv, o[db][4 * g + 1] * inv,
                   o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
}

// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap hands each lane
// its partner's value in one of the two results, its own in the other).
__device__ __forceinline__ float max_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum of x over each group of 16 consecutive lanes, in every lane of the
// group (DPP: swap neighbours, swap pairs, mirror the quads of each half,
// mirror the halves).
__device__ __forceinline__ float sum16(float x)
{
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
    return x;
}

// Maximum of x over each group of 16 consecutive lanes, in every lane of the
// group (the DPP pattern of sum16).
__device__ __forceinline__ float max16(float x)
{
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false)));
    return x;
}

__device__ __forceinline__ float sum_xor32(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row x of DitRMSNorm over 128 features (src/dit/shader/dit_rmsnorm.comp,
// src/dit/dit_precision.cpp:63-86) reproduced bit for bit: the shader's 128
// lanes each hold one square, which a tree adds at strides 64, 32, ..., 1
// (lane i += lane i + stride); then 1 / sqrt(sum / 128 + eps), correctly
// rounded. These helpers pair the same values (fp addition commutes, so the
// order within a pair does not matter) for the feature layouts the kernels
// hold, without contraction.
__device__ __forceinline__ float rms_coef(float sum, float eps)
{
#pragma clang fp contract(off)
    return 1.f / sqrtf(sum * (1.f / 128.f) + eps);
}

// 16 consecutive lanes hold a row, lane j (of the 16) features 8j + [0, 8).
// Strides 64, 32, 16, 8 pair lane j with lane j + 8, 4, 2, 1 (mod 16; DPP row
// rotations), strides 4, 2, 1 the lane's own values. Every lane of the 16
// returns the coefficient.
__device__ __forceinline__ float rms_coef_row16(const float (&x)[8], float eps)
{
#pragma clang fp contract(off)
    float a[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
        a[e] = x[e] * x[e];
#pragma unroll
    for (int e = 0; e < 8; e++)
        a[e] = a[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[e]), 0x128, 0xF, 0xF, false));
#pragma unroll
    for (int e = 0; e < 8; e++)
        a[e] = a[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[e]), 0x124, 0xF, 0xF, false));
#pragma unroll
    for (int e = 0; e < 8; e++)
        a[e] = a[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[e]), 0x122, 0xF, 0xF, false));
#pragma unroll
    for (int e = 0; e < 8; e++)
        a[e] = a[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[e]), 0x121, 0xF, 0xF, false));
#pragma unroll
    for (int e = 0; e < 4; e++)
        a[e] = a[e] + a[e + 4];
    a[0] = a[0] + a[2];
    a[1] = a[1] + a[3];
    return rms_coef(a[0] + a[1], eps);
}

// Bytes of the dynamic-LDS K gammas of the fused q/k RMSNorm (video, text).
template <bool NORM>
constexpr int kNormLdsBytes = NORM ? 2 * kHeadDim * 4 : 0;

// Bytes of the dynamic-LDS RoPE table: coords + 1 rows of 21 (cos, sin)
// pairs, rounded up to 16 bytes.
__host__ __device__ inline int rope_table_bytes(bool fused, int rope_coords)
{
    return fused ? ((rope_coords + 1) * kRopeRow * 4 + 15) & ~15 : 0;
}

} // namespace dev
} // namespace awa
