// QKV projection of a bf16 DiT block with the attention prologue in its
// epilogue (gfx950): Y = X W^T on bf16 MFMA with fp32 accumulation
// (tools/reference/dit_block.py:280-290, proj_qkv), then for the q and k
// heads the DitRMSNorm over head_dim times gamma (src/dit/dit_precision.cpp:63-86,
// src/dit/shader/dit_rmsnorm.comp) and the 3-axis MMRoPE rotation
// (src/awa/shader/mmrope.comp, src/awa/awa_layers.cpp:885-951), each result
// rounded to bf16 where the reference stores it: the GEMM output, the norm
// output, the rotated Q/K. V is the rounded GEMM output.
//
// A workgroup computes C^T = W_h X^T for 128 tokens and one 128-feature head
// of q, k or v (4 waves, 32 tokens each), so that after the k loop lane l of
// a wave holds 64 of the 128 features of token 32*wave + l % 32 and its
// partner lane l ^ 32 the other 64: the RMSNorm's sum over the head needs one
// lane swap, each RoPE pair sits in one lane. X and W are staged through LDS
// in 64-wide k slices, two at a time: the next two slices' loads are in
// flight while the two buffered ones are multiplied.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "awa_device.h"
#include "dit_kernels.h"

namespace awa
{
namespace
{

using namespace dev;

constexpr int kTokens = 128;        // tokens per workgroup
constexpr int kFeatures = 128;      // features per workgroup: one head
constexpr int kSlice = 64;          // k per LDS slice
constexpr int kPitch = kSlice + 8;  // LDS row pitch in elements (144 B: the 16-byte operand reads of 8 lanes hit distinct banks)
constexpr int kThreads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float round_bf16(float x)
{
    return bf16_lo(cvt_pk_bf16(x, 0.f));
}

__global__ __launch_bounds__(kThreads, 2) void qkv_rope_gemm_kernel(const QkvRopeGemm p)
{
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) uint16_t w_lds[2][kFeatures * kPitch];
    __shared__ __attribute__((aligned(16))) uint16_t x_lds[2][kTokens * kPitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;
    // Workgroup b runs on XCD b % 8 (round-robin dispatch). Each XCD takes
    // the heads h = xcd + 8 i and sweeps all token blocks of one head before
    // the next, so that a head's W rows are read into that XCD's L2 once and
    // the token blocks are shared by the heads in flight there.
    const int blocks_m = (p.m + kTokens - 1) / kTokens;
    const int head_blocks = 3 * p.heads;
    const int xcd = blockIdx.x % 8;
    const int slot = blockIdx.x / 8;
    const int head_block = xcd + 8 * (slot / blocks_m); // qkv * heads + head
    if (head_block >= head_blocks)
        return;
    const int m0 = (slot % blocks_m) * kTokens;
    const int f0 = head_block * kFeatures;

    // Slice staging: thread t moves 16 bytes (8 k) of rows t / 8 + 32 i
    // (i < 4) of the W and X slices; 8 consecutive threads cover one row's
    // 128 bytes.
    const int lr = tid >> 3;
    const int lk = 8 * (tid & 7);
    // Two register stages, each a slice of W and X rows on its way to LDS
    // (native vectors, which stay registers; arrays of the uint4 struct went
    // to private memory).
    u32x4 w0[4], x0[4], w1[4], x1[4];
    auto load_slice = [&](int s, u32x4 (&w)[4], u32x4 (&x)[4]) {
        const int k = s * kSlice + lk;
#pragma unroll
        for (int i = 0; i < 4; i++)
            w[i] = *reinterpret_cast<const u32x4*>(p.w + static_cast<long long>(f0 + lr + 32 * i) * p.ldw + k);
#pragma unroll
        for (int i = 0; i < 4; i++)
        {
            // Rows past the last token repeat it (never stored).
            const int token = min(m0 + lr + 32 * i, p.m - 1);
            x[i] = *reinterpret_cast<const u32x4*>(p.x + static_cast<long long>(token) * p.ldx + k);
        }
    };
    auto store_slice = [&](int buf, const u32x4 (&w)[4], const u32x4 (&x)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
        {
            *reinterpret_cast<u32x4*>(&w_lds[buf][(lr + 32 * i) * kPitch + lk]) = w[i];
            *reinterpret_cast<u32x4*>(&x_lds[buf][(lr + 32 * i) * kPitch + lk]) = x[i];
        }
    };

    // acc[fb]: C^T block of features 32 fb + [0, 32) x this wave's 32 tokens;
    // register i holds feature 32 fb + 8 (i / 4) + 4 half + i % 4 of token col.
    f32x16 acc[4];
#pragma unroll
    for (int fb = 0; fb < 4; fb++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            acc[fb][i] = 0.f;

    // Multiply the slice in LDS buffer buf.
    auto multiply = [&](int buf) {
        // A operand: W row 32 fb + col, k 8 half + [0, 8); B operand: X row
        // (this wave's token col), the same k.
        const uint16_t* const wl = w_lds[buf] + col * kPitch + 8 * half;
        const uint16_t* const xl = x_lds[buf] + (32 * wave + col) * kPitch + 8 * half;
#pragma unroll
        for (int kk = 0; kk < kSlice; kk += 16)
        {
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(xl + kk);
            bf16x8 a[4];
#pragma unroll
            for (int fb = 0; fb < 4; fb++)
                a[fb] = *reinterpret_cast<const bf16x8*>(wl + fb * 32 * kPitch + kk);
#pragma unroll
            for (int fb = 0; fb < 4; fb++)
                acc[fb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[fb], b, acc[fb], 0, 0, 0);
        }
    };
    // Two slices per iteration, slice t in LDS buffer t & 1: the next two
    // slices' loads are issued, the two buffered slices multiplied, and after
    // a barrier the loaded slices stored. The loaded registers never live
    // across iterations and the loads are unconditional (past the last slice
    // they re-read it, never stored), so the compiler keeps them as plain
    // registers, without copies that would wait for them.
    const int slices = p.k / kSlice; // even
    load_slice(0, w0, x0);
    load_slice(1, w1, x1);
    store_slice(0, w0, x0);
    store_slice(1, w1, x1);
    __syncthreads();
    for (int s = 0; s < slices; s += 2)
    {
        load_slice(min(s + 2, slices - 1), w0, x0);
        load_slice(min(s + 3, slices - 1), w1, x1);
        // Keep the loads ahead of the multiplies (the scheduler would sink
        // them next to the stores that wait for them).
        __builtin_amdgcn_sched_barrier(0);
        multiply(0);
        multiply(1);
        __syncthreads();
        if (s + 2 < slices)
        {
            store_slice(0, w0, x0);
            store_slice(1, w1, x1);
            __syncthreads();
        }
    }

    // ---- epilogue: this lane's token and its 64 features ----
    const int token = m0 + 32 * wave + col;
    const int kind = head_block / p.heads; // 0 q, 1 k, 2 v
    float v[4][16];
#pragma unroll
    for (int fb = 0; fb < 4; fb++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            v[fb][i] = round_bf16(acc[fb][i]); // the GEMM output as stored
    if (kind < 2)
    {
        // DitRMSNorm's sum of squares in its pairwise order: lane f of 128
        // holds x[f]^2, then sums[f] += sums[f + stride] for stride 64, 32,
        // ..., 1. Strides 64..8 stay in this lane (feature blocks, then
        // groups of 8); stride 4 pairs this lane's features 4 half + j with
        // the partner lane's; strides 2 and 1 are in-lane again.
        float sq[4][16];
#pragma unroll
        for (int fb = 0; fb < 4; fb++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                sq[fb][i] = v[fb][i] * v[fb][i];
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; i++)
            t[i] = (sq[0][i] + sq[2][i]) + (sq[1][i] + sq[3][i]); // strides 64 then 32
        // i = 4 g + j: feature 8 g + 4 half + j; stride 16 pairs g with g + 2,
        // stride 8 g with g + 1.
        float u[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            u[j] = (t[j] + t[8 + j]) + (t[4 + j] + t[12 + j]);
        // Stride 4: features j (half 0) + 4 + j (half 1), in both lanes.
        float w4[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
        {
            const float other = __shfl_xor(u[j], 32);
            w4[j] = half ? other + u[j] : u[j] + other; // half 0's value first
        }
        const float sum = (w4[0] + w4[2]) + (w4[1] + w4[3]);
        const float coefficient = 1.f / sqrtf(sum / static_cast<float>(kFeatures) + p.eps);
        const float* const gamma = kind == 0 ? p.gamma_q : p.gamma_k;
        // The token's RoPE coordinates (ct | ch << 8 | cw << 16).
        const uint32_t code = p.text ? static_cast<uint32_t>(min(token, p.m - 1)) * 0x010101u
                                     : p.token_code[min(token, p.m - 1)];
#pragma unroll
        for (int fb = 0; fb < 4; fb++)
#pragma unroll
            for (int i = 0; i < 16; i++)
            {
                const int f = 32 * fb + 8 * (i >> 2) + 4 * half + (i & 3);
                v[fb][i] = round_bf16((v[fb][i] * coefficient) * gamma[f]);
            }
        // Pairs (f, f + 1), f even, below kRopeDim: axis p / 21 of pair p.
#pragma unroll
        for (int fb = 0; fb < 4; fb++)
#pragma unroll
            for (int i = 0; i < 16; i += 2)
            {
                const int f = 32 * fb + 8 * (i >> 2) + 4 * half + (i & 3);
                const int pair = f >> 1;
                if (pair < kRopeDim / 2)
                {
                    const int axis = pair / kRopePairs;
                    const int pp = pair - axis * kRopePairs;
                    const int coord = static_cast<int>((code >> (8 * axis)) & 255u);
                    const float c = p.rope_cs[(coord * kRopePairs + pp) * 2];
                    const float sn = p.rope_cs[(coord * kRopePairs + pp) * 2 + 1];
                    const float x0 = v[fb][i];
                    const float x1 = v[fb][i + 1];
                    v[fb][i] = round_bf16(x0 * c - x1 * sn);
                    v[fb][i + 1] = round_bf16(x1 * c + x0 * sn);
                }
            }
    }
    if (token < p.m)
    {
        uint16_t* const dst = p.y + static_cast<long long>(token) * p.ldy + f0;
#pragma unroll
        for (int fb = 0; fb < 4; fb++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                store4(dst + 32 * fb + 8 * g + 4 * half, v[fb][4 * g], v[fb][4 * g + 1], v[fb][4 * g + 2],
                       v[fb][4 * g + 3]);
    }
}

} // namespace

hipError_t launch_qkv_rope_gemm(const QkvRopeGemm& p, hipStream_t stream)
{
    if (p.m <= 0)
        return hipSuccess;
    if (p.k % (2 * kSlice) || p.ldx % 8 || p.ldw % 8 || p.ldy % 4 || (!p.text && !p.token_code) || p.heads <= 0)
        return hipErrorInvalidValue;
    // 8 * ceil(head blocks / 8) * token blocks workgroups (see the kernel's
    // XCD mapping; the ones past the last head return at once).
    const int blocks_m = (p.m + kTokens - 1) / kTokens;
    const int per_xcd = (3 * p.heads + 7) / 8;
    hipLaunchKernelGGL(qkv_rope_gemm_kernel, dim3(8 * per_xcd * blocks_m), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

} // namespace awa
