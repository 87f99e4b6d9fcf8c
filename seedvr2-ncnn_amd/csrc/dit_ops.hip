// Row-wise kernels of the DiT block around the AWA layer (gfx950): the
// RMSNorm + Ada modulation feeding a GEMM, the bias + Ada gate + residual
// after one, and the SwiGLU between the MLP GEMMs. Activations are fp32 or
// bf16 (round to nearest even on store); arithmetic is fp32. Widths and row
// strides are multiples of 8 elements and rows 16-byte aligned: every thread
// moves 8 elements with 16-byte (bf16) or 2 x 16-byte (fp32) accesses.
//
// Ada modulation (tools/reference/dit_block.py:166-181): the block embedding
// emb[hidden * 6] is read as [c][layer][k] with layer 0 = attn, 1 = mlp and
// k = 0 shift, 1 scale, 2 gate; each branch adds its own learned vectors
// (ada_prepare_kernel, once per branch and block, so that the row kernels
// read contiguous vectors).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "dit_kernels.h"

namespace awa
{
namespace
{

__device__ __forceinline__ float load_act(const void* p, long long i, int elemsize)
{
    if (elemsize == 2)
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
    return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v)
{
    const uint32_t b = __float_as_uint(v);
    if ((b & 0x7f800000u) == 0x7f800000u) // inf / nan: keep, quiet nan
        return static_cast<uint16_t>((b >> 16) | ((b & 0xffffu) ? 0x40u : 0u));
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ void store_act(void* p, long long i, int elemsize, float v)
{
    if (elemsize == 2)
        static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
    else
        static_cast<float*>(p)[i] = v;
}

constexpr int kRowThreads = 256;

// Sum over the workgroup (256 threads, 4 waves): wave DPP-free shuffle tree,
// then the four wave sums in a fixed order.
__device__ __forceinline__ float block_sum(float v, float* red)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0)
        red[wave] = v;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return total;
}

// Eight consecutive activations (16-byte aligned) in and out.
__device__ __forceinline__ void load8(const void* p, long long i, int elemsize, float (&v)[8])
{
    if (elemsize == 2)
    {
        const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
        {
            v[2 * k] = __uint_as_float(a[k] << 16);
            v[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u);
        }
    }
    else
    {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    }
}

__device__ __forceinline__ void store8(void* p, long long i, int elemsize, const float (&v)[8])
{
    if (elemsize == 2)
    {
        uint32_t a[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            a[k] = static_cast<uint32_t>(f32_to_bf16_rne(v[2 * k])) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(v[2 * k + 1])) << 16);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = make_uint4(a[0], a[1], a[2], a[3]);
    }
    else
    {
        *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(static_cast<float*>(p) + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__device__ __forceinline__ void load8f(const float* p, int i, float (&v)[8])
{
    const float4 a = *reinterpret_cast<const float4*>(p + i);
    const float4 b = *reinterpret_cast<const float4*>(p + i + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// ada[r][c] = emb[c * 6 + r] + learned[r][c] (r = 3 * layer + k).
__global__ __launch_bounds__(kRowThreads) void ada_prepare_kernel(const void* emb, int emb_elemsize,
                                                                  const float* learned, float* ada, int width)
{
    const int i = blockIdx.x * kRowThreads + threadIdx.x;
    if (i >= 6 * width)
        return;
    const int r = i / width;
    const int c = i - r * width;
    ada[i] = load_act(emb, static_cast<long long>(c) * 6 + r, emb_elemsize) + learned[i];
}

constexpr int kRowChunks = 4; // chunks of 8 a thread keeps in registers (rows up to 8192 wide)

// y = rmsnorm(x) * (scale_a + scale_b) + (shift_a + shift_b), one workgroup
// per row; the row stays in registers between the two passes.
__global__ __launch_bounds__(kRowThreads) void rmsnorm_modulate_kernel(const RowNormModulate p)
{
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const int chunks = p.width / 8;
    const long long base_in = row * p.in_stride;
    float v[kRowChunks][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kRowChunks; j++)
    {
        const int ch = threadIdx.x + j * kRowThreads;
        if (ch < chunks)
        {
            load8(p.in, base_in + 8 * ch, p.in_elemsize, v[j]);
#pragma unroll
            for (int e = 0; e < 8; e++)
                ss = fmaf(v[j][e], v[j][e], ss);
        }
    }
    const float mean = block_sum(ss, red) / static_cast<float>(p.width);
    const float inv = 1.f / sqrtf(mean + p.eps);
    const long long base_out = row * p.out_stride;
#pragma unroll
    for (int j = 0; j < kRowChunks; j++)
    {
        const int ch = threadIdx.x + j * kRowThreads;
        if (ch >= chunks)
            continue;
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            y[e] = v[j][e] * inv;
        if (p.shift)
        {
            float shift[8], scale[8];
            load8f(p.shift, 8 * ch, shift);
            load8f(p.scale, 8 * ch, scale);
#pragma unroll
            for (int e = 0; e < 8; e++)
                y[e] = y[e] * scale[e] + shift[e];
        }
        store8(p.out, base_out + 8 * ch, p.out_elemsize, y);
    }
}

// out = (h + bias) * (gate_a + gate_b) + residual; one thread per 8 elements.
__global__ __launch_bounds__(kRowThreads) void gate_residual_kernel(const GateResidual p)
{
    const int chunks = p.width / 8;
    const long long n = static_cast<long long>(p.rows) * chunks;
    for (long long i = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kRowThreads)
    {
        const long long row = i / chunks;
        const int c0 = 8 * static_cast<int>(i - row * chunks);
        float h[8], r[8], bias[8], gate[8];
        load8(p.h, row * p.h_stride + c0, p.h_elemsize, h);
        load8(p.residual, row * p.residual_stride + c0, p.residual_elemsize, r);
#pragma unroll
        for (int e = 0; e < 8; e++)
            bias[e] = 0.f, gate[e] = 1.f;
        if (p.bias)
            load8f(p.bias, c0, bias);
        if (p.gate)
            load8f(p.gate, c0, gate);
#pragma unroll
        for (int e = 0; e < 8; e++)
            h[e] = (h[e] + bias[e]) * gate[e] + r[e];
        store8(p.out, row * p.out_stride + c0, p.out_elemsize, h);
    }
}

// out = silu(a) * b with a, b the two halves of one GEMM output row.
__global__ __launch_bounds__(kRowThreads) void swiglu_kernel(const SwiGlu p)
{
    const int chunks = p.width / 8;
    const long long n = static_cast<long long>(p.rows) * chunks;
    for (long long i = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kRowThreads)
    {
        const long long row = i / chunks;
        const int c0 = 8 * static_cast<int>(i - row * chunks);
        float a[8], b[8];
        load8(p.in, row * p.in_stride + c0, p.in_elemsize, a);
        load8(p.in, row * p.in_stride + p.width + c0, p.in_elemsize, b);
#pragma unroll
        for (int e = 0; e < 8; e++)
            a[e] = a[e] / (1.f + expf(-a[e])) * b[e];
        store8(p.out, row * p.out_stride + c0, p.out_elemsize, a);
    }
}

// out = x + x (the last block's text: its final residual doubles the
// post-attention text, tools/reference/dit_block.py:362-366).
__global__ __launch_bounds__(kRowThreads) void double_kernel(const void* in, int in_elemsize, long long in_stride,
                                                             void* out, int out_elemsize, long long out_stride,
                                                             int rows, int width)
{
    const long long n = static_cast<long long>(rows) * width;
    for (long long i = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kRowThreads)
    {
        const long long row = i / width;
        const int c = static_cast<int>(i - row * width);
        const float v = load_act(in, row * in_stride + c, in_elemsize);
        store_act(out, row * out_stride + c, out_elemsize, v + v);
    }
}

int elementwise_grid(long long n)
{
    const long long blocks = (n + kRowThreads - 1) / kRowThreads;
    return static_cast<int>(blocks < 8192 ? blocks : 8192);
}

} // namespace

hipError_t launch_ada_prepare(const void* emb, int emb_elemsize, const float* learned, float* ada, int width,
                              hipStream_t stream)
{
    if (width <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(ada_prepare_kernel, dim3((6 * width + kRowThreads - 1) / kRowThreads), dim3(kRowThreads), 0,
                       stream, emb, emb_elemsize, learned, ada, width);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_modulate(const RowNormModulate& p, hipStream_t stream)
{
    if (p.rows <= 0)
        return hipSuccess;
    if (p.width % 8 || p.width > 8 * kRowChunks * kRowThreads || p.in_stride % 8 || p.out_stride % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_modulate_kernel, dim3(p.rows), dim3(kRowThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_gate_residual(const GateResidual& p, hipStream_t stream)
{
    const long long n = static_cast<long long>(p.rows) * (p.width / 8);
    if (n <= 0)
        return hipSuccess;
    if (p.width % 8 || p.h_stride % 8 || p.residual_stride % 8 || p.out_stride % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gate_residual_kernel, dim3(elementwise_grid(n)), dim3(kRowThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_swiglu(const SwiGlu& p, hipStream_t stream)
{
    const long long n = static_cast<long long>(p.rows) * (p.width / 8);
    if (n <= 0)
        return hipSuccess;
    if (p.width % 8 || p.in_stride % 8 || p.out_stride % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(swiglu_kernel, dim3(elementwise_grid(n)), dim3(kRowThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_double(const void* in, int in_elemsize, long long in_stride, void* out, int out_elemsize,
                         long long out_stride, int rows, int width, hipStream_t stream)
{
    const long long n = static_cast<long long>(rows) * width;
    if (n <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(double_kernel, dim3(elementwise_grid(n)), dim3(kRowThreads), 0, stream, in, in_elemsize,
                       in_stride, out, out_elemsize, out_stride, rows, width);
    return hipGetLastError();
}

} // namespace awa
