// Row-wise kernels of the DiT block around the AWA layer (gfx950): the
// RMSNorm + Ada modulation feeding a GEMM, the bias + Ada gate + residual
// after one, and the SwiGLU between the MLP GEMMs. Activations are fp32 or
// bf16 (round to nearest even on store); arithmetic is fp32.
//
// Ada modulation (tools/reference/dit_block.py:166-181): the block embedding
// emb[hidden * 6] is read as [c][layer][k] with layer 0 = attn, 1 = mlp and
// k = 0 shift, 1 scale, 2 gate; each branch adds its own learned vectors.
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

// y = rmsnorm(x) * (scale_a + scale_b) + (shift_a + shift_b), one workgroup per row.
__global__ __launch_bounds__(kRowThreads) void rmsnorm_modulate_kernel(const RowNormModulate p)
{
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const void* x = p.in;
    const long long base_in = row * p.in_stride;
    float ss = 0.f;
    for (int c = threadIdx.x; c < p.width; c += kRowThreads)
    {
        const float v = load_act(x, base_in + c, p.in_elemsize);
        ss = fmaf(v, v, ss);
    }
    const float mean = block_sum(ss, red) / static_cast<float>(p.width);
    const float inv = 1.f / sqrtf(mean + p.eps);
    const long long base_out = row * p.out_stride;
    for (int c = threadIdx.x; c < p.width; c += kRowThreads)
    {
        const float v = load_act(x, base_in + c, p.in_elemsize) * inv;
        if (!p.shift_b)
        {
            store_act(p.out, base_out + c, p.out_elemsize, v); // no Ada modulation
            continue;
        }
        const long long e = static_cast<long long>(c) * 6 + p.layer * 3;
        const float shift = load_act(p.emb, e + 0, p.emb_elemsize) + p.shift_b[c];
        const float scale = load_act(p.emb, e + 1, p.emb_elemsize) + p.scale_b[c];
        store_act(p.out, base_out + c, p.out_elemsize, v * scale + shift);
    }
}

// out = (h + bias) * (gate_a + gate_b) + residual; elementwise.
__global__ __launch_bounds__(kRowThreads) void gate_residual_kernel(const GateResidual p)
{
    const long long n = static_cast<long long>(p.rows) * p.width;
    for (long long i = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kRowThreads)
    {
        const long long row = i / p.width;
        const int c = static_cast<int>(i - row * p.width);
        float h = load_act(p.h, row * p.h_stride + c, p.h_elemsize);
        if (p.bias)
            h += p.bias[c];
        const float gate =
            p.gate_b ? load_act(p.emb, static_cast<long long>(c) * 6 + p.layer * 3 + 2, p.emb_elemsize) + p.gate_b[c]
                     : 1.f;
        const float r = load_act(p.residual, row * p.residual_stride + c, p.residual_elemsize);
        store_act(p.out, row * p.out_stride + c, p.out_elemsize, h * gate + r);
    }
}

// out = silu(a) * b with a, b the two halves of one GEMM output row.
__global__ __launch_bounds__(kRowThreads) void swiglu_kernel(const SwiGlu p)
{
    const long long n = static_cast<long long>(p.rows) * p.width;
    for (long long i = static_cast<long long>(blockIdx.x) * kRowThreads + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kRowThreads)
    {
        const long long row = i / p.width;
        const int c = static_cast<int>(i - row * p.width);
        const float a = load_act(p.in, row * p.in_stride + c, p.in_elemsize);
        const float b = load_act(p.in, row * p.in_stride + p.width + c, p.in_elemsize);
        const float silu = a / (1.f + expf(-a));
        store_act(p.out, row * p.out_stride + c, p.out_elemsize, silu * b);
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

hipError_t launch_rmsnorm_modulate(const RowNormModulate& p, hipStream_t stream)
{
    if (p.rows <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_modulate_kernel, dim3(p.rows), dim3(kRowThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_gate_residual(const GateResidual& p, hipStream_t stream)
{
    const long long n = static_cast<long long>(p.rows) * p.width;
    if (n <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(gate_residual_kernel, dim3(elementwise_grid(n)), dim3(kRowThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_swiglu(const SwiGlu& p, hipStream_t stream)
{
    const long long n = static_cast<long long>(p.rows) * p.width;
    if (n <= 0)
        return hipSuccess;
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
