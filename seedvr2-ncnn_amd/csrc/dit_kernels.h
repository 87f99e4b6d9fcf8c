// Launch interface of the DiT block's row-wise kernels (gfx950). Pointers
// are device pointers; strides are in elements; activations are fp32
// (elemsize 4) or bf16 (elemsize 2), parameter vectors fp32.
#pragma once

#include <hip/hip_runtime.h>

namespace awa
{

// out = rmsnorm(in) * (emb scale + scale_b) + (emb shift + shift_b), per row
// of `width`; shift_b = scale_b = null skips the modulation.
struct RowNormModulate
{
    const void* in;
    int in_elemsize;
    long long in_stride;
    void* out;
    int out_elemsize;
    long long out_stride;
    int rows, width;
    float eps;
    const void* emb; // [width][2][3]
    int emb_elemsize;
    int layer;       // 0 attn, 1 mlp
    const float* shift_b;
    const float* scale_b;
};

// out = (h + bias) * (emb gate + gate_b) + residual (bias may be null;
// gate_b = null takes the gate as 1).
struct GateResidual
{
    const void* h;
    int h_elemsize;
    long long h_stride;
    const float* bias;
    const void* residual;
    int residual_elemsize;
    long long residual_stride;
    void* out;
    int out_elemsize;
    long long out_stride;
    int rows, width;
    const void* emb;
    int emb_elemsize;
    int layer;
    const float* gate_b;
};

// out[:, c] = silu(in[:, c]) * in[:, width + c].
struct SwiGlu
{
    const void* in;
    int in_elemsize;
    long long in_stride;
    void* out;
    int out_elemsize;
    long long out_stride;
    int rows, width;
};

hipError_t launch_rmsnorm_modulate(const RowNormModulate& p, hipStream_t stream);
hipError_t launch_gate_residual(const GateResidual& p, hipStream_t stream);
hipError_t launch_swiglu(const SwiGlu& p, hipStream_t stream);
hipError_t launch_double(const void* in, int in_elemsize, long long in_stride, void* out, int out_elemsize,
                         long long out_stride, int rows, int width, hipStream_t stream);

} // namespace awa
