// Launch interface of the DiT block's row-wise kernels (gfx950). Pointers
// are device pointers; strides are in elements; activations are fp32
// (elemsize 4) or bf16 (elemsize 2), parameter vectors fp32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace awa
{

// ada[r][c] = emb[c][r / 3][r % 3] + learned[r][c] for the 6 rows (attn
// shift, scale, gate, mlp shift, scale, gate) of one branch: the Ada vectors
// the row kernels below read.
hipError_t launch_ada_prepare(const void* emb, int emb_elemsize, const float* learned, float* ada, int width,
                              hipStream_t stream);

// out = rmsnorm(in) * scale + shift, per row of `width`; scale = shift = null
// skips the modulation.
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
    const float* shift;
    const float* scale;
};

// out = (h + bias) * gate + residual (bias may be null; gate = null takes it as 1).
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
    const float* gate;
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
