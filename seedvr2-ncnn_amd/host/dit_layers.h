// Host-side mirror of the DiT block's mixed-precision layers on the AWA input
// (src/dit/dit_precision.h, src/dit/dit_precision.cpp:22-142, :284-343):
// the same type names, params and checks, over the C ABI of
// include/seedvr2_awa.h.
//
// In a BF16 block the QKV enters the AWA chain as fp32: q and k come out of
// an affine RMSNorm in fp32, v stays bf16 and is promoted exactly by the
// concat (src/dit/dit_precision.cpp:92-94). The fused entry point
// awa_forward_qknorm does the same in one pass; these layers keep the
// reference's per-layer surface for graphs that run them one by one.
#pragma once

#include "awa_layers.h"

// RMSNorm over the row width, ncnn RMSNorm params: 0 = affine_size, 1 = eps,
// 2 = affine. gamma_data holds affine_size fp32 values on the device (the
// weight ncnn's load_model reads from the .bin); the caller sets it before
// upload_model. 1 -> 1: dims-2/3 Mat of width affine_size, fp32 or bf16 as
// the Option's storage says; output fp32 when affine, else the input's type
// (DitRMSNorm::forward, src/dit/dit_precision.cpp:59-86).
class DitRMSNorm final : public seedvr2::hip::Layer
{
public:
    DitRMSNorm();
    int load_param(const seedvr2::hip::ParamDict& pd) override;
    int upload_model(const seedvr2::hip::Option& opt) override;
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;

    int affine_size = 0;
    float eps = 0.001f;
    int affine = 1;
    seedvr2::hip::Mat gamma_data;

private:
    bool uploaded_ = false;
};

// Concat along axis 1 (heads) of q, k (fp32) and v (fp32 or bf16), each
// Mat(d, H, N), into fp32 Mat(d, 3H, N); param 0 = axis, which must be 1
// (DitQKVConcat, src/dit/dit_precision.cpp:95-137). 3 -> 1.
class DitQKVConcat final : public seedvr2::hip::Layer
{
public:
    DitQKVConcat();
    int load_param(const seedvr2::hip::ParamDict& pd) override;
    int create_pipeline(const seedvr2::hip::Option& opt) override;
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;

    int axis = 0;
};

namespace seedvr2
{

// Registers DitRMSNorm as "RMSNorm" and DitQKVConcat as "Concat", overriding
// the stock types for a DiT block graph (register_dit_block_precision_layers,
// src/dit/dit_precision.cpp:284-290). The Ada parameter sums (MemoryData,
// BinaryOp) belong to the block's modulation and MLP, which
// awa_dit_block_forward runs fused.
void register_dit_block_precision_layers(hip::Net& net);

// What configure_dit_block_precision_layers found in a loaded block graph.
struct DitBlockPrecision
{
    int sums = 0;    // BinaryOps fed by an Ada parameter: their output stays fp32
    int gemms = 0;   // Gemm layers
    int swishes = 0; // Swish layers (SwiGLU)
    std::vector<std::string> fp32_layers; // layers given featmask bit 2 (fp32 storage)
    std::vector<std::string> fp32_sums;   // BinaryOps with fp32 output
};

// configure_dit_block_precision_layers (src/dit/dit_precision.cpp:295-343):
// follows the Ada parameter views of a loaded block graph (MemoryData named
// constant_p_ada_*, then the Reshape / Split layers viewing them), sets
// featmask bit 2 on those views and on SeedVR2AWAPack (its QKV is promoted
// fp32), marks the BinaryOps that read a parameter as fp32-output sums, and
// counts Gemm and Swish layers. True for a paired block (12 sums, 10 Gemms,
// 2 Swishes) or the video-only last block (6, 7, 1).
bool configure_dit_block_precision_layers(hip::Net& net, DitBlockPrecision* found = nullptr);

} // namespace seedvr2
