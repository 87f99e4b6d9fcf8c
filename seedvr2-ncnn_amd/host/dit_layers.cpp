// Host-side mirror of the DiT mixed-precision layers on the AWA input
// (src/dit/dit_precision.cpp:22-142, :284-343) over the C ABI.
#include "dit_layers.h"

#include <cstdio>
#include <set>

using seedvr2::hip::Layer;
using seedvr2::hip::Mat;
using seedvr2::hip::Net;
using seedvr2::hip::Option;
using seedvr2::hip::ParamDict;
using seedvr2::hip::ParamLayer;

namespace
{

int report_failure(const char* type, int rc)
{
    if (rc != AWA_OK)
        std::fprintf(stderr, "%s: %s\n", type, awa_last_error());
    return rc;
}

} // namespace

DitRMSNorm::DitRMSNorm()
{
    type = "RMSNorm";
    one_blob_only = true;
    support_inplace = false;
}

int DitRMSNorm::load_param(const ParamDict& pd)
{
    // ncnn RMSNorm::load_param: 0 = affine_size, 1 = eps, 2 = affine.
    affine_size = pd.get(0, 0);
    eps = pd.get(1, 0.001f);
    affine = pd.get(2, 1);
    uploaded_ = false;
    return affine_size > 0 && eps >= 0.f ? 0 : -1;
}

int DitRMSNorm::upload_model(const Option&)
{
    // The gamma stays fp32 whatever the block's storage (dit_precision.cpp:48-56).
    if (affine && (gamma_data.empty() || gamma_data.elemsize != 4 || gamma_data.total() < affine_size))
    {
        std::fprintf(stderr, "RMSNorm: affine needs %d fp32 gamma values\n", affine_size);
        return -1;
    }
    uploaded_ = true;
    return 0;
}

int DitRMSNorm::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs, const Option& opt) const
{
    // Fixed DiT graphs normalise the last dimension (dit_precision.cpp:62-68).
    const size_t scalar_size = opt.use_bf16_storage ? 2 : 4;
    if (!uploaded_ || bottom_blobs.size() != 1)
        return -1;
    const Mat& in = bottom_blobs[0];
    if (in.w != affine_size || in.n != 1 || (in.dims != 2 && in.dims != 3) || in.elemsize != scalar_size)
    {
        std::fprintf(stderr, "RMSNorm: unsupported input %d:%dx%dx%d elemsize %zu\n", in.dims, in.w, in.h, in.c,
                     in.elemsize);
        return -1;
    }
    top_blobs.resize(1);
    const size_t out_size = affine ? 4 : in.elemsize;
    const int rc = in.dims == 2 ? top_blobs[0].create(in.w, in.h, out_size, opt.blob_allocator)
                                : top_blobs[0].create(in.w, in.h, in.c, out_size, opt.blob_allocator);
    if (rc != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob a = in.blob();
    const awa_blob b = top_blobs[0].blob();
    return report_failure("RMSNorm", awa_rmsnorm(&a, affine ? static_cast<const float*>(gamma_data.data) : nullptr,
                                                 eps, &b, opt.stream));
}

DitQKVConcat::DitQKVConcat()
{
    type = "Concat";
}

int DitQKVConcat::load_param(const ParamDict& pd)
{
    axis = pd.get(0, 0); // ncnn Concat: 0 = axis
    return 0;
}

int DitQKVConcat::create_pipeline(const Option&)
{
    return axis == 1 ? 0 : -1; // the heads axis of Mat(d, H, N) (dit_precision.cpp:100)
}

int DitQKVConcat::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs, const Option& opt) const
{
    if (axis != 1 || bottom_blobs.size() != 3)
        return -1;
    const Mat& q = bottom_blobs[0];
    for (const Mat& m : bottom_blobs)
        if (m.dims != 3 || m.n != 1 || m.w != q.w || m.h != q.h || m.c != q.c)
            return -1;
    if (q.elemsize != 4 || bottom_blobs[1].elemsize != 4 ||
        (bottom_blobs[2].elemsize != 2 && bottom_blobs[2].elemsize != 4))
        return -1;
    top_blobs.resize(1);
    if (top_blobs[0].create(q.w, 3 * q.h, q.c, 4, opt.blob_allocator) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob bq = q.blob(), bk = bottom_blobs[1].blob(), bv = bottom_blobs[2].blob();
    const awa_blob out = top_blobs[0].blob();
    return report_failure("Concat", awa_qkv_concat(&bq, &bk, &bv, &out, opt.stream));
}

namespace seedvr2
{

namespace
{

Layer* create_rmsnorm(void*)
{
    return new DitRMSNorm;
}

Layer* create_qkv_concat(void*)
{
    return new DitQKVConcat;
}

} // namespace

void register_dit_block_precision_layers(hip::Net& net)
{
    net.register_custom_layer("RMSNorm", create_rmsnorm);
    net.register_custom_layer("Concat", create_qkv_concat);
}

bool configure_dit_block_precision_layers(hip::Net& net, DitBlockPrecision* found)
{
    DitBlockPrecision r;
    std::set<std::string> parameters; // blobs carrying fp32 Ada parameters
    for (ParamLayer& layer : net.mutable_layers())
    {
        if (layer.type == "Gemm")
            r.gemms++;
        else if (layer.type == "Swish")
            r.swishes++;
        if (layer.type == "SeedVR2AWAPack")
        {
            layer.featmask |= 1 << 2; // promoted fp32 QKV
            r.fp32_layers.push_back(layer.name);
        }
        if (layer.type == "MemoryData" && layer.name.rfind("constant_p_ada_", 0) == 0)
        {
            parameters.insert(layer.tops.begin(), layer.tops.end());
        }
        else if ((layer.type == "Reshape" || layer.type == "Split") && !layer.bottoms.empty() &&
                 parameters.count(layer.bottoms[0]))
        {
            // Views of an fp32 parameter in a BF16 graph keep its type.
            layer.featmask |= 1 << 2;
            r.fp32_layers.push_back(layer.name);
            parameters.insert(layer.tops.begin(), layer.tops.end());
        }
        else if (layer.type == "BinaryOp")
        {
            bool fp32_output = false;
            for (const std::string& bottom : layer.bottoms)
                fp32_output = fp32_output || parameters.count(bottom) != 0;
            if (fp32_output)
            {
                r.sums++;
                r.fp32_sums.push_back(layer.name);
            }
        }
    }
    if (found)
        *found = r;
    if (r.sums != 6 && r.sums != 12)
        return false;
    return (r.sums == 12 && r.gemms == 10 && r.swishes == 2) || (r.sums == 6 && r.gemms == 7 && r.swishes == 1);
}

} // namespace seedvr2
