// C++ operator surface of the AWA path, mirroring the reference's ncnn custom
// layers (src/awa/awa_layers.h:19-223): the same four layer type names, the
// same param ids and meanings, the same multi-blob forward signature, the
// same 0 / -1 / -100 return codes and the same registration entry points.
// Blobs live in HIP device memory and forward enqueues on Option::stream;
// every layer reaches the GPU only through the C ABI of seedvr2_awa.h.
//
// ncnn itself is not a dependency: the few ncnn types the layers' interface
// needs (ParamDict, Option, Mat, Layer, Net's custom-layer registry) have
// device-memory counterparts in namespace seedvr2::hip with the same member
// names, so a host that drove the reference layers through ncnn drives these
// with the same calls.
#pragma once

#include <cstddef>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "seedvr2_awa.h"

namespace seedvr2
{

// Half-open window box (src/awa/awa_layers.h:20-28).
struct AwaWindow final
{
    int t0 = 0;
    int t1 = 0;
    int h0 = 0;
    int h1 = 0;
    int w0 = 0;
    int w1 = 0;
};

// Session token grid (src/awa/awa_layers.h:31-39); valid() as at
// src/awa/awa_layers.cpp:340-345.
struct AwaRuntimeSpec final
{
    int source_t = 0;
    int source_h = 0;
    int source_w = 0;
    int video_tokens = 0;

    bool valid() const;
};

// Windows in the layers' order: w outer, h, t inner; empty windows dropped
// (src/awa/awa_layers.cpp:347-359). Returns {} for invalid arguments.
std::vector<AwaWindow> make_awa_windows(int source_t, int source_h, int source_w, int windows_t, int windows_h,
                                        int windows_w, bool shifted);

namespace hip
{

// Device-memory allocator interface (ncnn::Allocator's fastMalloc/fastFree).
class Allocator
{
public:
    virtual ~Allocator() = default;
    virtual void* fastMalloc(size_t size) = 0;
    virtual void fastFree(void* ptr) = 0;
};

// awa_malloc / awa_free on the current device.
Allocator* default_device_allocator();

// Device blob with ncnn Mat geometry (elempack 1): dims 1..4, w fastest,
// cstep aligned to 16 bytes, NCNN_BATCH n / nstep. Storage is shared between
// copies; a Mat made by external() borrows caller memory.
class Mat
{
public:
    void* data = nullptr;
    int dims = 0;
    int w = 0, h = 0, d = 1, c = 1, n = 1;
    size_t elemsize = 4;
    long long cstep = 0;
    long long nstep = 0;

    bool empty() const { return data == nullptr || total() == 0; }
    long long total() const { return nstep * n; }

    // dims 1: Mat(w); dims 2: Mat(w, h); dims 3: Mat(w, h, c); dims 4: Mat(w, h, d, c); n > 1 adds batches.
    int create(int w, size_t elemsize, Allocator* allocator);
    int create(int w, int h, size_t elemsize, Allocator* allocator);
    int create(int w, int h, int c, size_t elemsize, Allocator* allocator, int n = 1);
    int create_4d(int w, int h, int d, int c, size_t elemsize, Allocator* allocator, int n = 1);
    void release();

    awa_blob blob() const;
    static Mat external(const awa_blob& blob);

private:
    std::shared_ptr<void> storage_;
    int allocate(Allocator* allocator);
};

// Parameters by id (ncnn::ParamDict::get / set): integers, floats and
// arrays, as a .param line gives them (`id=int`, `id=float`,
// `-23300-id=n,v1,...,vn`).
class ParamDict
{
public:
    int get(int id, int default_value) const;
    float get(int id, float default_value) const;
    void set(int id, int value);
    void set(int id, float value);
    // Array parameter id, empty when absent.
    std::vector<float> get_array(int id) const;
    // Parses one `key=value` field of a .param layer line; -1 when malformed.
    int load_field(const std::string& field);

private:
    std::map<int, int> ints_;
    std::map<int, float> floats_;
    std::map<int, std::vector<float>> arrays_;
};

// The ncnn::Option fields the AWA layers read, plus the HIP stream.
struct Option
{
    void* stream = nullptr;               // hipStream_t; nullptr = default stream
    bool use_bf16_storage = false;        // BF16 blocks: bf16 Unpack outputs, bf16 MFMA attention
    bool use_batch_video_layout = false;  // Unpack video as NCNN_BATCH Mat(d, H, w, h; n = t)
    Allocator* blob_allocator = nullptr;  // outputs (nullptr = default_device_allocator())
};

class Layer
{
public:
    virtual ~Layer() = default;
    virtual int load_param(const ParamDict& pd);
    virtual int upload_model(const Option& opt);
    virtual int create_pipeline(const Option& opt);
    virtual int destroy_pipeline(const Option& opt);
    virtual int forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                        const Option& opt) const;

    bool one_blob_only = false;
    bool support_inplace = false;
    bool support_batch = false;
    bool support_vulkan = false; // the device path here is HIP; kept false
    std::string type;
};

typedef Layer* (*layer_creator_func)(void* userdata);
typedef void (*layer_destroyer_func)(Layer* layer, void* userdata);

// One layer line of an ncnn .param file.
struct ParamLayer
{
    std::string type, name;
    std::vector<std::string> bottoms, tops;
    ParamDict pd;
    std::unique_ptr<Layer> layer; // registered types only; other types are recorded, not run
    int featmask = 0;             // ncnn Layer::featmask (param 31); bit 2 keeps a layer's storage fp32
};

class Extractor;

// Custom-layer registry with ncnn::Net's register_custom_layer signature, and
// ncnn::Net::load_param for the .param text format the reference's packages
// use (magic 7767517, "layer_count blob_count", then one line per layer:
// type name bottom_count top_count bottoms... tops... params...;
// tools/export_dit_block.py:38-124, :578-644; read by load_graph,
// src/dit/dit_stack.cpp:167-220). Layers of registered types are created and
// given their ParamDict; a layer's load_param failure fails the load.
// load_model then uploads and creates the pipelines of the created layers
// (the AWA layers carry no weights), and create_extractor runs the graph.
class Net
{
public:
    int register_custom_layer(const char* type, layer_creator_func creator, layer_destroyer_func destroyer = nullptr,
                              void* userdata = nullptr);
    // nullptr for an unknown type.
    std::unique_ptr<Layer> create_custom_layer(const char* type) const;
    std::vector<std::string> custom_layer_types() const;

    // 0, or -1 with the message in last_error() (the net is left empty).
    int load_param(const char* path);
    int load_param_mem(const char* text);
    const std::vector<ParamLayer>& layers() const { return layers_; }
    std::vector<ParamLayer>& mutable_layers() { return layers_; }
    const ParamLayer* find_layer(const std::string& name) const;
    int blob_count() const { return blob_count_; }
    const std::string& last_error() const { return error_; }

    // upload_model + create_pipeline of every created layer, with opt as the
    // net's option (ncnn::Net::load_model's role here: no weight file).
    int load_model(const Option& opt);
    const Option& option() const { return opt_; }
    Extractor create_extractor() const;

private:
    struct Entry
    {
        layer_creator_func creator;
        void* userdata;
    };
    std::map<std::string, Entry> registry_;
    std::vector<ParamLayer> layers_;
    int blob_count_ = 0;
    std::string error_;
    Option opt_;
};

// Runs a loaded net the way ncnn::Extractor does: input() binds blobs by
// name (the Input layers' tops), extract() runs the layers the requested blob
// depends on, in file order, and returns it. Runs the created layers,
// ncnn's Reshape (params 0 = w, 1 = h, 11 = d, 2 = c; -1 inferred, 0 keeps
// the input's extent; padded inputs are first copied dense, as ncnn's Reshape
// does with a flattened copy) and Split (every top shares the bottom); a
// needed layer of any other type fails the extraction with -1. Enqueued on
// the net option's stream.
class Extractor
{
public:
    explicit Extractor(const Net* net) : net_(net) {}
    int input(const char* blob_name, const Mat& in);
    int extract(const char* blob_name, Mat& out);
    const std::string& last_error() const { return error_; }

private:
    int run(const ParamLayer& layer);
    const Net* net_;
    std::map<std::string, Mat> blobs_;
    std::string error_;
};

} // namespace hip
} // namespace seedvr2

// Shared base of the four layers: params 0-7 (8 for MMRoPE), an optional
// runtime spec copied at construction, and the plan built in load_param.
class SeedVR2AwaLayerBase : public seedvr2::hip::Layer
{
public:
    ~SeedVR2AwaLayerBase() override;
    int load_param(const seedvr2::hip::ParamDict& pd) override;
    int upload_model(const seedvr2::hip::Option& opt) override;
    int destroy_pipeline(const seedvr2::hip::Option& opt) override;

    const awa_plan* plan() const { return plan_; }

protected:
    SeedVR2AwaLayerBase(const char* type_name, bool reads_rope_dim);
    SeedVR2AwaLayerBase(const char* type_name, bool reads_rope_dim, const seedvr2::AwaRuntimeSpec& spec);
    int require_uploaded() const;

    bool has_runtime_spec_ = false;
    seedvr2::AwaRuntimeSpec runtime_spec_;
    bool reads_rope_dim_ = false;
    awa_plan* plan_ = nullptr;
    awa_plan_info info_{};
    bool uploaded_ = false;
};

// 2 in (video QKV, text QKV) -> 2 out (packed Mat(d, 3H, S) fp32, cu_seqlens Mat(nwin+1) fp32).
class SeedVR2AWAPack final : public SeedVR2AwaLayerBase
{
public:
    SeedVR2AWAPack();
    explicit SeedVR2AWAPack(const seedvr2::AwaRuntimeSpec& runtime_spec);
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;
};

// 1 -> 1: Mat(d, 3H, S) -> fp32 Mat(d, 3H, S) with Q and K rotated.
class SeedVR2MMRoPE final : public SeedVR2AwaLayerBase
{
public:
    SeedVR2MMRoPE();
    explicit SeedVR2MMRoPE(const seedvr2::AwaRuntimeSpec& runtime_spec);
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;
};

// 1 -> 1: Mat(d, 3H, S) -> fp32 Mat(d, H, S).
class SeedVR2WindowAttention final : public SeedVR2AwaLayerBase
{
public:
    SeedVR2WindowAttention();
    explicit SeedVR2WindowAttention(const seedvr2::AwaRuntimeSpec& runtime_spec);
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;
};

// 1 -> 2: Mat(d, H, S) -> video Mat(d, H, N) (or the batch layout), text Mat(d, H, T_x).
class SeedVR2AWAUnpack final : public SeedVR2AwaLayerBase
{
public:
    SeedVR2AWAUnpack();
    explicit SeedVR2AWAUnpack(const seedvr2::AwaRuntimeSpec& runtime_spec);
    int forward(const std::vector<seedvr2::hip::Mat>& bottom_blobs, std::vector<seedvr2::hip::Mat>& top_blobs,
                const seedvr2::hip::Option& opt) const override;
};

// Registers the four type names (src/awa/awa_layers.cpp:1267-1291). With a
// runtime spec, layers created afterwards copy it at construction, so the
// spec only has to outlive the layers' creation.
void register_seedvr2_awa_layers(seedvr2::hip::Net& net);
void register_seedvr2_awa_layers(seedvr2::hip::Net& net, const seedvr2::AwaRuntimeSpec* runtime_spec);

// Runs Pack -> MMRoPE -> WindowAttention -> Unpack as the single fused
// entry point (awa_forward) when the four layers were loaded with the same
// geometry; returns -1 when they were not. Inputs and outputs as the Pack
// layer's bottoms and the Unpack layer's tops.
int seedvr2_awa_forward_chain(const SeedVR2AWAPack& pack, const SeedVR2AWAUnpack& unpack,
                              const std::vector<seedvr2::hip::Mat>& bottom_blobs,
                              std::vector<seedvr2::hip::Mat>& top_blobs, const seedvr2::hip::Option& opt);
