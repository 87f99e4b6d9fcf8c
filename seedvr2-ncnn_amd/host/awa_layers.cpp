// C++ operator surface of the AWA path over the C ABI (see awa_layers.h).
// Layer semantics follow src/awa/awa_layers.cpp: params (:90-114, :867-874),
// construction flags (:363-373, :581-590, :849-858, :1028-1037), registration
// (:1237-1291); the device work is the C ABI's.
#include "awa_layers.h"

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <limits>
#include <sstream>
#include <string>

namespace seedvr2
{

bool AwaRuntimeSpec::valid() const
{
    const long long computed = static_cast<long long>(source_t) * source_h * source_w;
    return source_t > 0 && source_h > 0 && source_w > 0 && video_tokens > 0 && computed == video_tokens &&
           computed <= std::numeric_limits<int>::max();
}

std::vector<AwaWindow> make_awa_windows(int source_t, int source_h, int source_w, int windows_t, int windows_h,
                                        int windows_w, bool shifted)
{
    awa_plan_desc desc{};
    desc.source_t = source_t;
    desc.source_h = source_h;
    desc.source_w = source_w;
    desc.windows_t = windows_t;
    desc.windows_h = windows_h;
    desc.windows_w = windows_w;
    desc.text_tokens = 1; // the partition does not depend on the text length
    desc.shifted = shifted ? 1 : 0;
    desc.rope_dim = 126;
    if (source_t <= 0 || source_h <= 0 || source_w <= 0)
        return {};
    awa_plan* plan = nullptr;
    if (awa_plan_create(&desc, &plan) != AWA_OK)
        return {};
    awa_plan_info info{};
    std::vector<AwaWindow> result;
    if (awa_plan_info_get(plan, &info) == AWA_OK)
    {
        std::vector<int> boxes(static_cast<size_t>(info.window_count) * 6);
        if (awa_plan_windows(plan, boxes.data()) == AWA_OK)
            for (int i = 0; i < info.window_count; i++)
            {
                const int* b = &boxes[static_cast<size_t>(i) * 6];
                result.push_back({b[0], b[1], b[2], b[3], b[4], b[5]});
            }
    }
    awa_plan_destroy(plan);
    return result;
}

namespace hip
{

namespace
{

class DeviceAllocator final : public Allocator
{
public:
    void* fastMalloc(size_t size) override
    {
        void* ptr = nullptr;
        return awa_malloc(&ptr, size) == AWA_OK ? ptr : nullptr;
    }
    void fastFree(void* ptr) override { awa_free(ptr); }
};

long long align16_elements(long long elements, size_t elemsize)
{
    const long long bytes = elements * static_cast<long long>(elemsize);
    return ((bytes + 15) / 16 * 16) / static_cast<long long>(elemsize);
}

} // namespace

Allocator* default_device_allocator()
{
    static DeviceAllocator allocator;
    return &allocator;
}

int Mat::allocate(Allocator* allocator)
{
    Allocator* a = allocator ? allocator : default_device_allocator();
    const size_t bytes = static_cast<size_t>(total()) * elemsize;
    void* ptr = bytes ? a->fastMalloc(bytes) : nullptr;
    if (bytes && !ptr)
    {
        release();
        return AWA_ERR_ALLOC;
    }
    storage_ = std::shared_ptr<void>(ptr, [a](void* p) {
        if (p)
            a->fastFree(p);
    });
    data = ptr;
    return AWA_OK;
}

int Mat::create(int w_, size_t elemsize_, Allocator* allocator)
{
    release();
    dims = 1;
    w = w_;
    h = d = c = n = 1;
    elemsize = elemsize_;
    cstep = nstep = w_;
    return allocate(allocator);
}

int Mat::create(int w_, int h_, size_t elemsize_, Allocator* allocator)
{
    release();
    dims = 2;
    w = w_;
    h = h_;
    d = c = n = 1;
    elemsize = elemsize_;
    cstep = nstep = static_cast<long long>(w_) * h_;
    return allocate(allocator);
}

int Mat::create(int w_, int h_, int c_, size_t elemsize_, Allocator* allocator, int n_)
{
    release();
    dims = 3;
    w = w_;
    h = h_;
    d = 1;
    c = c_;
    n = n_;
    elemsize = elemsize_;
    cstep = align16_elements(static_cast<long long>(w_) * h_, elemsize_);
    // Batches of the NCNN_BATCH layout start on 4 KiB boundaries (src/awa/awa_layers.cpp:537-539).
    nstep = n_ > 1 ? (static_cast<long long>((cstep * c_ * static_cast<long long>(elemsize_) + 4095) / 4096 * 4096) /
                      static_cast<long long>(elemsize_))
                   : cstep * c_;
    return allocate(allocator);
}

int Mat::create_4d(int w_, int h_, int d_, int c_, size_t elemsize_, Allocator* allocator, int n_)
{
    release();
    dims = 4;
    w = w_;
    h = h_;
    d = d_;
    c = c_;
    n = n_;
    elemsize = elemsize_;
    cstep = align16_elements(static_cast<long long>(w_) * h_ * d_, elemsize_);
    nstep = n_ > 1 ? (static_cast<long long>((cstep * c_ * static_cast<long long>(elemsize_) + 4095) / 4096 * 4096) /
                      static_cast<long long>(elemsize_))
                   : cstep * c_;
    return allocate(allocator);
}

void Mat::release()
{
    storage_.reset();
    data = nullptr;
    dims = 0;
    w = h = 0;
    d = c = n = 1;
    cstep = nstep = 0;
}

awa_blob Mat::blob() const
{
    awa_blob b{};
    b.data = data;
    b.dims = dims;
    b.w = w;
    b.h = h;
    b.d = d;
    b.c = c;
    b.n = n;
    b.elemsize = static_cast<int>(elemsize);
    b.cstep = cstep;
    b.nstep = nstep;
    return b;
}

Mat Mat::external(const awa_blob& b)
{
    Mat m;
    m.data = b.data;
    m.dims = b.dims;
    m.w = b.w;
    m.h = b.h;
    m.d = b.d;
    m.c = b.c;
    m.n = b.n;
    m.elemsize = static_cast<size_t>(b.elemsize);
    m.cstep = b.cstep;
    m.nstep = b.nstep;
    return m;
}

int ParamDict::get(int id, int default_value) const
{
    const auto it = ints_.find(id);
    return it == ints_.end() ? default_value : it->second;
}

float ParamDict::get(int id, float default_value) const
{
    const auto f = floats_.find(id);
    if (f != floats_.end())
        return f->second;
    const auto i = ints_.find(id);
    return i == ints_.end() ? default_value : static_cast<float>(i->second);
}

void ParamDict::set(int id, int value)
{
    ints_[id] = value;
}

void ParamDict::set(int id, float value)
{
    floats_[id] = value;
}

std::vector<float> ParamDict::get_array(int id) const
{
    const auto it = arrays_.find(id);
    return it == arrays_.end() ? std::vector<float>() : it->second;
}

namespace
{

// Whole-string integer / float parse (no trailing characters).
bool parse_int(const std::string& s, long long& out)
{
    if (s.empty())
        return false;
    char* end = nullptr;
    errno = 0;
    out = std::strtoll(s.c_str(), &end, 10);
    return errno == 0 && end == s.c_str() + s.size();
}

bool parse_float(const std::string& s, float& out)
{
    if (s.empty())
        return false;
    char* end = nullptr;
    errno = 0;
    out = std::strtof(s.c_str(), &end);
    return errno == 0 && end == s.c_str() + s.size();
}

bool is_float_text(const std::string& s)
{
    return s.find_first_of(".eE") != std::string::npos;
}

} // namespace

int ParamDict::load_field(const std::string& field)
{
    const size_t eq = field.find('=');
    long long key = 0;
    if (eq == std::string::npos || !parse_int(field.substr(0, eq), key))
        return -1;
    const std::string value = field.substr(eq + 1);
    if (key <= -23300)
    {
        // Array: -23300 - id = count,v1,...,vcount.
        const int id = static_cast<int>(-23300 - key);
        std::vector<std::string> parts;
        size_t start = 0;
        while (true)
        {
            const size_t comma = value.find(',', start);
            parts.push_back(value.substr(start, comma == std::string::npos ? std::string::npos : comma - start));
            if (comma == std::string::npos)
                break;
            start = comma + 1;
        }
        long long count = 0;
        if (!parse_int(parts[0], count) || count < 0 || static_cast<size_t>(count) + 1 != parts.size())
            return -1;
        std::vector<float> values;
        for (size_t i = 1; i < parts.size(); i++)
        {
            float v = 0.f;
            if (!parse_float(parts[i], v))
                return -1;
            values.push_back(v);
        }
        arrays_[id] = values;
        return 0;
    }
    if (key < 0 || key > 0x7fffffff)
        return -1;
    if (is_float_text(value))
    {
        float v = 0.f;
        if (!parse_float(value, v))
            return -1;
        floats_[static_cast<int>(key)] = v;
        return 0;
    }
    long long v = 0;
    if (!parse_int(value, v) || v < INT32_MIN || v > INT32_MAX)
        return -1;
    ints_[static_cast<int>(key)] = static_cast<int>(v);
    return 0;
}

int Layer::load_param(const ParamDict&)
{
    return 0;
}

int Layer::upload_model(const Option&)
{
    return 0;
}

int Layer::create_pipeline(const Option&)
{
    return 0;
}

int Layer::destroy_pipeline(const Option&)
{
    return 0;
}

int Layer::forward(const std::vector<Mat>&, std::vector<Mat>&, const Option&) const
{
    return -1;
}

int Net::register_custom_layer(const char* type, layer_creator_func creator, layer_destroyer_func, void* userdata)
{
    if (!type || !creator)
        return -1;
    registry_[type] = Entry{creator, userdata};
    return 0;
}

std::unique_ptr<Layer> Net::create_custom_layer(const char* type) const
{
    const auto it = type ? registry_.find(type) : registry_.end();
    if (it == registry_.end())
        return nullptr;
    return std::unique_ptr<Layer>(it->second.creator(it->second.userdata));
}

std::vector<std::string> Net::custom_layer_types() const
{
    std::vector<std::string> types;
    for (const auto& kv : registry_)
        types.push_back(kv.first);
    return types;
}

int Net::load_param(const char* path)
{
    std::ifstream in(path ? path : "");
    if (!in)
    {
        error_ = std::string("cannot open ") + (path ? path : "(null)");
        return -1;
    }
    std::stringstream text;
    text << in.rdbuf();
    return load_param_mem(text.str().c_str());
}

int Net::load_param_mem(const char* text)
{
    layers_.clear();
    blob_count_ = 0;
    auto fail_load = [&](const std::string& message) {
        layers_.clear();
        blob_count_ = 0;
        error_ = message;
        return -1;
    };
    if (!text)
        return fail_load("null text");
    std::istringstream lines(text);
    std::string line;
    if (!std::getline(lines, line) || line.substr(0, line.find_first_of(" \t\r")) != "7767517")
        return fail_load("not an ncnn param file (magic 7767517 expected)");
    long long layer_count = 0, blob_count = 0;
    {
        if (!std::getline(lines, line))
            return fail_load("missing layer and blob counts");
        std::istringstream counts(line);
        std::string a, b, extra;
        if (!(counts >> a >> b) || (counts >> extra) || !parse_int(a, layer_count) || !parse_int(b, blob_count) ||
            layer_count <= 0 || blob_count <= 0)
            return fail_load("invalid layer and blob counts: " + line);
    }
    std::map<std::string, int> produced;
    while (std::getline(lines, line))
    {
        std::istringstream fields(line);
        std::vector<std::string> f;
        for (std::string tok; fields >> tok;)
            f.push_back(tok);
        if (f.empty())
            continue;
        long long nb = 0, nt = 0;
        if (f.size() < 4 || !parse_int(f[2], nb) || !parse_int(f[3], nt) || nb < 0 || nt < 0 ||
            f.size() < 4 + static_cast<size_t>(nb + nt))
            return fail_load("invalid layer line: " + line);
        ParamLayer l;
        l.type = f[0];
        l.name = f[1];
        l.bottoms.assign(f.begin() + 4, f.begin() + 4 + nb);
        l.tops.assign(f.begin() + 4 + nb, f.begin() + 4 + nb + nt);
        for (size_t i = 4 + nb + nt; i < f.size(); i++)
            if (l.pd.load_field(f[i]) != 0)
                return fail_load("invalid parameter " + f[i] + " in layer " + l.name);
        l.featmask = l.pd.get(31, 0);
        for (const std::string& top : l.tops)
            if (!produced.emplace(top, 1).second)
                return fail_load("blob " + top + " produced twice");
        if (registry_.count(l.type))
        {
            l.layer = create_custom_layer(l.type.c_str());
            if (!l.layer || l.layer->load_param(l.pd) != 0)
                return fail_load("load_param failed for layer " + l.name + " (" + l.type + ")");
        }
        layers_.push_back(std::move(l));
    }
    if (static_cast<long long>(layers_.size()) != layer_count)
        return fail_load("layer count " + std::to_string(layer_count) + " but " + std::to_string(layers_.size()) +
                         " layer lines");
    if (static_cast<long long>(produced.size()) > blob_count)
        return fail_load("more blobs produced than the declared blob count");
    blob_count_ = static_cast<int>(blob_count);
    error_.clear();
    return 0;
}

const ParamLayer* Net::find_layer(const std::string& name) const
{
    for (const ParamLayer& l : layers_)
        if (l.name == name)
            return &l;
    return nullptr;
}

int Net::load_model(const Option& opt)
{
    opt_ = opt;
    for (ParamLayer& l : layers_)
        if (l.layer && (l.layer->upload_model(opt) != 0 || l.layer->create_pipeline(opt) != 0))
        {
            error_ = "upload_model / create_pipeline failed for layer " + l.name + " (" + l.type + ")";
            return -1;
        }
    return 0;
}

Extractor Net::create_extractor() const
{
    return Extractor(this);
}

namespace
{

// ncnn Reshape::forward for the shapes a DiT block uses: the output extents
// from params 0 (w), 1 (h), 11 (d), 2 (c), -1 inferred from the element
// count, 0 keeping the input's extent, dims set by the last given param.
// Dense inputs are reshaped in place (a view); inputs with channel or batch
// padding (the NCNN_BATCH video layout) are first copied dense on the device.
int reshape_forward(const ParamDict& pd, const Mat& in, Mat& out, const Option& opt, std::string& error)
{
    constexpr int kUnset = -233;
    const long long plane = static_cast<long long>(in.w) * in.h * in.d;
    const long long total = plane * in.c * in.n;
    int ext[4] = {pd.get(0, kUnset), pd.get(1, kUnset), pd.get(11, kUnset), pd.get(2, kUnset)}; // w h d c
    const int dims = ext[2] != kUnset ? 4 : ext[3] != kUnset ? 3 : ext[1] != kUnset ? 2 : 1;
    const int in_ext[4] = {in.w, in.h, in.d, in.c};
    const int used[4] = {1, dims >= 2, dims == 4, dims >= 3};
    long long known = 1;
    int infer = -1;
    for (int i = 0; i < 4; i++)
    {
        if (!used[i])
        {
            ext[i] = 1;
            continue;
        }
        if (ext[i] == 0)
            ext[i] = in_ext[i];
        if (ext[i] == -1)
        {
            if (infer >= 0)
            {
                error = "Reshape with more than one -1 extent";
                return -1;
            }
            infer = i;
            continue;
        }
        if (ext[i] <= 0)
        {
            error = "Reshape extent " + std::to_string(ext[i]) + " is invalid";
            return -1;
        }
        known *= ext[i];
    }
    if (infer >= 0)
    {
        if (known == 0 || total % known != 0)
        {
            error = "Reshape cannot infer an extent";
            return -1;
        }
        ext[infer] = static_cast<int>(total / known);
        known *= ext[infer];
    }
    if (known != total)
    {
        error = "Reshape to " + std::to_string(known) + " elements from " + std::to_string(total);
        return -1;
    }
    const long long out_plane = static_cast<long long>(ext[0]) * ext[1] * ext[2];
    if (dims >= 3 && (out_plane * static_cast<long long>(in.elemsize)) % 16 != 0)
    {
        error = "Reshape to a padded channel layout is not supported";
        return -1;
    }
    // A dense copy of the input (same shape, no channel or batch padding).
    Mat dense = in;
    const bool padded = (in.dims >= 3 && in.cstep != plane) || (in.n > 1 && in.nstep != plane * in.c);
    if (padded)
    {
        Mat flat;
        if (flat.create(static_cast<int>(total), in.elemsize, opt.blob_allocator) != 0)
        {
            error = "Reshape copy allocation failed";
            return -100;
        }
        awa_blob dst = in.blob();
        dst.data = flat.data;
        dst.cstep = plane;
        dst.nstep = plane * in.c;
        const awa_blob src = in.blob();
        if (awa_cast(&src, &dst, opt.stream) != AWA_OK)
        {
            error = std::string("Reshape copy: ") + awa_last_error();
            return -1;
        }
        dense = flat;
    }
    out = dense;
    out.dims = dims;
    out.w = ext[0];
    out.h = ext[1];
    out.d = ext[2];
    out.c = ext[3];
    out.n = 1;
    out.cstep = dims >= 3 ? out_plane : out_plane * ext[3];
    out.nstep = out.cstep * ext[3];
    return 0;
}

} // namespace

int Extractor::input(const char* blob_name, const Mat& in)
{
    if (!blob_name || in.empty())
    {
        error_ = "input: null blob name or empty Mat";
        return -1;
    }
    blobs_[blob_name] = in;
    return 0;
}

int Extractor::run(const ParamLayer& l)
{
    std::vector<Mat> bottoms;
    for (const std::string& b : l.bottoms)
    {
        const auto it = blobs_.find(b);
        if (it == blobs_.end())
        {
            error_ = "layer " + l.name + " needs blob " + b + ", which is neither an input nor produced";
            return -1;
        }
        bottoms.push_back(it->second);
    }
    std::vector<Mat> tops;
    int rc = 0;
    if (l.layer)
        rc = l.layer->forward(bottoms, tops, net_->option());
    else if (l.type == "Reshape" && bottoms.size() == 1 && l.tops.size() == 1)
    {
        tops.resize(1);
        rc = reshape_forward(l.pd, bottoms[0], tops[0], net_->option(), error_);
    }
    else if (l.type == "Split" && bottoms.size() == 1)
        tops.assign(l.tops.size(), bottoms[0]);
    else
    {
        error_ = "layer " + l.name + " of type " + l.type + " is not run by this runtime";
        return -1;
    }
    if (rc != 0 || tops.size() != l.tops.size())
    {
        if (error_.empty())
            error_ = "layer " + l.name + " (" + l.type + ") failed: " + std::to_string(rc);
        return rc != 0 ? rc : -1;
    }
    for (size_t i = 0; i < tops.size(); i++)
        blobs_[l.tops[i]] = tops[i];
    return 0;
}

int Extractor::extract(const char* blob_name, Mat& out)
{
    error_.clear();
    if (!blob_name)
    {
        error_ = "extract: null blob name";
        return -1;
    }
    const std::vector<ParamLayer>& layers = net_->layers();
    // The layers the blob depends on, found backwards from its producer.
    std::vector<char> needed(layers.size(), 0);
    std::vector<std::string> wanted{blob_name};
    while (!wanted.empty())
    {
        const std::string b = wanted.back();
        wanted.pop_back();
        if (blobs_.count(b))
            continue;
        bool found = false;
        for (size_t i = 0; i < layers.size() && !found; i++)
            for (const std::string& t : layers[i].tops)
                if (t == b)
                {
                    found = true;
                    if (!needed[i])
                    {
                        needed[i] = 1;
                        wanted.insert(wanted.end(), layers[i].bottoms.begin(), layers[i].bottoms.end());
                    }
                }
        if (!found)
        {
            error_ = "blob " + b + " is not produced by any layer";
            return -1;
        }
    }
    for (size_t i = 0; i < layers.size(); i++)
    {
        if (!needed[i] || std::all_of(layers[i].tops.begin(), layers[i].tops.end(),
                                      [&](const std::string& t) { return blobs_.count(t) != 0; }))
            continue;
        if (layers[i].type == "Input")
        {
            error_ = "input blob " + (layers[i].tops.empty() ? std::string("?") : layers[i].tops[0]) + " was not set";
            return -1;
        }
        const int rc = run(layers[i]);
        if (rc != 0)
            return rc;
    }
    out = blobs_.at(blob_name);
    return 0;
}

} // namespace hip
} // namespace seedvr2

using seedvr2::hip::Mat;
using seedvr2::hip::Option;
using seedvr2::hip::ParamDict;

namespace
{

void report(const char* layer, int rc)
{
    if (rc != AWA_OK)
        std::fprintf(stderr, "%s: %s\n", layer, awa_last_error());
}

} // namespace

SeedVR2AwaLayerBase::SeedVR2AwaLayerBase(const char* type_name, bool reads_rope_dim) : reads_rope_dim_(reads_rope_dim)
{
    type = type_name;
    one_blob_only = false;
    support_inplace = false;
}

SeedVR2AwaLayerBase::SeedVR2AwaLayerBase(const char* type_name, bool reads_rope_dim,
                                         const seedvr2::AwaRuntimeSpec& spec)
    : SeedVR2AwaLayerBase(type_name, reads_rope_dim)
{
    has_runtime_spec_ = true;
    runtime_spec_ = spec;
}

SeedVR2AwaLayerBase::~SeedVR2AwaLayerBase()
{
    awa_plan_destroy(plan_);
}

int SeedVR2AwaLayerBase::load_param(const ParamDict& pd)
{
    awa_plan_destroy(plan_);
    plan_ = nullptr;
    uploaded_ = false;
    awa_plan_desc desc{};
    desc.source_t = pd.get(0, 0);
    desc.source_h = pd.get(1, 0);
    desc.source_w = pd.get(2, 0);
    desc.windows_t = pd.get(3, 0);
    desc.windows_h = pd.get(4, 0);
    desc.windows_w = pd.get(5, 0);
    desc.text_tokens = pd.get(6, 0);
    desc.shifted = pd.get(7, 0) != 0 ? 1 : 0;
    // Only the MMRoPE layer reads param 8 (src/awa/awa_layers.cpp:872); the
    // others build their maps with the default.
    desc.rope_dim = reads_rope_dim_ ? pd.get(8, 126) : 126;
    if (has_runtime_spec_)
    {
        desc.runtime_t = runtime_spec_.source_t;
        desc.runtime_h = runtime_spec_.source_h;
        desc.runtime_w = runtime_spec_.source_w;
        desc.runtime_tokens = runtime_spec_.video_tokens;
    }
    const int rc = awa_plan_create(&desc, &plan_);
    if (rc != AWA_OK)
    {
        plan_ = nullptr;
        return rc;
    }
    return awa_plan_info_get(plan_, &info_);
}

int SeedVR2AwaLayerBase::upload_model(const Option& opt)
{
    if (!plan_)
        return -1;
    const int rc = awa_plan_upload(plan_, opt.stream);
    report(type.c_str(), rc);
    uploaded_ = rc == AWA_OK;
    return rc;
}

int SeedVR2AwaLayerBase::destroy_pipeline(const Option&)
{
    awa_plan_destroy(plan_);
    plan_ = nullptr;
    uploaded_ = false;
    return 0;
}

int SeedVR2AwaLayerBase::require_uploaded() const
{
    if (!plan_ || !uploaded_)
    {
        std::fprintf(stderr, "%s: forward before load_param/upload_model\n", type.c_str());
        return -1;
    }
    return 0;
}

SeedVR2AWAPack::SeedVR2AWAPack() : SeedVR2AwaLayerBase("SeedVR2AWAPack", false)
{
    support_batch = true;
}

SeedVR2AWAPack::SeedVR2AWAPack(const seedvr2::AwaRuntimeSpec& spec) : SeedVR2AwaLayerBase("SeedVR2AWAPack", false, spec)
{
    support_batch = true;
}

int SeedVR2AWAPack::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                            const Option& opt) const
{
    if (require_uploaded() != 0)
        return -1;
    if (bottom_blobs.size() != 2)
        return -1;
    const awa_blob video = bottom_blobs[0].blob();
    const awa_blob text = bottom_blobs[1].blob();
    int heads = 0, head_dim = 0;
    int rc = awa_qkv_shape(&video, info_.source_tokens, &heads, &head_dim);
    if (rc != AWA_OK)
    {
        report(type.c_str(), rc);
        return rc;
    }
    top_blobs.resize(2);
    if (top_blobs[0].create(head_dim, 3 * heads, info_.sequence_tokens, 4, opt.blob_allocator) != AWA_OK ||
        top_blobs[1].create(info_.window_count + 1, 4, opt.blob_allocator) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob packed = top_blobs[0].blob();
    const awa_blob cu = top_blobs[1].blob();
    rc = awa_pack(plan_, &video, &text, &packed, &cu, opt.stream);
    report(type.c_str(), rc);
    return rc;
}

SeedVR2MMRoPE::SeedVR2MMRoPE() : SeedVR2AwaLayerBase("SeedVR2MMRoPE", true)
{
}

SeedVR2MMRoPE::SeedVR2MMRoPE(const seedvr2::AwaRuntimeSpec& spec) : SeedVR2AwaLayerBase("SeedVR2MMRoPE", true, spec)
{
}

int SeedVR2MMRoPE::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                           const Option& opt) const
{
    if (require_uploaded() != 0 || bottom_blobs.size() != 1)
        return -1;
    const Mat& in = bottom_blobs[0];
    top_blobs.resize(1);
    if (top_blobs[0].create(in.w, in.h, in.c, 4, opt.blob_allocator) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob a = in.blob();
    const awa_blob b = top_blobs[0].blob();
    const int rc = awa_mmrope(plan_, &a, &b, opt.stream);
    report(type.c_str(), rc);
    return rc;
}

SeedVR2WindowAttention::SeedVR2WindowAttention() : SeedVR2AwaLayerBase("SeedVR2WindowAttention", false)
{
}

SeedVR2WindowAttention::SeedVR2WindowAttention(const seedvr2::AwaRuntimeSpec& spec)
    : SeedVR2AwaLayerBase("SeedVR2WindowAttention", false, spec)
{
}

int SeedVR2WindowAttention::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                                    const Option& opt) const
{
    if (require_uploaded() != 0 || bottom_blobs.size() != 1)
        return -1;
    const Mat& in = bottom_blobs[0];
    if (in.dims != 3 || in.h % 3 != 0)
        return -1;
    top_blobs.resize(1);
    if (top_blobs[0].create(in.w, in.h / 3, in.c, 4, opt.blob_allocator) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob a = in.blob();
    const awa_blob b = top_blobs[0].blob();
    const int rc = awa_window_attention(plan_, &a, &b, opt.use_bf16_storage ? AWA_COMPUTE_BF16 : AWA_COMPUTE_F32,
                                        opt.stream);
    report(type.c_str(), rc);
    return rc;
}

SeedVR2AWAUnpack::SeedVR2AWAUnpack() : SeedVR2AwaLayerBase("SeedVR2AWAUnpack", false)
{
}

SeedVR2AWAUnpack::SeedVR2AWAUnpack(const seedvr2::AwaRuntimeSpec& spec)
    : SeedVR2AwaLayerBase("SeedVR2AWAUnpack", false, spec)
{
}

namespace
{

// Video and text outputs of Unpack (src/awa/awa_layers.cpp:638-689, :743-846).
int create_unpack_outputs(const awa_plan_info& info, int heads, int head_dim, const Option& opt,
                          std::vector<Mat>& top_blobs)
{
    const size_t elemsize = opt.use_bf16_storage ? 2 : 4;
    top_blobs.resize(2);
    int rc = opt.use_batch_video_layout
                 ? top_blobs[0].create_4d(head_dim, heads, info.source_w, info.source_h, elemsize, opt.blob_allocator,
                                          info.source_t)
                 : top_blobs[0].create(head_dim, heads, info.source_tokens, elemsize, opt.blob_allocator);
    if (rc == AWA_OK)
        rc = top_blobs[1].create(head_dim, heads, info.text_tokens, elemsize, opt.blob_allocator);
    return rc;
}

} // namespace

int SeedVR2AWAUnpack::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                              const Option& opt) const
{
    if (require_uploaded() != 0 || bottom_blobs.size() != 1)
        return -1;
    const Mat& in = bottom_blobs[0];
    if (in.dims != 3)
        return -1;
    if (create_unpack_outputs(info_, in.h, in.w, opt, top_blobs) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob a = in.blob();
    const awa_blob v = top_blobs[0].blob();
    const awa_blob t = top_blobs[1].blob();
    const int rc = awa_unpack(plan_, &a, &v, &t, opt.stream);
    report(type.c_str(), rc);
    return rc;
}

int seedvr2_awa_forward_chain(const SeedVR2AWAPack& pack, const SeedVR2AWAUnpack& unpack,
                              const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs, const Option& opt)
{
    const awa_plan* p = pack.plan();
    const awa_plan* u = unpack.plan();
    if (!p || !u || bottom_blobs.size() != 2)
        return -1;
    awa_plan_info pi{}, ui{};
    awa_plan_info_get(p, &pi);
    awa_plan_info_get(u, &ui);
    if (pi.source_t != ui.source_t || pi.source_h != ui.source_h || pi.source_w != ui.source_w ||
        pi.window_count != ui.window_count || pi.sequence_tokens != ui.sequence_tokens || pi.shifted != ui.shifted ||
        pi.text_tokens != ui.text_tokens)
        return -1;
    const awa_blob video = bottom_blobs[0].blob();
    const awa_blob text = bottom_blobs[1].blob();
    int heads = 0, head_dim = 0;
    int rc = awa_qkv_shape(&video, pi.source_tokens, &heads, &head_dim);
    if (rc != AWA_OK)
        return rc;
    if (create_unpack_outputs(pi, heads, head_dim, opt, top_blobs) != AWA_OK)
        return AWA_ERR_ALLOC;
    const awa_blob v = top_blobs[0].blob();
    const awa_blob t = top_blobs[1].blob();
    rc = awa_forward(p, &video, &text, &v, &t, opt.use_bf16_storage ? AWA_COMPUTE_BF16 : AWA_COMPUTE_F32, opt.stream);
    report("SeedVR2AWA fused chain", rc);
    return rc;
}

namespace
{

template <class T>
seedvr2::hip::Layer* create_layer(void* userdata)
{
    const auto* spec = static_cast<const seedvr2::AwaRuntimeSpec*>(userdata);
    return spec ? new T(*spec) : new T();
}

} // namespace

void register_seedvr2_awa_layers(seedvr2::hip::Net& net)
{
    register_seedvr2_awa_layers(net, nullptr);
}

void register_seedvr2_awa_layers(seedvr2::hip::Net& net, const seedvr2::AwaRuntimeSpec* runtime_spec)
{
    void* userdata = const_cast<seedvr2::AwaRuntimeSpec*>(runtime_spec);
    net.register_custom_layer("SeedVR2AWAPack", create_layer<SeedVR2AWAPack>, nullptr, userdata);
    net.register_custom_layer("SeedVR2AWAUnpack", create_layer<SeedVR2AWAUnpack>, nullptr, userdata);
    net.register_custom_layer("SeedVR2MMRoPE", create_layer<SeedVR2MMRoPE>, nullptr, userdata);
    net.register_custom_layer("SeedVR2WindowAttention", create_layer<SeedVR2WindowAttention>, nullptr, userdata);
}
