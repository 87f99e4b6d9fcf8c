// Drives the C++ AWA layers (seedvr2-ncnn_amd/host/awa_layers.h) the way a
// host of the reference's ncnn layers does: register, create by type name,
// load_param with the .param ids, upload_model, forward blob vectors.
//
//   awa_layers_check params
//       Host-only checks of registration, params, runtime spec and windows.
//   awa_layers_check param
//       Host-only checks of .param loading: a DiT block's AWA lines in the
//       reference export's format, static and dynamic (-1) grids, and
//       malformed files.
//   awa_layers_check forward OUTDIR t h w nt nh nw text shifted heads bf16
//       Seeded inputs on device 0, the four-layer chain and the fused chain;
//       writes inputs and outputs as float32 files into OUTDIR and prints the
//       largest staged-vs-fused difference.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "awa_layers.h"

using seedvr2::hip::Mat;
using seedvr2::hip::Net;
using seedvr2::hip::Option;
using seedvr2::hip::ParamDict;

namespace
{

int failures = 0;

void expect(bool ok, const char* what)
{
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok)
        failures++;
}

ParamDict params(int t, int h, int w, int nt, int nh, int nw, int text, int shifted)
{
    ParamDict pd;
    const int v[8] = {t, h, w, nt, nh, nw, text, shifted};
    for (int i = 0; i < 8; i++)
        pd.set(i, v[i]);
    return pd;
}

int run_params()
{
    Net net;
    register_seedvr2_awa_layers(net);
    const std::vector<std::string> types = net.custom_layer_types();
    expect(types.size() == 4, "four layer types registered");
    for (const char* name : {"SeedVR2AWAPack", "SeedVR2MMRoPE", "SeedVR2WindowAttention", "SeedVR2AWAUnpack"})
    {
        auto layer = net.create_custom_layer(name);
        expect(layer && layer->type == name, name);
        expect(layer && !layer->one_blob_only && !layer->support_inplace, "multi-blob, not in place");
        expect(layer && layer->load_param(params(9, 16, 16, 3, 8, 8, 64, 1)) == 0, "load_param 9x16x16 shifted");
    }
    expect(net.create_custom_layer("Nope") == nullptr, "unknown type");
    auto pack = net.create_custom_layer("SeedVR2AWAPack");
    expect(pack->load_param(params(-1, -1, -1, 3, 8, 8, 64, 0)) == -1, "-1,-1,-1 without a runtime spec is invalid");
    expect(pack->load_param(params(9, 16, 16, 3, 8, 8, 0, 0)) == -1, "text tokens must be positive");
    expect(pack->load_param(params(9, 16, 16, 0, 8, 8, 64, 0)) == -1, "window counts must be positive");
    expect(pack->load_param(params(9, -1, 16, 3, 8, 8, 64, 0)) == -1, "partial -1 is invalid");
    {
        std::vector<Mat> top;
        expect(pack->forward({}, top, Option()) == -1, "forward before upload fails");
    }
    seedvr2::AwaRuntimeSpec spec{9, 16, 16, 9 * 16 * 16};
    expect(spec.valid(), "runtime spec valid");
    expect(!seedvr2::AwaRuntimeSpec{9, 16, 16, 100}.valid(), "runtime spec token mismatch");
    Net dyn;
    register_seedvr2_awa_layers(dyn, &spec);
    auto dpack = dyn.create_custom_layer("SeedVR2AWAPack");
    spec.source_t = 0; // layers copied the spec at creation
    expect(dpack->load_param(params(-1, -1, -1, 3, 8, 8, 64, 1)) == 0, "dynamic package takes the runtime grid");
    const auto* base = static_cast<const SeedVR2AwaLayerBase*>(dpack.get());
    awa_plan_info info{};
    awa_plan_info_get(base->plan(), &info);
    expect(info.source_t == 9 && info.window_count == 36 && info.sequence_tokens == 4608, "9x16x16 shifted: 36 windows, S 4608");
    auto rope = net.create_custom_layer("SeedVR2MMRoPE");
    ParamDict pd = params(2, 16, 16, 1, 8, 8, 64, 1);
    pd.set(8, 125);
    expect(rope->load_param(pd) == -1, "rope_dim must be a multiple of 6");
    pd.set(8, 126);
    expect(rope->load_param(pd) == 0, "rope_dim 126");
    const auto windows = seedvr2::make_awa_windows(2, 16, 16, 1, 8, 8, true);
    expect(windows.size() == 9 && windows[1].h0 == 4 && windows[1].h1 == 12 && windows[3].w0 == 4,
           "make_awa_windows 2x16x16 shifted");
    expect(seedvr2::make_awa_windows(0, 16, 16, 1, 8, 8, false).empty(), "make_awa_windows invalid");
    std::printf("%s\n", failures ? "params: FAILED" : "params: all passed");
    return failures ? 1 : 0;
}

// A DiT block's AWA section as the reference's export writes it
// (tools/export_dit_block.py:578-604, :639-644, :740-743): Pack, MMRoPE,
// WindowAttention, Unpack, the video batch reshape, and a consumer Gemm.
std::string block_param(const char* t, const char* h, const char* w, int shifted)
{
    const std::string grid = std::string("0=") + t + " 1=" + h + " 2=" + w;
    const std::string rest = " 3=3 4=8 5=8 6=64 7=" + std::to_string(shifted);
    return "7767517\n"
           "8 10\n"
           "Input in0 0 1 vid_qkv 0=128 1=60 2=2304\n"
           "Input in1 0 1 txt_qkv 0=128 1=60 2=64\n"
           "SeedVR2AWAPack awa_pack 2 2 vid_qkv txt_qkv packed awa_cu_seqlens " + grid + rest + "\n"
           "SeedVR2MMRoPE mmrope 1 1 packed roped " + grid + rest + " 8=126\n"
           "SeedVR2WindowAttention awa_attention 1 1 roped attended " + grid + rest + "\n"
           "SeedVR2AWAUnpack awa_unpack 1 2 attended vid_out txt_out " + grid + rest + "\n"
           "Reshape reshape_awa_video_batch 1 1 vid_out awa_video_batch 0=2560 1=-1\n"
           "Gemm gemm_0 1 1 awa_video_batch proj 10=-1 2=0 3=1 4=0 5=1 6=1 7=0 8=2560 9=2560 -23310=3,1.0,0.5,-2\n";
}

int run_param()
{
    for (const int shifted : {0, 1})
    {
        Net net;
        register_seedvr2_awa_layers(net);
        const std::string text = block_param("9", "16", "16", shifted);
        expect(net.load_param_mem(text.c_str()) == 0, "static 9x16x16 block loads");
        expect(net.layers().size() == 8 && net.blob_count() == 10, "8 layers, 10 blobs");
        const char* awa[4] = {"awa_pack", "mmrope", "awa_attention", "awa_unpack"};
        for (const char* name : awa)
        {
            const auto* l = net.find_layer(name);
            const auto* base = l && l->layer ? static_cast<const SeedVR2AwaLayerBase*>(l->layer.get()) : nullptr;
            awa_plan_info info{};
            expect(base && awa_plan_info_get(base->plan(), &info) == 0 && info.source_tokens == 2304 &&
                       info.window_count == (shifted ? 36 : 12) && info.sequence_tokens == (shifted ? 4608 : 3072),
                   name);
        }
        const auto* unpack = net.find_layer("awa_unpack");
        expect(unpack && unpack->bottoms.size() == 1 && unpack->tops.size() == 2 && unpack->tops[0] == "vid_out",
               "unpack blobs");
        const auto* reshape = net.find_layer("reshape_awa_video_batch");
        expect(reshape && !reshape->layer && reshape->bottoms[0] == "vid_out" && reshape->pd.get(1, 0) == -1,
               "video batch reshape recorded, height -1");
        const auto* gemm = net.find_layer("gemm_0");
        const std::vector<float> arr = gemm ? gemm->pd.get_array(10) : std::vector<float>();
        expect(gemm && arr.size() == 3 && arr[1] == 0.5f && arr[2] == -2.f && gemm->pd.get(8, 0) == 2560,
               "foreign layer params, array field");
    }
    // The dynamic package template: 0=-1 1=-1 2=-1 takes the session grid.
    seedvr2::AwaRuntimeSpec spec{9, 32, 32, 9 * 32 * 32};
    Net dyn;
    register_seedvr2_awa_layers(dyn, &spec);
    const std::string dyn_text = block_param("-1", "-1", "-1", 1);
    expect(dyn.load_param_mem(dyn_text.c_str()) == 0, "dynamic block loads with a runtime spec");
    {
        const auto* l = dyn.find_layer("awa_attention");
        awa_plan_info info{};
        expect(l && l->layer &&
                   awa_plan_info_get(static_cast<const SeedVR2AwaLayerBase*>(l->layer.get())->plan(), &info) == 0 &&
                   info.source_tokens == 9216 && info.window_count == 100,
               "dynamic grid 9x32x32 shifted: 100 windows");
    }
    Net nospec;
    register_seedvr2_awa_layers(nospec);
    expect(nospec.load_param_mem(dyn_text.c_str()) == -1 && nospec.layers().empty(),
           "dynamic block without a runtime spec fails");
    // Malformed files.
    Net bad;
    register_seedvr2_awa_layers(bad);
    std::string t = block_param("9", "16", "16", 0);
    expect(bad.load_param_mem(("123\n" + t.substr(t.find('\n') + 1)).c_str()) == -1, "bad magic");
    std::string wrong_count = t;
    wrong_count.replace(wrong_count.find("8 10"), 4, "9 10");
    expect(bad.load_param_mem(wrong_count.c_str()) == -1, "layer count mismatch");
    std::string short_line = t + "Split s 1\n";
    expect(bad.load_param_mem(short_line.c_str()) == -1, "truncated layer line");
    std::string bad_param = t;
    bad_param.replace(bad_param.find("7=0\nSeedVR2MMRoPE"), 3, "7=x");
    expect(bad.load_param_mem(bad_param.c_str()) == -1, "non-numeric parameter");
    std::string zero_windows = t;
    zero_windows.replace(zero_windows.find("3=3 4=8 5=8 6=64 7=0\nSeedVR2AWAUnpack") , 3, "3=0");
    expect(bad.load_param_mem(zero_windows.c_str()) == -1 && !bad.last_error().empty(),
           "layer load_param failure fails the load");
    std::string dup = t;
    dup.replace(dup.find("packed roped"), 12, "packed packed");
    expect(bad.load_param_mem(dup.c_str()) == -1, "blob produced twice");
    expect(bad.load_param("/nonexistent/dit_block_00.ncnn.param") == -1, "missing file");
    std::printf("%s\n", failures ? "param: FAILED" : "param: all passed");
    return failures ? 1 : 0;
}

std::vector<float> to_host_float(const Mat& m)
{
    // Dense rows of w elements: dims 3 -> [c][h][w], dims 4 -> [n][c][d][h][w], cstep gaps dropped.
    const long long row = static_cast<long long>(m.w) * m.h * (m.dims == 4 ? m.d : 1);
    const long long planes = static_cast<long long>(m.c) * m.n;
    std::vector<unsigned char> raw(static_cast<size_t>(m.total() * m.elemsize));
    awa_memcpy_d2h(raw.data(), m.data, raw.size(), nullptr);
    awa_stream_synchronize(nullptr);
    std::vector<float> out(static_cast<size_t>(row * planes));
    for (long long b = 0; b < m.n; b++)
        for (long long c = 0; c < m.c; c++)
            for (long long i = 0; i < row; i++)
            {
                const size_t src = static_cast<size_t>(b * m.nstep + c * m.cstep + i);
                float v;
                if (m.elemsize == 4)
                    std::memcpy(&v, &raw[src * 4], 4);
                else
                {
                    unsigned short h16;
                    std::memcpy(&h16, &raw[src * 2], 2);
                    const unsigned int bits = static_cast<unsigned int>(h16) << 16;
                    std::memcpy(&v, &bits, 4);
                }
                out[static_cast<size_t>((b * m.c + c) * row + i)] = v;
            }
    return out;
}

bool write_file(const std::string& path, const std::vector<float>& v)
{
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f)
        return false;
    const bool ok = std::fwrite(v.data(), sizeof(float), v.size(), f) == v.size();
    std::fclose(f);
    return ok;
}

int run_forward(int argc, char** argv)
{
    if (argc < 13)
    {
        std::fprintf(stderr, "usage: forward OUTDIR t h w nt nh nw text shifted heads bf16\n");
        return 2;
    }
    const std::string dir = argv[2];
    int a[10];
    for (int i = 0; i < 10; i++)
        a[i] = std::atoi(argv[3 + i]);
    const int t = a[0], h = a[1], w = a[2], text = a[6], heads = a[8];
    const bool bf16 = a[9] != 0;
    const int n = t * h * w, d = 128;
    const size_t es = bf16 ? 2 : 4;
    if (awa_runtime_init(0) != AWA_OK)
    {
        std::fprintf(stderr, "no device: %s\n", awa_last_error());
        return 1;
    }
    Option opt;
    opt.use_bf16_storage = bf16;
    Net net;
    register_seedvr2_awa_layers(net);
    const ParamDict pd = params(a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]);
    auto pack = net.create_custom_layer("SeedVR2AWAPack");
    auto rope = net.create_custom_layer("SeedVR2MMRoPE");
    auto attention = net.create_custom_layer("SeedVR2WindowAttention");
    auto unpack = net.create_custom_layer("SeedVR2AWAUnpack");
    for (auto* layer : {pack.get(), rope.get(), attention.get(), unpack.get()})
        if (layer->load_param(pd) != 0 || layer->upload_model(opt) != 0 || layer->create_pipeline(opt) != 0)
        {
            std::fprintf(stderr, "%s: load/upload failed\n", layer->type.c_str());
            return 1;
        }
    // Layout (a): Mat(d, 3H, tokens).
    Mat video, txt;
    if (video.create(d, 3 * heads, n, es, nullptr) != 0 || txt.create(d, 3 * heads, text, es, nullptr) != 0)
        return 1;
    awa_fill_normal(video.data, static_cast<size_t>(video.total()), static_cast<int>(es), 20260901ULL, nullptr);
    awa_fill_normal(txt.data, static_cast<size_t>(txt.total()), static_cast<int>(es), 20260902ULL, nullptr);

    std::vector<Mat> packed, roped, attended, staged, fused;
    int rc = pack->forward({video, txt}, packed, opt);
    if (rc == 0)
        rc = rope->forward({packed[0]}, roped, opt);
    if (rc == 0)
        rc = attention->forward({roped[0]}, attended, opt);
    if (rc == 0)
        rc = unpack->forward({attended[0]}, staged, opt);
    if (rc == 0)
        rc = seedvr2_awa_forward_chain(*static_cast<SeedVR2AWAPack*>(pack.get()),
                                       *static_cast<SeedVR2AWAUnpack*>(unpack.get()), {video, txt}, fused, opt);
    if (rc != 0 || awa_stream_synchronize(nullptr) != 0)
    {
        std::fprintf(stderr, "forward failed rc=%d: %s\n", rc, awa_last_error());
        return 1;
    }
    const auto sv = to_host_float(staged[0]), st = to_host_float(staged[1]);
    const auto fv = to_host_float(fused[0]), ft = to_host_float(fused[1]);
    double diff = 0.0;
    for (size_t i = 0; i < sv.size(); i++)
        diff = std::fmax(diff, std::fabs(static_cast<double>(sv[i]) - fv[i]));
    for (size_t i = 0; i < st.size(); i++)
        diff = std::fmax(diff, std::fabs(static_cast<double>(st[i]) - ft[i]));
    const auto cu = to_host_float(packed[1]);
    if (!write_file(dir + "/video_qkv.f32", to_host_float(video)) || !write_file(dir + "/text_qkv.f32", to_host_float(txt)) ||
        !write_file(dir + "/staged_video.f32", sv) || !write_file(dir + "/staged_text.f32", st) ||
        !write_file(dir + "/fused_video.f32", fv) || !write_file(dir + "/fused_text.f32", ft) ||
        !write_file(dir + "/cu_seqlens.f32", cu))
    {
        std::fprintf(stderr, "cannot write into %s\n", dir.c_str());
        return 1;
    }
    for (auto* layer : {pack.get(), rope.get(), attention.get(), unpack.get()})
        layer->destroy_pipeline(opt);
    std::printf("forward: staged vs fused max abs diff %.9g\n", diff);
    return 0;
}

} // namespace

int main(int argc, char** argv)
{
    if (argc >= 2 && std::strcmp(argv[1], "params") == 0)
        return run_params();
    if (argc >= 2 && std::strcmp(argv[1], "forward") == 0)
        return run_forward(argc, argv);
    if (argc >= 2 && std::strcmp(argv[1], "param") == 0)
        return run_param();
    std::fprintf(stderr, "usage: %s params | param | forward OUTDIR t h w nt nh nw text shifted heads bf16\n",
                 argv[0]);
    return 2;
}
