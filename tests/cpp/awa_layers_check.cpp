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
//   awa_layers_check paramforward OUTDIR t h w nt nh nw text shifted heads bf16 dynamic batch
//       A DiT block's AWA section as .param text (static grid, or the
//       dynamic 0=-1 1=-1 2=-1 template with a runtime spec), loaded with
//       Net::load_param_mem and Net::load_model and run by an Extractor on
//       seeded inputs, the Unpack video output in the NCNN_BATCH layout when
//       batch is 1; writes the inputs, the reshaped video matrix
//       (awa_video_batch) and the text output as float32 files into OUTDIR.
//   awa_layers_check dit
//       Host-only checks of the DiT precision layers (DitRMSNorm,
//       DitQKVConcat): registration, params, and
//       configure_dit_block_precision_layers on paired and last-block graphs.
//   awa_layers_check ditforward OUTDIR tokens heads bf16
//       Seeded raw q/k/v on device 0 through RMSNorm (q, k; affine) and the
//       QKV concat as a BF16 (bf16 = 1) or FP32 block runs them; writes the
//       inputs, gammas and output as float32 files into OUTDIR.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "awa_layers.h"
#include "dit_layers.h"

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
    pd.set(8, 0);
    expect(rope->load_param(pd) == -1, "rope_dim 0 is invalid (only an absent param 8 defaults to 126)");
    pd.set(8, -6);
    expect(rope->load_param(pd) == -1, "negative rope_dim is invalid");
    pd.set(8, 126);
    expect(rope->load_param(pd) == 0, "rope_dim 126");
    ParamDict absent = params(2, 16, 16, 1, 8, 8, 64, 1);
    expect(rope->load_param(absent) == 0, "absent param 8 defaults to 126");
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

// The same section for any grid and head count: grid strings "-1" give the
// dynamic template, whose video batch reshape infers its height (1=-1).
std::string block_param_for(const std::string& t, const std::string& h, const std::string& w, int nt, int nh, int nw,
                            int text, int shifted, int heads, long long tokens, bool dynamic)
{
    const std::string grid = "0=" + t + " 1=" + h + " 2=" + w;
    const std::string rest = " 3=" + std::to_string(nt) + " 4=" + std::to_string(nh) + " 5=" + std::to_string(nw) +
                             " 6=" + std::to_string(text) + " 7=" + std::to_string(shifted);
    const std::string hidden = std::to_string(heads * 128);
    return "7767517\n"
           "8 10\n"
           "Input in0 0 1 vid_qkv 0=128 1=" + std::to_string(3 * heads) + " 2=" + std::to_string(tokens) + "\n"
           "Input in1 0 1 txt_qkv 0=128 1=" + std::to_string(3 * heads) + " 2=" + std::to_string(text) + "\n"
           "SeedVR2AWAPack awa_pack 2 2 vid_qkv txt_qkv packed awa_cu_seqlens " + grid + rest + "\n"
           "SeedVR2MMRoPE mmrope 1 1 packed roped " + grid + rest + " 8=126\n"
           "SeedVR2WindowAttention awa_attention 1 1 roped attended " + grid + rest + "\n"
           "SeedVR2AWAUnpack awa_unpack 1 2 attended vid_out txt_out " + grid + rest + "\n"
           "Reshape reshape_awa_video_batch 1 1 vid_out awa_video_batch 0=" + hidden + " 1=" +
           (dynamic ? std::string("-1") : std::to_string(tokens)) + "\n"
           "Gemm gemm_0 1 1 awa_video_batch proj 10=-1 2=0 3=1 4=0 5=1 6=1 7=0 8=" + hidden + " 9=" + hidden + "\n";
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

int run_param_forward(int argc, char** argv)
{
    if (argc < 15)
    {
        std::fprintf(stderr, "usage: paramforward OUTDIR t h w nt nh nw text shifted heads bf16 dynamic batch\n");
        return 2;
    }
    const std::string dir = argv[2];
    int a[12];
    for (int i = 0; i < 12; i++)
        a[i] = std::atoi(argv[3 + i]);
    const int t = a[0], h = a[1], w = a[2], text = a[6], heads = a[8];
    const bool bf16 = a[9] != 0, dynamic = a[10] != 0, batch = a[11] != 0;
    const int n = t * h * w, d = 128;
    const size_t es = bf16 ? 2 : 4;
    if (awa_runtime_init(0) != AWA_OK)
    {
        std::fprintf(stderr, "no device: %s\n", awa_last_error());
        return 1;
    }
    const std::string text_param =
        dynamic ? block_param_for("-1", "-1", "-1", a[3], a[4], a[5], text, a[7], heads, n, true)
                : block_param_for(std::to_string(t), std::to_string(h), std::to_string(w), a[3], a[4], a[5], text,
                                  a[7], heads, n, false);
    seedvr2::AwaRuntimeSpec spec{t, h, w, n};
    Net net;
    register_seedvr2_awa_layers(net, dynamic ? &spec : nullptr);
    Option opt;
    opt.use_bf16_storage = bf16;
    opt.use_batch_video_layout = batch;
    if (net.load_param_mem(text_param.c_str()) != 0 || net.load_model(opt) != 0)
    {
        std::fprintf(stderr, "load failed: %s\n", net.last_error().c_str());
        return 1;
    }
    Mat video, txt;
    if (video.create(d, 3 * heads, n, es, nullptr) != 0 || txt.create(d, 3 * heads, text, es, nullptr) != 0)
        return 1;
    awa_fill_normal(video.data, static_cast<size_t>(video.total()), static_cast<int>(es), 20260911ULL, nullptr);
    awa_fill_normal(txt.data, static_cast<size_t>(txt.total()), static_cast<int>(es), 20260912ULL, nullptr);
    seedvr2::hip::Extractor ex = net.create_extractor();
    Mat vb, tt, proj;
    if (ex.input("vid_qkv", video) != 0 || ex.input("txt_qkv", txt) != 0 || ex.extract("awa_video_batch", vb) != 0 ||
        ex.extract("txt_out", tt) != 0 || awa_stream_synchronize(nullptr) != 0)
    {
        std::fprintf(stderr, "extract failed: %s %s\n", ex.last_error().c_str(), awa_last_error());
        return 1;
    }
    if (vb.dims != 2 || vb.w != heads * d || vb.h != n || tt.dims != 3 || tt.w != d || tt.h != heads || tt.c != text)
    {
        std::fprintf(stderr, "unexpected shapes: video batch dims %d %dx%d, text dims %d\n", vb.dims, vb.w, vb.h, tt.dims);
        return 1;
    }
    // The block's projection Gemm is not part of this runtime: extracting past it fails cleanly.
    if (ex.extract("proj", proj) == 0 || ex.last_error().find("Gemm") == std::string::npos)
    {
        std::fprintf(stderr, "extracting the Gemm output should fail: %s\n", ex.last_error().c_str());
        return 1;
    }
    if (!write_file(dir + "/video_qkv.f32", to_host_float(video)) || !write_file(dir + "/text_qkv.f32", to_host_float(txt)) ||
        !write_file(dir + "/video_batch.f32", to_host_float(vb)) || !write_file(dir + "/text_out.f32", to_host_float(tt)))
    {
        std::fprintf(stderr, "cannot write into %s\n", dir.c_str());
        return 1;
    }
    std::printf("paramforward: %s %dx%dx%d shifted=%d heads=%d bf16=%d batch=%d: video batch %dx%d\n",
                dynamic ? "dynamic" : "static", t, h, w, a[7], heads, bf16, batch, vb.h, vb.w);
    return 0;
}

// A DiT block graph in the export's shape, reduced to what the precision
// configuration reads: per modulated branch an Ada parameter (MemoryData
// constant_p_ada_*), a Split into its six vectors and six BinaryOp sums with
// the embedding; five Gemms and a Swish per branch with an MLP, two Gemms
// for the last block's text branch; residual BinaryOps that read no
// parameter; the AWA Pack.
std::string dit_graph(bool last_block, int extra_sums)
{
    std::vector<std::string> lines;
    int blobs = 0;
    auto add = [&](const std::string& line, int tops) {
        lines.push_back(line);
        blobs += tops;
    };
    add("Input in_video 0 1 video", 1);
    add("Input in_text 0 1 text", 1);
    add("Input in_emb 0 1 emb", 1);
    add("Split split_emb 1 6 emb e0 e1 e2 e3 e4 e5", 6);
    for (const char* br : {"vid", "txt"})
    {
        const std::string b = br;
        const bool modulated = !last_block || b == "vid";
        if (modulated)
        {
            add("MemoryData constant_p_ada_" + b + " 0 1 ada_" + b + " 0=2560 1=6", 1);
            add("Reshape view_ada_" + b + " 1 1 ada_" + b + " adar_" + b + " 0=2560 1=6", 1);
            std::string split = "Split split_ada_" + b + " 1 6 adar_" + b;
            for (int i = 0; i < 6; i++)
                split += " a" + b + std::to_string(i);
            add(split, 6);
            for (int i = 0; i < 6; i++)
                add("BinaryOp sum_" + b + std::to_string(i) + " 2 1 e" + std::to_string(i) + " a" + b +
                        std::to_string(i) + " s" + b + std::to_string(i) + " 0=0",
                    1);
        }
        add("Gemm qkv_" + b + " 1 1 " + (b == "vid" ? "video" : "text") + " qkv_" + b, 1);
        add("Gemm proj_" + b + " 1 1 att_" + b + " proj_" + b, 1);
        add("BinaryOp resid_" + b + " 2 1 proj_" + b + " " + (b == "vid" ? "video" : "text") + " y_" + b + " 0=0",
            1);
        if (modulated)
        {
            add("Gemm gate_" + b + " 1 1 y_" + b + " g_" + b, 1);
            add("Gemm in_" + b + " 1 1 y_" + b + " i_" + b, 1);
            add("Swish swish_" + b + " 1 1 g_" + b + " sw_" + b, 1);
            add("Gemm out_" + b + " 1 1 sw_" + b + " o_" + b, 1);
        }
    }
    add("SeedVR2AWAPack awa_pack 2 2 qkv_vid qkv_txt packed cu 0=9 1=16 2=16 3=3 4=8 5=8 6=64 7=0", 2);
    add("SeedVR2AWAUnpack awa_unpack 1 2 packed att_vid att_txt 0=9 1=16 2=16 3=3 4=8 5=8 6=64 7=0", 2);
    for (int i = 0; i < extra_sums; i++)
        add("BinaryOp extra_sum" + std::to_string(i) + " 2 1 e0 avid0 x" + std::to_string(i) + " 0=0", 1);
    std::string text = "7767517\n" + std::to_string(lines.size()) + " " + std::to_string(blobs) + "\n";
    for (const std::string& l : lines)
        text += l + "\n";
    return text;
}

int run_dit()
{
    Net net;
    seedvr2::register_dit_block_precision_layers(net);
    const auto types = net.custom_layer_types();
    expect(types.size() == 2 && types[0] == "Concat" && types[1] == "RMSNorm", "RMSNorm and Concat registered");

    auto norm = net.create_custom_layer("RMSNorm");
    ParamDict pd;
    pd.set(0, 128);
    pd.set(1, 1e-5f);
    expect(norm && norm->load_param(pd) == 0, "RMSNorm load_param");
    auto* rms = static_cast<DitRMSNorm*>(norm.get());
    expect(rms->affine_size == 128 && rms->eps == 1e-5f && rms->affine == 1, "RMSNorm params 0-2 and defaults");
    Option opt;
    expect(rms->upload_model(opt) != 0, "RMSNorm affine without gamma is rejected");
    std::vector<Mat> tops;
    expect(rms->forward({Mat()}, tops, opt) != 0, "RMSNorm forward before upload is rejected");
    ParamDict bad;
    expect(net.create_custom_layer("RMSNorm")->load_param(bad) != 0, "RMSNorm without affine_size is rejected");

    auto concat = net.create_custom_layer("Concat");
    expect(concat && concat->load_param(ParamDict()) == 0 && concat->create_pipeline(opt) != 0,
           "Concat on axis 0 is rejected at create_pipeline");
    ParamDict axis1;
    axis1.set(0, 1);
    expect(concat->load_param(axis1) == 0 && concat->create_pipeline(opt) == 0, "Concat on axis 1");
    expect(concat->forward({Mat(), Mat()}, tops, opt) != 0, "Concat needs three inputs");

    struct Case
    {
        bool last;
        int extra;
        bool ok;
        int sums, gemms, swishes;
    };
    for (const Case& c : {Case{false, 0, true, 12, 10, 2}, Case{true, 0, true, 6, 7, 1}, Case{false, 1, false, 13, 10, 2},
                          Case{true, 6, false, 12, 7, 1}})
    {
        Net g;
        seedvr2::register_dit_block_precision_layers(g);
        const std::string text = dit_graph(c.last, c.extra);
        if (g.load_param_mem(text.c_str()) != 0)
        {
            std::printf("FAIL graph load: %s\n", g.last_error().c_str());
            failures++;
            continue;
        }
        seedvr2::DitBlockPrecision found;
        const bool ok = seedvr2::configure_dit_block_precision_layers(g, &found);
        char what[160];
        std::snprintf(what, sizeof what, "configure last=%d extra=%d: %s (sums %d gemms %d swishes %d)", c.last,
                      c.extra, ok ? "accepted" : "rejected", found.sums, found.gemms, found.swishes);
        expect(ok == c.ok && found.sums == c.sums && found.gemms == c.gemms && found.swishes == c.swishes, what);
        const auto* pack = g.find_layer("awa_pack");
        const auto* view = g.find_layer("view_ada_vid");
        const auto* split = g.find_layer("split_ada_vid");
        const auto* emb_split = g.find_layer("split_emb");
        expect(pack && (pack->featmask & 4) && view && (view->featmask & 4) && split && (split->featmask & 4) &&
                   emb_split && emb_split->featmask == 0,
               "featmask bit 2 on the Pack and the Ada views only");
        bool residual_fp32 = false;
        for (const std::string& name : found.fp32_sums)
            residual_fp32 = residual_fp32 || name.rfind("resid_", 0) == 0;
        expect(!residual_fp32, "residual sums keep the block's storage");
    }
    std::printf("dit: %s\n", failures ? "FAILED" : "all passed");
    return failures ? 1 : 0;
}

int run_dit_forward(int argc, char** argv)
{
    if (argc < 6)
    {
        std::fprintf(stderr, "usage: ditforward OUTDIR tokens heads bf16\n");
        return 2;
    }
    const std::string dir = argv[2];
    const int tokens = std::atoi(argv[3]), heads = std::atoi(argv[4]), d = 128;
    const bool bf16 = std::atoi(argv[5]) != 0;
    const size_t es = bf16 ? 2 : 4;
    if (awa_runtime_init(0) != AWA_OK)
    {
        std::fprintf(stderr, "no device: %s\n", awa_last_error());
        return 1;
    }
    Option opt;
    opt.use_bf16_storage = bf16;
    Net net;
    seedvr2::register_dit_block_precision_layers(net);
    ParamDict pn;
    pn.set(0, d);
    pn.set(1, 1e-5f);
    ParamDict pc;
    pc.set(0, 1);
    auto norm_q = net.create_custom_layer("RMSNorm");
    auto norm_k = net.create_custom_layer("RMSNorm");
    auto concat = net.create_custom_layer("Concat");
    int seed = 0;
    for (auto* layer : {norm_q.get(), norm_k.get()})
    {
        auto* rms = static_cast<DitRMSNorm*>(layer);
        if (rms->load_param(pn) != 0 || rms->gamma_data.create(d, 4, nullptr) != 0)
            return 1;
        awa_fill_normal(rms->gamma_data.data, d, 4, 20261000ULL + seed++, nullptr);
        if (rms->upload_model(opt) != 0 || rms->create_pipeline(opt) != 0)
            return 1;
    }
    if (concat->load_param(pc) != 0 || concat->create_pipeline(opt) != 0)
        return 1;
    // Raw projections Mat(d, H, tokens) in the block's storage type.
    Mat q, k, v;
    for (Mat* m : {&q, &k, &v})
    {
        if (m->create(d, heads, tokens, es, nullptr) != 0)
            return 1;
        awa_fill_normal(m->data, static_cast<size_t>(m->total()), static_cast<int>(es), 20261010ULL + seed++, nullptr);
    }
    std::vector<Mat> nq, nk, qkv;
    int rc = norm_q->forward({q}, nq, opt);
    if (rc == 0)
        rc = norm_k->forward({k}, nk, opt);
    if (rc == 0)
        rc = concat->forward({nq[0], nk[0], v}, qkv, opt);
    if (rc != 0 || awa_stream_synchronize(nullptr) != 0)
    {
        std::fprintf(stderr, "dit forward failed rc=%d: %s\n", rc, awa_last_error());
        return 1;
    }
    const bool shapes = nq[0].elemsize == 4 && qkv[0].dims == 3 && qkv[0].w == d && qkv[0].h == 3 * heads &&
                        qkv[0].c == tokens && qkv[0].elemsize == 4;
    if (!shapes || !write_file(dir + "/q.f32", to_host_float(q)) || !write_file(dir + "/k.f32", to_host_float(k)) ||
        !write_file(dir + "/v.f32", to_host_float(v)) ||
        !write_file(dir + "/gamma_q.f32", to_host_float(static_cast<DitRMSNorm*>(norm_q.get())->gamma_data)) ||
        !write_file(dir + "/gamma_k.f32", to_host_float(static_cast<DitRMSNorm*>(norm_k.get())->gamma_data)) ||
        !write_file(dir + "/qkv.f32", to_host_float(qkv[0])))
    {
        std::fprintf(stderr, "bad output shape or cannot write into %s\n", dir.c_str());
        return 1;
    }
    std::printf("ditforward: qkv %dx%dx%d fp32 written\n", qkv[0].w, qkv[0].h, qkv[0].c);
    return 0;
}

} // namespace

int main(int argc, char** argv)
{
    if (argc >= 2 && std::strcmp(argv[1], "params") == 0)
        return run_params();
    if (argc >= 2 && std::strcmp(argv[1], "forward") == 0)
        return run_forward(argc, argv);
    if (argc >= 2 && std::strcmp(argv[1], "paramforward") == 0)
        return run_param_forward(argc, argv);
    if (argc >= 2 && std::strcmp(argv[1], "param") == 0)
        return run_param();
    if (argc >= 2 && std::strcmp(argv[1], "dit") == 0)
        return run_dit();
    if (argc >= 2 && std::strcmp(argv[1], "ditforward") == 0)
        return run_dit_forward(argc, argv);
    std::fprintf(stderr, "usage: %s params | param | dit | forward OUTDIR t h w nt nh nw text shifted heads bf16 | "
                 "ditforward OUTDIR tokens heads bf16\n",
                 argv[0]);
    return 2;
}
