"""The C++ layer surface (SeedVR2AWAPack / SeedVR2MMRoPE /
SeedVR2WindowAttention / SeedVR2AWAUnpack over the C ABI, and the DiT
precision layers DitRMSNorm / DitQKVConcat on the AWA input), driven by
tests/cpp/awa_layers_check the way a host of the reference's ncnn layers
drives them (src/awa/awa_layers.h:47-223, src/dit/dit_precision.cpp:22-343)."""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import oracle as O
from awa_cases import rel_err

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "cpp", "awa_layers_check")


def run_check(*args: str) -> subprocess.CompletedProcess:
    if not os.path.exists(CHECK):
        pytest.fail(f"{CHECK} missing: build it with `make -C tests/cpp` (part of __graft_entry__.build())")
    return subprocess.run([CHECK, *args], capture_output=True, text=True, timeout=300)


def test_layer_params_and_registration():
    r = run_check("params")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "params: all passed" in r.stdout


def test_param_file_loading():
    """ncnn .param text with a DiT block's AWA lines in the reference export's
    format (tools/export_dit_block.py:578-644): static and dynamic grids, the
    video batch reshape, foreign layers with array params, malformed files."""
    r = run_check("param")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "param: all passed" in r.stdout


FORWARD_CASES = [
    # t, h, w, nt, nh, nw, text, shifted, heads, bf16
    ((1, 16, 16, 1, 8, 8, 64, 0), 4, 0),
    ((2, 16, 16, 1, 8, 8, 64, 1), 3, 1),
    ((3, 11, 13, 2, 3, 3, 5, 1), 2, 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("params,heads,bf16", FORWARD_CASES)
def test_layer_chain_matches_oracle(gpu, tmp_path, params, heads, bf16):
    print(f"layer chain case {params} heads={heads} bf16={bf16}", flush=True)
    r = run_check("forward", str(tmp_path), *map(str, params), str(heads), str(bf16))
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    t, h, w, nt, nh, nw, text, shifted = params
    g = O.Geometry(t, h, w, nt, nh, nw, text, bool(shifted))
    n, d = g.source_tokens, 128

    def load(name, shape):
        return np.fromfile(os.path.join(tmp_path, name), np.float32).reshape(shape)

    video = load("video_qkv.f32", (n, 3, heads, d))
    txt = load("text_qkv.f32", (text, 3, heads, d))
    ref_v, ref_t = O.awa_layer(g, video, txt, heads, d)
    cu = load("cu_seqlens.f32", (-1,))
    assert np.array_equal(cu, O.build_maps(g).cu_seqlens.astype(np.float32))
    for kind in ("staged", "fused"):
        v = load(f"{kind}_video.f32", (n, heads, d))
        tt = load(f"{kind}_text.f32", (text, heads, d))
        if bf16:
            assert rel_err(v, ref_v) <= 2e-2 and rel_err(tt, ref_t) <= 2e-2, kind
        else:
            assert np.max(np.abs(v - ref_v)) <= 1e-4 and np.max(np.abs(tt - ref_t)) <= 1e-4, kind
    diff = float(r.stdout.strip().split()[-1])
    assert diff <= (1e-6 if not bf16 else 1e-2)


PARAM_FORWARD_CASES = [
    # t, h, w, nt, nh, nw, text, shifted, heads, bf16, dynamic, batch video layout
    ((2, 16, 16, 1, 8, 8, 64, 1), 4, 0, 0, 0),
    ((2, 16, 16, 1, 8, 8, 64, 0), 4, 1, 1, 1),
    ((9, 16, 16, 3, 8, 8, 64, 0), 4, 0, 1, 1),
    ((9, 16, 16, 3, 8, 8, 64, 1), 4, 1, 0, 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("params,heads,bf16,dynamic,batch", PARAM_FORWARD_CASES)
def test_param_package_runs_on_device(gpu, tmp_path, params, heads, bf16, dynamic, batch):
    """A DiT block's AWA section as the reference export writes it
    (tools/export_dit_block.py:578-644, :740-743; the dynamic template of
    :38-124), loaded by Net::load_param_mem (static grid, or 0=-1 1=-1 2=-1
    with the runtime spec), given its pipelines by Net::load_model and run by
    an Extractor, as load_graph and DitStackSession::run drive the reference
    package (src/dit/dit_stack.cpp:167-220, :951-963): Pack, MMRoPE,
    WindowAttention, Unpack, then reshape_awa_video_batch's [N][H*d] view of
    the video output (a dense copy of the NCNN_BATCH layout). Compared with
    the oracle."""
    print(f"param package case {params} heads={heads} bf16={bf16} dynamic={dynamic} batch={batch}", flush=True)
    r = run_check("paramforward", str(tmp_path), *map(str, params), str(heads), str(bf16), str(dynamic), str(batch))
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    t, h, w, nt, nh, nw, text, shifted = params
    g = O.Geometry(t, h, w, nt, nh, nw, text, bool(shifted))
    n, d = g.source_tokens, 128

    def load(name, shape):
        return np.fromfile(os.path.join(tmp_path, name), np.float32).reshape(shape)

    ref_v, ref_t = O.awa_layer(g, load("video_qkv.f32", (n, 3, heads, d)), load("text_qkv.f32", (text, 3, heads, d)),
                               heads, d)
    v = load("video_batch.f32", (n, heads * d)).reshape(n, heads, d)
    tt = load("text_out.f32", (text, heads, d))
    if bf16:
        assert rel_err(v, ref_v) <= 2e-2 and rel_err(tt, ref_t) <= 2e-2
    else:
        assert np.max(np.abs(v - ref_v)) <= 1e-4 and np.max(np.abs(tt - ref_t)) <= 1e-4


@pytest.mark.gpu
def test_shape_trace(gpu, tmp_path):
    """SEEDVR2_TRACE_OPS prints one line per layer blob, in the reference's format."""
    env = dict(os.environ, SEEDVR2_TRACE_OPS="1")
    r = subprocess.run([CHECK, "forward", str(tmp_path), "1", "16", "16", "1", "8", "8", "64", "0", "2", "0"],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr
    lines = [l for l in r.stderr.splitlines() if l.startswith("awa-trace op=")]
    ops = [l.split()[1][3:] for l in lines]
    for op in ("pack.video.in", "pack.text.in", "pack.out", "rope.in", "attention.in", "unpack.in",
               "unpack.video.out", "unpack.text.out", "forward.video.in"):
        assert op in ops, op
    assert "awa-trace op=pack.video.in dims=3 w=128 h=6 d=1 c=256 elemsize=4 pack=1" in lines


def test_dit_precision_layers():
    """DitRMSNorm / DitQKVConcat registration and params, and
    configure_dit_block_precision_layers on paired and last-block graphs
    (src/dit/dit_precision.cpp:284-343): the Ada parameter views get
    featmask bit 2, the parameter sums are counted, wrong counts reject."""
    r = run_check("dit")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "dit: all passed" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("bf16", [0, 1])
def test_dit_precision_layer_chain_bit_exact(gpu, tmp_path, bf16):
    """RMSNorm(q), RMSNorm(k) (affine, fp32 out) and the QKV concat through
    the layer surface as an FP32 or BF16 block runs them, against the
    oracle's rmsnorm and qkv_concat: bit for bit (the norm follows the
    shader's summation order; the concat moves and promotes exactly)."""
    tokens, heads, d = 45, 5, 128
    print(f"dit precision chain tokens={tokens} heads={heads} bf16={bf16}", flush=True)
    r = run_check("ditforward", str(tmp_path), str(tokens), str(heads), str(bf16))
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr

    def load(name, shape):
        return np.fromfile(os.path.join(tmp_path, name), np.float32).reshape(shape)

    q, k, v = (load(f"{x}.f32", (tokens, heads, d)) for x in "qkv")
    gq, gk = load("gamma_q.f32", (d,)), load("gamma_k.f32", (d,))
    want = O.qkv_concat(O.rmsnorm(q, gq, 1e-5), O.rmsnorm(k, gk, 1e-5), v)
    np.testing.assert_array_equal(load("qkv.f32", (tokens, 3 * heads, d)), want)
