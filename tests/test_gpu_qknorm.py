"""The DiT block's q/k RMSNorm on the GPU: the standalone DitRMSNorm
(src/dit/dit_precision.cpp:63-86, src/dit/shader/dit_rmsnorm.comp) and the
QKV prologue fused into the AWA gather (awa_forward_qknorm), against the CPU
oracle: RMSNorm in the shader's order, then the AWA layer.

Tolerances: the standalone norm is bit-exact; the fused layer, fp32 compute,
max abs error <= 1e-4 (its norm uses v_rsq_f32 and a lane-order sum, a few
ulp from the oracle's); bf16 compute, max|err| / max|ref| <= 2e-2.
"""

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import CONFIGS, HEAD_DIM, RAGGED, abs_err, geometry, qkv_inputs, rel_err
from device_blobs import DeviceMat, mat3, qkv_blob, read_mat3, read_video, upload_mat3, video_out_blob

pytestmark = pytest.mark.gpu

EPS = 1e-5


def bf16_round(x):
    return A.bf16_bits_to_f32(A.f32_to_bf16_bits(x))


def gamma_set(seed):
    rng = np.random.RandomState(seed)
    return [rng.uniform(0.25, 2.0, HEAD_DIM).astype(np.float32) for _ in range(4)]


class DeviceGammas:
    def __init__(self, gammas):
        self.bufs = [A.DeviceBuffer(HEAD_DIM * 4) for _ in gammas]
        for b, g in zip(self.bufs, gammas):
            b.upload(g)
        self.norm = A.AwaQkNorm(*[b.ptr for b in self.bufs], EPS)


def run_fused_qknorm(g, video, text, gammas, compute, in_elem=4, out_elem=4, layout="a"):
    heads = video.shape[2]
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    vq = qkv_blob(video, layout, in_elem)
    tq = qkv_blob(text, "a", in_elem)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, out_elem, False)
    to = mat3(HEAD_DIM, heads, g.text_tokens, out_elem)
    dg = DeviceGammas(gammas)
    plan.forward_qknorm(vq.blob, tq.blob, dg.norm, vo.blob, to.blob, compute)
    A.synchronize()
    return read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), read_mat3(to)


@pytest.mark.parametrize("elemsize", [4, 2])
@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("width", [128, 2560, 200])
def test_rmsnorm_bit_exact(gpu, elemsize, affine, width):
    print(f"case rmsnorm elem={elemsize} affine={affine} width={width}", flush=True)
    rng = np.random.RandomState(width + elemsize)
    rows, channels = 37, 3
    x = (rng.randn(channels, rows, width) * rng.uniform(0.1, 20, (channels, rows, 1))).astype(np.float32)
    if elemsize == 2:
        x = bf16_round(x)
    gamma = rng.uniform(-2, 2, width).astype(np.float32) if affine else None
    inp = mat3(width, rows, channels, elemsize)
    upload_mat3(inp, x)
    out_elem = 4 if affine else elemsize
    out = mat3(width, rows, channels, out_elem)
    gbuf = None
    if affine:
        gbuf = A.DeviceBuffer(width * 4)
        gbuf.upload(gamma)
    A.rmsnorm(inp.blob, gbuf.ptr if gbuf else None, EPS, out.blob)
    A.synchronize()
    want = O.rmsnorm(x.reshape(-1, width), gamma, EPS).reshape(channels, rows, width)
    if out_elem == 2:
        want = bf16_round(want)
    np.testing.assert_array_equal(read_mat3(out), want)


@pytest.mark.parametrize("shifted", [False, True])
def test_fused_qknorm_fp32(gpu, shifted):
    g = geometry(CONFIGS["clip_2x16x16"], shifted)
    print(f"case qknorm fp32 clip_2x16x16 shifted={shifted}", flush=True)
    heads = 4
    video, text = qkv_inputs(g, heads, HEAD_DIM, 4242)
    video[:, :2] *= 3.0  # raw projections are not unit-scale
    gammas = gamma_set(7)
    nv, nt = O.qk_norm_inputs(video, text, gammas, EPS)
    ref_v, ref_t = O.awa_layer(g, nv, nt, heads, HEAD_DIM)
    got_v, got_t = run_fused_qknorm(g, video, text, gammas, A.COMPUTE_F32)
    assert abs_err(got_v, ref_v) <= 1e-4
    assert abs_err(got_t, ref_t) <= 1e-4


@pytest.mark.parametrize("params", RAGGED[:3])
def test_fused_qknorm_ragged(gpu, params):
    g = geometry(params, True)
    print(f"case qknorm ragged {params}", flush=True)
    heads = 2
    video, text = qkv_inputs(g, heads, HEAD_DIM, 17 + sum(params))
    gammas = gamma_set(sum(params))
    nv, nt = O.qk_norm_inputs(video, text, gammas, EPS)
    ref_v, ref_t = O.awa_layer(g, nv, nt, heads, HEAD_DIM)
    got_v, got_t = run_fused_qknorm(g, video, text, gammas, A.COMPUTE_F32, layout="b")
    assert abs_err(got_v, ref_v) <= 1e-4
    assert abs_err(got_t, ref_t) <= 1e-4


@pytest.mark.parametrize("in_elem,out_elem", [(2, 2), (4, 2), (2, 4)])
def test_fused_qknorm_bf16(gpu, in_elem, out_elem):
    """bf16 MFMA on raw bf16 (or fp32) projections; Q/K stay fp32 through the
    norm and RoPE, as the reference's fp32 norm output feeds the AWA Pack."""
    g = geometry(CONFIGS["clip_9x16x16"], True)
    print(f"case qknorm bf16 clip_9x16x16 in={in_elem} out={out_elem}", flush=True)
    heads = 2
    video, text = qkv_inputs(g, heads, HEAD_DIM, 99)
    if in_elem == 2:
        video, text = bf16_round(video), bf16_round(text)
    gammas = gamma_set(3)
    nv, nt = O.qk_norm_inputs(video, text, gammas, EPS)
    ref_v, ref_t = O.awa_layer(g, nv, nt, heads, HEAD_DIM)
    got_v, got_t = run_fused_qknorm(g, video, text, gammas, A.COMPUTE_BF16, in_elem, out_elem)
    assert rel_err(got_v, ref_v) <= 2e-2
    assert rel_err(got_t, ref_t) <= 2e-2


@pytest.mark.parametrize("name,shifted,scale", [("image_1x16x16", False, 1.0), ("clip_9x16x16", True, 3.0),
                                               ("clip_9x16x16", False, 8.0)])
def test_fused_qknorm_matches_unfused_chain(gpu, name, shifted, scale):
    """fp32: the fused prologue gives the bits of the standalone norm of Q and
    K into an fp32 QKV followed by awa_forward (the reference's DitRMSNorm ->
    DitQKVConcat -> AWA data flow): the fused norm reproduces DitRMSNorm's
    tree-ordered sum and correctly rounded coefficient exactly, on raw
    projections of unit scale and scaled by 3 and 8 (gammas up to 20)."""
    g = geometry(CONFIGS[name], shifted)
    print(f"case qknorm fused vs unfused {name} shifted={shifted} scale={scale}", flush=True)
    heads = 4
    video, text = qkv_inputs(g, heads, HEAD_DIM, 5150)
    video[:, :2] *= scale
    text[:, :2] *= scale
    gammas = gamma_set(11) if scale == 1.0 else [
        np.random.RandomState(int(scale)).uniform(0.0, 20.0, HEAD_DIM).astype(np.float32) for _ in range(4)]
    fused_v, fused_t = run_fused_qknorm(g, video, text, gammas, A.COMPUTE_F32)
    # Unfused: layout 'b' keeps Q, K and V as three contiguous [T][H][d] blocks.
    dg = DeviceGammas(gammas)
    outs = []
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    blobs = []
    for qkv, gq, gk in ((video, dg.bufs[0], dg.bufs[1]), (text, dg.bufs[2], dg.bufs[3])):
        raw = qkv_blob(qkv, "b", 4)
        normed = qkv_blob(qkv, "b", 4)
        T = qkv.shape[0]
        for part, gbuf in ((0, gq), (1, gk)):
            rows = T * heads
            src = A.mat(raw.buf.ptr + part * rows * HEAD_DIM * 4, w=HEAD_DIM, h=rows, dims=2, elemsize=4)
            dst = A.mat(normed.buf.ptr + part * rows * HEAD_DIM * 4, w=HEAD_DIM, h=rows, dims=2, elemsize=4)
            A.rmsnorm(src, gbuf.ptr, EPS, dst)
        blobs.append((raw, normed))
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, False)
    to = mat3(HEAD_DIM, heads, g.text_tokens, 4)
    plan.forward(blobs[0][1].blob, blobs[1][1].blob, vo.blob, to.blob, A.COMPUTE_F32)
    A.synchronize()
    un_v = read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM)
    un_t = read_mat3(to)
    np.testing.assert_array_equal(fused_v, un_v)
    np.testing.assert_array_equal(fused_t, un_t)


def test_qknorm_invalid_arguments(gpu):
    g = geometry(CONFIGS["image_1x16x16"], False)
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    video, text = qkv_inputs(g, 1, HEAD_DIM, 1)
    vq, tq = qkv_blob(video, "a", 4), qkv_blob(text, "a", 4)
    vo = video_out_blob(g.t, g.h, g.w, 1, HEAD_DIM, 4, False)
    to = mat3(HEAD_DIM, 1, g.text_tokens, 4)
    dg = DeviceGammas(gamma_set(1))
    bad = A.AwaQkNorm(dg.bufs[0].ptr, None, dg.bufs[2].ptr, dg.bufs[3].ptr, EPS)
    with pytest.raises(RuntimeError):
        plan.forward_qknorm(vq.blob, tq.blob, bad, vo.blob, to.blob, A.COMPUTE_F32)
    misaligned = A.AwaQkNorm(dg.bufs[0].ptr + 4, dg.bufs[1].ptr, dg.bufs[2].ptr, dg.bufs[3].ptr, EPS)
    with pytest.raises(RuntimeError):
        plan.forward_qknorm(vq.blob, tq.blob, misaligned, vo.blob, to.blob, A.COMPUTE_F32)
    neg = A.AwaQkNorm(dg.bufs[0].ptr, dg.bufs[1].ptr, dg.bufs[2].ptr, dg.bufs[3].ptr, -1.0)
    with pytest.raises(RuntimeError):
        plan.forward_qknorm(vq.blob, tq.blob, neg, vo.blob, to.blob, A.COMPUTE_F32)


@pytest.mark.parametrize("v_elemsize", [4, 2])
@pytest.mark.parametrize("width,heads,tokens", [(128, 20, 37), (6, 3, 11)])
def test_qkv_concat_bit_exact(gpu, v_elemsize, width, heads, tokens):
    """DitQKVConcat (awa_qkv_concat) against the oracle, bit for bit: the
    16-byte path (width 128) and the per-element path (width 6)."""
    print(f"case qkv concat v_elem={v_elemsize} width={width} heads={heads} tokens={tokens}", flush=True)
    rng = np.random.RandomState(width + heads + v_elemsize)
    q, k, v = (rng.randn(tokens, heads, width).astype(np.float32) for _ in range(3))
    if v_elemsize == 2:
        v = bf16_round(v)
    mats = []
    for x, es in ((q, 4), (k, 4), (v, v_elemsize)):
        m = mat3(width, heads, tokens, es)
        upload_mat3(m, x)
        mats.append(m)
    out = mat3(width, 3 * heads, tokens, 4)
    A.qkv_concat(mats[0].blob, mats[1].blob, mats[2].blob, out.blob)
    A.synchronize()
    np.testing.assert_array_equal(read_mat3(out), O.qkv_concat(q, k, v))


def test_qkv_concat_rejects_bad_blobs(gpu):
    q, k = mat3(128, 4, 8, 4), mat3(128, 4, 8, 4)
    out = mat3(128, 12, 8, 4)
    for v in (mat3(128, 4, 7, 4), mat3(128, 5, 8, 4)):
        with pytest.raises(A.AwaError):
            A.qkv_concat(q.blob, k.blob, v.blob, out.blob)
    with pytest.raises(A.AwaError):  # q must be fp32
        A.qkv_concat(mat3(128, 4, 8, 2).blob, k.blob, mat3(128, 4, 8, 2).blob, out.blob)
    with pytest.raises(A.AwaError):  # output must be Mat(w, 3h, c)
        A.qkv_concat(q.blob, k.blob, mat3(128, 4, 8, 2).blob, mat3(128, 8, 8, 4).blob)
