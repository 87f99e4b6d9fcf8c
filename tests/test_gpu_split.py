"""Split layers: when an fp32 layer's (window, head) units are long but too
few to fill the device, each unit's keys are split into segments over several
workgroups, and a second kernel combines the segments (out = sum_s 2^(m_s - M)
O_s / sum_s 2^(m_s - M) l_s) in place of the text-mean kernel. Covers the
split factor the plans pick (the production 256x256 fp32 layer splits in
five; the image, short-clip, bf16 and 33-frame 20-head layers do not), oracle
parity of the production layer (one 320-row window, 20 heads) in both
precisions, the split result against the same layer with splitting turned off
(SEEDVR2_AWA_SPLIT=0), and the staged chain against the fused layer, bit for
bit in fp32, with both split.
"""

import os

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import CONFIGS, HEAD_DIM, abs_err, geometry, qkv_inputs, rel_err
from device_blobs import DeviceMat, mat3, qkv_blob, read_mat3, read_video, video_out_blob

pytestmark = pytest.mark.gpu


def bf16_round(x):
    return A.bf16_bits_to_f32(A.f32_to_bf16_bits(x))


def run_fused(g, video, text, compute, elem, split_on=True):
    """The fused layer; returns (video, text, split factor used)."""
    heads = video.shape[2]
    old = os.environ.pop("SEEDVR2_AWA_SPLIT", None)
    if not split_on:
        os.environ["SEEDVR2_AWA_SPLIT"] = "0"
    try:
        plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted), heads=heads)
        plan.upload()
        split = plan.attention_split(heads, compute)
    finally:
        os.environ.pop("SEEDVR2_AWA_SPLIT", None)
        if old is not None:
            os.environ["SEEDVR2_AWA_SPLIT"] = old
    vq, tq = qkv_blob(video, "a", elem), qkv_blob(text, "a", elem)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, elem, False)
    to = mat3(HEAD_DIM, heads, g.text_tokens, elem)
    plan.forward(vq.blob, tq.blob, vo.blob, to.blob, compute)
    A.synchronize()
    return read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), read_mat3(to), split


@pytest.mark.parametrize("name,shifted,compute,heads,expect", [
    ("production_256", False, A.COMPUTE_F32, 20, 5),
    ("production_256", False, A.COMPUTE_BF16, 20, 1),
    ("production_256", False, A.COMPUTE_F32_MFMA, 20, 1),
    ("image_1x16x16", False, A.COMPUTE_F32, 20, 1),
    ("clip_2x16x16", False, A.COMPUTE_F32, 20, 3),
    ("clip_2x16x16", True, A.COMPUTE_F32, 20, 1),
    ("clip_2x16x16", True, A.COMPUTE_BF16, 20, 1),
    ("clip_9x16x16", False, A.COMPUTE_F32, 20, 1),
    ("clip_9x16x16", True, A.COMPUTE_F32, 20, 1),
    ("clip_9x16x16", False, A.COMPUTE_F32, 4, 4),
    ("clip_9x16x16", True, A.COMPUTE_F32, 4, 1),
])
def test_split_factor(gpu, name, shifted, compute, heads, expect):
    """The production layer's 20 units of 320 rows split in five (one per
    64-key tile) in fp32, the unshifted 2x16x16 clip's 80 units of 192 rows
    in three; bf16 and the pipelined fp32-MFMA variant never split; units of
    under three 64-key tiles (image, shifted windows) do not; the 33-frame
    layer fills the device unsplit at 20 heads and splits in four (48 8-wave
    items) at 4."""
    g = geometry(CONFIGS[name], shifted)
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    assert plan.attention_split(heads, compute) == expect


@pytest.mark.parametrize("compute", [A.COMPUTE_F32, A.COMPUTE_BF16])
def test_production_layer_matches_oracle(gpu, compute):
    """The production 256x256 layer (windows (4, 3, 3): one 16 x 16 window of
    256 video rows + 64 text rows), 20 heads: fp32 (split in five) within 1e-4
    of the oracle, bf16 (not split) within 2e-2 relative of it on the same bf16
    inputs."""
    g = geometry(CONFIGS["production_256"], False)
    bf16 = compute == A.COMPUTE_BF16
    print(f"case production 256 bf16={bf16}", flush=True)
    video, text = qkv_inputs(g, 20, HEAD_DIM, 20260901)
    if bf16:
        video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, 20, HEAD_DIM)
    got_v, got_t, split = run_fused(g, video, text, compute, 2 if bf16 else 4)
    assert split == (1 if bf16 else 5)
    if bf16:
        assert rel_err(got_v, ref_v) <= 2e-2 and rel_err(got_t, ref_t) <= 2e-2
    else:
        assert abs_err(got_v, ref_v) <= 1e-4 and abs_err(got_t, ref_t) <= 1e-4


@pytest.mark.parametrize("name,shifted,heads,elem", [
    ("production_256", False, 20, 4),
    ("production_256", False, 20, 2),
    ("clip_2x16x16", False, 20, 4),
    ("clip_9x16x16", False, 4, 4),
])
def test_split_matches_unsplit(gpu, name, shifted, heads, elem):
    """The same fp32 layer and inputs with splitting off: within 1e-5 for fp32
    outputs (a tenth of the parity budget; only the summation order differs),
    and within one bf16 rounding (2^-8 relative) for bf16 outputs."""
    g = geometry(CONFIGS[name], shifted)
    print(f"case split vs unsplit {name} shifted={shifted} heads={heads} out elem={elem}", flush=True)
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260902)
    sv, st, s_split = run_fused(g, video, text, A.COMPUTE_F32, elem)
    uv, ut, s_plain = run_fused(g, video, text, A.COMPUTE_F32, elem, split_on=False)
    assert s_split > 1 and s_plain == 1
    if elem == 2:
        assert rel_err(sv, uv.astype(np.float64)) <= 2 ** -8 and rel_err(st, ut.astype(np.float64)) <= 2 ** -8
    else:
        assert abs_err(sv, uv.astype(np.float64)) <= 1e-5 and abs_err(st, ut.astype(np.float64)) <= 1e-5


def test_staged_split_matches_fused(gpu):
    """Pack -> MMRoPE -> WindowAttention -> Unpack on a split layer (the
    production layer, 20 heads) gives the fused layer's bits in fp32: both
    combine the same segments with the same kernel."""
    g = geometry(CONFIGS["production_256"], False)
    heads = 20
    print("case staged split production 256", flush=True)
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260903)
    fv, ft, split = run_fused(g, video, text, A.COMPUTE_F32, 4)
    assert split == 5
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    S = plan.info.sequence_tokens
    vq, tq = qkv_blob(video, "a", 4), qkv_blob(text, "a", 4)
    packed = mat3(HEAD_DIM, 3 * heads, S, 4)
    cu = DeviceMat(dict(w=plan.info.window_count + 1, dims=1), plan.info.window_count + 1, 4)
    roped = mat3(HEAD_DIM, 3 * heads, S, 4)
    att = mat3(HEAD_DIM, heads, S, 4)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, False)
    to = mat3(HEAD_DIM, heads, g.text_tokens, 4)
    plan.pack(vq.blob, tq.blob, packed.blob, cu.blob)
    plan.mmrope(packed.blob, roped.blob)
    plan.window_attention(roped.blob, att.blob, A.COMPUTE_F32)
    plan.unpack(att.blob, vo.blob, to.blob)
    A.synchronize()
    np.testing.assert_array_equal(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), fv)
    np.testing.assert_array_equal(read_mat3(to), ft)


@pytest.mark.parametrize("compute,elem,split_on", [(A.COMPUTE_F32, 4, False), (A.COMPUTE_BF16, 2, True),
                                                   (A.COMPUTE_BF16, 4, True)])
def test_single_window_text_written_directly(gpu, compute, elem, split_on):
    """A layer of one window (the production layer) writes its text rows
    straight to the text output, the mean of one row being that row: against
    the oracle, and in fp32 bit for bit against the staged chain, whose
    Unpack takes the mean."""
    g = geometry(CONFIGS["production_256"], False)
    heads = 8
    bf16 = compute == A.COMPUTE_BF16
    print(f"case single window text direct bf16={bf16} out elem={elem}", flush=True)
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260904)
    if bf16:
        video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, heads, HEAD_DIM)
    fv, ft, split = run_fused(g, video, text, compute, elem, split_on=split_on)
    assert split == 1
    if bf16:
        assert rel_err(fv, ref_v) <= 2e-2 and rel_err(ft, ref_t) <= 2e-2
        return
    assert abs_err(fv, ref_v) <= 1e-4 and abs_err(ft, ref_t) <= 1e-4
    old = os.environ.pop("SEEDVR2_AWA_SPLIT", None)
    os.environ["SEEDVR2_AWA_SPLIT"] = "0"
    try:
        plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted), heads=heads)
        plan.upload()
    finally:
        os.environ.pop("SEEDVR2_AWA_SPLIT", None)
        if old is not None:
            os.environ["SEEDVR2_AWA_SPLIT"] = old
    S = plan.info.sequence_tokens
    vq, tq = qkv_blob(video, "a", 4), qkv_blob(text, "a", 4)
    packed = mat3(HEAD_DIM, 3 * heads, S, 4)
    cu = DeviceMat(dict(w=plan.info.window_count + 1, dims=1), plan.info.window_count + 1, 4)
    roped = mat3(HEAD_DIM, 3 * heads, S, 4)
    att = mat3(HEAD_DIM, heads, S, 4)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, False)
    to = mat3(HEAD_DIM, heads, g.text_tokens, 4)
    plan.pack(vq.blob, tq.blob, packed.blob, cu.blob)
    plan.mmrope(packed.blob, roped.blob)
    plan.window_attention(roped.blob, att.blob, A.COMPUTE_F32)
    plan.unpack(att.blob, vo.blob, to.blob)
    A.synchronize()
    np.testing.assert_array_equal(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), fv)
    np.testing.assert_array_equal(read_mat3(to), ft)


@pytest.mark.parametrize("compute,elem,split_on", [(A.COMPUTE_BF16, 2, True), (A.COMPUTE_F32, 4, False),
                                                   (A.COMPUTE_F32, 4, True)])
def test_single_window_padded_text_output(gpu, compute, elem, split_on):
    """A text output with padded rows (cstep past H * d) cannot take the
    direct write of a one-window layer's text rows: the text-mean (or, split,
    the merge) kernel writes them instead, and the bits equal those of the
    dense output (the mean of one row is that row)."""
    g = geometry(CONFIGS["production_256"], False)
    heads = 4
    print(f"case single window padded text output compute={compute} elem={elem} split={split_on}", flush=True)
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260905)
    if compute == A.COMPUTE_BF16:
        video, text = bf16_round(video), bf16_round(text)
    dv, dt, split = run_fused(g, video, text, compute, elem, split_on=split_on)
    assert (split > 1) == (split_on and compute == A.COMPUTE_F32)
    old = os.environ.pop("SEEDVR2_AWA_SPLIT", None)
    if not split_on:
        os.environ["SEEDVR2_AWA_SPLIT"] = "0"
    try:
        plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted), heads=heads)
        plan.upload()
    finally:
        os.environ.pop("SEEDVR2_AWA_SPLIT", None)
        if old is not None:
            os.environ["SEEDVR2_AWA_SPLIT"] = old
    vq, tq = qkv_blob(video, "a", elem), qkv_blob(text, "a", elem)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, elem, False)
    cstep = heads * HEAD_DIM + 16 // elem
    to = DeviceMat(dict(w=HEAD_DIM, h=heads, c=g.text_tokens, dims=3, cstep=cstep), g.text_tokens * cstep, elem)
    plan.forward(vq.blob, tq.blob, vo.blob, to.blob, compute)
    A.synchronize()
    np.testing.assert_array_equal(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), dv)
    np.testing.assert_array_equal(read_mat3(to), dt)
