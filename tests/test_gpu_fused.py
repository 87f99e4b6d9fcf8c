"""Parity of the fused HIP layer (awa_forward) with the CPU oracle.

Tolerances: fp32 compute, max abs error <= 1e-4 against the oracle's Kahan
(shader-order) fp32 result; bf16 compute, max|err| / max|ref| <= 2e-2 against
the same oracle fed the identical bf16-rounded inputs.
"""

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import CONFIGS, HEAD_DIM, RAGGED, abs_err, geometry, qkv_inputs, rel_err
from device_blobs import DeviceMat, mat3, qkv_blob, read_mat3, read_video, video_out_blob

pytestmark = pytest.mark.gpu

FP32_ATOL = 1e-4
BF16_RTOL = 2e-2


def run_fused(g, video, text, compute, in_elem=4, out_elem=4, layout="a", batch_out=False, text_out_elem=None):
    heads = video.shape[2]
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    vq = qkv_blob(video, layout, in_elem)
    tq = qkv_blob(text, "a", in_elem)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, out_elem, batch_out)
    to = mat3(HEAD_DIM, heads, g.text_tokens, out_elem if text_out_elem is None else text_out_elem)
    plan.forward(vq.blob, tq.blob, vo.blob, to.blob, compute)
    A.synchronize()
    return read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), read_mat3(to)


def bf16_round(x):
    return A.bf16_bits_to_f32(A.f32_to_bf16_bits(x))


@pytest.mark.parametrize("shifted", [False, True])
def test_fp32_image_layer(gpu, shifted):
    g = geometry(CONFIGS["image_1x16x16"], shifted)
    print(f"case fp32 image shifted={shifted}", flush=True)
    video, text = qkv_inputs(g, 20, HEAD_DIM, 20260823)
    ref_v, ref_t = O.awa_layer(g, video, text, 20, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32)
    assert abs_err(got_v, ref_v) <= FP32_ATOL
    assert abs_err(got_t, ref_t) <= FP32_ATOL


@pytest.mark.parametrize("shifted", [False, True])
def test_bf16_clip_layer(gpu, shifted):
    g = geometry(CONFIGS["clip_2x16x16"], shifted)
    print(f"case bf16 clip_2x16x16 shifted={shifted}", flush=True)
    video, text = qkv_inputs(g, 20, HEAD_DIM, 20260824)
    video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, 20, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=2, out_elem=2)
    assert rel_err(got_v, ref_v) <= BF16_RTOL
    assert rel_err(got_t, ref_t) <= BF16_RTOL


@pytest.mark.parametrize("params", RAGGED)
@pytest.mark.parametrize("shifted", [False, True])
def test_fp32_ragged(gpu, params, shifted):
    g = geometry(params, shifted)
    print(f"case fp32 ragged {params} shifted={shifted}", flush=True)
    video, text = qkv_inputs(g, 2, HEAD_DIM, 7 + sum(params))
    ref_v, ref_t = O.awa_layer(g, video, text, 2, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32)
    assert abs_err(got_v, ref_v) <= FP32_ATOL
    assert abs_err(got_t, ref_t) <= FP32_ATOL


@pytest.mark.parametrize("params", RAGGED[:2])
def test_bf16_ragged(gpu, params):
    g = geometry(params, True)
    print(f"case bf16 ragged {params}", flush=True)
    video, text = qkv_inputs(g, 3, HEAD_DIM, 11 + sum(params))
    video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, 3, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=2, out_elem=4)
    assert rel_err(got_v, ref_v) <= BF16_RTOL
    assert rel_err(got_t, ref_t) <= BF16_RTOL


def test_production_single_window(gpu):
    """(4,3,3) at 256x256 is a single 1x16x16 window: plain attention over N+T_x tokens."""
    g = geometry(CONFIGS["production_256"], False)
    print("case production single window", flush=True)
    video, text = qkv_inputs(g, 4, HEAD_DIM, 666)
    ref_v, ref_t = O.awa_layer(g, video, text, 4, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32)
    assert abs_err(got_v, ref_v) <= FP32_ATOL
    assert abs_err(got_t, ref_t) <= FP32_ATOL


# The reference's production window setting (4, 3, 3) with 58 text tokens on
# the 720p latent grid (45 x 80): 13 latent frames give windows of 4 x 15 x
# 27 video tokens, 1678 rows with the text (tools/reference/dit_stack.py:20).
@pytest.mark.parametrize("shifted", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_production_720p_windows(gpu, shifted, bf16):
    g = geometry((13, 45, 80, 4, 3, 3, 58), shifted)
    print(f"case 13x45x80 (4,3,3) text 58 shifted={shifted} bf16={bf16}", flush=True)
    heads = 2
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    assert plan.info.max_window_tokens == 4 * 15 * 27 + 58
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260913)
    if bf16:
        video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, heads, HEAD_DIM)
    if bf16:
        got_v, got_t = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=2, out_elem=2)
        assert rel_err(got_v, ref_v) <= BF16_RTOL and rel_err(got_t, ref_t) <= BF16_RTOL
    else:
        got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32)
        assert abs_err(got_v, ref_v) <= FP32_ATOL and abs_err(got_t, ref_t) <= FP32_ATOL


@pytest.mark.parametrize("layout", ["a", "b", "c", "d"])
@pytest.mark.parametrize("batch_out", [False, True])
def test_layouts_identical(gpu, layout, batch_out):
    """All four accepted QKV layouts and both video output layouts give the same bits."""
    g = geometry((2, 8, 12, 1, 4, 4, 6), True)
    print(f"case layout {layout} batch_out={batch_out}", flush=True)
    video, text = qkv_inputs(g, 3, HEAD_DIM, 99)
    base_v, base_t = run_fused(g, video, text, A.COMPUTE_F32, layout="a", batch_out=False)
    got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32, layout=layout, batch_out=batch_out)
    np.testing.assert_array_equal(got_v, base_v)
    np.testing.assert_array_equal(got_t, base_t)


def packed_attention_f32(g, video, text):
    """Per-window attention rows [S][H][d] of the staged fp32 chain."""
    heads = video.shape[2]
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    S = plan.info.sequence_tokens
    vq = qkv_blob(video, "a", 4)
    tq = qkv_blob(text, "a", 4)
    packed = mat3(HEAD_DIM, 3 * heads, S, 4)
    cu = DeviceMat(dict(w=plan.info.window_count + 1, dims=1), plan.info.window_count + 1, 4)
    roped = mat3(HEAD_DIM, 3 * heads, S, 4)
    att = mat3(HEAD_DIM, heads, S, 4)
    plan.pack(vq.blob, tq.blob, packed.blob, cu.blob)
    plan.mmrope(packed.blob, roped.blob)
    plan.window_attention(roped.blob, att.blob, A.COMPUTE_F32)
    A.synchronize()
    return read_mat3(att)


def test_bf16_output_rounding(gpu):
    """bf16 video outputs are the fp32 outputs rounded to nearest even. A bf16
    text output is the window-order mean of the per-window rows rounded to
    bf16 (the packed attention output of a bf16 layer), itself rounded
    (src/awa/awa_layers.cpp:768-775, src/awa/shader/awa_unpack.comp:47-58)."""
    g = geometry((1, 8, 8, 1, 2, 2, 4), True)
    print("case bf16 output rounding", flush=True)
    heads = 2
    video, text = qkv_inputs(g, heads, HEAD_DIM, 5)
    v32, t32 = run_fused(g, video, text, A.COMPUTE_F32, out_elem=4)
    v16, t16 = run_fused(g, video, text, A.COMPUTE_F32, out_elem=2)
    np.testing.assert_array_equal(v16, bf16_round(v32))
    rows = packed_attention_f32(g, video, text)
    _, t_expect = O.unpack_forward(g, bf16_round(rows), heads, HEAD_DIM)
    np.testing.assert_array_equal(t16, bf16_round(t_expect))
    # Mixed outputs: fp32 text keeps fp32 rows.
    v16m, t32m = run_fused(g, video, text, A.COMPUTE_F32, out_elem=2, text_out_elem=4)
    np.testing.assert_array_equal(v16m, v16)
    np.testing.assert_array_equal(t32m, t32)


# The benchmark workloads themselves: 33 frames 256x256 (9x16x16), 9 frames
# 512x512 (9x32x32) and 121 frames 256x256 (31x16x16, windows of up to 320
# rows and a ragged temporal remainder), both partitions, both precisions.
@pytest.mark.parametrize("name", ["clip_9x16x16", "clip_9x32x32", "clip_31x16x16"])
@pytest.mark.parametrize("shifted", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_benchmark_shapes(gpu, name, shifted, bf16):
    heads = 20
    g = geometry(CONFIGS[name], shifted)
    print(f"case {name} shifted={shifted} bf16={bf16} heads={heads}", flush=True)
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260825)
    if bf16:
        video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, heads, HEAD_DIM)
    if bf16:
        got_v, got_t = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=2, out_elem=2)
        assert rel_err(got_v, ref_v) <= BF16_RTOL and rel_err(got_t, ref_t) <= BF16_RTOL
    else:
        got_v, got_t = run_fused(g, video, text, A.COMPUTE_F32)
        assert abs_err(got_v, ref_v) <= FP32_ATOL and abs_err(got_t, ref_t) <= FP32_ATOL


# Every input / output element size with either arithmetic, including fp32
# QKV into bf16 arithmetic (how QKV reaches AWA in the reference's BF16
# blocks: src/dit/dit_precision.cpp:22-142).
@pytest.mark.parametrize("in_elem", [4, 2])
@pytest.mark.parametrize("out_elem", [4, 2])
@pytest.mark.parametrize("compute", [A.COMPUTE_F32, A.COMPUTE_BF16])
def test_precision_combinations(gpu, in_elem, out_elem, compute):
    g = geometry((3, 11, 13, 2, 3, 3, 5), True)
    print(f"case precision in={in_elem} out={out_elem} compute={compute}", flush=True)
    video, text = qkv_inputs(g, 3, HEAD_DIM, 20260826)
    if in_elem == 2:
        video, text = bf16_round(video), bf16_round(text)
    ref_v, ref_t = O.awa_layer(g, video, text, 3, HEAD_DIM)
    got_v, got_t = run_fused(g, video, text, compute, in_elem=in_elem, out_elem=out_elem)
    if compute == A.COMPUTE_F32 and out_elem == 4:
        assert abs_err(got_v, ref_v) <= FP32_ATOL and abs_err(got_t, ref_t) <= FP32_ATOL
    else:
        assert rel_err(got_v, ref_v) <= BF16_RTOL and rel_err(got_t, ref_t) <= BF16_RTOL


def test_text_mean_repeated_launches(gpu):
    """The plan's lazily rebuilt work lists and text-row workspace give the
    same bits on repeated launches of one plan, in both arithmetics and with
    the head count changing between runs."""
    g = geometry(RAGGED[1], True)
    print(f"case repeated launches {RAGGED[1]} shifted", flush=True)
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    plan.upload()
    first = {}
    for heads in (2, 5, 2, 5):
        video, text = qkv_inputs(g, heads, HEAD_DIM, 90 + heads)
        vq = qkv_blob(video, "a", 4)
        tq = qkv_blob(text, "a", 4)
        for compute in (A.COMPUTE_F32, A.COMPUTE_BF16):
            for _ in range(3):
                vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, False)
                to = mat3(HEAD_DIM, heads, g.text_tokens, 4)
                plan.forward(vq.blob, tq.blob, vo.blob, to.blob, compute)
                A.synchronize()
                got_v = read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM)
                got_t = read_mat3(to)
                key = (heads, compute)
                if key not in first:
                    ref_v, ref_t = O.awa_layer(g, video, text, heads, HEAD_DIM)
                    tol = abs_err if compute == A.COMPUTE_F32 else rel_err
                    bound = FP32_ATOL if compute == A.COMPUTE_F32 else BF16_RTOL
                    assert tol(got_v, ref_v) <= bound and tol(got_t, ref_t) <= bound, key
                    first[key] = (got_v, got_t)
                np.testing.assert_array_equal(got_v, first[key][0])
                np.testing.assert_array_equal(got_t, first[key][1])


# Layers whose windows end in a last key tile of at most 32 keys (shifted: the
# 33-frame layer's windows of 80, 96 and 160 rows, the 5-frame clip's of 96, a
# ragged grid's of 140 and 406). On bf16
# inputs the bf16 kernel runs such a tile's first score block only; on fp32
# inputs it runs the whole tile with the second block masked. Fed the same
# bf16-representable values, the two must agree bit for bit.
@pytest.mark.parametrize("params", [CONFIGS["clip_9x16x16"], CONFIGS["clip_2x16x16"], RAGGED[1]])
def test_short_last_tile_same_bits(gpu, params):
    g = geometry(params, True)
    print(f"case short last tile {params} shifted", flush=True)
    video, text = qkv_inputs(g, 4, HEAD_DIM, 20260901)
    video, text = bf16_round(video), bf16_round(text)
    v2, t2 = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=2, out_elem=2)
    v4, t4 = run_fused(g, video, text, A.COMPUTE_BF16, in_elem=4, out_elem=2)
    assert np.array_equal(v2, v4) and np.array_equal(t2, t4)
    ref_v, ref_t = O.awa_layer(g, video, text, 4, HEAD_DIM)
    assert rel_err(v2, ref_v) <= BF16_RTOL and rel_err(t2, ref_t) <= BF16_RTOL
