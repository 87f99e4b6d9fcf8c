"""Parity of the staged entry points (the four reference layers one by one)
with the oracle: Pack, MMRoPE and Unpack are bit-exact; WindowAttention is
within the fp32 / bf16 tolerances."""

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import CONFIGS, HEAD_DIM, abs_err, geometry, qkv_inputs, rel_err
from device_blobs import DeviceMat, mat3, qkv_blob, read_mat3, read_video, upload_mat3, video_out_blob

pytestmark = pytest.mark.gpu


def make_plan(g, rope_dim=126):
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted, rope_dim))
    plan.upload()
    return plan


@pytest.mark.parametrize("shifted", [False, True])
@pytest.mark.parametrize("elemsize", [4, 2])
def test_pack_bit_exact(gpu, shifted, elemsize):
    g = geometry(CONFIGS["clip_2x16x16"], shifted)
    print(f"case pack shifted={shifted} elemsize={elemsize}", flush=True)
    heads = 4
    video, text = qkv_inputs(g, heads, HEAD_DIM, 1)
    if elemsize == 2:
        video = A.bf16_bits_to_f32(A.f32_to_bf16_bits(video))
        text = A.bf16_bits_to_f32(A.f32_to_bf16_bits(text))
    ref_packed, ref_cu = O.pack_forward(g, video, text, heads, HEAD_DIM)
    plan = make_plan(g)
    vq = qkv_blob(video, "b", elemsize)
    tq = qkv_blob(text, "a", elemsize)
    packed = mat3(HEAD_DIM, 3 * heads, plan.info.sequence_tokens, 4)
    cu = DeviceMat(dict(w=plan.info.window_count + 1, dims=1), plan.info.window_count + 1, 4)
    plan.pack(vq.blob, tq.blob, packed.blob, cu.blob)
    A.synchronize()
    got = read_mat3(packed).reshape(ref_packed.shape)
    np.testing.assert_array_equal(got, ref_packed)
    np.testing.assert_array_equal(cu.download_raw(), ref_cu)


@pytest.mark.parametrize("params,rope_dim", [(CONFIGS["clip_9x16x16"], 126), ((3, 11, 13, 2, 3, 3, 5), 126),
                                             ((2, 6, 6, 1, 2, 2, 3), 18)])
@pytest.mark.parametrize("shifted", [False, True])
def test_mmrope_bit_exact(gpu, params, rope_dim, shifted):
    g = geometry(params, shifted)
    print(f"case mmrope {params} rope_dim={rope_dim} shifted={shifted}", flush=True)
    heads = 2
    head_dim = HEAD_DIM if rope_dim == 126 else 24
    m = O.build_maps(g)
    x = O.fill_gaussian(m.sequence_tokens * 3 * heads * head_dim, 3).reshape(m.sequence_tokens, 3 * heads, head_dim)
    table = O.rope_table(g, rope_dim)
    ref = O.mmrope_forward(x, table, heads, head_dim, rope_dim)
    plan = make_plan(g, rope_dim)
    np.testing.assert_array_equal(plan.rope_table(), table)
    inp = mat3(head_dim, 3 * heads, m.sequence_tokens, 4)
    upload_mat3(inp, x)
    out = mat3(head_dim, 3 * heads, m.sequence_tokens, 4)
    plan.mmrope(inp.blob, out.blob)
    A.synchronize()
    np.testing.assert_array_equal(read_mat3(out), ref.reshape(m.sequence_tokens, 3 * heads, head_dim))


@pytest.mark.parametrize("compute", [A.COMPUTE_F32, A.COMPUTE_BF16])
@pytest.mark.parametrize("shifted", [False, True])
def test_window_attention_packed(gpu, compute, shifted):
    g = geometry(CONFIGS["clip_2x16x16"], shifted)
    print(f"case packed attention compute={compute} shifted={shifted}", flush=True)
    heads = 4
    m = O.build_maps(g)
    x = O.fill_gaussian(m.sequence_tokens * 3 * heads * HEAD_DIM, 17).reshape(m.sequence_tokens, 3, heads, HEAD_DIM)
    elem = 4
    if compute == A.COMPUTE_BF16:
        x = A.bf16_bits_to_f32(A.f32_to_bf16_bits(x))
        elem = 2
    ref = O.attention(x, m.cu_seqlens, heads, HEAD_DIM, "kahan")
    plan = make_plan(g)
    inp = mat3(HEAD_DIM, 3 * heads, m.sequence_tokens, elem)
    upload_mat3(inp, x.reshape(m.sequence_tokens, 3 * heads, HEAD_DIM))
    out = mat3(HEAD_DIM, heads, m.sequence_tokens, 4)
    plan.window_attention(inp.blob, out.blob, compute)
    A.synchronize()
    got = read_mat3(out)
    if compute == A.COMPUTE_F32:
        assert abs_err(got, ref) <= 1e-4
    else:
        assert rel_err(got, ref) <= 2e-2


def test_staged_chain_production_window(gpu):
    """The four staged layers at the production 121-frame 720p geometry:
    latent 31 x 45 x 80, windows (4, 3, 3) of up to 8 x 15 x 27 video tokens,
    58 text tokens: 3298-row windows (the fp32 kernel's 4-wave form)."""
    g = geometry((31, 45, 80, 4, 3, 3, 58), False)
    print("case staged chain 31x45x80 (4,3,3) text 58", flush=True)
    heads = 1
    video, text = qkv_inputs(g, heads, HEAD_DIM, 20260914)
    plan = make_plan(g)
    assert plan.info.max_window_tokens == 8 * 15 * 27 + 58
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
    ref_v, ref_t = O.awa_layer(g, video, text, heads, HEAD_DIM)
    assert abs_err(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), ref_v) <= 1e-4
    assert abs_err(read_mat3(to), ref_t) <= 1e-4


@pytest.mark.parametrize("head_dim", [8, 40])
def test_window_attention_generic_head_dim(gpu, head_dim):
    g = geometry((2, 6, 6, 1, 2, 2, 3), True)
    print(f"case generic attention head_dim={head_dim}", flush=True)
    heads = 2
    m = O.build_maps(g)
    x = O.fill_gaussian(m.sequence_tokens * 3 * heads * head_dim, 23).reshape(m.sequence_tokens, 3, heads, head_dim)
    ref = O.attention(x, m.cu_seqlens, heads, head_dim, "kahan")
    plan = make_plan(g, 6)
    inp = mat3(head_dim, 3 * heads, m.sequence_tokens, 4)
    upload_mat3(inp, x.reshape(m.sequence_tokens, 3 * heads, head_dim))
    out = mat3(head_dim, heads, m.sequence_tokens, 4)
    plan.window_attention(inp.blob, out.blob, A.COMPUTE_F32)
    A.synchronize()
    assert abs_err(read_mat3(out), ref) <= 1e-5


@pytest.mark.parametrize("shifted", [False, True])
@pytest.mark.parametrize("batch_out", [False, True])
def test_unpack_bit_exact(gpu, shifted, batch_out):
    g = geometry(CONFIGS["clip_9x16x16"], shifted)
    print(f"case unpack shifted={shifted} batch_out={batch_out}", flush=True)
    heads = 3
    m = O.build_maps(g)
    x = O.fill_gaussian(m.sequence_tokens * heads * HEAD_DIM, 29).reshape(m.sequence_tokens, heads, HEAD_DIM)
    ref_v, ref_t = O.unpack_forward(g, x, heads, HEAD_DIM, "gpu")
    plan = make_plan(g)
    inp = mat3(HEAD_DIM, heads, m.sequence_tokens, 4)
    upload_mat3(inp, x)
    vo = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, batch_out)
    to = mat3(HEAD_DIM, heads, g.text_tokens, 4)
    plan.unpack(inp.blob, vo.blob, to.blob)
    A.synchronize()
    np.testing.assert_array_equal(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM), ref_v)
    np.testing.assert_array_equal(read_mat3(to), ref_t)


def test_staged_chain_matches_fused(gpu):
    """Pack -> MMRoPE -> WindowAttention -> Unpack equals the fused layer (fp32)."""
    g = geometry(CONFIGS["clip_2x16x16"], True)
    print("case staged chain vs fused", flush=True)
    heads = 4
    video, text = qkv_inputs(g, heads, HEAD_DIM, 31)
    plan = make_plan(g)
    S = plan.info.sequence_tokens
    vq = qkv_blob(video, "a", 4)
    tq = qkv_blob(text, "a", 4)
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
    fv = video_out_blob(g.t, g.h, g.w, heads, HEAD_DIM, 4, False)
    ft = mat3(HEAD_DIM, heads, g.text_tokens, 4)
    plan.forward(vq.blob, tq.blob, fv.blob, ft.blob, A.COMPUTE_F32)
    A.synchronize()
    np.testing.assert_array_equal(read_video(vo, g.t, g.h, g.w, heads, HEAD_DIM),
                                  read_video(fv, g.t, g.h, g.w, heads, HEAD_DIM))
    np.testing.assert_array_equal(read_mat3(to), read_mat3(ft))


def test_cast_round_trip(gpu):
    x = O.fill_gaussian(3 * 5 * 40, 41).reshape(3, 5, 40)
    print("case cast", flush=True)
    a = mat3(40, 5, 3, 4)
    upload_mat3(a, x)
    b = mat3(40, 5, 3, 2)
    A.cast(a.blob, b.blob)
    c = mat3(40, 5, 3, 4)
    A.cast(b.blob, c.blob)
    A.synchronize()
    expect = A.bf16_bits_to_f32(A.f32_to_bf16_bits(x))
    np.testing.assert_array_equal(read_mat3(b), expect)
    np.testing.assert_array_equal(read_mat3(c), expect)
