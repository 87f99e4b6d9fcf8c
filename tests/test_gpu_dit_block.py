"""The DiT block around the AWA layer on the GPU (awa_dit_block_forward)
against the oracle block (FixedDitBlock.forward restated,
tools/reference/dit_block.py:344-378).

Tolerances, max|err| / max|ref| over each output:
- fp32 block: <= 1e-5. Everything is fp32 on the GPU against float64 in the
  oracle; the AWA layer itself is held to 1e-4 absolute elsewhere, and its
  output enters the block through a projection with weights ~0.05.
- bf16 block: <= 2e-2 (the bf16 budget). The oracle rounds to bf16 at the
  same points the GPU block stores bf16, so the remainder is accumulation
  order and the bf16 attention arithmetic.
"""

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import geometry
from test_dit_block_oracle import EPS, HEAD_DIM, HEADS, HIDDEN, MLP, case

pytestmark = pytest.mark.gpu


class DeviceBranch:
    """A branch's weights on the device: GEMM weights in the block's element
    size. adjacent_mlp stores proj_in right after proj_in_gate in one
    allocation (the block then runs the two as one GEMM); otherwise they are
    separate allocations (two GEMMs)."""

    def __init__(self, w: O.DitBranchWeights, elemsize: int, adjacent_mlp: bool = False):
        self.bufs = []

        def up(a, es):
            a = np.ascontiguousarray(a, np.float32)
            buf = A.DeviceBuffer(a.size * es)
            buf.upload(A.f32_to_bf16_bits(a) if es == 2 else a)
            self.bufs.append(buf)
            return buf.ptr

        if adjacent_mlp:
            gate = up(np.concatenate([w.mlp_gate, w.mlp_in]), elemsize)
            inp = gate + w.mlp_gate.size * elemsize
        else:
            gate, inp = up(w.mlp_gate, elemsize), up(w.mlp_in, elemsize)
        self.struct = A.AwaDitBranchWeights(
            up(w.qkv, elemsize), up(w.proj_out, elemsize), up(w.proj_out_bias, 4), gate, inp,
            up(w.mlp_out, elemsize), up(w.norm_q, 4), up(w.norm_k, 4), up(w.ada, 4))


def upload_act(x, es):
    x = np.ascontiguousarray(x, np.float32)
    buf = A.DeviceBuffer(x.size * es)
    buf.upload(A.f32_to_bf16_bits(x) if es == 2 else x)
    return buf


def download_act(buf, shape, es):
    n = int(np.prod(shape))
    if es == 2:
        return A.bf16_bits_to_f32(buf.download((n,), np.uint16)).reshape(shape)
    return buf.download((n,), np.float32).reshape(shape)


def run_block(g, video, text, emb, wv, wt, last_layer, precision):
    es = 2 if precision == A.COMPUTE_BF16 else 4
    blk = A.DitBlock(*g.args, g.text_tokens, g.shifted, HEADS, HEAD_DIM, HIDDEN, MLP, last_layer, precision, EPS)
    dv, dt = DeviceBranch(wv, es), DeviceBranch(wt, es)
    bv, bt, be = upload_act(video, es), upload_act(text, es), upload_act(emb, es)
    ov, ot = A.DeviceBuffer(video.size * es), A.DeviceBuffer(text.size * es)
    blk.forward(dv.struct, dt.struct, bv.ptr, bt.ptr, be.ptr, ov.ptr, ot.ptr)
    A.synchronize()
    out = download_act(ov, video.shape, es), download_act(ot, text.shape, es)
    blk.destroy()
    return out


def rel(a, b):
    """max|a - b| / max|b| (the gate), with the Frobenius relative error printed beside it."""
    d = np.abs(a.astype(np.float64) - b)
    fro = float(np.linalg.norm(d) / np.linalg.norm(np.asarray(b, np.float64)))
    print(f"  Frobenius rel {fro:.3g}, mean |d| {np.mean(d):.3g}", flush=True)
    return float(np.max(d) / np.max(np.abs(b)))


@pytest.mark.parametrize("last_layer", [False, True])
@pytest.mark.parametrize("shifted", [False, True])
@pytest.mark.parametrize("precision", [A.COMPUTE_F32, A.COMPUTE_BF16])
def test_dit_block_matches_oracle(gpu, precision, shifted, last_layer):
    bf16 = precision == A.COMPUTE_BF16
    print(f"case dit block bf16={bf16} shifted={shifted} last={last_layer}", flush=True)
    g, video, text, emb, wv, wt = case(100 + 4 * bf16 + 2 * shifted + last_layer, shifted)
    got_v, got_t = run_block(g, video, text, emb, wv, wt, last_layer, precision)
    ref_v, ref_t = O.dit_block(g, video, text, emb, wv, wt, HEADS, HEAD_DIM, EPS, last_layer, bf16=bf16)
    tol = 2e-2 if bf16 else 1e-5
    ev, et = rel(got_v, ref_v), rel(got_t, ref_t)
    print(f"  rel err video {ev:.3g} text {et:.3g}", flush=True)
    assert ev <= tol and et <= tol


def test_dit_block_rejects_bad_descriptions(gpu):
    for kw in ({"head_dim": 64}, {"hidden": 250}, {"precision": 7}):
        args = dict(t=2, h=16, w=16, nt=1, nh=8, nw=8, text_tokens=16, shifted=False, heads=HEADS,
                    head_dim=HEAD_DIM, hidden=HIDDEN, mlp_hidden=MLP, last_layer=False, precision=A.COMPUTE_F32)
        args.update(kw)
        with pytest.raises(A.AwaError):
            A.DitBlock(**args)


def test_dit_stack_matches_oracle_blocks(gpu):
    """Four blocks with the precision switch after two (fp32, fp32, bf16,
    bf16-last): the stack's outputs against the oracle block applied in turn,
    with the carried video, text and embedding rounded to bf16 at the switch
    (src/dit/dit_stack.cpp:934-950). The bf16 part is two blocks deep, so the
    bf16 budget is taken per block: <= 2 * 2e-2."""
    blocks, prefix = 4, 2
    print("case dit stack 4 blocks, 2 fp32", flush=True)
    rng = np.random.default_rng(77)
    from test_dit_block_oracle import make_weights
    g0, video, text, emb, _, _ = case(300, False)
    ws = [(make_weights(rng), make_weights(rng)) for _ in range(blocks)]
    stack = A.DitStack(*g0.args, g0.text_tokens, blocks, prefix, HEADS, HEAD_DIM, HIDDEN, MLP, EPS)
    dev = [(DeviceBranch(wv, 4 if b < prefix else 2, adjacent_mlp=b % 2 == 0),
            DeviceBranch(wt, 4 if b < prefix else 2, adjacent_mlp=b % 2 == 0)) for b, (wv, wt) in enumerate(ws)]
    bv, bt, be = upload_act(video, 4), upload_act(text, 4), upload_act(emb, 4)
    ov, ot = A.DeviceBuffer(video.size * 2), A.DeviceBuffer(text.size * 2)
    stack.run([d[0].struct for d in dev], [d[1].struct for d in dev], bv.ptr, bt.ptr, be.ptr, ov.ptr, ot.ptr)
    A.synchronize()
    got_v, got_t = download_act(ov, video.shape, 2), download_act(ot, text.shape, 2)
    stack.destroy()
    rv, rt, re = video, text, emb
    for b in range(blocks):
        g = geometry(g0.args + (g0.text_tokens,), b % 2 == 1)
        bf16 = b >= prefix
        if b == prefix:
            rv, rt, re = O.round_bf16(rv), O.round_bf16(rt), O.round_bf16(re)
        rv, rt = O.dit_block(g, rv, rt, re, ws[b][0], ws[b][1], HEADS, HEAD_DIM, EPS, b == blocks - 1, bf16=bf16)
        rv, rt = rv.astype(np.float32), rt.astype(np.float32)
    ev, et = rel(got_v, rv), rel(got_t, rt)
    print(f"  rel err video {ev:.3g} text {et:.3g}", flush=True)
    assert ev <= 4e-2 and et <= 4e-2


@pytest.mark.parametrize("precision,shifted", [(A.COMPUTE_F32, False), (A.COMPUTE_BF16, True)])
def test_dit_block_benchmark_shape(gpu, precision, shifted):
    """One block at the benchmark workload: latent 9x16x16, windows 3x8x8,
    64 text tokens, hidden 2560 = 20 x 128, SwiGLU 6912; weights N(0, 0.02)
    (the random init of the benchmark), inputs N(0, 1). Same tolerances."""
    bf16 = precision == A.COMPUTE_BF16
    print(f"case dit block benchmark shape bf16={bf16} shifted={shifted}", flush=True)
    heads, hidden, mlp = 20, 2560, 6912
    g = geometry((9, 16, 16, 3, 8, 8, 64), shifted)
    rng = np.random.default_rng(2026 + bf16)
    n = lambda *s, sd=0.02: (rng.standard_normal(s) * sd).astype(np.float32)

    def weights():
        return O.DitBranchWeights(qkv=n(3 * hidden, hidden), proj_out=n(hidden, hidden), proj_out_bias=n(hidden),
                                  mlp_gate=n(mlp, hidden), mlp_in=n(mlp, hidden), mlp_out=n(hidden, mlp),
                                  norm_q=rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32),
                                  norm_k=rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32), ada=n(6, hidden, sd=0.5))

    wv, wt = weights(), weights()
    video, text, emb = n(g.source_tokens, hidden, sd=1.0), n(g.text_tokens, hidden, sd=1.0), n(hidden * 6, sd=1.0)
    es = 2 if bf16 else 4
    blk = A.DitBlock(*g.args, g.text_tokens, g.shifted, heads, HEAD_DIM, hidden, mlp, False, precision, EPS)
    dv, dt = DeviceBranch(wv, es, adjacent_mlp=True), DeviceBranch(wt, es, adjacent_mlp=True)
    bv, bt, be = upload_act(video, es), upload_act(text, es), upload_act(emb, es)
    ov, ot = A.DeviceBuffer(video.size * es), A.DeviceBuffer(text.size * es)
    blk.forward(dv.struct, dt.struct, bv.ptr, bt.ptr, be.ptr, ov.ptr, ot.ptr)
    A.synchronize()
    got_v, got_t = download_act(ov, video.shape, es), download_act(ot, text.shape, es)
    blk.destroy()
    ref_v, ref_t = O.dit_block(g, video, text, emb, wv, wt, heads, HEAD_DIM, EPS, False, bf16=bf16)
    ev, et = rel(got_v, ref_v), rel(got_t, ref_t)
    print(f"  rel err video {ev:.3g} text {et:.3g}", flush=True)
    tol = 2e-2 if bf16 else 1e-5
    assert ev <= tol and et <= tol


def test_dit_stack_zero_gates_is_exact_at_benchmark_shape(gpu):
    """The whole 32-block loop at the benchmark workload (latent 9x16x16,
    windows 3x8x8, 64 text, hidden 2560 = 20 x 128, SwiGLU 6912, blocks 0-8
    fp32 and 9-31 bf16), checked by a property that holds at any size: with
    every Ada gate zero (the embedding's and the learned ones) each block
    returns its video and text inputs unchanged, (h + bias) * 0 + x = x
    exactly, and the last block, with its text output projection and bias
    zero, returns text as 2 * (0 + text). So video_out = bf16(video) and
    text_out = 2 * bf16(text) bit for bit, whatever the attention and the
    MLP compute in between (weights N(0, 0.02) on the device)."""
    t, h, w, nt, nh, nw, tx = 9, 16, 16, 3, 8, 8, 64
    blocks, prefix, heads, hidden, mlp = 32, 9, 20, 2560, 6912
    n = t * h * w
    print("case dit stack zero gates, 33f 256x256, 32 blocks", flush=True)
    stack = A.DitStack(t, h, w, nt, nh, nw, tx, blocks, prefix, heads, HEAD_DIM, hidden, mlp, EPS)
    rng = np.random.default_rng(5)
    keep = []
    seed = [700]

    def dev(count, es, stddev=0.02):
        b = A.DeviceBuffer(count * es)
        b.fill_normal(count, es, seed[0], None, stddev)
        seed[0] += 1
        keep.append(b)
        return b

    def host(a):
        a = np.ascontiguousarray(a, np.float32)
        b = A.DeviceBuffer(a.nbytes)
        b.upload(a)
        keep.append(b)
        return b

    wv, wt = [], []
    for blk in range(blocks):
        es = 4 if blk < prefix else 2
        for br in range(2):
            ada = (rng.standard_normal((6, hidden)) * 0.5).astype(np.float32)
            ada[[2, 5]] = 0.0  # learned attention and MLP gates
            proj = dev(hidden * hidden, es)
            bias = host(rng.standard_normal(hidden) * 0.1)
            if br == 1 and blk == blocks - 1:
                proj.zero()
                bias.zero()
            (wv if br == 0 else wt).append(A.AwaDitBranchWeights(
                dev(3 * hidden * hidden, es).ptr, proj.ptr, bias.ptr, dev(mlp * hidden, es).ptr,
                dev(mlp * hidden, es).ptr, dev(hidden * mlp, es).ptr,
                host(rng.uniform(0.5, 1.5, HEAD_DIM)).ptr, host(rng.uniform(0.5, 1.5, HEAD_DIM)).ptr, host(ada).ptr))
    video = rng.standard_normal((n, hidden)).astype(np.float32)
    text = rng.standard_normal((tx, hidden)).astype(np.float32)
    emb = (rng.standard_normal((hidden, 2, 3)) * 0.5).astype(np.float32)
    emb[:, :, 2] = 0.0  # embedding gates
    bv, bt, be = host(video), host(text), host(emb)
    ov, ot = A.DeviceBuffer(n * hidden * 2), A.DeviceBuffer(tx * hidden * 2)
    stack.run(wv, wt, bv.ptr, bt.ptr, be.ptr, ov.ptr, ot.ptr)
    A.synchronize()
    got_v = A.bf16_bits_to_f32(ov.download((n * hidden,), np.uint16)).reshape(n, hidden)
    got_t = A.bf16_bits_to_f32(ot.download((tx * hidden,), np.uint16)).reshape(tx, hidden)
    stack.destroy()
    np.testing.assert_array_equal(got_v, O.round_bf16(video))
    np.testing.assert_array_equal(got_t, 2.0 * O.round_bf16(text))


@pytest.mark.parametrize("precision", [A.COMPUTE_F32, A.COMPUTE_BF16])
def test_block_objects_share_gemm_algorithms(gpu, precision):
    """Two block objects of one shape (the second created after the first
    chose its GEMM algorithms) run the same algorithms: bit-identical
    outputs on the same weights and inputs."""
    print(f"case two block objects precision={precision}", flush=True)
    g, video, text, emb, wv, wt = case(20260917, False)
    first = run_block(g, video, text, emb, wv, wt, False, precision)
    second = run_block(g, video, text, emb, wv, wt, False, precision)
    for a, b in zip(first, second):
        assert np.array_equal(a, b)
