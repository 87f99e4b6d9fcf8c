"""Pins the oracle's DiT block (oracle.dit_block, a restatement of
FixedDitBlock.forward, tools/reference/dit_block.py:344-378) before the GPU
block is compared with it:

- closed forms: with every Ada gate zero the block is the identity (both
  residuals pass the input through); the last block returns text as
  2 * (text after attention + text), so with zero output-projection weights
  and bias it doubles the text;
- an independent float64 composition from torch's own routines
  (torch.nn.functional.rms_norm, linear, silu) following the reference
  module code, which must agree to rounding;
- planted mistakes (gate before the bias, eps outside the square root, SiLU
  replaced by sigmoid) that the comparison must reject.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from awa_cases import geometry

HEADS, HEAD_DIM = 2, 128
HIDDEN, MLP = HEADS * HEAD_DIM, 384
EPS = 1e-5


def make_weights(rng, hidden=HIDDEN, mlp=MLP, gate_scale=0.5):
    hd = HEADS * HEAD_DIM
    n = lambda *s, sd=0.05: (rng.standard_normal(s) * sd).astype(np.float32)
    ada = n(6, hidden, sd=0.3)
    ada[[2, 5]] *= gate_scale / 0.3
    return O.DitBranchWeights(
        qkv=n(3 * hd, hidden), proj_out=n(hidden, hd), proj_out_bias=n(hidden, sd=0.1),
        mlp_gate=n(mlp, hidden), mlp_in=n(mlp, hidden), mlp_out=n(hidden, mlp),
        norm_q=rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32),
        norm_k=rng.uniform(0.5, 1.5, HEAD_DIM).astype(np.float32), ada=ada)


def case(seed, shifted=True, params=(2, 16, 16, 1, 8, 8, 16)):
    rng = np.random.default_rng(seed)
    g = geometry(params, shifted)
    video = rng.standard_normal((g.source_tokens, HIDDEN)).astype(np.float32)
    text = rng.standard_normal((g.text_tokens, HIDDEN)).astype(np.float32)
    emb = (rng.standard_normal(HIDDEN * 6) * 0.5).astype(np.float32)
    return g, video, text, emb, make_weights(rng), make_weights(rng)


def torch_block(g, video, text, emb, wv, wt, last_layer, gate_first=False, eps_outside=False, sigmoid=False):
    """The reference module's arithmetic with torch routines, float64; the
    attention layer is the same pinned fp32 oracle."""
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    emb_t = t(emb)

    def rms(x):
        if eps_outside:
            return x / (x.pow(2).mean(-1, keepdim=True).sqrt() + EPS)
        return F.rms_norm(x, (x.shape[-1],), eps=EPS)

    def ada(h, w, layer, mode):
        dim = h.shape[-1]
        mod = emb_t.reshape(1, dim, 2, 3)[0, :, layer, :].transpose(0, 1)
        shift_a, scale_a, gate_a = mod.unbind(0)
        a = t(w.ada)
        shift_b, scale_b, gate_b = a[3 * layer], a[3 * layer + 1], a[3 * layer + 2]
        if mode == "in":
            return h * (scale_a + scale_b) + (shift_a + shift_b)
        return h * (gate_a + gate_b)

    ws = (wv, wt)
    xs = (t(video), t(text))
    attn_in = []
    for br in range(2):
        h = rms(xs[br])
        if br == 0 or not last_layer:
            h = ada(h, ws[br], 0, "in")
        attn_in.append(F.linear(h, t(ws[br].qkv)).reshape(-1, 3, HEADS, HEAD_DIM))
    gam = (wv.norm_q, wv.norm_k, wt.norm_q, wt.norm_k)
    qv, qt = O.qk_norm_inputs(attn_in[0].numpy().astype(np.float32), attn_in[1].numpy().astype(np.float32), gam, EPS)
    av, at = O.awa_layer(g, qv, qt, HEADS, HEAD_DIM)
    outs = []
    for br, att in enumerate((av, at)):
        w = ws[br]
        if gate_first:
            h = ada(F.linear(t(att.reshape(-1, HEADS * HEAD_DIM)), t(w.proj_out)), w, 0, "out") + t(w.proj_out_bias)
        else:
            h = F.linear(t(att.reshape(-1, HEADS * HEAD_DIM)), t(w.proj_out), t(w.proj_out_bias))
        if br == 1 and last_layer:
            y = h + xs[br]
            outs.append((y + y).numpy())
            continue
        if not gate_first:
            h = ada(h, w, 0, "out")
        y = h + xs[br]
        m = ada(rms(y), w, 1, "in")
        act = torch.sigmoid if sigmoid else F.silu
        m = F.linear(act(F.linear(m, t(w.mlp_gate))) * F.linear(m, t(w.mlp_in)), t(w.mlp_out))
        outs.append((ada(m, w, 1, "out") + y).numpy())
    return outs


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("last_layer", [False, True])
@pytest.mark.parametrize("shifted", [False, True])
def test_block_matches_torch_composition(last_layer, shifted):
    g, video, text, emb, wv, wt = case(11 + shifted + 2 * last_layer, shifted)
    ov, ot = O.dit_block(g, video, text, emb, wv, wt, HEADS, HEAD_DIM, EPS, last_layer)
    tv, tt = torch_block(g, video, text, emb, wv, wt, last_layer)
    assert rel(ov, tv) < 1e-12 and rel(ot, tt) < 1e-12


def test_zero_gates_make_the_block_the_identity():
    g, video, text, emb, wv, wt = case(5)
    e = emb.reshape(-1, 2, 3)
    e[:, :, 2] = 0.0  # embedding gates
    for w in (wv, wt):
        w.ada[[2, 5]] = 0.0  # learned gates
    ov, ot = O.dit_block(g, video, text, e.reshape(-1), wv, wt, HEADS, HEAD_DIM, EPS, False)
    np.testing.assert_array_equal(ov, video.astype(np.float64))
    np.testing.assert_array_equal(ot, text.astype(np.float64))


def test_last_block_doubles_text():
    g, video, text, emb, wv, wt = case(6)
    wt.proj_out[:] = 0.0
    wt.proj_out_bias[:] = 0.0
    _, ot = O.dit_block(g, video, text, emb, wv, wt, HEADS, HEAD_DIM, EPS, True)
    np.testing.assert_array_equal(ot, 2.0 * text.astype(np.float64))


@pytest.mark.parametrize("mistake", ["gate_first", "eps_outside", "sigmoid"])
def test_planted_mistakes_are_rejected(mistake):
    g, video, text, emb, wv, wt = case(7)
    ov, ot = O.dit_block(g, video, text, emb, wv, wt, HEADS, HEAD_DIM, EPS, False)
    tv, tt = torch_block(g, video, text, emb, wv, wt, False, **{mistake: True})
    assert max(rel(ov, tv), rel(ot, tt)) > 1e-6


def test_bf16_mode_rounds_to_bf16():
    """bf16 mode: every output is a bf16 value and stays within the bf16
    budget of the float64 block."""
    g, video, text, emb, wv, wt = case(8)
    ov, ot = O.dit_block(g, video, text, emb, wv, wt, HEADS, HEAD_DIM, EPS, False, bf16=True)
    fv, ft = O.dit_block(g, O.round_bf16(video), O.round_bf16(text), O.round_bf16(emb), wv, wt, HEADS, HEAD_DIM,
                         EPS, False)
    for a in (ov, ot):
        np.testing.assert_array_equal(O.round_bf16(a.astype(np.float32)).astype(np.float64), a)
    assert rel(ov, fv) < 2e-2 and rel(ot, ft) < 2e-2
