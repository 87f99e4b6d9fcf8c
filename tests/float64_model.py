"""The AWA layer in float64 from its definition (test infrastructure).

Per window: gather the window's video tokens and the text tokens, rotate Q
and K with window-local 3-D RoPE (interleaved pairs, 21 frequencies per axis,
10000^(-2p/42)), softmax attention scaled by 1/sqrt(d), scatter video rows
back and average the text rows over windows (src/awa/awa_layers.cpp:382-458,
:599-689, :867-953, :1062-1120). Independent of the oracle's C++ code: the
oracle tests pin the oracle against it, and the large-magnitude GPU tests use
it as the exact reference.
"""

from __future__ import annotations

import math

import numpy as np

import oracle as O


def rope_frequencies64(axis_dim: int = 42) -> np.ndarray:
    return 10000.0 ** (-(2.0 * np.arange(axis_dim // 2)) / axis_dim)


def rope_apply64(x: np.ndarray, coords: np.ndarray, mistake: str | None = None) -> np.ndarray:
    """Interleaved-pair rotation of features 0..125 (dims 126, 127 pass
    through) with per-axis angles coord * 10000^(-2p/42), in float64."""
    out = x.astype(np.float64).copy()
    f = rope_frequencies64()
    for a in range(3):
        c = coords[:, a].astype(np.float64)
        ang = c[:, None] * f[None, :]
        cs, sn = np.cos(ang), np.sin(ang)
        if mistake == "sin_sign":
            sn = -sn
        e = x[..., 42 * a:42 * a + 42:2].astype(np.float64)
        o = x[..., 42 * a + 1:42 * a + 42:2].astype(np.float64)
        shape = (-1,) + (1,) * (x.ndim - 2) + (21,)
        cs, sn = cs.reshape(shape), sn.reshape(shape)
        if mistake == "pair_swap":
            e, o = o, e
        out[..., 42 * a:42 * a + 42:2] = e * cs - o * sn
        out[..., 42 * a + 1:42 * a + 42:2] = o * cs + e * sn
    return out


def attention64(q, k, v, scale=None):
    """softmax(q k^T * scale) v in float64; q, k, v [L][H][d]."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = np.einsum("qhd,khd->hqk", q.astype(np.float64), k.astype(np.float64)) * scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, v.astype(np.float64))


def layer64(g: O.Geometry, video: np.ndarray, text: np.ndarray, mistake: str | None = None):
    """The whole AWA layer in float64 from its definition: per window, gather
    the window's video tokens and the text tokens, rotate Q and K with
    window-local 3-D RoPE, attend, scatter video rows back and average the
    text rows over windows."""
    N = g.source_tokens
    T = g.text_tokens
    heads, d = video.shape[2], video.shape[3]
    vid = np.zeros((N, heads, d))
    txt = np.zeros((T, heads, d))
    windows = O.make_windows(g)
    for t0, t1, h0, h1, w0, w1 in windows:
        tt, hh, ww = np.meshgrid(np.arange(t0, t1), np.arange(h0, h1), np.arange(w0, w1), indexing="ij")
        idx = ((tt * g.h + hh) * g.w + ww).reshape(-1)
        toff = 0 if mistake == "text_offset" else T
        coords = np.concatenate([
            np.stack([toff + (tt - t0).reshape(-1), (hh - h0).reshape(-1), (ww - w0).reshape(-1)], 1),
            np.repeat(np.arange(T)[:, None], 3, 1)])
        x = np.concatenate([video[idx], text])
        q = rope_apply64(x[:, 0], coords, mistake)
        k = rope_apply64(x[:, 1], coords, mistake)
        scale = 1.0 if mistake == "no_scale" else None
        o = attention64(q, k, x[:, 2], scale)
        vid[idx] = o[:len(idx)]
        txt += o[len(idx):]
    return vid, txt / len(windows)


def layer64_of_rotated(g: O.Geometry, video: np.ndarray, text: np.ndarray):
    """The layer in float64 after the reference's fp32 Pack and MMRoPE (the
    oracle's): Q and K carry the fp32 rotation's rounding, everything after
    it is exact. Its distance to a result measures that result's attention
    arithmetic alone (the fp32 rotation, which every fp32 implementation of
    the reference's data flow shares, cancels)."""
    heads, d = video.shape[2], video.shape[3]
    m = O.build_maps(g)
    packed, _ = O.pack_forward(g, video, text, heads, d)
    roped = O.mmrope_forward(packed, O.rope_table(g), heads, d).reshape(m.sequence_tokens, 3, heads, d)
    out = np.zeros((m.sequence_tokens, heads, d))
    cu = m.cu_seqlens
    for w in range(m.window_count):
        a, b = cu[w], cu[w + 1]
        out[a:b] = attention64(roped[a:b, 0], roped[a:b, 1], roped[a:b, 2])
    vid = out[m.video_positions]
    txt = out[m.text_positions.reshape(m.window_count, g.text_tokens)].mean(axis=0)
    return vid, txt
