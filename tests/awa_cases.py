"""Shared geometry cases and device helpers for the AWA tests."""

from __future__ import annotations

import numpy as np

import oracle as O

HEAD_DIM = 128
HEADS = 20
TEXT = 64

# Layer params (t, h, w, n_t, n_h, n_w, T_x) of the workloads the tests and the
# benchmark use: the production 256x256 image layer, then the 1-frame image,
# 5-frame, 33-frame, 512x512 and 121-frame clips.
CONFIGS = {
    "production_256": (1, 16, 16, 4, 3, 3, 64),
    "image_1x16x16": (1, 16, 16, 1, 8, 8, 64),
    "clip_2x16x16": (2, 16, 16, 1, 8, 8, 64),
    "clip_9x16x16": (9, 16, 16, 3, 8, 8, 64),
    "clip_9x32x32": (9, 32, 32, 3, 8, 8, 64),
    "clip_31x16x16": (31, 16, 16, 8, 8, 8, 64),
}

# Ragged grids whose windows do not divide the grid (clipped and shifted edges).
RAGGED = [
    (3, 11, 13, 2, 3, 3, 5),
    (5, 7, 19, 2, 2, 4, 7),
    (1, 9, 9, 1, 2, 2, 3),
    (4, 6, 10, 3, 5, 2, 17),
]


def geometry(params, shifted: bool) -> O.Geometry:
    t, h, w, nt, nh, nw, tx = params
    return O.Geometry(t, h, w, nt, nh, nw, tx, bool(shifted))


def qkv_inputs(g: O.Geometry, heads: int, head_dim: int, seed: int):
    """Seeded N(0,1) video [N][3][H][d] and text [T_x][3][H][d] fp32 QKV from the
    reference's generator (mt19937 + seed_seq + Box-Muller), stream 0 / 1."""
    n = g.source_tokens * 3 * heads * head_dim
    video = O.fill_gaussian(n, seed, 0).reshape(g.source_tokens, 3, heads, head_dim)
    text = O.fill_gaussian(g.text_tokens * 3 * heads * head_dim, seed, 1).reshape(g.text_tokens, 3, heads, head_dim)
    return video, text


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref|, the bf16 gate. Also prints the Frobenius
    relative error and per-element statistics of the same comparison."""
    d = np.abs(got.astype(np.float64) - np.asarray(ref, np.float64))
    r = np.asarray(ref, np.float64)
    gate = float(np.max(d) / max(np.max(np.abs(r)), 1e-30))
    fro = float(np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30))
    print(f"  bf16 check: max rel {gate:.3g}, Frobenius rel {fro:.3g}, mean |d| {np.mean(d):.3g}, "
          f"p99.9 |d| {np.quantile(d, 0.999):.3g}, max |d| {np.max(d):.3g} over {d.size} elements", flush=True)
    return gate


def abs_err(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.max(np.abs(got.astype(np.float64) - ref)))
