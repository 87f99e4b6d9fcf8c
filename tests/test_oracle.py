"""Pins the CPU oracle (CPU only).

Each part of the oracle is checked against something that does not restate
it: the reference's own compiled noise generator (oracle/_ref) and the golden
vectors it wrote, the window geometry the reference's partition yields at the
benchmark shapes, partition / permutation invariants, closed forms evaluated
in float64 (RoPE angles, softmax attention, the single-window layer, which is
plain full attention with 3-D RoPE), textbook algorithms implemented
independently here (std::seed_seq, MT19937 through numpy, Box-Muller), and
torch's round-to-nearest-even bf16 cast. The mutation tests plant plausible
mistakes in the float64 model and show the same comparisons reject them.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

import oracle as O
from awa_cases import CONFIGS, RAGGED
from float64_model import attention64, layer64, layer64_of_rotated, rope_apply64, rope_frequencies64

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# --------------------------------------------------------------------------
# Window geometry at the benchmark shapes. Each row: layer params, then for
# the unshifted and shifted partitions (window count, distinct window lengths
# L = video + text tokens, packed length S). Obtained from the reference's
# partition rule (src/awa/awa_layers.cpp:53-88) at these shapes.
GEOMETRY = {
    "production_256": ((1, 16, 16, 4, 3, 3, 64), (1, {320}, 320), (1, {320}, 320)),
    "image_1x16x16": ((1, 16, 16, 1, 8, 8, 64), (4, {128}, 512), None),
    "clip_2x16x16": ((2, 16, 16, 1, 8, 8, 64), (4, {192}, 768), (9, {96, 128, 192}, 1088)),
    "clip_9x16x16": ((9, 16, 16, 3, 8, 8, 64), (12, {256}, 3072),
                     (36, {80, 96, 112, 128, 160, 192, 256}, 4608)),
    "clip_9x32x32": ((9, 32, 32, 3, 8, 8, 64), (48, {256}, 12288), (100, None, 15616)),
    "clip_31x16x16": ((31, 16, 16, 8, 8, 8, 64), (32, {256, 320}, 9984), (81, {80, 96, 128, 192, 320}, 13120)),
}

# Per-axis intervals of shifted partitions at the benchmark shapes: half-window
# shift, bounds truncated toward zero, then clipped.
AXIS_SPLITS = {
    ("clip_2x16x16", "h"): [(0, 4), (4, 12), (12, 16)],
    ("clip_2x16x16", "t"): [(0, 2)],
    ("clip_9x16x16", "t"): [(0, 1), (1, 4), (4, 7), (7, 9)],
    ("clip_31x16x16", "t"): [(0, 2), (2, 6), (6, 10), (10, 14), (14, 18), (18, 22), (22, 26), (26, 30), (30, 31)],
}


def geometry(name: str, shifted: bool) -> O.Geometry:
    t, h, w, nt, nh, nw, tx = CONFIGS[name]
    return O.Geometry(t, h, w, nt, nh, nw, tx, shifted)


def check_partition(g: O.Geometry, windows: np.ndarray) -> None:
    """Windows are non-empty boxes inside the grid, cover every token exactly
    once, are Cartesian products of per-axis partitions and come in w-outer,
    h, t-inner order."""
    assert len(windows) > 0
    cover = np.zeros((g.t, g.h, g.w), np.int32)
    for t0, t1, h0, h1, w0, w1 in windows:
        assert 0 <= t0 < t1 <= g.t and 0 <= h0 < h1 <= g.h and 0 <= w0 < w1 <= g.w
        cover[t0:t1, h0:h1, w0:w1] += 1
    assert np.all(cover == 1)
    axes = []
    for a in range(3):
        iv = sorted({(int(r[2 * a]), int(r[2 * a + 1])) for r in windows})
        assert iv[0][0] == 0 and all(iv[i][1] == iv[i + 1][0] for i in range(len(iv) - 1))
        axes.append(iv)
    assert len(windows) == len(axes[0]) * len(axes[1]) * len(axes[2])
    order = [(int(r[4]), int(r[2]), int(r[0])) for r in windows]
    assert order == sorted(order), "window order must be w outer, h, t inner"


@pytest.mark.parametrize("name", list(GEOMETRY))
@pytest.mark.parametrize("shifted", [False, True])
def test_window_geometry_at_benchmark_shapes(name, shifted):
    params, unshifted, shifted_expect = GEOMETRY[name]
    expect = shifted_expect if shifted else unshifted
    if expect is None:
        pytest.skip("no shifted layer at this shape")
    g = geometry(name, shifted)
    windows = O.make_windows(g)
    check_partition(g, windows)
    m = O.build_maps(g)
    lengths = np.diff(m.cu_seqlens)
    nwin, lens, S = expect
    assert m.window_count == nwin == len(windows)
    if lens is not None:
        assert set(lengths.tolist()) == lens
    assert m.sequence_tokens == S
    assert np.array_equal(lengths, [(r[1] - r[0]) * (r[3] - r[2]) * (r[5] - r[4]) + g.text_tokens for r in windows])


def test_window_axis_splits_and_first_windows():
    for (name, axis), splits in AXIS_SPLITS.items():
        windows = O.make_windows(geometry(name, True))
        a = "thw".index(axis)
        assert sorted({(int(r[2 * a]), int(r[2 * a + 1])) for r in windows}) == splits, (name, axis)
    first = O.make_windows(geometry("clip_2x16x16", True))[:4].tolist()
    assert first == [[0, 2, 0, 4, 0, 4], [0, 2, 4, 12, 0, 4], [0, 2, 12, 16, 0, 4], [0, 2, 0, 4, 4, 12]]


def test_window_counts_other_nt():
    # n_t in {3, 4} gives a 3-frame window at T = 9; n_t in {8, 9} a 4-frame window at T = 31.
    for nt, expect in ((3, 3), (4, 3)):
        w = O.make_windows(O.Geometry(9, 16, 16, nt, 8, 8, 64, False))
        assert w[0][1] - w[0][0] == expect
    for nt in (8, 9):
        w = O.make_windows(O.Geometry(31, 16, 16, nt, 8, 8, 64, False))
        assert w[0][1] - w[0][0] == 4 and w[:, 1].max() == 31


@pytest.mark.parametrize("params", RAGGED + [(2, 5, 3, 1, 1, 1, 1), (30, 2, 2, 7, 1, 1, 4), (40, 3, 90, 6, 2, 9, 2)])
@pytest.mark.parametrize("shifted", [False, True])
def test_partition_invariants_ragged(params, shifted):
    g = O.Geometry(*params[:6], params[6], shifted)
    check_partition(g, O.make_windows(g))


def test_python_round_positive_is_bankers_rounding():
    values = [0.5, 1.5, 2.5, 3.5, 4.5, 59.5, 60.5, 44.999999999, 45.0000001, 0.49999999999999994, 2.675,
              1e6 + 0.5, 123456.5]
    rng = np.random.default_rng(7)
    values += (rng.random(2000) * 200).tolist() + (np.arange(0, 400) * 0.5).tolist()
    for v in values:
        if v <= 0:
            continue
        assert O.python_round_positive(v) == round(v), v


def test_window_size_uses_rescaled_area():
    # 16x16 and 32x32 grids both rescale to 60x60: 8 windows per axis give 8-token windows.
    for side in (16, 32, 24):
        w = O.make_windows(O.Geometry(1, side, side, 1, 8, 8, 1, False))
        assert w[0][3] - w[0][2] == min(8, side) and w[0][5] - w[0][4] == min(8, side)
    # 9x16 (non-square): scale = sqrt(3600/144) = 5 -> 45 x 80, windows ceil(45/3) = 15 -> clipped to 9, ceil(80/4) = 20
    w = O.make_windows(O.Geometry(1, 9, 16, 1, 3, 4, 1, False))
    assert len(w) == 1 and w[0].tolist() == [0, 1, 0, 9, 0, 16]


# --------------------------------------------------------------------------
# Index maps

@pytest.mark.parametrize("name", ["image_1x16x16", "clip_2x16x16", "clip_9x16x16", "clip_31x16x16"])
@pytest.mark.parametrize("shifted", [False, True])
def test_maps_are_consistent_permutations(name, shifted):
    g = geometry(name, shifted)
    m = O.build_maps(g)
    N, T = g.source_tokens, g.text_tokens
    assert m.status == 0
    cu = m.cu_seqlens
    assert cu[0] == 0 and cu[-1] == m.sequence_tokens and np.all(np.diff(cu) > T)
    windows = O.make_windows(g)
    video_order = []
    for wi, (t0, t1, h0, h1, w0, w1) in enumerate(windows):
        rows = m.sequence_index[cu[wi]:cu[wi + 1]]
        tt, hh, ww = np.meshgrid(np.arange(t0, t1), np.arange(h0, h1), np.arange(w0, w1), indexing="ij")
        video = ((tt * g.h + hh) * g.w + ww).reshape(-1)
        assert np.array_equal(rows[:-T], video), "video rows in t, h, w order inside the window"
        assert np.array_equal(rows[-T:], N + np.arange(T)), "text appended after each window"
        assert np.array_equal(m.text_positions[wi * T:(wi + 1) * T], cu[wi + 1] - T + np.arange(T))
        video_order.append(video)
    assert np.array_equal(m.target, np.concatenate(video_order)), "video tokens in packed order"
    assert np.array_equal(m.sequence_index[m.video_positions], np.arange(N))
    assert np.array_equal(np.sort(m.sequence_index[m.sequence_index < N]), np.arange(N))


def test_pack_is_a_gather_by_the_maps():
    g = geometry("clip_2x16x16", True)
    heads, d = 2, 8
    rng = np.random.default_rng(3)
    video = rng.standard_normal((g.source_tokens, 3, heads, d)).astype(np.float32)
    text = rng.standard_normal((g.text_tokens, 3, heads, d)).astype(np.float32)
    packed, cu = O.pack_forward(g, video, text, heads, d)
    m = O.build_maps(g)
    src = np.concatenate([video, text])[m.sequence_index]
    assert np.array_equal(packed, src)
    assert cu.dtype == np.float32 and np.array_equal(cu, m.cu_seqlens.astype(np.float32))


@pytest.mark.parametrize("text_order", ["cpu", "gpu"])
def test_pack_unpack_round_trip(text_order):
    """Unpack of the packed V rows returns the video V exactly and the text V
    up to the rounding of a mean of identical copies."""
    for shifted in (False, True):
        g = geometry("clip_9x16x16", shifted)
        heads, d = 2, 16
        rng = np.random.default_rng(11)
        video = rng.standard_normal((g.source_tokens, 3, heads, d)).astype(np.float32)
        text = rng.standard_normal((g.text_tokens, 3, heads, d)).astype(np.float32)
        packed, _ = O.pack_forward(g, video, text, heads, d)
        v_out, t_out = O.unpack_forward(g, np.ascontiguousarray(packed[:, 2]), heads, d, text_order)
        assert np.array_equal(v_out, video[:, 2])
        np.testing.assert_allclose(t_out, text[:, 2], rtol=4e-6, atol=1e-7)


# --------------------------------------------------------------------------
# RoPE


def window_coordinates(g: O.Geometry) -> np.ndarray:
    """[S][3] RoPE coordinates of every packed row, derived from the windows:
    video (T_x + t - t0, h - h0, w - w0), text (k, k, k)."""
    out = []
    for t0, t1, h0, h1, w0, w1 in O.make_windows(g):
        for t in range(t0, t1):
            for h in range(h0, h1):
                for w in range(w0, w1):
                    out.append((g.text_tokens + t - t0, h - h0, w - w0))
        out += [(k, k, k) for k in range(g.text_tokens)]
    return np.array(out, np.int64)


@pytest.mark.parametrize("name,shifted", [("clip_2x16x16", True), ("clip_9x16x16", False), ("production_256", False)])
def test_rope_table_closed_form(name, shifted):
    g = geometry(name, shifted)
    table = O.rope_table(g).astype(np.float64)
    coords = window_coordinates(g)
    assert table.shape == (len(coords), 252)
    f = rope_frequencies64()
    angle = coords[:, :, None] * f[None, None, :]            # [S][axis][pair]
    cos = np.repeat(np.cos(angle).reshape(len(coords), 63), 2, axis=1)  # pairs duplicated
    sin = np.repeat(np.sin(angle).reshape(len(coords), 63), 2, axis=1)
    # fp32 angle = fl(coord * fl(freq)): |error| <= |angle| * 2^-23 (+ freq rounding)
    tol = 2.5e-7 * (1.0 + np.repeat(np.abs(angle).reshape(len(coords), 63), 2, axis=1))
    assert np.all(np.abs(table[:, :126] - cos) <= tol)
    assert np.all(np.abs(table[:, 126:] - sin) <= tol)
    # Pair 0 of each axis has frequency 1: the table holds cos/sin of the coordinate itself.
    for a in range(3):
        np.testing.assert_allclose(table[:, 42 * a], np.cos(coords[:, a]), atol=1e-6)


def test_mmrope_forward_matches_closed_form():
    g = geometry("clip_2x16x16", True)
    heads, d = 2, 128
    rng = np.random.default_rng(5)
    S = O.build_maps(g).sequence_tokens
    packed = rng.standard_normal((S, 3, heads, d)).astype(np.float32)
    out = O.mmrope_forward(packed, O.rope_table(g), heads, d)
    coords = window_coordinates(g)
    expect = rope_apply64(packed[:, :2], coords)
    np.testing.assert_allclose(out[:, :2], expect, atol=5e-5)
    assert np.array_equal(out[:, :2, :, 126:], packed[:, :2, :, 126:]), "dims past rope_dim pass through"
    assert np.array_equal(out[:, 2], packed[:, 2]), "V is not rotated"


# --------------------------------------------------------------------------
# Attention


@pytest.mark.parametrize("order", ["cpu", "kahan"])
@pytest.mark.parametrize("d", [16, 64, 128])
def test_attention_brute_force(order, d):
    rng = np.random.default_rng(d)
    lengths = [5, 1, 33, 70]
    heads = 3
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    packed = (rng.standard_normal((cu[-1], 3, heads, d)) * 1.5).astype(np.float32)
    out = O.attention(packed, cu, heads, d, order)
    for i in range(len(lengths)):
        sl = slice(cu[i], cu[i + 1])
        ref = attention64(packed[sl, 0], packed[sl, 1], packed[sl, 2])
        np.testing.assert_allclose(out[sl], ref, atol=1e-5, rtol=0)


def test_attention_orders_agree_and_differ_only_in_rounding():
    g = geometry("clip_2x16x16", True)
    heads, d = 2, 128
    rng = np.random.default_rng(9)
    m = O.build_maps(g)
    packed = rng.standard_normal((m.sequence_tokens, 3, heads, d)).astype(np.float32)
    a = O.attention(packed, m.cu_seqlens, heads, d, "cpu")
    b = O.attention(packed, m.cu_seqlens, heads, d, "kahan")
    assert np.max(np.abs(a - b)) < 2e-6


def test_single_window_layer_is_full_attention_with_3d_rope():
    """Production 256x256 image layer: one window covers the grid, so the AWA
    layer is ordinary softmax attention over N + T_x tokens with 3-D RoPE."""
    g = geometry("production_256", False)
    heads, d = 2, 128
    video = O.fill_gaussian(g.source_tokens * 3 * heads * d, 20260823, 0).reshape(g.source_tokens, 3, heads, d)
    text = O.fill_gaussian(g.text_tokens * 3 * heads * d, 20260823, 1).reshape(g.text_tokens, 3, heads, d)
    N, T = g.source_tokens, g.text_tokens
    coords = np.concatenate([
        np.stack([T + np.zeros(N, np.int64), np.arange(N) // 16, np.arange(N) % 16], 1),
        np.repeat(np.arange(T)[:, None], 3, 1)])
    x = np.concatenate([video, text])
    ref = attention64(rope_apply64(x[:, 0], coords), rope_apply64(x[:, 1], coords), x[:, 2])
    for order in ("cpu", "kahan"):
        v, t = O.awa_layer(g, video, text, heads, d, attention_order=order, text_order="cpu" if order == "cpu" else "gpu")
        assert np.max(np.abs(v - ref[:N])) < 1e-5
        assert np.max(np.abs(t - ref[N:])) < 1e-5


@pytest.mark.parametrize("name,shifted", [("clip_2x16x16", True), ("image_1x16x16", False)])
def test_layer_matches_float64_definition(name, shifted):
    g = geometry(name, shifted)
    heads, d = 2, 128
    rng = np.random.default_rng(21)
    video = rng.standard_normal((g.source_tokens, 3, heads, d)).astype(np.float32)
    text = rng.standard_normal((g.text_tokens, 3, heads, d)).astype(np.float32)
    ref_v, ref_t = layer64(g, video, text)
    for order, text_order in (("cpu", "cpu"), ("kahan", "gpu")):
        v, t = O.awa_layer(g, video, text, heads, d, attention_order=order, text_order=text_order)
        assert np.max(np.abs(v - ref_v)) < 1e-5
        assert np.max(np.abs(t - ref_t)) < 1e-5


@pytest.mark.parametrize("name,shifted", [("clip_2x16x16", True), ("image_1x16x16", False)])
def test_layer_of_rotated_inputs(name, shifted):
    """The float64 layer after the fp32 rotation (the large-magnitude tests'
    attention-arithmetic reference) is the float64 layer up to that
    rotation's rounding (a few 1e-7 at unit scale), and the Kahan-order
    oracle, which rotates identically, is closer to it than to the fully
    float64 layer."""
    g = geometry(name, shifted)
    heads, d = 2, 128
    rng = np.random.default_rng(23)
    video = rng.standard_normal((g.source_tokens, 3, heads, d)).astype(np.float32)
    text = rng.standard_normal((g.text_tokens, 3, heads, d)).astype(np.float32)
    rv, rt = layer64_of_rotated(g, video, text)
    ev, et = layer64(g, video, text)
    assert np.max(np.abs(rv - ev)) < 2e-6 and np.max(np.abs(rt - et)) < 2e-6
    ov, ot = O.awa_layer(g, video, text, heads, d)
    assert np.max(np.abs(ov - rv)) < np.max(np.abs(ov - ev)) and np.max(np.abs(ov - rv)) < 1e-6
    # A planted mistake (text rows summed over windows, not averaged) is caught.
    m = O.build_maps(g)
    assert np.max(np.abs(rt * m.window_count - et)) > 1e-2


@pytest.mark.parametrize("mistake", ["sin_sign", "pair_swap", "text_offset", "no_scale"])
def test_planted_mistakes_are_caught(mistake):
    """The float64 model with one plausible mistake planted disagrees with the
    oracle far beyond the tolerances used above."""
    g = geometry("clip_2x16x16", True)
    heads, d = 1, 128
    rng = np.random.default_rng(21)
    video = rng.standard_normal((g.source_tokens, 3, heads, d)).astype(np.float32)
    text = rng.standard_normal((g.text_tokens, 3, heads, d)).astype(np.float32)
    v, t = O.awa_layer(g, video, text, heads, d)
    bad_v, bad_t = layer64(g, video, text, mistake)
    assert max(np.max(np.abs(v - bad_v)), np.max(np.abs(t - bad_t))) > 1e-2


# --------------------------------------------------------------------------
# Noise generator (src/sampler/sampler.cpp:37-61)

def seed_seq_generate(seeds, n=624):
    """std::seed_seq::generate as specified by the C++ standard ([rand.util.seedseq])."""
    mask = 0xFFFFFFFF
    b = [0x8B8B8B8B] * n
    s = len(seeds)
    t = 11 if n >= 623 else (7 if n >= 68 else (5 if n >= 39 else (3 if n >= 7 else (n - 1) // 2)))
    p = (n - t) // 2
    q = p + t
    m = max(s + 1, n)

    def T(x):
        return x ^ (x >> 27)

    for k in range(m):
        r1 = (1664525 * T(b[k % n] ^ b[(k + p) % n] ^ b[(k - 1) % n])) & mask
        if k == 0:
            r2 = (r1 + s) & mask
        elif k <= s:
            r2 = (r1 + k % n + seeds[k - 1]) & mask
        else:
            r2 = (r1 + k % n) & mask
        b[(k + p) % n] = (b[(k + p) % n] + r1) & mask
        b[(k + q) % n] = (b[(k + q) % n] + r2) & mask
        b[k % n] = r2
    for k in range(m, m + n):
        r3 = (1566083941 * T((b[k % n] + b[(k + p) % n] + b[(k - 1) % n]) & mask)) & mask
        r4 = (r3 - k % n) & mask
        b[(k + p) % n] ^= r3
        b[(k + q) % n] ^= r4
        b[k % n] = r4
    return np.array(b, np.uint32)


def gaussian_numpy(count: int, seed: int, stream: int) -> np.ndarray:
    """MT19937 (numpy's implementation) seeded with the seed_seq words, then
    Box-Muller in float64 with midpoint uniforms, cast to float32."""
    words = seed_seq_generate([seed, stream & 0xFFFFFFFF, (stream >> 32) & 0xFFFFFFFF])
    bg = np.random.MT19937(0)
    bg.state = {"bit_generator": "MT19937", "state": {"key": words, "pos": 624}}
    raw = bg.random_raw(2 * ((count + 1) // 2)).astype(np.float64)
    u = (raw + 0.5) / 4294967296.0
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    a = 2.0 * math.pi * u[1::2]
    out = np.empty(2 * len(r), np.float32)
    out[0::2] = (r * np.cos(a)).astype(np.float32)
    out[1::2] = (r * np.sin(a)).astype(np.float32)
    return out[:count]


@pytest.mark.parametrize("seed,stream", [(666, 7), (20260825, (1 << 32) + 3), (0, 0)])
def test_seed_seq_words_match_the_standard_algorithm(seed, stream):
    assert np.array_equal(O.seed_seq_words(seed, stream),
                          seed_seq_generate([seed, stream & 0xFFFFFFFF, stream >> 32]))


@pytest.mark.parametrize("seed,stream,count", [(666, 7, 4097), (20260824, 1, 1000), (1, (1 << 40) + 9, 33)])
def test_gaussian_matches_independent_mt19937_box_muller(seed, stream, count):
    a = O.fill_gaussian(count, seed, stream)
    b = gaussian_numpy(count, seed, stream)
    ulp = np.spacing(np.abs(b).astype(np.float32))
    assert np.all(np.abs(a - b) <= ulp)
    assert np.mean(a == b) > 0.999


def test_gaussian_matches_reference_golden_vectors():
    with open(os.path.join(GOLDEN, "sampler_vectors.json")) as f:
        cases = json.load(f)["cases"]
    assert cases
    for c in cases:
        expect = np.array([int(x, 16) for x in c["bits"]], np.uint32)
        got = O.fill_gaussian(c["count"], c["seed"], c["stream"]).view(np.uint32)
        assert np.array_equal(got, expect), (c["seed"], c["stream"])


def test_gaussian_matches_compiled_reference():
    ref = O.ref_sampler()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    for seed, stream, count in ((666, 7, 131073), (20260825, 64, 50001), (3, (1 << 33) + 1, 7)):
        buf = np.zeros(count, np.float32)
        assert ref.ref_fill_gaussian_noise(buf.ctypes.data, count, seed, stream) == 0
        assert np.array_equal(O.fill_gaussian(count, seed, stream).view(np.uint32), buf.view(np.uint32))


def test_gaussian_statistics_as_the_reference_smoke_test():
    # tools/sampler_smoke.cpp:40-70
    n = 131073
    x = O.fill_gaussian(n, 666, 7).astype(np.float64)
    assert np.all(np.isfinite(x))
    assert abs(x.mean()) < 0.02 and abs(x.var() - 1.0) < 0.04
    assert np.array_equal(O.fill_gaussian(n, 666, 7), O.fill_gaussian(n, 666, 7))
    for stream in (8, (1 << 32) + 7):
        assert not np.array_equal(O.fill_gaussian(n, 666, stream), O.fill_gaussian(n, 666, 7))
    assert not np.array_equal(O.fill_gaussian(n, 667, 7), O.fill_gaussian(n, 666, 7))
    with pytest.raises(ValueError):
        O.fill_gaussian(0, 0, 0)


# --------------------------------------------------------------------------
# bf16 rounding

def test_round_bf16_matches_torch_rne():
    torch = pytest.importorskip("torch")
    import awa_hip

    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        # exact ties between two bf16 values, both parities
        ((np.arange(1, 2000, dtype=np.uint32) << 16) | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1e-40, -1e-40, 3.3895314e38, -3.3895314e38, np.inf, -np.inf], np.float32),
    ])
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.round_bf16_bits(x), t)
    assert np.array_equal(awa_hip.f32_to_bf16_bits(x), t)


# ---- DitRMSNorm restatement (src/dit/shader/dit_rmsnorm.comp) ----

def _rms_f64(x, gamma, eps):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return y if gamma is None else y * np.asarray(gamma, np.float64)


@pytest.mark.parametrize("width", [128, 200, 2560])
@pytest.mark.parametrize("affine", [False, True])
def test_rmsnorm_matches_float64_definition(width, affine):
    rng = np.random.RandomState(width + affine)
    x = (rng.randn(33, width) * rng.uniform(0.01, 50, (33, 1))).astype(np.float32)
    gamma = rng.uniform(-2, 2, width).astype(np.float32) if affine else None
    got = O.rmsnorm(x, gamma, 1e-5)
    ref = _rms_f64(x, gamma, 1e-5)
    scale = np.abs(ref).max(-1, keepdims=True) + 1e-30
    # Each output is a few fp32 roundings away from the exact value.
    assert np.max(np.abs(got - ref) / scale) < 4e-6 * (1 + (gamma is not None))


def test_rmsnorm_closed_forms():
    eps = 1e-5
    # A constant row c gives c / sqrt(c^2 + eps) times gamma.
    for c in (0.0, 1.0, -3.5, 1e3):
        x = np.full((1, 128), c, np.float32)
        g = np.linspace(-1, 1, 128).astype(np.float32)
        got = O.rmsnorm(x, g, eps)
        want = (np.float64(c) / np.sqrt(np.float64(c) * c + eps)) * g.astype(np.float64)
        assert np.allclose(got, want, rtol=1e-6, atol=1e-7), c
    # With eps = 0 the norm is scale-invariant and the mean square of the
    # output is 1.
    x = np.random.RandomState(3).randn(7, 128).astype(np.float32)
    a = O.rmsnorm(x, None, 0.0)
    b = O.rmsnorm(np.float32(8.0) * x, None, 0.0)
    assert np.array_equal(a, b)  # a power-of-two scale is exact
    assert np.allclose((a.astype(np.float64) ** 2).mean(-1), 1.0, atol=1e-6)


def test_rmsnorm_rejects_planted_mistakes():
    """A sum instead of a mean, or eps outside the root, fails the float64 check."""
    rng = np.random.RandomState(9)
    x = rng.randn(4, 128).astype(np.float32)
    ref = _rms_f64(x, None, 1e-5)
    wrong_sum = x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-5)
    wrong_eps = x / (np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True)) + 1e-5)
    got = O.rmsnorm(x, None, 1e-5)
    assert np.max(np.abs(got - ref)) < 1e-5
    assert np.max(np.abs(wrong_sum - ref)) > 1e-2
    x_small = (rng.randn(4, 128) * 1e-3).astype(np.float32)
    ref_small = _rms_f64(x_small, None, 1e-5)
    wrong_small = x_small / (np.sqrt((x_small.astype(np.float64) ** 2).mean(-1, keepdims=True)) + 1e-5)
    assert np.max(np.abs(O.rmsnorm(x_small, None, 1e-5) - ref_small)) < 1e-5
    assert np.max(np.abs(wrong_small - ref_small)) > 1e-2


def test_qk_norm_inputs_normalises_q_and_k_only():
    rng = np.random.RandomState(5)
    video = rng.randn(6, 3, 2, 128).astype(np.float32)
    text = rng.randn(3, 3, 2, 128).astype(np.float32)
    gammas = [rng.uniform(0.5, 1.5, 128).astype(np.float32) for _ in range(4)]
    v, t = O.qk_norm_inputs(video, text, gammas, 1e-5)
    assert np.array_equal(v[:, 2], video[:, 2]) and np.array_equal(t[:, 2], text[:, 2])
    for src, dst, gq, gk in ((video, v, gammas[0], gammas[1]), (text, t, gammas[2], gammas[3])):
        assert np.allclose(dst[:, 0], _rms_f64(src[:, 0], gq, 1e-5), rtol=1e-5, atol=1e-6)
        assert np.allclose(dst[:, 1], _rms_f64(src[:, 1], gk, 1e-5), rtol=1e-5, atol=1e-6)


def test_qkv_concat_is_the_qkv_interleave():
    """DitQKVConcat against numpy's concatenation along the head axis (an
    independent formulation), with distinct values per (tensor, token, head,
    feature); a planted head mapping y // 3 instead of y % heads is rejected."""
    tokens, heads, d = 5, 3, 6
    base = np.arange(tokens * heads * d, dtype=np.float32).reshape(tokens, heads, d)
    q, k, v = base, base + 1000.0, base + 2000.0
    got = O.qkv_concat(q, k, v)
    assert np.array_equal(got, np.concatenate([q, k, v], axis=1))
    planted = np.stack([(q, k, v)[y // heads][:, y // 3] for y in range(3 * heads)], axis=1)
    assert not np.array_equal(got, planted)
    with pytest.raises(ValueError):
        O.qkv_concat(q, k, v[:, :2])
