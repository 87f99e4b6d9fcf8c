"""Integer arithmetic the attention kernels do in fp32, checked
exhaustively on the CPU with the same IEEE single-precision operations
(correctly rounded reciprocal, round-to-nearest-even product, truncation).

The attention kernels decode window-local row i into (t, h, w) with
floor(i / d) = int((i + 0.5) * fl(1 / d)) for d = h*w and d = w of the
window box. The host admits windows of fewer than 2^14 rows (their LDS row
tables stop far below that), and a box's spatial area h*w is at most the
rescaled 3600-cell grid; the check covers every i < 2^14 and d <= 4096.
"""

import numpy as np


def test_reciprocal_quotient_is_exact():
    i = np.arange(1 << 14, dtype=np.int64)
    fi = i.astype(np.float32) + np.float32(0.5)
    for d in range(1, 4097):
        inv = np.float32(1.0) / np.float32(d)
        q = (fi * inv).astype(np.int64)  # truncation of a positive float
        np.testing.assert_array_equal(q, i // d, err_msg=f"d={d}")


def test_plain_reciprocal_without_offset_fails():
    """Without the +0.5 offset the product can land just below an integer:
    the check above would catch a decode that dropped it."""
    bad = 0
    i = np.arange(4096, dtype=np.int64)
    for d in range(1, 1025):
        inv = np.float32(1.0) / np.float32(d)
        bad += int(np.count_nonzero((i.astype(np.float32) * inv).astype(np.int64) != i // d))
    assert bad > 0


# ---- The fp32 kernel's integer digit slices (awa_attention_x.hip) ----
# A row value becomes X = trunc(x * 2^(30-e)) (|X| < 2^30) plus the offset
# 128 (1 + 2^8 + 2^16); four such words are byte-transposed by eight
# v_perm_b32 (byte i of the result = byte sel_i of the pair (hi, lo), lo the
# low four bytes) into four int8 slices, the lower three with bit 7 flipped.


def _perm(hi, lo, sel):
    b = [(lo >> (8 * i)) & 255 for i in range(4)] + [(hi >> (8 * i)) & 255 for i in range(4)]
    return sum(b[(sel >> (8 * i)) & 255] << (8 * i) for i in range(4))


def _transpose_digits(x):
    a = _perm(x[1], x[0], 0x06020400)
    b = _perm(x[1], x[0], 0x07030501)
    c = _perm(x[3], x[2], 0x06020400)
    d = _perm(x[3], x[2], 0x07030501)
    return [_perm(d, b, 0x07060302), _perm(c, a, 0x07060302) ^ 0x80808080,
            _perm(d, b, 0x05040100) ^ 0x80808080, _perm(c, a, 0x05040100) ^ 0x80808080]


def _int8(word, i):
    v = (word >> (8 * i)) & 255
    return v - 256 if v >= 128 else v


def test_digit_slices_reconstruct_every_value():
    """Byte i of slice s is digit s of value i; the digits rebuild X exactly
    (X = d1 2^24 + d2 2^16 + d3 2^8 + d4), with d1 in [-64, 64] and the
    balanced lower digits in [-128, 127]."""
    rng = np.random.default_rng(7)
    edge = [2**30 - 1, -(2**30) + 1, 0, -1, 1, 0x7F7F7F, -0x808080, 0x808080, -0x7F7F7F, 2**24, -(2**24)]
    values = edge + [int(v) for v in rng.integers(-(2**30) + 1, 2**30, 40000)]
    values += [0] * (-len(values) % 4)
    for q in range(0, len(values), 4):
        xs = values[q:q + 4]
        w = _transpose_digits([(x + 0x808080) & 0xFFFFFFFF for x in xs])
        for i, x in enumerate(xs):
            d = [_int8(w[s], i) for s in range(4)]
            assert -64 <= d[0] <= 64 and all(-128 <= v <= 127 for v in d[1:]), (x, d)
            assert ((d[0] * 256 + d[1]) * 256 + d[2]) * 256 + d[3] == x, (x, d)


def test_digit_slices_fail_without_the_flip():
    """Leaving out the bit-7 flip of the lower slices breaks reconstruction:
    the check above would catch it."""
    x = [12345, -6789, 2**29, -(2**29)]
    w = _transpose_digits([(v + 0x808080) & 0xFFFFFFFF for v in x])
    w[1] ^= 0x80808080
    d = [_int8(w[s], 0) for s in range(4)]
    assert ((d[0] * 256 + d[1]) * 256 + d[2]) * 256 + d[3] != x[0]


def test_score_classes_fit_exact_int32_and_fp32():
    """With |d1| <= 64 and |d2..d4| <= 128 over 128 features, every weight
    class C_w (w = 2..5, at most four slice products per feature) stays below
    2^23: exact in the int32 MFMA accumulator and in its fp32 conversion."""
    bound = {2: 64 * 64, 3: 2 * 64 * 128, 4: 2 * 64 * 128 + 128 * 128, 5: 2 * 64 * 128 + 2 * 128 * 128}
    for w, per_feature in bound.items():
        assert per_feature * 128 < 2**23, w


def test_class_four_and_five_merge_exactly_in_int32():
    """The exact-score kernel forms C4 * 2^8 + C5 in int32 and converts it
    once: the sum stays below 2^31 at the class bounds, and its rounded
    conversion divided by 2^8 equals the correctly rounded C4 + C5 / 2^8 (the
    single fused multiply-add it replaces) for extreme and random classes."""
    c4_max = 2 * 64 * 128 * 128 + 128 * 128 * 128
    c5_max = (2 * 64 * 128 + 2 * 128 * 128) * 128
    assert c4_max * 256 + c5_max < 2**31
    rng = np.random.default_rng(5)
    c4 = np.concatenate([rng.integers(-c4_max, c4_max + 1, 200000), [c4_max, -c4_max, 0, 1, -1]])
    c5 = np.concatenate([rng.integers(-c5_max, c5_max + 1, 200000), [c5_max, -c5_max, 255, -255, 127]])
    merged = (c4 * 256 + c5).astype(np.int64)
    assert np.all(np.abs(merged) < 2**31)
    got = merged.astype(np.float32) / np.float32(256)
    # C4 + C5 / 2^8 is exact in float64 (at most 31 significant bits); its
    # float32 rounding is the fused multiply-add's result.
    want = (c4.astype(np.float64) + c5.astype(np.float64) / 256.0).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
