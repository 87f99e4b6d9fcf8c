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
