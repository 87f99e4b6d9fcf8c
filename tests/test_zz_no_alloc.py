"""awa_forward_noalloc: the fused layer with its text rows in the library's
static per-GPU scratch buffer instead of the plan's workspace. It runs the
same kernels as awa_forward, so its outputs must be bit-identical to
awa_forward's on the same inputs. Each no-alloc call runs first, on a fresh
plan whose work list awa_plan_upload built (awa_plan_desc.heads), and the
device's free memory is the same before and after it; awa_forward then runs on
the same plan for the comparison. Two calls in a row, the second on a smaller
layer, then the clean rejections (text rows beyond the buffer, a plan with no
work list for the head count)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import awa_hip as A
from awa_cases import CONFIGS, HEAD_DIM

pytestmark = pytest.mark.gpu


class Layer:
    """Device QKV (seeded N(0,1)) and outputs for one layer geometry."""

    def __init__(self, params, shifted, heads, in_elem, out_elem, seed):
        t, h, w, nt, nh, nw, tx = params
        self.params, self.shifted = params, shifted
        self.n, self.tx, self.heads, self.out_elem = t * h * w, tx, heads, out_elem
        self.plan = A.Plan(A.LayerParams(t, h, w, nt, nh, nw, tx, shifted), heads=heads)
        self.plan.upload()
        row = 3 * heads * HEAD_DIM
        self.vq = A.DeviceBuffer(self.n * row * in_elem)
        self.tq = A.DeviceBuffer(tx * row * in_elem)
        self.vq.fill_normal(self.n * row, in_elem, seed)
        self.tq.fill_normal(tx * row, in_elem, seed + 1)
        self.vq_blob = A.mat(self.vq.ptr, HEAD_DIM, 3 * heads, self.n, in_elem)
        self.tq_blob = A.mat(self.tq.ptr, HEAD_DIM, 3 * heads, tx, in_elem)

    def outputs(self):
        vo = A.DeviceBuffer(self.n * self.heads * HEAD_DIM * self.out_elem)
        to = A.DeviceBuffer(self.tx * self.heads * HEAD_DIM * self.out_elem)
        return (vo, to, A.mat(vo.ptr, HEAD_DIM, self.heads, self.n, self.out_elem),
                A.mat(to.ptr, HEAD_DIM, self.heads, self.tx, self.out_elem))

    def read(self, vo, to):
        dt = np.float32 if self.out_elem == 4 else np.uint16
        return (vo.download((self.n * self.heads * HEAD_DIM,), dt), to.download((self.tx * self.heads * HEAD_DIM,), dt))


def free_device_bytes() -> int:
    """hipMemGetInfo's free bytes on the current device."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def warm_kernels(layer: Layer, compute: int) -> None:
    """Loads the kernels the layer's forward launches (their first launch
    may load code objects) through awa_forward on a separate plan, so that
    the no-alloc call's memory check sees only what that call does."""
    t, h, w, nt, nh, nw, tx = layer.params
    other = A.Plan(A.LayerParams(t, h, w, nt, nh, nw, tx, layer.shifted), heads=layer.heads)
    other.upload()
    _, _, vb, tb = layer.outputs()
    other.forward(layer.vq_blob, layer.tq_blob, vb, tb, compute)
    A.synchronize()
    other.destroy()


def run_both(layer: Layer, compute: int):
    """The no-alloc call first (the plan's work list comes from
    awa_plan_upload), then awa_forward on the same plan and inputs."""
    warm_kernels(layer, compute)
    vo_a, to_a, vb_a, tb_a = layer.outputs()
    vo_b, to_b, vb_b, tb_b = layer.outputs()
    A.synchronize()
    before = free_device_bytes()
    rc = layer.plan.forward_noalloc(layer.vq_blob, layer.tq_blob, vb_b, tb_b, compute)
    A.synchronize()
    after = free_device_bytes()
    assert rc == A.AWA_OK, A.lib().awa_last_error()
    assert after == before, f"the no-alloc call changed free device memory by {before - after} bytes"
    layer.plan.forward(layer.vq_blob, layer.tq_blob, vb_a, tb_a, compute)
    A.synchronize()
    return layer.read(vo_a, to_a), layer.read(vo_b, to_b)


def test_noalloc_matches_awa_forward_twice(gpu):
    """First call: the 33-frame shifted layer in fp32 (36 windows, 20 heads:
    23.6 MB of text rows). Second call on the same GPU: a smaller 5-frame
    shifted layer, bf16 in and out, 4 heads; the buffer keeps the first
    call's contents, which the second overwrites where it reads."""
    print("case noalloc 9x16x16 shifted fp32, 20 heads", flush=True)
    big = Layer(CONFIGS["clip_9x16x16"], True, 20, 4, 4, 20260902)
    ref, got = run_both(big, A.COMPUTE_F32)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])
    print("case noalloc 2x16x16 shifted bf16, 4 heads", flush=True)
    small = Layer(CONFIGS["clip_2x16x16"], True, 4, 2, 2, 20260903)
    ref, got = run_both(small, A.COMPUTE_BF16)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])


def test_noalloc_rejects_what_it_cannot_hold(gpu):
    # 9x32x32 shifted, fp32 text rows: 100 windows x 64 x 20 x 128 x 4 B = 65.5 MB > 32 MiB.
    print("case noalloc rejects 9x32x32 shifted fp32 text rows", flush=True)
    too_big = Layer(CONFIGS["clip_9x32x32"], True, 20, 4, 4, 20260904)
    _, _, vb, tb = too_big.outputs()
    assert too_big.plan.forward_noalloc(too_big.vq_blob, too_big.tq_blob, vb, tb, A.COMPUTE_F32) == A.AWA_ERR_INVALID
    assert b"no-alloc scratch" in A.lib().awa_last_error()
    # A plan created without the head count has no work list until an allocating forward.
    print("case noalloc rejects a plan without its work list", flush=True)
    t, h, w, nt, nh, nw, tx = CONFIGS["clip_2x16x16"]
    plan = A.Plan(A.LayerParams(t, h, w, nt, nh, nw, tx, False))
    plan.upload()
    small = Layer(CONFIGS["clip_2x16x16"], False, 4, 4, 4, 20260905)
    _, _, vb, tb = small.outputs()
    assert plan.forward_noalloc(small.vq_blob, small.tq_blob, vb, tb, A.COMPUTE_F32) == A.AWA_ERR_INVALID
    assert b"work list" in A.lib().awa_last_error()
    A.synchronize()
