"""The product plan (host side of libseedvr2_awa.so) against the oracle: every
map bit-exact, error codes as the reference's load_param. No GPU needed."""

import ctypes
import itertools

import numpy as np
import pytest

import awa_hip as A
import oracle as O
from awa_cases import CONFIGS, RAGGED, geometry


def header_symbols():
    import os
    import re

    path = os.path.join(os.path.dirname(A.HERE), "include", "seedvr2_awa.h")
    text = open(path).read()
    return sorted(set(re.findall(r"\b(awa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = A.lib()
    declared = header_symbols()
    assert set(declared) == set(A.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def all_cases():
    cases = []
    for p in list(CONFIGS.values()) + RAGGED:
        for s in (False, True):
            cases.append((p, s))
    # small exhaustive sweep of grids and window counts
    for t, h, w in [(1, 1, 1), (1, 3, 5), (2, 4, 4), (7, 5, 3), (31, 9, 16), (40, 6, 7)]:
        for nt, nh, nw in [(1, 1, 1), (2, 3, 3), (4, 8, 8), (3, 5, 2)]:
            for s in (False, True):
                cases.append(((t, h, w, nt, nh, nw, 3), s))
    return cases


@pytest.mark.parametrize("params,shifted", all_cases())
def test_plan_maps_bit_exact(params, shifted):
    g = geometry(params, shifted)
    m = O.build_maps(g)
    assert m.status == 0
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted))
    assert plan.info.window_count == m.window_count
    assert plan.info.sequence_tokens == m.sequence_tokens
    np.testing.assert_array_equal(plan.windows(), O.make_windows(g))
    np.testing.assert_array_equal(plan.sequence_index(), m.sequence_index)
    np.testing.assert_array_equal(plan.cu_seqlens(), m.cu_seqlens)
    np.testing.assert_array_equal(plan.video_positions(), m.video_positions)
    np.testing.assert_array_equal(plan.text_positions(), m.text_positions)
    assert plan.info.max_window_tokens == int(np.diff(m.cu_seqlens).max())


@pytest.mark.parametrize("params,shifted", list(itertools.product(
    [CONFIGS["clip_9x16x16"], CONFIGS["clip_31x16x16"], (3, 11, 13, 2, 3, 3, 5)], [False, True])))
@pytest.mark.parametrize("rope_dim", [126, 18, 6])
def test_plan_rope_table_bit_exact(params, shifted, rope_dim):
    g = geometry(params, shifted)
    plan = A.Plan(A.LayerParams(*g.args, g.text_tokens, g.shifted, rope_dim))
    np.testing.assert_array_equal(plan.rope_table(), O.rope_table(g, rope_dim))


def test_runtime_spec_dynamic_params():
    """params 0/1/2 = -1 take the grid from the runtime spec (awa_layers.cpp:97-104)."""
    plan = A.Plan(A.LayerParams(-1, -1, -1, 3, 8, 8, 64, True), runtime=(9, 16, 16, 9 * 16 * 16))
    ref = O.build_maps(geometry(CONFIGS["clip_9x16x16"], True))
    np.testing.assert_array_equal(plan.sequence_index(), ref.sequence_index)


@pytest.mark.parametrize("params,runtime", [
    ((0, 16, 16, 1, 8, 8, 64, False, 126), None),
    ((1, 16, 16, 0, 8, 8, 64, False, 126), None),
    ((1, 16, 16, 1, 8, 8, 0, False, 126), None),
    ((1, 16, 16, 1, 8, 8, 64, False, 100), None),   # rope_dim not a multiple of 6
    ((1, 16, 16, 1, 8, 8, 64, False, -6), None),
    ((1, 16, 16, 1, 8, 8, 64, False, 0), None),     # rope_dim 0 (src/awa/awa_layers.cpp:873-874)
    ((-1, -1, -1, 1, 8, 8, 64, False, 126), None),  # dynamic without runtime spec
    ((-1, -1, -1, 1, 8, 8, 64, False, 126), (2, 16, 16, 500)),  # inconsistent spec
    ((-1, 16, 16, 1, 8, 8, 64, False, 126), None),  # partial -1
    ((70000, 70000, 1, 1, 1, 1, 4, False, 126), None),  # token count overflows int
])
def test_plan_rejects_invalid_params(params, runtime):
    with pytest.raises(A.AwaError) as e:
        A.Plan(A.LayerParams(*params), runtime=runtime)
    assert e.value.code == A.AWA_ERR_INVALID


def test_plan_rejects_negative_heads():
    """awa_plan_desc.heads: 0 (unknown) or a positive head count."""
    with pytest.raises(A.AwaError) as e:
        A.Plan(A.LayerParams(1, 16, 16, 1, 8, 8, 64), heads=-1)
    assert e.value.code == A.AWA_ERR_INVALID


def test_forward_requires_uploaded_plan():
    """Entry points refuse a plan that was never uploaded (the reference's
    'uninitialized Vulkan state', awa_layers.cpp:506-510), before touching memory."""
    plan = A.Plan(A.LayerParams(1, 16, 16, 1, 8, 8, 64))
    blob = A.mat(0, 128, 60, 256)
    rc = A.lib().awa_forward(plan.h, ctypes.byref(blob), ctypes.byref(blob), ctypes.byref(blob),
                             ctypes.byref(blob), A.COMPUTE_F32, None)
    assert rc != A.AWA_OK
