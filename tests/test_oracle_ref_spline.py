"""The oracle's cubic Hermite spline set against the reference's own
CubicSplineSetT (libsymmetrix/source/cubic_spline_set.cpp, compiled from the
reference sources into oracle/_ref/ by `make -C oracle ref`; skipped where the
reference is absent, e.g. on the GPU box).

Random nodal values and derivatives on a 256-knot grid (the compact radial
grid of the model format, spacing r_cut / 255 from x0 = 1e-12), evaluated
inside the grid, exactly on knots and outside both ends (clamped to the first
and last interval, cubic_spline_set.cpp:32-47).
"""

import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_spline.so")

pytestmark = pytest.mark.skipif(not os.path.exists(REF_LIB), reason="reference spline build absent (make -C oracle ref)")


def _ref_eval(precision, h, x0, values, derivs, r):
    lib = ctypes.CDLL(REF_LIB)
    v = np.ascontiguousarray(values, dtype=np.float64)
    d = np.ascontiguousarray(derivs, dtype=np.float64)
    rr = np.ascontiguousarray(r, dtype=np.float64)
    nfn, nodes = v.shape
    out_v = np.zeros((len(rr), nfn))
    out_d = np.zeros((len(rr), nfn))
    dp = ctypes.POINTER(ctypes.c_double)
    rc = lib.ref_spline_eval(ctypes.c_int(precision), ctypes.c_double(h), ctypes.c_double(x0), ctypes.c_int(nfn),
                             ctypes.c_int(nodes), v.ctypes.data_as(dp), d.ctypes.data_as(dp), ctypes.c_int(len(rr)),
                             rr.ctypes.data_as(dp), out_v.ctypes.data_as(dp), out_d.ctypes.data_as(dp))
    assert rc == 0
    return out_v, out_d


def _grid_case(seed, nfn=12, nodes=256, r_cut=6.0):
    rng = np.random.default_rng(seed)
    x0 = 1e-12
    h = (r_cut - x0) / (nodes - 1)
    values = rng.normal(size=(nfn, nodes))
    derivs = rng.normal(size=(nfn, nodes)) * 3.0
    inside = rng.uniform(x0, r_cut, size=400)
    knots = x0 + h * rng.integers(0, nodes, size=50)
    outside = np.concatenate([rng.uniform(-1.0, x0, size=20), rng.uniform(r_cut, r_cut + 1.0, size=20),
                              [x0, r_cut, r_cut + 1e-9]])
    return h, x0, values, derivs, np.concatenate([inside, knots, outside])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_spline_matches_reference_double(oracle_lib, seed):
    h, x0, values, derivs, r = _grid_case(seed)
    want_v, want_d = _ref_eval(8, h, x0, values, derivs, r)
    got_v, got_d = oracle_lib.spline_eval(h, x0, values, derivs, r)
    np.testing.assert_allclose(got_v, want_v, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(got_d, want_d, rtol=1e-13, atol=1e-12)


def test_reference_float_spline_agrees_with_oracle_double(oracle_lib):
    """The FP32 instantiation of the reference builds its Hermite
    coefficients in float; at h = r_cut / 255 the c2, c3 formulas cancel
    (cubic_spline_set.cpp:23-26), so it agrees with the double evaluation
    only to ~1e-4 of the value scale.  (The GPU tables are built in double and
    stored in FP32, which keeps the FP32 rounding of the evaluation only.)"""
    h, x0, values, derivs, r = _grid_case(3)
    want_v, want_d = _ref_eval(4, h, x0, values, derivs, r)
    got_v, got_d = oracle_lib.spline_eval(h, x0, values, derivs, r)
    scale_v = np.max(np.abs(got_v))
    scale_d = np.max(np.abs(got_d))
    assert np.max(np.abs(got_v - want_v)) < 1e-4 * scale_v
    assert np.max(np.abs(got_d - want_d)) < 1e-3 * scale_d
