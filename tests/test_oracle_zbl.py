"""The oracle's ZBL pair term (restating zbl_kokkos.cpp:76-126 in double)
against the reference's own known answers (symmetrix/test/test_zbl.py:5-48:
a_exp 0.3, a_prefactor 0.4543, c = (0.1818, 0.5099, 0.2802, 0.02817), the
covalent radii listed there, p = 6, Z = 5 and 10), its finite-difference
derivative and the Coulomb limit at short range."""

import numpy as np
import pytest

RADII = [0.2, 0.31, 0.28, 1.28, 0.96, 0.84, 0.76, 0.71, 0.66, 0.57, 0.58]
C = [0.1818, 0.5099, 0.2802, 0.02817]
ZU, ZV = 5, 10
R_MAX = RADII[ZU] + RADII[ZV]


def zbl(oracle_lib, r, a_prefactor=0.4543, c=C):
    return oracle_lib.zbl_pair(0.3, a_prefactor, c, RADII, 6, ZU, ZV, r)


def test_known_values(oracle_lib):
    v, g = zbl(oracle_lib, [1.0, R_MAX, R_MAX + 0.3])
    assert v[0] == pytest.approx(0.3166652764835175, rel=1e-14)   # test_zbl.py:38
    assert v[1] == 0.0 and g[1] == 0.0                            # test_zbl.py:36, 42
    assert v[2] == 0.0 and g[2] == 0.0


def test_envelope_known_value(oracle_lib):
    # with a screening length so large that phi = sum(c) and c = (1, 0, 0, 0),
    # V r / (0.5 * 14.3996 Zu Zv) is the envelope alone (test_zbl.py:17)
    r = 1.0
    v, _ = zbl(oracle_lib, [r], a_prefactor=1e12, c=[1.0, 0.0, 0.0, 0.0])
    envelope = v[0] * r / (0.5 * 14.3996 * ZU * ZV)
    assert envelope == pytest.approx(0.4374788794430078, rel=1e-9)


def test_gradient_matches_finite_differences(oracle_lib):
    h = 1e-6
    for r in [0.3, 0.8, 1.0, 1.3]:
        _, g = zbl(oracle_lib, [r])
        vp, _ = zbl(oracle_lib, [r + h])
        vm, _ = zbl(oracle_lib, [r - h])
        assert g[0] == pytest.approx((vp[0] - vm[0]) / (2 * h), rel=1e-7)


def test_coulomb_limit(oracle_lib):
    # r -> 0: phi -> sum(c), envelope -> 1, so V r -> 0.5 * 14.3996 Zu Zv sum(c)
    r = 1e-7
    v, _ = zbl(oracle_lib, [r])
    assert v[0] * r == pytest.approx(0.5 * 14.3996 * ZU * ZV * sum(C), rel=1e-5)
