"""The oracle's spherical harmonics: MACE convention pinned independently.

The reference evaluates sphericart 1.0.3 (an un-vendored dependency) on the
permuted direction (z, x, y) and scales by 2 sqrt(pi)
(libsymmetrix/source/mace.cpp:1268-1299).  sphericart is not installed; its
published real basis (orthonormal, no Condon-Shortley phase) is pinned here
against scipy's complex harmonics, the e3nn l=1 form sqrt(3)(x, y, z), the
zero-vector rule (reference test_device_environment.py:92-100),
orthonormality by quadrature and finite-difference gradients.
"""

import numpy as np
import pytest
from scipy.special import sph_harm_y


def scipy_real_sh(lmax, xyz):
    """Real orthonormal harmonics without the Condon-Shortley phase of the
    permuted unit direction, times 2 sqrt(pi), from scipy's complex ones."""
    u = xyz / np.linalg.norm(xyz, axis=1, keepdims=True)
    x, y, z = u[:, 2], u[:, 0], u[:, 1]  # permuted (z, x, y)
    theta = np.arccos(np.clip(z, -1, 1))
    phi = np.arctan2(y, x)
    out = np.zeros((len(u), (lmax + 1) ** 2))
    for l in range(lmax + 1):
        for m in range(-l, l + 1):
            c = sph_harm_y(l, abs(m), theta, phi)  # includes (-1)^m
            if m > 0:
                v = np.sqrt(2.0) * (-1) ** m * c.real
            elif m < 0:
                v = np.sqrt(2.0) * (-1) ** m * c.imag
            else:
                v = c.real
            out[:, l * l + l + m] = v
    return out * 2.0 * np.sqrt(np.pi)


def test_matches_independent_complex_harmonics(oracle_lib):
    rng = np.random.default_rng(0)
    xyz = np.vstack([[0.37, -0.41, 0.83], rng.normal(size=(200, 3)) * 2.5])
    Y, _ = oracle_lib.harmonics(3, xyz)
    np.testing.assert_allclose(Y, scipy_real_sh(3, xyz), atol=2e-13)


def test_l1_is_sqrt3_xyz_and_l0_is_one(oracle_lib):
    xyz = np.array([[0.37, -0.41, 0.83], [1.0, 2.0, -2.0]])
    Y, _ = oracle_lib.harmonics(1, xyz)
    u = xyz / np.linalg.norm(xyz, axis=1, keepdims=True)
    np.testing.assert_allclose(Y[:, 0], 1.0, atol=1e-15)
    np.testing.assert_allclose(Y[:, 1:4], np.sqrt(3.0) * u, atol=1e-14)


def test_zero_vector(oracle_lib):
    # reference: raw Y00 = 0.282094791773878 at the zero vector, others zero
    Y, dY = oracle_lib.harmonics(3, np.zeros((1, 3)))
    assert Y[0, 0] == pytest.approx(0.282094791773878 * 2 * np.sqrt(np.pi))
    assert np.all(Y[0, 1:] == 0) and np.all(dY == 0)


def test_orthonormal_by_quadrature(oracle_lib):
    # Gauss-Legendre in cos(theta) x uniform phi integrates degree <= 6 exactly
    nodes, weights = np.polynomial.legendre.leggauss(12)
    phis = np.linspace(0, 2 * np.pi, 24, endpoint=False)
    ct, ph = np.meshgrid(nodes, phis, indexing="ij")
    st = np.sqrt(1 - ct**2)
    xyz = np.stack([st * np.cos(ph), st * np.sin(ph), ct], -1).reshape(-1, 3)
    w = (weights[:, None] * np.full_like(ph, 2 * np.pi / len(phis))).reshape(-1)
    Y, _ = oracle_lib.harmonics(3, xyz)
    gram = (Y * w[:, None]).T @ Y
    np.testing.assert_allclose(gram, 4 * np.pi * np.eye(16), atol=1e-12)


def test_gradients_match_finite_differences(oracle_lib):
    rng = np.random.default_rng(1)
    xyz = rng.normal(size=(20, 3)) * 3.0
    _, dY = oracle_lib.harmonics(3, xyz)
    eps = 1e-6
    for axis in range(3):
        d = np.zeros(3)
        d[axis] = eps
        yp, _ = oracle_lib.harmonics(3, xyz + d)
        ym, _ = oracle_lib.harmonics(3, xyz - d)
        np.testing.assert_allclose(dY[:, axis, :], (yp - ym) / (2 * eps), atol=2e-9)


def test_rotation_covariance(oracle_lib):
    from symmetrix_amd import irreps

    rng = np.random.default_rng(2)
    xyz = rng.normal(size=(30, 3))
    R = irreps.random_rotation(5)
    Y, _ = oracle_lib.harmonics(3, xyz)
    YR, _ = oracle_lib.harmonics(3, xyz @ R.T)
    for l in range(4):
        D = irreps.wigner_d(l, R)
        block = slice(l * l, (l + 1) ** 2)
        np.testing.assert_allclose(YR[:, block], Y[:, block] @ D.T, atol=1e-11)
        np.testing.assert_allclose(D @ D.T, np.eye(2 * l + 1), atol=1e-11)


def test_python_generator_uses_the_same_harmonics(oracle_lib):
    from symmetrix_amd import irreps

    xyz = np.random.default_rng(4).normal(size=(50, 3))
    np.testing.assert_allclose(irreps.mace_sph_harm(3, xyz), oracle_lib.harmonics(3, xyz)[0], atol=1e-13)
