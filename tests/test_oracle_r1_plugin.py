"""The oracle's restatement of the reference's R1 plugin operator
(oracle.plugin_r1_forward / _source / _edge; jit_codegen.py:884-1110,
1314-1424), pinned by what the mathematics fixes rather than by retyping it:

- the packet's cubic pieces reproduce the oracle's Hermite spline set (itself
  checked against the reference's own CubicSplineSetT in
  test_oracle_ref_spline.py), inside the grid and clamped beyond both ends;
- the source owner is the transpose of the receiver owner:
  <A, forward(H)> = <source(A), H> for every A and H (an index or path slip
  in one of them breaks it);
- the edge owner is minus the gradient of <A, forward> with respect to each
  edge vector (central differences of the forward with harmonics and radial
  functions re-evaluated at the moved vector);
- with the medium contract's couplings the forward is rotation covariant:
  each output vector of one path and l_out keeps its length when the edges
  and the l = 1 source features rotate (a wrong coefficient breaks it).
"""

import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _contract():
    with open(os.path.join(HERE, "golden", "jit_r1_mace_mpa0_medium_contract.json")) as f:
        return json.load(f)


def _case(oracle_lib, seed=0, n=10, per=6, channels=3, types=2, cutoff=5.0):
    """Random receiver-major graph with edge vectors of lengths 0.8..5.6 A
    (some beyond the cutoff), random radial pieces per unordered type pair."""
    rng = np.random.default_rng(seed)
    receivers = np.repeat(np.arange(n), per)
    sources = rng.integers(0, n, size=n * per)
    xyz = rng.normal(size=(n * per, 3))
    xyz *= (rng.uniform(0.8, 5.6, size=n * per) / np.linalg.norm(xyz, axis=1))[:, None]
    radius = np.linalg.norm(xyz, axis=1)
    node_type = rng.integers(0, types, size=n)
    a, b = node_type[receivers], node_type[sources]
    lo, hi = np.minimum(a, b), np.maximum(a, b)
    edge_type = lo * (2 * types - lo - 1) // 2 + hi
    contract = _contract()
    P = len(contract["paths"])
    knots, h, x0 = 41, cutoff / 40, 0.0
    pieces = np.stack([oracle_lib.hermite_pieces(rng.normal(size=(P * channels, knots)),
                                                 rng.normal(size=(P * channels, knots)), h)
                       for _ in range(types * (types + 1) // 2)])
    return dict(rng=rng, n=n, receivers=receivers, sources=sources, xyz=xyz, radius=radius, edge_type=edge_type,
                pieces=pieces, h=h, x0=x0, channels=channels, cutoff=cutoff, contract=contract,
                terms=oracle_lib.plugin_terms(contract), num_lme=40, num_lm2=4)


def _forward(oracle_lib, c, xyz, H):
    radius = np.linalg.norm(xyz, axis=1)
    R, _ = oracle_lib.plugin_spline(c["pieces"], c["edge_type"], radius, c["x0"], c["h"])
    Y, _ = oracle_lib.harmonics(3, xyz)
    return oracle_lib.plugin_r1_forward(c["terms"], c["channels"], c["n"], c["receivers"], c["sources"],
                                        radius < c["cutoff"], R, Y, H, c["num_lme"])


def test_pieces_reproduce_the_oracle_spline_set(oracle_lib):
    rng = np.random.default_rng(1)
    fns, knots, h, x0 = 5, 30, 0.2, 0.3
    values, derivs = rng.normal(size=(fns, knots)), rng.normal(size=(fns, knots))
    r = np.concatenate([rng.uniform(x0, x0 + h * (knots - 1), 200), [0.1, x0, x0 + h * (knots - 1), 9.0]])
    want_v, want_d = oracle_lib.spline_eval(h, x0, values, derivs, r)
    got_v, got_d = oracle_lib.plugin_spline(oracle_lib.hermite_pieces(values, derivs, h)[None],
                                            np.zeros(len(r), int), r, x0, h)
    np.testing.assert_allclose(got_v, want_v, atol=1e-12)
    np.testing.assert_allclose(got_d, want_d, atol=1e-11)


def test_source_owner_is_the_transpose_of_the_forward(oracle_lib):
    c = _case(oracle_lib)
    rng, C = c["rng"], c["channels"]
    H = rng.normal(size=(c["n"], 4, C))
    A = rng.normal(size=(c["n"], 40, C))
    R, _ = oracle_lib.plugin_spline(c["pieces"], c["edge_type"], c["radius"], c["x0"], c["h"])
    Y, _ = oracle_lib.harmonics(3, c["xyz"])
    active = c["radius"] < c["cutoff"]
    assert 0 < active.sum() < len(active)
    out = oracle_lib.plugin_r1_forward(c["terms"], C, c["n"], c["receivers"], c["sources"], active, R, Y, H, 40)
    sadj = oracle_lib.plugin_r1_source(c["terms"], C, c["n"], 4, c["receivers"], c["sources"], active, R, Y, A)
    assert np.sum(A * out) == pytest.approx(np.sum(sadj * H), rel=1e-12)
    assert np.abs(out).max() > 0 and np.abs(sadj).max() > 0


def test_edge_owner_is_minus_the_edge_gradient(oracle_lib):
    c = _case(oracle_lib, seed=2)
    rng, C = c["rng"], c["channels"]
    H = rng.normal(size=(c["n"], 4, C))
    A = rng.normal(size=(c["n"], 40, C))
    R, dR = oracle_lib.plugin_spline(c["pieces"], c["edge_type"], c["radius"], c["x0"], c["h"])
    Y, dY = oracle_lib.harmonics(3, c["xyz"])
    active = c["radius"] < c["cutoff"]
    force = oracle_lib.plugin_r1_edge(c["terms"], C, c["receivers"], c["sources"], active, c["xyz"], c["radius"],
                                      R, dR, Y, dY, H, A)
    eps = 1e-6
    for e in np.flatnonzero(active)[:12]:
        for k in range(3):
            plus, minus = c["xyz"].copy(), c["xyz"].copy()
            plus[e, k] += eps
            minus[e, k] -= eps
            fd = (np.sum(A * _forward(oracle_lib, c, plus, H)) - np.sum(A * _forward(oracle_lib, c, minus, H))) / (2 * eps)
            assert -fd == pytest.approx(force[e, k], rel=1e-5, abs=1e-7)
    assert np.all(force[~active] == 0.0)


def test_forward_with_the_medium_couplings_is_rotation_covariant(oracle_lib):
    from symmetrix_amd import irreps

    c = _case(oracle_lib, seed=3)
    rng, C = c["rng"], c["channels"]
    H = rng.normal(size=(c["n"], 4, C))
    out = _forward(oracle_lib, c, c["xyz"], H)
    rot = irreps.random_rotation(7)
    Hr = H.copy()
    Hr[:, 1:4] = np.einsum("ab,nbk->nak", irreps.wigner_d(1, rot), H[:, 1:4])
    out_r = _forward(oracle_lib, c, c["xyz"] @ rot.T, Hr)
    # output vectors: per l_out (groups in order) the components are m-major,
    # lme = offset + m * instances + instance, one vector per path instance
    offset = 0
    for group in c["contract"]["groups"]:
        m, count = 2 * group["l"] + 1, len(group["path_indices"])
        for instance in range(count):
            block = offset + np.arange(m) * count + instance
            np.testing.assert_allclose(np.linalg.norm(out_r[:, block], axis=1), np.linalg.norm(out[:, block], axis=1),
                                       rtol=1e-9, atol=1e-12)
        offset += m * count
    assert offset == 40
