"""Symmetric-contraction polynomials and coupling tables.

* The oracle's polynomial value/gradient against a direct numpy evaluation
  and finite differences (reference multivariate_polynomial.cpp:313-355).
* The generated real coupling (CG) tables against the reference's medium R1
  contract fixture, all 86 terms (tests/golden, copied from
  symmetrix/test/data/execution_contracts/jit_r1_mace_mpa0_medium_contract.json).
* The generated M0 monomial tables against standard_m0_contract.json
  (tests/golden): identical for the scalar and m=0 outputs; the fixture's
  m=+-1 tables carry 6 extra cubic monomials each that no O(3)-equivariant
  polynomial contains (shown by brute force below).
* Equivariance of the generated polynomials.
"""

import itertools
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_oracle_polynomial_value_and_gradient(oracle_lib):
    rng = np.random.default_rng(0)
    monos = [[0], [3], [0, 0], [1, 2], [2, 2], [0, 1, 2], [1, 1, 1], [0, 3, 3]]
    coef = rng.normal(size=len(monos))
    x = rng.normal(size=4)
    f, g = oracle_lib.poly_eval(monos, coef, x)
    want = sum(c * np.prod(x[m]) for c, m in zip(coef, monos))
    assert f == pytest.approx(want, abs=1e-13)
    eps = 1e-6
    for v in range(4):
        dx = np.zeros(4)
        dx[v] = eps
        fd = (oracle_lib.poly_eval(monos, coef, x + dx)[0] - oracle_lib.poly_eval(monos, coef, x - dx)[0]) / (2 * eps)
        assert g[v] == pytest.approx(fd, abs=1e-8)


def test_cg_tables_match_reference_contract():
    from symmetrix_amd import irreps

    ref = load("jit_r1_mace_mpa0_medium_contract.json")
    t = irreps.phi1_tables(3, 1)
    assert [tuple(p) for p in t["paths"]] == [(p["edge_l"], p["source_l"], p["output_l"]) for p in ref["paths"]]
    mine = {(x["lm1"], x["lm2"], x["row"], x["lme"]): x["coefficient"] for x in t["terms"]}
    theirs = {(x["lm1"], x["lm2"], x["row"], x["lme"]): x["coefficient"] for x in ref["sparse_coupling"]["terms"]}
    assert set(mine) == set(theirs) and len(theirs) == ref["sparse_coupling"]["term_count"] == 86
    for k in theirs:
        assert mine[k] == pytest.approx(theirs[k], abs=1e-12)


def test_r0_contract_rows_are_the_edge_harmonics():
    ref = load("standard_r0_contract.json")
    terms = ref["sparse_coupling"]["terms"]
    assert [(t["lm1"], t["lm2"], t["lme"], t["coefficient"]) for t in terms] == [(k, 0, k, 1.0) for k in range(16)]


def test_m0_monomials_match_reference_contract():
    from symmetrix_amd import irreps

    ref = load("standard_m0_contract.json")
    extra = {}
    for group in ref["monomial_groups"]:
        LM = group["output_component"]
        L = int(np.sqrt(LM))
        monos, _ = irreps.equivariant_polynomials(3, L, 3)[LM - L * L]
        mine = {tuple(m) for m in monos}
        theirs = {tuple(m) for m in group["terms"]}
        assert mine <= theirs
        extra[LM] = theirs - mine
    assert extra[0] == set() and extra[2] == set()
    assert extra[1] == {(3, 4, 8), (3, 9, 15), (3, 10, 14), (4, 8, 13), (9, 13, 15), (10, 13, 14)}
    assert len(extra[3]) == 6


@pytest.mark.slow
def test_extra_reference_monomials_are_not_equivariant():
    """Brute force: the full space of O(3)-equivariant cubic polynomials of 16
    harmonic inputs (l <= 3) with an l=1 output has no (3,4,8)-type term."""
    from symmetrix_amd import irreps

    monos = list(itertools.combinations_with_replacement(range(16), 3))
    rng = np.random.default_rng(0)
    parity = np.array([(-1) ** l for l in range(4) for _ in range(2 * l + 1)])
    rows = []
    for s in range(900):  # 2700 equations > 2448 unknowns
        R = irreps.random_rotation(s)
        Ds = [irreps.wigner_d(l, R) for l in range(4)]
        DL = irreps.wigner_d(1, R)
        A = rng.normal(size=16)
        A2 = np.concatenate([Ds[l] @ A[l * l:(l + 1) ** 2] for l in range(4)])
        if s % 2:
            A2, DL = A2 * parity, -DL
        mv = np.array([A[a] * A[b] * A[c] for a, b, c in monos])
        mv2 = np.array([A2[a] * A2[b] * A2[c] for a, b, c in monos])
        for M in range(3):
            row = np.zeros((3, len(monos)))
            row[M] += mv2
            for Mp in range(3):
                row[Mp] -= DL[M, Mp] * mv
            rows.append(row.reshape(-1))
    _, sv, vt = np.linalg.svd(np.array(rows), full_matrices=False)
    null = vt[sv < 1e-8 * sv[0]].reshape(-1, 3, len(monos))
    present = np.max(np.abs(null[:, 0, :]), axis=0) > 1e-8
    for t in [(3, 4, 8), (3, 9, 15), (3, 10, 14), (4, 8, 13), (9, 13, 15), (10, 13, 14)]:
        assert not present[monos.index(t)]
    mine, _ = irreps.equivariant_polynomials(3, 1, 3)[0]
    assert {m for m, p in zip(monos, present) if p} == {tuple(m) for m in mine if len(m) == 3}


@pytest.mark.parametrize("out_l", [0, 1, 2])
def test_generated_polynomials_are_equivariant(out_l):
    from symmetrix_amd import irreps

    comps = irreps.equivariant_polynomials(3, out_l, 3)
    rng = np.random.default_rng(out_l)
    w = rng.normal(size=comps[0][1].shape[0])

    def evaluate(A):
        return np.array([sum(c * np.prod(A[list(m)]) for c, m in zip(w @ basis, monos))
                         for monos, basis in comps])

    A = rng.normal(size=16)
    R = irreps.random_rotation(11)
    A2 = np.concatenate([irreps.wigner_d(l, R) @ A[l * l:(l + 1) ** 2] for l in range(4)])
    np.testing.assert_allclose(evaluate(A2), irreps.wigner_d(out_l, R) @ evaluate(A), atol=1e-10)
