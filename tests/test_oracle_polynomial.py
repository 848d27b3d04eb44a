"""Symmetric-contraction polynomials and coupling tables.

* The oracle's polynomial value/gradient against a direct numpy evaluation
  and finite differences (reference multivariate_polynomial.cpp:313-355), and
  the reference's repeated-monomial rule (first coefficient kept, exact index
  vectors as keys; multivariate_polynomial.cpp:36-46) on its own fixture.
* The generated real coupling (CG) tables against the reference's R1
  contract fixtures, every term and sign (tests/golden, copied from
  symmetrix/test/data/execution_contracts/jit_r1_*_contract.json): the
  medium (3,1) shape, 86 terms; the wide (3,2) shape, 215 terms; the
  L_max = 0 (3,0) shape, 16 terms; the 1-term l = 0 fixture.
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


def test_repeated_monomial_retains_first_coefficient(oracle_lib):
    # the reference's own known answer (symmetrix/test/test_multivariate_polynomial.py:65-68):
    # [0] listed twice keeps 2.0, so f = 2*4 + 3*4*5 = 68 (summing both would give 104)
    f, g = oracle_lib.poly_eval([[0], [0], [0, 1]], [2.0, 9.0, 3.0], [4.0, 5.0])
    assert f == pytest.approx(68.0, abs=1e-12)
    np.testing.assert_allclose(g, [2.0 + 3.0 * 5.0, 3.0 * 4.0], atol=1e-12)


def test_permuted_monomials_are_distinct_terms(oracle_lib):
    # map keys are exact index vectors: [0,1] and [1,0] are two terms, [1,0] again is a repeat
    monos = [[0, 1], [1, 0], [1, 0], [2, 2, 1], [1, 2, 2], [2, 1, 2], [2, 2, 1]]
    coef = [2.0, 3.0, 100.0, 0.5, 0.25, 0.125, 100.0]
    x = np.array([4.0, 5.0, -1.5])
    f, g = oracle_lib.poly_eval(monos, coef, x)
    want = (2.0 + 3.0) * x[0] * x[1] + (0.5 + 0.25 + 0.125) * x[1] * x[2] ** 2
    assert f == pytest.approx(want, abs=1e-12)
    eps = 1e-6
    for v in range(3):
        dx = np.zeros(3)
        dx[v] = eps
        fd = (oracle_lib.poly_eval(monos, coef, x + dx)[0] - oracle_lib.poly_eval(monos, coef, x - dx)[0]) / (2 * eps)
        assert g[v] == pytest.approx(fd, abs=1e-7)


# The reference's R1 coupling contracts (symmetrix/test/data/execution_contracts/,
# copied into tests/golden): (file, edge l_max, source l_max, terms, tolerance).
# jit_r1_contract.json stores its values to 8 significant digits.
R1_CONTRACTS = [
    ("jit_r1_mace_mpa0_medium_contract.json", 3, 1, 86, 1e-12),
    ("jit_r1_contract.json", 3, 1, 86, 5e-8),
    ("jit_r1_mace_mp0b2_large_contract.json", 3, 2, 215, 1e-12),
    ("jit_r1_mace_off23_large_contract.json", 3, 2, 215, 1e-12),
    ("jit_r1_mace_omat0_small_contract.json", 3, 0, 16, 1e-12),
    ("jit_r1_mace_off23_small_contract.json", 3, 0, 16, 1e-12),
    ("jit_r1_fixture_c4_e3_l0_contract.json", 0, 0, 1, 1e-12),
]


@pytest.mark.parametrize("name,edge_lmax,source_lmax,count,tol", R1_CONTRACTS)
def test_cg_tables_match_reference_contract(name, edge_lmax, source_lmax, count, tol):
    # every path, row, output row and coefficient (sign included) of the
    # generated table equals the reference's contract
    from symmetrix_amd import irreps

    ref = load(name)
    t = irreps.phi1_tables(edge_lmax, source_lmax)
    assert [tuple(p) for p in t["paths"]] == [(p["edge_l"], p["source_l"], p["output_l"]) for p in ref["paths"]]
    mine = {(x["lm1"], x["lm2"], x["row"], x["lme"]): x["coefficient"] for x in t["terms"]}
    theirs = {(x["lm1"], x["lm2"], x["row"], x["lme"]): x["coefficient"] for x in ref["sparse_coupling"]["terms"]}
    assert set(mine) == set(theirs) and len(theirs) == ref["sparse_coupling"]["term_count"] == count
    for k in theirs:
        assert mine[k] == pytest.approx(theirs[k], abs=tol)


def test_cg_sign_rule_is_not_the_largest_entry_rule():
    # the two paths of the wide shape on which "largest entry positive" and
    # the reference's convention (m=0 x m=0 -> m=0 entry positive) disagree
    from symmetrix_amd import irreps

    for triple in [(2, 2, 2), (3, 2, 3)]:
        c = irreps.coupling_tensor(*triple)
        flat = c.reshape(-1)
        assert c[triple[0], triple[1], triple[2]] > 0
        peak = np.max(np.abs(flat))
        first_peak = flat[np.flatnonzero(np.abs(flat) > peak - 1e-9)[0]]
        assert first_peak < 0


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
