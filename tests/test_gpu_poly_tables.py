"""GPU parity for symmetric-contraction tables the compiled monomial tables do
not describe exactly.

The node kernels evaluate the terms of a model's M0 / M1 monomial lists that
match a compiled table in registers and every other term in a runtime loop.
These tests rewrite the generated model JSON so that both paths carry
weight, and compare the HIP result with the CPU oracle (which evaluates the
JSON lists as given):

- monomial order shuffled within each output, and the variable order inside
  each monomial permuted (same polynomial, compiled slots found by value);
- extra monomials that no compiled slot holds, plus a repeated monomial
  (first coefficient kept, as the reference's polynomial does) and a
  permutation of an existing one (a distinct term);
- a correlation order with no compiled table (every term runs in the loop).

Tolerances as in test_gpu_parity.py (FP32).
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _write(tmp_path, name, model):
    path = tmp_path / f"{name}.json"
    path.write_text(json.dumps(model))
    return str(path)


def _generated(preset_or_shape, seed=0):
    from symmetrix_amd import synthetic

    return json.loads(synthetic.model_json(synthetic.random_mace_model(preset_or_shape, seed=seed)))


def _check(oracle_lib, path, model, structure):
    from symmetrix_amd import Symmetrix, synthetic

    got = Symmetrix(path).calculate(structure)
    types = synthetic.node_types(structure, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, structure, model["r_cut"] + 0.5)
    n = len(structure)
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    return got


def _shuffle(model, rng):
    """Same polynomials, terms and variables in another order."""
    C = model["num_channels"]
    ne = model["num_elements"]
    for LM, monos in model["M0_monomials"].items():
        perm = rng.permutation(len(monos))
        model["M0_monomials"][LM] = [[int(v) for v in rng.permutation(monos[p])] for p in perm]
        for a in range(ne):
            w = model["M0_weights"][str(a)][LM]
            for k in range(C):
                w[str(k)] = [w[str(k)][p] for p in perm]
    monos = model["M1_monomials"]
    perm = rng.permutation(len(monos))
    model["M1_monomials"] = [[int(v) for v in rng.permutation(monos[p])] for p in perm]
    for a in range(ne):
        w = model["M1_weights"][str(a)]
        for k in range(C):
            w[str(k)] = [w[str(k)][p] for p in perm]


def _add_terms(model, rng, extra):
    """Appends `extra` monomials, then a repeat of an existing one and a
    permutation of another, to the M0 outputs with LM >= 1 and to M1, with
    small random coefficients.  The repeat is of the output's first (linear)
    monomial with a large coefficient: the reference keeps the first
    coefficient of a repeated monomial (multivariate_polynomial.cpp:36-46), and
    summing the repeat instead moves the energy by ~1e-3 eV/atom, far outside
    the tolerance."""
    C = model["num_channels"]
    ne = model["num_elements"]
    nlm = (model["l_max"] + 1) ** 2

    def new_terms(existing):
        have = {tuple(sorted(m)) for m in existing}
        out = []
        while len(out) < extra:
            deg = int(rng.integers(2, 4))
            m = sorted(int(v) for v in rng.integers(0, nlm, size=deg))
            if tuple(m) not in have:
                have.add(tuple(m))
                out.append(m)
        repeat = list(existing[0])  # the output's first (linear) monomial
        permuted = next(list(reversed(m)) for m in list(existing) + out if len(m) > 1 and m[0] != m[-1])
        return out + [repeat, permuted]

    def coefficients(n):
        c = list(0.05 * rng.normal(size=n))
        c[-2] = 2.0  # the repeat
        return c

    for LM, monos in model["M0_monomials"].items():
        if LM == "0":
            continue
        add = new_terms(monos)
        model["M0_monomials"][LM] = monos + add
        for a in range(ne):
            w = model["M0_weights"][str(a)][LM]
            for k in range(C):
                w[str(k)] = w[str(k)] + coefficients(len(add))
    add = new_terms(model["M1_monomials"])
    model["M1_monomials"] = model["M1_monomials"] + add
    for a in range(ne):
        w = model["M1_weights"][str(a)]
        for k in range(C):
            w[str(k)] = w[str(k)] + coefficients(len(add))


def _summed_repeats(model):
    """The same tables with each repeated monomial's coefficients added to its
    first entry (the semantics the reference does not have)."""
    model = json.loads(json.dumps(model))
    ne, C = model["num_elements"], model["num_channels"]

    def fold(monos, weight_lists):
        first, keep = {}, []
        for j, m in enumerate(monos):
            key = tuple(m)
            if key in first:
                for w in weight_lists:
                    for k in range(C):
                        w[str(k)][first[key]] += w[str(k)][j]
            else:
                first[key] = j
                keep.append(j)
        for w in weight_lists:
            for k in range(C):
                w[str(k)] = [w[str(k)][j] for j in keep]
        return [monos[j] for j in keep]

    for LM in model["M0_monomials"]:
        model["M0_monomials"][LM] = fold(
            model["M0_monomials"][LM], [model["M0_weights"][str(a)][LM] for a in range(ne)])
    model["M1_monomials"] = fold(model["M1_monomials"], [model["M1_weights"][str(a)] for a in range(ne)])
    return model


@pytest.mark.parametrize("preset,cells", [("tiny", 2), ("medium3", 2)])
def test_shuffled_monomial_tables_match_oracle_and_generated_order(oracle_lib, tmp_path, preset, cells):
    from symmetrix_amd import Symmetrix, synthetic

    s = synthetic.srtio3_supercell(cells, sigma=0.05, seed=3)
    model = _generated(preset)
    base = Symmetrix(_write(tmp_path, "base", model)).calculate(s)
    _shuffle(model, np.random.default_rng(7))
    print(f"{preset}: shuffled M0/M1 tables, SrTiO3 {cells}^3", flush=True)
    got = _check(oracle_lib, _write(tmp_path, "shuffled", model), model, s)
    # the same polynomial in another term order: FP32 summation-order noise only
    assert abs(got["energy"] - base["energy"]) / len(s) < E_TOL
    np.testing.assert_allclose(got["forces"], base["forces"], atol=F_TOL)


@pytest.mark.parametrize("preset,cells", [("tiny", 2), ("medium3", 2)])
def test_extra_monomials_run_in_the_remainder_loop(oracle_lib, tmp_path, preset, cells):
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(cells, sigma=0.05, seed=4)
    model = _generated(preset, seed=1)
    _add_terms(model, np.random.default_rng(11), extra=6)
    print(f"{preset}: M0/M1 tables with extra, repeated and permuted monomials, SrTiO3 {cells}^3", flush=True)
    got = _check(oracle_lib, _write(tmp_path, "extra", model), model, s)
    # summing the repeats instead would give a clearly different result
    summed = _summed_repeats(model)
    types = synthetic.node_types(s, summed["atomic_numbers"])
    orc = oracle_lib.MaceOracle(summed, np.unique(types), "float32")
    other = oracle_lib.evaluate(orc, s, summed["r_cut"] + 0.5)
    assert abs(got["energy"] - other["energy"]) / len(s) > 10 * E_TOL


def test_uncompiled_correlation_order_matches_oracle(oracle_lib, tmp_path):
    from symmetrix_amd import synthetic

    shape = synthetic.ModelShape(
        atomic_numbers=(38, 22, 8), channels=64, l_max=3, L_max=1, correlation=2,
        radial_hidden=(32, 32), r_cut=5.0, avg_num_neighbors=40.0,
    )
    model = _generated(shape, seed=2)
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=5)
    print("l_max 3, correlation 2 (no compiled table), SrTiO3 2^3", flush=True)
    _check(oracle_lib, _write(tmp_path, "corr2", model), model, s)


def _reference_m0_table(model, seed=7):
    """The model's M0 polynomial with exactly the reference's own monomial lists
    (tests/golden/standard_m0_contract.json, from libsymmetrix/source/
    standard_m0.hpp:35-60: 422 terms, 94/118/92/118 per output component):
    generated weights where the generated table has the term, random ones of
    the same spread for the 12 others (in m = +-1 of the l = 1 output), which
    no compiled slot holds and the runtime loop evaluates."""
    import os

    golden = os.path.join(os.path.dirname(__file__), "golden", "standard_m0_contract.json")
    with open(golden) as f:
        contract = json.load(f)
    rng = np.random.default_rng(seed)
    C = model["num_channels"]
    extra = 0
    for group in contract["monomial_groups"]:
        LM = str(group["output_component"])
        old = {tuple(m): j for j, m in enumerate(model["M0_monomials"][LM])}
        terms = [list(t) for t in group["terms"]]
        for a in range(model["num_elements"]):
            w = model["M0_weights"][str(a)][LM]
            spread = float(np.std(np.concatenate([np.asarray(w[str(k)]) for k in range(C)]))) or 1e-2
            for k in range(C):
                wk = w[str(k)]
                w[str(k)] = [wk[old[tuple(t)]] if tuple(t) in old else float(rng.normal(scale=spread)) for t in terms]
        extra += sum(1 for t in terms if tuple(t) not in old)
        model["M0_monomials"][LM] = terms
    assert sum(g["term_count"] for g in contract["monomial_groups"]) == 422 and extra == 12
    return model


def test_reference_m0_table_matches_oracle(oracle_lib, tmp_path):
    from symmetrix_amd import synthetic

    model = _reference_m0_table(_generated("medium3"))
    path = _write(tmp_path, "medium3_reference_m0", model)
    print("medium shape with the reference's 422-term M0 table, SrTiO3 3^3", flush=True)
    _check(oracle_lib, path, model, synthetic.srtio3_supercell(3, sigma=0.05, seed=4))


def test_reference_m0_table_stage_cost_at_the_headline_size(tmp_path):
    """Stage times of the M0 kernels with the generated table (every term in a
    compiled slot) and with the reference's table (12 terms in the runtime
    loop) on the headline workload: the 89-element medium model on SrTiO3 10^3
    (5,000 atoms), median of 5 profiled calls after 3 untimed."""
    import statistics

    from symmetrix_amd import MACEKokkosFloat, synthetic

    s = synthetic.srtio3_supercell(10, sigma=0.05, seed=0)
    generated = _generated("medium")
    times = {}
    for name, model in (("generated", generated), ("reference", _reference_m0_table(json.loads(json.dumps(generated))))):
        path = _write(tmp_path, f"medium_{name}", model)
        ev = MACEKokkosFloat(path)
        types = synthetic.node_types(s, model["atomic_numbers"])
        gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                    model["r_cut"] + 0.5)["generation"]
        for _ in range(3):
            ev._compute_prepared_factorized_positions(gen, s.positions)
        samples = []
        for _ in range(5):
            ev._set_profiling(True)
            ev._compute_prepared_factorized_positions(gen, s.positions)
            samples.append({k: ms / c if c else 0.0 for k, (ms, c) in ev._stage_times().items()})
        ev._set_profiling(False)
        times[name] = {k: statistics.median(x[k] for x in samples) for k in samples[0]}
        total = sum(times[name].values())
        print(f"  {name} M0 table: m0_forward {times[name]['m0_forward']:.4f} ms, m0_reverse "
              f"{times[name]['m0_reverse']:.4f} ms, stages {total:.4f} ms", flush=True)
    for stage in ("m0_forward", "m0_reverse"):
        assert times["reference"][stage] > 0.0
