"""GPU parity of the unfolded layer-0 table.

With many active element types the folded layer-0 table (H0[source type] and
A0_W[receiver type] folded into the spline rows per ordered pair of types)
grows past what stays in cache, and the untiled plan switches to the unfolded
table: one row set per unordered radial table, H0 of the source's type applied
per edge, A0_W applied to each node's sums by per-type GEMMs (and its
transpose to the adjoint).  The evaluator chooses it by the folded table's
size (the 10-type irregular box of test_gpu_configs.py takes it);
SXL_A0_UNFOLDED=1 forces it here on small systems, =0 forces the folded path.

Checked against the CPU oracle (BASELINE north-star tolerances, FP32) with the
model options that touch layer 0 (A0 density scaling, per-pair Agnesi
tables, everything together), on the tiny, medium and wide shapes, against
the folded path on the same inputs, and in the tiled plan, which keeps the
folded table.
"""

import dataclasses
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3

OPTIONS = {
    "plain": dict(),
    "A0": dict(density=("A0",)),
    "agnesi": dict(agnesi=True),
    "all": dict(zbl=True, density=("A0", "A1"), agnesi=True, h1_basis="pre_linear_up", residual=True),
}


def _model(tmp_path, preset, option, seed=0):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS[preset], **OPTIONS[option])
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=seed))
    path = tmp_path / f"{preset}_{option}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _structure(preset, seed):
    from symmetrix_amd import synthetic

    if preset == "wide":
        return synthetic.water_box(num_molecules=60, seed=seed)
    return synthetic.srtio3_supercell(3, sigma=0.1, seed=seed)


def _oracle(oracle_lib, model, s, skin=0.5):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + skin)


def _compare(got, want, n, e_tol=E_TOL, f_tol=F_TOL, s_tol=S_TOL):
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < e_tol and df < f_tol and ds < s_tol


@pytest.mark.parametrize("preset,option", [("tiny", "plain"), ("tiny", "A0"), ("tiny", "agnesi"), ("tiny", "all"),
                                           ("medium3", "plain"), ("medium3", "all"), ("wide", "plain")])
def test_unfolded_layer0_matches_oracle(oracle_lib, tmp_path, monkeypatch, preset, option):
    from symmetrix_amd import Symmetrix

    monkeypatch.setenv("SXL_A0_UNFOLDED", "1")
    path, model = _model(tmp_path, preset, option)
    s = _structure(preset, seed=11)
    print(f"unfolded layer 0, {preset} + {option}: {len(s)} atoms", flush=True)
    _compare(Symmetrix(path).calculate(s), _oracle(oracle_lib, model, s), len(s))


def test_unfolded_and_folded_layer0_agree(tmp_path, monkeypatch):
    from symmetrix_amd import Symmetrix

    path, _ = _model(tmp_path, "medium3", "all", seed=2)
    s = _structure("medium3", seed=12)
    monkeypatch.setenv("SXL_A0_UNFOLDED", "1")
    unfolded = Symmetrix(path).calculate(s)
    monkeypatch.setenv("SXL_A0_UNFOLDED", "0")
    folded = Symmetrix(path).calculate(s)
    # the two paths round differently (the sums over input channels run
    # before or after the edge sum); both are FP32 evaluations of one model
    _compare(unfolded, folded, len(s), e_tol=1e-6, f_tol=2e-5, s_tol=2e-7)


@pytest.mark.parametrize("limit", [7, 32])
def test_tiled_plan_keeps_the_folded_table(oracle_lib, tmp_path, monkeypatch, limit):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    monkeypatch.setenv("SXL_A0_UNFOLDED", "1")
    path, model = _model(tmp_path, "tiny", "all", seed=4)
    s = _structure("tiny", seed=13)
    want = _oracle(oracle_lib, model, s)
    ev = MACEKokkosFloat(path)
    ev._set_allow_fixed_workspace(True)
    ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    assert ev.stats["num_tiles"] > 1
    ev._compute_prepared_factorized_positions(gen, s.positions)
    n = len(s)
    assert abs(ev._total_energy(gen) - want["energy"]) / n < E_TOL
    np.testing.assert_allclose(ev._reduce_atom_forces(n, None, None, gen), want["forces"], atol=F_TOL)
