"""GPU parity of the l_max = 2 shapes beside the tiny preset's (2, 1): scalar
hidden features (L_max = 0, paths (l, 0, l)) and hidden features up to l = 2
(L_max = 2, 11 paths, 83 coupling terms), each at correlation 2 (the
compiled symmetric-contraction table) and 3 (every M0 term in the kernels'
runtime remainder loop), against the CPU oracle on the same structure with
the standard FP32 tolerances; and the (2, 2) shape under the tiled plan.
"""

import dataclasses
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _model(tmp_path, L_max, correlation, channels=64, seed=3):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["tiny"], channels=channels, L_max=L_max,
                                correlation=correlation)
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=seed))
    path = tmp_path / f"shape_2{L_max}_c{correlation}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _oracle(oracle_lib, model, s):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)


@pytest.mark.parametrize("L_max,correlation", [(0, 2), (0, 3), (2, 2), (2, 3)])
def test_lmax2_shape_matches_oracle(oracle_lib, tmp_path, L_max, correlation):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = _model(tmp_path, L_max, correlation)
    assert (model["l_max"], model["L_max"]) == (2, L_max)
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=4)
    n = len(s)
    print(f"(l_max, L_max) = (2, {L_max}), correlation {correlation}, C = 64: SrTiO3 3^3 ({n} atoms)",
          flush=True)
    got = Symmetrix(path).calculate(s)
    want = _oracle(oracle_lib, model, s)
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    assert np.max(np.abs(got["forces"].sum(axis=0))) < 1e-6 * n


def test_lmax2_hidden_l2_shape_tiled_matches_oracle(oracle_lib, tmp_path):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = _model(tmp_path, 2, 2)
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=5)
    n = len(s)
    limit = 40
    print(f"(2, 2) shape, tiled plan with {limit} receivers per tile: SrTiO3 3^3 ({n} atoms)", flush=True)
    ev = MACEKokkosFloat(path)
    ev._set_allow_fixed_workspace(True)
    ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    assert ev.stats["num_tiles"] == -(-n // limit)
    energy = float(ev.node_energies.sum())
    forces = ev._reduce_atom_forces(n, None, None, gen)
    stress = ev._reduce_stress(s.volume, None, gen)
    want = _oracle(oracle_lib, model, s)
    de = abs(energy - want["energy"]) / n
    df = float(np.max(np.abs(forces - want["forces"])))
    ds = float(np.max(np.abs(stress - want["stress_3x3"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL
