"""GPU parity for the optional terms of the model format, against the CPU
oracle on the same seeded inputs (BASELINE north-star tolerances, FP32):

- ZBL pair repulsion (has_zbl; reference zbl_kokkos.cpp, double precision),
- A0 and A1 density normalisation (A0_scaled / A1_scaled with tanh-square
  density networks; mace.cpp:1561-1636, 2380-2458),
- the Agnesi distance transform of the radial features
  (compact_radial.cpp:150-170, 238-247),
- the pre_linear_up H1 basis and the first-interaction residual
  (h1_affine_schema.hpp:9-24, mace.cpp:1759-1813, 1845-1875),

each alone and all together, on the tiny, medium and wide shapes, in the
untiled and the tiled plan, plus the directed forces edge by edge and the
closed-form energy of isolated atoms of a residual-first model.
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
    "zbl": dict(zbl=True),
    "A0": dict(density=("A0",)),
    "A1": dict(density=("A1",)),
    "agnesi": dict(agnesi=True),
    "pre_linear_up": dict(h1_basis="pre_linear_up"),
    "residual": dict(h1_basis="pre_linear_up", residual=True),
    "all": dict(zbl=True, density=("A0", "A1"), agnesi=True, h1_basis="pre_linear_up", residual=True),
}


def _model(tmp_path, preset, option, seed=0):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS[preset], **OPTIONS[option])
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=seed))
    path = tmp_path / f"{preset}_{option}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _oracle(oracle_lib, model, s, skin=0.5):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + skin)


def _compare(got, want, n):
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL


@pytest.mark.parametrize("option", list(OPTIONS))
def test_tiny_options_match_oracle(oracle_lib, tmp_path, option):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = _model(tmp_path, "tiny", option)
    s = synthetic.srtio3_supercell(3, sigma=0.1, seed=6)
    print(f"tiny + {option}: SrTiO3 3^3", flush=True)
    _compare(Symmetrix(path).calculate(s), _oracle(oracle_lib, model, s), len(s))


@pytest.mark.parametrize("preset,option", [("medium3", "all"), ("medium3", "A1"), ("medium3", "residual"),
                                           ("wide", "all")])
def test_larger_shapes_with_options_match_oracle(oracle_lib, tmp_path, preset, option):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = _model(tmp_path, preset, option)
    if preset == "wide":
        s = synthetic.water_box(num_molecules=60, seed=1)
    else:
        s = synthetic.srtio3_supercell(3, sigma=0.1, seed=7)
    print(f"{preset} + {option}: {len(s)} atoms", flush=True)
    _compare(Symmetrix(path).calculate(s), _oracle(oracle_lib, model, s), len(s))


def test_all_options_directed_forces_edge_by_edge(oracle_lib, tmp_path):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = _model(tmp_path, "tiny", "all", seed=3)
    s = synthetic.srtio3_supercell(3, sigma=0.1, seed=8)
    want = _oracle(oracle_lib, model, s)
    gi = want["inputs"]
    ev = MACEKokkosFloat(path)
    ev.compute_node_energies_forces(len(s), gi["node_types"], gi["num_neigh"], gi["neigh_indices"],
                                    gi["neigh_types"], gi["xyz"], gi["r"])
    np.testing.assert_allclose(ev.node_energies, want["energies"], atol=E_TOL)
    np.testing.assert_allclose(ev.node_forces.reshape(-1, 3), want["directed_forces"], atol=F_TOL)


@pytest.mark.parametrize("limit", [7, 32])
def test_all_options_tiled_plan_matches_oracle(oracle_lib, tmp_path, limit):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = _model(tmp_path, "tiny", "all", seed=4)
    s = synthetic.srtio3_supercell(3, sigma=0.1, seed=9)
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


def test_isolated_atoms_of_residual_model_closed_form(tmp_path):
    """No neighbours: A0 = M0 = M1 = 0, so the energy is E0 + r0 . b0 +
    readout_2(S0_z^T b0) with b0 the element's scalar residual."""
    from symmetrix_amd import Symmetrix, synthetic

    path, model = _model(tmp_path, "tiny", "residual", seed=3)
    pos = np.array([[1.0, 1.0, 1.0], [13.0, 1.0, 1.0], [1.0, 13.0, 1.0]])
    s = synthetic.Structure(pos, np.array([38, 22, 8]), np.eye(3) * 36.0)
    C, ne = model["num_channels"], model["num_elements"]
    nLM = (model["L_max"] + 1) ** 2
    b = np.asarray(model["H1_first_residual_weights"]).reshape(ne, nLM, C)
    r0 = np.asarray(model["readout_1_weights_for_H1_pre_linear_up"])
    S0 = np.asarray(model["H2_weights_for_H1_pre_linear_up"]).reshape(ne, C, C)
    W1 = np.asarray(model["readout_2_weights_1"]).reshape(-1, C)
    W2 = np.asarray(model["readout_2_weights_2"])
    want = 0.0
    for z in (38, 22, 8):
        t = model["atomic_numbers"].index(z)
        zh = W1 @ (S0[t].T @ b[t, 0])
        want += model["atomic_energies"][t] + r0 @ b[t, 0] + model["readout_2_scale_factor"] * (
            W2 @ (zh / (1.0 + np.exp(-zh))))
    got = Symmetrix(path).calculate(s)
    print(f"  |dE|={abs(got['energy'] - want):.3e}", flush=True)
    assert abs(got["energy"] - want) / 3 < E_TOL
    np.testing.assert_array_equal(got["forces"], np.zeros((3, 3)))
