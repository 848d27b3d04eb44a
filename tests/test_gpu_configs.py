"""GPU parity on the benchmark configurations at their full sizes, and on the
degenerate inputs the reference's tests exercise.

- headline: the 89-element medium model on SrTiO3 10^3 (5,000 atoms,
  BASELINE configs[1]), the workload bench.py times;
- the wide shape carrying the reference's own 215 coupling terms
  (jit_r1_mace_mp0b2_large_contract.json) on 300 water molecules;
- irregular: 20,000 atoms uniform at 0.08 /A^3 with 1.8 A minimum separation,
  10 elements, the 89-element medium-shape model: a
  wide neighbour-count distribution and 100 ordered element pairs;
- water: 10,000 rigid H2O (30,000 atoms) at 1.0 g/cm^3, the wide model
  (C = 256, hidden 0e+1o+2e).

Both are compared with the CPU oracle on the same inputs (BASELINE north-star
tolerances, FP32), plus the size-independent checks: the atom forces of a
periodic system sum to zero and the stress is symmetric.  The degenerate
cases follow the reference's zero / empty graph tests
(test_device_environment.py:200-226): an atom without neighbours carries
E0 + readout of zero features and no force, a single atom sees only its own
periodic images, and a structure without atoms is rejected at prepare.
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _model(tmp_path_factory, preset):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model(preset, seed=0))
    path = tmp_path_factory.mktemp(preset) / f"{preset}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _full_size_check(oracle_lib, path, model, s, label):
    from symmetrix_amd import Symmetrix, synthetic

    print(f"{label}: {len(s)} atoms", flush=True)
    got = Symmetrix(path).calculate(s)
    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    n = len(s)
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    # size-independent properties
    assert np.all(np.isfinite(got["forces"]))
    assert np.max(np.abs(got["forces"].sum(axis=0))) < 1e-6 * n
    sigma = got["stress_3x3"] if "stress_3x3" in got else None
    if sigma is not None:
        np.testing.assert_allclose(sigma, sigma.T, atol=1e-9)


@pytest.fixture(scope="module")
def medium(tmp_path_factory):
    return _model(tmp_path_factory, "medium")


def test_headline_config_full_size(oracle_lib, medium):
    # the workload bench.py times: the 89-element medium model on the perturbed
    # SrTiO3 10^3 supercell, sigma 0.05 A, seed 0
    from symmetrix_amd import synthetic

    path, model = medium
    s = synthetic.srtio3_supercell(10, sigma=0.05, seed=0)
    _full_size_check(oracle_lib, path, model, s, "SrTiO3 10^3, medium model (89 elements, 3 active)")


@pytest.mark.parametrize("contract_name", ["jit_r1_mace_mp0b2_large_contract.json",
                                           "jit_r1_mace_off23_large_contract.json"])
def test_wide_model_with_reference_coupling_values(oracle_lib, tmp_path, contract_name):
    # the wide (3,2) shape with the coupling terms and channel count of the
    # reference's own contracts (tests/golden, from
    # symmetrix/test/data/execution_contracts/: mp0b2-large, 128 channels, and
    # off23-large, 224 channels -- an unsliced R1 forward over a 15.5 MB
    # table; 17 paths, 215 terms each) in place of the generated ones
    import dataclasses
    import os

    from symmetrix_amd import synthetic

    golden = os.path.join(os.path.dirname(__file__), "golden", contract_name)
    with open(golden) as f:
        contract = json.load(f)
    shape = dataclasses.replace(synthetic.PRESETS["wide"], channels=contract["channels"])
    model = json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=5)))
    assert [(l1, l2, lo) for l1, l2, lo in zip(model["Phi1_l1"], model["Phi1_l2"], model["Phi1_l"])] == [
        (p["edge_l"], p["source_l"], p["output_l"]) for p in contract["paths"]]
    terms = contract["sparse_coupling"]["terms"]
    assert len(terms) == 215
    model["Phi1_lme"] = [t["lme"] for t in terms]
    model["Phi1_lelm1lm2"] = [t["row"] for t in terms]
    model["Phi1_clebsch_gordan"] = [t["coefficient"] for t in terms]
    path = tmp_path / "wide_contract.json"
    path.write_text(json.dumps(model))
    s = synthetic.water_box(300, seed=2)
    _full_size_check(oracle_lib, str(path), model, s,
                     f"water 300 H2O, wide shape, C={contract['channels']}, the reference's 215 coupling terms")


@pytest.mark.parametrize("contract_name", ["jit_r1_mace_omat0_small_contract.json",
                                           "jit_r1_mace_off23_small_contract.json"])
def test_scalar_model_with_reference_coupling_values(oracle_lib, tmp_path, contract_name):
    # the scalar (3,0) shape with the coupling terms and channel count of the
    # reference's omat0-small (128 channels) and off23-small (96 channels)
    # contracts (tests/golden, from symmetrix/test/data/execution_contracts/:
    # 4 paths, 16 terms)
    import dataclasses
    import os

    from symmetrix_amd import synthetic

    golden = os.path.join(os.path.dirname(__file__), "golden", contract_name)
    with open(golden) as f:
        contract = json.load(f)
    shape = dataclasses.replace(synthetic.PRESETS["scalar"], channels=contract["channels"])
    model = json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=5)))
    assert model["num_channels"] == contract["channels"]
    assert [(l1, l2, lo) for l1, l2, lo in zip(model["Phi1_l1"], model["Phi1_l2"], model["Phi1_l"])] == [
        (p["edge_l"], p["source_l"], p["output_l"]) for p in contract["paths"]]
    terms = contract["sparse_coupling"]["terms"]
    assert len(terms) == 16
    model["Phi1_lme"] = [t["lme"] for t in terms]
    model["Phi1_lelm1lm2"] = [t["row"] for t in terms]
    model["Phi1_clebsch_gordan"] = [t["coefficient"] for t in terms]
    path = tmp_path / "scalar_contract.json"
    path.write_text(json.dumps(model))
    s = synthetic.srtio3_supercell(6, sigma=0.05, seed=2)
    _full_size_check(oracle_lib, str(path), model, s,
                     f"SrTiO3 6^3, scalar shape, C={contract['channels']}, the reference's 16 coupling terms")


def test_irregular_config_full_size(oracle_lib, medium):
    from symmetrix_amd import synthetic

    path, model = medium
    s = synthetic.irregular_box(seed=0)
    _full_size_check(oracle_lib, path, model, s, "irregular box, medium model (89 elements, 10 active)")


def test_water_config_full_size(oracle_lib, tmp_path_factory):
    from symmetrix_amd import synthetic

    path, model = _model(tmp_path_factory, "wide")
    s = synthetic.water_box(seed=0)
    _full_size_check(oracle_lib, path, model, s, "water box, wide model (C=256, L_max 2)")


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    return _model(tmp_path_factory, "tiny")


def _isolated_energy(model, z):
    """E0 + readout of a node with A0 = 0 (M0 = 0, M1 = 0, H2 = 0):
    readout_2(0) = sum_h w2[h] * scale * silu(0) = 0, readout_1 . 0 = 0."""
    return model["atomic_energies"][model["atomic_numbers"].index(z)]


def test_isolated_atoms_carry_only_e0(tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = tiny
    # three atoms 12 A apart in a 36 A cube: no neighbours within 5.5 A
    pos = np.array([[1.0, 1.0, 1.0], [13.0, 1.0, 1.0], [1.0, 13.0, 1.0]])
    s = synthetic.Structure(pos, np.array([38, 22, 8]), np.eye(3) * 36.0)
    got = Symmetrix(path).calculate(s)
    want = sum(_isolated_energy(model, z) for z in (38, 22, 8))
    assert abs(got["energy"] - want) < 1e-9
    np.testing.assert_array_equal(got["forces"], np.zeros((3, 3)))
    np.testing.assert_array_equal(got["stress"], np.zeros(6))


def test_single_atom_with_periodic_images_matches_oracle(oracle_lib, tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = tiny
    # one Sr atom in a 3.9 A cube: every neighbour is a periodic image of itself
    s = synthetic.Structure(np.array([[0.3, 0.2, 0.1]]), np.array([38]), np.eye(3) * 3.9)
    got = Symmetrix(path).calculate(s)
    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    assert abs(got["energy"] - want["energy"]) < E_TOL
    np.testing.assert_allclose(got["forces"], want["forces"], atol=F_TOL)
    np.testing.assert_allclose(got["stress"], want["stress"], atol=S_TOL)


def test_empty_structure_is_rejected_like_the_reference(tiny):
    """No atoms means no active element types: the reference raises
    invalid_argument at prepare (mace_kokkos_factorized_lifecycle.cpp:3956-3957)."""
    from symmetrix_amd import MACEKokkosFloat

    path, _ = tiny
    ev = MACEKokkosFloat(path)
    empty = np.zeros(0, np.int32)
    with pytest.raises(ValueError, match="at least one active type"):
        ev._prepare_factorized_graph(0, empty, empty, empty, empty)
