"""GPU parity: the HIP path (through libsymmetrix_amd.so's C ABI) against the
CPU oracle on the same seeded inputs.

Tolerances (FP32): energy 1e-5 eV/atom, forces 1e-4 eV/A,
stress 1e-6 eV/A^3; neighbour lists bit-exact.
"""

import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


@pytest.fixture(scope="module")
def native():
    from symmetrix_amd import _native

    return _native.library()


def _model_file(tmp_path_factory, preset, seed=0):
    from symmetrix_amd import synthetic

    model = synthetic.random_mace_model(preset, seed=seed)
    text = synthetic.model_json(model)
    path = tmp_path_factory.mktemp(preset) / f"{preset}.json"
    path.write_text(text)
    return str(path), json.loads(text)


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    return _model_file(tmp_path_factory, "tiny")


@pytest.fixture(scope="module")
def medium3(tmp_path_factory):
    return _model_file(tmp_path_factory, "medium3")


@pytest.fixture(scope="module")
def wide(tmp_path_factory):
    return _model_file(tmp_path_factory, "wide")


def _compare(calc_result, oracle_result, n):
    de = abs(calc_result["energy"] - oracle_result["energy"]) / n
    df = float(np.max(np.abs(calc_result["forces"] - oracle_result["forces"])))
    ds = float(np.max(np.abs(calc_result["stress"] - oracle_result["stress"])))
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL
    assert df < F_TOL
    assert ds < S_TOL


# --------------------------------------------------------------------------
# neighbour graph: reference known answers and bit-exact agreement
# --------------------------------------------------------------------------


def test_neighbor_graph_small_known_answer(native):
    # reference symmetrix/test/test_device_environment.py:168-196
    from symmetrix_amd import periodic_neighbor_graph

    cell = np.eye(3) * 4.0
    positions = np.array([[0.1, 0.0, 0.0], [0.3, 0.0, 0.0], [3.9, 0.0, 0.0]])
    g = periodic_neighbor_graph(positions, cell, np.linalg.inv(cell), 0.5)
    np.testing.assert_array_equal(g["receiver_offsets"], [0, 2, 4, 6])
    np.testing.assert_array_equal(g["sources"], [2, 1, 2, 0, 0, 1])
    np.testing.assert_array_equal(
        g["shifts"], [[-1, 0, 0], [0, 0, 0], [-1, 0, 0], [0, 0, 0], [1, 0, 0], [1, 0, 0]])
    np.testing.assert_allclose(
        g["fractional_xyz"],
        [[-0.05, 0, 0], [0.05, 0, 0], [-0.1, 0, 0], [-0.05, 0, 0], [0.05, 0, 0], [0.1, 0, 0]],
        atol=1e-15)


def test_neighbor_graph_zero_and_empty(native):
    # reference test_device_environment.py:200-226
    from symmetrix_amd import periodic_neighbor_graph

    cell = np.eye(3) * 10.0
    g = periodic_neighbor_graph(np.array([[0.0, 0, 0], [4.0, 4, 4]]), cell, np.linalg.inv(cell), 0.5)
    assert g["sources"].size == 0 and g["shifts"].shape == (0, 3)
    np.testing.assert_array_equal(g["num_neigh"], [0, 0])
    np.testing.assert_array_equal(g["receiver_offsets"], [0, 0, 0])
    e = periodic_neighbor_graph(np.empty((0, 3)), cell, np.linalg.inv(cell), 0.5)
    assert e["sources"].size == 0
    np.testing.assert_array_equal(e["receiver_offsets"], [0])


def test_neighbor_graph_rejects_invalid_inputs(native):
    # reference test_device_environment.py:228-245
    from symmetrix_amd import periodic_neighbor_graph

    cell = np.eye(3) * 4.0
    with pytest.raises(ValueError, match="cutoff must be finite and positive"):
        periodic_neighbor_graph(np.zeros((1, 3)), cell, np.linalg.inv(cell), 0.0)
    with pytest.raises(ValueError, match="cell and inverse cell are inconsistent"):
        periodic_neighbor_graph(np.zeros((1, 3)), cell, np.zeros((3, 3)), 1.0)


@pytest.mark.parametrize("case", ["srtio3", "triclinic", "small_cell", "one_bin"])
def test_neighbor_graph_bit_exact_vs_oracle(native, oracle_lib, case):
    from symmetrix_amd import periodic_neighbor_graph, synthetic

    rng = np.random.default_rng(7)
    if case == "srtio3":
        s = synthetic.srtio3_supercell(4, sigma=0.05, seed=3)
        pos, cell, cutoff = s.positions, s.cell, 6.5
    elif case == "one_bin":
        # a cutoff above half the cell: one bin holding all 1,080 atoms, more
        # than the device sort stages per segment
        s = synthetic.srtio3_supercell(6, sigma=0.05, seed=4)
        pos, cell, cutoff = s.positions, s.cell, 12.0
    elif case == "triclinic":
        cell = np.array([[9.2, 0.0, 0.0], [1.7, 8.1, 0.0], [-0.9, 1.3, 10.3]])
        pos = rng.uniform(-2.0, 12.0, size=(200, 3))  # includes atoms outside the cell
        cutoff = 4.7
    else:
        cell = np.array([[3.2, 0.0, 0.0], [0.7, 4.1, 0.0], [-0.4, 0.6, 5.3]])
        pos = rng.uniform(0.0, 1.0, size=(4, 3)) @ cell
        cutoff = 4.7
    inv = np.linalg.inv(cell)
    got = periodic_neighbor_graph(pos, cell, inv, cutoff)
    want = oracle_lib.neighbor_graph(pos, cell, inv, cutoff)
    for key in ("num_neigh", "receiver_offsets", "sources", "shifts"):
        np.testing.assert_array_equal(got[key], want[key])
    # bit-exact doubles
    assert got["fractional_xyz"].tobytes() == want["fractional_xyz"].tobytes()


# --------------------------------------------------------------------------
# full E + F + stress parity
# --------------------------------------------------------------------------


def _oracle_eval(oracle_lib, model, structure, skin=0.5):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(structure, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    return oracle_lib.evaluate(orc, structure, model["r_cut"] + skin)


@pytest.mark.parametrize("n", [2, 3])
def test_tiny_srtio3_parity(native, oracle_lib, tiny, n):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(n, sigma=0.05, seed=0)
    print(f"tiny SrTiO3 {n}^3 ({len(s)} atoms)", flush=True)
    got = Symmetrix(path).calculate(s)
    _compare(got, _oracle_eval(oracle_lib, model, s), len(s))


def test_tiny_directed_forces_match_oracle_edge_by_edge(native, oracle_lib, tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=2)
    want = _oracle_eval(oracle_lib, model, s)
    gi = want["inputs"]
    ev = MACEKokkosFloat(path)
    ev.compute_node_energies_forces(len(s), gi["node_types"], gi["num_neigh"], gi["neigh_indices"],
                                    gi["neigh_types"], gi["xyz"], gi["r"])
    np.testing.assert_allclose(ev.node_energies, want["energies"], atol=E_TOL)
    np.testing.assert_allclose(ev.node_forces.reshape(-1, 3), want["directed_forces"], atol=F_TOL)


def test_medium_shape_parity(native, oracle_lib, medium3):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = medium3
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=0)
    print(f"medium shape SrTiO3 3^3 ({len(s)} atoms)", flush=True)
    got = Symmetrix(path).calculate(s)
    _compare(got, _oracle_eval(oracle_lib, model, s), len(s))


def test_wide_shape_parity(native, oracle_lib, wide):
    # C = 256 with a 17.8 MB coupling-radial table: the second interaction
    # runs in four 64-channel slices (forward and reverse), the reverse's
    # per-slice force parts added in slice order, so repeats agree bitwise
    from symmetrix_amd import Symmetrix, synthetic

    path, model = wide
    s = synthetic.water_box(num_molecules=60, seed=0)
    print(f"wide shape water ({len(s)} atoms)", flush=True)
    calc = Symmetrix(path)
    got = calc.calculate(s)
    _compare(got, _oracle_eval(oracle_lib, model, s), len(s))
    again = calc.calculate(s.copy())
    assert np.array_equal(got["forces"], again["forces"])
    assert got["energy"] == again["energy"]


def test_wide_shape_sliced_reverse_equals_unsliced(native, wide, monkeypatch):
    """The channel-sliced R1 reverse (four one-wave workgroups per receiver,
    force parts added in slice order) against the one-workgroup grouped
    reverse (SXL_R1_REVERSE_SLICES=1) on the same graph: node energies are
    identical (the reverse does not touch them); directed forces, atom forces
    and the virial differ only by FP64 summation order."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = wide
    s = synthetic.water_box(num_molecules=60, seed=3)
    types = synthetic.node_types(s, model["atomic_numbers"])

    def run():
        ev = MACEKokkosFloat(path)
        gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                    model["r_cut"] + 0.5)["generation"]
        ev._compute_prepared_factorized_positions(gen, s.positions)
        return (ev.node_energies.copy(), ev.node_forces.reshape(-1, 3).copy(),
                ev._reduce_atom_forces(len(s), None, None, gen), ev._reduce_stress(s.volume, None, gen))

    sliced = run()
    monkeypatch.setenv("SXL_R1_REVERSE_SLICES", "1")
    whole = run()
    print(f"wide water ({len(s)} atoms): max|df_ij| = {np.max(np.abs(sliced[1] - whole[1])):.2e}", flush=True)
    assert np.array_equal(sliced[0], whole[0])
    scale = float(np.max(np.abs(whole[1])))
    assert scale > 0.0
    assert np.max(np.abs(sliced[1] - whole[1])) <= 1e-12 * scale
    assert np.max(np.abs(sliced[2] - whole[2])) <= 1e-11 * scale
    assert np.max(np.abs(sliced[3] - whole[3])) <= 1e-11 * max(1.0, float(np.max(np.abs(whole[3]))))
    monkeypatch.setenv("SXL_R1_REVERSE_SLICES", "3")
    with pytest.raises(ValueError, match="SXL_R1_REVERSE_SLICES"):
        run()


def test_scalar_shape_parity(native, oracle_lib, tmp_path_factory):
    # L_max = 0: scalar H1, 4 coupling paths (l, 0 -> l), 16 terms
    from symmetrix_amd import Symmetrix, synthetic

    path, model = _model_file(tmp_path_factory, "scalar")
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=0)
    print(f"scalar shape SrTiO3 3^3 ({len(s)} atoms)", flush=True)
    got = Symmetrix(path).calculate(s)
    _compare(got, _oracle_eval(oracle_lib, model, s), len(s))


def test_repeat_evaluation_is_bitwise_deterministic(native, tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=4)
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    info = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)
    gen = info["generation"]
    outs = []
    for _ in range(3):
        ev._compute_prepared_factorized_positions(gen, s.positions)
        outs.append((ev.node_energies.tobytes(), ev.node_forces.tobytes(),
                     ev._reduce_stress(s.volume, None, gen).tobytes()))
    assert outs[0] == outs[1] == outs[2]


def test_stale_generation_is_rejected(native, tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=4)
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    g1 = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    g2 = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    assert g2 != g1
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_positions(g1, s.positions)


def test_failed_preparation_makes_earlier_tokens_stale(native, tiny):
    """A preparation that raises after it has started to change the graph
    state (here: a neighbour type outside the model, found while the edge
    pair table is formed) leaves no earlier generation usable."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=4)
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    g1 = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    ev._compute_prepared_factorized_positions(g1, s.positions)
    n = len(s)
    num_neigh = np.ones(n, dtype=np.int32)
    neigh = ((np.arange(n) + 1) % n).astype(np.int32)
    bad_types = np.full(n, model["num_elements"], dtype=np.int32)  # out of range
    with pytest.raises(IndexError):
        ev._prepare_factorized_graph(n, types, num_neigh, neigh, bad_types)
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_positions(g1, s.positions)


def test_skin_reuse_matches_fresh_graph(native, tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, _ = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=5)
    calc = Symmetrix(path, neighbor_skin=0.5)
    calc.calculate(s)
    moved = s.copy()
    moved.positions = moved.positions + np.random.default_rng(1).normal(scale=0.05, size=moved.positions.shape)
    reused = calc.calculate(moved)
    assert calc.neighbor_rebuild_count == 1
    fresh = Symmetrix(path, neighbor_skin=0.5).calculate(moved)
    # same active edges, possibly in another order: FP32 summation-order noise only
    assert abs(reused["energy"] - fresh["energy"]) < E_TOL * len(s)
    np.testing.assert_allclose(reused["forces"], fresh["forces"], atol=F_TOL)
    far = s.copy()
    far.positions[0] += 0.3  # more than skin/2
    calc.calculate(far)
    assert calc.neighbor_rebuild_count == 2
