"""GPU: the calculator's neighbour-graph reuse across wrapped atoms, cell
changes and isolated-system motion (reference calculator.py:2838-3093), each
against a freshly built graph and the CPU oracle on the same inputs, plus the
invalid-geometry error of the prepared-positions path
(mace_kokkos_factorized_lifecycle.cpp:3078-3085)."""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("calc") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _close(a, b, n, stress=True):
    de = abs(a["energy"] - b["energy"]) / n
    df = float(np.max(np.abs(a["forces"] - b["forces"])))
    ds = float(np.max(np.abs(a["stress"] - b["stress"]))) if stress else 0.0
    print(f"  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL


def _oracle(oracle_lib, model, s):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)


def test_wrapped_atoms_reuse_the_graph(tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, _ = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=11)
    calc = Symmetrix(path, neighbor_skin=0.5)
    base = calc.calculate(s)
    wrapped = s.copy()
    # whole lattice vectors on a few atoms, then every atom wrapped into the cell
    wrapped.positions[[0, 7, 40]] += s.cell[0] - 2 * s.cell[2]
    frac = wrapped.positions @ np.linalg.inv(s.cell)
    wrapped.positions = (frac - np.floor(frac)) @ s.cell
    print("wrapped atoms, unchanged cell", flush=True)
    assert calc.evaluator._max_displacement(calc._cache["generation"], wrapped.positions) < 1e-9
    got = calc.calculate(wrapped)
    assert calc.neighbor_cache_build_count == 1 and calc.neighbor_cache_reuse_count == 1
    _close(got, base, len(s))


@pytest.mark.parametrize("strain", [0.01, -0.01, "shear"])
def test_cell_change_reuses_the_graph(oracle_lib, tiny, strain):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=12)
    calc = Symmetrix(path, neighbor_skin=0.5)
    calc.calculate(s)
    F = np.eye(3)
    if strain == "shear":
        F[0, 1] = 0.02
    else:
        F *= 1.0 + strain
    t = s.copy()
    t.cell = s.cell @ F.T
    t.positions = s.positions @ F.T + np.random.default_rng(3).normal(scale=0.03, size=s.positions.shape)
    print(f"cell change {strain}", flush=True)
    got = calc.calculate(t)
    assert calc.neighbor_cache_build_count == 1 and calc.neighbor_cache_reuse_count == 1
    assert calc.neighbor_cache_geometry_update_count == 2
    _close(got, Symmetrix(path, neighbor_skin=0.5).calculate(t), len(s))
    _close(got, _oracle(oracle_lib, model, t), len(s))


def test_large_compression_rebuilds(tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, _ = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=13)
    calc = Symmetrix(path, neighbor_skin=0.5)
    calc.calculate(s)
    t = s.copy()
    t.cell = s.cell * 0.9
    t.positions = s.positions * 0.9
    got = calc.calculate(t)
    assert calc.neighbor_cache_build_count == 2
    _close(got, Symmetrix(path, neighbor_skin=0.5).calculate(t), len(s))


def test_isolated_cluster_reuses_its_box(oracle_lib, tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, model = tiny
    rng = np.random.default_rng(5)
    pos = synthetic.srtio3_supercell(2, sigma=0.05, seed=14).positions[:20]
    nums = np.array([38, 22, 8, 8, 8] * 4)
    cluster = synthetic.Structure(pos, nums, np.zeros((3, 3)), pbc=(False, False, False))
    calc = Symmetrix(path, neighbor_skin=0.5)
    calc.calculate(cluster)
    moved = cluster.copy()
    # within skin/2 = 0.25 A of the build positions (a rigid shift counts as motion)
    moved.positions = moved.positions + rng.normal(scale=0.03, size=pos.shape) + np.array([0.05, -0.03, 0.02])
    assert np.max(np.linalg.norm(moved.positions - cluster.positions, axis=1)) < 0.25
    print("isolated cluster, small motion", flush=True)
    got = calc.calculate(moved)
    assert calc.neighbor_cache_build_count == 1
    fresh = Symmetrix(path, neighbor_skin=0.5).calculate(moved)
    _close(got, fresh, len(nums), stress=False)
    # the oracle in a box large enough to hold no images within the cutoff
    boxed = synthetic.Structure(moved.positions - moved.positions.min(axis=0) + 7.0, nums, np.eye(3) * 40.0)
    want = _oracle(oracle_lib, model, boxed)
    _close(got, want, len(nums), stress=False)


def test_coincident_atoms_raise_invalid_geometry(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.0, seed=0)
    s.positions[1] = s.positions[0]
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    with pytest.raises(ValueError, match="invalid edge geometry"):
        ev._compute_prepared_factorized_positions(gen, s.positions)
    # the next valid evaluation of a separated configuration succeeds
    s.positions[1] += np.array([0.9, 0.0, 0.0])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    assert np.isfinite(ev._total_energy(gen))


def test_fused_totals_and_displacement_match_separate_calls(tiny):
    """An evaluation from positions reduces energy and stress for the cell
    volume and measures the displacement in the same pass: both equal the
    separate reductions and the separate displacement check."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=15)
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    moved = s.positions + np.random.default_rng(2).normal(scale=0.04, size=s.positions.shape)
    ev._compute_prepared_factorized_positions(gen, moved)
    fused_d = ev._last_max_displacement()
    fused_e = ev._total_energy(gen)
    fused_s = ev._reduce_stress(s.volume, None, gen)
    assert fused_d == pytest.approx(ev._max_displacement(gen, moved), rel=0, abs=1e-14)
    assert fused_d == pytest.approx(float(np.max(np.linalg.norm(moved - s.positions, axis=1))), abs=1e-12)
    # a different volume reduces again; stress scales as 1/V
    other = ev._reduce_stress(2.0 * s.volume, None, gen)
    np.testing.assert_allclose(other, 0.5 * fused_s, rtol=1e-12, atol=1e-15)
    again = ev._reduce_stress(s.volume, None, gen)
    np.testing.assert_allclose(again, fused_s, rtol=1e-12, atol=1e-15)
    assert ev._total_energy(gen) == fused_e
    # an evaluation from edge vectors has no displacement of its own
    gi = ev._periodic_graph_arrays(gen)
    assert gi["num_neigh"].sum() == ev._graph_size()[1]


def test_long_neighbour_cutoff_gives_the_same_results(tiny):
    """A neighbour cutoff far beyond r_cut (sources with more than 1,024
    edges, beyond what the device sort stages per segment) changes the graph
    but not the physics: energies, forces and stress agree with the graph at
    r_cut + skin."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(5, sigma=0.05, seed=16)
    types = synthetic.node_types(s, model["atomic_numbers"])
    inv = np.linalg.inv(s.cell)
    out = []
    for cutoff in (model["r_cut"] + 0.5, 15.0):
        ev = MACEKokkosFloat(path)
        info = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, inv, cutoff)
        gen = info["generation"]
        ev._compute_prepared_factorized_positions(gen, s.positions)
        out.append((info["num_edges"], ev._total_energy(gen), ev._reduce_atom_forces(len(s), None, None, gen),
                    ev._reduce_stress(s.volume, None, gen)))
    (e0, E0, F0, S0), (e1, E1, F1, S1) = out
    print(f"  edges {e0} -> {e1} ({e1 / len(s):.0f} per atom)", flush=True)
    assert e1 / len(s) > 1024
    assert abs(E1 - E0) / len(s) < E_TOL
    np.testing.assert_allclose(F1, F0, atol=F_TOL)
    np.testing.assert_allclose(S1, S0, atol=S_TOL)


def _slab(pbc, vacuum=15.0, seed=31, tilt=0.0):
    """SrTiO3 3 x 3 x 2 cells with vacuum added along the open axes (more than
    cutoff + skin: no interaction across them), periodic along the others."""
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=seed)
    a = synthetic.SRTIO3_A
    keep = s.positions[:, 2] < 2.0 * a - 0.5 * a  # two of the three layers of cells
    positions = s.positions[keep]
    cell = s.cell.copy()
    for axis in range(3):
        if not pbc[axis]:
            cell[axis] = cell[axis] / np.linalg.norm(cell[axis]) * (np.ptp(positions[:, axis]) + vacuum)
    cell[1, 0] += tilt  # an oblique in-plane lattice
    return synthetic.Structure(positions.copy(), s.numbers[keep].copy(), cell, tuple(bool(p) for p in pbc))


@pytest.mark.parametrize("pbc,tiles", [((True, True, False), None), ((True, True, False), 16),
                                       ((True, False, False), None), ((False, True, True), None)])
def test_partly_periodic_cell_equals_the_periodic_box_and_oracle(oracle_lib, tiny, pbc, tiles):
    from symmetrix_amd import Symmetrix

    path, model = tiny
    slab = _slab(pbc, tilt=0.3 if pbc[0] and pbc[1] else 0.0)
    box = slab.copy()
    box.pbc = (True, True, True)
    print(f"pbc {pbc}: {len(slab)} atoms, vacuum along the open axes, tiles {tiles}", flush=True)
    calc = Symmetrix(path, neighbor_skin=0.5, allow_fixed_workspace=tiles is not None)
    if tiles:
        calc.evaluator._set_dual_layer_workspace_receiver_limit_for_testing(tiles)
    got = calc.calculate(slab)
    assert (calc.evaluator.stats["tile_receivers"] > 0) == bool(tiles)
    periodic = Symmetrix(path, neighbor_skin=0.5).calculate(box)
    _close(got, periodic, len(slab))
    _close(got, _oracle(oracle_lib, model, box), len(slab))


def test_slab_reuses_its_graph_and_rebuilds_on_a_cell_change(oracle_lib, tiny):
    from symmetrix_amd import Symmetrix

    path, model = tiny
    slab = _slab((True, True, False), seed=32)
    calc = Symmetrix(path, neighbor_skin=0.5)
    calc.calculate(slab)
    rng = np.random.default_rng(5)
    moved = slab.copy()
    moved.positions = slab.positions + rng.normal(scale=0.05, size=slab.positions.shape)
    moved.positions[[1, 9]] += slab.cell[0]  # whole periodic lattice vectors: not a move
    print("slab: small moves and periodic wraps reuse the graph", flush=True)
    got = calc.calculate(moved)
    assert calc.neighbor_cache_build_count == 1 and calc.neighbor_cache_reuse_count == 1
    _close(got, Symmetrix(path, neighbor_skin=0.5).calculate(moved), len(slab))
    # an atom moved past skin/2 along the open axis: rebuilt
    far = moved.copy()
    far.positions[4, 2] += 0.4
    got = calc.calculate(far)
    assert calc.neighbor_cache_build_count == 2
    _close(got, Symmetrix(path, neighbor_skin=0.5).calculate(far), len(slab))
    # an in-plane strain: the partly periodic graph is rebuilt, as the reference's
    strained = far.copy()
    F = np.array([[1.01, 0.004, 0.0], [0.004, 0.995, 0.0], [0.0, 0.0, 1.0]])
    strained.cell = far.cell @ F.T
    strained.positions = far.positions @ F.T
    print("slab: in-plane strain", flush=True)
    got = calc.calculate(strained)
    assert calc.neighbor_cache_build_count == 3
    box = strained.copy()
    box.pbc = (True, True, True)
    _close(got, _oracle(oracle_lib, model, box), len(slab))
