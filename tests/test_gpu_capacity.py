"""Capacity paths of the tiled plan: graphs past the untiled plan's 32-bit
edge index, the planner's refusal on its memory estimate, the graph arrays
of a tiled graph, and a size-independent check of large tiled runs.

The tiled plan indexes edges per tile (tile-local int32 ids, 64-bit tile
bases on the host), so a graph beyond 2^31 - 1 edges runs the same code as a
small one.  SXL_EDGE_INDEX_LIMIT lowers the untiled plan's edge ceiling (a
test hook read when an evaluator is created): a 135-atom graph of 6,750
edges then takes the path of a graph past 2^31 edges -- the planner must
tile, the untiled plan and the int32 array export are refused -- and the
tiled results must match the CPU oracle (energy 1e-5 eV/atom, forces
1e-4 eV/A, stress 1e-6 eV/A^3).  SXL_DEVICE_MEMORY_LIMIT caps the memory the
planner may plan for (bytes), so its refusal can be forced on a small graph.
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5
F_TOL = 1e-4
S_TOL = 1e-6


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("tiny") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _prepare(path, model, s, limit=None, fixed=True):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    ev = MACEKokkosFloat(path)
    if fixed:
        ev._set_allow_fixed_workspace(True)
    if limit:
        ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    return ev, gen, types


def test_graph_past_the_edge_index_is_tiled_and_matches_oracle(oracle_lib, tiny, monkeypatch):
    from symmetrix_amd import synthetic

    monkeypatch.setenv("SXL_EDGE_INDEX_LIMIT", "2000")
    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=21)
    n = len(s)
    print(f"tiny SrTiO3 3^3 ({n} atoms), edge index limit 2000, 16 receivers per tile", flush=True)
    ev, gen, types = _prepare(path, model, s, limit=16)
    rep = ev.execution_plan_report
    assert rep["selected_id"] == "mh0-dual-layer-tiled-v1"
    assert "32-bit edge index" in rep["selection_reason"]
    assert not rep["candidates"][0]["qualified"]
    assert ev.stats["num_edges"] > 2000 and ev.stats["tile_receivers"] == 16
    ev._compute_prepared_factorized_positions(gen, s.positions)
    energy = ev.node_energies.sum()
    forces = ev._reduce_atom_forces(n, None, None, gen)
    stress = ev._reduce_stress(s.volume, None, gen)
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    de = abs(energy - want["energy"]) / n
    dF = float(np.max(np.abs(forces - want["forces"])))
    ds = float(np.max(np.abs(stress - want["stress_3x3"])))
    print(f"  vs oracle |dE|/atom={de:.2e} max|dF|={dF:.2e} max|dS|={ds:.2e}", flush=True)
    assert de < E_TOL and dF < F_TOL and ds < S_TOL
    # the int32 CSR export is refused past the limit, as the reference's
    with pytest.raises(OverflowError, match="32-bit"):
        ev._periodic_graph_arrays(gen)


def test_graph_past_the_edge_index_without_tiles_is_refused(tiny, monkeypatch):
    from symmetrix_amd import synthetic

    monkeypatch.setenv("SXL_EDGE_INDEX_LIMIT", "2000")
    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=22)
    print("edge index limit 2000: untiled, and tiles of 64 receivers (about 3,200 edges)", flush=True)
    with pytest.raises(OverflowError, match="32-bit edge indexing"):
        _prepare(path, model, s, fixed=False)
    with pytest.raises(OverflowError, match="smaller workspace receiver limit"):
        _prepare(path, model, s, limit=64)


def test_planner_refuses_a_tiled_plan_beyond_device_memory(tiny, monkeypatch):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=23)
    types = synthetic.node_types(s, model["atomic_numbers"])
    print("device memory limit 64 KiB, 16 receivers per tile", flush=True)
    monkeypatch.setenv("SXL_DEVICE_MEMORY_LIMIT", str(1 << 16))
    ev = MACEKokkosFloat(path)
    ev._set_allow_fixed_workspace(True)
    ev._set_dual_layer_workspace_receiver_limit_for_testing(16)
    with pytest.raises(MemoryError, match="tiled execution plan needs an estimated"):
        ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                              model["r_cut"] + 0.5)
    rep = ev.execution_plan_report
    assert rep["state"] == "refused" and rep["available_bytes"] <= 1 << 16
    assert rep["candidates"][1]["estimated_bytes"] > rep["available_bytes"]
    # the evaluator stays usable: with the cap lifted the same graph prepares
    monkeypatch.delenv("SXL_DEVICE_MEMORY_LIMIT")
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    assert ev.stats["num_tiles"] == -(-len(s) // 16)


@pytest.mark.parametrize("cells", [3, 4])
def test_tiled_graph_arrays_equal_the_build_bit_for_bit(tiny, cells):
    """Under the tiled plan the fractional edge vectors are formed from the
    int8 cell shifts and the build's fractional positions exactly as the build
    formed them: every array equals the untiled plan's and the model-free
    builder's bit for bit."""
    from symmetrix_amd import periodic_neighbor_graph, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(cells, sigma=0.07, seed=24)
    s.positions[::9] += s.cell[1] * 1.0 - s.cell[2] * 2.0  # atoms outside the cell: nonzero wraps
    print(f"SrTiO3 {cells}^3, graph arrays tiled (16 receivers) vs untiled", flush=True)
    arrays = {}
    for limit in (None, 16):
        ev, gen, _ = _prepare(path, model, s, limit=limit, fixed=limit is not None)
        assert (ev.stats["tile_receivers"] > 0) == bool(limit)
        arrays[limit] = ev._periodic_graph_arrays(gen)
    free = periodic_neighbor_graph(s.positions, s.cell, np.linalg.inv(s.cell), model["r_cut"] + 0.5)
    for key in ("num_neigh", "receiver_offsets", "sources", "shifts", "fractional_xyz"):
        a, b = np.asarray(arrays[16][key]), np.asarray(arrays[None][key])
        assert a.dtype == b.dtype and np.array_equal(a, b), key
        if key in free:
            assert np.array_equal(a, np.asarray(free[key])), key


def test_perfect_lattice_energy_is_size_independent_under_tiles(tiny):
    """A perfect lattice has the same energy per atom at every size and zero
    forces: the property a capacity run (beyond any oracle's reach) is
    checked by.  3^3 untiled against 6^3 tiled in 64-receiver tiles."""
    from symmetrix_amd import synthetic

    path, model = tiny
    out = {}
    for cells, limit in ((3, None), (6, 64)):
        s = synthetic.srtio3_supercell(cells, sigma=0.0, seed=0)
        ev, gen, _ = _prepare(path, model, s, limit=limit, fixed=limit is not None)
        ev._compute_prepared_factorized_positions(gen, s.positions)
        out[cells] = (ev.node_energies.sum() / len(s), float(np.max(np.abs(ev._reduce_atom_forces(len(s), None, None,
                                                                                                  gen)))))
        print(f"  perfect SrTiO3 {cells}^3 tiles {limit}: E/atom {out[cells][0]:.9f}, max|F| {out[cells][1]:.2e}",
              flush=True)
    assert abs(out[3][0] - out[6][0]) < 1e-6
    assert out[3][1] < 1e-5 and out[6][1] < 1e-5
