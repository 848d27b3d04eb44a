"""Tiled (fixed-workspace) execution on the GPU: the three-sweep tiled plan
against the untiled plan and the CPU oracle.

The reference checks its tiled plan at tile boundaries with a receiver
capacity of 4 and N in {3, 4, 5, 8, 9} (test_dual_layer_fixed_workspace.py:
62-130, rtol 2e-4 / atol 2e-5); here tiles of 1..16 receivers over 5- and
40-atom SrTiO3 cells, plus the medium and wide shapes, with the standard
FP32 tolerances (energy 1e-5 eV/atom, forces 1e-4 eV/A, stress 1e-6 eV/A^3).
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5
F_TOL = 1e-4
S_TOL = 1e-6


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


def _evaluate(path, model, structure, limit=None, skin=0.5):
    """Energies, directed forces, atom forces, stress and stats of one call."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    ev = MACEKokkosFloat(path)
    if limit is not None:
        ev._set_allow_fixed_workspace(True)
        ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    types = synthetic.node_types(structure, model["atomic_numbers"])
    cell = structure.cell
    gen = ev._prepare_periodic_factorized_graph(types, structure.positions, cell, np.linalg.inv(cell),
                                                model["r_cut"] + skin)["generation"]
    ev._compute_prepared_factorized_positions(gen, structure.positions)
    if limit is not None and ev.stats["tile_receivers"] > 0:
        # the tiled plan folds directed forces into atom forces tile by tile
        with pytest.raises(ValueError, match="tiled plan"):
            ev.node_forces
        directed = None
    else:
        directed = ev.node_forces.reshape(-1, 3)
    return {
        "energies": ev.node_energies,
        "directed": directed,
        "forces": ev._reduce_atom_forces(len(structure), None, None, gen),
        "stress": ev._reduce_stress(structure.volume, None, gen),
        "stats": ev.stats,
        "tiled_count": ev.dual_layer_tiled_evaluation_count,
    }


def _assert_close(a, b, n):
    de = abs(a["energies"].sum() - b["energies"].sum()) / n
    dn = float(np.max(np.abs(a["energies"] - b["energies"])))
    df = 0.0
    if a["directed"] is not None and b["directed"] is not None and a["directed"].size:
        df = float(np.max(np.abs(a["directed"] - b["directed"])))
    dF = float(np.max(np.abs(a["forces"] - b["forces"])))
    ds = float(np.max(np.abs(a["stress"] - b["stress"])))
    print(f"  |dE|/atom={de:.2e} max|dE_i|={dn:.2e} max|df_ij|={df:.2e} max|dF|={dF:.2e} max|dS|={ds:.2e}",
          flush=True)
    assert de < E_TOL and dn < E_TOL
    assert df < F_TOL and dF < F_TOL
    assert ds < S_TOL


@pytest.mark.parametrize("cells,limit", [(1, 1), (1, 2), (1, 4), (2, 3), (2, 4), (2, 8), (2, 9), (2, 16)])
def test_tiled_matches_untiled_at_tile_boundaries(tiny, cells, limit):
    from symmetrix_amd import synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(cells, sigma=0.05, seed=11)
    n = len(s)
    print(f"tiny SrTiO3 {cells}^3 ({n} atoms), {limit} receivers per tile", flush=True)
    untiled = _evaluate(path, model, s)
    tiled = _evaluate(path, model, s, limit=limit)
    assert untiled["stats"]["tile_receivers"] == 0 and untiled["tiled_count"] == 0
    assert tiled["stats"]["tile_receivers"] == limit
    assert tiled["stats"]["num_tiles"] == -(-n // limit)
    assert tiled["tiled_count"] == 1
    _assert_close(tiled, untiled, n)


def test_tiled_plan_keeps_no_graph_wide_edge_state(tiny):
    """The tiled plan holds per edge only the sources, the cell shifts (int8)
    and the tiles' source-grouped lists (11 bytes); geometry, pair codes,
    directed forces and messages live in the tile arena.  Its estimate matches the memory held,
    and the per-atom footprint is a fraction of the untiled plan's."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(8, sigma=0.05, seed=12)
    n = len(s)
    # baseline: the model and radial tables of the same element types (an
    # evaluator prepared on one unit cell; freed after)
    base = MACEKokkosFloat(path)
    unit = synthetic.srtio3_supercell(1, sigma=0.05, seed=12)
    base._prepare_periodic_factorized_graph(synthetic.node_types(unit, model["atomic_numbers"]), unit.positions,
                                            unit.cell, np.linalg.inv(unit.cell), model["r_cut"] + 0.5)
    before = base.stats["device_bytes"]
    del base
    held = {}
    for limit in (None, 256):
        ev = MACEKokkosFloat(path)
        if limit:
            ev._set_allow_fixed_workspace(True)
            ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
        types = synthetic.node_types(s, model["atomic_numbers"])
        gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                    model["r_cut"] + 0.5)["generation"]
        ev._compute_prepared_factorized_positions(gen, s.positions)
        rep = ev.execution_plan_report
        held[limit] = ev.stats["device_bytes"] - before
        est = rep["candidates"][1 if limit else 0]["estimated_bytes"]
        print(f"  limit {limit}: plan {rep['selected_id']}, held {held[limit] / n:.0f} B/atom, "
              f"estimate {est / n:.0f} B/atom", flush=True)
        assert 0.8 * held[limit] <= est <= 1.2 * held[limit]
        del ev
    assert held[256] < 0.6 * held[None]


def test_receiver_limit_at_or_above_node_count_keeps_untiled_plan(tiny):
    from symmetrix_amd import synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(1, sigma=0.05, seed=11)
    out = _evaluate(path, model, s, limit=len(s))
    assert out["stats"]["tile_receivers"] == 0 and out["tiled_count"] == 0


@pytest.mark.parametrize("preset,limit", [("medium3", 32), ("wide", 50), ("scalar", 40)])
def test_tiled_matches_oracle(oracle_lib, tmp_path_factory, preset, limit):
    from symmetrix_amd import synthetic

    path, model = _model_file(tmp_path_factory, preset)
    if preset == "wide":
        s = synthetic.water_box(num_molecules=60, seed=0)
    else:
        s = synthetic.srtio3_supercell(3, sigma=0.05, seed=0)
    n = len(s)
    print(f"{preset}: {n} atoms, {limit} receivers per tile", flush=True)
    tiled = _evaluate(path, model, s, limit=limit)
    assert tiled["stats"]["num_tiles"] == -(-n // limit)
    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    de = abs(tiled["energies"].sum() - want["energy"]) / n
    dF = float(np.max(np.abs(tiled["forces"] - want["forces"])))
    ds = float(np.max(np.abs(tiled["stress"] - want["stress_3x3"])))
    print(f"  vs oracle |dE|/atom={de:.2e} max|dF|={dF:.2e} max|dS|={ds:.2e}", flush=True)
    assert de < E_TOL and dF < F_TOL and ds < S_TOL


def test_plan_setters_invalidate_the_prepared_graph(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(1, sigma=0.05, seed=3)
    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    assert not ev.allow_fixed_workspace
    ev._set_allow_fixed_workspace(True)
    assert ev.allow_fixed_workspace
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_positions(gen, s.positions)
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell), 5.5)["generation"]
    ev._set_dual_layer_workspace_receiver_limit_for_testing(2)
    with pytest.raises(ValueError, match="stale"):
        ev._compute_prepared_factorized_positions(gen, s.positions)
    with pytest.raises(ValueError, match="receiver limit must be positive"):
        ev._set_dual_layer_workspace_receiver_limit_for_testing(0)
