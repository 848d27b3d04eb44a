"""GPU: the execution planner and its report (reference execution_plan.hpp,
mace_kokkos_runtime.cpp:3843-3915, calculator.py:1691-1725): candidate
memory estimates against the device memory actually held, the selection
rules (capacity / speed profiles, fixed-workspace opt-in, debug pins) and
that a pinned tiled plan gives the untiled plan's results."""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5
F_TOL = 1e-4


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("plan") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _prepare(ev, s, model):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    return ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                 model["r_cut"] + 0.5)["generation"]


def test_report_pending_then_untiled_with_estimate(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    before = MACEKokkosFloat(path).stats["device_bytes"]  # tables of one evaluator (freed after)
    ev = MACEKokkosFloat(path)
    rep = ev.execution_plan_report
    assert rep["state"] == "pending" and rep["selected_id"] == ""
    s = synthetic.srtio3_supercell(8, sigma=0.05, seed=41)
    gen = _prepare(ev, s, model)
    ev._compute_prepared_factorized_positions(gen, s.positions)
    rep = ev.execution_plan_report
    print(json.dumps(rep, indent=1), flush=True)
    assert rep["state"] == "active" and rep["selected_id"] == "mh0-direct-speed"
    assert rep["requested_algorithm"] == "direct" and rep["requested_profile"] == "capacity"
    assert rep["available_bytes"] > rep["reserve_bytes"] > 0 and not rep["boundary_attempt"]
    ids = [c["id"] for c in rep["candidates"]]
    assert ids == ["mh0-direct-speed", "mh0-dual-layer-tiled-v1"]
    tiled = rep["candidates"][1]
    assert not tiled["qualified"] and "allow_fixed_workspace" in tiled["reason"]
    # the untiled estimate accounts for the graph and work arrays actually held
    held = ev.stats["device_bytes"] - before
    est = rep["candidates"][0]["estimated_bytes"]
    print(f"  estimate {est / 2**20:.1f} MiB, held {held / 2**20:.1f} MiB", flush=True)
    assert 0.8 * held <= est <= 1.2 * held


def test_selection_rules_and_pinned_tiles_match(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(4, sigma=0.05, seed=42)
    base = MACEKokkosFloat(path)
    gen = _prepare(base, s, model)
    base._compute_prepared_factorized_positions(gen, s.positions)
    e0 = base._total_energy(gen)
    f0 = base._reduce_atom_forces(len(s), None, None, gen)

    ev = MACEKokkosFloat(path)
    ev._set_dual_layer_workspace_receiver_limit_for_testing(48)
    # speed: untiled even with a receiver limit and fixed workspace allowed
    ev._set_allow_fixed_workspace(True)
    ev._set_execution_plan_request("direct", "speed")
    _prepare(ev, s, model)
    assert ev.execution_plan_report["selected_id"] == "mh0-direct-speed"
    # capacity with the limit: tiles
    ev._set_execution_plan_request("direct", "capacity")
    _prepare(ev, s, model)
    rep = ev.execution_plan_report
    assert rep["selected_id"] == "mh0-dual-layer-tiled-v1" and rep["candidates"][1]["qualified"]
    assert ev.stats["num_tiles"] == -(-len(s) // 48)
    # a debug pin selects tiles without the fixed-workspace opt-in
    ev._set_allow_fixed_workspace(False)
    ev._set_execution_plan_request("direct", "capacity", "mh0-dual-layer-tiled-v1")
    gen = _prepare(ev, s, model)
    rep = ev.execution_plan_report
    assert rep["selection_source"] == "debug_override" and rep["selected_id"] == "mh0-dual-layer-tiled-v1"
    ev._compute_prepared_factorized_positions(gen, s.positions)
    assert abs(ev._total_energy(gen) - e0) / len(s) < E_TOL
    np.testing.assert_allclose(ev._reduce_atom_forces(len(s), None, None, gen), f0, atol=F_TOL)


def test_invalid_plan_requests(tiny):
    from symmetrix_amd import MACEKokkosFloat

    path, _ = tiny
    ev = MACEKokkosFloat(path)
    with pytest.raises(ValueError, match="direct"):
        ev._set_execution_plan_request("generic", "capacity")
    with pytest.raises(ValueError, match="execution_profile"):
        ev._set_execution_plan_request("direct", "fastest")
    with pytest.raises(ValueError, match="_debug_execution_plan"):
        ev._set_execution_plan_request("direct", "capacity", "mh0-direct-capacity-y-only")
    with pytest.raises(ValueError, match="capacity"):
        ev._set_execution_plan_request("direct", "speed", "mh0-dual-layer-tiled-v1")


def test_calculator_exposes_the_plan(tiny):
    from symmetrix_amd import Symmetrix, synthetic

    path, _ = tiny
    calc = Symmetrix(path, execution_profile="speed")
    assert calc.execution_plan["state"] == "pending"
    calc.calculate(synthetic.srtio3_supercell(2, sigma=0.05, seed=43))
    plan = calc.execution_plan
    assert plan["requested_profile"] == "speed" and plan["selected_id"] == "mh0-direct-speed"
