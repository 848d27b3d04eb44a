"""Workspace and policy properties of MACEKokkosFloat on the GPU: the
reference's read-only properties (symmetrix/source/cpp/mace_kokkos.cpp:
459-723) report the buffers and plan of the prepared graph, untiled and
tiled, and go back to "no graph" when a setter invalidates it."""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    model = synthetic.random_mace_model("tiny", seed=0)
    text = synthetic.model_json(model)
    path = tmp_path_factory.mktemp("ws") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _prepare(ev, model, s):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    return gen


def test_untiled_plan_properties(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=1)
    n = len(s)
    ev = MACEKokkosFloat(path)
    assert not ev.factorized_ready and ev.factorized_graph_generation == 0
    assert ev.low_memory_policy == "disabled" and not ev.low_memory_requested
    gen = _prepare(ev, model, s)
    print(f"untiled: phi1 {ev.phi1_workspace_bytes} B, work {ev.factorized_workspace_bytes} B, "
          f"graph {ev.factorized_graph_device_capacity_bytes} B", flush=True)
    assert ev.factorized_ready and not ev.factorized_tiled_ready
    assert ev.factorized_graph_generation == gen
    C = ev.num_channels
    assert ev.phi1_workspace_bytes > 0 and ev.phi1_workspace_bytes % (n * C * 4) == 0
    assert ev.phi1_policy == "retained"
    assert ev.readout_workspace_bytes == n * 8 + n * C * 4  # node energies (f64) + direct adjoint (f32)
    edges = ev.stats["num_edges"]
    assert ev.execution_active_edge_count == edges and ev.execution_active_receiver_count == n
    assert ev.execution_planned_receiver_capacity == n and ev.execution_planned_edge_capacity == edges
    assert ev.execution_planned_capacity_bytes == ev.low_memory_selected_estimated_bytes > 0
    assert ev.execution_planned_capacity_bytes == ev.low_memory_speed_estimated_bytes
    assert ev.dual_layer_workspace_batch_count == 0 and ev.dual_layer_workspace_bytes == 0
    assert not ev.low_memory
    assert ev.execution_geometry_workspace_bytes >= edges * 4 * 8  # xyz and r in f64
    assert ev.edge_geometry_policy == "cartesian-f64-v1" and ev.compact_edge_geometry_bytes == 0
    assert ev.harmonic_value_bytes == 0 and ev.harmonic_gradient_bytes == 0
    assert 0 < ev.low_memory_device_free_bytes <= ev.low_memory_device_total_bytes
    assert ev.factorized_fallback_evaluation_count == 0 and not ev.factorized_jit_ready
    assert ev.factorized_schedule_build_count == ev.factorized_prepared_graph_count == 1
    assert ev.execution_capacity_selection_reason == ev.execution_plan_report["selection_reason"]
    # a setter invalidates the prepared graph
    ev._set_allow_fixed_workspace(True)
    assert not ev.factorized_ready and ev.factorized_graph_generation == 0
    assert ev.low_memory_requested and ev.low_memory_policy == "pending"


def test_tiled_plan_properties(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=1)
    n = len(s)
    limit = 8
    ev = MACEKokkosFloat(path)
    ev._set_allow_fixed_workspace(True)
    ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    _prepare(ev, model, s)
    tiles = -(-n // limit)
    print(f"tiled: {tiles} tiles, arena {ev.dual_layer_workspace_bytes} B, "
          f"{ev.dual_layer_workspace_bytes_per_receiver} B/receiver, {ev.dual_layer_workspace_bytes_per_edge} B/edge, "
          f"{ev.dual_layer_source_segment_count} runs", flush=True)
    assert ev.factorized_tiled_ready and ev.low_memory and ev.low_memory_policy == "capacity"
    assert ev.dual_layer_workspace_batch_count == tiles
    assert ev.dual_layer_workspace_planned_receivers == ev.execution_planned_receiver_capacity == limit
    C = ev.num_channels
    assert ev.phi1_policy == "receiver-local"
    assert ev.phi1_workspace_bytes > 0 and ev.phi1_workspace_bytes % (limit * C * 4) == 0
    assert ev.phi1_workspace_bytes < n * C * 4 * (ev.phi1_workspace_bytes // (limit * C * 4))
    # the arena's edge capacity is the largest tile's edge count
    edges = ev.stats["num_edges"]
    assert 0 < ev.dual_layer_workspace_planned_edges < edges
    assert ev.execution_planned_edge_capacity == ev.dual_layer_workspace_planned_edges
    assert ev.dual_layer_workspace_bytes_per_receiver > 0 and ev.dual_layer_workspace_bytes_per_edge > 0
    assert ev.dual_layer_workspace_bytes >= (ev.dual_layer_workspace_bytes_per_receiver * limit
                                             + ev.dual_layer_workspace_bytes_per_edge
                                             * ev.dual_layer_workspace_planned_edges)
    # every (source, tile) pair of the graph is one run of 3 ints
    assert ev.dual_layer_source_segment_count >= n
    assert ev.dual_layer_schedule_bytes >= 12 * ev.dual_layer_source_segment_count
    assert ev.execution_planned_capacity_bytes == ev.low_memory_capacity_estimated_bytes > 0
