"""Observability counters (reference factorized_prepared_graph_count,
factorized_prepared_evaluation_count, factorized_preparation_fence_count,
factorized_evaluation_fence_count, mace_kokkos.cpp:925-970; the reference's
repeat-evaluation test test_mace_streamed_edges.py:3700-3740 checks that
repeated evaluations of one prepared graph change no workspace and wait on
the device once each).

Here: a prepared graph evaluated again from positions allocates nothing,
issues the same number of kernel launches every time, waits on the host
exactly once (the result copy) and returns bitwise identical results (the
evaluation is deterministic), for the untiled and the tiled plan alike.
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("obs") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _prepared(tiny, tiled):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(4, sigma=0.05, seed=21)
    ev = MACEKokkosFloat(path)
    if tiled:
        ev._set_allow_fixed_workspace(True)
        ev._set_dual_layer_workspace_receiver_limit_for_testing(100)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"])
    return ev, gen["generation"], s


@pytest.mark.parametrize("tiled", [False, True], ids=["untiled", "tiled"])
def test_repeat_evaluations_allocate_nothing_and_fence_once(tiny, tiled):
    ev, gen, s = _prepared(tiny, tiled)
    st = ev.stats
    assert ev.factorized_prepared_graph_count == 1
    assert ev.factorized_prepared_evaluation_count == 0
    # waits: the previous graph's work, the edge counts read back (with the
    # runs per tile), the prepared graph; the tiled plan also waits before
    # dropping graph-wide per-edge arrays and checks its tile lists
    assert ev.factorized_preparation_fence_count == (5 if tiled else 3), ev.factorized_preparation_fence_count
    assert ev.factorized_evaluation_fence_count == 0
    assert ev.factorized_last_graph_prepare_ms > 0.0
    assert (st["tile_receivers"] > 0) == tiled
    print(f"{'tiled' if tiled else 'untiled'}: preparation fences {ev.factorized_preparation_fence_count}",
          flush=True)

    x = s.positions + np.random.default_rng(3).normal(scale=0.02, size=s.positions.shape)
    ev._compute_prepared_factorized_positions(gen, x)  # first evaluation may size buffers
    first = (ev.node_energies.copy(), ev._reduce_atom_forces(len(s)).copy())
    launches = ev.last_evaluation_launch_count
    assert launches > 0
    fences0 = ev.factorized_evaluation_fence_count
    prep_fences = ev.factorized_preparation_fence_count
    for k in range(3):
        ev._compute_prepared_factorized_positions(gen, x)
        st = ev.stats
        print(f"repeat {k}: launches {st['last_evaluation_launches']} allocations "
              f"{st['last_evaluation_allocations']} fences {st['last_evaluation_fences']} "
              f"{st['last_evaluation_ms']:.3f} ms", flush=True)
        assert st["last_evaluation_allocations"] == 0
        assert st["last_evaluation_launches"] == launches
        assert st["last_evaluation_fences"] == 1
        np.testing.assert_array_equal(ev.node_energies, first[0])
        np.testing.assert_array_equal(ev._reduce_atom_forces(len(s)), first[1])
    assert ev.factorized_evaluation_fence_count - fences0 == 3
    assert ev.factorized_prepared_evaluation_count == 4
    assert ev.factorized_preparation_fence_count == prep_fences
    assert ev.factorized_prepared_graph_count == 1
    if tiled:
        assert ev.dual_layer_tiled_evaluation_count == 4


def test_preparation_counts_are_reproducible(tiny):
    # the same graph prepared again costs the same host waits; a caller's
    # CSR graph waits twice (the previous graph's work, the prepared graph)
    from symmetrix_amd import periodic_neighbor_graph, synthetic

    ev, gen, s = _prepared(tiny, False)
    first = ev.factorized_preparation_fence_count
    types = synthetic.node_types(s, tiny[1]["atomic_numbers"])
    gen2 = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                 tiny[1]["r_cut"])["generation"]
    assert gen2 != gen
    assert ev.factorized_prepared_graph_count == 2
    assert ev.factorized_preparation_fence_count == 2 * first
    g = periodic_neighbor_graph(s.positions, s.cell, np.linalg.inv(s.cell), tiny[1]["r_cut"])
    ev._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]])
    assert ev.factorized_prepared_graph_count == 3
    assert ev.factorized_preparation_fence_count == 2 * first + 2


def test_live_evaluators_block_finalization(tiny):
    # the reference counts live evaluators and refuses to finalize while any
    # is alive (tools_kokkos.cpp:57-66); the runtime is not finalized here
    import symmetrix_amd as s
    from symmetrix_amd import MACEKokkosFloat

    base = s._kokkos_live_object_count()
    ev = MACEKokkosFloat(tiny[0])
    assert s._kokkos_is_initialized()
    assert s._kokkos_live_object_count() == base + 1
    with pytest.raises(RuntimeError, match=r"Cannot finalize Kokkos while \d+ Symmetrix evaluator"):
        s._finalize_kokkos()
    ev.close()
    assert s._kokkos_live_object_count() == base
    assert s._kokkos_is_initialized()
