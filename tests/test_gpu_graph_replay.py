"""HIP graph replay of evaluations from positions (sxl_set_graph_replay):
every replay equals an eager evaluation of the same positions bit for bit.
The replays run with eager work between them on the same evaluator (an
evaluation from explicit edge vectors and a displacement query), with new
positions in the same array, after a cell update (a new capture), on host
and on device positions, with all model options, and report the kernels
they ran in the launch count."""

import dataclasses
import json
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(__file__))
from hip_memory import Hip  # noqa: E402

pytestmark = pytest.mark.gpu


def _model(tmp_path, **options):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["medium3"], **options)
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=5))
    path = tmp_path / "m.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _prepared(path, model, s, replay):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    ev = MACEKokkosFloat(path)
    if replay:
        ev._set_graph_replay(True)
        assert ev.graph_replay
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    return ev, gen


def _results(ev, gen, n, volume):
    return (ev.node_energies.copy(), ev._reduce_atom_forces(n, None, None, gen),
            ev._reduce_stress(volume, None, gen), ev._total_energy(gen))


def _same(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(np.asarray(x), np.asarray(y))


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("options", ["plain", "all"])
def test_replays_equal_eager_evaluations(tmp_path, device, options):
    from symmetrix_amd import synthetic

    extra = {} if options == "plain" else dict(zbl=True, density=("A0", "A1"), agnesi=True,
                                                h1_basis="pre_linear_up", residual=True)
    path, model = _model(tmp_path, **extra)
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=9)
    n = len(s)
    replay, gen = _prepared(path, model, s, True)
    eager, gen_e = _prepared(path, model, s, False)
    hip = Hip()
    d_pos = hip.alloc(n * 3 * 8)
    rng = np.random.default_rng(1)
    try:
        cell = s.cell.copy()
        for step in range(6):
            pos = s.positions + rng.normal(scale=0.04, size=(n, 3))
            if step == 4:
                # a cell update: the replay is captured again for the new volume
                cell = cell * 1.01
                pos = pos * 1.01
                for ev, g in ((replay, gen), (eager, gen_e)):
                    ev._update_factorized_cell(g, cell, np.linalg.inv(cell))
            if device:
                hip.lib.hipMemcpy(d_pos, np.ascontiguousarray(pos).ctypes.data, n * 3 * 8, 1)
                replay._compute_prepared_factorized_positions_device(gen, d_pos)
                eager._compute_prepared_factorized_positions_device(gen_e, d_pos)
            else:
                replay._compute_prepared_factorized_positions(gen, pos)
                eager._compute_prepared_factorized_positions(gen_e, pos)
            volume = abs(np.linalg.det(cell))
            got, want = _results(replay, gen, n, volume), _results(eager, gen_e, n, volume)
            print(f"{options}, {'device' if device else 'host'} positions, replay {step}: "
                  f"E {got[3]:.9f}, launches {replay.last_evaluation_launch_count} / "
                  f"{eager.last_evaluation_launch_count}", flush=True)
            _same(got, want)
            assert replay.last_evaluation_launch_count == eager.last_evaluation_launch_count
            assert replay._last_max_displacement() == eager._last_max_displacement()
            # eager work on the replaying evaluator between its replays
            g = replay._periodic_graph_arrays(gen)
            receivers = np.repeat(np.arange(n), g["num_neigh"])
            xyz = pos[g["sources"]] - pos[receivers] + g["shifts"].astype(np.float64) @ cell
            r = np.linalg.norm(xyz, axis=1)
            replay._compute_prepared_factorized(gen, xyz, r)
            replay._max_displacement(gen, pos)
    finally:
        hip.free_all()


def test_replay_is_off_by_default_and_follows_new_graphs(tmp_path):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = _model(tmp_path)
    assert not MACEKokkosFloat(path).graph_replay
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=2)
    replay, gen = _prepared(path, model, s, True)
    eager, gen_e = _prepared(path, model, s, False)
    for ev, g in ((replay, gen), (eager, gen_e)):
        ev._compute_prepared_factorized_positions(g, s.positions)
    _same(_results(replay, gen, len(s), s.volume), _results(eager, gen_e, len(s), s.volume))
    # a new graph (another structure) on the same evaluator captures again
    s2 = synthetic.srtio3_supercell(3, sigma=0.05, seed=3)
    types = synthetic.node_types(s2, model["atomic_numbers"])
    for i, ev in enumerate((replay, eager)):
        g = ev._prepare_periodic_factorized_graph(types, s2.positions, s2.cell, np.linalg.inv(s2.cell),
                                                  model["r_cut"] + 0.5)["generation"]
        ev._compute_prepared_factorized_positions(g, s2.positions)
        if i == 0:
            gen2 = g
        else:
            gen2_e = g
    _same(_results(replay, gen2, len(s2), s2.volume), _results(eager, gen2_e, len(s2), s2.volume))
    replay._set_graph_replay(False)
    assert not replay.graph_replay
