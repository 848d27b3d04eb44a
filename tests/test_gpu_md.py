"""GPU: the device velocity-Verlet NVE driver (sxl_md_nve).

- Against a host velocity-Verlet loop written here over the same evaluator's
  forces (graph built at r_cut + skin, rebuilt past skin/2): the device
  integrator evaluates the same expressions with FP contraction off, so the
  trajectories are identical bit for bit.
- Energy conservation of a 20-step run at 1 fs (the capacity configuration's
  protocol) and argument validation.
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MASSES = {38: 87.62, 22: 47.867, 8: 15.999}
ACC = 9.648533212e-3  # 1 eV/(A amu) in A/fs^2
KB = 8.617333262e-5


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("md") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _system(n, seed, temperature=300.0):
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(n, sigma=0.05, seed=seed)
    m = np.array([MASSES[int(z)] for z in s.numbers])
    rng = np.random.default_rng(seed + 1)
    v = rng.normal(size=(len(s), 3)) * np.sqrt(KB * temperature * ACC / m)[:, None]
    v -= (m[:, None] * v).sum(0) / m.sum()
    return s, m, v


@pytest.mark.parametrize("tile_receivers", [None, 40])
def test_device_md_matches_host_velocity_verlet(tiny, tile_receivers):
    """Untiled, and under the tiled plan (tiles of 40 receivers): the device
    driver evaluates on the current graph, then reads the displacement that
    evaluation measured and rebuilds and evaluates again past skin/2, which
    gives the host loop's trajectory (check first, then evaluate)."""
    from symmetrix_amd import MACEKokkosFloat, synthetic

    def evaluator():
        ev = MACEKokkosFloat(path)
        if tile_receivers:
            ev._set_allow_fixed_workspace(True)
            ev._set_dual_layer_workspace_receiver_limit_for_testing(tile_receivers)
        return ev

    path, model = tiny
    s, m, v0 = _system(3, seed=21, temperature=600.0)
    types = synthetic.node_types(s, model["atomic_numbers"])
    skin, dt, steps = 0.1, 2.0, 12   # small skin: the run rebuilds its graph
    print(f"device MD vs host loop: {len(s)} atoms, {steps} steps, tile receivers {tile_receivers}", flush=True)
    dev = evaluator()._md_nve(types, m, s.positions, v0, s.cell, skin, dt, steps)

    ev = evaluator()
    inv_cell = np.linalg.inv(s.cell)
    cutoff = model["r_cut"] + skin
    x, v = s.positions.copy(), v0.copy()
    inv_m = (ACC / m)[:, None]
    gen = ev._prepare_periodic_factorized_graph(types, x, s.cell, inv_cell, cutoff)["generation"]
    ev._compute_prepared_factorized_positions(gen, x)
    f = ev._reduce_atom_forces(len(s), None, None, gen)
    epot = [ev._total_energy(gen)]
    rebuilds = 0
    dtf = 0.5 * dt
    for _ in range(steps):
        v = v + dtf * f * inv_m
        x = x + dt * v
        if not ev._max_displacement(gen, x) <= 0.5 * skin:
            gen = ev._prepare_periodic_factorized_graph(types, x, s.cell, inv_cell, cutoff)["generation"]
            rebuilds += 1
        ev._compute_prepared_factorized_positions(gen, x)
        f = ev._reduce_atom_forces(len(s), None, None, gen)
        v = v + dtf * f * inv_m
        epot.append(ev._total_energy(gen))
    if tile_receivers:
        assert ev.stats["tile_receivers"] == tile_receivers
    print(f"  rebuilds device {dev['rebuilds']} host {rebuilds}", flush=True)
    assert rebuilds >= 1 and dev["rebuilds"] == rebuilds
    np.testing.assert_array_equal(dev["positions"], x)
    np.testing.assert_array_equal(dev["velocities"], v)
    np.testing.assert_array_equal(dev["potential_energy"], epot)
    ekin = 0.5 * (m[:, None] * v * v).sum() / ACC
    assert dev["kinetic_energy"][-1] == pytest.approx(ekin, rel=1e-12)


def test_nve_energy_is_conserved(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s, m, v0 = _system(4, seed=22)
    types = synthetic.node_types(s, model["atomic_numbers"])
    res = MACEKokkosFloat(path)._md_nve(types, m, s.positions, v0, s.cell, 0.5, 1.0, 20)
    etot = res["potential_energy"] + res["kinetic_energy"]
    drift = float(np.max(np.abs(etot - etot[0]))) / len(s)
    swing = float(np.max(np.abs(res["potential_energy"] - res["potential_energy"][0]))) / len(s)
    print(f"  {len(s)} atoms: max |dE_tot|/atom = {drift:.2e} eV (|dE_pot|/atom up to {swing:.2e})", flush=True)
    assert np.all(np.isfinite(etot))
    assert drift < 0.05 * swing + 1e-6


def test_md_argument_validation(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s, m, v0 = _system(2, seed=23)
    types = synthetic.node_types(s, model["atomic_numbers"])
    ev = MACEKokkosFloat(path)
    with pytest.raises(ValueError, match="time step"):
        ev._md_nve(types, m, s.positions, v0, s.cell, 0.5, 0.0, 3)
    bad = m.copy()
    bad[3] = -1.0
    with pytest.raises(ValueError, match="masses"):
        ev._md_nve(types, bad, s.positions, v0, s.cell, 0.5, 1.0, 3)
    with pytest.raises(ValueError, match="step count"):
        ev._md_nve(types, m, s.positions, v0, s.cell, 0.5, 1.0, -1)


def test_md_progress_reports_every_step_and_can_stop_the_run(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s, m, v0 = _system(2, seed=24)
    types = synthetic.node_types(s, model["atomic_numbers"])
    full = MACEKokkosFloat(path)._md_nve(types, m, s.positions, v0, s.cell, 0.5, 1.0, 6)
    seen = []

    def progress(step, epot, ekin, seconds):
        seen.append((step, epot, ekin, seconds))
        return step == 4  # stop after the fourth step

    print("MD with a progress callback stopping after step 4 of 6", flush=True)
    ev = MACEKokkosFloat(path)
    part = ev._md_nve(types, m, s.positions, v0, s.cell, 0.5, 1.0, 6, progress=progress)
    assert [q[0] for q in seen] == [1, 2, 3, 4]
    for step, epot, ekin, seconds in seen:
        assert epot == full["potential_energy"][step] and ekin == full["kinetic_energy"][step]
        assert seconds > 0.0
    np.testing.assert_array_equal(part["potential_energy"][:5], full["potential_energy"][:5])
    assert np.all(part["potential_energy"][5:] == 0.0)
    # the callback is removed after the run: a plain run on the same evaluator works
    again = ev._md_nve(types, m, s.positions, v0, s.cell, 0.5, 1.0, 2)
    np.testing.assert_array_equal(again["potential_energy"], full["potential_energy"][:3])
