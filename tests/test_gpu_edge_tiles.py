"""Edge-tile launches of the reverse edge kernels (the R1 reverse of the
single-pass shapes, the channel-sliced R1 reverse of the wide shape and the
A0 reverse): one workgroup per 16-, 32- or 64-edge
tile of a receiver instead of one per receiver, chosen for graphs of at most
ten receiver waves per compute unit (SXL_EDGE_TILE_LAUNCH=1 / 0 forces it,
SXL_EDGE_TILE the tile).  Neither kernel reduces over a receiver's edges:
each edge's force and message are sums over the channels alone, whichever
tile holds it, so node energies, directed forces, atom forces and stress
equal the one-workgroup-per-receiver launches bit for bit: on the medium
shape, with every model option (A0/A1 density terms, ZBL, Agnesi,
pre_linear_up, residual), on the unfolded layer-0 path, on the scalar shape,
on the wide shape (per-slice force parts) and with receivers of 0, 1, 15,
16, 17, 63, 64, 65 and 129 edges."""

import dataclasses
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _model(tmp_path, preset, **options):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS[preset], **options)
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=4))
    path = tmp_path / f"{preset}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _periodic(path, model, s):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    return ev, gen


def _results(ev, gen, n, volume):
    return (ev.node_energies.copy(), ev.node_forces.copy(), ev._reduce_atom_forces(n, None, None, gen),
            ev._reduce_stress(volume, None, gen))


def _assert_identical(a, b):
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("tile", [16, 64])
@pytest.mark.parametrize("case", ["medium3", "all_options", "unfolded", "scalar", "wide"])
def test_edge_tile_launch_equals_receiver_launch(tmp_path, monkeypatch, case, tile):
    from symmetrix_amd import synthetic

    if case == "all_options":
        path, model = _model(tmp_path, "medium3", zbl=True, density=("A0", "A1"), agnesi=True,
                             h1_basis="pre_linear_up", residual=True)
    elif case == "wide":
        # A1 density term: the channel-sliced reverse's slice 0 carries the
        # density-scale force of every edge
        path, model = _model(tmp_path, "wide", density=("A1",))
    else:
        path, model = _model(tmp_path, "scalar" if case == "scalar" else "medium3")
    if case == "unfolded":
        monkeypatch.setenv("SXL_A0_UNFOLDED", "1")
    monkeypatch.setenv("SXL_EDGE_TILE_LAUNCH", "1")
    monkeypatch.setenv("SXL_EDGE_TILE", str(tile))
    s = synthetic.water_box(num_molecules=45, seed=7) if case == "wide" else \
        synthetic.srtio3_supercell(3, sigma=0.05, seed=7)
    n = len(s)
    ev, gen = _periodic(path, model, s)
    tiles = ev.stats["num_edges"]  # edges > 64 per receiver at this cutoff: several tiles each
    tiled = _results(ev, gen, n, s.volume)
    monkeypatch.setenv("SXL_EDGE_TILE_LAUNCH", "0")
    ev0, gen0 = _periodic(path, model, s)
    whole = _results(ev0, gen0, n, s.volume)
    print(f"{case}, {tile}-edge tiles: {n} atoms, {tiles} edges; max |dF| {np.max(np.abs(tiled[2] - whole[2])):.1e}",
          flush=True)
    _assert_identical(tiled, whole)


@pytest.mark.parametrize("tile", [16, 32, 64])
def test_edge_tiles_at_tile_boundaries(tmp_path, monkeypatch, tile):
    """A caller graph whose receivers have 0, 1, 15, 16, 17, 63, 64, 65 and
    129 edges."""
    from symmetrix_amd import MACEKokkosFloat

    path, model = _model(tmp_path, "medium3")
    rng = np.random.default_rng(3)
    degrees = [0, 1, 63, 64, 65, 129, 5, 0, 64, 15, 16, 17, 32, 33]
    n = 140
    num_neigh = np.zeros(n, dtype=np.int32)
    num_neigh[:len(degrees)] = degrees
    num_neigh[len(degrees):] = rng.integers(0, 4, n - len(degrees))
    sources = np.concatenate([rng.choice(np.delete(np.arange(n), i), d, replace=d > n - 1)
                              for i, d in enumerate(num_neigh)]).astype(np.int32)
    node_types = rng.integers(0, min(3, model["num_elements"]), n).astype(np.int32)
    xyz = rng.normal(scale=1.8, size=(len(sources), 3))
    r = np.linalg.norm(xyz, axis=1)

    monkeypatch.setenv("SXL_EDGE_TILE_LAUNCH", "1")
    monkeypatch.setenv("SXL_EDGE_TILE", str(tile))

    def run():
        ev = MACEKokkosFloat(path)
        gen = ev._prepare_factorized_graph(n, node_types, num_neigh, sources, node_types[sources])
        ev._compute_prepared_factorized(gen, xyz, r)
        return ev.node_energies.copy(), ev.node_forces.copy()

    tiled = run()
    monkeypatch.setenv("SXL_EDGE_TILE_LAUNCH", "0")
    whole = run()
    print(f"caller graph, {tile}-edge tiles: {n} receivers, {len(sources)} edges", flush=True)
    _assert_identical(tiled, whole)
