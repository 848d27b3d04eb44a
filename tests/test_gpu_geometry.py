"""Caller-built graphs evaluated from positions (the reference's
_prepare_factorized_geometry / _fractional_geometry / _shift_geometry and
_validate_graph_cardinality, symmetrix/source/cpp/mace_kokkos.cpp:1604-1669;
semantics mace_kokkos_factorized_lifecycle.cpp:2455-2780, 2915-3074).

A receiver-major CSR graph is prepared from the caller's lists; its geometry
is given as reference positions plus reference edge vectors (Cartesian or
fractional) or plus integer cell shifts.  An evaluation at new positions must
equal the evaluation of the same graph from explicit edge vectors formed on
the host (xyz = x[src] - x[recv] + shift . cell, r = |xyz|): energies and
directed forces to FP64 rounding of the edge vectors (the device forms them
from displacements, the host directly), far inside the north-star tolerances.
Each case also runs under the tiled plan (tiles of a few receivers, which
keeps no directed forces: energies and atom forces are compared), where the
geometry is formed per tile from the same reference arrays and explicit edge
vectors are copied into the tile arena per tile.
"""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("tiny") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _caller_graph(model, s, cutoff):
    """The caller's CSR (from the model-free device builder) and its arrays."""
    from symmetrix_amd import periodic_neighbor_graph, synthetic

    g = periodic_neighbor_graph(s.positions, s.cell, np.linalg.inv(s.cell), cutoff)
    types = synthetic.node_types(s, model["atomic_numbers"])
    return types, g


def _evaluator(path, limit):
    from symmetrix_amd import MACEKokkosFloat

    ev = MACEKokkosFloat(path)
    if limit:
        ev._set_allow_fixed_workspace(True)
        ev._set_dual_layer_workspace_receiver_limit_for_testing(limit)
    return ev


def _results(ev, gen):
    """Node energies and directed forces (untiled) or atom forces (tiled)."""
    if ev.stats["tile_receivers"] > 0:
        n = ev.stats["num_nodes"]
        return ev.node_energies.copy(), np.asarray(ev._reduce_atom_forces(n, None, None, gen)).copy()
    return ev.node_energies.copy(), ev.node_forces.copy()


def _explicit(ev, gen, types, g, positions, cell):
    receivers = np.repeat(np.arange(len(types)), g["num_neigh"])
    xyz = positions[g["sources"]] - positions[receivers] + g["shifts"].astype(np.float64) @ cell
    r = np.linalg.norm(xyz, axis=1)
    ev._compute_prepared_factorized(gen, xyz, r)
    return _results(ev, gen)


def _moved(s, seed, amount=0.08):
    rng = np.random.default_rng(seed)
    return s.positions + rng.normal(scale=amount, size=s.positions.shape)


def _close(a, b):
    (ea, fa), (eb, fb) = a, b
    np.testing.assert_allclose(ea, eb, atol=1e-9, rtol=0)
    np.testing.assert_allclose(fa, fb, atol=1e-8, rtol=0)


@pytest.mark.parametrize("limit", [None, 16])
@pytest.mark.parametrize("kind", ["cartesian", "fractional", "shifts"])
def test_caller_graph_geometry_equals_explicit_edge_vectors(tiny, kind, limit):
    from symmetrix_amd import synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=11)
    cutoff = model["r_cut"] + 0.5
    types, g = _caller_graph(model, s, cutoff)
    cell, inv = s.cell, np.linalg.inv(s.cell)
    ev = _evaluator(path, limit)
    ev._validate_graph_cardinality(len(types), len(types), len(g["sources"]))
    gen = ev._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]])
    pbc = np.ones(3, dtype=np.int32)
    receivers = np.repeat(np.arange(len(types)), g["num_neigh"])
    if kind == "cartesian":
        ref_xyz = s.positions[g["sources"]] - s.positions[receivers] + g["shifts"] @ cell
        ev._prepare_factorized_geometry(gen, s.positions, ref_xyz, cell, inv, pbc)
    elif kind == "fractional":
        ev._prepare_factorized_fractional_geometry(gen, s.positions @ inv, g["fractional_xyz"], cell, inv, pbc)
    else:
        ev._prepare_factorized_shift_geometry(gen, s.positions, g["shifts"], cell, inv, pbc)
    assert (ev.stats["tile_receivers"] > 0) == bool(limit)
    for seed in (1, 2):
        x = _moved(s, seed)
        print(f"{kind} geometry, SrTiO3 3^3, displacement seed {seed}, tile receivers {limit}", flush=True)
        ev._compute_prepared_factorized_positions(gen, x)
        got = _results(ev, gen)
        _close(got, _explicit(ev, gen, types, g, x, cell))
    # atoms moved by a lattice vector: the minimum-image displacement wraps
    x = _moved(s, 3)
    ev._compute_prepared_factorized_positions(gen, x)
    base = _results(ev, gen)
    x_wrapped = x.copy()
    x_wrapped[::7] += cell[0] - cell[2]
    ev._compute_prepared_factorized_positions(gen, x_wrapped)
    _close(_results(ev, gen), base)


@pytest.mark.parametrize("limit", [None, 16])
@pytest.mark.parametrize("kind", ["fractional", "shifts"])
def test_cell_update_follows_fractional_and_shift_geometry(tiny, kind, limit):
    from symmetrix_amd import synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=12)
    cutoff = model["r_cut"] + 0.5
    types, g = _caller_graph(model, s, cutoff)
    cell, inv = s.cell, np.linalg.inv(s.cell)
    ev = _evaluator(path, limit)
    gen = ev._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]])
    pbc = np.ones(3, dtype=np.int32)
    if kind == "fractional":
        ev._prepare_factorized_fractional_geometry(gen, s.positions @ inv, g["fractional_xyz"], cell, inv, pbc)
    else:
        ev._prepare_factorized_shift_geometry(gen, s.positions, g["shifts"], cell, inv, pbc)
    strain = np.eye(3) + np.array([[0.01, 0.004, 0.0], [0.004, -0.006, 0.002], [0.0, 0.002, 0.008]])
    new_cell = cell @ strain
    new_inv = np.linalg.inv(new_cell)
    ev._update_factorized_cell(gen, new_cell, new_inv)
    x = s.positions @ strain + np.random.default_rng(4).normal(scale=0.03, size=s.positions.shape)
    print(f"{kind} geometry after a cell update, tile receivers {limit}", flush=True)
    ev._compute_prepared_factorized_positions(gen, x)
    got = _results(ev, gen)
    _close(got, _explicit(ev, gen, types, g, x, new_cell))


@pytest.mark.parametrize("device_arrays", [False, True])
def test_tiled_neighbour_types_and_explicit_vectors_equal_untiled(tiny, device_arrays):
    """A caller graph whose neighbour types differ from its sources' (the pair
    codes are then kept graph-wide and read per tile), evaluated from
    explicit edge vectors (host or device arrays, copied into the tile arena
    per tile): the tiled plan equals the untiled one."""
    from hip_memory import Hip
    from symmetrix_amd import synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=15)
    types, g = _caller_graph(model, s, model["r_cut"] + 0.5)
    elements = np.unique(types)
    neigh_types = types[g["sources"]].copy()
    # every fifth neighbour is read as the next active element
    rank = np.searchsorted(elements, neigh_types[::5])
    neigh_types[::5] = elements[(rank + 1) % elements.size]
    receivers = np.repeat(np.arange(len(types)), g["num_neigh"])
    xyz = s.positions[g["sources"]] - s.positions[receivers] + g["shifts"].astype(np.float64) @ s.cell
    r = np.linalg.norm(xyz, axis=1)
    out = {}
    hip = Hip()
    for limit in (None, 16):
        ev = _evaluator(path, limit)
        gen = ev._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], neigh_types)
        assert (ev.stats["tile_receivers"] > 0) == bool(limit)
        print(f"explicit edge vectors ({'device' if device_arrays else 'host'} arrays), tile receivers {limit}",
              flush=True)
        if device_arrays:
            ev._compute_prepared_factorized_device(gen, hip.upload(xyz), hip.upload(r))
        else:
            ev._compute_prepared_factorized(gen, xyz, r)
        e = ev.node_energies.copy()
        f = np.asarray(ev._reduce_atom_forces(len(types), None, None, gen)).copy()
        out[limit] = (e, f)
    hip.free_all()
    # the tiled plan sums each source's H1-adjoint messages per tile (FP32, in
    # another order): atom forces agree to a few FP32 ulps of their size
    np.testing.assert_allclose(out[16][0], out[None][0], atol=1e-9, rtol=0)
    np.testing.assert_allclose(out[16][1], out[None][1], atol=1e-6, rtol=0)


def test_open_boundary_cluster_with_cartesian_geometry(tiny):
    # a cluster with no periodic axis: displacements are not wrapped
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=13)
    n = len(s)
    cutoff = model["r_cut"]
    d = s.positions[None, :, :] - s.positions[:, None, :]
    dist = np.linalg.norm(d, axis=2)
    adj = (dist < cutoff) & ~np.eye(n, dtype=bool)
    num_neigh = adj.sum(1).astype(np.int32)
    recv, src = np.nonzero(adj)
    types = synthetic.node_types(s, model["atomic_numbers"])
    ev = MACEKokkosFloat(path)
    gen = ev._prepare_factorized_graph(n, types, num_neigh, src.astype(np.int32), types[src])
    ref_xyz = s.positions[src] - s.positions[recv]
    ev._prepare_factorized_geometry(gen, s.positions, ref_xyz, np.zeros(9), np.zeros(9), np.zeros(3, np.int32))
    x = _moved(s, 5, amount=0.05) + np.array([40.0, -25.0, 7.0])  # translated far beyond any cell
    print("open-boundary cluster, Cartesian geometry", flush=True)
    ev._compute_prepared_factorized_positions(gen, x)
    got = (ev.node_energies.copy(), ev.node_forces.copy())
    xyz = x[src] - x[recv]
    ev._compute_prepared_factorized(gen, xyz, np.linalg.norm(xyz, axis=1))
    _close(got, (ev.node_energies.copy(), ev.node_forces.copy()))


def test_geometry_errors_follow_the_reference(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=14)
    types, g = _caller_graph(model, s, model["r_cut"] + 0.5)
    cell, inv = s.cell, np.linalg.inv(s.cell)
    n, e = len(types), len(g["sources"])
    ev = MACEKokkosFloat(path)
    gen = ev._prepare_factorized_graph(n, types, g["num_neigh"], g["sources"], types[g["sources"]])
    pbc = np.ones(3, dtype=np.int32)
    with pytest.raises(ValueError, match="geometry tokens"):
        ev._compute_prepared_factorized_positions(gen, s.positions)
    with pytest.raises(ValueError, match="current prepared graph token"):
        ev._prepare_factorized_geometry(gen + 1, s.positions, np.zeros((e, 3)), cell, inv, pbc)
    with pytest.raises(ValueError, match="extents are inconsistent"):
        ev._prepare_factorized_geometry(gen, s.positions, np.zeros((e - 1, 3)), cell, inv, pbc)
    bad = s.positions.copy()
    bad[0, 0] = np.nan
    with pytest.raises(ValueError, match="non-finite"):
        ev._prepare_factorized_geometry(gen, bad, np.zeros((e, 3)), cell, inv, pbc)
    with pytest.raises(ValueError, match="fully periodic"):
        ev._prepare_factorized_fractional_geometry(gen, s.positions @ inv, g["fractional_xyz"], cell, inv,
                                                   np.array([1, 1, 0], np.int32))
    with pytest.raises(ValueError, match="extents are inconsistent"):
        ev._prepare_factorized_shift_geometry(gen, s.positions[1:], g["shifts"], cell, inv, pbc)
    # Cartesian geometry cannot follow a new cell
    receivers = np.repeat(np.arange(n), g["num_neigh"])
    ref_xyz = s.positions[g["sources"]] - s.positions[receivers] + g["shifts"] @ cell
    ev._prepare_factorized_geometry(gen, s.positions, ref_xyz, cell, inv, pbc)
    with pytest.raises(ValueError, match="fractional or shift geometry"):
        ev._update_factorized_cell(gen, cell, inv)
    # a new graph drops the geometry of the old one
    gen2 = ev._prepare_factorized_graph(n, types, g["num_neigh"], g["sources"], types[g["sources"]])
    with pytest.raises(ValueError, match="geometry tokens"):
        ev._compute_prepared_factorized_positions(gen2, s.positions)


def test_graph_cardinality_limits(tiny):
    from symmetrix_amd import MACEKokkosFloat

    path, _ = tiny
    ev = MACEKokkosFloat(path)
    int_max = 2**31 - 1
    ev._validate_graph_cardinality(10, 10, int_max)
    with pytest.raises(OverflowError, match="atom count"):
        ev._validate_graph_cardinality(int_max, int_max, 10)
    with pytest.raises(OverflowError, match="feature-node count"):
        ev._validate_graph_cardinality(10, int_max, 10)
    with pytest.raises(ValueError, match="smaller than its receiver count"):
        ev._validate_graph_cardinality(10, 9, 10)
    with pytest.raises(OverflowError, match="directed-edge count"):
        ev._validate_graph_cardinality(10, 10, int_max + 1)
