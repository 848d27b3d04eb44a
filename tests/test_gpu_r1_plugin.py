"""GPU: the ahead-of-time R1 HIP plugin of the reference's medium contract
(libsymmetrix_amd_r1_mpa0_medium.so, symmetrix_jit_hip_plugin_query_v1;
ABI symmetrix/source/symmetrix/jit_hip_plugin_abi.h) driven through ctypes
exactly as the reference's loader would: the descriptor's ABI fields and the
contract's fingerprints (tests/golden), then r1_forward_launch and
r1_coordinate_reverse_launch on packets filled from oracle arrays (the medium
shape's radial functions as cubic pieces, the oracle's harmonics and their
gradients, random features and adjoints) against the oracle's restatement of
the three owners.  FP32 plugin vs FP64 restatement: every output within 1e-5
of its largest magnitude.  A second test times the plugin's source- and
edge-owned reverse against this evaluator's message path on the headline
workload."""

import ctypes
import json
import os
import statistics

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PLUGIN = os.path.join(ROOT, "symmetrix-xl_amd", "symmetrix_amd", "libsymmetrix_amd_r1_mpa0_medium.so")

i32p = ctypes.c_void_p


class Radial(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("edge_types", ctypes.c_uint32), ("intervals", ctypes.c_uint32),
                ("functions", ctypes.c_uint32), ("h", ctypes.c_double), ("x0", ctypes.c_double),
                ("coefficients", ctypes.c_void_p)]


class Forward(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("active_type_count", ctypes.c_uint32),
                ("num_nodes", ctypes.c_int64), ("num_edges", ctypes.c_int64), ("node_types", i32p),
                ("num_neigh", i32p), ("first_neigh", i32p), ("neigh_indices", i32p), ("neigh_types", i32p),
                ("type_to_active", i32p), ("radius", ctypes.c_void_p), ("radial", Radial),
                ("harmonics_values", ctypes.c_void_p), ("neighbor_features", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("cutoff", ctypes.c_double)]


class Source(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("active_type_count", ctypes.c_uint32),
                ("num_nodes", ctypes.c_int64), ("num_edges", ctypes.c_int64), ("node_types", i32p),
                ("neigh_types", i32p), ("source_offsets", i32p), ("source_edges", i32p), ("edge_receivers", i32p),
                ("type_to_active", i32p), ("radius", ctypes.c_void_p), ("radial", Radial),
                ("harmonics_values", ctypes.c_void_p), ("output_adjoint", ctypes.c_void_p),
                ("source_adjoint", ctypes.c_void_p), ("cutoff", ctypes.c_double)]


class Edge(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("active_type_count", ctypes.c_uint32),
                ("coordinate_scalar_size", ctypes.c_uint32), ("coordinates_are_unit", ctypes.c_uint32),
                ("num_nodes", ctypes.c_int64), ("num_edges", ctypes.c_int64), ("node_types", i32p),
                ("neigh_indices", i32p), ("neigh_types", i32p), ("edge_receivers", i32p), ("type_to_active", i32p),
                ("xyz", ctypes.c_void_p), ("radius", ctypes.c_void_p), ("radial", Radial),
                ("harmonics_values", ctypes.c_void_p), ("harmonics_gradients", ctypes.c_void_p),
                ("neighbor_features", ctypes.c_void_p), ("output_adjoint", ctypes.c_void_p),
                ("directed_forces", ctypes.c_void_p), ("cutoff", ctypes.c_double)]


FORWARD_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.POINTER(Forward), ctypes.c_void_p, ctypes.c_int32)
REVERSE_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.POINTER(Source), ctypes.POINTER(Edge), ctypes.c_void_p,
                              ctypes.c_int32)


class Plugin(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("struct_size", ctypes.c_uint32), ("pointer_size", ctypes.c_uint32),
                ("byte_order", ctypes.c_uint32), ("capabilities", ctypes.c_uint32), ("scalar_kind", ctypes.c_uint32),
                ("scalar_size", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("abi_tag", ctypes.c_char_p),
                ("artifact_id", ctypes.c_char_p), ("contract_fingerprint", ctypes.c_char_p),
                ("semantic_fingerprint", ctypes.c_char_p), ("structure_fingerprint", ctypes.c_char_p),
                ("channels", ctypes.c_int32), ("embedding", ctypes.c_int32), ("edge_l_max", ctypes.c_int32),
                ("source_l_max", ctypes.c_int32), ("target_architecture", ctypes.c_char_p),
                ("target_features", ctypes.c_char_p), ("native_subgroup_width", ctypes.c_int32),
                ("forward_threads_per_block", ctypes.c_int32), ("source_threads_per_block", ctypes.c_int32),
                ("edge_threads_per_block", ctypes.c_int32), ("persistent_blocks_per_compute_unit", ctypes.c_int32),
                ("r1_forward_launch", FORWARD_FN), ("r1_coordinate_reverse_launch", REVERSE_FN)]


def _plugin():
    lib = ctypes.CDLL(PLUGIN)
    lib.symmetrix_jit_hip_plugin_query_v1.restype = ctypes.POINTER(Plugin)
    return lib, lib.symmetrix_jit_hip_plugin_query_v1().contents


def _contract():
    with open(os.path.join(HERE, "golden", "jit_r1_mace_mpa0_medium_contract.json")) as f:
        return json.load(f)


def test_descriptor_carries_the_contract(tmp_path):
    _, p = _plugin()
    c = _contract()
    assert p.abi_version == 1 and p.struct_size == ctypes.sizeof(Plugin) and p.pointer_size == 8
    assert p.byte_order == 0x01020304 and p.abi_tag == b"symmetrix.jit.hip-plugin/1"
    assert p.capabilities & 3 == 3 and p.scalar_kind == 1 and p.scalar_size == 4
    assert p.contract_fingerprint.decode() == c["generation_fingerprint"]
    assert p.semantic_fingerprint.decode() == c["fingerprint"]
    assert p.structure_fingerprint.decode() == c["structure_fingerprint"]
    assert (p.channels, p.embedding, p.edge_l_max, p.source_l_max) == (128, 64, 3, 1)
    assert p.target_architecture == b"gfx950" and p.native_subgroup_width == 64
    print(f"  artifact {p.artifact_id.decode()}, contract {p.contract_fingerprint.decode()}", flush=True)


def _packets(oracle_lib, hip, cells, seed):
    """Packets of the medium shape (3 active types, 6 edge types) on SrTiO3
    cells^3 at a 6.5 A list cutoff, with their host copies."""
    from symmetrix_amd import periodic_neighbor_graph, synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model("medium3", seed=seed)))
    s = synthetic.srtio3_supercell(cells, sigma=0.05, seed=seed)
    g = periodic_neighbor_graph(s.positions, s.cell, np.linalg.inv(s.cell), model["r_cut"] + 0.5)
    n = len(s)
    receivers = np.repeat(np.arange(n), g["num_neigh"]).astype(np.int32)
    sources = g["sources"].astype(np.int32)
    xyz = s.positions[sources] - s.positions[receivers] + g["shifts"].astype(np.float64) @ s.cell
    radius = np.linalg.norm(xyz, axis=1)
    types = synthetic.node_types(s, model["atomic_numbers"]).astype(np.int32)
    active = np.unique(types)
    type_to_active = np.full(model["num_elements"], -1, np.int32)
    type_to_active[active] = np.arange(len(active))
    na = len(active)
    grid_min, h, _ = oracle_lib.compact_radial_grid(model)
    pieces = []
    for a in range(na):
        for b in range(a, na):
            v, d = oracle_lib.compact_radial_tables(model, int(active[a]), int(active[b]), "R1")
            pieces.append(oracle_lib.hermite_pieces(v, d, h))
    pieces = np.stack(pieces).astype(np.float32)  # [6][intervals][4][1280]
    Y, dY = oracle_lib.harmonics(3, xyz)
    rng = np.random.default_rng(seed)
    H = rng.normal(size=(n, 4, 128)).astype(np.float32)
    A = rng.normal(size=(n, 40, 128)).astype(np.float32)
    order = np.argsort(sources, kind="stable").astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(np.bincount(sources, minlength=n))]).astype(np.int32)
    neigh_types = types[sources]
    host = dict(n=n, receivers=receivers, sources=sources, xyz=xyz, radius=radius, types=types,
                neigh_types=neigh_types, pieces=pieces, h=h, x0=grid_min, Y=Y.astype(np.float32),
                dY=dY.astype(np.float32), H=H, A=A, cutoff=float(model["r_cut"]), na=na,
                type_to_active=type_to_active, model=model, structure=s)
    radial = Radial(ctypes.sizeof(Radial), pieces.shape[0], pieces.shape[1], pieces.shape[3], h, grid_min,
                    hip.upload(pieces))
    d = {k: hip.upload(v) for k, v in dict(types=types, num_neigh=g["num_neigh"].astype(np.int32),
                                            first=g["receiver_offsets"][:-1].astype(np.int32), sources=sources,
                                            neigh_types=neigh_types, t2a=type_to_active, radius=radius,
                                            Y=host["Y"], dY=host["dY"], H=H, A=A, offsets=offsets, order=order,
                                            receivers=receivers, xyz=xyz).items()}
    n64, e64 = n, len(radius)
    fwd = Forward(ctypes.sizeof(Forward), na, n64, e64, d["types"], d["num_neigh"], d["first"], d["sources"],
                  d["neigh_types"], d["t2a"], d["radius"], radial, d["Y"], d["H"], hip.alloc(n * 40 * 128 * 4),
                  host["cutoff"])
    src = Source(ctypes.sizeof(Source), na, n64, e64, d["types"], d["neigh_types"], d["offsets"], d["order"],
                 d["receivers"], d["t2a"], d["radius"], radial, d["Y"], d["A"], 0, host["cutoff"])
    edge = Edge(ctypes.sizeof(Edge), na, 8, 0, n64, e64, d["types"], d["sources"], d["neigh_types"], d["receivers"],
                d["t2a"], d["xyz"], d["radius"], radial, d["Y"], d["dY"], d["H"], d["A"], 0, host["cutoff"])
    return host, fwd, src, edge


def _restated(oracle_lib, host):
    C = 128
    terms = oracle_lib.plugin_terms(_contract())
    a = host["type_to_active"][host["types"]]
    ra, sa = a[host["receivers"]], a[host["sources"]]
    lo, hi = np.minimum(ra, sa), np.maximum(ra, sa)
    edge_type = lo * (2 * host["na"] - lo - 1) // 2 + hi
    R, dR = oracle_lib.plugin_spline(host["pieces"], edge_type, host["radius"], host["x0"], host["h"])
    active = host["radius"] < host["cutoff"]
    Y, dY = host["Y"].astype(np.float64), host["dY"].astype(np.float64)
    H, A = host["H"].astype(np.float64), host["A"].astype(np.float64)
    out = oracle_lib.plugin_r1_forward(terms, C, host["n"], host["receivers"], host["sources"], active, R, Y, H, 40)
    sadj = oracle_lib.plugin_r1_source(terms, C, host["n"], 4, host["receivers"], host["sources"], active, R, Y, A)
    force = oracle_lib.plugin_r1_edge(terms, C, host["receivers"], host["sources"], active, host["xyz"],
                                      host["radius"], R, dR, Y, dY, H, A)
    return out, sadj, force


def _close(got, want, what):
    scale = float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"  {what}: max error {err:.3e} of max {scale:.3e}", flush=True)
    assert err <= 1e-5 * scale


@pytest.mark.parametrize("gradients", ["given", "formed from xyz"])
def test_plugin_matches_the_restated_operator(oracle_lib, gradients):
    from hip_memory import Hip

    lib, p = _plugin()
    hip = Hip()
    print(f"plugin on SrTiO3 3^3, medium contract, harmonic gradients {gradients}", flush=True)
    host, fwd, src, edge = _packets(oracle_lib, hip, 3, seed=5)
    n, E = host["n"], len(host["radius"])
    if gradients != "given":
        edge.harmonics_gradients = None
    rng = np.random.default_rng(9)
    s0 = rng.normal(size=(n, 4, 128)).astype(np.float32)
    f0 = rng.normal(size=(E, 3))
    src.source_adjoint = hip.upload(s0)
    edge.directed_forces = hip.upload(f0)
    assert p.r1_forward_launch(ctypes.byref(fwd), None, 1024) == 0
    assert p.r1_coordinate_reverse_launch(ctypes.byref(src), ctypes.byref(edge), None, 1024) == 0
    out = hip.download(fwd.output, (n, 40, 128), np.float32)
    sadj = hip.download(src.source_adjoint, (n, 4, 128), np.float32)
    force = hip.download(edge.directed_forces, (E, 3), np.float64)
    hip.free_all()
    want_out, want_sadj, want_force = _restated(oracle_lib, host)
    _close(out, want_out, "output")
    _close(sadj - s0, want_sadj, "source adjoint (accumulated)")
    _close(force - f0, want_force, "directed forces (accumulated)")
    # invalid packets are refused before any launch
    bad = Forward.from_buffer_copy(fwd)
    bad.struct_size = 8
    assert p.r1_forward_launch(ctypes.byref(bad), None, 1024) != 0
    assert p.r1_forward_launch(ctypes.byref(fwd), None, 0) != 0


def test_source_owned_reverse_against_the_message_path_at_the_headline_size(oracle_lib):
    """The plugin's reverse (source-owned feature adjoint + edge-owned forces,
    no per-edge messages) and this evaluator's reverse (r1_reverse writing
    per-edge messages + gather_messages) on SrTiO3 10^3 with the medium
    shape: device time per launch, median of 10 after 3 warmups."""
    from hip_memory import Hip
    from symmetrix_amd import MACEKokkosFloat, synthetic

    lib, p = _plugin()
    hip = Hip()
    host, fwd, src, edge = _packets(oracle_lib, hip, 10, seed=6)
    n, E = host["n"], len(host["radius"])
    src.source_adjoint = hip.alloc(n * 4 * 128 * 4)
    edge.directed_forces = hip.alloc(E * 3 * 8)
    hl = hip.lib
    hl.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hl.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hl.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hl.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    hl.hipEventCreate(ctypes.byref(ev0))
    hl.hipEventCreate(ctypes.byref(ev1))
    blocks = 256 * p.persistent_blocks_per_compute_unit

    def timed(launch):
        times = []
        for k in range(13):
            hl.hipEventRecord(ev0, None)
            assert launch() == 0
            hl.hipEventRecord(ev1, None)
            hl.hipEventSynchronize(ev1)
            ms = ctypes.c_float()
            hl.hipEventElapsedTime(ctypes.byref(ms), ev0, ev1)
            if k >= 3:
                times.append(ms.value)
        return statistics.median(times)

    plugin_fwd = timed(lambda: p.r1_forward_launch(ctypes.byref(fwd), None, blocks))
    plugin_rev = timed(lambda: p.r1_coordinate_reverse_launch(ctypes.byref(src), ctypes.byref(edge), None, blocks))
    hip.free_all()
    # this evaluator on the same structure and shape
    model, s = host["model"], host["structure"]
    path = os.path.join(os.environ.get("TMPDIR", "/tmp"), "medium3_plugin_ab.json")
    with open(path, "w") as f:
        json.dump(model, f)
    ev = MACEKokkosFloat(path)
    gen = ev._prepare_periodic_factorized_graph(host["types"], s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    for _ in range(3):
        ev._compute_prepared_factorized_positions(gen, s.positions)
    samples = []
    for _ in range(10):
        ev._set_profiling(True)
        ev._compute_prepared_factorized_positions(gen, s.positions)
        samples.append({k: ms / c if c else 0.0 for k, (ms, c) in ev._stage_times().items()})
    ev._set_profiling(False)
    st = {k: statistics.median(x[k] for x in samples) for k in samples[0]}
    own_rev = st["r1_reverse"] + st["h1_adjoint_gather"]
    print(f"  {n} atoms, {E} edges: plugin forward {plugin_fwd:.3f} ms, reverse (source + edge owners) "
          f"{plugin_rev:.3f} ms; this evaluator's r1_forward {st['r1_forward']:.3f} ms, r1_reverse "
          f"{st['r1_reverse']:.3f} + gather {st['h1_adjoint_gather']:.3f} = {own_rev:.3f} ms", flush=True)
    assert plugin_rev > 0 and own_rev > 0
