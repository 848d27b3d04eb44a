"""The allocation-free neighbour-graph entry point
(sxl_neighbor_graph_build_noalloc, include/symmetrix_amd.h) against the
allocating one (sxl_neighbor_graph_build) through the C ABI: positions and
outputs in device memory the test owns, two calls in a row (the second on a
smaller system, after the first has left its data in the library's scratch
array), each bit-identical to the allocating builder; the capacity, atom-limit
and empty-input paths.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SXL_LENGTH_ERROR = 3


class Hip:
    """Device memory for the caller's side of the ABI (plumbing)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.lib.hipFree.argtypes = [ctypes.c_void_p]
        self.lib.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipStreamDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipDeviceSynchronize.argtypes = []
        self.held = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)) == 0
        self.held.append(p.value)
        return p.value

    def upload(self, array):
        a = np.ascontiguousarray(array)
        p = self.alloc(a.nbytes)
        if a.nbytes:
            assert self.lib.hipMemcpy(ctypes.c_void_p(p), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1) == 0
        return p

    def download(self, ptr, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            assert self.lib.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), out.nbytes, 2) == 0
        return out

    def free_all(self):
        assert self.lib.hipDeviceSynchronize() == 0
        for p in self.held:
            self.lib.hipFree(ctypes.c_void_p(p))
        self.held = []


@pytest.fixture
def hip():
    h = Hip()
    yield h
    h.free_all()


def _c(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _allocating(positions, cell, cutoff):
    from symmetrix_amd import periodic_neighbor_graph

    return periodic_neighbor_graph(positions, cell, np.linalg.inv(cell), cutoff)


def _noalloc(hip, positions, cell, cutoff, capacity, stream=None, sentinel=False):
    from symmetrix_amd import _native

    lib = _native.library()
    pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
    n = pos.shape[0]
    c = np.ascontiguousarray(cell, dtype=np.float64).reshape(-1)
    ic = np.ascontiguousarray(np.linalg.inv(cell), dtype=np.float64).reshape(-1)
    d_pos = hip.upload(pos)
    if sentinel:
        d_off = hip.upload(np.full(n + 1, -7, np.int32))
        d_src = hip.upload(np.full(max(capacity, 1), -7, np.int32))
    else:
        d_off = hip.alloc((n + 1) * 4)
        d_src = hip.alloc(max(capacity, 1) * 4)
    d_sh = hip.alloc(max(capacity, 1) * 12)
    d_fr = hip.alloc(max(capacity, 1) * 24)
    ne = ctypes.c_int64(-1)
    status = lib.sxl_neighbor_graph_build_noalloc(
        ctypes.c_void_p(d_pos), n, _c(c, ctypes.c_double), _c(ic, ctypes.c_double), float(cutoff),
        int(capacity), ctypes.c_void_p(d_off), ctypes.c_void_p(d_src), ctypes.c_void_p(d_sh),
        ctypes.c_void_p(d_fr), ctypes.byref(ne), ctypes.c_void_p(stream))
    e = int(ne.value)
    out = {"status": status, "num_edges": e, "message": lib.sxl_last_error().decode()}
    if status == 0:
        out["receiver_offsets"] = hip.download(d_off, n + 1, np.int32)
        out["sources"] = hip.download(d_src, e, np.int32)
        out["shifts"] = hip.download(d_sh, (e, 3), np.int32)
        out["fractional_xyz"] = hip.download(d_fr, (e, 3), np.float64)
    elif sentinel:
        out["receiver_offsets"] = hip.download(d_off, n + 1, np.int32)
        out["sources"] = hip.download(d_src, max(capacity, 1), np.int32)
    return out


def _triclinic_box(n, seed):
    rng = np.random.default_rng(seed)
    cell = np.array([[14.0, 0.0, 0.0], [2.5, 13.0, 0.0], [-1.5, 2.0, 15.0]])
    frac = rng.uniform(size=(n, 3))
    return frac @ cell + rng.normal(scale=0.01, size=(n, 3)), cell


def _assert_same(got, want):
    assert got["status"] == 0, got["message"]
    assert got["num_edges"] == len(want["sources"])
    np.testing.assert_array_equal(got["receiver_offsets"], want["receiver_offsets"])
    np.testing.assert_array_equal(got["sources"], want["sources"])
    np.testing.assert_array_equal(got["shifts"], want["shifts"])
    # bit-identical doubles
    np.testing.assert_array_equal(got["fractional_xyz"].view(np.uint64), want["fractional_xyz"].view(np.uint64))


def test_noalloc_graph_equals_allocating_builder_on_two_calls(hip):
    from symmetrix_amd import synthetic

    # first call: 600 atoms in a triclinic cell
    pos1, cell1 = _triclinic_box(600, seed=1)
    want1 = _allocating(pos1, cell1, 5.5)
    print(f"call 1: {len(pos1)} atoms, {len(want1['sources'])} edges", flush=True)
    got1 = _noalloc(hip, pos1, cell1, 5.5, capacity=len(want1["sources"]) + 17)
    _assert_same(got1, want1)
    # second call, smaller: SrTiO3 2^3 (40 atoms, many periodic images), on a stream
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=2)
    want2 = _allocating(s.positions, s.cell, 6.5)
    stream = ctypes.c_void_p()
    assert hip.lib.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        print(f"call 2: {len(s)} atoms, {len(want2['sources'])} edges", flush=True)
        got2 = _noalloc(hip, s.positions, s.cell, 6.5, capacity=len(want2["sources"]), stream=stream.value)
    finally:
        hip.lib.hipStreamDestroy(stream)
    _assert_same(got2, want2)


def test_noalloc_graph_reports_the_needed_capacity(hip):
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=3)
    want = _allocating(s.positions, s.cell, 5.0)
    e = len(want["sources"])
    got = _noalloc(hip, s.positions, s.cell, 5.0, capacity=e - 1, sentinel=True)
    assert got["status"] == SXL_LENGTH_ERROR
    assert got["num_edges"] == e
    assert "capacity" in got["message"]
    # no output written
    assert np.all(got["receiver_offsets"] == -7) and np.all(got["sources"] == -7)
    # the same arrays with enough room
    _assert_same(_noalloc(hip, s.positions, s.cell, 5.0, capacity=e), want)


def test_noalloc_graph_limits_and_empty_input(hip):
    from symmetrix_amd import _native

    max_atoms, max_bins = ctypes.c_int(), ctypes.c_int()
    nbytes = _native.library().sxl_neighbor_graph_noalloc_limits(ctypes.byref(max_atoms), ctypes.byref(max_bins))
    assert (max_atoms.value, max_bins.value, nbytes) == (131072, 262144, 18353408)
    # one atom more than the limit: refused before any device work
    n = max_atoms.value + 1
    rng = np.random.default_rng(4)
    cell = np.eye(3) * 200.0
    got = _noalloc(hip, rng.uniform(0, 200.0, size=(n, 3)), cell, 5.0, capacity=16)
    assert got["status"] == SXL_LENGTH_ERROR and "at most" in got["message"]
    # a cell with more bins than the limit
    got = _noalloc(hip, rng.uniform(0, 400.0, size=(8, 3)), np.eye(3) * 400.0, 0.5, capacity=16)
    assert got["status"] == SXL_LENGTH_ERROR and "cell bins" in got["message"]
    # no atoms: no edges, receiver_offsets = [0]
    got = _noalloc(hip, np.zeros((0, 3)), np.eye(3) * 10.0, 5.0, capacity=0)
    assert got["status"] == 0 and got["num_edges"] == 0
    np.testing.assert_array_equal(got["receiver_offsets"], [0])
