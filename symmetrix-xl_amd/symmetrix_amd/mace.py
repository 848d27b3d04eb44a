"""Python face of the evaluator, mirroring the reference's native class.

``MACEKokkosFloat`` keeps the method names, argument meaning and result
layout of the reference's pybind11 class of the same name
(``symmetrix/source/cpp/mace_kokkos.cpp:1561-1840, 2086-2203, 2762``) for the
model-evaluation path, so callers written against the reference run
unchanged.  All work runs in ``libsymmetrix_amd.so`` on the GPU; nothing here
computes model quantities.
"""

from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _native
from ._native import c_double_p, c_i64, c_int_p, c_u64, check, library

# sxl_md_progress_fn: int (int step, double epot, double ekin, double seconds, void* user)
_PROGRESS_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                ctypes.c_void_p)


def _i32(a, n=None, name="array"):
    a = np.ascontiguousarray(a, dtype=np.int32).reshape(-1)
    if n is not None and a.size != n:
        raise ValueError(f"{name} must hold {n} values, got {a.size}")
    return a


def _f64(a, n=None, name="array"):
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    if n is not None and a.size != n:
        raise ValueError(f"{name} must hold {n} values, got {a.size}")
    return a


def _p(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


class MACEKokkosFloat:
    """FP32 MACE evaluator on one MI355X (reference class ``MACEKokkosFloat``)."""

    streamed_edges_mode = "direct"

    def __init__(self, filename, head: str = ""):
        lib = library()
        handle = ctypes.c_void_p()
        check(lib.sxl_create(str(filename).encode(), (head or "").encode(), ctypes.byref(handle)))
        self._h = handle
        info = _native.ModelInfo()
        check(lib.sxl_model_info(self._h, ctypes.byref(info)))
        self._info = info
        z = np.zeros(info.num_elements, dtype=np.int32)
        check(lib.sxl_atomic_numbers(self._h, _p(z, ctypes.c_int)))
        e0 = np.zeros(info.num_elements, dtype=np.float64)
        check(lib.sxl_atomic_energies(self._h, _p(e0, ctypes.c_double)))
        self._atomic_numbers = [int(v) for v in z]
        self._atomic_energies = [float(v) for v in e0]
        self._generation = 0
        self._evaluated = False

    def close(self):
        if getattr(self, "_h", None):
            library().sxl_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- model metadata ----------------------------------------------------
    @property
    def atomic_numbers(self):
        return list(self._atomic_numbers)

    @property
    def atomic_energies(self):
        return list(self._atomic_energies)

    @property
    def r_cut(self):
        return self._info.r_cut

    @property
    def l_max(self):
        return self._info.l_max

    @property
    def L_max(self):
        return self._info.L_max

    @property
    def num_channels(self):
        return self._info.num_channels

    @property
    def num_elements(self):
        return self._info.num_elements

    # ---- graphs --------------------------------------------------------------
    def _prepare_factorized_graph(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types):
        types = _i32(node_types, num_nodes, "node_types")
        nn = _i32(num_neigh, num_nodes, "num_neigh")
        e = int(nn.sum())
        idx = _i32(neigh_indices, e, "neigh_indices")
        nt = _i32(neigh_types, e, "neigh_types")
        gen = c_u64(0)
        check(library().sxl_prepare_graph(self._h, int(num_nodes), _p(types, ctypes.c_int),
                                          _p(nn, ctypes.c_int), _p(idx, ctypes.c_int),
                                          _p(nt, ctypes.c_int), ctypes.byref(gen)))
        self._generation = int(gen.value)
        self._evaluated = False
        return self._generation

    def _prepare_factorized_graph_device(self, num_nodes, node_types_ptr, num_neigh_ptr, neigh_indices_ptr,
                                         neigh_types_ptr):
        """_prepare_factorized_graph with the four arrays in device memory
        (pointers; reference prepare_factorized_graph_device)."""
        gen = c_u64(0)
        check(library().sxl_prepare_graph_device(self._h, int(num_nodes), ctypes.c_void_p(int(node_types_ptr)),
                                                 ctypes.c_void_p(int(num_neigh_ptr)),
                                                 ctypes.c_void_p(int(neigh_indices_ptr)),
                                                 ctypes.c_void_p(int(neigh_types_ptr)), ctypes.byref(gen)))
        self._generation = int(gen.value)
        self._evaluated = False
        return self._generation

    def _prepare_periodic_factorized_graph(self, node_types, positions, cell, inverse_cell, neighbor_cutoff):
        types = _i32(node_types)
        n = types.size
        pos = _f64(positions, 3 * n, "positions")
        c = _f64(cell, 9, "cell")
        ic = _f64(inverse_cell, 9, "inverse_cell")
        gen = c_u64(0)
        ne = c_i64(0)
        check(library().sxl_prepare_periodic_graph(self._h, n, _p(types, ctypes.c_int), _p(pos, ctypes.c_double),
                                                   _p(c, ctypes.c_double), _p(ic, ctypes.c_double),
                                                   float(neighbor_cutoff), ctypes.byref(gen), ctypes.byref(ne)))
        self._generation = int(gen.value)
        self._evaluated = False
        return {"generation": self._generation, "num_edges": int(ne.value)}

    def _prepare_periodic_factorized_graph_device(self, node_types, positions_ptr, cell, inverse_cell,
                                                  neighbor_cutoff):
        """As ``_prepare_periodic_factorized_graph`` with positions already on
        the device (an integer device address, e.g. ``tensor.data_ptr()``)."""
        types = _i32(node_types)
        c = _f64(cell, 9, "cell")
        ic = _f64(inverse_cell, 9, "inverse_cell")
        gen = c_u64(0)
        ne = c_i64(0)
        check(library().sxl_prepare_periodic_graph_device(
            self._h, types.size, _p(types, ctypes.c_int), ctypes.c_void_p(int(positions_ptr)),
            _p(c, ctypes.c_double), _p(ic, ctypes.c_double), float(neighbor_cutoff), ctypes.byref(gen),
            ctypes.byref(ne)))
        self._generation = int(gen.value)
        self._evaluated = False
        return {"generation": self._generation, "num_edges": int(ne.value)}

    def _update_factorized_cell(self, generation, cell, inverse_cell):
        c = _f64(cell, 9, "cell")
        ic = _f64(inverse_cell, 9, "inverse_cell")
        check(library().sxl_update_cell(self._h, c_u64(int(generation)), _p(c, ctypes.c_double),
                                        _p(ic, ctypes.c_double)))

    def _validate_graph_cardinality(self, num_receivers, num_feature_nodes, num_edges):
        """32-bit cardinality checks (reference ``_validate_graph_cardinality``,
        mace_kokkos.cpp:1604-1607): OverflowError (length_error) or ValueError."""
        check(library().sxl_validate_graph_cardinality(self._h, int(num_receivers), int(num_feature_nodes),
                                                       int(num_edges)))

    def _geometry_arrays(self, positions, second, cell, inverse_cell, pbc, second_kind):
        pos = np.ascontiguousarray(np.asarray(positions, dtype=np.float64).reshape(-1))
        if second_kind == "shifts":
            other = np.ascontiguousarray(np.asarray(second, dtype=np.int32).reshape(-1))
            other_p = _p(other, ctypes.c_int)
        else:
            other = np.ascontiguousarray(np.asarray(second, dtype=np.float64).reshape(-1))
            other_p = _p(other, ctypes.c_double)
        c = _f64(cell, 9, "cell")
        ic = _f64(inverse_cell, 9, "inverse_cell")
        pb = _i32(pbc, 3, "pbc")
        keep = (pos, other, c, ic, pb)
        return keep, (_p(pos, ctypes.c_double), pos.size, other_p, other.size, _p(c, ctypes.c_double),
                      _p(ic, ctypes.c_double), _p(pb, ctypes.c_int))

    def _prepare_factorized_geometry(self, execution_graph_generation, reference_positions, reference_xyz, cell,
                                     inverse_cell, pbc):
        """Geometry of a caller's graph for evaluations from positions: the
        positions and edge vectors at which it was built (reference
        ``_prepare_factorized_geometry``, mace_kokkos.cpp:1608-1629)."""
        keep, args = self._geometry_arrays(reference_positions, reference_xyz, cell, inverse_cell, pbc, "xyz")
        check(library().sxl_prepare_geometry(self._h, c_u64(int(execution_graph_generation)), *args))
        del keep

    def _prepare_factorized_fractional_geometry(self, execution_graph_generation, fractional_positions,
                                                fractional_xyz, cell, inverse_cell, pbc):
        """As ``_prepare_factorized_geometry`` in fractional coordinates of a
        fully periodic cell (reference mace_kokkos.cpp:1650-1669)."""
        keep, args = self._geometry_arrays(fractional_positions, fractional_xyz, cell, inverse_cell, pbc, "xyz")
        check(library().sxl_prepare_fractional_geometry(self._h, c_u64(int(execution_graph_generation)), *args))
        del keep

    def _prepare_factorized_shift_geometry(self, execution_graph_generation, reference_positions, shifts, cell,
                                           inverse_cell, pbc):
        """As ``_prepare_factorized_geometry`` with integer cell shifts per
        edge in place of edge vectors (reference mace_kokkos.cpp:1630-1649)."""
        keep, args = self._geometry_arrays(reference_positions, shifts, cell, inverse_cell, pbc, "shifts")
        check(library().sxl_prepare_shift_geometry(self._h, c_u64(int(execution_graph_generation)), *args))
        del keep

    def _graph_size(self):
        n = ctypes.c_int(0)
        e = c_i64(0)
        g = c_u64(0)
        check(library().sxl_graph_size(self._h, ctypes.byref(n), ctypes.byref(e), ctypes.byref(g)))
        return int(n.value), int(e.value), int(g.value)

    def _periodic_graph_arrays(self, generation):
        """The prepared periodic graph: num_neigh, receiver_offsets, sources,
        shifts, fractional_xyz (reference neighbour-graph output layout)."""
        n, e, _ = self._graph_size()
        num_neigh = np.zeros(n, dtype=np.int32)
        offsets = np.zeros(n + 1, dtype=np.int32)
        sources = np.zeros(e, dtype=np.int32)
        shifts = np.zeros((e, 3), dtype=np.int32)
        frac = np.zeros((e, 3), dtype=np.float64)
        check(library().sxl_graph_arrays(self._h, c_u64(int(generation)), _p(num_neigh, ctypes.c_int),
                                         _p(offsets, ctypes.c_int), _p(sources, ctypes.c_int),
                                         _p(shifts, ctypes.c_int), _p(frac, ctypes.c_double)))
        return {"num_neigh": num_neigh, "receiver_offsets": offsets, "sources": sources, "shifts": shifts,
                "fractional_xyz": frac}

    # ---- evaluation -----------------------------------------------------------
    def _compute_prepared_factorized_positions(self, generation, positions):
        n, _, _ = self._graph_size()
        pos = _f64(positions, 3 * n, "positions")
        check(library().sxl_compute_prepared_positions(self._h, c_u64(int(generation)), _p(pos, ctypes.c_double)))
        self._evaluated = True

    def _compute_prepared_factorized_positions_device(self, generation, positions_ptr):
        check(library().sxl_compute_prepared_positions_device(self._h, c_u64(int(generation)),
                                                              ctypes.c_void_p(int(positions_ptr))))
        self._evaluated = True

    def _compute_prepared_factorized(self, generation, xyz, r):
        _, e, _ = self._graph_size()
        x = _f64(xyz, 3 * e, "xyz")
        rr = _f64(r, e, "r")
        check(library().sxl_compute_prepared(self._h, c_u64(int(generation)), _p(x, ctypes.c_double),
                                             _p(rr, ctypes.c_double)))
        self._evaluated = True

    def _compute_prepared_factorized_device(self, generation, xyz_ptr, r_ptr):
        """As _compute_prepared_factorized with xyz [E][3] and r [E] doubles
        in device memory (pointers), read during the call."""
        check(library().sxl_compute_prepared_device(self._h, c_u64(int(generation)), ctypes.c_void_p(int(xyz_ptr)),
                                                    ctypes.c_void_p(int(r_ptr))))
        self._evaluated = True

    def compute_node_energies_forces(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                                     execution_graph_generation=0):
        """Evaluate energies and directed forces (reference
        ``compute_node_energies_forces``, mace_kokkos.cpp:2169-2203).  With a
        nonzero generation the prepared graph of that token is reused."""
        if execution_graph_generation:
            self._compute_prepared_factorized(execution_graph_generation, xyz, r)
            return
        types = _i32(node_types, num_nodes, "node_types")
        nn = _i32(num_neigh, num_nodes, "num_neigh")
        e = int(nn.sum())
        idx = _i32(neigh_indices, e, "neigh_indices")
        nt = _i32(neigh_types, e, "neigh_types")
        x = _f64(xyz, 3 * e, "xyz")
        rr = _f64(r, e, "r")
        check(library().sxl_compute_node_energies_forces(
            self._h, int(num_nodes), _p(types, ctypes.c_int), _p(nn, ctypes.c_int), _p(idx, ctypes.c_int),
            _p(nt, ctypes.c_int), _p(x, ctypes.c_double), _p(rr, ctypes.c_double)))
        _, _, self._generation = self._graph_size()
        self._evaluated = True

    def _set_execution_plan_request(self, algorithm, profile, debug_plan=""):
        check(library().sxl_set_execution_plan_request(self._h, str(algorithm).encode(), str(profile).encode(),
                                                       str(debug_plan or "").encode()))
        self._evaluated = False

    def _heads(self):
        length = c_i64(0)
        check(library().sxl_model_heads_json(self._h, None, 0, ctypes.byref(length)))
        buf = ctypes.create_string_buffer(int(length.value) + 1)
        check(library().sxl_model_heads_json(self._h, buf, len(buf), ctypes.byref(length)))
        return json.loads(buf.value.decode())

    @property
    def selected_head(self):
        """Prediction head whose parameters were loaded (reference selected_head)."""
        return self._heads()["selected_head"]

    @property
    def available_heads(self):
        """Prediction heads stored in the model file (reference available_heads)."""
        return self._heads()["available_heads"]

    @property
    def execution_plan_report(self):
        """The planner's candidates, memory estimates and selection for the
        prepared graph (reference execution_plan_report)."""
        length = c_i64(0)
        check(library().sxl_execution_plan_json(self._h, None, 0, ctypes.byref(length)))
        buf = ctypes.create_string_buffer(int(length.value) + 1)
        check(library().sxl_execution_plan_json(self._h, buf, len(buf), ctypes.byref(length)))
        return json.loads(buf.value.decode())

    def _pair_compute(self, ilist, numneigh, firstneigh, x, atom_type, local_of, mace_types, f=None):
        """One pair_style symmetrix/mace force call on a LAMMPS-style full
        neighbour list (sxl_pair_compute): ilist [inum], numneigh [nall] and
        firstneigh (nall integer arrays) indexed by atom, x [nall][3], 1-based
        types, local_of [nall], mace_types [ntypes].  Returns the forces
        [nall][3] (accumulated into f when given), eng_vdwl, eatom [nall] and
        the virial [6]."""
        il = _i32(ilist, name="ilist")
        nall = int(np.asarray(atom_type).size)
        nn = _i32(numneigh, nall, "numneigh")
        lists = [_i32(firstneigh[i], int(nn[i]), "firstneigh") for i in range(nall)]
        ptrs = (c_int_p * nall)(*[_p(a, ctypes.c_int) if a.size else c_int_p() for a in lists])
        xx = _f64(x, 3 * nall, "x")
        tt = _i32(atom_type, nall, "type")
        lo = _i32(local_of, nall, "local_of")
        mt = _i32(mace_types, name="mace_types")
        out = np.zeros(3 * nall) if f is None else _f64(f, 3 * nall, "f").copy()
        energy = ctypes.c_double(0.0)
        eatom = np.zeros(nall)
        virial = np.zeros(6)
        check(library().sxl_pair_compute(self._h, il.size, _p(il, ctypes.c_int), _p(nn, ctypes.c_int), ptrs, nall,
                                         _p(xx, ctypes.c_double), _p(tt, ctypes.c_int), _p(lo, ctypes.c_int),
                                         mt.size, _p(mt, ctypes.c_int), _p(out, ctypes.c_double),
                                         ctypes.byref(energy), _p(eatom, ctypes.c_double),
                                         _p(virial, ctypes.c_double)))
        self._evaluated = True
        return {"f": out.reshape(nall, 3), "energy": float(energy.value), "eatom": eatom, "virial": virial}

    def _pair_compute_device(self, inum, ilist_ptr, numneigh_ptr, neighbors_ptr, stride_atom, stride_slot, nall,
                             x_ptr, type_ptr, local_of_ptr, mace_types, f_ptr, eatom_ptr=0):
        """The LAMMPS KOKKOS pair style's compute on device arrays (pointers):
        forces accumulated into f and per-atom energies set in eatom (when
        given) on the device; returns the energy and the virial [6]."""
        mt = _i32(mace_types, name="mace_types")
        energy = ctypes.c_double(0.0)
        virial = np.zeros(6)
        check(library().sxl_pair_compute_device(
            self._h, int(inum), ctypes.c_void_p(int(ilist_ptr)), ctypes.c_void_p(int(numneigh_ptr)),
            ctypes.c_void_p(int(neighbors_ptr)), c_i64(int(stride_atom)), c_i64(int(stride_slot)), int(nall),
            ctypes.c_void_p(int(x_ptr)), ctypes.c_void_p(int(type_ptr)), ctypes.c_void_p(int(local_of_ptr)),
            mt.size, _p(mt, ctypes.c_int), ctypes.c_void_p(int(f_ptr)), ctypes.byref(energy),
            ctypes.c_void_p(int(eatom_ptr)) if eatom_ptr else None, _p(virial, ctypes.c_double)))
        self._evaluated = True
        return {"energy": float(energy.value), "virial": virial}

    def _pair_compute_device_prepared(self, neighbor_ago, inum, ilist_ptr, numneigh_ptr, neighbors_ptr, stride_atom,
                                      stride_slot, nall, x_ptr, type_ptr, local_of_ptr, mace_types, f_ptr,
                                      eatom_ptr=0):
        """The LAMMPS KOKKOS pair style's prepared execution on device arrays:
        every listed pair an edge (those beyond r_cut scaled to it), the graph
        rebuilt when neighbor_ago is 0 (or the list's counts changed) and
        otherwise only the edge vectors updated.  Returns the energy, the
        virial [6] and whether the graph was rebuilt."""
        mt = _i32(mace_types, name="mace_types")
        energy = ctypes.c_double(0.0)
        virial = np.zeros(6)
        rebuilt = ctypes.c_int(0)
        check(library().sxl_pair_compute_device_prepared(
            self._h, int(neighbor_ago), int(inum), ctypes.c_void_p(int(ilist_ptr)), ctypes.c_void_p(int(numneigh_ptr)),
            ctypes.c_void_p(int(neighbors_ptr)), c_i64(int(stride_atom)), c_i64(int(stride_slot)), int(nall),
            ctypes.c_void_p(int(x_ptr)), ctypes.c_void_p(int(type_ptr)), ctypes.c_void_p(int(local_of_ptr)),
            mt.size, _p(mt, ctypes.c_int), ctypes.c_void_p(int(f_ptr)), ctypes.byref(energy),
            ctypes.c_void_p(int(eatom_ptr)) if eatom_ptr else None, _p(virial, ctypes.c_double),
            ctypes.byref(rebuilt)))
        self._evaluated = True
        return {"energy": float(energy.value), "virial": virial, "rebuilt": bool(rebuilt.value)}

    def _md_nve(self, node_types, masses, positions, velocities, cell, skin, dt, steps, progress=None):
        """Velocity-Verlet NVE run on the device (the `fix nve` update of the
        reference's LAMMPS capacity runs).  positions (A), velocities (A/fs),
        masses (amu), dt (fs).  Returns the final positions and velocities,
        the potential and kinetic energies (eV) at the start and after every
        step, each step's wall time and the number of neighbour-graph
        rebuilds.  progress(step, epot, ekin, seconds), when given, is called
        after every step; a true return ends the run after that step."""
        types = _i32(node_types, name="node_types")
        n = types.size
        m = _f64(masses, n, "masses")
        x = _f64(positions, 3 * n, "positions").copy()
        v = _f64(velocities, 3 * n, "velocities").copy()
        c = _f64(cell, 9, "cell")
        inv = _f64(np.linalg.inv(c.reshape(3, 3)), 9, "inverse_cell")
        steps = int(steps)
        epot = np.zeros(max(steps, 0) + 1)
        ekin = np.zeros(max(steps, 0) + 1)
        seconds = np.zeros(max(steps, 1))
        rebuilds = ctypes.c_int(0)
        callback = None
        if progress is not None:
            def relay(step, ep, ek, sec, _user):
                try:
                    return 1 if progress(int(step), float(ep), float(ek), float(sec)) else 0
                except BaseException:  # an exception must not cross the C ABI: stop the run
                    return 1
            callback = _PROGRESS_FN(relay)
            check(library().sxl_set_md_progress(self._h, ctypes.cast(callback, ctypes.c_void_p), None))
        try:
            check(library().sxl_md_nve(self._h, n, _p(types, ctypes.c_int), _p(m, ctypes.c_double),
                                       _p(x, ctypes.c_double), _p(v, ctypes.c_double), _p(c, ctypes.c_double),
                                       _p(inv, ctypes.c_double), float(skin), float(dt), steps,
                                       _p(epot, ctypes.c_double), _p(ekin, ctypes.c_double),
                                       _p(seconds, ctypes.c_double), ctypes.byref(rebuilds)))
        finally:
            if callback is not None:
                check(library().sxl_set_md_progress(self._h, None, None))
        self._evaluated = True
        return {"positions": x.reshape(n, 3), "velocities": v.reshape(n, 3), "potential_energy": epot,
                "kinetic_energy": ekin, "step_seconds": seconds[:max(steps, 0)], "rebuilds": int(rebuilds.value)}

    def _max_displacement(self, generation, positions):
        n, _, _ = self._graph_size()
        pos = _f64(positions, 3 * n, "positions")
        out = ctypes.c_double(0.0)
        check(library().sxl_max_displacement(self._h, c_u64(int(generation)),
                                             ctypes.cast(pos.ctypes.data, ctypes.c_void_p), 0,
                                             ctypes.byref(out)))
        return float(out.value)

    def _max_displacement_device(self, generation, positions_ptr):
        out = ctypes.c_double(0.0)
        check(library().sxl_max_displacement(self._h, c_u64(int(generation)), ctypes.c_void_p(int(positions_ptr)),
                                             1, ctypes.byref(out)))
        return float(out.value)

    # ---- results ----------------------------------------------------------------
    @property
    def node_energies(self):
        n, _, _ = self._graph_size()
        out = np.zeros(n, dtype=np.float64)
        check(library().sxl_node_energies(self._h, _p(out, ctypes.c_double), n))
        return out

    @property
    def node_forces(self):
        _, e, _ = self._graph_size()
        out = np.zeros(3 * e, dtype=np.float64)
        check(library().sxl_node_forces(self._h, _p(out, ctypes.c_double), e))
        return out

    def _reduce_atom_forces(self, num_nodes, receivers=None, sources=None, execution_graph_generation=0):
        gen = int(execution_graph_generation) or self._generation
        out = np.zeros((int(num_nodes), 3), dtype=np.float64)
        n, _, _ = self._graph_size()
        if n != int(num_nodes):
            raise ValueError("Atom-force reduction extents are inconsistent.")
        check(library().sxl_reduce_atom_forces(self._h, c_u64(gen), _p(out, ctypes.c_double)))
        return out

    def _reduce_stress(self, volume, xyz=None, execution_graph_generation=0):
        gen = int(execution_graph_generation) or self._generation
        out = np.zeros(9, dtype=np.float64)
        check(library().sxl_reduce_stress(self._h, c_u64(gen), float(volume), _p(out, ctypes.c_double)))
        return out.reshape(3, 3)

    def _total_energy(self, execution_graph_generation=0):
        gen = int(execution_graph_generation) or self._generation
        out = ctypes.c_double(0.0)
        check(library().sxl_total_energy(self._h, c_u64(gen), ctypes.byref(out)))
        return float(out.value)

    def _device_results(self):
        """Device addresses of (atom forces [N][3], totals [10]) of the last
        evaluation (valid until the next call)."""
        f = ctypes.c_void_p()
        t = ctypes.c_void_p()
        check(library().sxl_device_results(self._h, ctypes.byref(f), ctypes.byref(t)))
        return f.value, t.value

    def _synchronize(self):
        check(library().sxl_synchronize(self._h))

    def _set_profiling(self, enable=True, stages=None):
        """Per-stage HIP-event timing (counters reset); `stages` limits it
        to the named stages (two events per stage and evaluation)."""
        if stages is None:
            check(library().sxl_set_profiling(self._h, 1 if enable else 0))
            return
        names = [library().sxl_stage_name(i).decode() for i in range(library().sxl_num_stages())]
        mask = 0
        for name in stages:
            mask |= 1 << names.index(name)
        check(library().sxl_set_profiling_stages(self._h, mask if enable else 0))

    def _last_max_displacement(self):
        """Largest displacement measured by the last evaluation from positions."""
        out = ctypes.c_double(0.0)
        check(library().sxl_last_max_displacement(self._h, ctypes.byref(out)))
        return float(out.value)

    def _stage_times(self):
        """{stage: (accumulated device ms, count)} of profiled evaluations."""
        lib = library()
        n = lib.sxl_num_stages()
        ms = np.zeros(n, dtype=np.float64)
        counts = np.zeros(n, dtype=np.int32)
        check(lib.sxl_stage_times(self._h, _p(ms, ctypes.c_double), _p(counts, ctypes.c_int)))
        return {lib.sxl_stage_name(i).decode(): (float(ms[i]), int(counts[i])) for i in range(n)}

    # --- execution plan (reference mace_kokkos.cpp:436-447, 619-620) ---------
    def _set_allow_fixed_workspace(self, enabled):
        """Permit the tiled (fixed-workspace) plan; invalidates the prepared
        graph (reference ``_set_allow_fixed_workspace``)."""
        check(library().sxl_set_allow_fixed_workspace(self._h, 1 if enabled else 0))

    @property
    def allow_fixed_workspace(self):
        v = ctypes.c_int(0)
        check(library().sxl_allow_fixed_workspace(self._h, ctypes.byref(v)))
        return bool(v.value)

    def _set_graph_replay(self, enabled=True):
        """Replay untiled evaluations from positions as one HIP graph launch
        (captured per graph generation, positions array and cell)."""
        check(library().sxl_set_graph_replay(self._h, 1 if enabled else 0))

    @property
    def graph_replay(self):
        v = ctypes.c_int(0)
        check(library().sxl_graph_replay(self._h, ctypes.byref(v)))
        return bool(v.value)

    def _set_dual_layer_workspace_receiver_limit_for_testing(self, receivers):
        """Receivers per tile of the tiled plan; invalidates the prepared
        graph.  Non-positive limits raise ValueError like the reference."""
        check(library().sxl_set_workspace_receiver_limit(self._h, int(receivers)))

    @property
    def dual_layer_tiled_evaluation_count(self):
        return self.stats["tiled_evaluations"]

    # --- observability (reference mace_kokkos.cpp:925-970) ---------------------
    @property
    def factorized_prepared_graph_count(self):
        return self.stats["graph_builds"]

    @property
    def factorized_prepared_evaluation_count(self):
        return self.stats["evaluations"]

    @property
    def factorized_preparation_fence_count(self):
        """Host waits on the evaluator's stream over all graph preparations."""
        return self.stats["preparation_fences"]

    @property
    def factorized_evaluation_fence_count(self):
        """Host waits on the evaluator's stream over all evaluations."""
        return self.stats["evaluation_fences"]

    @property
    def factorized_last_evaluation_ms(self):
        return self.stats["last_evaluation_ms"]

    @property
    def factorized_last_graph_prepare_ms(self):
        return self.stats["last_graph_prepare_ms"]

    @property
    def last_evaluation_launch_count(self):
        """Kernel launches of the last evaluation."""
        return self.stats["last_evaluation_launches"]

    @property
    def last_evaluation_allocation_count(self):
        """Device allocations of the last evaluation (0 once the workspace
        of the prepared graph exists)."""
        return self.stats["last_evaluation_allocations"]

    @property
    def stats(self):
        s = _native.Stats()
        check(library().sxl_stats(self._h, ctypes.byref(s)))
        return {name: getattr(s, name) for name, _ in _native.Stats._fields_}

    # --- workspace and policy properties (reference mace_kokkos.cpp:459-723;
    # accessors libsymmetrix/source/mace_kokkos_runtime.cpp:2366-2511,
    # 3919-3937, 4093-4390).  Each reports what this evaluator holds for the
    # prepared graph; subsystems it does not have (JIT plugins, stored
    # harmonics) report their inactive value.
    def _workspace(self):
        length = c_i64(0)
        check(library().sxl_workspace_json(self._h, None, 0, ctypes.byref(length)))
        buf = ctypes.create_string_buffer(int(length.value) + 1)
        check(library().sxl_workspace_json(self._h, buf, len(buf), ctypes.byref(length)))
        return json.loads(buf.value.decode())

    def _candidate_bytes(self, plan_id):
        for c in self.execution_plan_report["candidates"]:
            if c["id"] == plan_id:
                return int(c["estimated_bytes"])
        return 0

    @property
    def factorized_graph_generation(self):
        """Generation of the prepared graph (0: none)."""
        return self._workspace()["graph_generation"]

    @property
    def factorized_ready(self):
        return self._workspace()["graph_generation"] != 0

    @property
    def factorized_tiled_ready(self):
        w = self._workspace()
        return w["graph_generation"] != 0 and bool(w["tiled"])

    @property
    def factorized_fallback_evaluation_count(self):
        """Evaluations that left the native kernels: none (there is no fallback path)."""
        return 0

    @property
    def factorized_schedule_build_count(self):
        """Node-block and tile schedules built: one per prepared graph."""
        return self.stats["graph_builds"]

    @property
    def factorized_source_owned_reverse(self):
        """The R1 reverse is receiver-owned (per-edge H1-adjoint messages
        gathered per source)."""
        return False

    @property
    def factorized_jit_ready(self):
        """No JIT plugin is loaded by the evaluator (the R1 plugin ABI is a
        separate ahead-of-time library)."""
        return False

    @property
    def factorized_jit_launch_count(self):
        return 0

    @property
    def factorized_jit_forward_launch_count(self):
        return 0

    @property
    def factorized_jit_reverse_launch_count(self):
        return 0

    @property
    def factorized_workspace_bytes(self):
        """Device bytes of the evaluation's work arrays (node and edge work,
        features, reductions) for the prepared graph."""
        w = self._workspace()
        return w["node_work_bytes"] + w["edge_work_bytes"] + w["feature_bytes"] + w["reduction_bytes"]

    @property
    def factorized_graph_device_capacity_bytes(self):
        return self._workspace()["graph_bytes"]

    @property
    def phi1_workspace_bytes(self):
        """Bytes of Phi1 (its adjoint reuses the buffer)."""
        return self._workspace()["phi1_bytes"]

    @property
    def phi1_policy(self):
        """"receiver-local" under the tiled plan (Phi1 per tile), else "retained"."""
        return "receiver-local" if self._workspace()["tiled"] else "retained"

    @property
    def readout_workspace_bytes(self):
        """Bytes the readout writes besides the A1 adjoint: node energies and
        the direct scalar adjoint."""
        return self._workspace()["readout_bytes"]

    @property
    def readout_policy(self):
        """"fused": one kernel computes the readout and its adjoint per node
        block; nothing of the forward is kept for the reverse."""
        return "fused"

    @property
    def edge_geometry_policy(self):
        """Edge vectors and lengths held as float64 (the reference's
        "cartesian-f64-v1" layout)."""
        return "cartesian-f64-v1"

    @property
    def compact_edge_geometry_bytes(self):
        return 0

    @property
    def execution_geometry_workspace_bytes(self):
        return self._workspace()["geometry_bytes"]

    @property
    def harmonic_value_bytes(self):
        """Harmonics are formed per edge tile in LDS; no array holds them."""
        return 0

    @property
    def harmonic_gradient_bytes(self):
        return 0

    @property
    def shuffled_coordinate_bytes(self):
        return 0

    @property
    def scalar_size_bytes(self):
        return 4

    @property
    def dual_layer_workspace_planned_receivers(self):
        return self._workspace()["tile_receivers"]

    @property
    def dual_layer_workspace_active_receivers(self):
        return self._workspace()["tile_receivers"]

    @property
    def dual_layer_workspace_planned_edges(self):
        """Edges of the largest tile (the arena's edge capacity)."""
        return self._workspace()["max_tile_edges"]

    @property
    def dual_layer_workspace_active_edges(self):
        return self._workspace()["max_tile_edges"]

    @property
    def dual_layer_workspace_batch_count(self):
        """Receiver tiles of the prepared graph (0 untiled)."""
        return self._workspace()["num_tiles"]

    @property
    def dual_layer_workspace_bytes(self):
        """The tiled plan's reused arena: per-receiver work arrays and per-edge
        geometry, pair codes, directed forces and messages (0 untiled)."""
        w = self._workspace()
        return w["node_work_bytes"] + w["edge_work_bytes"] if w["tiled"] else 0

    @property
    def dual_layer_workspace_bytes_per_receiver(self):
        w = self._workspace()
        return w["node_work_bytes"] // w["tile_receivers"] if w["tiled"] else 0

    @property
    def dual_layer_workspace_bytes_per_edge(self):
        w = self._workspace()
        return w["edge_work_bytes"] // max(w["max_tile_edges"], 1) if w["tiled"] else 0

    @property
    def dual_layer_schedule_bytes(self):
        """Bytes of the tiles' (source, start, length) runs."""
        return self._workspace()["run_bytes"]

    @property
    def dual_layer_source_segment_count(self):
        """(source, tile) runs of the tiled plan's source-grouped edge lists."""
        return self._workspace()["tile_runs"]

    @property
    def execution_active_receiver_count(self):
        return self._workspace()["num_nodes"]

    @property
    def execution_active_feature_node_count(self):
        return self._workspace()["num_nodes"]

    @property
    def execution_active_edge_count(self):
        return self._workspace()["num_edges"]

    @property
    def execution_planned_receiver_capacity(self):
        w = self._workspace()
        return w["tile_receivers"] if w["tiled"] else w["num_nodes"]

    @property
    def execution_planned_feature_node_capacity(self):
        return self._workspace()["num_nodes"]

    @property
    def execution_planned_edge_capacity(self):
        w = self._workspace()
        return w["max_tile_edges"] if w["tiled"] else w["num_edges"]

    @property
    def execution_planned_capacity_bytes(self):
        """The selected plan's memory estimate."""
        return self._candidate_bytes(self.execution_plan_report["selected_id"])

    @property
    def execution_capacity_selection_reason(self):
        return self.execution_plan_report["selection_reason"]

    @property
    def low_memory(self):
        """The prepared graph runs the tiled (capacity) plan."""
        return bool(self._workspace()["tiled"])

    @property
    def low_memory_requested(self):
        return self.execution_plan_report["requested_profile"] == "capacity" and self.allow_fixed_workspace

    @property
    def low_memory_policy(self):
        """"disabled" (tiles not allowed), "pending" (no graph), "capacity"
        (tiled plan) or "speed" (untiled plan)."""
        if not self.low_memory_requested:
            return "disabled"
        w = self._workspace()
        if w["graph_generation"] == 0:
            return "pending"
        return "capacity" if w["tiled"] else "speed"

    @property
    def low_memory_selection_reason(self):
        return self.execution_plan_report["selection_reason"]

    @property
    def low_memory_device_free_bytes(self):
        return self._workspace()["device_free_bytes"]

    @property
    def low_memory_device_total_bytes(self):
        return self._workspace()["device_total_bytes"]

    @property
    def low_memory_available_bytes(self):
        return int(self.execution_plan_report["available_bytes"])

    @property
    def low_memory_reserve_bytes(self):
        return int(self.execution_plan_report["reserve_bytes"])

    @property
    def low_memory_speed_estimated_bytes(self):
        return self._candidate_bytes("mh0-direct-speed")

    @property
    def low_memory_capacity_estimated_bytes(self):
        return self._candidate_bytes("mh0-dual-layer-tiled-v1")

    @property
    def low_memory_selected_estimated_bytes(self):
        return self.execution_planned_capacity_bytes


# --- runtime lifecycle (reference tools_kokkos.cpp:522-534) ---------------------
def _init_kokkos():
    """Initialise the HIP runtime (reference ``_init_kokkos``); creating an
    evaluator does this too."""
    check(library().sxl_runtime_initialize())


def _finalize_kokkos():
    """Finalise the runtime (reference ``_finalize_kokkos``): RuntimeError
    while evaluators are alive; no evaluator can be created afterwards."""
    check(library().sxl_runtime_finalize())


def _kokkos_is_initialized():
    return bool(library().sxl_runtime_is_initialized())


def _kokkos_live_object_count():
    """Evaluator objects alive in this process."""
    return int(library().sxl_live_evaluator_count())


def _kokkos_default_execution_space():
    return library().sxl_default_execution_space().decode()


def periodic_neighbor_graph(positions, cell, inverse_cell, cutoff):
    """Periodic neighbour graph on the device in the reference's edge order
    (reference ``_kokkos_periodic_neighbor_graph``): dict of num_neigh,
    receiver_offsets, sources, shifts, fractional_xyz."""
    lib = library()
    pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
    n = pos.shape[0]
    c = _f64(cell, 9, "cell")
    ic = _f64(inverse_cell, 9, "inverse_cell")
    handle = ctypes.c_void_p()
    ne = c_i64(0)
    check(lib.sxl_neighbor_graph_build(_p(pos, ctypes.c_double), n, _p(c, ctypes.c_double),
                                       _p(ic, ctypes.c_double), float(cutoff), ctypes.byref(handle),
                                       ctypes.byref(ne)))
    try:
        e = int(ne.value)
        num_neigh = np.zeros(n, dtype=np.int32)
        offsets = np.zeros(n + 1, dtype=np.int32)
        sources = np.zeros(e, dtype=np.int32)
        shifts = np.zeros((e, 3), dtype=np.int32)
        frac = np.zeros((e, 3), dtype=np.float64)
        check(lib.sxl_neighbor_graph_copy(handle, _p(num_neigh, ctypes.c_int), _p(offsets, ctypes.c_int),
                                          _p(sources, ctypes.c_int), _p(shifts, ctypes.c_int),
                                          _p(frac, ctypes.c_double)))
    finally:
        lib.sxl_neighbor_graph_free(handle)
    return {"num_neigh": num_neigh, "receiver_offsets": offsets, "sources": sources, "shifts": shifts,
            "fractional_xyz": frac}


# reference binding name (symmetrix._kokkos_periodic_neighbor_graph)
_kokkos_periodic_neighbor_graph = periodic_neighbor_graph
