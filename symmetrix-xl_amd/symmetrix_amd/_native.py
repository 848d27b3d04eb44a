"""ctypes binding of libsymmetrix_amd.so (include/symmetrix_amd.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
symmetrix-xl_amd/csrc``).  There is no fallback: if the library is missing or
does not export the declared symbols, importing the evaluator raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libsymmetrix_amd.so")

SXL_OK = 0
_ERRORS = {
    1: ValueError,        # invalid_argument
    2: IndexError,        # out_of_range
    3: OverflowError,     # length_error (32-bit cardinality)
    4: RuntimeError,      # runtime_error / device failures
    5: RuntimeError,      # logic_error
    6: MemoryError,       # allocation failure
}

c_int_p = ctypes.POINTER(ctypes.c_int)
c_double_p = ctypes.POINTER(ctypes.c_double)
c_u64 = ctypes.c_uint64
c_i64 = ctypes.c_int64


class ModelInfo(ctypes.Structure):
    _fields_ = [
        ("num_elements", ctypes.c_int), ("num_channels", ctypes.c_int), ("l_max", ctypes.c_int),
        ("L_max", ctypes.c_int), ("num_paths", ctypes.c_int), ("spline_points", ctypes.c_int),
        ("r_cut", ctypes.c_double),
    ]


class Stats(ctypes.Structure):
    _fields_ = [
        ("device_bytes", ctypes.c_int64), ("num_nodes", ctypes.c_int), ("num_edges", ctypes.c_int64),
        ("graph_builds", ctypes.c_int), ("evaluations", ctypes.c_int),
        ("last_evaluation_ms", ctypes.c_double), ("tiled_evaluations", ctypes.c_int),
        ("tile_receivers", ctypes.c_int), ("num_tiles", ctypes.c_int),
        ("last_graph_prepare_ms", ctypes.c_double), ("preparation_fences", ctypes.c_int64),
        ("evaluation_fences", ctypes.c_int64), ("last_evaluation_launches", ctypes.c_int64),
        ("last_evaluation_allocations", ctypes.c_int64), ("last_evaluation_fences", ctypes.c_int64),
    ]


# name -> (restype, argtypes); exactly the entry points of include/symmetrix_amd.h
SIGNATURES = {
    "sxl_last_error": (ctypes.c_char_p, []),
    "sxl_create": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "sxl_destroy": (None, [ctypes.c_void_p]),
    "sxl_runtime_initialize": (ctypes.c_int, []),
    "sxl_runtime_finalize": (ctypes.c_int, []),
    "sxl_runtime_is_initialized": (ctypes.c_int, []),
    "sxl_live_evaluator_count": (ctypes.c_int64, []),
    "sxl_default_execution_space": (ctypes.c_char_p, []),
    "sxl_model_info": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ModelInfo)]),
    "sxl_atomic_numbers": (ctypes.c_int, [ctypes.c_void_p, c_int_p]),
    "sxl_atomic_energies": (ctypes.c_int, [ctypes.c_void_p, c_double_p]),
    "sxl_prepare_graph": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p, c_int_p, c_int_p, c_int_p,
                                         ctypes.POINTER(c_u64)]),
    "sxl_prepare_periodic_graph": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p, c_double_p,
                                                  c_double_p, c_double_p, ctypes.c_double,
                                                  ctypes.POINTER(c_u64), ctypes.POINTER(c_i64)]),
    "sxl_prepare_periodic_graph_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p,
                                                         ctypes.c_void_p, c_double_p, c_double_p,
                                                         ctypes.c_double, ctypes.POINTER(c_u64),
                                                         ctypes.POINTER(c_i64)]),
    "sxl_graph_arrays": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_int_p, c_int_p, c_int_p, c_int_p,
                                        c_double_p]),
    "sxl_update_cell": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p, c_double_p]),
    "sxl_neighbor_graph_build_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_double_p, c_double_p,
                                                        ctypes.c_double, c_i64, ctypes.c_void_p, ctypes.c_void_p,
                                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(c_i64),
                                                        ctypes.c_void_p]),
    "sxl_neighbor_graph_noalloc_limits": (c_i64, [c_int_p, c_int_p]),
    "sxl_validate_graph_cardinality": (ctypes.c_int, [ctypes.c_void_p, c_i64, c_i64, c_i64]),
    "sxl_prepare_geometry": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p, c_i64, c_double_p, c_i64,
                                            c_double_p, c_double_p, c_int_p]),
    "sxl_prepare_fractional_geometry": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p, c_i64, c_double_p,
                                                       c_i64, c_double_p, c_double_p, c_int_p]),
    "sxl_prepare_shift_geometry": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p, c_i64, c_int_p, c_i64,
                                                  c_double_p, c_double_p, c_int_p]),
    "sxl_compute_prepared_positions": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p]),
    "sxl_compute_prepared_positions_device": (ctypes.c_int, [ctypes.c_void_p, c_u64, ctypes.c_void_p]),
    "sxl_compute_prepared": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p, c_double_p]),
    "sxl_compute_prepared_device": (ctypes.c_int, [ctypes.c_void_p, c_u64, ctypes.c_void_p, ctypes.c_void_p]),
    "sxl_compute_node_energies_forces": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p, c_int_p,
                                                        c_int_p, c_int_p, c_double_p, c_double_p]),
    "sxl_max_displacement": (ctypes.c_int, [ctypes.c_void_p, c_u64, ctypes.c_void_p, ctypes.c_int,
                                            c_double_p]),
    "sxl_set_profiling_stages": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
    "sxl_last_max_displacement": (ctypes.c_int, [ctypes.c_void_p, c_double_p]),
    "sxl_set_execution_plan_request": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_char_p,
                                                      ctypes.c_char_p]),
    "sxl_model_heads_json": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, c_i64, ctypes.POINTER(c_i64)]),
    "sxl_execution_plan_json": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, c_i64, ctypes.POINTER(c_i64)]),
    "sxl_workspace_json": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, c_i64, ctypes.POINTER(c_i64)]),
    "sxl_set_graph_replay": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "sxl_graph_replay": (ctypes.c_int, [ctypes.c_void_p, c_int_p]),
    "sxl_pair_compute": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p, c_int_p,
                                        ctypes.POINTER(c_int_p), ctypes.c_int, c_double_p, c_int_p, c_int_p,
                                        ctypes.c_int, c_int_p, c_double_p, c_double_p, c_double_p, c_double_p]),
    "sxl_pair_compute_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, c_i64, c_i64, ctypes.c_int, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, c_int_p,
                                               ctypes.c_void_p, c_double_p, ctypes.c_void_p, c_double_p]),
    "sxl_pair_compute_device_prepared": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, c_i64,
                                                        c_i64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                                        ctypes.c_void_p, ctypes.c_int, c_int_p, ctypes.c_void_p,
                                                        c_double_p, ctypes.c_void_p, c_double_p, c_int_p]),
    "sxl_prepare_graph_device": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(c_u64)]),
    "sxl_md_nve": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_int_p, c_double_p, c_double_p, c_double_p,
                                  c_double_p, c_double_p, ctypes.c_double, ctypes.c_double, ctypes.c_int,
                                  c_double_p, c_double_p, c_double_p, c_int_p]),
    "sxl_set_md_progress": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "sxl_node_energies": (ctypes.c_int, [ctypes.c_void_p, c_double_p, ctypes.c_int]),
    "sxl_node_forces": (ctypes.c_int, [ctypes.c_void_p, c_double_p, c_i64]),
    "sxl_reduce_atom_forces": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p]),
    "sxl_reduce_stress": (ctypes.c_int, [ctypes.c_void_p, c_u64, ctypes.c_double, c_double_p]),
    "sxl_total_energy": (ctypes.c_int, [ctypes.c_void_p, c_u64, c_double_p]),
    "sxl_device_results": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                          ctypes.POINTER(ctypes.c_void_p)]),
    "sxl_graph_size": (ctypes.c_int, [ctypes.c_void_p, c_int_p, ctypes.POINTER(c_i64), ctypes.POINTER(c_u64)]),
    "sxl_stats": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Stats)]),
    "sxl_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "sxl_neighbor_graph_build": (ctypes.c_int, [c_double_p, ctypes.c_int, c_double_p, c_double_p,
                                                ctypes.c_double, ctypes.POINTER(ctypes.c_void_p),
                                                ctypes.POINTER(c_i64)]),
    "sxl_neighbor_graph_copy": (ctypes.c_int, [ctypes.c_void_p, c_int_p, c_int_p, c_int_p, c_int_p,
                                               c_double_p]),
    "sxl_neighbor_graph_free": (None, [ctypes.c_void_p]),
    "sxl_set_profiling": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "sxl_num_stages": (ctypes.c_int, []),
    "sxl_stage_name": (ctypes.c_char_p, [ctypes.c_int]),
    "sxl_stage_times": (ctypes.c_int, [ctypes.c_void_p, c_double_p, c_int_p]),
    "sxl_set_allow_fixed_workspace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "sxl_allow_fixed_workspace": (ctypes.c_int, [ctypes.c_void_p, c_int_p]),
    "sxl_set_workspace_receiver_limit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
}

_lib = None


def library():
    """The loaded evaluator library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(
                f"{LIBRARY_PATH} is missing: build it with __graft_entry__.build() "
                "(hipcc for gfx950); there is no CPU fallback"
            )
        lib = ctypes.CDLL(LIBRARY_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != SXL_OK:
        message = library().sxl_last_error().decode(errors="replace")
        raise _ERRORS.get(status, RuntimeError)(message)
