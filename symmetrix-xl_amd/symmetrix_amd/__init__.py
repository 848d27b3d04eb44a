"""MI355X-native MACE evaluator: a drop-in for the model-evaluation path of
Symmetrix-XL (energy, forces and stress of two-interaction compact MACE
models, FP32, one GPU).

    from symmetrix_amd import Symmetrix, MACEKokkosFloat

``MACEKokkosFloat`` mirrors the reference's native evaluator class and
``Symmetrix`` its calculator; both run on the hand-written gfx950 kernels of
``libsymmetrix_amd.so`` and raise if that library has not been built.
"""

from .calculator import Symmetrix, full_3x3_to_voigt_6_stress
from .mace import (
    MACEKokkosFloat,
    _finalize_kokkos,
    _init_kokkos,
    _kokkos_default_execution_space,
    _kokkos_is_initialized,
    _kokkos_live_object_count,
    _kokkos_periodic_neighbor_graph,
    periodic_neighbor_graph,
)

__all__ = [
    "MACEKokkosFloat",
    "Symmetrix",
    "full_3x3_to_voigt_6_stress",
    "periodic_neighbor_graph",
    "_kokkos_periodic_neighbor_graph",
    "_init_kokkos",
    "_finalize_kokkos",
    "_kokkos_is_initialized",
    "_kokkos_live_object_count",
    "_kokkos_default_execution_space",
]
