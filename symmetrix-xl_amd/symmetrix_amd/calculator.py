"""Energy / forces / stress calculator with neighbour-list skin reuse.

Counterpart of the reference's ASE calculator ``Symmetrix``
(``symmetrix/source/symmetrix/calculator.py:539-757, 2838-3093, 3821-4021``)
for the model-evaluation path: the neighbour graph is built on the device at
cutoff + skin and reused across calls, also across cell changes
(``calculator.py:2851-2898``): edge vectors are the build's fractional edge
vectors in the current cell plus the atoms' minimum-image non-affine
displacements, and the graph stays valid while
``||cell^-1 cell_build||_2 (cutoff + 2 max|non-affine|) <= cutoff + skin``
(with an unchanged cell: no atom moved more than skin/2; atoms wrapped back
into the cell count as not moved).  Every call evaluates at the current
positions; energy is the FP64 sum of node energies, forces are reduced from
the directed edge forces, stress is -(1/V) sum f (x) xyz in Voigt order
(``calculator.py:3821-3894``).

ASE is optional: ``calculate`` accepts an ``ase.Atoms`` or any object with
``positions``, ``numbers`` and ``cell`` (e.g. ``synthetic.Structure``).
"""

from __future__ import annotations

import numpy as np

from .mace import MACEKokkosFloat


def _arrays(atoms):
    if hasattr(atoms, "get_positions"):
        positions = np.asarray(atoms.get_positions(), dtype=np.float64)
        numbers = np.asarray(atoms.get_atomic_numbers())
        cell = np.asarray(atoms.get_cell(), dtype=np.float64)
        pbc = np.asarray(atoms.get_pbc(), dtype=bool)
    else:
        positions = np.asarray(atoms.positions, dtype=np.float64)
        numbers = np.asarray(atoms.numbers)
        cell = np.asarray(atoms.cell, dtype=np.float64)
        pbc = np.asarray(getattr(atoms, "pbc", (True, True, True)), dtype=bool)
    return positions, numbers, cell, pbc


def topology_valid(cell, topology_cell, max_non_affine, cutoff, skin):
    """Whether a graph built at cutoff + skin in ``topology_cell`` still holds
    every pair within ``cutoff`` in ``cell`` after non-affine displacements of
    at most ``max_non_affine`` (reference calculator.py:2872-2877): a pair
    within cutoff now was within contraction * (cutoff + 2 max_non_affine) in
    the build's cell, contraction = ||cell^-1 topology_cell||_2."""
    cell = np.asarray(cell, dtype=float)
    topology_cell = np.asarray(topology_cell, dtype=float)
    if np.array_equal(cell, topology_cell):
        contraction = 1.0  # the identity deformation (the common case: no cell change)
    else:
        try:
            deformation = np.linalg.solve(cell, topology_cell)
        except np.linalg.LinAlgError:
            return False
        contraction = float(np.linalg.norm(deformation, ord=2))
    if not np.isfinite(contraction) or not np.isfinite(max_non_affine):
        return False
    return contraction * (cutoff + 2.0 * max_non_affine) <= cutoff + skin


def full_3x3_to_voigt_6_stress(stress):
    s = np.asarray(stress).reshape(3, 3)
    return np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]), 0.5 * (s[0, 2] + s[2, 0]),
                     0.5 * (s[0, 1] + s[1, 0])])


class Symmetrix:
    """MACE calculator on one MI355X (reference ``symmetrix.Symmetrix``)."""

    implemented_properties = ["energy", "free_energy", "energies", "forces", "stress"]

    def __init__(self, model_file, dtype="float32", use_kokkos=True, streamed_edges="direct",
                 neighbor_skin=0.5, head=None, allow_fixed_workspace=False, execution_profile="capacity",
                 _debug_execution_plan=None, **unused):
        if dtype not in ("float32", np.float32):
            raise ValueError("the MI355X evaluator computes in float32 (dtype='float32')")
        if streamed_edges not in ("direct", "generic", True):
            raise ValueError(f"unsupported streamed_edges mode {streamed_edges!r}")
        if not (neighbor_skin >= 0.0):
            raise ValueError("neighbor_skin must be non-negative")
        self.evaluator = MACEKokkosFloat(model_file, head or "")
        # plan request (reference calculator.py:740-889): the planner picks
        # untiled or receiver-tiled execution per prepared graph
        self.execution_profile = execution_profile
        self.evaluator._set_execution_plan_request("direct", execution_profile, _debug_execution_plan or "")
        if allow_fixed_workspace:
            # tiled plan when the untiled workspace would not fit
            # (reference calculator.py:578-582)
            self.evaluator._set_allow_fixed_workspace(True)
        self.cutoff = float(self.evaluator.r_cut)
        self.neighbor_skin = float(neighbor_skin)
        self._type_of_z = {z: i for i, z in enumerate(self.evaluator.atomic_numbers)}
        self._cache = None
        self.results = {}
        # counters of the reference calculator (calculator.py:2900-3040)
        self.neighbor_cache_build_count = 0
        self.neighbor_cache_reuse_count = 0
        self.neighbor_cache_geometry_update_count = 0
        self.calculation_count = 0

    @property
    def execution_plan(self):
        """Current execution selection and its memory diagnostics (reference
        calculator.py:1691-1725): pending until the first graph is prepared."""
        return dict(self.evaluator.execution_plan_report)

    @property
    def neighbor_rebuild_count(self):
        return self.neighbor_cache_build_count

    # ---- neighbour cache -----------------------------------------------------
    def _node_types(self, numbers):
        try:
            return np.array([self._type_of_z[int(z)] for z in numbers], dtype=np.int32)
        except KeyError as err:
            raise ValueError(f"atomic number {err.args[0]} is not supported by the model") from None

    def _isolated_box(self, positions):
        """Cubic box of an isolated system: side = extent + 2 (cutoff + skin) + 1,
        so no periodic image lies within cutoff + skin while the graph is
        valid (atoms move at most skin/2 each before a rebuild)."""
        reach = self.cutoff + self.neighbor_skin
        lo = positions.min(axis=0) if len(positions) else np.zeros(3)
        hi = positions.max(axis=0) if len(positions) else np.zeros(3)
        side = float(np.max(hi - lo)) + 2.0 * reach + 1.0
        return lo - reach, np.eye(3) * side

    def _geometry(self, atoms):
        positions, numbers, cell, pbc = _arrays(atoms)
        if np.any(pbc) and not np.all(pbc):
            raise NotImplementedError("mixed periodic boundary conditions are not supported")
        return positions, numbers, cell, bool(np.all(pbc))

    def _compatible(self, numbers, cell, periodic):
        """Whether the cached graph may serve these atoms (same species in the
        same order, same periodicity); a changed cell is moved to the device."""
        c = self._cache
        if c is None or c["periodic"] != periodic or len(numbers) != len(c["numbers"]) or \
                np.any(numbers != c["numbers"]):
            return False
        if periodic and not np.array_equal(cell, c["cell"]):
            try:
                inverse = np.linalg.inv(cell)
            except np.linalg.LinAlgError:
                return False
            self.evaluator._update_factorized_cell(c["generation"], cell, inverse)
            c["cell"] = cell.copy()
            self.neighbor_cache_geometry_update_count += 1
        return True

    def _still_valid(self, cell, periodic, moved):
        if not periodic:
            return moved <= 0.5 * self.neighbor_skin
        return topology_valid(cell, self._cache["topology_cell"], moved, self.cutoff, self.neighbor_skin)

    def _build(self, positions, numbers, cell, periodic):
        offset = np.zeros(3)
        if not periodic:
            offset, cell = self._isolated_box(positions)
        types = self._node_types(numbers)
        info = self.evaluator._prepare_periodic_factorized_graph(
            types, positions - offset, cell, np.linalg.inv(cell), self.cutoff + self.neighbor_skin)
        self._cache = {"generation": info["generation"], "numbers": numbers.copy(), "periodic": periodic,
                       "cell": cell.copy(), "topology_cell": cell.copy(), "offset": offset,
                       "num_edges": info["num_edges"]}
        self.neighbor_cache_build_count += 1
        self.neighbor_cache_geometry_update_count += 1

    def _evaluate(self, atoms):
        """Evaluates at the atoms' positions: on the cached graph when it is
        still valid, else on a rebuilt one.  The validity check uses the
        displacement the evaluation itself measured, so a reused graph costs
        one device pass; the rare failed check rebuilds and evaluates again.
        Returns the positions and cell the evaluator saw (isolated systems are
        shifted into their cached box) and the periodicity."""
        positions, numbers, cell, periodic = self._geometry(atoms)
        ev = self.evaluator
        if self._compatible(numbers, cell, periodic):
            c = self._cache
            x = positions if periodic else positions - c["offset"]
            ev._compute_prepared_factorized_positions(c["generation"], x)
            if self._still_valid(cell, periodic, ev._last_max_displacement()):
                self.neighbor_cache_reuse_count += 1
                return x, c["cell"], periodic
        self._build(positions, numbers, cell, periodic)
        c = self._cache
        x = positions if periodic else positions - c["offset"]
        ev._compute_prepared_factorized_positions(c["generation"], x)
        return x, c["cell"], periodic

    # ---- evaluation -----------------------------------------------------------------
    def calculate(self, atoms=None, properties=("energy", "forces", "stress"), system_changes=None):
        positions, cell, periodic = self._evaluate(atoms)
        gen = self._cache["generation"]
        ev = self.evaluator
        energy = ev._total_energy(gen)
        results = {
            "energy": energy,
            "free_energy": energy,
            "energies": ev.node_energies,
            "forces": ev._reduce_atom_forces(len(positions), execution_graph_generation=gen),
        }
        if "stress" in properties and periodic:
            volume = abs(float(np.linalg.det(cell)))
            results["stress"] = full_3x3_to_voigt_6_stress(ev._reduce_stress(volume, None, gen))
        self.results = results
        self.calculation_count += 1
        return results

    def get_potential_energy(self, atoms=None, force_consistent=False):
        return self.calculate(atoms, ("energy",))["energy"]

    def get_forces(self, atoms=None):
        return self.calculate(atoms, ("forces",))["forces"]

    def get_stress(self, atoms=None):
        return self.calculate(atoms, ("stress",))["stress"]

    def get_property(self, name, atoms=None, allow_calculation=True):
        return self.calculate(atoms)[name]
