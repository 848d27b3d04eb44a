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
into the cell count as not moved).  A partly periodic cell (a slab or a wire,
which the reference serves with a host neighbour list,
``calculator.py:2934-2990``) is built on the device in a cell whose open axes
are replaced by vectors orthogonal to the periodic ones and longer than the
atoms' extent plus 2 (cutoff + skin), and evaluated through the graph's cell
shifts with displacements wrapped along the periodic axes only; like the
reference, it is rebuilt when the cell changes.  Every call evaluates at the current
positions; energy is the FP64 sum of node energies, forces are reduced from
the directed edge forces, stress is -(1/V) sum f (x) xyz in Voigt order
(``calculator.py:3821-3894``).

ASE is optional: ``calculate`` accepts an ``ase.Atoms`` or any object with
``positions``, ``numbers`` and ``cell`` (e.g. ``synthetic.Structure``).
"""

from __future__ import annotations

import numpy as np

from .mace import MACEKokkosFloat, periodic_neighbor_graph


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

    def _open_axes_cell(self, positions, cell, pbc):
        """Build cell of a partly periodic system: the periodic lattice vectors
        are kept; each open axis becomes a unit vector orthogonal to them (and
        to the other open one) times the atoms' extent along it plus
        2 (cutoff + skin) + 1, and the positions are offset into that box, so
        no image across an open axis lies within cutoff + skin while the graph
        is valid (atoms move at most skin/2 each before a rebuild)."""
        reach = self.cutoff + self.neighbor_skin
        periodic_vectors = np.array([cell[k] for k in range(3) if pbc[k]]).T
        q, _ = np.linalg.qr(periodic_vectors, mode="complete")
        directions = q[:, periodic_vectors.shape[1]:].T
        build_cell = np.array(cell, dtype=float, copy=True)
        offset = np.zeros(3)
        for axis, d in zip([k for k in range(3) if not pbc[k]], directions):
            projection = positions @ d if len(positions) else np.zeros(1)
            lo, hi = float(projection.min()), float(projection.max())
            build_cell[axis] = d * (hi - lo + 2.0 * reach + 1.0)
            offset += d * (lo - reach)
        return build_cell, offset

    def _geometry(self, atoms):
        positions, numbers, cell, pbc = _arrays(atoms)
        mode = "periodic" if np.all(pbc) else "open" if not np.any(pbc) else "mixed"
        return positions, numbers, cell, pbc, mode

    def _compatible(self, numbers, cell, pbc, mode):
        """Whether the cached graph may serve these atoms (same species in the
        same order, same periodicity); a changed cell is moved to the device
        (a partly periodic cell that changed is rebuilt, as the reference's)."""
        c = self._cache
        if c is None or c["mode"] != mode or np.any(c["pbc"] != pbc) or len(numbers) != len(c["numbers"]) or \
                np.any(numbers != c["numbers"]):
            return False
        if mode == "mixed" and not np.array_equal(cell, c["cell"]):
            return False
        if mode == "periodic" and not np.array_equal(cell, c["cell"]):
            try:
                inverse = np.linalg.inv(cell)
            except np.linalg.LinAlgError:
                return False
            self.evaluator._update_factorized_cell(c["generation"], cell, inverse)
            c["cell"] = cell.copy()
            self.neighbor_cache_geometry_update_count += 1
        return True

    def _still_valid(self, cell, mode, moved):
        if mode != "periodic":
            return moved <= 0.5 * self.neighbor_skin
        return topology_valid(cell, self._cache["topology_cell"], moved, self.cutoff, self.neighbor_skin)

    def _build(self, positions, numbers, cell, pbc, mode):
        types = self._node_types(numbers)
        reach = self.cutoff + self.neighbor_skin
        offset = np.zeros(3)
        if mode == "mixed":
            # the device graph of the open-axes box, then evaluated from the
            # caller's positions through its cell shifts (zero along the open
            # axes), displacements wrapped along the periodic axes only
            build_cell, shift_origin = self._open_axes_cell(positions, cell, pbc)
            inverse = np.linalg.inv(build_cell)
            g = periodic_neighbor_graph(positions - shift_origin, build_cell, inverse, reach)
            if np.any(g["shifts"][:, ~pbc]):
                raise RuntimeError("an edge crosses an open axis of the build cell")
            ev = self.evaluator
            gen = ev._prepare_factorized_graph(len(types), types, g["num_neigh"], g["sources"], types[g["sources"]])
            ev._prepare_factorized_shift_geometry(gen, positions, g["shifts"], build_cell, inverse,
                                                  pbc.astype(np.int32))
            info = {"generation": gen, "num_edges": len(g["sources"])}
            geometry_cell = build_cell
        else:
            geometry_cell = cell
            if mode == "open":
                offset, geometry_cell = self._isolated_box(positions)
            info = self.evaluator._prepare_periodic_factorized_graph(
                types, positions - offset, geometry_cell, np.linalg.inv(geometry_cell), reach)
        self._cache = {"generation": info["generation"], "numbers": numbers.copy(), "mode": mode,
                       "pbc": pbc.copy(), "cell": (cell if mode != "open" else geometry_cell).copy(),
                       "topology_cell": geometry_cell.copy(), "offset": offset, "num_edges": info["num_edges"]}
        self.neighbor_cache_build_count += 1
        self.neighbor_cache_geometry_update_count += 1

    def _evaluate(self, atoms):
        """Evaluates at the atoms' positions: on the cached graph when it is
        still valid, else on a rebuilt one.  The validity check uses the
        displacement the evaluation itself measured, so a reused graph costs
        one device pass; the rare failed check rebuilds and evaluates again.
        Returns the positions and cell the evaluator saw (isolated systems are
        shifted into their cached box) and the periodicity."""
        positions, numbers, cell, pbc, mode = self._geometry(atoms)
        ev = self.evaluator
        if self._compatible(numbers, cell, pbc, mode):
            c = self._cache
            x = positions - c["offset"]
            ev._compute_prepared_factorized_positions(c["generation"], x)
            if self._still_valid(cell, mode, ev._last_max_displacement()):
                self.neighbor_cache_reuse_count += 1
                return x, c["cell"], mode
        self._build(positions, numbers, cell, pbc, mode)
        c = self._cache
        x = positions - c["offset"]
        ev._compute_prepared_factorized_positions(c["generation"], x)
        return x, c["cell"], mode

    # ---- evaluation -----------------------------------------------------------------
    def calculate(self, atoms=None, properties=("energy", "forces", "stress"), system_changes=None):
        positions, cell, mode = self._evaluate(atoms)
        gen = self._cache["generation"]
        ev = self.evaluator
        energy = ev._total_energy(gen)
        results = {
            "energy": energy,
            "free_energy": energy,
            "energies": ev.node_energies,
            "forces": ev._reduce_atom_forces(len(positions), execution_graph_generation=gen),
        }
        # stress of a periodic or partly periodic cell: -(1/V) sum f (x) xyz
        # with the caller's cell volume (reference calculator.py:3878-3893)
        volume = abs(float(np.linalg.det(cell))) if mode != "open" else 0.0
        if "stress" in properties and volume > 0.0:
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
