"""Seeded synthetic inputs: random-init compact MACE JSON and test structures.

No checkpoint converter is available offline, so models are written directly
in the compact JSON format version 4 with ``h1_affine_mode`` "m0_composite"
(or "pre_linear_up", optionally residual-first) that the evaluator loads (keys and layouts: reference
``libsymmetrix/source/mace.cpp:2659-2959``, ``h1_affine_schema.hpp:1-62``,
``symmetrix/test/compact_r1_model.py:97-170``).  Weights are random with the
fan-in scaling of a freshly initialised MACE; the message-passing sums are
divided by ``avg_num_neighbors`` through the A0/A1 weights, as the converter
folds them (``extract_mace_data.py:1443``).  The symmetric-contraction
polynomials (M0, M1) are equivariant combinations built from real coupling
tensors, so a generated model is rotation invariant.

Structures replace ASE builders (ASE is not installed): the cubic SrTiO3
supercell, the irregular random-density box and the rigid-water box of the
benchmark configurations.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field

import numpy as np

from . import irreps

SILU_NORMALIZATION = 1.6791767923989418  # 2nd-moment normalisation of SiLU


@dataclass(frozen=True)
class ModelShape:
    atomic_numbers: tuple
    channels: int
    l_max: int
    L_max: int
    correlation: int
    num_bessel: int = 8
    radial_hidden: tuple = (64, 64, 64)
    r_cut: float = 6.0
    cutoff_p: int = 5
    num_spline_points: int = 256
    avg_num_neighbors: float = 50.0
    readout_hidden: int = 16
    energy_scale: float = 10.0
    m1_correlation: int | None = None
    zbl: bool = False            # ZBL pair repulsion (has_zbl)
    density: tuple = ()          # density-normalised layers: subset of ("A0", "A1")
    agnesi: bool = False         # Agnesi distance transform of the radial features
    # H1 affine basis of format 4: "m0_composite", or "pre_linear_up" with split
    # H1 weights (H1_weights = P U) and readout_1 / skip on M0_scalar P0 (+ residual)
    h1_basis: str = "m0_composite"
    residual: bool = False       # first-interaction residual (pre_linear_up basis only)
    extra: dict = field(default_factory=dict)


# Single-bond covalent radii (A) by atomic number, Z = 0..89, of Cordero et al.,
# Dalton Trans. (2008) 2832 (index 0 is a placeholder); the ZBL envelope and
# the Agnesi transform of a synthetic model take their radii from here.
COVALENT_RADII = (
    0.20, 0.31, 0.28, 1.28, 0.96, 0.84, 0.76, 0.71, 0.66, 0.57, 0.58, 1.66, 1.41, 1.21, 1.11, 1.07,
    1.05, 1.02, 1.06, 2.03, 1.76, 1.70, 1.60, 1.53, 1.39, 1.39, 1.32, 1.26, 1.24, 1.32, 1.22, 1.22,
    1.20, 1.19, 1.20, 1.20, 1.16, 2.20, 1.95, 1.90, 1.75, 1.64, 1.54, 1.47, 1.46, 1.42, 1.39, 1.45,
    1.44, 1.42, 1.39, 1.39, 1.38, 1.39, 1.40, 2.44, 2.15, 2.07, 2.04, 2.03, 2.01, 1.99, 1.98, 1.98,
    1.96, 1.94, 1.92, 1.92, 1.89, 1.90, 1.87, 1.87, 1.75, 1.70, 1.62, 1.51, 1.44, 1.41, 1.36, 1.36,
    1.32, 1.45, 1.46, 1.48, 1.40, 1.50, 1.50, 2.60, 2.21, 2.15,
)
# ZBL screening constants of the MACE ZBL basis (universal screening function
# coefficients, a = 0.4543 * 0.529 / (Zu^0.3 + Zv^0.3)) and envelope power
ZBL_C = (0.1818, 0.5099, 0.2802, 0.02817)
ZBL_A_EXP, ZBL_A_PREFACTOR, ZBL_P = 0.3, 0.4543, 6
# Agnesi transform parameters of the MACE Agnesi distance transform
AGNESI_A, AGNESI_Q, AGNESI_P = 1.0805, 0.9183, 4.5791

PRESETS = {
    # 3 elements, 32x0e+32x1o, lmax 2, correlation 2.
    "tiny": ModelShape(
        atomic_numbers=(38, 22, 8), channels=32, l_max=2, L_max=1, correlation=2,
        radial_hidden=(32, 32), r_cut=5.0, avg_num_neighbors=40.0,
    ),
    # 128x0e+128x1o, lmax 3, correlation 3, 89 elements.
    "medium": ModelShape(
        atomic_numbers=tuple(range(1, 90)), channels=128, l_max=3, L_max=1,
        correlation=3, radial_hidden=(64, 64, 64), r_cut=6.0, avg_num_neighbors=70.0,
    ),
    # Medium shape restricted to the SrTiO3 elements (same kernels, small file).
    "medium3": ModelShape(
        atomic_numbers=(38, 22, 8), channels=128, l_max=3, L_max=1,
        correlation=3, radial_hidden=(64, 64, 64), r_cut=6.0, avg_num_neighbors=70.0,
    ),
    # Medium shape with the Agnesi distance transform: the radial tables are
    # per unordered element pair (6 pairs on SrTiO3) instead of shared.
    "medium_agnesi": ModelShape(
        atomic_numbers=tuple(range(1, 90)), channels=128, l_max=3, L_max=1,
        correlation=3, radial_hidden=(64, 64, 64), r_cut=6.0, avg_num_neighbors=70.0,
        agnesi=True,
    ),
    # Scalar hidden features (L_max = 0, 128x0e, lmax 3, correlation 3): the
    # shape of the reference's omat0-small and off23-small models, whose
    # second interaction has 4 paths and 16 coupling terms.
    "scalar": ModelShape(
        atomic_numbers=(38, 22, 8), channels=128, l_max=3, L_max=0,
        correlation=3, radial_hidden=(64, 64, 64), r_cut=6.0, avg_num_neighbors=70.0,
    ),
    # 256 channels, 0e+1o+2e, lmax 3, correlation 3.
    "wide": ModelShape(
        atomic_numbers=(1, 8), channels=256, l_max=3, L_max=2, correlation=3,
        radial_hidden=(64, 64, 64), r_cut=5.0, avg_num_neighbors=50.0,
    ),
}


def _f32(a):
    return np.asarray(a, dtype=np.float32)


class _Array:
    """JSON leaf holding a float array, written with 9 significant digits
    (exact for float32 values)."""

    __slots__ = ("values",)

    def __init__(self, values):
        self.values = _f32(values).ravel()


def _format_floats(values: np.ndarray) -> str:
    if values.size == 0:
        return "[]"
    return "[" + (("%.9g," * values.size) % tuple(values.tolist()))[:-1] + "]"


def _dump(obj) -> str:
    if isinstance(obj, _Array):
        return _format_floats(obj.values)
    if isinstance(obj, dict):
        return "{" + ",".join(json.dumps(str(k)) + ":" + _dump(v) for k, v in obj.items()) + "}"
    if isinstance(obj, (list, tuple)):
        return "[" + ",".join(_dump(v) for v in obj) + "]"
    if isinstance(obj, (np.floating, float)):
        return repr(float(obj))
    if isinstance(obj, (np.integer,)):
        return str(int(obj))
    return json.dumps(obj)


def _poly_weights(rng, n_poly, degrees, scale_by_degree):
    w = rng.normal(size=n_poly)
    return w * np.array([scale_by_degree[d] for d in degrees])


def _poly_degrees(basis, monomials):
    """Degree of each polynomial (the degree of its monomials)."""
    deg = np.array([len(m) for m in monomials])
    out = []
    for row in basis:
        nz = np.flatnonzero(np.abs(row) > 0)
        out.append(int(deg[nz[0]]) if nz.size else 1)
    return out


def _polynomial_block(rng, num_elements, channels, input_lmax, out_l_max, correlation,
                      scale_by_degree):
    """Monomials and per-element/per-channel coefficients of an equivariant
    symmetric contraction with outputs l = 0..out_l_max.

    Returns (monomials[LM], weights[element][LM] -> array (channels, n_mono)).
    """
    monomials = {}
    weights = [dict() for _ in range(num_elements)]
    for out_l in range(out_l_max + 1):
        comps = irreps.equivariant_polynomials(input_lmax, out_l, correlation)
        n_poly = comps[0][1].shape[0]
        degrees = _poly_degrees(comps[0][1], comps[0][0])
        scale = np.array([scale_by_degree[d] for d in degrees])
        w = rng.normal(size=(num_elements, channels, n_poly)) * scale
        for mo, (monos, basis) in enumerate(comps):
            lm = out_l * out_l + mo
            monomials[str(lm)] = monos
            for a in range(num_elements):
                weights[a][str(lm)] = w[a] @ basis
    return monomials, weights


def random_mace_model(shape: ModelShape | str = "tiny", seed: int = 0) -> dict:
    """Random-init compact MACE model dict (format version 4, m0_composite or
    pre_linear_up basis per ``shape.h1_basis``)."""
    if isinstance(shape, str):
        shape = PRESETS[shape]
    rng = np.random.default_rng(seed)
    z = list(shape.atomic_numbers)
    ne = len(z)
    C = shape.channels
    lmax, Lmax = shape.l_max, shape.L_max
    nlm, nLM = (lmax + 1) ** 2, (Lmax + 1) ** 2
    avg = shape.avg_num_neighbors
    tables = irreps.phi1_tables(lmax, Lmax)
    num_paths = len(tables["paths"])
    num_e = tables["num_e"]

    def mlp(widths):
        return [
            _Array(rng.normal(size=(widths[i + 1], widths[i])) / math.sqrt(widths[i]))
            for i in range(len(widths) - 1)
        ]

    radial_in = shape.num_bessel
    hidden = list(shape.radial_hidden)
    networks = {
        "R0": {
            "shape": [radial_in, *hidden, (lmax + 1) * C],
            "activation": "silu",
            "activation_scale": SILU_NORMALIZATION,
        },
        "R1": {
            "shape": [radial_in, *hidden, num_paths * C],
            "activation": "silu",
            "activation_scale": SILU_NORMALIZATION,
        },
    }
    for name in shape.density:
        if name not in ("A0", "A1"):
            raise ValueError(f"unknown density-normalised layer {name!r}")
        networks[name] = {
            "shape": [radial_in, hidden[0], 1],
            "activation": "silu",
            "activation_scale": SILU_NORMALIZATION,
            "postprocess": "tanh-square",
        }
    for net in networks.values():
        net["weights"] = mlp(net["shape"])

    poly_scale = {1: 1.0, 2: 0.5, 3: 0.25}
    m0_monomials, m0_w = _polynomial_block(rng, ne, C, lmax, Lmax, shape.correlation, poly_scale)
    m1_corr = shape.m1_correlation or shape.correlation
    m1_monomials, m1_w = _polynomial_block(rng, ne, C, lmax, 0, m1_corr, poly_scale)

    model = {
        "symmetrix_format_version": 4,
        "h1_affine_mode": "m0_composite",
        "h1_affine_version": 1,
        "model_type": "MACE",
        "radial_representation": "compact",
        "num_interactions": 2,
        "num_elements": ne,
        "num_channels": C,
        "r_cut": float(shape.r_cut),
        "l_max": lmax,
        "L_max": Lmax,
        "atomic_numbers": z,
        "atomic_energies": [float(v) for v in _f32(rng.uniform(-5.0, -1.0, size=ne))],
        "has_zbl": False,
        "has_field_coupling": False,
        "compact_radial": {
            "spline_grid_min": 1e-12,
            "num_spline_points": shape.num_spline_points,
            "basis": {
                "type": "bessel",
                "weights": [float(n * math.pi / shape.r_cut) for n in range(1, radial_in + 1)],
                "prefactor": float(math.sqrt(2.0 / shape.r_cut)),
            },
            "cutoff": {"type": "polynomial", "r_max": float(shape.r_cut), "p": shape.cutoff_p},
            "distance_transform": (
                {"type": "agnesi", "a": AGNESI_A, "q": AGNESI_Q, "p": AGNESI_P,
                 "covalent_radii": [COVALENT_RADII[zz] for zz in z]}
                if shape.agnesi else {"type": "none"}
            ),
            "networks": networks,
        },
        "H0_weights": _Array(rng.normal(size=(ne, C))),
        "A0_weights": [
            [_Array(rng.normal(size=(C, C)) / (math.sqrt(C) * avg)) for _ in range(lmax + 1)]
            for _ in range(ne)
        ],
        "A0_scaled": "A0" in shape.density,
        "M0_monomials": m0_monomials,
        "M0_weights": {
            str(a): {lm: {str(k): _Array(m0_w[a][lm][k]) for k in range(C)} for lm in m0_monomials}
            for a in range(ne)
        },
        "H1_weights": _Array(rng.normal(size=(Lmax + 1, C, C)) / math.sqrt(C)),
        "Phi1_l": tables["Phi1_l"],
        "Phi1_l1": tables["Phi1_l1"],
        "Phi1_l2": tables["Phi1_l2"],
        "Phi1_lme": tables["Phi1_lme"],
        "Phi1_lelm1lm2": tables["Phi1_lelm1lm2"],
        "Phi1_clebsch_gordan": tables["Phi1_clebsch_gordan"],
        "A1_weights": [
            _Array(rng.normal(size=(num_e[l] * C, C)) / (math.sqrt(num_e[l] * C) * avg))
            for l in range(lmax + 1)
        ],
        "A1_scaled": "A1" in shape.density,
        "M1_monomials": m1_monomials["0"],
        "M1_weights": {
            str(a): {str(k): _Array(m1_w[a]["0"][k]) for k in range(C)} for a in range(ne)
        },
        "H2_weights_for_M0": [_Array(rng.normal(size=(C, C)) / math.sqrt(C)) for _ in range(ne)],
        "H2_weights_for_M1": _Array(rng.normal(size=(C, C)) / math.sqrt(C)),
        "readout_1_weights_for_M0": _Array(
            rng.normal(size=C) * shape.energy_scale / math.sqrt(C)
        ),
        "readout_2_hidden_size": shape.readout_hidden,
        "readout_2_weights_1": _Array(
            rng.normal(size=(shape.readout_hidden, C)) / math.sqrt(C)
        ),
        "readout_2_weights_2": _Array(
            rng.normal(size=shape.readout_hidden)
            * shape.energy_scale / math.sqrt(shape.readout_hidden)
        ),
        "readout_2_scale_factor": SILU_NORMALIZATION,
    }
    if shape.h1_basis == "pre_linear_up":
        _split_h1(model, shape, np.random.default_rng([seed, 1]))
    elif shape.h1_basis != "m0_composite" or shape.residual:
        raise ValueError("the first-interaction residual requires the pre_linear_up basis")
    if shape.zbl:
        model.update({
            "has_zbl": True, "zbl_a_exp": ZBL_A_EXP, "zbl_a_prefactor": ZBL_A_PREFACTOR,
            "zbl_c": list(ZBL_C), "zbl_covalent_radii": list(COVALENT_RADII), "zbl_p": ZBL_P,
        })
    model.update(shape.extra)
    return model


def _split_h1(model: dict, shape: ModelShape, rng) -> None:
    """Rewrite a model in the pre_linear_up basis (h1_affine_schema.hpp:14-24):
    H1_weights = P U per l with the product (P) and linear_up (U) weights kept,
    readout_1 r0 and skip S0_z on the pre-linear_up scalar features, and, for a
    residual-first model, per-element residual constants on the scalar block
    (the first interaction's skip of the scalar node embedding; the blocks of
    l > 0 are zero as in a MACE whose first-layer features are scalars)."""
    C, Lmax = shape.channels, shape.L_max
    ne = len(shape.atomic_numbers)
    P = _f32(rng.normal(size=(Lmax + 1, C, C)) / math.sqrt(C))
    U = _f32(rng.normal(size=(Lmax + 1, C, C)) / math.sqrt(C))
    model["H1_weights"] = _Array(np.einsum("lij,ljk->lik", P.astype(np.float64), U.astype(np.float64)))
    model["H1_product_weights"] = _Array(P)
    model["H1_linear_up_weights"] = _Array(U)
    del model["readout_1_weights_for_M0"], model["H2_weights_for_M0"]
    model["h1_affine_mode"] = "pre_linear_up"
    model["readout_1_weights_for_H1_pre_linear_up"] = _Array(
        rng.normal(size=C) * shape.energy_scale / math.sqrt(C))
    model["H2_weights_for_H1_pre_linear_up"] = [
        _Array(rng.normal(size=(C, C)) / math.sqrt(C)) for _ in range(ne)]
    model["first_interaction_residual"] = bool(shape.residual)
    if shape.residual:
        b = np.zeros((ne, (Lmax + 1) ** 2, C))
        b[:, 0, :] = rng.normal(size=(ne, C)) * 0.5
        model["H1_first_residual_weights"] = _Array(b)


def multihead_model(model: dict, names=("default", "other"), default=None, seed: int = 1) -> dict:
    """A multi-head file (prediction_heads schema 1, reference
    prediction_heads.hpp:10-89) from a single-head model: the first head keeps
    the model's own per-head fields, the others get fresh random readouts and
    atomic energies of the same shapes."""
    rng = np.random.default_rng([seed, 7])
    pre = model.get("h1_affine_mode") == "pre_linear_up"
    readout_1 = "readout_1_weights_for_H1_pre_linear_up" if pre else "readout_1_weights_for_M0"
    fields = ["atomic_energies", readout_1, "readout_2_weights_1", "readout_2_weights_2"]
    if model.get("has_zbl"):
        fields.append("zbl_c")
    out = dict(model)
    params = {}
    for i, name in enumerate(names):
        head = {}
        for f in fields:
            v = model[f]
            if i == 0 or f == "zbl_c":
                head[f] = v
            else:
                arr = np.asarray(v if not isinstance(v, _Array) else v.values, dtype=np.float64)
                head[f] = _Array(arr + rng.normal(size=arr.shape) * (0.5 * np.std(arr) + 1e-3))
        params[name] = head
    out["prediction_heads"] = {"schema_version": 1, "names": list(names),
                               "default": default or names[0], "parameters": params}
    return out


def model_json(model: dict) -> str:
    return _dump(model)


def write_model(path, shape: ModelShape | str = "tiny", seed: int = 0) -> str:
    text = model_json(random_mace_model(shape, seed))
    with open(path, "w") as f:
        f.write(text)
    return str(path)


def load_model(path) -> dict:
    with open(path) as f:
        return json.load(f)


# --------------------------------------------------------------------------
# Structures
# --------------------------------------------------------------------------


@dataclass
class Structure:
    positions: np.ndarray  # (N, 3) Angstrom
    numbers: np.ndarray  # (N,) atomic numbers
    cell: np.ndarray  # (3, 3) rows are lattice vectors
    pbc: tuple = (True, True, True)

    def __len__(self):
        return len(self.numbers)

    @property
    def volume(self) -> float:
        return float(abs(np.linalg.det(self.cell)))

    def copy(self):
        return Structure(self.positions.copy(), self.numbers.copy(), self.cell.copy(), self.pbc)


SRTIO3_A = 3.905
_SRTIO3_BASIS = (
    (38, (0.0, 0.0, 0.0)),
    (22, (0.5, 0.5, 0.5)),
    (8, (0.5, 0.5, 0.0)),
    (8, (0.5, 0.0, 0.5)),
    (8, (0.0, 0.5, 0.5)),
)


def srtio3_supercell(n: int, sigma: float = 0.05, seed: int = 0, a: float = SRTIO3_A) -> Structure:
    """Cubic SrTiO3 n x n x n supercell with Gaussian displacements (sigma, Angstrom)."""
    frac = np.array([b for _, b in _SRTIO3_BASIS])
    nums = np.array([zz for zz, _ in _SRTIO3_BASIS])
    grid = np.stack(np.meshgrid(np.arange(n), np.arange(n), np.arange(n), indexing="ij"), -1)
    cells = grid.reshape(-1, 3)
    pos = ((cells[:, None, :] + frac[None, :, :]).reshape(-1, 3)) * a
    numbers = np.tile(nums, len(cells))
    rng = np.random.default_rng(seed)
    pos = pos + rng.normal(scale=sigma, size=pos.shape)
    return Structure(pos, numbers, np.eye(3) * (a * n))


def irregular_box(num_atoms: int = 20000, density: float = 0.08, min_distance: float = 1.8,
                  elements=(1, 6, 7, 8, 13, 14, 22, 26, 29, 38), seed: int = 0) -> Structure:
    """Atoms placed uniformly at random in a periodic cube, rejection-sampled
    to a minimum separation, species uniform over ``elements``."""
    length = (num_atoms / density) ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    nb = max(1, int(length // min_distance))
    width = length / nb
    bins = {}
    pos = np.empty((num_atoms, 3))
    count = 0
    d2 = min_distance * min_distance
    attempts = 0
    while count < num_atoms:
        attempts += 1
        if attempts > 200 * num_atoms:
            raise RuntimeError("rejection sampling did not converge")
        p = rng.uniform(0.0, length, size=3)
        b = tuple((p // width).astype(int) % nb)
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    key = ((b[0] + dx) % nb, (b[1] + dy) % nb, (b[2] + dz) % nb)
                    for j in bins.get(key, ()):
                        d = pos[j] - p
                        d -= length * np.round(d / length)
                        if d @ d < d2:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pos[count] = p
            bins.setdefault(b, []).append(count)
            count += 1
    numbers = rng.choice(np.asarray(elements), size=num_atoms)
    return Structure(pos, numbers, np.eye(3) * length)


def water_box(num_molecules: int = 10000, density_g_cm3: float = 1.0, seed: int = 0,
              oh: float = 0.957, angle_deg: float = 104.5) -> Structure:
    """Rigid H2O molecules with random orientations on a jittered grid."""
    mass = 15.999 + 2 * 1.008  # g/mol
    volume = num_molecules * mass / 6.02214076e23 / density_g_cm3 * 1e24  # A^3
    length = volume ** (1.0 / 3.0)
    per_axis = int(math.ceil(num_molecules ** (1.0 / 3.0)))
    spacing = length / per_axis
    rng = np.random.default_rng(seed)
    grid = np.stack(np.meshgrid(*(np.arange(per_axis),) * 3, indexing="ij"), -1).reshape(-1, 3)
    sites = grid[rng.permutation(len(grid))[:num_molecules]]
    centers = (sites + 0.5) * spacing + rng.uniform(-0.1, 0.1, size=(num_molecules, 3)) * spacing
    half = math.radians(angle_deg) / 2.0
    local = np.array(
        [[0.0, 0.0, 0.0], [oh * math.sin(half), 0.0, oh * math.cos(half)],
         [-oh * math.sin(half), 0.0, oh * math.cos(half)]]
    )
    pos = np.empty((num_molecules * 3, 3))
    for i in range(num_molecules):
        rot = irreps._random_rotation(rng)
        pos[3 * i : 3 * i + 3] = centers[i] + local @ rot.T
    numbers = np.tile(np.array([8, 1, 1]), num_molecules)
    return Structure(pos, numbers, np.eye(3) * length)


def node_types(structure: Structure, atomic_numbers) -> np.ndarray:
    """Model element indices of the structure's atoms (not atomic numbers)."""
    lookup = {int(zz): i for i, zz in enumerate(atomic_numbers)}
    present = np.unique(structure.numbers)
    missing = sorted(set(int(zz) for zz in present) - set(lookup))
    if missing:
        raise ValueError(f"atomic numbers {missing} are not supported by the model")
    table = np.full(int(present.max()) + 1, -1, dtype=np.int32)
    for zz in present:
        table[int(zz)] = lookup[int(zz)]
    return table[np.asarray(structure.numbers, dtype=np.int64)]
