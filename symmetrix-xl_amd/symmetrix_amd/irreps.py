"""Real spherical harmonics, real Wigner matrices and coupling tensors.

Conventions follow the evaluator this package replaces:

* Y_lm is the orthonormal real spherical harmonic without the Condon-Shortley
  phase, evaluated on the permuted direction (z, x, y) and multiplied by
  2*sqrt(pi) (reference ``libsymmetrix/source/mace.cpp:1268-1299``;
  normalisation constant ``spherical_harmonic_device.hpp:15-16``).  With this
  permutation Y_1 = sqrt(3) * (x, y, z) / r.
* Components are indexed lm = l*l + l + m, m = -l..l
  (``edge_harmonics.layout`` "lm=l*l+l+m" in the reference's execution
  contracts).
* Coupling tensors C[m1, m2, M] are "component" normalised: for every output
  component M the squares over (m1, m2) sum to one.  This is the
  normalisation of the coefficients stored in the reference's R1 contract
  (``symmetrix/test/data/execution_contracts/jit_r1_mace_mpa0_medium_contract.json``).

Wigner matrices and coupling tensors are derived numerically from the
harmonics themselves, so they are consistent with Y_lm by construction.
"""

from __future__ import annotations

import functools
import math

import numpy as np

SH_NORMALIZATION = 3.5449077018110318  # 2*sqrt(pi)
MAX_L = 3

# Orthonormal real spherical-harmonic prefactors (no Condon-Shortley phase).
_C00 = 0.5 / math.sqrt(math.pi)
_C1 = math.sqrt(3.0 / (4.0 * math.pi))
_C2A = math.sqrt(15.0 / (4.0 * math.pi))
_C20 = math.sqrt(5.0 / (16.0 * math.pi))
_C22 = math.sqrt(15.0 / (16.0 * math.pi))
_C33 = math.sqrt(35.0 / (32.0 * math.pi))
_C32 = math.sqrt(105.0 / (4.0 * math.pi))
_C31 = math.sqrt(21.0 / (32.0 * math.pi))
_C30 = math.sqrt(7.0 / (16.0 * math.pi))


def num_lm(lmax: int) -> int:
    return (lmax + 1) * (lmax + 1)


def real_sph_harm_unit(lmax: int, u: np.ndarray) -> np.ndarray:
    """Orthonormal real SH of unit vectors ``u`` (n, 3) in their own frame.

    This is the textbook real basis (the one sphericart evaluates): m > 0 goes
    with Re((x+iy)^m), m < 0 with Im((x+iy)^|m|), positive prefactors.
    """
    if lmax > MAX_L:
        raise ValueError(f"l_max {lmax} exceeds the supported maximum {MAX_L}")
    u = np.asarray(u, dtype=np.float64).reshape(-1, 3)
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    out = np.zeros((u.shape[0], num_lm(lmax)))
    out[:, 0] = _C00
    if lmax >= 1:
        out[:, 1] = _C1 * y
        out[:, 2] = _C1 * z
        out[:, 3] = _C1 * x
    if lmax >= 2:
        out[:, 4] = _C2A * x * y
        out[:, 5] = _C2A * y * z
        out[:, 6] = _C20 * (3.0 * z * z - 1.0)
        out[:, 7] = _C2A * x * z
        out[:, 8] = _C22 * (x * x - y * y)
    if lmax >= 3:
        out[:, 9] = _C33 * y * (3.0 * x * x - y * y)
        out[:, 10] = _C32 * x * y * z
        out[:, 11] = _C31 * y * (5.0 * z * z - 1.0)
        out[:, 12] = _C30 * z * (5.0 * z * z - 3.0)
        out[:, 13] = _C31 * x * (5.0 * z * z - 1.0)
        out[:, 14] = 0.5 * _C32 * z * (x * x - y * y)
        out[:, 15] = _C33 * x * (x * x - 3.0 * y * y)
    return out


def mace_sph_harm(lmax: int, xyz: np.ndarray) -> np.ndarray:
    """MACE-convention harmonics of edge vectors ``xyz`` (n, 3).

    The direction is normalised, permuted to (z, x, y) and the orthonormal
    value is scaled by 2*sqrt(pi) (``mace.cpp:1268-1299``).
    """
    xyz = np.asarray(xyz, dtype=np.float64).reshape(-1, 3)
    r = np.linalg.norm(xyz, axis=1)
    unit = np.zeros_like(xyz)
    nz = r > 0
    unit[nz] = xyz[nz] / r[nz, None]
    shuffled = unit[:, [2, 0, 1]]
    values = real_sph_harm_unit(lmax, shuffled) * SH_NORMALIZATION
    # the zero vector has only the constant harmonic (reference zero-vector rule)
    values[~nz, 1:] = 0.0
    return values


def _random_rotation(rng: np.random.Generator) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array(
        [
            [a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
            [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
            [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d],
        ]
    )


def random_rotation(seed: int = 0) -> np.ndarray:
    return _random_rotation(np.random.default_rng(seed))


def _real_block_any_l(l: int, u: np.ndarray) -> np.ndarray:
    """Some orthonormal real basis of degree-l harmonics (any l).

    Used only for intermediate irreps of nested couplings (l > 3), where the
    basis convention cancels between the two couplings that share it.
    """
    from scipy.special import sph_harm_y

    theta = np.arccos(np.clip(u[:, 2], -1.0, 1.0))
    phi = np.arctan2(u[:, 1], u[:, 0])
    out = np.zeros((u.shape[0], 2 * l + 1))
    for m in range(-l, l + 1):
        y = sph_harm_y(l, abs(m), theta, phi)
        if m > 0:
            out[:, l + m] = math.sqrt(2.0) * y.real
        elif m < 0:
            out[:, l + m] = math.sqrt(2.0) * y.imag
        else:
            out[:, l] = y.real
    return out


def _harmonic_block(l: int, xyz: np.ndarray) -> np.ndarray:
    if l <= MAX_L:
        return mace_sph_harm(l, xyz)[:, l * l : (l + 1) * (l + 1)]
    unit = xyz / np.linalg.norm(xyz, axis=1, keepdims=True)
    return _real_block_any_l(l, unit[:, [2, 0, 1]])


def wigner_d(l: int, rotation: np.ndarray) -> np.ndarray:
    """Real Wigner matrix D with Y_l(R x) = D @ Y_l(x) for MACE harmonics."""
    rng = np.random.default_rng(12345 + l)
    points = rng.normal(size=(16 * (2 * l + 1), 3))
    points /= np.linalg.norm(points, axis=1, keepdims=True)
    a = _harmonic_block(l, points)
    b = _harmonic_block(l, points @ np.asarray(rotation).T)
    dt, *_ = np.linalg.lstsq(a, b, rcond=None)
    return dt.T


def triangle(l1: int, l2: int, l3: int) -> bool:
    return abs(l1 - l2) <= l3 <= l1 + l2


@functools.lru_cache(maxsize=None)
def coupling_tensor(l1: int, l2: int, lout: int) -> np.ndarray:
    """Real coupling tensor C[m1, m2, M] of l1 x l2 -> lout.

    Solved as the one-dimensional null space of the equivariance constraint
    over a few random rotations, normalised per output component.  Sign: for
    a natural-parity triple (l1 + l2 + lout even) the m = 0 x m = 0 -> m = 0
    entry, C[l1, l2, lout], is nonzero (the 3j symbol (l1 l2 lout; 0 0 0)
    vanishes only for odd sums) and is made positive.  This is the convention
    of the reference's coupling values: it reproduces every term of its
    contracts for the (3,1), (3,2) and (3,0) shapes
    (symmetrix/test/data/execution_contracts/jit_r1_*_contract.json), where
    the previous "largest entry positive" rule flipped the (2,2,2) and (3,2,3)
    paths.  Other triples keep the entry of largest magnitude (first in C
    order on ties) positive.
    """
    if not triangle(l1, l2, lout):
        raise ValueError(f"({l1}, {l2}) cannot couple to {lout}")
    d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * lout + 1
    rows = []
    for seed in range(3):
        rot = random_rotation(1000 + seed)
        w1, w2, w3 = wigner_d(l1, rot), wigner_d(l2, rot), wigner_d(lout, rot)
        lhs = np.kron(w1.T, np.kron(w2.T, np.eye(d3)))
        rhs = np.kron(np.eye(d1), np.kron(np.eye(d2), w3))
        rows.append(lhs - rhs)
    constraint = np.concatenate(rows, axis=0)
    _, sing, vt = np.linalg.svd(constraint)
    if sing[-1] > 1e-8 or (len(sing) > 1 and sing[-2] < 1e-6):
        raise RuntimeError("coupling null space is not one-dimensional")
    tensor = vt[-1].reshape(d1, d2, d3) * math.sqrt(d3)
    if (l1 + l2 + lout) % 2 == 0:
        if tensor[l1, l2, lout] < 0:
            tensor = -tensor
    else:
        flat = tensor.reshape(-1)
        peak = np.max(np.abs(flat))
        first = int(np.flatnonzero(np.abs(flat) > peak - 1e-9)[0])
        if flat[first] < 0:
            tensor = -tensor
    tensor[np.abs(tensor) < 1e-12] = 0.0
    return tensor


def r1_paths(edge_lmax: int, source_lmax: int, output_lmax: int | None = None):
    """Ordered (edge_l, source_l, output_l) paths of the second interaction.

    The order is the one of MACE's tensor-product instructions sorted by output
    irrep, which is the order of the reference contract's ``paths`` list: for
    each source irrep, each edge irrep, each admissible output (natural parity,
    output l <= ``output_lmax``), then a stable sort on output l.
    """
    if output_lmax is None:
        output_lmax = edge_lmax
    paths = []
    for source_l in range(source_lmax + 1):
        for edge_l in range(edge_lmax + 1):
            for out_l in range(abs(edge_l - source_l), edge_l + source_l + 1):
                if out_l > output_lmax or (edge_l + source_l + out_l) % 2:
                    continue
                paths.append((edge_l, source_l, out_l))
    return sorted(paths, key=lambda p: p[2])


def phi1_tables(edge_lmax: int, source_lmax: int):
    """Sparse CG terms of the second interaction in the JSON layout.

    Returns a dict with ``Phi1_l``/``Phi1_l1``/``Phi1_l2`` (per path) and the
    term lists ``Phi1_lme``/``Phi1_lelm1lm2``/``Phi1_clebsch_gordan``.  Rows
    (lelm1lm2) run over paths, then edge m1, then source m2; output rows (lme)
    are grouped by output l, then m, then path within that l
    (``mace.cpp:1969-2020`` and ``mace.cpp:2304-2340`` consume this layout).
    """
    paths = r1_paths(edge_lmax, source_lmax)
    num_e = [0] * (edge_lmax + 1)
    path_e = []
    for _, _, lo in paths:
        path_e.append(num_e[lo])
        num_e[lo] += 1
    lme_offset = []
    offset = 0
    for l in range(edge_lmax + 1):
        lme_offset.append(offset)
        offset += (2 * l + 1) * num_e[l]
    terms = []
    row = 0
    for p, (l1, l2, lo) in enumerate(paths):
        cg = coupling_tensor(l1, l2, lo)
        for m1 in range(2 * l1 + 1):
            for m2 in range(2 * l2 + 1):
                for mo in range(2 * lo + 1):
                    c = cg[m1, m2, mo]
                    if c != 0.0:
                        lme = lme_offset[lo] + mo * num_e[lo] + path_e[p]
                        terms.append(
                            {
                                "lm1": l1 * l1 + m1,
                                "lm2": l2 * l2 + m2,
                                "row": row,
                                "lme": lme,
                                "coefficient": float(c),
                            }
                        )
                row += 1
    terms.sort(key=lambda t: (t["lm1"], t["lm2"], t["row"], t["lme"]))
    return {
        "paths": paths,
        "num_e": num_e,
        "Phi1_l": [p[2] for p in paths],
        "Phi1_l1": [p[0] for p in paths],
        "Phi1_l2": [p[1] for p in paths],
        "Phi1_lme": [t["lme"] for t in terms],
        "Phi1_lelm1lm2": [t["row"] for t in terms],
        "Phi1_clebsch_gordan": [t["coefficient"] for t in terms],
        "terms": terms,
    }


def _poly_from_tensor(indices_per_slot, tensor):
    """Expand sum T[a,b,..,M] x[i_a] x[i_b].. into {monomial: coef[M]}."""
    out = {}
    dims = tensor.shape[:-1]
    for idx in np.ndindex(*dims):
        vec = tensor[idx]
        if not np.any(vec != 0.0):
            continue
        mono = tuple(sorted(indices_per_slot[s][i] for s, i in enumerate(idx)))
        acc = out.get(mono)
        out[mono] = vec.copy() if acc is None else acc + vec
    return out


def equivariant_polynomials(input_lmax: int, out_l: int, correlation: int):
    """Equivariant polynomials of one channel's harmonics A[lm], lm < (input_lmax+1)^2.

    Each polynomial maps the inputs to the 2*out_l+1 components of one output
    irrep of natural parity, built from products of coupling tensors (degree 1:
    the input itself; degree 2: one coupling; degree 3: two nested couplings
    over every choice of last factor and intermediate l).  Returns, for each
    output component M, (monomials, basis): the monomials with a nonzero
    coefficient in component M, sorted by degree then lexicographically (the
    order of ``standard_m0_contract.json``), and the coefficients of every
    polynomial on them, shape (num_polynomials, num_monomials).  A weight
    vector w over polynomials gives the equivariant map w @ basis_M.
    """
    slots = {l: list(range(l * l, (l + 1) * (l + 1))) for l in range(input_lmax + 1)}
    polys = []
    if out_l <= input_lmax:
        eye = np.eye(2 * out_l + 1)
        polys.append(_poly_from_tensor([slots[out_l]], eye))
    if correlation >= 2:
        for l1 in range(input_lmax + 1):
            for l2 in range(l1, input_lmax + 1):
                if (l1 + l2 + out_l) % 2 or not triangle(l1, l2, out_l):
                    continue
                polys.append(
                    _poly_from_tensor([slots[l1], slots[l2]], coupling_tensor(l1, l2, out_l))
                )
    if correlation >= 3:
        for l1 in range(input_lmax + 1):
            for l2 in range(l1, input_lmax + 1):
                for l3 in range(l2, input_lmax + 1):
                    if (l1 + l2 + l3 + out_l) % 2:
                        continue
                    for last in sorted({(l1, l2, l3)[k] for k in range(3)}):
                        rest = [l1, l2, l3]
                        rest.remove(last)
                        la, lb = rest
                        for lam in range(abs(la - lb), la + lb + 1):
                            if not triangle(lam, last, out_l):
                                continue
                            inner = coupling_tensor(la, lb, lam)
                            outer = coupling_tensor(lam, last, out_l)
                            tensor = np.einsum("abm,mcM->abcM", inner, outer)
                            polys.append(
                                _poly_from_tensor([slots[la], slots[lb], slots[last]], tensor)
                            )
    if correlation > 3:
        raise ValueError("correlation order above 3 is not supported")
    keep = []
    for poly in polys:
        poly = {m: c for m, c in poly.items() if np.max(np.abs(c)) > 1e-12}
        if poly:
            keep.append(poly)
    components = []
    for mo in range(2 * out_l + 1):
        monomials = sorted(
            {m for poly in keep for m, c in poly.items() if abs(c[mo]) > 1e-12},
            key=lambda m: (len(m), m),
        )
        index = {m: i for i, m in enumerate(monomials)}
        basis = np.zeros((len(keep), len(monomials)))
        for p, poly in enumerate(keep):
            for m, c in poly.items():
                if m in index:
                    basis[p, index[m]] = c[mo]
        components.append(([list(m) for m in monomials], basis))
    return components
