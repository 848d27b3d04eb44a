"""TEST INFRASTRUCTURE ONLY -- CPU oracle driver.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, and only as the checker (or the timed CPU baseline).
The product never imports it.

Contents:

* ``neighbor_graph``: the C restatement of the reference's periodic
  neighbour graph (``neighbor_oracle.c``).
* ``compact_radial_tables``: numpy restatement of the compact radial model's
  tabulation (``libsymmetrix/source/compact_radial.cpp``):
  Bessel features with polynomial cutoff ``:227-267``, SiLU MLP
  ``multilayer_perceptron.cpp:78-140``, knot derivatives ``:326-370``.
* ``MaceOracle``: the C++ restatement of ``MACECPU`` (``mace_oracle.cpp``)
  built from a model JSON dict, in float32 or float64.
* ``reduce``: atom forces and stress from directed edge forces
  (``mace_kokkos_evaluate.cpp:87-106, 156-186``), and the Voigt order of
  ``calculator.py:3821-3894``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS = {}


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    return os.path.join(_HERE, "liboracle.so")


def _lib(timed=False):
    """The checker build, or with timed=True the vectorised build of the same
    source that bench.py's CPU baseline times (never the checker)."""
    if timed not in _LIBS:
        path = os.path.join(_HERE, "liboracle_timed.so" if timed else "liboracle.so")
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.oracle_neighbor_last_error.restype = ctypes.c_char_p
        lib.oracle_mace_last_error.restype = ctypes.c_char_p
        for name in ("oracle_mace_create_f32", "oracle_mace_create_f64"):
            getattr(lib, name).restype = ctypes.c_void_p
            getattr(lib, name).argtypes = [ctypes.c_void_p]
        for name in ("oracle_mace_destroy_f32", "oracle_mace_destroy_f64"):
            getattr(lib, name).argtypes = [ctypes.c_void_p]
        _LIBS[timed] = lib
    return _LIBS[timed]


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ---------------------------------------------------------------------------
# neighbour graph
# ---------------------------------------------------------------------------


def neighbor_graph(positions, cell, inverse_cell, cutoff):
    """Receiver-major periodic neighbour graph in the reference's edge order.

    Returns dict(num_neigh, receiver_offsets, sources, shifts, fractional_xyz).
    Raises ValueError for inputs the reference rejects.
    """
    lib = _lib()
    pos = np.ascontiguousarray(positions, dtype=np.float64).reshape(-1, 3)
    c = np.ascontiguousarray(cell, dtype=np.float64).reshape(9)
    ic = np.ascontiguousarray(inverse_cell, dtype=np.float64).reshape(9)
    n = pos.shape[0]
    num_neigh = np.zeros(n, dtype=np.int32)
    offsets = np.zeros(n + 1, dtype=np.int32)
    total = ctypes.c_longlong(0)
    status = lib.oracle_neighbor_count(
        _ptr(pos, ctypes.c_double), ctypes.c_int(n), _ptr(c, ctypes.c_double),
        _ptr(ic, ctypes.c_double), ctypes.c_double(cutoff), _ptr(num_neigh, ctypes.c_int),
        _ptr(offsets, ctypes.c_int), ctypes.byref(total))
    if status != 0:
        raise ValueError(lib.oracle_neighbor_last_error().decode())
    e = total.value
    sources = np.zeros(e, dtype=np.int32)
    shifts = np.zeros((e, 3), dtype=np.int32)
    frac = np.zeros((e, 3), dtype=np.float64)
    status = lib.oracle_neighbor_fill(
        _ptr(pos, ctypes.c_double), ctypes.c_int(n), _ptr(c, ctypes.c_double),
        _ptr(ic, ctypes.c_double), ctypes.c_double(cutoff), _ptr(offsets, ctypes.c_int),
        _ptr(sources, ctypes.c_int), _ptr(shifts, ctypes.c_int), _ptr(frac, ctypes.c_double))
    if status != 0:
        raise ValueError(lib.oracle_neighbor_last_error().decode())
    return {
        "num_neigh": num_neigh,
        "receiver_offsets": offsets,
        "sources": sources,
        "shifts": shifts,
        "fractional_xyz": frac,
    }


# ---------------------------------------------------------------------------
# compact radial tabulation
# ---------------------------------------------------------------------------


def _silu_mlp(features, weights, scale, penultimate=False):
    x = features
    for w in weights[:-1]:
        z = x @ w.T
        x = scale * z / (1.0 + np.exp(-z))
    if penultimate:
        return x
    return x @ weights[-1].T


def spline_derivatives(values, h):
    """Knot derivatives by the reference's tridiagonal rule
    (compact_radial.cpp:326-370): not-a-knot-like left end, zero derivative at
    the right end."""
    values = np.asarray(values, dtype=np.float64)
    n = values.shape[-1]
    unknowns = n - 2
    out = np.zeros_like(values)
    flat = values.reshape(-1, n)
    res = out.reshape(-1, n)
    for f in range(flat.shape[0]):
        v = flat[f]
        lower = np.zeros(unknowns)
        diag = np.full(unknowns, 4.0)
        upper = np.zeros(unknowns)
        rhs = np.zeros(unknowns)
        left = 2.0 * (-v[0] + 2.0 * v[1] - v[2]) / h
        upper[0] = 2.0
        rhs[0] = 3.0 * (v[2] - v[0]) / h - left
        for node in range(2, n - 1):
            row = node - 1
            lower[row] = 1.0
            if node + 1 <= n - 2:
                upper[row] = 1.0
            rhs[row] = 3.0 * (v[node + 1] - v[node - 1]) / h
        for row in range(1, unknowns):
            factor = lower[row] / diag[row - 1]
            diag[row] -= factor * upper[row - 1]
            rhs[row] -= factor * rhs[row - 1]
        sol = np.zeros(unknowns)
        sol[-1] = rhs[-1] / diag[-1]
        for row in range(unknowns - 2, -1, -1):
            sol[row] = (rhs[row] - upper[row] * sol[row + 1]) / diag[row]
        d = np.zeros(n)
        d[1 : n - 1] = sol
        d[0] = d[2] + left
        d[-1] = 0.0
        res[f] = d
    return out


def spline_derivatives_fast(values, h):
    """Vectorised form of ``spline_derivatives`` over many functions (same
    elimination, same operation order per function)."""
    v = np.asarray(values, dtype=np.float64)
    n = v.shape[-1]
    u = n - 2
    left = 2.0 * (-v[..., 0] + 2.0 * v[..., 1] - v[..., 2]) / h
    diag = np.full(u, 4.0)
    upper = np.zeros(u)
    lower = np.zeros(u)
    upper[0] = 2.0
    for node in range(2, n - 1):
        row = node - 1
        lower[row] = 1.0
        if node + 1 <= n - 2:
            upper[row] = 1.0
    rhs = np.empty(v.shape[:-1] + (u,))
    rhs[..., 0] = 3.0 * (v[..., 2] - v[..., 0]) / h - left
    for node in range(2, n - 1):
        rhs[..., node - 1] = 3.0 * (v[..., node + 1] - v[..., node - 1]) / h
    for row in range(1, u):
        factor = lower[row] / diag[row - 1]
        diag[row] -= factor * upper[row - 1]
        rhs[..., row] -= factor * rhs[..., row - 1]
    sol = np.empty_like(rhs)
    sol[..., -1] = rhs[..., -1] / diag[-1]
    for row in range(u - 2, -1, -1):
        sol[..., row] = (rhs[..., row] - upper[row] * sol[..., row + 1]) / diag[row]
    d = np.zeros_like(v)
    d[..., 1 : n - 1] = sol
    d[..., 0] = d[..., 2] + left
    d[..., -1] = 0.0
    return d


def compact_radial_grid(model):
    cr = model["compact_radial"]
    grid_min = float(cr["spline_grid_min"])
    points = int(cr["num_spline_points"])
    h = (float(model["r_cut"]) - grid_min) / (points - 1)
    return grid_min, h, points


def agnesi_transform(r, r0, a, q, p):
    """Agnesi distance transform t = 1 / (1 + a s^q / (1 + s^(q - p))),
    s = r / r0 (compact_radial.cpp:238-247)."""
    s = r / r0
    return 1.0 / (1.0 + a * s**q / (1.0 + s ** (q - p)))


def radial_features(model, type_i, type_j):
    """Bessel x polynomial-cutoff features on the spline knots
    (compact_radial.cpp:227-267), shape (knots, num_bessel); with the Agnesi
    transform the Bessel functions take the transformed distance and the
    cutoff the plain one."""
    cr = model["compact_radial"]
    grid_min, h, points = compact_radial_grid(model)
    w = np.asarray(cr["basis"]["weights"], dtype=np.float64)
    pref = float(cr["basis"]["prefactor"])
    rmax = float(cr["cutoff"]["r_max"])
    p = int(cr["cutoff"]["p"])
    tr = cr["distance_transform"]
    r = grid_min + np.arange(points) * h
    t = r
    if tr["type"] == "agnesi":
        radii = np.asarray(tr["covalent_radii"], dtype=np.float64)
        r0 = 0.5 * (radii[type_i] + radii[type_j])
        t = agnesi_transform(r, r0, float(tr["a"]), float(tr["q"]), float(tr["p"]))
    elif tr["type"] != "none":
        raise NotImplementedError(f"distance_transform {tr['type']!r} is not restated")
    scaled = r / rmax
    cut = np.where(
        r < rmax,
        1.0
        - ((p + 1.0) * (p + 2.0) / 2.0) * scaled**p
        + p * (p + 2.0) * scaled ** (p + 1)
        - (p * (p + 1.0) / 2.0) * scaled ** (p + 2),
        0.0,
    )
    return pref * np.sin(w[None, :] * t[:, None]) / t[:, None] * cut[:, None]


def _network(model, name):
    net = model["compact_radial"]["networks"][name]
    shape = net["shape"]
    weights = [
        np.asarray(w, dtype=np.float64).reshape(shape[i + 1], shape[i])
        for i, w in enumerate(net["weights"])
    ]
    return weights, float(net["activation_scale"]), net.get("postprocess", "") == "tanh-square"


def compact_radial_tables(model, type_i, type_j, name):
    """Nodal values and derivatives (functions, knots) of network ``name`` for
    the unordered pair (type_i, type_j); a density network's output is
    postprocessed by tanh(y^2) before the derivative rule
    (compact_radial.cpp:271-289)."""
    _, h, _ = compact_radial_grid(model)
    feats = radial_features(model, type_i, type_j)
    weights, scale, tanh_square = _network(model, name)
    values = _silu_mlp(feats, weights, scale).T.copy()  # (functions, knots)
    if tanh_square:
        values = np.tanh(values * values)
    return values, spline_derivatives_fast(values, h)


# ---------------------------------------------------------------------------
# MACE oracle
# ---------------------------------------------------------------------------


class _Spec(ctypes.Structure):
    _fields_ = [
        ("num_elements", ctypes.c_int), ("channels", ctypes.c_int), ("l_max", ctypes.c_int),
        ("L_max", ctypes.c_int), ("r_cut", ctypes.c_double), ("num_active", ctypes.c_int),
        ("type_to_active", ctypes.c_void_p), ("spline_nodes", ctypes.c_int),
        ("spline_h", ctypes.c_double), ("spline_x0", ctypes.c_double),
        ("r0_values", ctypes.c_void_p), ("r0_derivs", ctypes.c_void_p),
        ("r1_values", ctypes.c_void_p), ("r1_derivs", ctypes.c_void_p),
        ("H0", ctypes.c_void_p), ("A0W", ctypes.c_void_p), ("m0_offsets", ctypes.c_void_p),
        ("m0_degree", ctypes.c_void_p), ("m0_index", ctypes.c_void_p),
        ("m0_coef", ctypes.c_void_p), ("H1W", ctypes.c_void_p), ("num_paths", ctypes.c_int),
        ("num_terms", ctypes.c_int), ("path_l", ctypes.c_void_p), ("path_l1", ctypes.c_void_p),
        ("path_l2", ctypes.c_void_p), ("term_lme", ctypes.c_void_p),
        ("term_row", ctypes.c_void_p), ("term_cg", ctypes.c_void_p), ("A1W", ctypes.c_void_p),
        ("m1_terms", ctypes.c_int), ("m1_degree", ctypes.c_void_p),
        ("m1_index", ctypes.c_void_p), ("m1_coef", ctypes.c_void_p), ("H2M0", ctypes.c_void_p),
        ("H2M1", ctypes.c_void_p), ("readout_q", ctypes.c_void_p),
        ("readout_hidden", ctypes.c_int), ("readout_w1", ctypes.c_void_p),
        ("readout_w2", ctypes.c_void_p), ("readout_scale", ctypes.c_double),
        ("atomic_energies", ctypes.c_void_p),
        ("atomic_numbers", ctypes.c_void_p),
        ("has_zbl", ctypes.c_int), ("zbl_a_exp", ctypes.c_double), ("zbl_a_prefactor", ctypes.c_double),
        ("zbl_c", ctypes.c_double * 4), ("zbl_num_radii", ctypes.c_int), ("zbl_radii", ctypes.c_void_p),
        ("zbl_p", ctypes.c_int),
        ("A0_scaled", ctypes.c_int), ("a0s_values", ctypes.c_void_p), ("a0s_derivs", ctypes.c_void_p),
        ("A1_scaled", ctypes.c_int), ("a1s_values", ctypes.c_void_p), ("a1s_derivs", ctypes.c_void_p),
        ("pre_linear_up", ctypes.c_int), ("H1P0", ctypes.c_void_p),
        ("first_residual", ctypes.c_int), ("residual", ctypes.c_void_p), ("residual_fused", ctypes.c_void_p),
    ]


def _monomial_arrays(monomial_lists):
    deg, idx = [], []
    for m in monomial_lists:
        if not 1 <= len(m) <= 3:
            raise NotImplementedError("oracle restates polynomials of degree 1..3")
        deg.append(len(m))
        idx.append(list(m) + [0] * (3 - len(m)))
    return np.asarray(deg, dtype=np.int32), np.asarray(idx, dtype=np.int32).reshape(-1, 3)


class MaceOracle:
    """CPU restatement of MACECPU for one model and a set of active types."""

    def __init__(self, model: dict, active_types, precision="float32", timed=False):
        mode = model.get("h1_affine_mode")
        if model.get("symmetrix_format_version") != 4 or mode not in ("m0_composite", "pre_linear_up"):
            raise NotImplementedError("the oracle restates format-4 models (m0_composite or pre_linear_up basis)")
        if model.get("has_field_coupling"):
            raise NotImplementedError("the oracle does not restate field coupling")
        pre = mode == "pre_linear_up"
        residual = bool(model.get("first_interaction_residual"))
        if residual and not pre:
            raise ValueError("first-interaction residual models use the pre_linear_up basis")
        self.precision = precision
        self.model = model
        ne = int(model["num_elements"])
        C = int(model["num_channels"])
        lmax, Lmax = int(model["l_max"]), int(model["L_max"])
        nlm, nLM = (lmax + 1) ** 2, (Lmax + 1) ** 2
        self.C, self.lmax, self.Lmax = C, lmax, Lmax
        active = sorted(set(int(t) for t in active_types))
        self.active = active
        t2a = np.full(ne, -1, dtype=np.int32)
        for a, t in enumerate(active):
            t2a[t] = a
        grid_min, h, points = compact_radial_grid(model)
        r0v, r0d, r1v, r1d = [], [], [], []
        a0sv, a0sd, a1sv, a1sd = [], [], [], []
        a0s, a1s = bool(model.get("A0_scaled")), bool(model.get("A1_scaled"))
        for ai in range(len(active)):
            for aj in range(ai, len(active)):
                v, d = compact_radial_tables(model, active[ai], active[aj], "R0")
                r0v.append(v)
                r0d.append(d)
                v, d = compact_radial_tables(model, active[ai], active[aj], "R1")
                r1v.append(v)
                r1d.append(d)
                if a0s:
                    v, d = compact_radial_tables(model, active[ai], active[aj], "A0")
                    a0sv.append(v)
                    a0sd.append(d)
                if a1s:
                    v, d = compact_radial_tables(model, active[ai], active[aj], "A1")
                    a1sv.append(v)
                    a1sd.append(d)
        keep = {}

        def arr(a, dtype=np.float64):
            a = np.ascontiguousarray(a, dtype=dtype)
            keep[id(a)] = a
            return a.ctypes.data

        m0_lists, m0_coef_blocks, m0_off = [], [], [0]
        for LM in range(nLM):
            monos = model["M0_monomials"][str(LM)]
            m0_lists.extend(monos)
            m0_off.append(m0_off[-1] + len(monos))
        m0_deg, m0_idx = _monomial_arrays(m0_lists)
        m0_coef = np.zeros((ne, C, m0_off[-1]))
        for a in range(ne):
            wa = model["M0_weights"][str(a)]
            for LM in range(nLM):
                block = np.asarray([wa[str(LM)][str(k)] for k in range(C)], dtype=np.float64)
                m0_coef[a, :, m0_off[LM] : m0_off[LM + 1]] = block
        m1_deg, m1_idx = _monomial_arrays(model["M1_monomials"])
        m1_coef = np.asarray(
            [[model["M1_weights"][str(a)][str(k)] for k in range(C)] for a in range(ne)],
            dtype=np.float64,
        )
        a1 = [np.ascontiguousarray(w, dtype=np.float64) for w in model["A1_weights"]]
        self._a1 = a1
        a1_ptrs = (ctypes.c_void_p * len(a1))(*[w.ctypes.data for w in a1])
        self._a1_ptrs = a1_ptrs
        spec = _Spec(
            num_elements=ne, channels=C, l_max=lmax, L_max=Lmax, r_cut=float(model["r_cut"]),
            num_active=len(active), type_to_active=arr(t2a, np.int32), spline_nodes=points,
            spline_h=h, spline_x0=grid_min, r0_values=arr(np.stack(r0v)),
            r0_derivs=arr(np.stack(r0d)), r1_values=arr(np.stack(r1v)),
            r1_derivs=arr(np.stack(r1d)), H0=arr(model["H0_weights"]),
            A0W=arr(np.asarray(model["A0_weights"], dtype=np.float64)),
            m0_offsets=arr(m0_off, np.int32), m0_degree=arr(m0_deg, np.int32),
            m0_index=arr(m0_idx, np.int32), m0_coef=arr(m0_coef), H1W=arr(model["H1_weights"]),
            num_paths=len(model["Phi1_l"]), num_terms=len(model["Phi1_lme"]),
            path_l=arr(model["Phi1_l"], np.int32), path_l1=arr(model["Phi1_l1"], np.int32),
            path_l2=arr(model["Phi1_l2"], np.int32), term_lme=arr(model["Phi1_lme"], np.int32),
            term_row=arr(model["Phi1_lelm1lm2"], np.int32),
            term_cg=arr(model["Phi1_clebsch_gordan"]),
            A1W=ctypes.cast(a1_ptrs, ctypes.c_void_p).value, m1_terms=len(m1_deg),
            m1_degree=arr(m1_deg, np.int32), m1_index=arr(m1_idx, np.int32),
            m1_coef=arr(m1_coef),
            H2M0=arr(np.asarray(model["H2_weights_for_H1_pre_linear_up" if pre else "H2_weights_for_M0"])),
            H2M1=arr(model["H2_weights_for_M1"]),
            readout_q=arr(model["readout_1_weights_for_H1_pre_linear_up" if pre else "readout_1_weights_for_M0"]),
            readout_hidden=int(model.get("readout_2_hidden_size", 16)),
            readout_w1=arr(model["readout_2_weights_1"]),
            readout_w2=arr(model["readout_2_weights_2"]),
            readout_scale=float(model["readout_2_scale_factor"]),
            atomic_energies=arr(model["atomic_energies"]),
            atomic_numbers=arr(model["atomic_numbers"], np.int32),
            has_zbl=int(bool(model.get("has_zbl"))),
            A0_scaled=int(a0s), A1_scaled=int(a1s),
        )
        if model.get("has_zbl"):
            radii = np.asarray(model["zbl_covalent_radii"], dtype=np.float64)
            spec.zbl_a_exp = float(model["zbl_a_exp"])
            spec.zbl_a_prefactor = float(model["zbl_a_prefactor"])
            for q, c in enumerate(model["zbl_c"]):
                spec.zbl_c[q] = float(c)
            spec.zbl_num_radii = len(radii)
            spec.zbl_radii = arr(radii)
            spec.zbl_p = int(model["zbl_p"])
        if pre:
            P = np.asarray(model["H1_product_weights"], dtype=np.float64).reshape(Lmax + 1, C, C)
            spec.pre_linear_up = 1
            spec.H1P0 = arr(P[0])
        if residual:
            # fused residual (mace.cpp:2808-2822): residual of element a, row lm,
            # times H1_linear_up_weights of l(lm)
            res = np.asarray(model["H1_first_residual_weights"], dtype=np.float64).reshape(ne, nLM, C)
            U = np.asarray(model["H1_linear_up_weights"], dtype=np.float64).reshape(Lmax + 1, C, C)
            l_of = np.repeat(np.arange(Lmax + 1), 2 * np.arange(Lmax + 1) + 1)
            fused = np.einsum("alk,lko->alo", res, U[l_of])
            spec.first_residual = 1
            spec.residual = arr(res)
            spec.residual_fused = arr(fused)
        if a0s:
            spec.a0s_values = arr(np.stack(a0sv))
            spec.a0s_derivs = arr(np.stack(a0sd))
        if a1s:
            spec.a1s_values = arr(np.stack(a1sv))
            spec.a1s_derivs = arr(np.stack(a1sd))
        lib = _lib(timed)
        self._lib = lib
        suffix = "f32" if precision == "float32" else "f64"
        self._destroy = getattr(lib, f"oracle_mace_destroy_{suffix}")
        self._compute = getattr(lib, f"oracle_mace_compute_{suffix}")
        handle = getattr(lib, f"oracle_mace_create_{suffix}")(ctypes.byref(spec))
        del keep
        if not handle:
            raise ValueError(lib.oracle_mace_last_error().decode())
        self._handle = handle

    def __del__(self):
        if getattr(self, "_handle", None):
            self._destroy(self._handle)
            self._handle = None

    def compute(self, node_types, num_neigh, neigh_indices, neigh_types, xyz, r, num_threads=0):
        """Node energies (N,) and directed edge forces (E, 3), both float64."""
        types = np.ascontiguousarray(node_types, dtype=np.int32)
        nn = np.ascontiguousarray(num_neigh, dtype=np.int32)
        idx = np.ascontiguousarray(neigh_indices, dtype=np.int32)
        nt = np.ascontiguousarray(neigh_types, dtype=np.int32)
        xyz = np.ascontiguousarray(xyz, dtype=np.float64).reshape(-1, 3)
        r = np.ascontiguousarray(r, dtype=np.float64)
        n = len(types)
        energies = np.zeros(n)
        forces = np.zeros((len(r), 3))
        status = self._compute(
            ctypes.c_void_p(self._handle), ctypes.c_int(n), _ptr(types, ctypes.c_int),
            _ptr(nn, ctypes.c_int), _ptr(idx, ctypes.c_int), _ptr(nt, ctypes.c_int),
            _ptr(xyz, ctypes.c_double), _ptr(r, ctypes.c_double), _ptr(energies, ctypes.c_double),
            _ptr(forces, ctypes.c_double), ctypes.c_int(num_threads))
        if status != 0:
            raise RuntimeError(self._lib.oracle_mace_last_error().decode())
        return energies, forces


def harmonics(lmax, xyz):
    """The oracle's harmonics Y (n, num_lm) and gradients dY (n, 3, num_lm)."""
    x = np.ascontiguousarray(xyz, dtype=np.float64).reshape(-1, 3)
    nlm = (lmax + 1) ** 2
    Y = np.zeros((len(x), nlm))
    dY = np.zeros((len(x), 3, nlm))
    _lib().oracle_harmonics(ctypes.c_int(lmax), ctypes.c_longlong(len(x)), _ptr(x, ctypes.c_double),
                            _ptr(Y, ctypes.c_double), _ptr(dY, ctypes.c_double))
    return Y, dY


def spline_eval(h, x0, values, derivs, r):
    """The oracle's Hermite spline set at points r: values, derivatives (n, nfn)."""
    v = np.ascontiguousarray(values, dtype=np.float64)
    d = np.ascontiguousarray(derivs, dtype=np.float64)
    nfn, nodes = v.shape
    rr = np.ascontiguousarray(r, dtype=np.float64)
    out_v = np.zeros((len(rr), nfn))
    out_d = np.zeros((len(rr), nfn))
    _lib().oracle_spline_eval(ctypes.c_double(h), ctypes.c_double(x0), ctypes.c_int(nodes), ctypes.c_int(nfn),
                              _ptr(v, ctypes.c_double), _ptr(d, ctypes.c_double), ctypes.c_longlong(len(rr)),
                              _ptr(rr, ctypes.c_double), _ptr(out_v, ctypes.c_double),
                              _ptr(out_d, ctypes.c_double))
    return out_v, out_d


def zbl_pair(a_exp, a_prefactor, c, covalent_radii, p, Zu, Zv, r):
    """The oracle's ZBL pair term 0.5 V envelope and its r-derivative at r."""
    rr = np.ascontiguousarray(np.atleast_1d(r), dtype=np.float64)
    cc = np.ascontiguousarray(c, dtype=np.float64)
    radii = np.ascontiguousarray(covalent_radii, dtype=np.float64)
    value, grad = np.zeros(len(rr)), np.zeros(len(rr))
    lib = _lib()
    status = lib.oracle_zbl_pair(ctypes.c_double(a_exp), ctypes.c_double(a_prefactor), _ptr(cc, ctypes.c_double),
                                 ctypes.c_int(len(radii)), _ptr(radii, ctypes.c_double), ctypes.c_int(p),
                                 ctypes.c_int(Zu), ctypes.c_int(Zv), ctypes.c_longlong(len(rr)),
                                 _ptr(rr, ctypes.c_double), _ptr(value, ctypes.c_double), _ptr(grad, ctypes.c_double))
    if status != 0:
        raise ValueError(lib.oracle_mace_last_error().decode())
    return value, grad


def poly_eval(monomials, coefficients, x):
    """The oracle's polynomial value and gradient."""
    deg, idx = _monomial_arrays(monomials)
    c = np.ascontiguousarray(coefficients, dtype=np.float64)
    xv = np.ascontiguousarray(x, dtype=np.float64)
    g = np.zeros(len(xv))
    lib = _lib()
    lib.oracle_poly_eval.restype = ctypes.c_double
    f = lib.oracle_poly_eval(ctypes.c_int(len(deg)), _ptr(deg, ctypes.c_int), _ptr(idx, ctypes.c_int),
                             _ptr(c, ctypes.c_double), ctypes.c_int(len(xv)), _ptr(xv, ctypes.c_double),
                             _ptr(g, ctypes.c_double))
    return f, g


def reduce(num_neigh, neigh_indices, forces, xyz, volume):
    """Atom forces (N, 3) and the 3x3 stress from directed edge forces."""
    lib = _lib()
    nn = np.ascontiguousarray(num_neigh, dtype=np.int32)
    idx = np.ascontiguousarray(neigh_indices, dtype=np.int32)
    f = np.ascontiguousarray(forces, dtype=np.float64)
    x = np.ascontiguousarray(xyz, dtype=np.float64)
    n = len(nn)
    atom = np.zeros((n, 3))
    stress = np.zeros(9)
    lib.oracle_reduce(ctypes.c_int(n), _ptr(nn, ctypes.c_int), _ptr(idx, ctypes.c_int),
                      _ptr(f, ctypes.c_double), _ptr(x, ctypes.c_double), ctypes.c_double(volume),
                      _ptr(atom, ctypes.c_double), _ptr(stress, ctypes.c_double))
    return atom, stress.reshape(3, 3)


def voigt(stress):
    """3x3 -> (xx, yy, zz, yz, xz, xy), symmetrised (ASE's convention)."""
    s = np.asarray(stress).reshape(3, 3)
    return np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]),
                     0.5 * (s[0, 2] + s[2, 0]), 0.5 * (s[0, 1] + s[1, 0])])


def graph_inputs(structure, cutoff, atomic_numbers):
    """Neighbour graph (oracle order) and edge geometry of a periodic structure.

    Returns dict with node_types, num_neigh, neigh_indices, neigh_types, xyz, r.
    """
    cell = np.asarray(structure.cell, dtype=np.float64)
    inv = np.linalg.inv(cell)
    g = neighbor_graph(structure.positions, cell, inv, cutoff)
    lookup = {int(z): i for i, z in enumerate(atomic_numbers)}
    types = np.array([lookup[int(z)] for z in structure.numbers], dtype=np.int32)
    receivers = np.repeat(np.arange(len(types)), g["num_neigh"])
    xyz = (
        structure.positions[g["sources"]] - structure.positions[receivers]
        + g["shifts"].astype(np.float64) @ cell
    )
    r = np.linalg.norm(xyz, axis=1)
    return {
        "node_types": types,
        "num_neigh": g["num_neigh"],
        "neigh_indices": g["sources"],
        "neigh_types": types[g["sources"]],
        "xyz": xyz,
        "r": r,
        "receivers": receivers,
        "graph": g,
    }


def evaluate(oracle: MaceOracle, structure, cutoff, num_threads=0):
    """Energy, atom forces and Voigt stress of a periodic structure."""
    gi = graph_inputs(structure, cutoff, oracle.model["atomic_numbers"])
    energies, forces = oracle.compute(gi["node_types"], gi["num_neigh"], gi["neigh_indices"],
                                      gi["neigh_types"], gi["xyz"], gi["r"], num_threads)
    atom, stress = reduce(gi["num_neigh"], gi["neigh_indices"], forces, gi["xyz"],
                          abs(np.linalg.det(structure.cell)))
    return {
        "energy": float(np.sum(energies, dtype=np.float64)),
        "energies": energies,
        "forces": atom,
        "stress": voigt(stress),
        "stress_3x3": stress,
        "directed_forces": forces,
        "inputs": gi,
    }


# ---------------------------------------------------------------------------
# The R1 operator of the reference's plugin ABI, over its packets
# (jit_hip_plugin_abi.h:37-85, 201-221; owners jit_codegen.py:884-1016
# receiver, 1018-1110 source, 1314-1424 edge; spline helpers :2382-2497)
# ---------------------------------------------------------------------------


def hermite_pieces(values, derivs, h):
    """Cubic pieces [intervals][4][functions] (c0 + c1 x + c2 x^2 + c3 x^3,
    x in [0, h] from each interval's left knot) of knot values and
    derivatives [functions][knots] (the Hermite form of
    cubic_spline_set.cpp:20-29)."""
    v = np.asarray(values, dtype=np.float64)
    d = np.asarray(derivs, dtype=np.float64)
    v0, v1, d0, d1 = v[:, :-1], v[:, 1:], d[:, :-1], d[:, 1:]
    c2 = (3.0 * (v1 - v0) / h - 2.0 * d0 - d1) / h
    c3 = (2.0 * (v0 - v1) / h + d0 + d1) / (h * h)
    return np.stack([v0, d0, c2, c3], axis=0).transpose(2, 0, 1).copy()  # [intervals][4][fns]


def plugin_spline(pieces, edge_type, radius, x0, h):
    """Values and slopes [E][functions] of the packet's radial functions:
    evaluation_point (interval clamped to the grid, x = 0 below, x = h above)
    and the cubic piece of each edge's type (jit_codegen.py:2406-2497), in FP64."""
    pieces = np.asarray(pieces, dtype=np.float64)  # [types][intervals][4][fns]
    intervals = pieces.shape[1]
    r = np.asarray(radius, dtype=np.float64)
    iv = np.floor((r - x0) / h).astype(np.int64)
    x = r - x0 - h * iv
    low, high = iv < 0, iv >= intervals
    iv = np.where(low, 0, np.where(high, intervals - 1, iv))
    x = np.where(low, 0.0, np.where(high, h, x))
    c = pieces[np.asarray(edge_type), iv]  # [E][4][fns]
    xc = x[:, None]
    value = c[:, 0] + c[:, 1] * xc + c[:, 2] * xc**2 + c[:, 3] * xc**3
    slope = c[:, 1] + 2.0 * c[:, 2] * xc + 3.0 * c[:, 3] * xc**2
    return value, slope


def plugin_terms(contract):
    """(path, lm1, lm2, lme, coefficient) of a contract's coupling terms; a
    term's path is the one owning its row (rows run path by path,
    (2 l1 + 1)(2 l2 + 1) per path)."""
    row_path = []
    for p, path in enumerate(contract["paths"]):
        row_path += [p] * ((2 * path["edge_l"] + 1) * (2 * path["source_l"] + 1))
    return [(row_path[t["row"]], t["lm1"], t["lm2"], t["lme"], t["coefficient"])
            for t in contract["sparse_coupling"]["terms"]]


def plugin_r1_forward(terms, channels, num_nodes, receivers, sources, active, R, Y, H, num_lme):
    """Receiver owner: output[i][lme][k] = sum over the active edges of i of
    sum_t cg_t R[e][p_t C + k] Y[e][lm1_t] H[src][lm2_t][k]."""
    out = np.zeros((num_nodes, num_lme, channels))
    e = np.flatnonzero(active)
    for p, lm1, lm2, lme, cg in terms:
        contrib = cg * R[e, p * channels:(p + 1) * channels] * Y[e, lm1][:, None] * H[sources[e], lm2]
        np.add.at(out[:, lme], receivers[e], contrib)
    return out


def plugin_r1_source(terms, channels, num_nodes, num_lm2, receivers, sources, active, R, Y, A):
    """Source owner: source_adjoint[s][lm2][k] = sum over the active edges
    from s of sum_t cg_t R[e][p_t C + k] Y[e][lm1_t] A[recv][lme_t][k]."""
    out = np.zeros((num_nodes, num_lm2, channels))
    e = np.flatnonzero(active)
    for p, lm1, lm2, lme, cg in terms:
        contrib = cg * R[e, p * channels:(p + 1) * channels] * Y[e, lm1][:, None] * A[receivers[e], lme]
        np.add.at(out[:, lm2], sources[e], contrib)
    return out


def plugin_r1_edge(terms, channels, receivers, sources, active, xyz, radius, R, dR, Y, dY, H, A):
    """Edge owner: the directed force -dE/dxyz_e of E = <A, output> on each
    active edge: -sum_k sum_t cg_t H[src][lm2_t][k] A[recv][lme_t][k]
    (R'_p Y[lm1] r_hat + R_p grad Y[lm1]); dY [E][3][lm]."""
    force = np.zeros((len(radius), 3))
    e = np.flatnonzero(active)
    u = xyz[e] / radius[e][:, None]
    for p, lm1, lm2, lme, cg in terms:
        w = cg * H[sources[e], lm2] * A[receivers[e], lme]  # [E][C]
        radial = (w * dR[e, p * channels:(p + 1) * channels]).sum(1) * Y[e, lm1]
        angular = (w * R[e, p * channels:(p + 1) * channels]).sum(1)
        force[e] -= radial[:, None] * u + angular[:, None] * dY[e, :, lm1]
    return force
