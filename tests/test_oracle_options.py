"""Closed-form pins of two model options of the oracle: the Agnesi distance
transform (compact_radial.cpp:150-170, 227-247) and the density
normalisation of A0 / A1 (mace.cpp:1561-1636, 2380-2458;
compact_radial.cpp:271-289).  The GPU runs both against the oracle
(tests/test_gpu_model_options.py); these tests fix the oracle itself by what
the mathematics implies, chosen so that a plausible slip fails:

- Agnesi t(s) = 1 / (1 + a s^q / (1 + s^(q - p))), s = r / r0: with
  lo = min(p, q), hi = max(p, q), t -> 1 - a s^hi as s -> 0 and
  t -> s^(-lo) / a as s -> infinity (the MACE parameters have q < p; an
  exponent sign slip in the inner power, or a dropped outer 1, breaks one of
  them); t(1) = 1 / (1 + a/2); the pair radius r0 is the mean of the two
  covalent radii (not their max, min or geometric mean).  The transform is
  symmetric in p and q -- the identity a s^q / (1 + s^(q-p)) =
  a s^p / (1 + s^(p-q)) -- so a swap of p and q is no error and is asserted
  as such.
- Density: the scaled model's A0 (A1) is the plain model's divided by
  s_i = 1 + sum_j tanh(y(r_ij)^2), y the density network's output.  On a dimer
  and an equilateral trimer at a spline knot (splines exact there) the scaled
  model's energy must equal the plain model's with its R0 network (A1
  weights) divided by s computed here from the network weights (to 1e-10 eV
  in FP64); a missing "1 +", a product for the quotient, tanh(|y|) for
  tanh(y^2) or one neighbour for two must each miss it by more than 1e-8 eV.
"""

import dataclasses
import json

import numpy as np
import pytest

A, Q, P = 1.0805, 0.9183, 4.5791  # the MACE Agnesi parameters


def test_agnesi_asymptotes_and_unit_point(oracle_lib):
    t = oracle_lib.agnesi_transform
    lo, hi = min(P, Q), max(P, Q)
    for s in (0.02, 0.01):  # 1 - t ~ 1e-8..1e-9: well above double rounding
        assert (1.0 - t(s, 1.0, A, Q, P)) / (A * s**hi) == pytest.approx(1.0, rel=1e-5)
    for s in (1e6, 1e7):  # corrections ~ 1 / (a s^lo)
        assert t(s, 1.0, A, Q, P) * A * s**lo == pytest.approx(1.0, rel=1e-4)
    assert t(1.0, 1.0, A, Q, P) == pytest.approx(1.0 / (1.0 + A / 2.0), abs=1e-15)
    # s = r / r0
    assert t(2.4, 1.2, A, Q, P) == pytest.approx(t(2.0, 1.0, A, Q, P), rel=1e-15)
    # the transform is monotone decreasing from 1 to 0
    s = np.linspace(1e-3, 50.0, 2000)
    v = t(s, 1.0, A, Q, P)
    assert v[0] <= 1.0 and np.all(np.diff(v) < 0) and v[-1] > 0.0


def test_agnesi_slips_fail_the_asymptotes(oracle_lib):
    lo, hi = min(P, Q), max(P, Q)
    # an inner exponent p - q (instead of q - p) misses both limits
    def slip(s):
        return 1.0 / (1.0 + A * s**Q / (1.0 + s ** (P - Q)))

    assert abs(slip(1e6) * A * 1e6**lo - 1.0) > 0.5
    assert abs((1.0 - slip(0.01)) / (A * 0.01**hi) - 1.0) > 0.5
    # without the outer 1 the transform diverges at s -> 0 instead of -> 1
    s = 0.01
    assert abs(1.0 / (A * s**Q / (1.0 + s ** (Q - P))) - 1.0) > 1.0


def test_agnesi_is_symmetric_in_p_and_q(oracle_lib):
    s = np.geomspace(1e-3, 1e3, 61)
    np.testing.assert_allclose(oracle_lib.agnesi_transform(s, 1.0, A, Q, P),
                               oracle_lib.agnesi_transform(s, 1.0, A, P, Q), rtol=1e-13)


def _agnesi_model():
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["tiny"], agnesi=True)
    return json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=3)))


def test_agnesi_pair_radius_is_the_mean(oracle_lib):
    model = _agnesi_model()
    radii = model["compact_radial"]["distance_transform"]["covalent_radii"]
    i, j = 0, 2
    assert radii[i] != radii[j]
    got = oracle_lib.radial_features(model, i, j)
    np.testing.assert_array_equal(got, oracle_lib.radial_features(model, j, i))

    def with_radius(r0):
        m = json.loads(json.dumps(model))
        m["compact_radial"]["distance_transform"]["covalent_radii"][1] = r0
        return oracle_lib.radial_features(m, 1, 1)

    np.testing.assert_allclose(got, with_radius(0.5 * (radii[i] + radii[j])), rtol=0, atol=1e-15)
    for wrong in (max(radii[i], radii[j]), min(radii[i], radii[j]), float(np.sqrt(radii[i] * radii[j]))):
        assert np.max(np.abs(got - with_radius(wrong))) > 1e-3


def _density_model(layer, r, y_target=1.3):
    """A density-normalised tiny model whose density network is rescaled (its
    last, linear layer) to output |y| = y_target at distance r, so that the
    divisor is of order 2 and the energy depends on it strongly."""
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["tiny"], density=(layer,))
    model = json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=4)))
    y0 = _network_output(model, layer, r)
    net = model["compact_radial"]["networks"][layer]
    net["weights"][-1] = (np.asarray(net["weights"][-1], dtype=np.float64) * (y_target / abs(y0))).tolist()
    return model


def _network_output(model, name, r):
    """The density network at distance r: features from the oracle's radial
    basis (pinned by its closed forms elsewhere), then a dense SiLU network
    written out here."""
    net = model["compact_radial"]["networks"][name]
    shape = net["shape"]
    weights = [np.asarray(w, dtype=np.float64).reshape(shape[k + 1], shape[k]) for k, w in enumerate(net["weights"])]
    grid_min, h, points = (float(model["compact_radial"]["spline_grid_min"]), None,
                           int(model["compact_radial"]["num_spline_points"]))
    h = (float(model["r_cut"]) - grid_min) / (points - 1)
    k = int(round((r - grid_min) / h))
    x = np.asarray(__import__("oracle.oracle", fromlist=["radial_features"]).radial_features(model, 0, 0))[k]
    scale = float(net["activation_scale"])
    for w in weights[:-1]:
        z = w @ x
        x = scale * z / (1.0 + np.exp(-z))
    return float((weights[-1] @ x)[0])


def _structure(kind, r):
    from symmetrix_amd import synthetic

    if kind == "dimer":
        pos = np.array([[10.0, 10.0, 10.0], [10.0 + r, 10.0, 10.0]])
        numbers = np.array([38, 8])
    else:  # equilateral triangle: every atom has two neighbours at r
        pos = np.array([[10.0, 10.0, 10.0], [10.0 + r, 10.0, 10.0], [10.0 + 0.5 * r, 10.0 + 0.5 * np.sqrt(3) * r, 10.0]])
        numbers = np.array([38, 22, 8])
    return synthetic.Structure(pos, numbers, np.eye(3) * 40.0)


def _energy(oracle_lib, model, s):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float64")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)["energy"]


def _plain(model, layer, factor):
    """The same model without density normalisation, its R0 network (A0) or
    its A1 weights (A1) multiplied by factor."""
    m = json.loads(json.dumps(model))
    m[f"{layer}_scaled"] = False
    del m["compact_radial"]["networks"][layer]
    if layer == "A0":
        last = m["compact_radial"]["networks"]["R0"]["weights"]
        last[-1] = (np.asarray(last[-1], dtype=np.float64) * factor).tolist()
    else:
        m["A1_weights"] = [(np.asarray(w, dtype=np.float64) * factor).tolist() for w in m["A1_weights"]]
    return m


@pytest.mark.parametrize("layer", ["A0", "A1"])
@pytest.mark.parametrize("kind,neighbours", [("dimer", 1), ("trimer", 2)])
def test_density_divides_by_one_plus_the_neighbour_sum(oracle_lib, layer, kind, neighbours):
    from symmetrix_amd import synthetic

    r_cut = synthetic.PRESETS["tiny"].r_cut
    points = synthetic.PRESETS["tiny"].num_spline_points
    grid_min = 1e-12
    h = (r_cut - grid_min) / (points - 1)
    r = grid_min + 150 * h  # a spline knot (about 2.94 A)
    model = _density_model(layer, r)
    assert float(model["compact_radial"]["spline_grid_min"]) == grid_min
    y = _network_output(model, layer, r)
    assert abs(abs(y) - 1.3) < 1e-12
    density = np.tanh(y * y)
    s = 1.0 + neighbours * density
    structure = _structure(kind, r)
    got = _energy(oracle_lib, model, structure)
    want = _energy(oracle_lib, _plain(model, layer, 1.0 / s), structure)
    print(f"{layer} {kind}: y = {y:.6f}, divisor {s:.9f}, E {got:.12f} vs {want:.12f}", flush=True)
    assert got == pytest.approx(want, abs=1e-10)
    # the slips a restatement could make each move the energy at least 100
    # times beyond that (the A1 path moves a dimer's energy least)
    for wrong in (neighbours * density, s, 1.0 + neighbours * np.tanh(abs(y)), 1.0 + density):
        if wrong == s and wrong != 1.0 / s:
            factor = s  # a product for the quotient
        else:
            factor = 1.0 / wrong
        if abs(factor - 1.0 / s) < 1e-12:
            continue  # the trimer's one-neighbour slip only differs from the dimer's divisor
        assert abs(_energy(oracle_lib, _plain(model, layer, factor), structure) - got) > 1e-8
