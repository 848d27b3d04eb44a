"""The oracle's pre_linear_up basis and first-interaction residual (CPU),
pinned by identities the model format fixes rather than by restating the
oracle's arithmetic:

- basis change (h1_affine_schema.hpp:9-24; reference check
  test_h1_affine.py:352-375): a pre_linear_up model with maps r0, S0_z on
  x = M0_scalar P0 evaluates exactly like the m0_composite model with
  q = P0 r0 and T_z = P0 S0_z on M0_scalar, with the same H1_weights;
- gauge invariance of the split: replacing P_l, U_l, the residual b, r0, S0_z
  by P_l G_l, G_l^-1 U_l, b G_l, G_0^-1 r0, G_0^-1 S0_z leaves H1_weights,
  the fused residual b U and x r0, x S0_z unchanged, so energies, forces and
  stress must not move (a transposed U, a fused/unfused mix-up or a residual
  on the wrong block breaks it);
- isolated atoms (no neighbours: A0 = M0 = M1 = 0): E = E0 + r0 . b0 +
  readout_2(S0_z^T b0) in closed form, which pins the residual on the scalar
  readout input.

All in FP64; the equalities hold to rounding.
"""

import dataclasses
import json
import math

import numpy as np
import pytest


def _split_model(seed=0, residual=True):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["tiny"], h1_basis="pre_linear_up", residual=residual)
    return json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=seed)))


def _evaluate(oracle_lib, model, s, skin=0.5):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float64")
    return oracle_lib.evaluate(orc, s, model["r_cut"] + skin)


def _assert_same(a, b, n):
    assert abs(a["energy"] - b["energy"]) < 1e-9 * n
    np.testing.assert_allclose(a["forces"], b["forces"], atol=1e-9)
    np.testing.assert_allclose(a["stress"], b["stress"], atol=1e-11)


@pytest.fixture(scope="module")
def structure():
    from symmetrix_amd import synthetic

    return synthetic.srtio3_supercell(2, sigma=0.1, seed=5)


def test_pre_linear_up_equals_m0_composite_with_composed_maps(oracle_lib, structure):
    pre = _split_model(seed=1, residual=False)
    C, ne = pre["num_channels"], pre["num_elements"]
    P0 = np.asarray(pre["H1_product_weights"]).reshape(-1, C, C)[0]
    r0 = np.asarray(pre["readout_1_weights_for_H1_pre_linear_up"])
    S0 = np.asarray(pre["H2_weights_for_H1_pre_linear_up"]).reshape(ne, C, C)
    comp = dict(pre)
    for key in ("readout_1_weights_for_H1_pre_linear_up", "H2_weights_for_H1_pre_linear_up",
                "H1_product_weights", "H1_linear_up_weights", "first_interaction_residual"):
        del comp[key]
    comp["h1_affine_mode"] = "m0_composite"
    comp["readout_1_weights_for_M0"] = (P0 @ r0).tolist()
    comp["H2_weights_for_M0"] = [(P0 @ S0[z]).reshape(-1).tolist() for z in range(ne)]
    a = _evaluate(oracle_lib, pre, structure)
    b = _evaluate(oracle_lib, comp, structure)
    _assert_same(a, b, len(structure))
    # and the maps matter: with P0 transposed the results move
    wrong = dict(comp)
    wrong["readout_1_weights_for_M0"] = (P0.T @ r0).tolist()
    assert abs(_evaluate(oracle_lib, wrong, structure)["energy"] - a["energy"]) > 1e-3


def test_split_gauge_invariance_with_residual(oracle_lib, structure):
    A = _split_model(seed=2, residual=True)
    C, ne, Lmax = A["num_channels"], A["num_elements"], A["L_max"]
    nLM = (Lmax + 1) ** 2
    P = np.asarray(A["H1_product_weights"]).reshape(Lmax + 1, C, C)
    U = np.asarray(A["H1_linear_up_weights"]).reshape(Lmax + 1, C, C)
    b = np.asarray(A["H1_first_residual_weights"]).reshape(ne, nLM, C).copy()
    rng = np.random.default_rng(7)
    # a residual on every block, so the l > 0 fused products are exercised too
    # (rotation invariance is not needed for this identity)
    b[:, 1:, :] = rng.normal(size=(ne, nLM - 1, C)) * 0.2
    A = dict(A)
    A["H1_first_residual_weights"] = b.reshape(-1).tolist()
    r0 = np.asarray(A["readout_1_weights_for_H1_pre_linear_up"])
    S0 = np.asarray(A["H2_weights_for_H1_pre_linear_up"]).reshape(ne, C, C)
    G = np.eye(C)[None] + 0.3 * rng.normal(size=(Lmax + 1, C, C)) / math.sqrt(C)
    Gi = np.linalg.inv(G)
    l_of = np.repeat(np.arange(Lmax + 1), 2 * np.arange(Lmax + 1) + 1)
    B = dict(A)
    B["H1_product_weights"] = np.einsum("lij,ljk->lik", P, G).reshape(-1).tolist()
    B["H1_linear_up_weights"] = np.einsum("lij,ljk->lik", Gi, U).reshape(-1).tolist()
    B["H1_first_residual_weights"] = np.einsum("alk,lko->alo", b, G[l_of]).reshape(-1).tolist()
    B["readout_1_weights_for_H1_pre_linear_up"] = (Gi[0] @ r0).tolist()
    B["H2_weights_for_H1_pre_linear_up"] = [(Gi[0] @ S0[z]).reshape(-1).tolist() for z in range(ne)]
    a = _evaluate(oracle_lib, A, structure)
    bb = _evaluate(oracle_lib, B, structure)
    _assert_same(a, bb, len(structure))
    # the residual contributes: without it the energy moves
    C0 = dict(A)
    C0["H1_first_residual_weights"] = np.zeros_like(b).reshape(-1).tolist()
    assert abs(_evaluate(oracle_lib, C0, structure)["energy"] - a["energy"]) > 1e-3


def _isolated_energy(model, z):
    """E0 + r0 . b0 + readout_2(S0_z^T b0) of a node without neighbours."""
    C, ne = model["num_channels"], model["num_elements"]
    t = model["atomic_numbers"].index(z)
    nLM = (model["L_max"] + 1) ** 2
    b0 = np.asarray(model["H1_first_residual_weights"]).reshape(ne, nLM, C)[t, 0]
    r0 = np.asarray(model["readout_1_weights_for_H1_pre_linear_up"])
    S0 = np.asarray(model["H2_weights_for_H1_pre_linear_up"]).reshape(ne, C, C)[t]
    h2 = S0.T @ b0
    W1 = np.asarray(model["readout_2_weights_1"]).reshape(-1, C)
    W2 = np.asarray(model["readout_2_weights_2"])
    zh = W1 @ h2
    silu = zh / (1.0 + np.exp(-zh))
    return model["atomic_energies"][t] + r0 @ b0 + model["readout_2_scale_factor"] * (W2 @ silu)


def test_isolated_atoms_with_residual_closed_form(oracle_lib):
    from symmetrix_amd import synthetic

    model = _split_model(seed=3, residual=True)
    pos = np.array([[1.0, 1.0, 1.0], [13.0, 1.0, 1.0], [1.0, 13.0, 1.0]])
    s = synthetic.Structure(pos, np.array([38, 22, 8]), np.eye(3) * 36.0)
    res = _evaluate(oracle_lib, model, s)
    want = [_isolated_energy(model, z) for z in (38, 22, 8)]
    np.testing.assert_allclose(res["energies"], want, rtol=0, atol=1e-10)
    np.testing.assert_array_equal(res["forces"], np.zeros((3, 3)))
