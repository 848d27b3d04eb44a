"""The MACE oracle end to end (CPU): forces and stress against finite
differences of its own energy (the reference method,
symmetrix/test/test_mace.py:687-750, rtol 1e-4 / atol 1e-6 in FP64), global
invariances, FP32 vs FP64 (reference test_mace_streamed_edges.py:556, atol
3e-5), and skin-masked vs exact graphs (reference :4592-4675).

Every test runs on
- the plain tiny model (l_max 2, L_max 1, correlation 2), on one with the
  optional terms of the format (ZBL pair repulsion, A0 and A1 density
  normalisation, Agnesi distance transform) and on a residual-first model in
  the pre_linear_up basis, on SrTiO3 2^3;
- the medium shape (l_max 3, L_max 1, correlation 3, 128 channels; the
  headline model's kernels) on SrTiO3 2^3;
- the wide shape (l_max 3, L_max 2: H1 with an l = 2 block, A1 with L = 2
  blocks, 17 coupling paths and 215 terms, 256 channels) on 12 rigid water
  molecules;
- the scalar shape (l_max 3, L_max 0: scalar H1, 4 coupling paths and 16
  terms, 128 channels; the reference's omat0-small / off23-small models) on
  SrTiO3 2^3;
so the reverse passes of every shape the evaluator compiles are pinned by
finite differences of the forward, and the forward's l = 2 / l = 3 blocks by
rotation invariance (a wrong row, sign or index in one block breaks the
equivariance that energy invariance and force covariance test).
"""

import json

import numpy as np
import pytest

CASES = ["tiny", "tiny+zbl+density+agnesi", "tiny+pre_linear_up+residual", "medium3", "wide", "scalar"]


@pytest.fixture(scope="module", params=CASES)
def case(request):
    import dataclasses

    from symmetrix_amd import synthetic

    preset = request.param.split("+")[0]
    shape = synthetic.PRESETS[preset]
    if request.param == "tiny+zbl+density+agnesi":
        shape = dataclasses.replace(shape, zbl=True, density=("A0", "A1"), agnesi=True)
    elif request.param == "tiny+pre_linear_up+residual":
        shape = dataclasses.replace(shape, h1_basis="pre_linear_up", residual=True)
    model = json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=0)))
    if preset == "wide":
        structure = synthetic.water_box(12, seed=3)
    else:
        structure = synthetic.srtio3_supercell(2, sigma=0.1, seed=3)
    return model, structure


def make(oracle_lib, model, structure, precision="float64"):
    from symmetrix_amd import synthetic

    types = synthetic.node_types(structure, model["atomic_numbers"])
    return oracle_lib.MaceOracle(model, np.unique(types), precision)


def energy(oracle_lib, orc, model, s, skin=0.5):
    return oracle_lib.evaluate(orc, s, model["r_cut"] + skin)["energy"]


def test_forces_match_finite_differences(oracle_lib, case):
    tiny, structure = case
    orc = make(oracle_lib, tiny, structure)
    base = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.5)
    h = 1e-4
    for atom, axis in [(0, 0), (5, 1), (17, 2), (33, 0)]:
        sp, sm = structure.copy(), structure.copy()
        sp.positions[atom, axis] += h
        sm.positions[atom, axis] -= h
        fd = -(energy(oracle_lib, orc, tiny, sp) - energy(oracle_lib, orc, tiny, sm)) / (2 * h)
        assert base["forces"][atom, axis] == pytest.approx(fd, rel=1e-4, abs=1e-6)


def test_directed_forces_are_edge_gradients(oracle_lib, case):
    tiny, structure = case
    orc = make(oracle_lib, tiny, structure)
    res = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.5)
    gi = res["inputs"]
    h = 1e-5
    for e in [0, 7, 123]:
        for axis in range(3):
            xp, xm = gi["xyz"].copy(), gi["xyz"].copy()
            xp[e, axis] += h
            xm[e, axis] -= h
            ep = orc.compute(gi["node_types"], gi["num_neigh"], gi["neigh_indices"], gi["neigh_types"], xp,
                             np.linalg.norm(xp, axis=1))[0].sum()
            em = orc.compute(gi["node_types"], gi["num_neigh"], gi["neigh_indices"], gi["neigh_types"], xm,
                             np.linalg.norm(xm, axis=1))[0].sum()
            assert res["directed_forces"][e, axis] == pytest.approx(-(ep - em) / (2 * h), rel=1e-4, abs=1e-7)


def test_stress_matches_strain_derivative(oracle_lib, case):
    tiny, structure = case
    orc = make(oracle_lib, tiny, structure)
    base = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.5)
    eps = 1e-5
    for i, j in [(0, 0), (1, 1), (0, 2), (1, 2)]:
        def strained(e):
            F = np.eye(3)
            F[i, j] += e / 2
            F[j, i] += e / 2
            s = structure.copy()
            s.positions = structure.positions @ F.T
            s.cell = structure.cell @ F.T
            return s

        fd = (energy(oracle_lib, orc, tiny, strained(eps)) - energy(oracle_lib, orc, tiny, strained(-eps))) / (2 * eps)
        assert base["stress_3x3"][i, j] == pytest.approx(fd / structure.volume, rel=1e-4, abs=1e-8)
    s = base["stress_3x3"]
    np.testing.assert_allclose(s, s.T, atol=1e-9)


def test_forces_sum_to_zero_and_translation_invariance(oracle_lib, case):
    tiny, structure = case
    orc = make(oracle_lib, tiny, structure)
    base = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.5)
    np.testing.assert_allclose(base["forces"].sum(axis=0), 0.0, atol=1e-10)
    moved = structure.copy()
    moved.positions = moved.positions + np.array([0.31, -1.7, 2.2])
    assert energy(oracle_lib, orc, tiny, moved) == pytest.approx(base["energy"], abs=1e-9)


def test_rotation_invariance(oracle_lib, case):
    tiny, structure = case
    # energy invariant and forces covariant under a global rotation of atoms and
    # cell: pins harmonics, coupling tables and polynomial equivariance together
    from symmetrix_amd import irreps

    orc = make(oracle_lib, tiny, structure)
    base = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.5)
    R = irreps.random_rotation(9)
    rot = structure.copy()
    rot.positions = structure.positions @ R.T
    rot.cell = structure.cell @ R.T
    res = oracle_lib.evaluate(orc, rot, tiny["r_cut"] + 0.5)
    assert res["energy"] == pytest.approx(base["energy"], abs=1e-9)
    np.testing.assert_allclose(res["forces"], base["forces"] @ R.T, atol=1e-10)
    np.testing.assert_allclose(res["stress_3x3"], R @ base["stress_3x3"] @ R.T, atol=1e-10)


def test_float32_matches_float64(oracle_lib, case):
    tiny, structure = case
    r64 = oracle_lib.evaluate(make(oracle_lib, tiny, structure, "float64"), structure, tiny["r_cut"] + 0.5)
    r32 = oracle_lib.evaluate(make(oracle_lib, tiny, structure, "float32"), structure, tiny["r_cut"] + 0.5)
    np.testing.assert_allclose(r32["energies"], r64["energies"], atol=3e-5)
    np.testing.assert_allclose(r32["directed_forces"], r64["directed_forces"], atol=3e-5)


def test_skin_masked_graph_equals_exact_graph(oracle_lib, case):
    tiny, structure = case
    orc = make(oracle_lib, tiny, structure)
    exact = oracle_lib.evaluate(orc, structure, tiny["r_cut"])
    skin = oracle_lib.evaluate(orc, structure, tiny["r_cut"] + 0.7)
    assert skin["energy"] == pytest.approx(exact["energy"], abs=1e-10)
    np.testing.assert_allclose(skin["forces"], exact["forces"], atol=1e-12)


def test_rejects_unsupported_models(oracle_lib, case):
    tiny, structure = case
    bad = dict(tiny)
    bad["has_field_coupling"] = True
    with pytest.raises(NotImplementedError):
        make(oracle_lib, bad, structure)
    bad = dict(tiny)
    bad["symmetrix_format_version"] = 2
    with pytest.raises(NotImplementedError):
        make(oracle_lib, bad, structure)
