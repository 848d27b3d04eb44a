"""Seeded synthetic inputs: model JSON writer and structure builders."""

import json

import numpy as np
import pytest


def test_model_json_is_format4_and_deterministic():
    from symmetrix_amd import synthetic

    a = synthetic.model_json(synthetic.random_mace_model("tiny", seed=3))
    b = synthetic.model_json(synthetic.random_mace_model("tiny", seed=3))
    assert a == b
    m = json.loads(a)
    assert m["symmetrix_format_version"] == 4 and m["h1_affine_mode"] == "m0_composite"
    C, lmax, Lmax = m["num_channels"], m["l_max"], m["L_max"]
    assert len(m["A0_weights"]) == 3 and len(m["A0_weights"][0]) == lmax + 1
    assert len(m["A0_weights"][0][0]) == C * C
    assert len(m["H1_weights"]) == (Lmax + 1) * C * C
    assert m["compact_radial"]["networks"]["R1"]["shape"][-1] == len(m["Phi1_l"]) * C
    # weights are float32 values written with 9 significant digits, which
    # round-trip exactly through float32
    w = np.asarray(m["H1_weights"])
    f32 = w.astype(np.float32)
    assert np.all(np.array([float("%.9g" % v) for v in f32.tolist()]) == w)


@pytest.mark.parametrize("preset, paths", [("tiny", 7), ("medium3", 10), ("wide", 17)])
def test_preset_shapes(preset, paths):
    from symmetrix_amd import irreps, synthetic

    shape = synthetic.PRESETS[preset]
    assert len(irreps.r1_paths(shape.l_max, shape.L_max)) == paths


def test_srtio3_supercell():
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(10, sigma=0.0)
    assert len(s) == 5000 and s.volume == pytest.approx((10 * 3.905) ** 3)
    counts = {z: int(np.sum(s.numbers == z)) for z in (38, 22, 8)}
    assert counts == {38: 1000, 22: 1000, 8: 3000}


def test_water_geometry():
    from symmetrix_amd import synthetic

    w = synthetic.water_box(num_molecules=50, seed=1)
    p = w.positions.reshape(-1, 3, 3)
    d1 = np.linalg.norm(p[:, 1] - p[:, 0], axis=1)
    d2 = np.linalg.norm(p[:, 2] - p[:, 0], axis=1)
    cosang = np.sum((p[:, 1] - p[:, 0]) * (p[:, 2] - p[:, 0]), axis=1) / (d1 * d2)
    np.testing.assert_allclose(d1, 0.957, atol=1e-12)
    np.testing.assert_allclose(d2, 0.957, atol=1e-12)
    np.testing.assert_allclose(np.degrees(np.arccos(cosang)), 104.5, atol=1e-9)
    # 1.0 g/cm^3
    mass = 50 * (15.999 + 2 * 1.008) / 6.02214076e23
    assert mass / (w.volume * 1e-24) == pytest.approx(1.0, rel=1e-9)


def test_irregular_box_min_distance():
    from symmetrix_amd import synthetic

    s = synthetic.irregular_box(num_atoms=400, density=0.08, seed=2)
    L = s.cell[0, 0]
    d = s.positions[:, None, :] - s.positions[None, :, :]
    d -= L * np.round(d / L)
    r = np.linalg.norm(d, axis=-1) + np.eye(len(s)) * 100
    assert r.min() >= 1.8
    assert set(np.unique(s.numbers)) <= {1, 6, 7, 8, 13, 14, 22, 26, 29, 38}
