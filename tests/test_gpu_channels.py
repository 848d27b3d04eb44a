"""GPU parity at the channel counts between the tested ones.

The kernels take any channel count C <= 256 that is a multiple of 32: one
thread per channel rounded up to whole waves (the lanes past C idle), GEMM
column tiles of 128 with a partial last tile, message rows of n_LM x C
floats gathered as float4s.  32, 96, 128 and 256 are covered by the other
tests; here C = 160, 192 and 224 on the medium shape (SrTiO3 3^3) and
C = 192 on the wide shape (water), against the CPU oracle at the BASELINE
north-star tolerances.
"""

import dataclasses
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _check(oracle_lib, tmp_path, preset, channels, s, seed):
    from symmetrix_amd import Symmetrix, synthetic

    shape = dataclasses.replace(synthetic.PRESETS[preset], channels=channels)
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=seed))
    model = json.loads(text)
    assert model["num_channels"] == channels
    path = tmp_path / f"{preset}_C{channels}.json"
    path.write_text(text)
    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    got = Symmetrix(str(path)).calculate(s)
    n = len(s)
    de = abs(got["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(got["forces"] - want["forces"])))
    ds = float(np.max(np.abs(got["stress"] - want["stress"])))
    print(f"{preset} C={channels}: {n} atoms  |dE|/atom={de:.3e}  max|dF|={df:.3e}  max|dS|={ds:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL


@pytest.mark.parametrize("channels", [160, 192, 224])
def test_medium_shape_channel_counts(oracle_lib, tmp_path, channels):
    from symmetrix_amd import synthetic

    _check(oracle_lib, tmp_path, "medium3", channels, synthetic.srtio3_supercell(3, sigma=0.1, seed=14), seed=6)


def test_wide_shape_192_channels(oracle_lib, tmp_path):
    from symmetrix_amd import synthetic

    _check(oracle_lib, tmp_path, "wide", 192, synthetic.water_box(num_molecules=40, seed=15), seed=7)
