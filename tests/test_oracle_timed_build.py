"""The oracle's timing build (oracle/liboracle_timed.so: the same restatement
vectorised for x86-64-v3 with -ffast-math, timed by bench.py's CPU baseline)
agrees with the checker build to FP32 rounding, so the baseline times the
same computation the checker pins.  Skipped where the host lacks AVX2/FMA
(bench.py then times the checker build)."""

import json

import numpy as np
import pytest


def _host_has_x86_64_v3():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f" {f}" in flags for f in ("avx2", "fma", "bmi2", "movbe"))


@pytest.mark.skipif(not _host_has_x86_64_v3(), reason="host CPU lacks x86-64-v3 (AVX2/FMA)")
@pytest.mark.parametrize("preset", ["medium", "wide"])
def test_timed_build_equals_checker_to_fp32_rounding(preset):
    from oracle import oracle
    from symmetrix_amd import synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model(preset, seed=1)))
    if preset == "wide":
        s = synthetic.water_box(num_molecules=8, seed=2)
    else:
        s = synthetic.srtio3_supercell(2, sigma=0.05, seed=2)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gi = oracle.graph_inputs(s, model["r_cut"] + 0.5, model["atomic_numbers"])
    args = (gi["node_types"], gi["num_neigh"], gi["neigh_indices"], gi["neigh_types"], gi["xyz"], gi["r"], 2)
    e_ref, f_ref = oracle.MaceOracle(model, np.unique(types), "float32").compute(*args)
    e_fast, f_fast = oracle.MaceOracle(model, np.unique(types), "float32", timed=True).compute(*args)
    n = len(s)
    de = abs(e_fast.sum() - e_ref.sum()) / n
    df = float(np.max(np.abs(f_fast - f_ref)))
    print(f"{preset}: |dE|/atom {de:.2e}, max|df_ij| {df:.2e}")
    assert de < 1e-5 and float(np.max(np.abs(e_fast - e_ref))) < 1e-5
    assert df < 1e-4
    # a different build, not the same library
    assert not np.array_equal(f_fast, f_ref) or not np.array_equal(e_fast, e_ref)
