"""GPU: prediction-head selection (reference prediction_heads.hpp:10-89,
selected_head / available_heads of mace_kokkos.cpp:1904-1905): the selected
head's per-head fields replace the top-level ones, checked against the CPU
oracle on the model with that head's fields copied over."""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5
F_TOL = 1e-4
S_TOL = 1e-6


@pytest.fixture(scope="module")
def multihead(tmp_path_factory):
    from symmetrix_amd import synthetic

    model = synthetic.multihead_model(synthetic.random_mace_model("tiny", seed=2), names=("a", "b"), default="a")
    text = synthetic.model_json(model)
    path = tmp_path_factory.mktemp("heads") / "heads.json"
    path.write_text(text)
    return str(path), json.loads(text)


@pytest.mark.parametrize("head", ["", "a", "b"])
def test_selected_head_matches_oracle(oracle_lib, multihead, head):
    from symmetrix_amd import MACEKokkosFloat, Symmetrix, synthetic

    path, model = multihead
    chosen = head or model["prediction_heads"]["default"]
    merged = {k: v for k, v in model.items() if k != "prediction_heads"}
    merged.update(model["prediction_heads"]["parameters"][chosen])
    ev = MACEKokkosFloat(path, head)
    assert ev.selected_head == chosen and ev.available_heads == ["a", "b"]
    s = synthetic.srtio3_supercell(2, sigma=0.1, seed=4)
    got = Symmetrix(path, head=head or None).calculate(s)
    types = synthetic.node_types(s, merged["atomic_numbers"])
    orc = oracle_lib.MaceOracle(merged, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, merged["r_cut"] + 0.5)
    n = len(s)
    print(f"head {chosen!r}: E={got['energy']:.6f}", flush=True)
    assert abs(got["energy"] - want["energy"]) / n < E_TOL
    np.testing.assert_allclose(got["forces"], want["forces"], atol=F_TOL)
    np.testing.assert_allclose(got["stress"], want["stress"], atol=S_TOL)


def test_heads_differ(multihead):
    from symmetrix_amd import Symmetrix, synthetic

    path, _ = multihead
    s = synthetic.srtio3_supercell(2, sigma=0.1, seed=4)
    ea = Symmetrix(path, head="a").calculate(s)["energy"]
    eb = Symmetrix(path, head="b").calculate(s)["energy"]
    assert abs(ea - eb) > 1e-3
