"""Launch shapes of small graphs, whose receivers would leave most SIMDs idle
with one workgroup per receiver: the layer-0 forward in 64-channel slices
whose four waves split each receiver's edges (LayerArgs::a0_slices, chosen
at up to one receiver wave per SIMD; SXL_A0_FORWARD_SLICES=1 / 0 forces it),
the reverse edge kernels in 16-edge tiles (up to ten receiver waves per
compute unit) and the node kernels in one-node workgroups (up to one wave per
SIMD).  The sliced layer-0 forward sums a receiver's edges in
another order than the one-workgroup kernel, so it is checked against the
CPU oracle (FP32 tolerances) on the medium shape, with every model option
(A0 density term, ZBL, Agnesi, pre_linear_up, residual), on the unfolded
layer-0 path and on the wide shape (four slices), and against the unsliced
kernel within FP32 rounding."""

import dataclasses
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


def _model(tmp_path, preset, **options):
    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS[preset], **options)
    text = synthetic.model_json(synthetic.random_mace_model(shape, seed=6))
    path = tmp_path / f"{preset}.json"
    path.write_text(text)
    return str(path), json.loads(text)


def _evaluate(path, model, s):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    ev = MACEKokkosFloat(path)
    types = synthetic.node_types(s, model["atomic_numbers"])
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                model["r_cut"] + 0.5)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    n = len(s)
    return {
        "energies": ev.node_energies.copy(),
        "forces": ev._reduce_atom_forces(n, None, None, gen),
        "stress": ev._reduce_stress(s.volume, None, gen),
        "workspace": ev._workspace(),
    }


def test_small_and_large_graph_launch_choices(tmp_path):
    from symmetrix_amd import synthetic

    path, model = _model(tmp_path, "medium3")
    small = _evaluate(path, model, synthetic.srtio3_supercell(3, sigma=0.05, seed=1))["workspace"]
    print(f"135 atoms: {small}", flush=True)
    assert small["a0_forward_slices"] == 2 and small["r1_forward_slices"] == 2 and small["edge_tile"] == 16
    large = _evaluate(path, model, synthetic.srtio3_supercell(8, sigma=0.05, seed=1))["workspace"]
    print(f"2,560 atoms: {large}", flush=True)
    assert large["a0_forward_slices"] == 1 and large["r1_forward_slices"] == 1 and large["edge_tile"] == 0


@pytest.mark.parametrize("case", ["medium3", "all_options", "unfolded", "wide"])
def test_sliced_layer0_forward_matches_oracle(oracle_lib, tmp_path, monkeypatch, case):
    from symmetrix_amd import synthetic

    if case == "all_options":
        path, model = _model(tmp_path, "medium3", zbl=True, density=("A0",), agnesi=True,
                             h1_basis="pre_linear_up", residual=True)
    else:
        path, model = _model(tmp_path, "wide" if case == "wide" else "medium3")
    if case == "unfolded":
        monkeypatch.setenv("SXL_A0_UNFOLDED", "1")
    s = synthetic.water_box(num_molecules=45, seed=2) if case == "wide" else \
        synthetic.srtio3_supercell(3, sigma=0.05, seed=2)
    n = len(s)
    monkeypatch.setenv("SXL_A0_FORWARD_SLICES", "1")
    sliced = _evaluate(path, model, s)
    assert sliced["workspace"]["a0_forward_slices"] == model["num_channels"] // 64
    monkeypatch.setenv("SXL_A0_FORWARD_SLICES", "0")
    whole = _evaluate(path, model, s)
    assert whole["workspace"]["a0_forward_slices"] == 1
    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    de = abs(sliced["energies"].sum() - want["energy"]) / n
    df = float(np.max(np.abs(sliced["forces"] - want["forces"])))
    ds = float(np.max(np.abs(sliced["stress"] - want["stress_3x3"])))
    dn = float(np.max(np.abs(sliced["energies"] - whole["energies"])))
    dw = float(np.max(np.abs(sliced["forces"] - whole["forces"])))
    print(f"{case}: {n} atoms; vs oracle |dE|/atom={de:.2e} max|dF|={df:.2e} max|dS|={ds:.2e}; "
          f"vs unsliced max|dE_i|={dn:.2e} max|dF|={dw:.2e}", flush=True)
    assert de < E_TOL and df < F_TOL and ds < S_TOL
    scale = max(1.0, float(np.max(np.abs(whole["energies"]))))
    assert dn < 1e-5 * scale and dw < 1e-4


@pytest.mark.parametrize("case", ["tiny", "medium3", "all_options", "wide", "wide300"])
def test_one_node_blocks_equal_wider_blocks(tmp_path, monkeypatch, case):
    """The node kernels (M0 forward and reverse, readout) of launches with at
    most one wave per SIMD run one node per workgroup (SXL_NODE_BLOCK=1 / 0
    forces it); each node's terms are evaluated alone in either form, so the
    results are the same bit for bit.  wide300: the wide shape on 300 atoms,
    whose wider blocks are the eight-node M0 forward and readout blocks of
    large graphs."""
    from symmetrix_amd import synthetic

    if case == "all_options":
        path, model = _model(tmp_path, "medium3", zbl=True, density=("A0", "A1"), agnesi=True,
                             h1_basis="pre_linear_up", residual=True)
    else:
        path, model = _model(tmp_path, "wide" if case == "wide300" else case)
    if case.startswith("wide"):
        s = synthetic.water_box(num_molecules=100 if case == "wide300" else 45, seed=3)
    else:
        s = synthetic.srtio3_supercell(3, sigma=0.05, seed=3)
    monkeypatch.setenv("SXL_NODE_BLOCK", "1")
    one = _evaluate(path, model, s)
    monkeypatch.setenv("SXL_NODE_BLOCK", "0")
    wide = _evaluate(path, model, s)
    print(f"{case}: {len(s)} atoms; max |dE_i| {np.max(np.abs(one['energies'] - wide['energies'])):.1e}",
          flush=True)
    for key in ("energies", "forces", "stress"):
        assert np.array_equal(one[key], wide[key])
