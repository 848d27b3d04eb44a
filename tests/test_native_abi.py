"""The C-ABI library without a GPU: it loads, exports exactly the entry points
declared in include/symmetrix_amd.h, and reports loader errors (which happen
before any device work) with the reference's error classes."""

import ctypes
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "symmetrix_amd.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(sxl_[a-z_0-9]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    from symmetrix_amd import _native

    lib = _native.library()
    names = declared()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name
    assert set(_native.SIGNATURES) == names


def test_stage_names():
    from symmetrix_amd import _native

    lib = _native.library()
    n = lib.sxl_num_stages()
    names = [lib.sxl_stage_name(i).decode() for i in range(n)]
    assert "r1_reverse" in names and "a0_forward" in names and len(set(names)) == n


def _create(path, head=""):
    from symmetrix_amd import _native

    h = ctypes.c_void_p()
    status = _native.library().sxl_create(path.encode(), head.encode(), ctypes.byref(h))
    msg = _native.library().sxl_last_error().decode()
    if status == 0:
        _native.library().sxl_destroy(h)
    return status, msg


def test_missing_model_file_is_invalid_argument():
    status, msg = _create("/nonexistent/model.json")
    assert status == 1 and "cannot open model file" in msg


@pytest.mark.parametrize(
    "change, message",
    [
        ({"symmetrix_format_version": 2}, "format version 4"),
        ({"h1_affine_mode": "other"}, "h1_affine_mode"),
        ({"has_zbl": True}, "zbl_a_exp"),
        ({"has_zbl": True, "zbl_a_exp": 0.3, "zbl_a_prefactor": 0.4543, "zbl_c": [0.2, 0.5, 0.3],
          "zbl_covalent_radii": [0.5] * 100, "zbl_p": 6}, "four screening coefficients"),
        ({"has_zbl": True, "zbl_a_exp": 0.3, "zbl_a_prefactor": 0.4543, "zbl_c": [0.2, 0.5, 0.3, 0.0],
          "zbl_covalent_radii": [0.5] * 10, "zbl_p": 6}, "do not cover"),
        ({"A0_scaled": True}, "A0 network does not match A0_scaled"),
        ({"A1_scaled": True}, "A1 network does not match A1_scaled"),
        ({"radial_representation": "pair-splines"}, "compact radial"),
        ({"l_max": 5}, "L_max <= l_max <= 3"),
        ({"readout_1_weights": [0.0]}, "old-basis"),
        ({"first_interaction_residual": True}, "m0_composite basis cannot represent"),
        ({"h1_affine_mode": "pre_linear_up"}, "must not contain readout_1_weights_for_M0"),
        ({"has_field_coupling": True}, "MACEField coupling is not supported"),
    ],
)
def test_model_validation_errors(tmp_path, change, message):
    from symmetrix_amd import synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model("tiny", seed=0)))
    model.update(change)
    path = tmp_path / "m.json"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path))
    assert status == 1, msg
    assert message in msg


@pytest.mark.parametrize(
    "edit, message",
    [
        (lambda cr: cr["distance_transform"].update({"type": "exponential"}), "unsupported distance transform"),
        (lambda cr: cr["distance_transform"].update({"type": "agnesi", "a": 1.0, "q": 0.9, "p": 4.5,
                                                     "covalent_radii": [1.0]}), "covalent radii do not match"),
        (lambda cr: cr["networks"]["R0"].update({"postprocess": "tanh-square"}), "cannot use postprocessing"),
        (lambda cr: cr["networks"]["R1"].update({"postprocess": "cube"}), "unsupported postprocessing"),
    ],
)
def test_compact_radial_validation_errors(tmp_path, edit, message):
    from symmetrix_amd import synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model("tiny", seed=0)))
    edit(model["compact_radial"])
    path = tmp_path / "m.json"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path))
    assert status == 1, msg
    assert message in msg


def _split_edit(key, value):
    def edit(model):
        if value is None:
            del model[key]
        else:
            model[key] = value
    return edit


@pytest.mark.parametrize(
    "edit, message",
    [
        (_split_edit("H1_product_weights", None), "requires H1_product_weights"),
        (_split_edit("H1_linear_up_weights", None), "requires split H1 weights"),
        (_split_edit("H1_first_residual_weights", [0.0] * 7), "invalid H1 residual extent"),
        (_split_edit("first_interaction_residual", False), "must not contain H1 residual weights"),
        (_split_edit("readout_1_weights_for_H1_pre_linear_up", [0.0] * 3), "must hold num_channels values"),
        (_split_edit("H2_weights_for_H1_pre_linear_up", [[0.0] * 4] * 3), "num_channels^2 values"),
        (_split_edit("H2_weights_for_H1_pre_linear_up", None), "requires readout_1_weights_for_H1_pre_linear_up"),
        (_split_edit("readout_1_weights_for_M0", [0.0]), "must not contain readout_1_weights_for_M0"),
    ],
)
def test_pre_linear_up_validation_errors(tmp_path, edit, message):
    """The reference's format-4 / residual validation (h1_affine_schema.hpp:
    191-258, mace.cpp:2796-2829) on a residual-first pre_linear_up model."""
    import dataclasses

    from symmetrix_amd import synthetic

    shape = dataclasses.replace(synthetic.PRESETS["tiny"], h1_basis="pre_linear_up", residual=True)
    model = json.loads(synthetic.model_json(synthetic.random_mace_model(shape, seed=0)))
    path = tmp_path / "ok.json"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path))
    # a valid model fails only at device creation (no GPU here) or succeeds
    assert "pre_linear_up" not in msg and "residual" not in msg, msg
    edit(model)
    path = tmp_path / "m.json"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path))
    assert status == 1, msg
    assert message in msg


def _multihead(**edits):
    from symmetrix_amd import synthetic

    model = synthetic.multihead_model(synthetic.random_mace_model("tiny", seed=0), names=("a", "b"))
    model = json.loads(synthetic.model_json(model))
    section = model["prediction_heads"]
    for key, value in edits.items():
        if key == "drop_field":
            del section["parameters"]["b"][value]
        else:
            section[key] = value
    return model


@pytest.mark.parametrize(
    "edits, head, message",
    [
        ({}, "c", "Requested prediction head 'c' is unavailable"),
        ({"schema_version": 2}, "", "unsupported schema version"),
        ({"names": ["a", "a"]}, "", "unique non-empty strings"),
        ({"default": "z"}, "", "default must name a stored head"),
        ({"drop_field": "readout_2_weights_2"}, "", "exactly the supported fields"),
    ],
)
def test_prediction_head_validation(tmp_path, edits, head, message):
    """Head selection errors of the reference (prediction_heads.hpp:30-82)."""
    path = tmp_path / "m.json"
    path.write_text(json.dumps(_multihead(**edits)))
    status, msg = _create(str(path), head)
    assert status == 1, msg
    assert message in msg


def test_single_head_file_rejects_a_named_head(tmp_path):
    from symmetrix_amd import synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model("tiny", seed=0)))
    path = tmp_path / "m.json"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path), "x")
    assert status == 1 and "does not identify a prediction head" in msg
    model["head"] = "pbe"
    path.write_text(json.dumps(model))
    status, msg = _create(str(path), "x")
    assert status == 1 and "the JSON contains 'pbe'" in msg


def test_malformed_json(tmp_path):
    path = tmp_path / "m.json"
    path.write_text('{"num_elements": 1, ')
    status, msg = _create(str(path))
    assert status == 1 and "parse error" in msg


def test_null_arguments_are_rejected():
    from symmetrix_amd import _native

    lib = _native.library()
    assert lib.sxl_create(None, None, None) == 1
    assert lib.sxl_stats(None, None) == 1


def test_runtime_lifecycle_without_a_device():
    # the reference's module lifecycle (tools_kokkos.cpp:44-99), in a fresh
    # process that never touches a device: finalization is final -- neither
    # the runtime nor an evaluator can be created after it
    import subprocess
    import sys

    code = """
import sys
sys.path.insert(0, {pkg!r})
import symmetrix_amd as s
assert s._kokkos_default_execution_space() == "HIP"
assert not s._kokkos_is_initialized()
assert s._kokkos_live_object_count() == 0
s._finalize_kokkos()
assert not s._kokkos_is_initialized()
try:
    s.MACEKokkosFloat({model!r})
except RuntimeError as e:
    assert "after Kokkos finalization" in str(e), e
else:
    raise AssertionError("constructed after finalization")
try:
    s._init_kokkos()
except RuntimeError as e:
    assert "after finalization" in str(e), e
else:
    raise AssertionError("initialized after finalization")
assert s._kokkos_live_object_count() == 0
print("lifecycle ok")
""".format(pkg=os.path.join(ROOT, "symmetrix-xl_amd"), model=os.path.join(ROOT, "no_such_model.json"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "lifecycle ok" in out.stdout


def test_reference_workspace_and_policy_properties_exist():
    """The reference's read-only workspace and policy properties that this
    evaluator reports (symmetrix/source/cpp/mace_kokkos.cpp:459-723) are
    properties of MACEKokkosFloat; their values are checked on the GPU."""
    from symmetrix_amd import MACEKokkosFloat

    names = """factorized_graph_generation factorized_ready factorized_tiled_ready
        factorized_fallback_evaluation_count factorized_schedule_build_count factorized_source_owned_reverse
        factorized_jit_ready factorized_jit_launch_count factorized_jit_forward_launch_count
        factorized_jit_reverse_launch_count factorized_workspace_bytes factorized_graph_device_capacity_bytes
        phi1_workspace_bytes phi1_policy readout_workspace_bytes readout_policy edge_geometry_policy
        compact_edge_geometry_bytes execution_geometry_workspace_bytes harmonic_value_bytes
        harmonic_gradient_bytes shuffled_coordinate_bytes scalar_size_bytes
        dual_layer_workspace_planned_receivers dual_layer_workspace_active_receivers
        dual_layer_workspace_planned_edges dual_layer_workspace_active_edges dual_layer_workspace_batch_count
        dual_layer_workspace_bytes dual_layer_workspace_bytes_per_receiver dual_layer_workspace_bytes_per_edge
        dual_layer_schedule_bytes dual_layer_source_segment_count dual_layer_tiled_evaluation_count
        execution_active_receiver_count execution_active_feature_node_count execution_active_edge_count
        execution_planned_receiver_capacity execution_planned_feature_node_capacity
        execution_planned_edge_capacity execution_planned_capacity_bytes execution_capacity_selection_reason
        low_memory low_memory_requested low_memory_policy low_memory_selection_reason
        low_memory_device_free_bytes low_memory_device_total_bytes low_memory_available_bytes
        low_memory_reserve_bytes low_memory_speed_estimated_bytes low_memory_capacity_estimated_bytes
        low_memory_selected_estimated_bytes""".split()
    for name in names:
        assert isinstance(getattr(MACEKokkosFloat, name, None), property), name
