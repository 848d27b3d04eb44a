"""The R1 plugin's compiled contract constants (csrc/r1_plugin_mpa0_medium.inc)
equal what gen_r1_plugin.py writes from the reference's medium contract
(tests/golden/jit_r1_mace_mpa0_medium_contract.json): fingerprints, channels,
embedding and every coupling coefficient in the compiled shape's term order.
A contract whose terms leave the compiled pattern is refused."""

import importlib.util
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "symmetrix-xl_amd", "csrc")


def _generator():
    spec = importlib.util.spec_from_file_location("gen_r1_plugin", os.path.join(CSRC, "gen_r1_plugin.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _contract(name="jit_r1_mace_mpa0_medium_contract.json"):
    with open(os.path.join(HERE, "golden", name)) as f:
        return json.load(f)


def test_committed_constants_equal_the_generator():
    with open(os.path.join(CSRC, "r1_plugin_mpa0_medium.inc")) as f:
        committed = f.read()
    assert committed == _generator().render(_contract(), "mpa0_medium")


def test_coefficients_follow_the_compiled_term_order():
    gen = _generator()
    contract = _contract()
    order, _ = gen.shape_term_order(3, 1)
    text = gen.render(contract, "mpa0_medium")
    values = [float(v) for v in text.split("kCoefficients[kTerms] = {")[1].split("}")[0].replace("\n", "").split(",")]
    coef = {(t["lm1"], t["lm2"], t["row"], t["lme"]): t["coefficient"] for t in contract["sparse_coupling"]["terms"]}
    assert values == [coef[k] for k in order] and len(values) == 86
    for key in ("generation_fingerprint", "fingerprint", "structure_fingerprint"):
        assert contract[key] in text


def test_a_contract_outside_the_compiled_pattern_is_refused():
    gen = _generator()
    bad = _contract()
    bad["sparse_coupling"]["terms"] = bad["sparse_coupling"]["terms"][:-1]
    with pytest.raises(ValueError, match="pattern"):
        gen.render(bad, "broken")
    with pytest.raises(ValueError, match="paths"):
        gen.render(_contract("jit_r1_mace_mp0b2_large_contract.json") | {"source_harmonics": {"l_max": 1}}, "mixed")


def test_plugin_library_exports_the_query_and_its_descriptor():
    """The built plugin exports the symbol include/symmetrix_amd_r1_plugin.h
    declares; its descriptor is static data, read here without a GPU."""
    import ctypes

    path = os.path.join(os.path.dirname(CSRC), "symmetrix_amd", "libsymmetrix_amd_r1_mpa0_medium.so")
    if not os.path.exists(path):
        pytest.skip("plugin not built (python -c 'import __graft_entry__ as g; g.build()')")
    with open(os.path.join(os.path.dirname(os.path.dirname(CSRC)), "include", "symmetrix_amd_r1_plugin.h")) as f:
        assert "symmetrix_jit_hip_plugin_query_v1(void);" in f.read()
    lib = ctypes.CDLL(path)
    query = lib.symmetrix_jit_hip_plugin_query_v1
    query.restype = ctypes.POINTER(ctypes.c_uint32 * 8)
    head = list(query().contents)
    # abi_version, struct_size (8 u32, 5 strings, 4 i32, 2 strings, 5 i32, 2 pointers), pointer size, byte order,
    # capabilities (forward | coordinate reverse), FP32
    assert head[0] == 1 and head[1] == 8 * 4 + 5 * 8 + 4 * 4 + 2 * 8 + 5 * 4 + 4 + 2 * 8
    assert head[2] == 8 and head[3] == 0x01020304 and head[4] == 3 and head[5] == 1 and head[6] == 4
