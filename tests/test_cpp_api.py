"""The C++ facade (include/symmetrix_amd.hpp): the reference's MACEKokkos<float>
method names over the C-ABI (mace_kokkos.hpp:91-97, 339-460, 489-501,
654-710), exercised through the check program built next to the library
(symmetrix-xl_amd/csrc/cpp_api_check.cpp).

- CPU: the header compiles on its own; loader errors reach C++ callers as the
  reference's exception types with the library's message.
- GPU: one periodic evaluation through the facade gives, bit for bit, the
  results of the same library driven from Python, and the model properties
  and prediction heads the Python binding reports."""

import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "symmetrix-xl_amd", "symmetrix_amd", "cpp_api_check")


def _check_program():
    if not os.path.exists(CHECK):
        raise RuntimeError("cpp_api_check is not built: run __graft_entry__.build()")
    return CHECK


def _write_input(path, types, positions, cell, cutoff):
    cell = np.asarray(cell, dtype=np.float64)
    with open(path, "wb") as f:
        f.write(np.int32(len(types)).tobytes())
        f.write(np.asarray(types, dtype=np.int32).tobytes())
        f.write(np.asarray(positions, dtype=np.float64).reshape(-1).tobytes())
        f.write(cell.reshape(-1).tobytes())
        f.write(np.linalg.inv(cell).reshape(-1).tobytes())
        f.write(np.array([cutoff, abs(np.linalg.det(cell))], dtype=np.float64).tobytes())


def _run(model, head, inp, out):
    return subprocess.run([_check_program(), str(model), head, str(inp), str(out)], capture_output=True,
                          text=True, timeout=120)


def test_header_compiles_alone(tmp_path):
    src = tmp_path / "use.cpp"
    src.write_text('#include "symmetrix_amd.hpp"\n'
                   "int main() { return sizeof(symmetrix_amd::MACEKokkosFloat) > 0 ? 0 : 1; }\n")
    r = subprocess.run(["g++", "-std=c++20", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("edit, kind, message", [
    ("malformed", "invalid_argument", "parse error"),
    ("format", "invalid_argument", "format"),
    ("missing", "invalid_argument", "cannot open model file"),
])
def test_loader_errors_reach_cpp_callers(tmp_path, edit, kind, message):
    from symmetrix_amd import synthetic

    model = json.loads(synthetic.model_json(synthetic.random_mace_model("tiny", seed=0)))
    path = tmp_path / "m.json"
    if edit == "malformed":
        path.write_text("{ not json")
    elif edit == "format":
        model["symmetrix_format_version"] = 99
        path.write_text(json.dumps(model))
    s = synthetic.srtio3_supercell(1, sigma=0.0, seed=0)
    inp = tmp_path / "in.bin"
    _write_input(inp, synthetic.node_types(s, model["atomic_numbers"]), s.positions, s.cell, 5.5)
    r = _run(path, "", inp, tmp_path / "out.bin")
    assert r.returncode == 3, (r.returncode, r.stderr)
    assert r.stderr.startswith(kind + ":"), r.stderr
    assert message in r.stderr


@pytest.mark.gpu
def test_facade_matches_the_python_binding(tmp_path):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    base = synthetic.random_mace_model("tiny", seed=3)
    model = synthetic.multihead_model(base, names=("pbe", "r2scan"), default="pbe")
    path = tmp_path / "m.json"
    path.write_text(synthetic.model_json(model))
    loaded = json.loads(path.read_text())
    s = synthetic.srtio3_supercell(3, sigma=0.08, seed=5)
    types = synthetic.node_types(s, loaded["atomic_numbers"])
    cutoff = loaded["r_cut"] + 0.5
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    _write_input(inp, types, s.positions, s.cell, cutoff)
    print(f"C++ facade: {len(s)} atoms, head r2scan", flush=True)
    r = _run(path, "r2scan", inp, out)
    assert r.returncode == 0, r.stderr
    info = r.stdout.split()
    assert float(info[0]) == loaded["r_cut"] and int(info[3]) == 32
    assert info[5] == "r2scan" and info[6:] == ["pbe", "r2scan"]

    raw = out.read_bytes()
    n = len(s)
    f64 = np.frombuffer(raw, dtype=np.float64, count=1 + n + 3 * n + 9)
    energy, energies = f64[0], f64[1:1 + n]
    forces = f64[1 + n:1 + 4 * n].reshape(n, 3)
    stress = f64[1 + 4 * n:].reshape(3, 3)
    off = 8 * (1 + 4 * n + 9)
    e = int(np.frombuffer(raw[off:off + 8], dtype=np.int64)[0])
    directed = np.frombuffer(raw[off + 8:], dtype=np.float64)
    assert directed.size == 3 * e

    ev = MACEKokkosFloat(str(path), "r2scan")
    gen = ev._prepare_periodic_factorized_graph(types, s.positions, s.cell, np.linalg.inv(s.cell),
                                                cutoff)["generation"]
    ev._compute_prepared_factorized_positions(gen, s.positions)
    assert ev._graph_size()[1] == e
    np.testing.assert_array_equal(energies, ev.node_energies)
    np.testing.assert_array_equal(directed, ev.node_forces)
    np.testing.assert_array_equal(forces, ev._reduce_atom_forces(n, None, None, gen))
    np.testing.assert_array_equal(stress, ev._reduce_stress(abs(np.linalg.det(s.cell)), None, gen))
    assert energy == ev._total_energy(gen)
