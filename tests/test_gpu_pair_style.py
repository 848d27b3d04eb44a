"""GPU: the single-rank LAMMPS pair-style driver (sxl_pair_compute,
counterpart of PairSymmetrixMACE::compute_no_domain_decomposition,
pair_symmetrix_mace.cpp:309-441) on a LAMMPS-style full neighbour list with
ghost atoms, special-bond bits and a shuffled ilist, against the calculator
and the CPU oracle on the same structure: energy, forces (ghost forces folded
into local atoms) and the global virial (= -V stress)."""

import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

E_TOL = 1e-5   # eV/atom
F_TOL = 1e-4   # eV/A
S_TOL = 1e-6   # eV/A^3


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from symmetrix_amd import synthetic

    text = synthetic.model_json(synthetic.random_mace_model("tiny", seed=0))
    path = tmp_path_factory.mktemp("pair") / "tiny.json"
    path.write_text(text)
    return str(path), json.loads(text)


def lammps_lists(s, cutoff, seed=0):
    """Local atoms, one shell of periodic ghost images and a full neighbour
    list of the local atoms over all atoms within cutoff (as LAMMPS builds
    with cutoff = force cutoff + skin)."""
    rng = np.random.default_rng(seed)
    n = len(s)
    shifts = [np.array([a, b, c]) for a in (-1, 0, 1) for b in (-1, 0, 1) for c in (-1, 0, 1)
              if (a, b, c) != (0, 0, 0)]
    x = np.concatenate([s.positions] + [s.positions + sh @ s.cell for sh in shifts])
    nall = len(x)
    local_of = np.arange(nall) % n
    species = [38, 22, 8]
    atom_type = np.array([species.index(int(z)) + 1 for z in s.numbers])[local_of]
    firstneigh = [np.zeros(0, np.int32) for _ in range(nall)]
    numneigh = np.zeros(nall, np.int32)
    for i in range(n):
        d = np.linalg.norm(x - x[i], axis=1)
        js = np.nonzero((d < cutoff) & (np.arange(nall) != i))[0]
        rng.shuffle(js)
        js = js.astype(np.int64)
        js[::7] |= 1 << 30  # special-bond bits above NEIGHMASK
        firstneigh[i] = js.astype(np.int32)
        numneigh[i] = len(js)
    ilist = rng.permutation(n).astype(np.int32)
    return ilist, numneigh, firstneigh, x, atom_type, local_of


def test_pair_style_matches_calculator_and_oracle(oracle_lib, tiny):
    from symmetrix_amd import MACEKokkosFloat, Symmetrix, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.08, seed=31)
    n = len(s)
    ilist, numneigh, firstneigh, x, atom_type, local_of = lammps_lists(s, model["r_cut"] + 1.0)
    mace_types = [model["atomic_numbers"].index(z) for z in (38, 22, 8)]
    print(f"pair style: {n} local + {len(x) - n} ghost atoms, {int(numneigh.sum())} list entries", flush=True)
    ev = MACEKokkosFloat(path)
    res = ev._pair_compute(ilist, numneigh, firstneigh, x, atom_type, local_of, mace_types)
    assert np.all(res["f"][n:] == 0.0)  # forces land on local atoms only
    assert np.all(res["eatom"][n:] == 0.0)
    assert res["energy"] == pytest.approx(res["eatom"][:n].sum(), abs=1e-9)

    calc = Symmetrix(path).calculate(s)
    V = s.volume
    sigma = calc["stress"]  # Voigt xx yy zz yz xz xy
    want_virial = -V * np.array([sigma[0], sigma[1], sigma[2], sigma[5], sigma[4], sigma[3]])
    de = abs(res["energy"] - calc["energy"]) / n
    df = float(np.max(np.abs(res["f"][:n] - calc["forces"])))
    dv = float(np.max(np.abs(res["virial"] - want_virial))) / V
    print(f"  vs calculator: |dE|/atom={de:.3e} max|dF|={df:.3e} max|dvirial|/V={dv:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL and dv < S_TOL
    np.testing.assert_allclose(res["eatom"][:n], calc["energies"], atol=E_TOL)

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    assert abs(res["energy"] - want["energy"]) / n < E_TOL
    np.testing.assert_allclose(res["f"][:n], want["forces"], atol=F_TOL)


def test_pair_style_accumulates_and_validates(tiny):
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=32)
    ilist, numneigh, firstneigh, x, atom_type, local_of = lammps_lists(s, model["r_cut"])
    mace_types = [model["atomic_numbers"].index(z) for z in (38, 22, 8)]
    ev = MACEKokkosFloat(path)
    base = ev._pair_compute(ilist, numneigh, firstneigh, x, atom_type, local_of, mace_types)
    prior = np.random.default_rng(0).normal(size=base["f"].shape)
    again = ev._pair_compute(ilist, numneigh, firstneigh, x, atom_type, local_of, mace_types, f=prior)
    np.testing.assert_allclose(again["f"], prior + base["f"], atol=1e-12)
    bad = local_of.copy()
    bad[len(s):] = len(s)  # ghosts mapped to a ghost, not to their local atoms
    with pytest.raises(ValueError, match="not in the local list"):
        ev._pair_compute(ilist, numneigh, firstneigh, x, atom_type, bad, mace_types)
    with pytest.raises(ValueError, match="outside the model"):
        ev._pair_compute(ilist, numneigh, firstneigh, x, atom_type, local_of, [0, 1, 99])


def _kokkos_list(numneigh, firstneigh, layout):
    """The list as a Kokkos 2-D neighbour view [nall][maxneigh]: LayoutRight
    (strides maxneigh, 1) or LayoutLeft (strides 1, nall), padded with -1."""
    nall = len(numneigh)
    width = max(1, int(numneigh.max()))
    table = np.full((nall, width), -1, dtype=np.int32)
    for i, js in enumerate(firstneigh):
        table[i, :len(js)] = js
    if layout == "right":
        return np.ascontiguousarray(table), width, 1
    return np.ascontiguousarray(table.T), 1, nall


@pytest.mark.parametrize("layout", ["right", "left"])
def test_device_pair_entry_equals_the_host_entry_bit_for_bit(oracle_lib, tiny, layout):
    from hip_memory import Hip
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.08, seed=33)
    n = len(s)
    ilist, numneigh, firstneigh, x, atom_type, local_of = lammps_lists(s, model["r_cut"] + 1.0, seed=3)
    nall = len(x)
    mace_types = [model["atomic_numbers"].index(z) for z in (38, 22, 8)]
    prior = np.random.default_rng(1).normal(size=(nall, 3))
    print(f"device pair entry ({layout} layout): {n} local + {nall - n} ghost atoms", flush=True)
    host = MACEKokkosFloat(path)._pair_compute(ilist, numneigh, firstneigh, x, atom_type, local_of, mace_types,
                                               f=prior.copy())
    hip = Hip()
    table, stride_atom, stride_slot = _kokkos_list(numneigh, firstneigh, layout)
    d_f = hip.upload(prior)
    d_eatom = hip.upload(np.full(nall, 7.0))
    ev = MACEKokkosFloat(path)
    dev = ev._pair_compute_device(n, hip.upload(ilist), hip.upload(numneigh), hip.upload(table), stride_atom,
                                  stride_slot, nall, hip.upload(x), hip.upload(atom_type.astype(np.int32)),
                                  hip.upload(local_of.astype(np.int32)), mace_types, d_f, d_eatom)
    f = hip.download(d_f, (nall, 3), np.float64)
    eatom = hip.download(d_eatom, nall, np.float64)
    hip.free_all()
    assert dev["energy"] == host["energy"]
    np.testing.assert_array_equal(dev["virial"], host["virial"])
    np.testing.assert_array_equal(f, host["f"])
    np.testing.assert_array_equal(eatom[ilist], host["eatom"][ilist])
    assert np.all(eatom[n:] == 7.0) and np.all(f[n:] == prior[n:])  # ghosts untouched

    types = synthetic.node_types(s, model["atomic_numbers"])
    orc = oracle_lib.MaceOracle(model, np.unique(types), "float32")
    want = oracle_lib.evaluate(orc, s, model["r_cut"] + 0.5)
    de = abs(dev["energy"] - want["energy"]) / n
    df = float(np.max(np.abs(f[:n] - prior[:n] - want["forces"])))
    print(f"  vs oracle: |dE|/atom={de:.3e} max|dF|={df:.3e}", flush=True)
    assert de < E_TOL and df < F_TOL


def test_device_pair_entry_validates_like_the_host_entry(tiny):
    from hip_memory import Hip
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(2, sigma=0.05, seed=34)
    ilist, numneigh, firstneigh, x, atom_type, local_of = lammps_lists(s, model["r_cut"])
    nall = len(x)
    mace_types = [model["atomic_numbers"].index(z) for z in (38, 22, 8)]
    table, sa, ss = _kokkos_list(numneigh, firstneigh, "right")
    hip = Hip()
    ev = MACEKokkosFloat(path)

    def call(local=local_of, types=mace_types, tab=table, ilist_=ilist):
        return ev._pair_compute_device(len(s), hip.upload(ilist_), hip.upload(numneigh), hip.upload(tab), sa, ss,
                                       nall, hip.upload(x), hip.upload(atom_type.astype(np.int32)),
                                       hip.upload(local.astype(np.int32)), types, hip.alloc(nall * 24))

    bad = local_of.copy()
    bad[len(s):] = len(s)  # ghosts mapped to a ghost, not to their local atoms
    with pytest.raises(ValueError, match="not in the local list"):
        call(local=bad)
    with pytest.raises(ValueError, match="outside the model"):
        call(types=[0, 1, 99])
    wild = table.copy()
    wild[ilist[0], 0] = nall + 5
    with pytest.raises(IndexError, match="neighbour index out of range"):
        call(tab=wild)
    twice = ilist.copy()
    twice[1] = twice[0]
    with pytest.raises(IndexError, match="ilist"):
        call(ilist_=twice)
    call()  # the evaluator is still usable
    hip.free_all()


def test_prepared_device_pair_entry_reuses_its_graph(tiny):
    """The KOKKOS pair style's prepared execution
    (pair_symmetrix_mace_kokkos.cpp:1043-1160): every listed pair an edge,
    those beyond r_cut scaled to it (inactive), the graph rebuilt only when
    neighbor_ago is 0.  With the list of the previous call and moved atoms
    it updates only the edge vectors and matches the filtering entry on the
    same list and positions to FP32 rounding (the scaled pairs change which
    of a receiver's edges share a kernel tile, so the sums run in another
    order); a list that changed without a rebuild is refused, and the next
    call rebuilds."""
    from hip_memory import Hip
    from symmetrix_amd import MACEKokkosFloat, synthetic

    path, model = tiny
    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=41)
    n = len(s)
    ilist, numneigh, firstneigh, x, atom_type, local_of = lammps_lists(s, model["r_cut"] + 1.0, seed=5)
    nall = len(x)
    mace_types = [model["atomic_numbers"].index(z) for z in (38, 22, 8)]
    table, stride_atom, stride_slot = _kokkos_list(numneigh, firstneigh, "right")
    hip = Hip()
    d_ilist, d_table = hip.upload(ilist), hip.upload(table)
    d_type, d_local = hip.upload(atom_type.astype(np.int32)), hip.upload(local_of.astype(np.int32))
    prepared, filtering = MACEKokkosFloat(path), MACEKokkosFloat(path)
    delta = np.random.default_rng(2).normal(scale=0.03, size=(n, 3))
    within = [int(np.sum(np.linalg.norm(x[js & 0x1FFFFFFF] - x[i], axis=1) < model["r_cut"]))
              for i, js in enumerate(firstneigh[:n])]
    print(f"prepared pair entry: {n} local atoms, {int(numneigh.sum())} list entries, {sum(within)} within r_cut",
          flush=True)

    def both(xs, ago, counts=numneigh):
        d_x, d_nn = hip.upload(xs), hip.upload(counts)
        d_fp, d_ff = hip.upload(np.zeros((nall, 3))), hip.upload(np.zeros((nall, 3)))
        d_ep, d_ef = hip.upload(np.zeros(nall)), hip.upload(np.zeros(nall))
        a = prepared._pair_compute_device_prepared(ago, n, d_ilist, d_nn, d_table, stride_atom, stride_slot, nall,
                                                   d_x, d_type, d_local, mace_types, d_fp, d_ep)
        b = filtering._pair_compute_device(n, d_ilist, d_nn, d_table, stride_atom, stride_slot, nall, d_x, d_type,
                                           d_local, mace_types, d_ff, d_ef)
        a.update(f=hip.download(d_fp, (nall, 3), np.float64), eatom=hip.download(d_ep, nall, np.float64))
        b.update(f=hip.download(d_ff, (nall, 3), np.float64), eatom=hip.download(d_ef, nall, np.float64))
        return a, b

    for step, ago in enumerate([0, 1, 2, 3]):
        xs = x + step * delta[local_of]  # ghosts move with their local atoms
        a, b = both(xs, ago)
        print(f"  step {step} (ago {ago}): rebuilt {a['rebuilt']}, E {a['energy']:.8f}", flush=True)
        assert a["rebuilt"] == (ago == 0)
        print(f"    vs filtering entry: |dE| {abs(a['energy'] - b['energy']):.1e}, "
              f"max|dF| {np.max(np.abs(a['f'] - b['f'])):.1e}, max|dW| {np.max(np.abs(a['virial'] - b['virial'])):.1e}",
              flush=True)
        assert abs(a["energy"] - b["energy"]) < 1e-8 * n
        np.testing.assert_allclose(a["virial"], b["virial"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(a["f"], b["f"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(a["eatom"], b["eatom"], rtol=0, atol=1e-6)
    shorter = numneigh.copy()
    shorter[ilist[0]] -= 1
    with pytest.raises(ValueError, match="neighbour list changed"):
        both(x, 4, shorter)
    a, _ = both(x, 5)
    assert a["rebuilt"]
    hip.free_all()
