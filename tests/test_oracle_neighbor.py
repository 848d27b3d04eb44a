"""The CPU oracle's neighbour graph against the reference's known answers,
a brute-force periodic image search, and graph invariants.

Known answers: reference symmetrix/test/test_device_environment.py:168-245.
"""

import itertools

import numpy as np
import pytest


def brute_force_edges(positions, cell, cutoff):
    """All (receiver, source, shift) with |x_s - x_r + shift . cell| <= cutoff,
    excluding self at zero shift (direct enumeration of images)."""
    inv = np.linalg.inv(cell)
    frac = positions @ inv
    reach = [int(np.ceil(cutoff * np.linalg.norm(inv[:, a]))) + 4 for a in range(3)]
    out = set()
    n = len(positions)
    for i in range(n):
        for j in range(n):
            for s in itertools.product(*(range(-r, r + 1) for r in reach)):
                if i == j and s == (0, 0, 0):
                    continue
                # shift that the graph reports is relative to the unwrapped positions
                d = positions[j] - positions[i] + np.asarray(s, dtype=float) @ cell
                if d @ d <= cutoff * cutoff:
                    out.add((i, j, *s))
    return out


def edge_records(g):
    recv = np.repeat(np.arange(len(g["num_neigh"])), g["num_neigh"])
    return {(int(a), int(b), *map(int, s)) for a, b, s in zip(recv, g["sources"], g["shifts"])}


def test_small_graph_known_answer(oracle_lib):
    cell = np.eye(3) * 4.0
    positions = np.array([[0.1, 0.0, 0.0], [0.3, 0.0, 0.0], [3.9, 0.0, 0.0]])
    g = oracle_lib.neighbor_graph(positions, cell, np.linalg.inv(cell), 0.5)
    np.testing.assert_array_equal(g["receiver_offsets"], [0, 2, 4, 6])
    np.testing.assert_array_equal(g["sources"], [2, 1, 2, 0, 0, 1])
    np.testing.assert_array_equal(
        g["shifts"], [[-1, 0, 0], [0, 0, 0], [-1, 0, 0], [0, 0, 0], [1, 0, 0], [1, 0, 0]])
    np.testing.assert_allclose(
        g["fractional_xyz"],
        [[-0.05, 0, 0], [0.05, 0, 0], [-0.1, 0, 0], [-0.05, 0, 0], [0.05, 0, 0], [0.1, 0, 0]],
        atol=1e-15)


def test_zero_edges_and_empty(oracle_lib):
    cell = np.eye(3) * 10.0
    g = oracle_lib.neighbor_graph(np.array([[0.0, 0, 0], [4.0, 4, 4]]), cell, np.linalg.inv(cell), 0.5)
    assert g["sources"].size == 0 and g["shifts"].shape == (0, 3)
    np.testing.assert_array_equal(g["receiver_offsets"], [0, 0, 0])
    e = oracle_lib.neighbor_graph(np.empty((0, 3)), cell, np.linalg.inv(cell), 0.5)
    np.testing.assert_array_equal(e["receiver_offsets"], [0])


def test_invalid_inputs(oracle_lib):
    cell = np.eye(3) * 4.0
    with pytest.raises(ValueError, match="cutoff must be finite and positive"):
        oracle_lib.neighbor_graph(np.zeros((1, 3)), cell, np.linalg.inv(cell), 0.0)
    with pytest.raises(ValueError, match="cell and inverse cell are inconsistent"):
        oracle_lib.neighbor_graph(np.zeros((1, 3)), cell, np.zeros((3, 3)), 1.0)
    with pytest.raises(ValueError, match="positions must be finite"):
        oracle_lib.neighbor_graph(np.array([[np.nan, 0, 0]]), cell, np.linalg.inv(cell), 1.0)


@pytest.mark.parametrize(
    "cell",
    [
        [[3.2, 0.0, 0.0], [0.0, 4.1, 0.0], [0.0, 0.0, 5.3]],
        [[3.2, 0.0, 0.0], [0.7, 4.1, 0.0], [-0.4, 0.6, 5.3]],
    ],
)
def test_matches_brute_force_images(oracle_lib, cell):
    # the reference compares with matscipy on this H4 system
    # (test_device_environment.py:104-165); matscipy is not installed, the
    # brute-force image enumeration is the independent check
    cell = np.asarray(cell)
    frac = np.array([[0.02, 0.15, 0.35], [0.43, 0.21, 0.87], [0.78, 0.72, 0.04], [0.91, 0.47, 0.61]])
    positions = frac @ cell
    positions[0] += cell[0]
    cutoff = 4.7
    g = oracle_lib.neighbor_graph(positions, cell, np.linalg.inv(cell), cutoff)
    assert edge_records(g) == brute_force_edges(positions, cell, cutoff)
    np.testing.assert_array_equal(np.diff(g["receiver_offsets"]), g["num_neigh"])
    recv = np.repeat(np.arange(len(positions)), g["num_neigh"])
    fp = positions @ np.linalg.inv(cell)
    np.testing.assert_allclose(g["fractional_xyz"], fp[g["sources"]] - fp[recv] + g["shifts"], atol=1e-15)


def test_random_triclinic_against_brute_force_and_symmetry(oracle_lib):
    rng = np.random.default_rng(3)
    cell = np.array([[7.5, 0.0, 0.0], [1.1, 6.9, 0.0], [-0.8, 0.9, 8.2]])
    positions = rng.uniform(-3.0, 10.0, size=(18, 3))
    cutoff = 3.9
    g = oracle_lib.neighbor_graph(positions, cell, np.linalg.inv(cell), cutoff)
    rec = edge_records(g)
    assert rec == brute_force_edges(positions, cell, cutoff)
    # (i, j, S) <=> (j, i, -S)
    assert {(j, i, -a, -b, -c) for i, j, a, b, c in rec} == rec
    # determinism
    g2 = oracle_lib.neighbor_graph(positions, cell, np.linalg.inv(cell), cutoff)
    for k in g:
        assert g[k].tobytes() == g2[k].tobytes()


def test_edges_are_receiver_major_and_within_cutoff(oracle_lib):
    from symmetrix_amd import synthetic

    s = synthetic.srtio3_supercell(3, sigma=0.05, seed=1)
    g = oracle_lib.neighbor_graph(s.positions, s.cell, np.linalg.inv(s.cell), 5.5)
    recv = np.repeat(np.arange(len(s)), g["num_neigh"])
    d = s.positions[g["sources"]] - s.positions[recv] + g["shifts"] @ s.cell
    assert np.all(np.linalg.norm(d, axis=1) <= 5.5 + 1e-12)
    assert np.all(np.diff(recv) >= 0)
