"""Host rules of the calculator's neighbour-graph reuse (CPU): the
cell-change validity bound of the reference (calculator.py:2855-2877)."""

import numpy as np
import pytest


def test_unchanged_cell_reduces_to_half_skin():
    from symmetrix_amd.calculator import topology_valid

    cell = np.diag([10.0, 11.0, 12.0])
    assert topology_valid(cell, cell, 0.25, 5.0, 0.5)
    assert not topology_valid(cell, cell, 0.2501, 5.0, 0.5)


@pytest.mark.parametrize("scale", [0.95, 0.99, 1.0, 1.05])
def test_isotropic_scaling_bound(scale):
    from symmetrix_amd.calculator import topology_valid

    build = np.eye(3) * 10.0
    cell = build * scale
    # contraction = 1/scale: valid iff (1/scale) (rc + 2d) <= rc + skin
    rc, skin, d = 5.0, 0.5, 0.1
    assert topology_valid(cell, build, d, rc, skin) == ((rc + 2 * d) / scale <= rc + skin)


def test_shear_uses_the_spectral_norm():
    from symmetrix_amd.calculator import topology_valid

    build = np.eye(3) * 10.0
    shear = build.copy()
    shear[1, 0] = 1.5  # second lattice vector tilted
    contraction = np.linalg.norm(np.linalg.solve(shear, build), 2)
    assert contraction > 1.0
    rc = 5.0
    skin = (contraction - 1.0) * rc
    assert topology_valid(shear, build, 0.0, rc, skin * 1.001)
    assert not topology_valid(shear, build, 0.0, rc, skin * 0.999)


def test_singular_or_nonfinite_cells_are_invalid():
    from symmetrix_amd.calculator import topology_valid

    build = np.eye(3) * 10.0
    assert not topology_valid(np.zeros((3, 3)), build, 0.0, 5.0, 0.5)
    assert not topology_valid(build, build, float("nan"), 5.0, 0.5)
