"""Multi-block live topology (orin/orin/multi_block.py:36-127).

No reference test covers it; the splits are pinned by hand-worked cases
and by the properties the reference's docstring states: owned boxes are
disjoint and cover the grid, processed windows are owned +- 2 clamped, and
from three strips on every strip processes the same width when the extent
divides evenly.
"""
import numpy as np
import pytest

from ssla_hip.topology import HALO, balanced_splits, grid_topology


@pytest.mark.parametrize("extent,n,want", [
    (20, 1, [0, 20]),
    (20, 2, [0, 10, 20]),
    (21, 2, [0, 10, 21]),
    (16, 4, [0, 5, 8, 11, 16]),            # middle 3, corner 3 + 2
    (120, 4, [0, 31, 60, 89, 120]),        # 640x480 s2 height
    (19, 4, [0, 6, 9, 12, 19]),            # spare 3: lower corner +1, upper +2
    (5, 4, [0, 1, 2, 3, 5]),               # middle 0: uniform, last takes the rest
    (12, 3, [0, 5, 7, 12]),
])
def test_balanced_splits_cases(extent, n, want):
    assert balanced_splits(extent, n) == want


@pytest.mark.parametrize("extent,n", [(16, 3), (16, 4), (40, 4), (120, 4), (64, 6)])
def test_equal_processed_width_when_even(extent, n):
    s = balanced_splits(extent, n)
    if (extent - 2 * HALO) % n:
        pytest.skip("remainder goes to the corners")
    widths = [min(extent, s[i + 1] + HALO) - max(0, s[i] - HALO) for i in range(n)]
    assert len(set(widths)) == 1, widths


@pytest.mark.parametrize("nb,W2,H2", [(1, 20, 16), (2, 20, 16), (4, 20, 16), (8, 20, 16),
                                      (8, 160, 120), (16, 160, 120)])
def test_grid_topology_covers_grid(nb, W2, H2):
    topo = grid_topology(nb, W2, H2)
    assert len(topo) == nb
    cover = np.zeros((H2, W2), int)
    for t in topo:
        cover[t.owned_y_lo:t.owned_y_hi, t.owned_x_lo:t.owned_x_hi] += 1
        assert t.proc == (max(0, t.owned_x_lo - HALO), min(W2, t.owned_x_hi + HALO),
                          max(0, t.owned_y_lo - HALO), min(H2, t.owned_y_hi + HALO))
    assert np.all(cover == 1)
    # x-major order: 8 blocks = 2 x-strips of 4 y-strips
    if nb == 8:
        assert [t.owned_x_lo for t in topo] == [0] * 4 + [W2 // 2] * 4


def test_grid_topology_rejects_other_counts():
    with pytest.raises(ValueError):
        grid_topology(3, 20, 16)
