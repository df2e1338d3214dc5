"""Multi-block live topology: the s2 grid split into owned strips with a
2-cell halo, one GPU workgroup (ring, hidden state, predictions) per strip.

Same splits as orin/orin/multi_block.py:36-127 (BlockTopo, the balanced
split that gives boundary strips HALO extra owned cells so every strip
processes the same width, and the 2W x 1H / 2W x 2H / 2W x 4H presets for
2 / 4 / 8 blocks), plus n_blocks = 1 (the whole grid, no halo) and 16
(4W x 4H, for the full-resolution grid).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

HALO = 2


@dataclass(frozen=True)
class BlockTopo:
    """Owned and processed (owned +- halo, clamped) s2 ranges of one block."""
    owned_x_lo: int
    owned_x_hi: int
    owned_y_lo: int
    owned_y_hi: int
    proc_x_lo: int
    proc_x_hi: int
    proc_y_lo: int
    proc_y_hi: int

    @property
    def owned(self):
        return (self.owned_x_lo, self.owned_x_hi, self.owned_y_lo, self.owned_y_hi)

    @property
    def proc(self):
        return (self.proc_x_lo, self.proc_x_hi, self.proc_y_lo, self.proc_y_hi)


def balanced_splits(extent: int, n_strips: int, halo: int = HALO) -> List[int]:
    """n_strips + 1 boundaries over [0, extent].  Up to two strips split
    evenly (each touches a boundary, one-sided halo).  From three strips on,
    the two boundary strips own `halo` more cells than a middle strip
    (middle = (extent - 2*halo) // n), the remainder going to the boundary
    strips (the lower one gets the floor half), so processed widths match;
    when middle would be < 1 the split is uniform with the last strip
    taking the rest."""
    if n_strips < 1:
        raise ValueError("n_strips must be >= 1")
    if n_strips == 1:
        return [0, extent]
    if n_strips == 2:
        return [0, extent // 2, extent]
    middle = (extent - 2 * halo) // n_strips
    if middle < 1:
        size = extent // n_strips
        return [i * size for i in range(n_strips)] + [extent]
    corner = middle + halo
    spare = extent - (2 * corner + (n_strips - 2) * middle)
    sizes = [middle] * n_strips
    sizes[0] = corner + spare // 2
    sizes[-1] = corner + spare - spare // 2
    out = [0]
    for s in sizes:
        out.append(out[-1] + s)
    assert out[-1] == extent
    return out


# blocks -> (x strips, y strips); 16 (4 x 4) has no counterpart in the
# reference, whose live runner offers 2, 4 and 8
_PRESETS = {1: (1, 1), 2: (2, 1), 4: (2, 2), 8: (2, 4), 16: (4, 4)}


def grid_topology(n_blocks: int, W2: int, H2: int, halo: int = HALO) -> List[BlockTopo]:
    """Blocks in x-major order (all y strips of the first x strip first),
    owned boxes disjoint and covering the grid."""
    if n_blocks not in _PRESETS:
        raise ValueError(f"unsupported n_blocks={n_blocks}; use 1, 2, 4, 8 or 16")
    nw, nh = _PRESETS[n_blocks]
    xs, ys = balanced_splits(W2, nw, halo), balanced_splits(H2, nh, halo)
    out = []
    for bw in range(nw):
        for bh in range(nh):
            xl, xh, yl, yh = xs[bw], xs[bw + 1], ys[bh], ys[bh + 1]
            out.append(BlockTopo(xl, xh, yl, yh,
                                 max(0, xl - halo), min(W2, xh + halo),
                                 max(0, yl - halo), min(H2, yh + halo)))
    return out
