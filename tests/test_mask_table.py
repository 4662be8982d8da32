"""The tile-mask table's range (corr_split.hip, k_mask_table / tile_mask_of):
the batched correlation looks up a source's target-tile mask by its floored
coordinates in a table over [-32, w + 32) x [-32, h + 32) and takes the mask
as empty outside it. That is exact only if no source outside the range has a
window cell at any level: level l's 8x8 window starts at (f >> l) - 3
(main.cu:1175-1217 samples 7x7 bilinear taps, whose corners span those 8
cells) on a (h >> l) x (w >> l) grid. Checked here by brute force over a
wide band of positions for several map sizes and level counts."""
import numpy as np
import pytest

PAD = 32  # kTabPad


def has_cell(f, n, levels):
    """True where a source floored to f (one axis) has a window cell on an
    axis of n pixels at some level."""
    hit = np.zeros_like(f, dtype=bool)
    for l in range(levels):
        nl = n >> l
        o = (f >> l) - 3
        hit |= (np.maximum(o, 0) <= np.minimum(o + 7, nl - 1)) & (nl > 0)
    return hit


@pytest.mark.parametrize("n", [7, 9, 12, 20, 48, 54, 64, 96, 256])
@pytest.mark.parametrize("levels", [1, 2, 3, 4])
def test_no_cell_outside_the_table(n, levels):
    f = np.arange(-400, n + 400, dtype=np.int64)
    hit = has_cell(f, n, levels)
    assert not hit[(f < -PAD) | (f >= n + PAD)].any()
    # the bound is tight at the deepest level the grid has: cells reach
    # 4 * 2^l pixels before the first pixel
    deep = max(l for l in range(levels) if n >> l > 0)
    reach = 4 << deep
    assert hit[f == -reach].all() and not hit[f == -reach - 1].any()


def test_rows_and_columns_are_independent():
    """A source has a cell at level l iff its window meets the grid in both
    axes, so the 2-D range is the product of the 1-D ones checked above."""
    h, w = 48, 64
    fy, fx = np.meshgrid(np.arange(-60, h + 60), np.arange(-60, w + 60), indexing="ij")
    any2 = np.zeros(fx.shape, bool)
    for l in range(4):
        ox, oy = (fx >> l) - 3, (fy >> l) - 3
        okx = np.maximum(ox, 0) <= np.minimum(ox + 7, (w >> l) - 1)
        oky = np.maximum(oy, 0) <= np.minimum(oy + 7, (h >> l) - 1)
        any2 |= okx & oky
    outside = (fx < -PAD) | (fx >= w + PAD) | (fy < -PAD) | (fy >= h + PAD)
    assert not any2[outside].any()
