"""Pins the CPU oracle's correlation, pyramid and lookup (oracle/oracle.c) with
checks that do not restate its code:

* volume: fp64 numpy matmul (closed form), symmetry corr(i,j) = corr(j,i)^T,
  diagonal = alpha*|f_p|^2, the fp16 variant against float16->float64 matmul;
* pyramid: integer-coded volumes (2x2 means of multiples of 4 are exact, so
  bitwise), floor shapes 54->27->13->6, numpy reshape-mean;
* lookup: integer coords make the output a window copy (channel a*7+b with a
  the x offset, bitwise); half-integer coords give exact averages; far-away and
  non-finite coords give zeros; random coords against scipy's zero-padded
  bilinear interpolation (map_coordinates, order=1, mode='grid-constant').
"""
import numpy as np
import pytest
from scipy import ndimage

from oracle import oracle as orc
import workloads as wl


@pytest.fixture(scope="module", autouse=True)
def _build():
    orc.build()


def test_volume_closed_form_and_invariants():
    f = wl.frames(2, C=16, h=6, w=8, seed=11)
    fi, fj = f[0].reshape(16, -1), f[1].reshape(16, -1)
    for alpha in (1 / 16, 1 / np.sqrt(16)):
        vol = orc.corr_volume(fi, fj, alpha)
        ref = alpha * (fi.astype(np.float64).T @ fj.astype(np.float64))
        np.testing.assert_allclose(vol, ref, rtol=1e-6, atol=1e-7)
    # corr(i,j) = corr(j,i)^T, exactly (same fp64 sums, same rounding)
    a = orc.corr_volume(fi, fj, 1 / 16)
    b = orc.corr_volume(fj, fi, 1 / 16)
    np.testing.assert_array_equal(a, b.T)
    # diagonal of corr(f,f) = alpha*|f_p|^2
    s = orc.corr_volume(fi, fi, 0.25)
    np.testing.assert_allclose(np.diag(s), 0.25 * (fi.astype(np.float64) ** 2).sum(0), rtol=1e-6)


def test_volume_f16():
    f = wl.frames(2, C=32, h=4, w=8, seed=12).astype(np.float16)
    vol = orc.corr_volume(f[0].reshape(32, -1), f[1].reshape(32, -1), 1 / 16)
    ref = (f[0].reshape(32, -1).astype(np.float64).T @ f[1].reshape(32, -1).astype(np.float64)) / 16
    np.testing.assert_allclose(vol, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("h,w", [(48, 64), (54, 96), (7, 9)])
def test_pool_shapes_and_exact_integers(h, w):
    rng = np.random.default_rng(0)
    x = (4 * rng.integers(-50, 50, size=(5, h, w))).astype(np.float32)
    cur = x
    for l in range(1, 4):
        nxt = orc.avg_pool_2x2(cur)
        assert nxt.shape == (5, h >> l, w >> l)
        H2, W2 = nxt.shape[1:]
        ref = cur[:, :2 * H2, :2 * W2].reshape(5, H2, 2, W2, 2).astype(np.float64).mean((2, 4))
        if l == 1:  # multiples of 4 -> exact means
            np.testing.assert_array_equal(nxt, ref.astype(np.float32))
        else:
            np.testing.assert_allclose(nxt, ref, rtol=1e-6, atol=1e-6)
        cur = nxt


def _pyr_for(h, w, seed=0, integer=False):
    rng = np.random.default_rng(seed)
    HW = h * w
    if integer:
        vol = (64 * rng.integers(-20, 20, size=(HW, HW))).astype(np.float32)
    else:
        vol = rng.standard_normal((HW, HW)).astype(np.float32)
    return orc.pyramid(vol, h, w)


def test_lookup_integer_coords_is_window_copy():
    h, w = 12, 16
    pyr = _pyr_for(h, w, integer=True)
    rng = np.random.default_rng(1)
    coords = wl.grid_coords(h, w) + rng.integers(-5, 6, size=(2, h * w)).astype(np.float32)
    coords *= 8  # integer at every level (scale 1/2^l, l<=3)
    out = orc.lookup(pyr, coords)
    for l, lev in enumerate(pyr):
        H2, W2 = lev.shape[1:]
        for p in range(0, h * w, 7):
            x0 = int(coords[0, p]) >> l
            y0 = int(coords[1, p]) >> l
            for a in range(7):
                for b in range(7):
                    x, y = x0 - 3 + a, y0 - 3 + b
                    want = lev[p, y, x] if (0 <= x < W2 and 0 <= y < H2) else 0.0
                    assert out[l * 49 + a * 7 + b, p] == want


def test_lookup_half_integer_exact():
    h, w = 6, 8
    pyr = _pyr_for(h, w, integer=True)
    coords = wl.grid_coords(h, w) + 0.5
    out = orc.lookup(pyr[:1], coords)
    lev = pyr[0]
    for p in range(h * w):
        x0, y0 = int(np.floor(coords[0, p])), int(np.floor(coords[1, p]))
        for a in range(7):
            for b in range(7):
                acc = 0.0
                for dxi in (0, 1):
                    for dyi in (0, 1):
                        x, y = x0 - 3 + a + dxi, y0 - 3 + b + dyi
                        if 0 <= x < w and 0 <= y < h:
                            acc += 0.25 * lev[p, y, x]
                assert out[a * 7 + b, p] == np.float32(acc)


def test_lookup_out_of_bounds_and_nonfinite_are_zero():
    h, w = 6, 8
    pyr = _pyr_for(h, w)
    coords = wl.grid_coords(h, w)
    coords[0, 0] = 1e30
    coords[1, 1] = -1e30
    coords[0, 2] = np.nan
    coords[1, 3] = np.inf
    coords[0, 4] = -np.inf
    coords[0, 5] = 100.0
    out = orc.lookup(pyr, coords)
    for p in range(6):
        assert not np.any(out[:, p]), p
    assert np.any(out[:, 6])


def test_lookup_matches_scipy_bilinear():
    """Zero-padded bilinear sampling at (x0-3+a, y0-3+b) for every level."""
    h, w = 12, 16
    pyr = _pyr_for(h, w, seed=5)
    coords = wl.flow_coords(1, h, w, seed=9)[0]
    out = orc.lookup(pyr, coords)
    for l, lev in enumerate(pyr):
        s = 1.0 / (1 << l)
        for p in range(0, h * w, 5):
            x0 = np.float32(coords[0, p] * np.float32(s))
            y0 = np.float32(coords[1, p] * np.float32(s))
            aa, bb = np.meshgrid(np.arange(7), np.arange(7), indexing="ij")
            xs = (x0 - 3 + aa).reshape(-1).astype(np.float64)
            ys = (y0 - 3 + bb).reshape(-1).astype(np.float64)
            ref = ndimage.map_coordinates(lev[p].astype(np.float64), [ys, xs], order=1,
                                          mode="grid-constant", cval=0.0, prefilter=False)
            np.testing.assert_allclose(out[l * 49:(l + 1) * 49, p], ref, rtol=1e-5, atol=1e-5)


def test_corr_batch_composes_volume_pyramid_lookup():
    n, C, h, w = 4, 16, 12, 16
    f = wl.frames(n, C=C, h=h, w=w, seed=2)
    ii, jj = np.array([0, 1, 3], np.int32), np.array([1, 3, 2], np.int32)
    coords = wl.flow_coords(3, h, w, seed=3)
    out = orc.corr_batch(f, ii, jj, coords, 1 / 16)
    for e in range(3):
        vol = orc.corr_volume(f[ii[e]].reshape(C, -1), f[jj[e]].reshape(C, -1), 1 / 16)
        ref = orc.lookup(orc.pyramid(vol, h, w), coords[e])
        np.testing.assert_array_equal(out[e], ref)
