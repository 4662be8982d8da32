"""Pins of the oracle's update-pass glue (oracle.c, orc_compute_motion ..
orc_ba_edge_set) by hand-worked values, exact arithmetic and numpy's own
routines, chosen so that a wrong plane order, a dropped clamp, a different
summation order, an unfused multiply-add or an off-by-one in the inactive
edge filter fails one of them.

Reference: cuda_slam/main.cu:1246-1301 (compute_motion_kernel,
compute_target_kernel), 2150-2163 (alloc_coords0), 2186-2390
(run_update_pass: per-edge copies, GraphAgg scatter_mean, BA edge set),
nn.cuh:382-385 (scale_add_kernel, built with --use_fast_math).
"""
import numpy as np
import pytest

from oracle import oracle as orc


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


def test_motion_hand_worked_planes_and_clamp():
    # one edge on a 2x3 grid: identity x = [0,1,2,0,1,2], y = [0,0,0,1,1,1]
    c1 = np.array([[[0.5, 2.0, 70.0, -1.0, 1.0, 2.0],
                    [0.0, -80.0, 0.25, 1.0, 3.0, 1.5]]], np.float32)
    tg = np.array([[[1.5, 2.0, 0.0, -1.0, 101.0, 2.0],
                    [0.0, -80.0, 0.25, 2.0, 3.0, 0.5]]], np.float32)
    m = orc.compute_motion(c1, tg, 2, 3)
    np.testing.assert_array_equal(m[0, 0], [0.5, 1.0, 64.0, -1.0, 0.0, 0.0])     # flow x
    np.testing.assert_array_equal(m[0, 1], [0.0, -64.0, 0.25, 0.0, 2.0, 0.5])    # flow y
    np.testing.assert_array_equal(m[0, 2], [1.0, 0.0, -64.0, 0.0, 64.0, 0.0])    # resid x
    np.testing.assert_array_equal(m[0, 3], [0.0, 0.0, 0.0, 1.0, 0.0, -1.0])      # resid y


def test_motion_identity_and_explicit_grid_agree():
    h, w, B = 5, 7, 3
    rng = np.random.default_rng(0)
    gx, gy = np.meshgrid(np.arange(w, dtype=np.float32), np.arange(h, dtype=np.float32))
    c0 = np.broadcast_to(np.stack([gx.ravel(), gy.ravel()]), (B, 2, h * w)).copy()
    # coords1 on the grid and target = coords1: no flow, no residual
    np.testing.assert_array_equal(orc.compute_motion(c0, c0, h, w), 0.0)
    c1 = c0 + rng.normal(0, 10, c0.shape).astype(np.float32)
    tg = c1 + rng.normal(0, 10, c0.shape).astype(np.float32)
    np.testing.assert_array_equal(orc.compute_motion(c1, tg, h, w),
                                  orc.compute_motion(c1, tg, h, w, coords0=c0))


def test_motion_antisymmetry_and_nan():
    h, w = 4, 4
    rng = np.random.default_rng(1)
    a = rng.normal(0, 20, (2, 2, 16)).astype(np.float32)
    b = rng.normal(0, 20, (2, 2, 16)).astype(np.float32)
    # swapping coords1 and coords0 negates the flow planes exactly (IEEE
    # subtraction is sign-symmetric; the clamp is symmetric)
    np.testing.assert_array_equal(orc.compute_motion(a, a, h, w, coords0=b)[:, :2],
                                  -orc.compute_motion(b, b, h, w, coords0=a)[:, :2])
    # fmaxf(NaN, -64) is -64 (IEEE maxNum), so a NaN coordinate clamps to -64
    c = np.zeros((1, 2, 16), np.float32)
    c[0, 0, 3] = np.nan
    m = orc.compute_motion(c, np.zeros_like(c), h, w, coords0=np.zeros_like(c))
    assert m[0, 0, 3] == -64.0 and m[0, 2, 3] == -64.0


def test_target_hand_worked():
    coords = np.array([[[1.0, 2.0], [3.0, 4.0]]], np.float32)
    delta = np.array([[[0.5, -2.0], [1.0, 0.0], [np.nan, np.nan]]], np.float32)
    wt = np.array([[[0.1, 0.2], [0.3, 0.4], [np.nan, np.nan]]], np.float32)
    t, wo = orc.compute_target(coords, delta, wt)
    np.testing.assert_array_equal(t, [[[1.5, 0.0], [4.0, 4.0]]])  # third plane ignored
    np.testing.assert_array_equal(wo, np.float32([[[0.1, 0.2], [0.3, 0.4]]]))


def test_gather_scatter_match_numpy_indexing():
    rng = np.random.default_rng(2)
    src = rng.normal(size=(9, 3, 5)).astype(np.float32)
    idx = np.array([4, 0, 8, 4, 2], np.int32)
    np.testing.assert_array_equal(orc.gather_rows(src, idx), src[idx])
    np.testing.assert_array_equal(orc.gather_rows(src, None, n=4), src[:4])
    perm = rng.permutation(9).astype(np.int32)
    dst = orc.scatter_rows(np.zeros_like(src), src, perm)
    ref = np.zeros_like(src)
    ref[perm] = src
    np.testing.assert_array_equal(dst, ref)
    # scatter undoes gather for a permutation
    np.testing.assert_array_equal(orc.scatter_rows(np.zeros_like(src), src[perm], perm), src)


def test_scatter_mean_power_of_two_counts_are_exact_means():
    rng = np.random.default_rng(3)
    ii = np.array([5, 2, 5, 9, 2, 5, 5, 2, 2, 1], np.int32)  # counts 4, 4, 1, 1
    src = rng.integers(-1000, 1000, size=(10, 2, 6)).astype(np.float32)
    dst, act = orc.scatter_mean(src, ii)
    np.testing.assert_array_equal(act, np.unique(ii))
    for a, k in enumerate(act):
        np.testing.assert_array_equal(dst[a], src[ii == k].astype(np.float64).mean(0))


def test_scatter_mean_is_one_fused_multiply_add_on_the_edge_order_sum():
    # count 3: dst = fma(inv - 1, S, S), inv = fl(1/3); with integer S the
    # product (inv - 1) * S and the sum are exact in fp64, so rounding the
    # fp64 value once to fp32 is the fused result
    inv = np.float32(1.0) / np.float32(3.0)
    a = np.float32(inv - np.float32(1.0))
    S = np.arange(1, 65, dtype=np.float32)
    fused = (np.float64(a) * S.astype(np.float64) + S.astype(np.float64)).astype(np.float32)
    unfused = (a * S) + S  # fp32 product rounded, then the sum
    assert np.any(fused != unfused)  # the sample tells the two apart
    src = np.stack([S, np.zeros_like(S), np.zeros_like(S)])[:, None, :]
    dst, act = orc.scatter_mean(src, np.array([7, 7, 7], np.int32))
    np.testing.assert_array_equal(act, [7])
    np.testing.assert_array_equal(dst[0, 0], fused)
    # edge order: 1e8 + 1 rounds back to 1e8 in fp32, so the edge-order sum
    # of [1e8, 1, -1e8] is 0 (another order would give 1)
    src = np.array([1e8, 1.0, -1e8], np.float32).reshape(3, 1)
    dst, _ = orc.scatter_mean(src, np.array([0, 0, 0], np.int32))
    assert dst[0, 0] == 0.0


def _rows(n, hw, base):
    # row e holds base + e everywhere: shows which row went where
    return (base + np.arange(n, dtype=np.float32))[:, None, None] * np.ones((1, 2, hw),
                                                                            np.float32)


def test_ba_edge_set_filter_boundary_order_and_rows():
    hw = 3
    ii, jj = np.array([6, 7, 5], np.int32), np.array([7, 6, 6], np.int32)
    ii_in = np.array([2, 1, 3, 2, 9, 4], np.int32)
    jj_in = np.array([3, 4, 2, 1, 2, 5], np.int32)
    t, w = _rows(3, hw, 0), _rows(3, hw, 100)
    ti, wi = _rows(6, hw, 10), _rows(6, hw, 110)
    r = orc.ba_edge_set(ii, jj, ii_in, jj_in, t, w, ti, wi, num_keyframes=8, forced_t0=5)
    # t0 - 3 = 2: (2,3) kept, (1,4) ii below, (3,2) kept, (2,1) jj below, (9,2) kept, (4,5) kept
    keep = [0, 2, 4, 5]
    assert r["t0"] == 5
    np.testing.assert_array_equal(r["ii"], np.r_[ii, ii_in[keep]])
    np.testing.assert_array_equal(r["jj"], np.r_[jj, jj_in[keep]])
    np.testing.assert_array_equal(r["target"][:, 0, 0], np.r_[0, 1, 2, 10 + np.array(keep)])
    np.testing.assert_array_equal(r["weight"][:, 1, 2], np.r_[100, 101, 102, 110 + np.array(keep)])


def test_ba_edge_set_dynamic_t0_and_switches():
    hw = 2
    e = np.zeros(0, np.int32)
    ii, jj = np.array([4, 3, 6], np.int32), np.array([5, 4, 7], np.int32)
    t, w = _rows(3, hw, 0), _rows(3, hw, 0)
    empty = np.zeros((0, 2, hw), np.float32)
    r = orc.ba_edge_set(ii, jj, e, e, t, w, empty, empty, num_keyframes=8)
    assert r["t0"] == 4 and len(r["ii"]) == 3  # max(1, min(ii) + 1)
    r = orc.ba_edge_set(np.array([0], np.int32), np.array([1], np.int32), e, e, t[:1], w[:1],
                        empty, empty, num_keyframes=8)
    assert r["t0"] == 1
    r = orc.ba_edge_set(e, e, e, e, empty, empty, empty, empty, num_keyframes=8)
    assert r["t0"] == 9 and len(r["ii"]) == 0
    # use_inactive off: the active set alone even with eligible inactive edges
    r = orc.ba_edge_set(ii, jj, np.array([5], np.int32), np.array([6], np.int32), t, w,
                        _rows(1, hw, 9), _rows(1, hw, 9), num_keyframes=8, use_inactive=False)
    np.testing.assert_array_equal(r["ii"], ii)
