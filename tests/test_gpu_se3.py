"""GPU parity of the SE3 reprojection kernels (cuda_slam/se3.cuh) through the
C ABI against the CPU oracle on identical seeded inputs.

Bars: valid masks, retraction indices and clamps bitwise; projected
coordinates and frame distances within helpers.TOL = 1e-4 relative to
max(|r|, rms(r)); fp64-evaluated pose retraction within 1e-6.
"""
import numpy as np
import pytest

from helpers import TOL, Pins, announce, assert_close_rel, assert_valid_mask, gpu_or_fail
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


@pytest.mark.parametrize("trans_sigma", [0.1, 1.0])
def test_projmap(slk, trans_sigma):
    """trans_sigma 0.1: the BA window (every pixel valid); 1.0: translations
    that push ~21% of the homogeneous depths below 0.25, so the mask is mixed
    and is checked exactly outside the fp32 rounding band of the threshold."""
    announce(f"projmap 48 edges trans_sigma={trans_sigma}")
    p = wl.ba_problem(seed=3 if trans_sigma == 0.1 else 13, trans_sigma=trans_sigma)
    h, w = 48, 64
    M = len(p["ii"])
    d = {k: slk.DeviceArray.from_host(p[k]) for k in ("poses", "disps", "intr", "ii", "jj")}
    coords = slk.DeviceArray((M, h, w, 2))
    valid = slk.DeviceArray((M, h, w))
    slk.check(slk.lib().slk_projmap(d["poses"].ptr, d["disps"].ptr, d["intr"].ptr, d["ii"].ptr,
                                    d["jj"].ptr, coords.ptr, valid.ptr, M, h, w, None))
    slk.hip().sync()
    rc, rv = orc.projmap(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], h, w)
    assert_close_rel(coords.to_host(), rc, what="coords")
    got_valid = valid.to_host()
    assert_valid_mask(got_valid, p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], h, w)
    if trans_sigma > 0.5:
        assert 0.5 < got_valid.mean() < 0.95
    # the oracle's own fp32 mask agrees with the fp64 one outside the band too
    assert_valid_mask(rv, p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], h, w)


def test_pose_retr_disp_retr_clamp(slk):
    pin = Pins(slk)
    rng = np.random.default_rng(1)
    poses = wl.ba_problem(n=8, h=6, w=8)["poses"]
    dx = rng.normal(0, 0.05, (5, 6)).astype(np.float32)
    pd = slk.DeviceArray.from_host(poses)
    dd = slk.DeviceArray.from_host(dx)
    slk.check(slk.lib().slk_pose_retr(pd.ptr, dd.ptr, 2, 7, None))
    slk.hip().sync()
    np.testing.assert_allclose(pd.to_host(), orc.pose_retr(poses, dx, 2, 7), atol=1e-6)
    disps = rng.uniform(0.0, 1.0, (6, 48)).astype(np.float32)
    dz = rng.normal(0, 0.5, (3, 48)).astype(np.float32)
    inds = np.array([4, 0, 2], np.int32)
    ds = slk.DeviceArray.from_host(disps)
    slk.check(slk.lib().slk_disp_retr(ds.ptr, pin(dz),
                                      pin(inds), 3, 48, None))
    slk.hip().sync()
    np.testing.assert_array_equal(ds.to_host(), orc.disp_retr(disps, dz, inds))
    x = rng.normal(0, 0.01, 1000).astype(np.float32)
    xd = slk.DeviceArray.from_host(x)
    slk.check(slk.lib().slk_clamp_disps(xd.ptr, 1000, 0.001, None))
    slk.hip().sync()
    np.testing.assert_array_equal(xd.to_host(), np.maximum(x, np.float32(0.001)))


def test_frame_distance(slk):
    pin = Pins(slk)
    p = wl.ba_problem(n=6, h=48, w=64, seed=5)
    ii = np.array([0, 1, 2, 3, 5, 4], np.int32)
    jj = np.array([1, 0, 4, 5, 2, 4], np.int32)
    d = {k: slk.DeviceArray.from_host(p[k]) for k in ("poses", "disps", "intr")}
    dist = slk.DeviceArray((6,))
    slk.check(slk.lib().slk_frame_distance(d["poses"].ptr, d["disps"].ptr, d["intr"].ptr,
                                           pin(ii),
                                           pin(jj), dist.ptr, 6, 48, 64,
                                           0.3, None))
    slk.hip().sync()
    ref = orc.frame_distance(p["poses"], p["disps"], p["intr"], ii, jj, 48, 64, 0.3)
    np.testing.assert_allclose(dist.to_host(), ref, rtol=TOL, atol=1e-5)


@pytest.mark.parametrize("case", ["translation", "rotation", "coverage_0.8", "coverage_0.6",
                                  "coverage_0.75"])
def test_frame_distance_known_answers(slk, case):
    """The hand-derived cases of the oracle's pins (test_oracle_se3_ba.py), on
    the GPU: fx = fy = 10, cx = cy = 0, frame 0 at the identity."""
    announce(f"frame_distance known answer {case}")
    th = 0.1
    cases = {
        "translation": ([0.2, 0, 0, 0, 0, 0, 1], [0.5] * 6, 2, 1.0),
        "rotation": ([0, 0, 0, 0.0, np.sin(th / 2), 0.0, np.cos(th / 2)], [0.7], 1,
                     0.3 * 10.0 * np.tan(th)),
        "coverage_0.8": ([0, 0, -0.5, 0, 0, 0, 1], [1, 1, 1, 1, 10], 1, 1.5),
        "coverage_0.6": ([0, 0, -0.5, 0, 0, 0, 1], [1, 1, 1, 10, 10], 1, 1000.0),
        "coverage_0.75": ([0, 0, -0.5, 0, 0, 0, 1], [1, 1, 1, 1.5], 1, 1.0),
    }
    pose_j, row, H, want = cases[case]
    W = len(row) // H
    poses = np.array([[0, 0, 0, 0, 0, 0, 1], pose_j], np.float32)
    disps = np.zeros((2, H, W), np.float32)
    disps[0] = np.asarray(row, np.float32).reshape(H, W)
    intr = np.array([10.0, 10.0, 0.0, 0.0], np.float32)
    pin = Pins(slk)
    D = slk.DeviceArray.from_host
    dp, dd, di = D(poses), D(disps), D(intr)
    dist = slk.DeviceArray((1,))
    slk.check(slk.lib().slk_frame_distance(dp.ptr, dd.ptr, di.ptr, pin(np.array([0], np.int32)),
                                           pin(np.array([1], np.int32)), dist.ptr, 1, H, W, 0.3,
                                           None))
    slk.hip().sync()
    got = float(dist.to_host()[0])
    assert got == pytest.approx(want, rel=1e-5)
    assert got == pytest.approx(float(orc.frame_distance(poses, disps, intr, [0], [1], H, W,
                                                         0.3)[0]), rel=1e-5)
