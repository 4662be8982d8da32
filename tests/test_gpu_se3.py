"""GPU parity of the SE3 reprojection kernels (cuda_slam/se3.cuh) through the
C ABI against the CPU oracle on identical seeded inputs.

Bars: valid masks, retraction indices and clamps bitwise; projected
coordinates and frame distances within helpers.TOL = 1e-4 relative to
max(|r|, rms(r)); fp64-evaluated pose retraction within 1e-6.
"""
import numpy as np
import pytest

from helpers import TOL, Pins, announce, assert_close_rel, gpu_or_fail
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


def test_projmap(slk):
    announce("projmap 48 edges")
    p = wl.ba_problem()
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
    assert np.mean(valid.to_host() == rv) > 0.9999


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
