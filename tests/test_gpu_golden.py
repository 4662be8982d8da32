"""The HIP path through the C ABI against the committed golden fixtures
(tests/golden/*.npz): the same bars as the oracle-comparison tests --
corr and lookup within helpers.TOL = 1e-4 relative to max(|r|, rms(r)),
bitwise for the integer-coded case; SE3 within TOL; BA poses, disps and dx
normwise within TOL."""
import os

import numpy as np
import pytest

from helpers import TOL, Pins, announce, assert_close_rel, assert_valid_mask, gpu_or_fail, norm_rel

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def slk():
    return gpu_or_fail()


@pytest.mark.parametrize("name", ["corr_window", "corr_integer"])
def test_corr_window_fixture(slk, name):
    announce(f"golden {name}")
    g = load(name)
    n, C, h, w = g["fmaps"].shape
    B = len(g["ii"])
    ctx = slk.Context(h, w, C=C, max_batch=B, corr_scale=float(g["alpha"]))
    fd = slk.DeviceArray.from_host(g["fmaps"])
    cd = slk.DeviceArray.from_host(g["coords"])
    out = slk.DeviceArray((B, 196, h * w))
    ctx.batch_build_and_sample_correlation(fd, g["ii"], g["jj"], cd, out)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    if name == "corr_integer":
        np.testing.assert_array_equal(got, g["out"])
    else:
        assert_close_rel(got, g["out"], what=name)


def test_se3_fixture(slk):
    g = load("se3")
    h, w = int(g["h"]), int(g["w"])
    M = len(g["ii"])
    D = Pins(slk)
    coords = slk.DeviceArray((M, h, w, 2))
    valid = slk.DeviceArray((M, h, w))
    slk.check(slk.lib().slk_projmap(D(g["poses"]), D(g["disps"]), D(g["intr"]), D(g["ii"]),
                                    D(g["jj"]), coords.ptr, valid.ptr, M, h, w, None))
    dist = slk.DeviceArray((M,))
    slk.check(slk.lib().slk_frame_distance(D(g["poses"]), D(g["disps"]), D(g["intr"]),
                                           D(g["ii"]), D(g["jj"]), dist.ptr, M, h, w,
                                           float(g["beta"]), None))
    poses = slk.DeviceArray.from_host(g["poses"])
    slk.check(slk.lib().slk_pose_retr(poses.ptr, D(g["dx"]), int(g["t0"]), int(g["t1"]), None))
    slk.hip().sync()
    assert_close_rel(coords.to_host(), g["coords"], what="projmap")
    assert_valid_mask(valid.to_host(), g["poses"], g["disps"], g["intr"], g["ii"], g["jj"], h, w)
    assert_close_rel(dist.to_host(), g["dist"], what="frame_distance")
    np.testing.assert_allclose(poses.to_host(), g["poses_retr"], rtol=1e-6, atol=1e-6)


def test_ba_iteration_fixture(slk):
    g = load("ba_iter")
    h, w = int(g["h"]), int(g["w"])
    ctx = slk.Context(h, w, C=128, max_batch=1, levels=1, corr_scale=1.0 / 16.0)
    d = {k: slk.DeviceArray.from_host(g[k])
         for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
    ctx.ba_iterate(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                   d["ii"], d["jj"], g["ii"], g["jj"], int(g["t0"]), int(g["t1"]),
                   float(g["lm"]), float(g["ep"]))
    assert ctx.ba_status() == slk.SLK_OK
    S, b, dx = ctx.ba_last_system()
    poses, disps = d["poses"].to_host(), d["disps"].to_host()
    ctx.close()
    assert norm_rel(S, g["S"]) < 1e-7
    assert norm_rel(dx, g["dx"]) < 1e-5
    assert norm_rel(poses, g["poses_out"]) < TOL
    assert norm_rel(disps, g["disps_out"]) < TOL
