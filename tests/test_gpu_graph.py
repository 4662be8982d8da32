"""GPU parity of slk_proximity_factors (CudaDroid::add_proximity_factors,
cuda_slam/main.cu:1655-1779, up to the edge-state update): the frame
distances of every pair in one launch, against the oracle's frame_distance
(within helpers.TOL), and the chosen edges, bitwise equal to the oracle's
selection run on the same raw distances. Parameter sets follow the
reference's three callers: initialisation (0, 0, rad 2, nms 2; main.cu:1847),
the frontend window (t1 - 5, t1 - window; main.cu:2056-2062) with existing
active and inactive edges and max_factors, and the backend (0, 0, radius 2,
nms 3; main.cu:2462-2471)."""
import ctypes

import numpy as np
import pytest

from helpers import TOL, announce, gpu_or_fail
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


def _trajectory(n, h, w, seed):
    """Keyframes moving along x with small rotations: distances grow with |i - j|."""
    rng = np.random.default_rng(seed)
    poses = np.zeros((n, 7), np.float32)
    poses[:, 0] = 0.06 * np.arange(n) + rng.normal(0, 0.01, n)
    poses[:, 1:3] = rng.normal(0, 0.01, (n, 2))
    poses[:, 3:] = wl.quat_from_rotvec(rng.normal(0, 0.02, (n, 3)))
    disps = rng.uniform(0.2, 2.0, (n, h, w)).astype(np.float32)
    intr = np.array([60.0, 60.0, 32.0, 24.0], np.float32)
    return poses, disps, intr


CASES = [  # (name, t0, t1, rad, nms, thresh, n_active, n_inac, max_factors)
    ("init", 0, 0, 2, 2, 16.0, 0, 0, 0),
    ("frontend", 11, 4, 2, 1, 16.0, 30, 10, 48),
    ("backend", 0, 0, 2, 3, 20.0, 40, 25, 0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_proximity_factors(slk, case):
    name, t0, t1, rad, nms, thresh, na, ni, maxf = case
    announce(f"proximity factors {name}")
    h, w, t = 48, 64, 16
    poses, disps, intr = _trajectory(t, h, w, seed=7)
    rng = np.random.default_rng(8)
    ii = rng.integers(0, t, na).astype(np.int32)
    jj = rng.integers(0, t, na).astype(np.int32)
    ii_in = rng.integers(0, t, ni).astype(np.int32)
    jj_in = rng.integers(0, t, ni).astype(np.int32)
    ctx = slk.Context(h, w, C=128, max_batch=1)
    dp, dd, di = (slk.DeviceArray.from_host(a) for a in (poses, disps, intr))
    npairs = (t - t0) * (t - t1)
    cap = 2 * (t - t0) * (t - t1 + rad + 1)
    new_i, new_j = np.zeros(cap, np.int32), np.zeros(cap, np.int32)
    dist = np.zeros(npairs, np.float32)
    n_new, n_es = ctypes.c_int(-1), ctypes.c_int(-1)
    ptr = lambda a: a.ctypes.data if a.size else None  # noqa: E731
    slk.check(slk.lib().slk_proximity_factors(
        ctx.ptr, dp.ptr, dd.ptr, di.ptr, t, t0, t1, rad, nms, thresh, 0.3, ptr(ii), ptr(jj), na,
        ptr(ii_in), ptr(jj_in), ni, maxf, new_i.ctypes.data, new_j.ctypes.data, cap,
        ctypes.byref(n_new), ctypes.byref(n_es), dist.ctypes.data, None))
    ctx.close()
    pi = np.repeat(np.arange(t0, t), t - t1).astype(np.int32)
    pj = np.tile(np.arange(t1, t), t - t0).astype(np.int32)
    ref_d = orc.frame_distance(poses, disps, intr, pi, pj, h, w, 0.3)
    np.testing.assert_allclose(dist, ref_d, rtol=TOL, atol=1e-5)
    ref_new, ref_ne = orc.proximity_select(dist, t, t0, t1, rad, nms, thresh, ii, jj, ii_in,
                                           jj_in, max_factors=maxf)
    assert n_es.value == ref_ne
    got = np.stack([new_i[:n_new.value], new_j[:n_new.value]], 1)
    np.testing.assert_array_equal(got, ref_new)
    assert np.sum(dist[(pi - pj) > rad + 1] <= thresh) > 0  # the greedy step had candidates
