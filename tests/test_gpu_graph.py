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


# ------------------------------------------- edge-state update (main.cu:795-836)
EDGE_CASES = [  # (name, n, removed, inactive already held, max_inac)
    ("age_removal", 48, [3, 17, 18, 40], 5, 64),
    ("first_edge_chain", 48, [0], 0, 64),
    ("inactive_full", 32, [1, 2, 9, 30, 31], 62, 64),  # room for two; three dropped
    ("nothing_masked", 16, [], 3, 64),
]


@pytest.mark.parametrize("case", EDGE_CASES, ids=[c[0] for c in EDGE_CASES])
def test_store_and_remove_edges_matches_oracle(slk, case):
    name, n, removed, n_in, max_inac = case
    h, w = 48, 64
    hw = h * w
    announce(f"store_and_remove_edges {name}: n={n} removed={removed} inac={n_in}/{max_inac}")
    rng = np.random.default_rng(11)
    ii = rng.integers(0, 20, n).astype(np.int32)
    jj = rng.integers(0, 20, n).astype(np.int32)
    age = rng.integers(0, 30, n).astype(np.int32)
    nets = rng.normal(size=(n, 128, hw)).astype(np.float32)
    tg = rng.normal(size=(n, 2, hw)).astype(np.float32)
    wt = rng.uniform(size=(n, 2, hw)).astype(np.float32)
    tin = np.zeros((max_inac, 2, hw), np.float32)
    win = np.zeros((max_inac, 2, hw), np.float32)
    tin[:n_in] = rng.normal(size=(n_in, 2, hw))
    win[:n_in] = rng.uniform(size=(n_in, 2, hw))
    iin = np.zeros(max_inac, np.int32)
    jin = np.zeros(max_inac, np.int32)
    iin[:n_in] = rng.integers(0, 20, n_in)
    jin[:n_in] = rng.integers(0, 20, n_in)
    mask = np.zeros(n, np.uint8)
    mask[removed] = 1
    ref = orc.store_and_remove_edges(mask, ii, jj, age, iin[:n_in], jin[:n_in], max_inac, nets,
                                     tg, wt, tin[:n_in], win[:n_in])
    D = slk.DeviceArray.from_host
    dn, dt, dw, dti, dwi = D(nets), D(tg), D(wt), D(tin), D(win)
    hii, hjj, hage, hiin, hjin = ii.copy(), jj.copy(), age.copy(), iin.copy(), jin.copy()
    num_inac, n_kept = ctypes.c_int(n_in), ctypes.c_int(-1)
    ctx = slk.Context(h, w, C=128, max_batch=48)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    slk.check(slk.lib().slk_store_and_remove_edges(
        ctx.ptr, P(mask), n, P(hii), P(hjj), P(hage), P(hiin), P(hjin), ctypes.byref(num_inac),
        max_inac, dn.ptr, 128 * hw, dt.ptr, dw.ptr, dti.ptr, dwi.ptr, 2 * hw,
        ctypes.byref(n_kept), None))
    slk.hip().sync()
    k, m = n_kept.value, num_inac.value
    assert (k, m) == (ref["n_kept"], ref["num_inac"])
    np.testing.assert_array_equal(hii[:k], ref["ii"])
    np.testing.assert_array_equal(hjj[:k], ref["jj"])
    np.testing.assert_array_equal(hage[:k], ref["age"])
    np.testing.assert_array_equal(hiin[:m], ref["ii_inac"])
    np.testing.assert_array_equal(hjin[:m], ref["jj_inac"])
    # rows are copies: bitwise
    np.testing.assert_array_equal(dn.to_host()[:k], ref["nets"])
    np.testing.assert_array_equal(dt.to_host()[:k], ref["target"])
    np.testing.assert_array_equal(dw.to_host()[:k], ref["weight"])
    np.testing.assert_array_equal(dti.to_host()[:m], ref["target_inac"])
    np.testing.assert_array_equal(dwi.to_host()[:m], ref["weight_inac"])
    # rows past the kept ones and past the inactive ones are left as they were
    np.testing.assert_array_equal(dti.to_host()[m:], tin[m:])
    ctx.close()


def test_init_new_edges_matches_oracle(slk):
    h, w = 48, 64
    hw = h * w
    announce("init_new_edges: 40 edges, 8 new")
    rng = np.random.default_rng(12)
    nets = rng.normal(size=(12, 128, hw)).astype(np.float32)
    en = rng.normal(size=(40, 128, hw)).astype(np.float32)
    wt = rng.uniform(size=(40, 2, hw)).astype(np.float32)
    ii = rng.integers(0, 12, 40).astype(np.int32)
    ref_en, ref_w = orc.init_new_edges(nets, en, wt, ii, 32, 8)
    D = slk.DeviceArray.from_host
    dn, de, dw = D(nets), D(en), D(wt)
    ctx = slk.Context(h, w, C=128, max_batch=48)
    slk.check(slk.lib().slk_init_new_edges(ctx.ptr, dn.ptr, de.ptr, dw.ptr,
                                           ii.ctypes.data_as(ctypes.c_void_p), 32, 8, 128 * hw,
                                           2 * hw, None))
    slk.hip().sync()
    np.testing.assert_array_equal(de.to_host(), ref_en)
    np.testing.assert_array_equal(dw.to_host(), ref_w)
    ctx.close()


@pytest.mark.parametrize("ix", [9, 0, 11])
def test_rm_keyframe_matches_oracle(slk, ix):
    """CudaDroid::rm_keyframe (main.cu:866-941) on a 12-keyframe window with
    48 active and 20 inactive edges at 48x64: every array and list bitwise
    equal to the oracle's (ix = 9 is the frontend's nk - 3)."""
    h, w, t, ne, ni = 48, 64, 12, 48, 20
    hw = h * w
    announce(f"rm_keyframe ix={ix}")
    rng = np.random.default_rng(13 + ix)
    st = {"poses": rng.normal(size=(t, 7)).astype(np.float32),
          "disps": rng.uniform(size=(t, hw)).astype(np.float32),
          "fmaps": rng.normal(size=(t, 128, hw)).astype(np.float16),
          "nets": rng.normal(size=(t, 128, hw)).astype(np.float32),
          "inps": rng.normal(size=(t, 128, hw)).astype(np.float32),
          "ii": rng.integers(0, t, ne).astype(np.int32),
          "jj": rng.integers(0, t, ne).astype(np.int32),
          "age": rng.integers(0, 25, ne).astype(np.int32),
          "ii_inac": rng.integers(0, t, ni).astype(np.int32),
          "jj_inac": rng.integers(0, t, ni).astype(np.int32),
          "edge_nets": rng.normal(size=(ne, 128, hw)).astype(np.float32),
          "target": rng.normal(size=(ne, 2, hw)).astype(np.float32),
          "weight": rng.uniform(size=(ne, 2, hw)).astype(np.float32),
          "target_inac": rng.normal(size=(ni, 2, hw)).astype(np.float32),
          "weight_inac": rng.uniform(size=(ni, 2, hw)).astype(np.float32)}
    ref = orc.rm_keyframe(ix, st)
    D = slk.DeviceArray.from_host
    arrs = ("poses", "disps", "nets", "inps", "edge_nets", "target", "weight", "target_inac",
            "weight_inac")
    dv = {k: D(st[k]) for k in arrs}
    dfm = D(st["fmaps"].view(np.uint16))
    lists = {k: st[k].copy() for k in ("ii", "jj", "age", "ii_inac", "jj_inac")}
    nk, nik = ctypes.c_int(-1), ctypes.c_int(-1)
    ctx = slk.Context(h, w, C=128, max_batch=48)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    slk.check(slk.lib().slk_rm_keyframe(
        ctx.ptr, ix, t, dv["poses"].ptr, dv["disps"].ptr, dfm.ptr, slk.SLK_F16, dv["nets"].ptr,
        dv["inps"].ptr, 128 * hw, P(lists["ii"]), P(lists["jj"]), P(lists["age"]), ne,
        ctypes.byref(nk), P(lists["ii_inac"]), P(lists["jj_inac"]), ni, ctypes.byref(nik),
        dv["edge_nets"].ptr, dv["target"].ptr, dv["weight"].ptr, dv["target_inac"].ptr,
        dv["weight_inac"].ptr, None))
    slk.hip().sync()
    assert (nk.value, nik.value) == (len(ref["ii"]), len(ref["ii_inac"]))
    for k in ("ii", "jj", "age"):
        np.testing.assert_array_equal(lists[k][:nk.value], ref[k])
    for k in ("ii_inac", "jj_inac"):
        np.testing.assert_array_equal(lists[k][:nik.value], ref[k])
    for k in arrs:
        np.testing.assert_array_equal(dv[k].to_host(), ref[k], err_msg=k)
    np.testing.assert_array_equal(dfm.to_host().view(np.float16), ref["fmaps"])
    ctx.close()
