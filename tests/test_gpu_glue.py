"""GPU parity of the update-pass glue (slk_compute_motion, slk_fill_coords0,
slk_compute_target, slk_gather_rows, slk_scatter_rows, slk_scatter_mean,
slk_ba_edge_set) through the C ABI against the CPU oracle on the same seeded
inputs. Every output is compared bitwise: the kernels perform the reference's
fp32 operations in the reference's order (cuda_slam/main.cu:1246-1301,
2150-2163, 2186-2390), including the fused multiply-add of the keyframe mean.
Sizes: the 48-edge 48x64 window with 128-channel rows (the cfg2 update
pass), a 2000-edge / 200-keyframe scatter-mean (the backend's edge count),
and odd shapes that take the scalar (non-float4) paths.
"""
import ctypes

import numpy as np
import pytest

from helpers import announce, gpu_or_fail
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


@pytest.fixture(scope="module")
def ctx(slk):
    c = slk.Context(48, 64, C=128, max_batch=48)
    yield c
    c.close()


def _dev(slk, a):
    return slk.DeviceArray.from_host(np.ascontiguousarray(a))


def _grid(B, h, w):
    gx, gy = np.meshgrid(np.arange(w, dtype=np.float32), np.arange(h, dtype=np.float32))
    return np.broadcast_to(np.stack([gx.ravel(), gy.ravel()]), (B, 2, h * w)).copy()


@pytest.mark.parametrize("h,w", [(48, 64), (7, 9)])
def test_motion_and_coords0(slk, h, w):
    announce(f"glue motion {h}x{w}")
    B, HW = 48, h * w
    rng = np.random.default_rng(10)
    c1 = (_grid(B, h, w) + rng.normal(0, 30, (B, 2, HW))).astype(np.float32)
    tg = (c1 + rng.normal(0, 30, (B, 2, HW))).astype(np.float32)
    c1[0, 0, :3] = [np.nan, np.inf, -np.inf]
    L = slk.lib()
    c1d, tgd = _dev(slk, c1), _dev(slk, tg)
    c0d = slk.DeviceArray((B, 2, HW))
    slk.check(L.slk_fill_coords0(c0d.ptr, B, h, w, None))
    m_id = slk.DeviceArray((B, 4, HW))
    m_c0 = slk.DeviceArray((B, 4, HW))
    m_s0 = slk.DeviceArray((B, 4, HW))
    slk.check(L.slk_compute_motion(m_id.ptr, c1d.ptr, None, tgd.ptr, B, h, w, None))
    slk.check(L.slk_compute_motion(m_c0.ptr, c1d.ptr, c0d.ptr, tgd.ptr, B, h, w, None))
    # step 0 of the update pass: target = coords1
    slk.check(L.slk_compute_motion(m_s0.ptr, c1d.ptr, None, c1d.ptr, B, h, w, None))
    slk.hip().sync()
    np.testing.assert_array_equal(c0d.to_host(), _grid(B, h, w))
    ref = orc.compute_motion(c1, tg, h, w)
    np.testing.assert_array_equal(m_id.to_host(), ref)
    np.testing.assert_array_equal(m_c0.to_host(), ref)
    np.testing.assert_array_equal(m_s0.to_host(), orc.compute_motion(c1, c1, h, w))


@pytest.mark.parametrize("hw", [3072, 63])
def test_target(slk, hw):
    n = 48
    rng = np.random.default_rng(11)
    coords = rng.normal(0, 20, (n, 2, hw)).astype(np.float32)
    delta = rng.normal(0, 2, (n, 3, hw)).astype(np.float32)
    wt = rng.random((n, 3, hw)).astype(np.float32)
    t = slk.DeviceArray((n, 2, hw))
    w = slk.DeviceArray((n, 2, hw))
    cd, dd, wd = _dev(slk, coords), _dev(slk, delta), _dev(slk, wt)  # alive until the sync
    slk.check(slk.lib().slk_compute_target(t.ptr, w.ptr, cd.ptr, dd.ptr, wd.ptr, n, hw, None))
    slk.hip().sync()
    rt, rw = orc.compute_target(coords, delta, wt)
    np.testing.assert_array_equal(t.to_host(), rt)
    np.testing.assert_array_equal(w.to_host(), rw)


def test_gather_scatter_hidden_state_rows(slk):
    """The per-edge copy loops of one 48-edge batch at bs = 16 of 96 edges:
    batch_nets = edge_nets[bs:bs+48], batch_inps = inps[ii[bs:bs+48]], then
    edge_nets[bs:bs+48] = batch_nets (main.cu:2216-2224, 2245-2252)."""
    announce("glue gather/scatter 48 rows of 128x3072")
    L = slk.lib()
    row = 128 * 3072
    rng = np.random.default_rng(12)
    nets = rng.normal(size=(96, row)).astype(np.float32)
    inps = rng.normal(size=(12, row)).astype(np.float32)
    ii, _ = wl.cyclic_edges(12)
    ii = np.concatenate([ii, ii]).astype(np.int32)
    bs, B = 16, 48
    netsd, inpsd, iid = _dev(slk, nets), _dev(slk, inps), _dev(slk, ii)
    bn = slk.DeviceArray((B, row))
    bi = slk.DeviceArray((B, row))
    slk.check(L.slk_gather_rows(bn.ptr, netsd.ptr + bs * row * 4, None, B, row, None))
    slk.check(L.slk_gather_rows(bi.ptr, inpsd.ptr, iid.ptr + bs * 4, B, row, None))
    slk.hip().sync()
    np.testing.assert_array_equal(bn.to_host(), orc.gather_rows(nets[bs:], None, n=B))
    np.testing.assert_array_equal(bi.to_host(), orc.gather_rows(inps, ii[bs:bs + B]))
    upd = rng.normal(size=(B, row)).astype(np.float32)
    bn.upload(upd)
    slk.check(L.slk_scatter_rows(netsd.ptr + bs * row * 4, bn.ptr, None, B, row, None))
    slk.hip().sync()
    ref = nets.copy()
    ref[bs:bs + B] = orc.scatter_rows(nets[bs:bs + B], upd, None)
    np.testing.assert_array_equal(netsd.to_host(), ref)


def test_gather_scatter_scalar_paths(slk):
    """Row lengths that are not a multiple of 4 and rows at an address that is
    not 16-byte aligned take the one-float path."""
    L = slk.lib()
    rng = np.random.default_rng(13)
    src = rng.normal(size=(10, 1001)).astype(np.float32)
    idx = rng.permutation(10).astype(np.int32)
    sd, idd = _dev(slk, src), _dev(slk, idx)
    g = slk.DeviceArray((10, 1001))
    slk.check(L.slk_gather_rows(g.ptr, sd.ptr, idd.ptr, 10, 1001, None))
    s = slk.DeviceArray((10, 1001))
    s.zero()
    slk.check(L.slk_scatter_rows(s.ptr, sd.ptr, idd.ptr, 10, 1001, None))
    # 4-float rows starting one float into the buffer
    src4 = rng.normal(size=(6 * 8 + 1,)).astype(np.float32)
    s4 = _dev(slk, src4)
    g4 = slk.DeviceArray((6 * 8 + 1,))
    g4.zero()
    slk.check(L.slk_gather_rows(g4.ptr + 4, s4.ptr + 4, None, 6, 8, None))
    slk.hip().sync()
    np.testing.assert_array_equal(g.to_host(), orc.gather_rows(src, idx))
    np.testing.assert_array_equal(s.to_host(), orc.scatter_rows(np.zeros_like(src), src, idx))
    np.testing.assert_array_equal(g4.to_host()[1:], src4[1:])


def _scatter_mean(slk, ctx, src, ii):
    L = slk.lib()
    n = len(ii)
    row = int(np.prod(src.shape[1:]))
    dst = slk.DeviceArray((max(n, 1), row))
    act_d = slk.DeviceArray((max(n, 1),), np.int32)
    act_h = np.zeros(max(n, 1), np.int32)
    na = ctypes.c_int(-1)
    sd = _dev(slk, src)  # alive until the sync
    slk.check(L.slk_scatter_mean(ctx.ptr, dst.ptr, sd.ptr,
                                 np.ascontiguousarray(ii, np.int32).ctypes.data, n, row,
                                 act_d.ptr, act_h.ctypes.data, ctypes.byref(na), None))
    slk.hip().sync()
    k = na.value
    return dst.to_host()[:k].reshape((k,) + src.shape[1:]), act_d.to_host()[:k], act_h[:k]


def test_scatter_mean_window(slk, ctx):
    """GraphAgg over the 48-edge window: 12 keyframes, 4 edges each, rows of
    128 x 3072 conv1 features (count 4: the fused mean step runs)."""
    announce("glue scatter_mean 48 x 128x3072")
    rng = np.random.default_rng(14)
    ii, _ = wl.cyclic_edges(12)
    src = rng.normal(size=(48, 128, 3072)).astype(np.float32)
    got, act_d, act_h = _scatter_mean(slk, ctx, src, ii)
    ref, act = orc.scatter_mean(src, ii)
    np.testing.assert_array_equal(act_h, act)
    np.testing.assert_array_equal(act_d, act)
    np.testing.assert_array_equal(got, ref)


def test_scatter_mean_backend_counts(slk, ctx):
    """2000 edges over 200 keyframes with uneven counts (1 to 20, odd ones
    included), rows of 4 x 61 floats (scalar path)."""
    ii, _ = wl.backend_edges(200, 2000)
    rng = np.random.default_rng(15)
    src = rng.normal(0, 100, size=(2000, 4, 61)).astype(np.float32)
    got, _, act_h = _scatter_mean(slk, ctx, src, ii)
    ref, act = orc.scatter_mean(src, ii)
    np.testing.assert_array_equal(act_h, act)
    np.testing.assert_array_equal(got, ref)


def test_ba_edge_set(slk, ctx):
    announce("glue ba_edge_set")
    L = slk.lib()
    hw = 3072
    rng = np.random.default_rng(16)
    ii = rng.integers(4, 12, 48).astype(np.int32)
    jj = rng.integers(4, 12, 48).astype(np.int32)
    ii_in = rng.integers(0, 12, 30).astype(np.int32)
    jj_in = rng.integers(0, 12, 30).astype(np.int32)
    t = rng.normal(size=(48, 2, hw)).astype(np.float32)
    w = rng.random((48, 2, hw)).astype(np.float32)
    ti = rng.normal(size=(30, 2, hw)).astype(np.float32)
    wi = rng.random((30, 2, hw)).astype(np.float32)
    td, wd, tid, wid = _dev(slk, t), _dev(slk, w), _dev(slk, ti), _dev(slk, wi)
    for forced, use in [(-1, 1), (6, 1), (-1, 0)]:
        cap = 78
        bi_h, bj_h = np.zeros(cap, np.int32), np.zeros(cap, np.int32)
        bi, bj = slk.DeviceArray((cap,), np.int32), slk.DeviceArray((cap,), np.int32)
        bt, bw = slk.DeviceArray((cap, 2, hw)), slk.DeviceArray((cap, 2, hw))
        cnt, t0 = ctypes.c_int(-1), ctypes.c_int(-1)
        slk.check(L.slk_ba_edge_set(ctx.ptr, ii.ctypes.data, jj.ctypes.data, 48,
                                    ii_in.ctypes.data, jj_in.ctypes.data, 30, td.ptr, wd.ptr,
                                    tid.ptr, wid.ptr, hw, 12, forced, use, bi_h.ctypes.data,
                                    bj_h.ctypes.data, bi.ptr, bj.ptr, bt.ptr, bw.ptr,
                                    ctypes.byref(cnt), ctypes.byref(t0), None))
        slk.hip().sync()
        ref = orc.ba_edge_set(ii, jj, ii_in, jj_in, t, w, ti, wi, 12, forced_t0=forced,
                              use_inactive=bool(use))
        m = cnt.value
        assert m == len(ref["ii"]) and t0.value == ref["t0"]
        np.testing.assert_array_equal(bi_h[:m], ref["ii"])
        np.testing.assert_array_equal(bj_h[:m], ref["jj"])
        np.testing.assert_array_equal(bi.to_host()[:m], ref["ii"])
        np.testing.assert_array_equal(bj.to_host()[:m], ref["jj"])
        np.testing.assert_array_equal(bt.to_host()[:m], ref["target"])
        np.testing.assert_array_equal(bw.to_host()[:m], ref["weight"])


def test_empty_calls_are_no_ops(slk, ctx):
    L = slk.lib()
    na = ctypes.c_int(-1)
    assert L.slk_compute_motion(None, None, None, None, 0, 4, 4, None) == 0
    assert L.slk_compute_target(None, None, None, None, None, 0, 16, None) == 0
    assert L.slk_gather_rows(None, None, None, 0, 16, None) == 0
    assert L.slk_scatter_rows(None, None, None, 0, 16, None) == 0
    assert L.slk_scatter_mean(ctx.ptr, None, None, None, 0, 16, None, None, ctypes.byref(na),
                              None) == 0 and na.value == 0
