"""The no-allocation batched correlation entry point
(slk_corr_batch_build_and_sample_dev_noalloc): its scratch is one static
64 MiB device array, so it must give bitwise the results of the context path
(slk_corr_batch_build_and_sample_dev, same kernels) on two calls in a row,
the second smaller than the first (the array keeps the first call's
contents), and must reject map sizes whose one-edge scratch does not fit."""
import ctypes

import numpy as np
import pytest

from helpers import announce, assert_close_rel, gpu_or_fail
from oracle import oracle as orc
import workloads as wl

P = ctypes.c_void_p


def _fn(slk):
    return slk.lib().slk_corr_batch_build_and_sample_dev_noalloc


def test_rejects_maps_beyond_the_scratch_without_a_gpu():
    import slk
    fn = _fn(slk)
    # 256 x 256: one edge's lookup windows alone are 64 MiB
    st = fn(None, 0, 128 * 65536, P(1), P(1), 4, None, None, 256, 256, 128, 0.0625, None)
    assert st == slk.SLK_E_ARG
    assert b"64 MiB" in slk.lib().slk_last_error()
    assert fn(None, 0, 0, P(1), P(1), 4, None, None, 48, 64, 120, 0.0625, None) == slk.SLK_E_ARG
    assert fn(None, 0, 0, None, None, 4, None, None, 48, 64, 128, 0.0625, None) == slk.SLK_E_ARG


def _context_path(slk, f, ii, jj, coords, dtype):
    n, C, h, w = f.shape
    B = len(ii)
    ctx = slk.Context(h, w, C=C, max_batch=48, corr_scale=wl.CORR_ALPHA_REF)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    iid, jjd = slk.DeviceArray.from_host(ii), slk.DeviceArray.from_host(jj)
    out = slk.DeviceArray((B, 196, h * w))
    ctx.batch_build_and_sample_correlation_dev(fd, iid, jjd, B, cd, out, dtype=dtype)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    return got


@pytest.mark.gpu
def test_noalloc_matches_context_path_two_calls():
    slk = gpu_or_fail()
    orc.build()
    fn = _fn(slk)
    cases = [
        # 20 edges at 48x64 (9 per launch fit the scratch: three launches)
        (wl.frames(8, C=128, h=48, w=64, seed=90), 20, slk.SLK_F32, 91),
        # then 5 edges of smaller fp16 maps over the same array
        (wl.frames(5, C=128, h=24, w=32, seed=92).astype(np.float16), 5, slk.SLK_F16, 93),
    ]
    for k, (f, B, dtype, seed) in enumerate(cases):
        n, C, h, w = f.shape
        announce(f"corr noalloc call {k}: {B} edges at {h}x{w} dtype {dtype}")
        ii, jj = wl.cyclic_edges(n)
        ii, jj = np.ascontiguousarray(ii[:B]), np.ascontiguousarray(jj[:B])
        coords = wl.flow_coords(B, h, w, seed=seed)
        fd = slk.DeviceArray.from_host(f)
        cd = slk.DeviceArray.from_host(coords)
        iid, jjd = slk.DeviceArray.from_host(ii), slk.DeviceArray.from_host(jj)
        out = slk.DeviceArray((B, 196, h * w))
        slk.check(fn(fd.ptr, dtype, C * h * w, iid.ptr, jjd.ptr, B, cd.ptr, out.ptr, h, w, C,
                     wl.CORR_ALPHA_REF, None))
        slk.hip().sync()
        got = out.to_host()
        want = _context_path(slk, f, ii, jj, coords, dtype)
        np.testing.assert_array_equal(got, want)
        ref = orc.corr_batch(f.astype(np.float32), ii[:1], jj[:1], coords[:1],
                             wl.CORR_ALPHA_REF)
        assert_close_rel(got[0], ref[0], what=f"call {k} edge 0 vs oracle")
