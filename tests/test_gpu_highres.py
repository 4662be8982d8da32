"""GPU parity at the high-resolution window (128x54x96 features, 16 frames,
64 edges) and at the backend scale (200 keyframes, 2000 edges), through the
C ABI against the CPU oracle on the same seeded inputs.

* The 64-edge launch is the largest one batched launch takes (one prefix
  scan and slot count over 64 edges); every edge is checked on sampled source
  pixels by a direct fp64 evaluation of their windows, and four edges in full
  against orc.corr_batch.
* BA at 54x96 with poses 0 and 1 fixed has P = 14 free poses (an 84 x 84
  Schur system), the size class solved by one workgroup with S in LDS.
* The backend correlation runs its 2000 edges through the prepared-frames
  path (every keyframe split once) and is checked on sampled pixels of every
  edge.
Bars as in the other parity tests: helpers.TOL relative to max(|r|, rms(r))
for correlation values, 1e-4 normwise for BA poses and inverse depths.
"""
import numpy as np
import pytest

from helpers import TOL, announce, assert_close_rel, gpu_or_fail, norm_rel
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


def lookup_rows(pyr, coords):
    """Oracle lookup of selected source rows: pyr[l] is [n, h>>l, w>>l] for n
    chosen source pixels whose coords are [2, n]."""
    n = pyr[0].shape[0]
    out = np.zeros((len(pyr) * 49, n), np.float32)
    for l, lev in enumerate(pyr):
        H2, W2 = lev.shape[1:]
        orc.lib().orc_corr_lookup_level(np.ascontiguousarray(lev).reshape(-1),
                                        np.ascontiguousarray(coords, np.float32).reshape(-1), out,
                                        3, 1, n, H2, W2, float(np.float32(1.0 / (1 << l))), l)
    return out


def sampled_reference(fi, fj, coords, pix, h, w, alpha):
    """Windows of the chosen source pixels: rows alpha * fi[:, p] . fj of the
    fp64 volume, pooled by the oracle's 2x2 mean, then the oracle lookup."""
    C = fi.shape[0]
    vol = (fi.reshape(C, -1)[:, pix].astype(np.float64).T
           @ fj.reshape(C, -1).astype(np.float64)) * alpha
    pyr = [vol.reshape(len(pix), h, w).astype(np.float32)]
    for _ in range(3):
        pyr.append(orc.avg_pool_2x2(pyr[-1]))
    return lookup_rows(pyr, coords[:, pix])


def test_highres_window_64_edges(slk):
    """Config highres: 16 frames of 128x54x96, the 64 cyclic edges in one launch."""
    h, w, n, B = 54, 96, 16, 64
    announce(f"highres window {h}x{w}, {B} edges in one launch")
    f = wl.frames(n, C=128, h=h, w=w, seed=70)
    ii, jj = wl.cyclic_edges(n)
    assert len(ii) == B
    coords = wl.flow_coords(B, h, w, seed=71)
    alpha = wl.CORR_ALPHA_REF
    ctx = slk.Context(h, w, C=128, max_batch=B, corr_scale=alpha)
    fd = slk.DeviceArray.from_host(f)
    cd = slk.DeviceArray.from_host(coords)
    out = slk.DeviceArray((B, 196, h * w))
    ctx.batch_build_and_sample_correlation(fd, ii, jj, cd, out)
    slk.hip().sync()
    got = out.to_host()
    ctx.close()
    assert np.all(np.isfinite(got))
    full = [0, 21, 42, 63]
    ref = orc.corr_batch(f, ii[full], jj[full], coords[full], alpha)
    for k, e in enumerate(full):
        assert_close_rel(got[e], ref[k], what=f"highres edge {e}")
    rng = np.random.default_rng(2)
    pix = rng.choice(h * w, 48, replace=False)
    for e in range(B):
        assert_close_rel(got[e][:, pix],
                         sampled_reference(f[ii[e]], f[jj[e]], coords[e], pix, h, w, alpha),
                         what=f"highres edge {e} sampled")


def test_highres_ba_three_iterations(slk):
    """Config highres BA: 16 frames, inverse depth 54x96, poses 0 and 1 fixed
    (P = 14, n = 84), 64 cyclic edges, 3 chained iterations."""
    announce("highres BA 54x96, P=14 (n=84), 3 iterations")
    p = wl.ba_problem(n=16, h=54, w=96, seed=72)
    assert p["t1"] - p["t0"] == 14
    D = slk.DeviceArray.from_host
    d = {k: D(p[k]) for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
    ctx = slk.Context(54, 96, max_batch=1)
    poses, disps = p["poses"], p["disps"]
    for it in range(3):
        ctx.ba_iterate(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                       d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1)
        ref = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                             p["ii"], p["jj"], 54, 96, p["t0"], p["t1"], 1e-4, 0.1)
        assert ref["status"] == 0
        S, b, dx = ctx.ba_last_system()
        assert S.shape == (84, 84)
        assert norm_rel(S, ref["S"]) < 1e-7, it
        assert norm_rel(b, ref["b"]) < 1e-7, it
        assert norm_rel(dx, ref["dx"]) < 1e-5, it
        poses, disps = ref["poses"], ref["disps"]
    assert ctx.ba_status() == slk.SLK_OK
    assert norm_rel(d["poses"].to_host(), poses) < TOL
    assert norm_rel(d["disps"].to_host(), disps) < TOL
    assert_close_rel(d["poses"].to_host(), poses, what="highres poses after 3")
    assert norm_rel(d["poses"].to_host() - p["poses"], poses - p["poses"]) < TOL
    ctx.close()
    # the same three iterations as one slk_ba_iterate_n call (fused iteration)
    d = {k: D(p[k]) for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
    ctx = slk.Context(54, 96, max_batch=1)
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 3)
    assert ctx.ba_status() == slk.SLK_OK
    assert norm_rel(d["poses"].to_host(), poses) < TOL
    assert norm_rel(d["disps"].to_host(), disps) < TOL
    assert_close_rel(d["poses"].to_host(), poses, what="highres poses after iterate_n(3)")
    assert_close_rel(d["disps"].to_host(), disps, what="highres disps after iterate_n(3)")
    ctx.close()


def test_backend_correlation_sampled(slk):
    """Config backend's correlation: 200 keyframes of 128x48x64, 2000 edges
    (|i-j| <= 2 plus long-range pairs) in 48-edge launches over frames split
    once (slk_corr_prepare_frames), every edge checked on 16 sampled source
    pixels, two edges in full."""
    h, w, n = 48, 64, 200
    announce(f"backend correlation {n} keyframes, 2000 edges, sampled")
    ii, jj = wl.backend_edges(n, 2000)
    M = len(ii)
    f = wl.frames(n, C=128, h=h, w=w, seed=80)
    coords = wl.flow_coords(M, h, w, seed=81)
    alpha = wl.CORR_ALPHA_REF
    ctx = slk.Context(h, w, C=128, max_batch=48, corr_scale=alpha)
    fd = slk.DeviceArray.from_host(f)
    ctx.prepare_frames(fd, n)
    rng = np.random.default_rng(3)
    pix = rng.choice(h * w, 16, replace=False)
    chunk = 400
    out = slk.DeviceArray((chunk, 196, h * w))
    full = {5, 1733}
    for c0 in range(0, M, chunk):
        sel = slice(c0, min(M, c0 + chunk))
        cd = slk.DeviceArray.from_host(np.ascontiguousarray(coords[sel]))
        ctx.batch_build_and_sample_prepared(np.ascontiguousarray(ii[sel]),
                                            np.ascontiguousarray(jj[sel]), cd, out)
        slk.hip().sync()
        got = out.to_host()
        assert np.all(np.isfinite(got))
        for k, e in enumerate(range(sel.start, sel.stop)):
            assert_close_rel(got[k][:, pix],
                             sampled_reference(f[ii[e]], f[jj[e]], coords[e], pix, h, w, alpha),
                             what=f"backend edge {e} sampled")
            if e in full:
                ref = orc.corr_batch(f, ii[e:e + 1], jj[e:e + 1], coords[e:e + 1], alpha)
                assert_close_rel(got[k], ref[0], what=f"backend edge {e}")
        cd.free()
    ctx.close()
