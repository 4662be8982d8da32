"""GPU parity of bundle adjustment (cuda_slam/ba.cuh) through the C ABI against
the CPU oracle on identical seeded inputs.

The GPU evaluates the linearization and all reductions in fp64 from the fp32
inputs, so S and b agree with the fp64 oracle to summation-order rounding
(asserted at 1e-7 normwise) and dx to 1e-5 normwise
(1e-4 relative) is asserted on the updated poses and disparities after 1 and
3 chained iterations. Stage kernels with the reference's fp32 storage are
held to 1e-5 relative (their outputs are fp32-rounded fp64 values).
"""
import numpy as np
import pytest

from helpers import TOL, Pins, announce, assert_close_rel, gpu_or_fail, norm_rel
from oracle import oracle as orc
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def slk():
    orc.build()
    return gpu_or_fail()


class Dev:
    """Device copies of a BA problem."""

    def __init__(self, slk, p):
        self.slk = slk
        self.p = p
        self.d = {k: slk.DeviceArray.from_host(p[k])
                  for k in ("poses", "disps", "intr", "target", "weight", "eta", "ii", "jj")}
        self.keep = []  # index copies stay alive while queued work may read them

    def iterate(self, ctx, lm, ep, motion_only=False, ii=None, jj=None):
        d = self.d
        ii = self.p["ii"] if ii is None else ii
        jj = self.p["jj"] if jj is None else jj
        iid = d["ii"] if ii is self.p["ii"] else self.slk.DeviceArray.from_host(ii)
        jjd = d["jj"] if jj is self.p["jj"] else self.slk.DeviceArray.from_host(jj)
        self.keep += [iid, jjd]
        ctx.ba_iterate(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                       iid, jjd, ii, jj, self.p["t0"], self.p["t1"], lm, ep, motion_only)

    def poses(self):
        return self.d["poses"].to_host()

    def disps(self):
        return self.d["disps"].to_host()


def oracle_iter(p, poses, disps, lm, ep, motion_only=False):
    return orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"], p["ii"],
                          p["jj"], p["h"], p["w"], p["t0"], p["t1"], lm, ep, motion_only)


@pytest.mark.parametrize("motion_only", [False, True])
def test_one_iteration_system_and_update(slk, motion_only):
    announce(f"ba_window one iteration motion_only={motion_only}")
    p = wl.ba_problem()
    dev = Dev(slk, p)
    ctx = slk.Context(p["h"], p["w"], max_batch=1)
    dev.iterate(ctx, 1e-4, 0.1, motion_only)
    assert ctx.ba_status() == slk.SLK_OK
    S, b, dx = ctx.ba_last_system()
    ref = oracle_iter(p, p["poses"], p["disps"], 1e-4, 0.1, motion_only)
    assert ref["status"] == 0
    assert norm_rel(S, ref["S"]) < 1e-7, norm_rel(S, ref["S"])
    assert norm_rel(b, ref["b"]) < 1e-7, norm_rel(b, ref["b"])
    assert norm_rel(dx, ref["dx"]) < 1e-5, norm_rel(dx, ref["dx"])
    assert_close_rel(dev.poses(), ref["poses"], what="poses")
    assert_close_rel(dev.disps(), ref["disps"], what="disps")
    if motion_only:
        np.testing.assert_array_equal(dev.disps(), p["disps"])
    ctx.close()


def test_three_iterations_chained(slk):
    announce("ba_window three chained iterations")
    p = wl.ba_problem()
    dev = Dev(slk, p)
    ctx = slk.Context(p["h"], p["w"], max_batch=1)
    poses, disps = p["poses"], p["disps"]
    for _ in range(3):
        dev.iterate(ctx, 1e-4, 0.1)
        ref = oracle_iter(p, poses, disps, 1e-4, 0.1)
        poses, disps = ref["poses"], ref["disps"]
    assert ctx.ba_status() == slk.SLK_OK
    assert norm_rel(dev.poses(), poses) < TOL
    assert norm_rel(dev.disps(), disps) < TOL
    assert_close_rel(dev.poses(), poses, what="poses after 3")
    assert_close_rel(dev.disps(), disps, what="disps after 3")
    # the pose updates themselves (not only the updated values)
    assert norm_rel(dev.poses() - p["poses"], poses - p["poses"]) < TOL
    ctx.close()


def _path_kernels(ctx):
    return set(ctx.profile())


def _dense_keyframe_problem(duplicate=False):
    """Keyframe 0 with edges to 9 free poses (10 E rows): more than the fused
    path's 7 per keyframe, so the window takes the five-kernel iteration.
    With `duplicate`, edge (0, 5) appears twice: E row (pose 5, keyframe 0)
    then belongs to two edges, which the one-wave-per-edge linearization
    cannot store, so the edge-serial k_ba_lin_kf runs."""
    n = 11
    ii = [0] * 9 + [k for k in range(1, n - 1)] + ([0] if duplicate else [])
    jj = [k for k in range(2, n)] + [k + 1 for k in range(1, n - 1)] + ([5] if duplicate else [])
    ii, jj = np.asarray(ii, np.int32), np.asarray(jj, np.int32)
    return wl.ba_problem(n=n, h=12, w=16, ii=ii, jj=jj, seed=17, fixed=2)


@pytest.mark.parametrize("case", ["window", "dense_keyframe", "dense_keyframe_dup"])
def test_iterate_n_matches_oracle_and_single_calls(slk, case):
    """slk_ba_iterate_n(3) against three chained oracle iterations and against
    three slk_ba_iterate calls: the cfg3 window runs the fused iteration (E
    rows and Schur products kept on chip, back-substitution folded into the
    next linearization, each solve in one launch with the next
    linearization), the dense keyframe the five-kernel one with one wave per
    edge (k_ba_lin_wv), and the dense keyframe with a duplicated edge the
    five-kernel one with the edge-serial linearization (k_ba_lin_kf)."""
    announce(f"ba iterate_n(3) {case}")
    p = (wl.ba_problem() if case == "window"
         else _dense_keyframe_problem(duplicate=case == "dense_keyframe_dup"))
    h, w = p["h"], p["w"]
    ref_p, ref_d = p["poses"], p["disps"]
    for _ in range(3):
        ref = oracle_iter(p, ref_p, ref_d, 1e-4, 0.1)
        assert ref["status"] == 0
        ref_p, ref_d = ref["poses"], ref["disps"]
    a, b = Dev(slk, p), Dev(slk, p)
    ctx_a = slk.Context(h, w, max_batch=1)
    ctx_b = slk.Context(h, w, max_batch=1)
    ctx_a.profile_enable(True)
    d = a.d
    ctx_a.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                       d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 3)
    assert ctx_a.ba_status() == slk.SLK_OK
    kernels = _path_kernels(ctx_a)
    if case == "window":
        assert {"ba_fz_lin", "ba_fz_asm", "ba_fz_step", "ba_fz_last"} <= kernels, kernels
    elif case == "dense_keyframe":
        assert {"ba_lin_wv", "ba_schur", "ba_backsub"} <= kernels, kernels
        assert "ba_lin_kf" not in kernels, kernels
    else:
        assert {"ba_lin_kf", "ba_schur", "ba_backsub"} <= kernels, kernels
        assert "ba_lin_wv" not in kernels, kernels
    for _ in range(3):
        b.iterate(ctx_b, 1e-4, 0.1)
    assert ctx_b.ba_status() == slk.SLK_OK
    assert norm_rel(a.poses(), ref_p) < TOL
    assert norm_rel(a.disps(), ref_d) < TOL
    assert_close_rel(a.poses(), ref_p, what="poses after iterate_n(3)")
    assert_close_rel(a.disps(), ref_d, what="disps after iterate_n(3)")
    assert norm_rel(a.poses() - p["poses"], ref_p - p["poses"]) < TOL
    # the same steps either way, up to fp64 summation order
    assert norm_rel(a.poses(), b.poses()) < 1e-6
    assert norm_rel(a.disps(), b.disps()) < 1e-6
    ctx_a.close()
    ctx_b.close()


def test_iterate_n_not_spd_leaves_state_untouched(slk):
    """A rejected step in the fused iteration: no retraction, and the
    back-substitution folded into the next launch is skipped as well."""
    p = wl.ba_problem(n=4, h=6, w=8, seed=2)
    p["weight"] = np.zeros_like(p["weight"])
    dev = Dev(slk, p)
    ctx = slk.Context(6, 8, C=128, max_batch=1, levels=2)
    d = dev.d
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 0.0, 0.0, 2)
    assert ctx.ba_status() == slk.SLK_E_NOT_SPD
    np.testing.assert_array_equal(dev.poses(), p["poses"])
    np.testing.assert_array_equal(dev.disps(), p["disps"])
    with pytest.raises(slk.SlkError):
        ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                         d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 0)
    ctx.close()


def test_iterate_n_wait_give_up_is_reported(slk):
    """The bounded wait inside an overlapped step launch: with the limit set to
    zero from the host, every linearization workgroup gives up without a poll,
    skipping its chunk's depth update and its next linearization, and every
    launch still ends; slk_ba_status reports it as SLK_E_HIP. The state left
    is the one slk.h states: the first step's solve ran (the poses take its
    step), no chunk applied its depth update, and the call's later steps took
    no step (the solve of the last launch saw the give-up). With the default
    limit restored, the next call on the same context runs normally and
    matches the oracle."""
    announce("ba iterate_n wait give-up (limit 0)")
    p = wl.ba_problem()
    dev = Dev(slk, p)
    ctx = slk.Context(p["h"], p["w"], max_batch=1)
    d = dev.d
    args = (d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"], d["ii"],
            d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1)
    ctx.ba_set_wait_limit(0)
    for iters in (2, 3):
        dev.d["poses"].upload(p["poses"])
        dev.d["disps"].upload(p["disps"])
        ctx.ba_iterate_n(*args, iters)
        assert ctx.ba_status() == slk.SLK_E_HIP
        assert b"stopped waiting" in slk.lib().slk_last_error()
        one = oracle_iter(p, p["poses"], p["disps"], 1e-4, 0.1)
        assert norm_rel(dev.poses(), one["poses"]) < TOL, iters
        assert norm_rel(dev.poses() - p["poses"], one["poses"] - p["poses"]) < TOL, iters
        np.testing.assert_array_equal(dev.disps(), p["disps"])
    ctx.ba_set_wait_limit(-1)
    dev2 = Dev(slk, p)
    d2 = dev2.d
    ctx.ba_iterate_n(d2["poses"], d2["disps"], d2["intr"], d2["target"], d2["weight"],
                     d2["eta"], d2["ii"], d2["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4,
                     0.1, 2)
    assert ctx.ba_status() == slk.SLK_OK
    ref_p, ref_d = p["poses"], p["disps"]
    for _ in range(2):
        ref = oracle_iter(p, ref_p, ref_d, 1e-4, 0.1)
        ref_p, ref_d = ref["poses"], ref["disps"]
    assert norm_rel(dev2.poses(), ref_p) < TOL
    assert norm_rel(dev2.disps(), ref_d) < TOL
    ctx.close()


@pytest.mark.parametrize("duplicate", [True, False])
def test_edge_cases_stereo_duplicates_absent_frame(slk, duplicate):
    # A stereo edge (1, 1), a frame (3) that is no keyframe and, optionally, a
    # duplicated (2, 3) edge. Every keyframe here has at most 7 E-row slots,
    # so a single iteration runs the fused path (k_ba_fz), whose E rows live
    # in LDS; the duplicate's two edges then add into the same slot. The
    # five-kernel path with a duplicated edge (k_ba_lin_kf) is the
    # dense_keyframe_dup case of test_iterate_n_matches_oracle_and_single_calls.
    ii = np.array([0, 1, 2, 1, 2, 0, 1] + ([2] if duplicate else []), np.int32)
    jj = np.array([1, 2, 3, 0, 1, 2, 1] + ([3] if duplicate else []), np.int32)
    p = wl.ba_problem(n=4, h=6, w=8, ii=ii, jj=jj, seed=8, fixed=1)
    p["eta"] = np.random.default_rng(9).uniform(0, 1e-3, p["eta"].shape).astype(np.float32)
    dev = Dev(slk, p)
    ctx = slk.Context(6, 8, C=128, max_batch=1, levels=2)
    ctx.profile_enable(True)
    dev.iterate(ctx, 1e-4, 0.1)
    assert "ba_fz_lin" in _path_kernels(ctx)
    S, b, dx = ctx.ba_last_system()
    ref = oracle_iter(p, p["poses"], p["disps"], 1e-4, 0.1)
    assert norm_rel(S, ref["S"]) < 1e-7
    assert norm_rel(dx, ref["dx"]) < 1e-5
    assert_close_rel(dev.poses(), ref["poses"])
    assert_close_rel(dev.disps(), ref["disps"])
    np.testing.assert_array_equal(dev.disps()[3], p["disps"][3])  # frame 3 not in ii
    ctx.close()


def test_not_spd_leaves_state_untouched(slk):
    p = wl.ba_problem(n=4, h=6, w=8, seed=2)
    p["weight"] = np.zeros_like(p["weight"])
    dev = Dev(slk, p)
    ctx = slk.Context(6, 8, C=128, max_batch=1, levels=2)
    dev.iterate(ctx, 0.0, 0.0)
    assert ctx.ba_status() == slk.SLK_E_NOT_SPD
    assert ctx.ba_status() == slk.SLK_OK  # flag cleared
    np.testing.assert_array_equal(dev.poses(), p["poses"])
    np.testing.assert_array_equal(dev.disps(), p["disps"])
    with pytest.raises(slk.SlkError):
        ctx.ba_iterate(*([dev.d["poses"]] * 6), dev.d["ii"], dev.d["jj"], p["ii"], p["jj"], 3, 3,
                       1e-4, 0.1)
    ctx.close()


@pytest.mark.parametrize("P", [11, 14, 15, 20, 21])
def test_lds_solver_sizes(slk, P):
    """P = 11 to 20 free poses (n = 66 to 120) take the one-workgroup LDL^T
    solve with the bordered system in LDS: n = 66, 84 and 90 are padded to
    72, 88 and 96 (identity rows), n = 120 is the largest (59 KB of LDS);
    P = 21 (n = 126): the first size of the blocked solve over many
    workgroups. One iteration against the oracle, then a second from the
    updated state."""
    announce(f"ba lds solver P={P} (n={6 * P})")
    n = P + 2
    p = wl.ba_problem(n=n, h=12, w=16, seed=30 + P)
    dev = Dev(slk, p)
    ctx = slk.Context(12, 16, max_batch=1, levels=2)
    poses, disps = p["poses"], p["disps"]
    for it in range(2):
        dev.iterate(ctx, 1e-4, 0.1)
        ref = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                             p["ii"], p["jj"], 12, 16, p["t0"], p["t1"], 1e-4, 0.1)
        assert ref["status"] == 0
        S, b, dx = ctx.ba_last_system()
        assert S.shape == (6 * P, 6 * P)
        assert norm_rel(S, ref["S"]) < 1e-7, it
        assert norm_rel(b, ref["b"]) < 1e-7, it
        assert norm_rel(dx, ref["dx"]) < 1e-5, it
        poses, disps = ref["poses"], ref["disps"]
        assert_close_rel(dev.poses(), poses, what=f"poses it {it}")
        assert_close_rel(dev.disps(), disps, what=f"disps it {it}")
    assert ctx.ba_status() == slk.SLK_OK
    ctx.close()
    if P > 20:
        return
    # three chained steps as one slk_ba_iterate_n call: the overlapped fused
    # steps, each solve (the panel solver from n = 66) in one launch with the
    # next linearization; the oracle's third step after the two above
    ref = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                         p["ii"], p["jj"], 12, 16, p["t0"], p["t1"], 1e-4, 0.1)
    assert ref["status"] == 0
    poses, disps = ref["poses"], ref["disps"]
    dev = Dev(slk, p)
    ctx = slk.Context(12, 16, max_batch=1, levels=2)
    ctx.profile_enable(True)
    d = dev.d
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 3)
    assert ctx.ba_status() == slk.SLK_OK
    assert {"ba_fz_step", "ba_fz_last"} <= _path_kernels(ctx)
    assert norm_rel(dev.poses(), poses) < TOL
    assert norm_rel(dev.disps(), disps) < TOL
    assert_close_rel(dev.poses(), poses, what="poses after iterate_n(3)")
    assert_close_rel(dev.disps(), disps, what="disps after iterate_n(3)")
    ctx.close()


def test_lds_solver_not_spd_late_pivot(slk):
    """P = 12 (n = 72, the one-workgroup LDS solve) with every edge that touches frames 12
    and 13 at zero weight and no damping: the rows of those two poses are
    zero, so the factorization fails at pivot 60, in a later column block than
    the first. Reported as SLK_E_NOT_SPD, poses and inverse depths untouched."""
    announce("ba lds solver P=12 late-pivot not SPD")
    p = wl.ba_problem(n=14, h=12, w=16, seed=41)
    dead = (p["ii"] >= 12) | (p["jj"] >= 12)
    assert dead.any() and not dead.all()
    p["weight"][dead] = 0.0
    ref = orc.ba_iterate(p["poses"], p["disps"], p["intr"], p["target"], p["weight"], p["eta"],
                         p["ii"], p["jj"], 12, 16, p["t0"], p["t1"], 0.0, 0.0)
    assert ref["status"] != 0
    dev = Dev(slk, p)
    ctx = slk.Context(12, 16, max_batch=1, levels=2)
    dev.iterate(ctx, 0.0, 0.0)
    assert ctx.ba_status() == slk.SLK_E_NOT_SPD
    np.testing.assert_array_equal(dev.poses(), p["poses"])
    np.testing.assert_array_equal(dev.disps(), p["disps"])
    # the same context then solves a well-posed system of the same size
    dev.d["weight"].upload(wl.ba_problem(n=14, h=12, w=16, seed=41)["weight"])
    q = wl.ba_problem(n=14, h=12, w=16, seed=41)
    dev.iterate(ctx, 1e-4, 0.1)
    assert ctx.ba_status() == slk.SLK_OK
    ref = orc.ba_iterate(q["poses"], q["disps"], q["intr"], q["target"], q["weight"], q["eta"],
                         q["ii"], q["jj"], 12, 16, q["t0"], q["t1"], 1e-4, 0.1)
    assert_close_rel(dev.poses(), ref["poses"], what="poses after recovery")
    assert_close_rel(dev.disps(), ref["disps"], what="disps after recovery")
    ctx.close()


def test_large_system_and_plan_cache(slk):
    """30 frames, P = 28 free poses (n = 168, the global-memory solve), then a
    different edge set and back (index structures rebuilt and reused)."""
    announce("ba large n=168 + plan cache")
    n = 30
    ii, jj = wl.cyclic_edges(n)
    p = wl.ba_problem(n=n, h=24, w=32, ii=ii, jj=jj, seed=12)
    dev = Dev(slk, p)
    ctx = slk.Context(24, 32, max_batch=1)
    poses, disps = p["poses"], p["disps"]
    for step, sel in enumerate([slice(None), slice(0, 80), slice(None)]):
        q = dict(p, ii=ii[sel], jj=jj[sel], target=p["target"][sel], weight=p["weight"][sel],
                 poses=poses, disps=disps)
        dev.d["target"].upload(np.ascontiguousarray(np.concatenate(
            [q["target"], np.zeros((len(ii) - len(q["ii"]),) + p["target"].shape[1:], np.float32)])))
        dev.d["weight"].upload(np.ascontiguousarray(np.concatenate(
            [q["weight"], np.zeros((len(ii) - len(q["ii"]),) + p["weight"].shape[1:], np.float32)])))
        dev.iterate(ctx, 1e-4, 0.1, ii=np.ascontiguousarray(q["ii"]), jj=np.ascontiguousarray(q["jj"]))
        ref = orc.ba_iterate(poses, disps, p["intr"], q["target"], q["weight"], p["eta"], q["ii"],
                             q["jj"], 24, 32, p["t0"], p["t1"], 1e-4, 0.1)
        S, b, dx = ctx.ba_last_system()
        assert S.shape == (168, 168)
        assert norm_rel(S, ref["S"]) < 1e-7, step
        assert norm_rel(dx, ref["dx"]) < 1e-5, step
        poses, disps = ref["poses"], ref["disps"]
        assert_close_rel(dev.poses(), poses, what=f"poses step {step}")
        assert_close_rel(dev.disps(), disps, what=f"disps step {step}")
    ctx.close()


def test_backend_geometry_1188(slk):
    """Config backend's BA geometry: 200 keyframes, 2000 edges (|i-j| <= 2 plus
    random long-range pairs), 198 free poses -> a 1188 x 1188 Schur system, at
    6x8 pixels per frame so the oracle's dense fp64 Cholesky stays quick. The
    reference backend's lm = 1e-5, ep = 1e-2 (main.cu:2487-2488); two chained
    iterations."""
    announce("ba backend geometry n=1188")
    ii, jj = wl.backend_edges(200, 2000)
    p = wl.ba_problem(n=200, h=6, w=8, ii=ii, jj=jj, seed=21)
    dev = Dev(slk, p)
    ctx = slk.Context(6, 8, max_batch=1, levels=1)
    poses, disps = p["poses"], p["disps"]
    for step in range(2):
        dev.iterate(ctx, 1e-5, 1e-2)
        assert ctx.ba_status() == slk.SLK_OK
        ref = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                             p["ii"], p["jj"], 6, 8, p["t0"], p["t1"], 1e-5, 1e-2)
        assert ref["status"] == 0
        S, b, dx = ctx.ba_last_system()
        assert S.shape == (1188, 1188)
        assert norm_rel(S, ref["S"]) < 1e-7, step
        assert norm_rel(dx, ref["dx"]) < 1e-5, step
        poses, disps = ref["poses"], ref["disps"]
        assert norm_rel(dev.poses(), poses) < TOL, step
        assert norm_rel(dev.disps(), disps) < TOL, step
    ctx.close()


def _homogeneous_depth(p):
    """Homogeneous depth of every edge-pixel at the problem's poses: the
    camera-j depth times the source pixel's inverse depth, the quantity
    ba.cuh:117-122 compares with MIN_DEPTH = 0.25 (se3.cuh:6)."""
    _, depth = wl.project(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], p["h"], p["w"])
    return depth * p["disps"][p["ii"]].reshape(len(p["ii"]), -1)


def test_iterate_n_masked_pixels_overlapped_steps(slk):
    """The cfg3 window with the free frames moving forward (tz_step 0.1), so
    5.5% of its edge-pixels, on five edges, lie behind MIN_DEPTH: their
    weights and inverse depth are masked (ba.cuh:117-122) in every
    linearization, including the overlapped step launches (k_ba_fz_step), whose
    relinearization and depth update see them too. slk_ba_iterate_n(3)
    against three chained oracle iterations, and S, b, dx of a single
    iteration."""
    announce("ba iterate_n(3) masked pixels (cfg3 window, tz_step 0.1)")
    p = wl.ba_problem(seed=23, tz_step=0.1)
    zh = _homogeneous_depth(p)
    assert (zh < 0.25).mean() >= 0.05, (zh < 0.25).mean()
    assert np.abs(zh - 0.25).min() > 1e-4  # no pixel the fp64 orders could classify apart
    ref_p, ref_d = p["poses"], p["disps"]
    refs = []
    for _ in range(3):
        ref = oracle_iter(p, ref_p, ref_d, 1e-4, 0.1)
        assert ref["status"] == 0
        refs.append(ref)
        ref_p, ref_d = ref["poses"], ref["disps"]
    one = Dev(slk, p)
    ctx1 = slk.Context(p["h"], p["w"], max_batch=1)
    one.iterate(ctx1, 1e-4, 0.1)
    assert ctx1.ba_status() == slk.SLK_OK
    S, b, dx = ctx1.ba_last_system()
    assert norm_rel(S, refs[0]["S"]) < 1e-7
    assert norm_rel(b, refs[0]["b"]) < 1e-7
    assert norm_rel(dx, refs[0]["dx"]) < 1e-5
    ctx1.close()
    dev = Dev(slk, p)
    ctx = slk.Context(p["h"], p["w"], max_batch=1)
    ctx.profile_enable(True)
    d = dev.d
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 3)
    assert ctx.ba_status() == slk.SLK_OK
    assert {"ba_fz_lin", "ba_fz_step", "ba_fz_last"} <= _path_kernels(ctx)
    assert norm_rel(dev.poses(), ref_p) < TOL
    assert norm_rel(dev.disps(), ref_d) < TOL
    assert norm_rel(dev.poses() - p["poses"], ref_p - p["poses"]) < TOL
    assert_close_rel(dev.poses(), ref_p, what="poses after iterate_n(3), masked")
    assert_close_rel(dev.disps(), ref_d, what="disps after iterate_n(3), masked")
    ctx.close()


def test_iterate_n_all_pixels_masked(slk):
    """Every edge-pixel behind MIN_DEPTH (SURVEY's forcible case): all
    weights are masked, so H and the gradients vanish, S is the damping
    ep * I, dx = 0 and every inverse depth stays as it was. Run through the
    overlapped fused steps of slk_ba_iterate_n(3)."""
    announce("ba iterate_n(3) every pixel masked")
    ii = np.array([0, 1, 0, 1, 2], np.int32)
    jj = np.array([2, 3, 3, 2, 3], np.int32)
    p = wl.ba_problem(n=4, h=12, w=16, ii=ii, jj=jj, seed=6, fixed=1, tz_step=1.0,
                      disp_range=(1.0, 2.0))
    assert (_homogeneous_depth(p) < 0.25).all()
    ref = oracle_iter(p, p["poses"], p["disps"], 1e-4, 0.1)
    assert ref["status"] == 0
    assert not ref["dx"].any() and not ref["b"].any()
    np.testing.assert_array_equal(ref["disps"], p["disps"])
    dev = Dev(slk, p)
    ctx = slk.Context(12, 16, max_batch=1, levels=2)
    ctx.profile_enable(True)
    d = dev.d
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-4, 0.1, 3)
    assert ctx.ba_status() == slk.SLK_OK
    assert {"ba_fz_step", "ba_fz_last"} <= _path_kernels(ctx)
    S, b, dx = ctx.ba_last_system()
    assert not dx.any() and not b.any()
    np.testing.assert_array_equal(S, np.diag(np.diag(S)))  # the damping alone
    np.testing.assert_allclose(np.diag(S), np.float32(0.1), rtol=1e-12)
    np.testing.assert_array_equal(S, ref["S"])
    np.testing.assert_array_equal(dev.disps(), p["disps"])
    assert_close_rel(dev.poses(), ref["poses"], what="poses, every pixel masked")
    ctx.close()


def test_backend_full_size_iterate_n5(slk):
    """Config backend's BA leg at its real size: 200 keyframes of 48x64,
    backend_edges(200, 2000), 198 free poses (a 1188 x 1188 Schur system),
    the reference backend's lm = 1e-5, ep = 1e-2 (main.cu:2486-2489), five
    iterations in one slk_ba_iterate_n call against five chained oracle
    iterations; S and b (1e-7) and dx (1e-5) of a single iteration first."""
    announce("ba backend full size: 200 x 48x64, 2000 edges, iterate_n(5)")
    ii, jj = wl.backend_edges(200, 2000)
    p = wl.ba_problem(n=200, h=48, w=64, ii=ii, jj=jj, seed=21)
    one = Dev(slk, p)
    ctx1 = slk.Context(48, 64, max_batch=1)
    one.iterate(ctx1, 1e-5, 1e-2)
    assert ctx1.ba_status() == slk.SLK_OK
    S, b, dx = ctx1.ba_last_system()
    ctx1.close()
    dev = Dev(slk, p)
    ctx = slk.Context(48, 64, max_batch=1)
    d = dev.d
    ctx.ba_iterate_n(d["poses"], d["disps"], d["intr"], d["target"], d["weight"], d["eta"],
                     d["ii"], d["jj"], p["ii"], p["jj"], p["t0"], p["t1"], 1e-5, 1e-2, 5)
    assert ctx.ba_status() == slk.SLK_OK
    got_p, got_d = dev.poses(), dev.disps()
    ctx.close()
    poses, disps = p["poses"], p["disps"]
    for it in range(5):
        ref = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                             p["ii"], p["jj"], 48, 64, p["t0"], p["t1"], 1e-5, 1e-2)
        announce(f"  oracle iteration {it + 1} of 5 done")
        assert ref["status"] == 0
        if it == 0:
            assert S.shape == (1188, 1188)
            assert norm_rel(S, ref["S"]) < 1e-7
            assert norm_rel(b, ref["b"]) < 1e-7
            assert norm_rel(dx, ref["dx"]) < 1e-5
            assert_close_rel(one.poses(), ref["poses"], what="poses after one iteration")
            assert_close_rel(one.disps(), ref["disps"], what="disps after one iteration")
        poses, disps = ref["poses"], ref["disps"]
    assert norm_rel(got_p, poses) < TOL
    assert norm_rel(got_d, disps) < TOL
    assert norm_rel(got_p - p["poses"], poses - p["poses"]) < TOL
    assert_close_rel(got_p, poses, what="poses after iterate_n(5)")
    assert_close_rel(got_d, disps, what="disps after iterate_n(5)")


# ------------------------------------------------------------ stage kernels --
def test_projective_transform_stage(slk):
    p = wl.ba_problem(n=6, h=24, w=32, seed=4)
    M = len(p["ii"])
    HW = 24 * 32
    d = {k: slk.DeviceArray.from_host(p[k])
         for k in ("target", "weight", "poses", "disps", "intr", "ii", "jj")}
    outs = {"Hs": (4, M, 36), "vs": (2, M, 6), "Eii": (M, 6, HW), "Eij": (M, 6, HW),
            "Cii": (M, HW), "bz": (M, HW)}
    o = {k: slk.DeviceArray(s) for k, s in outs.items()}
    slk.check(slk.lib().slk_ba_projective_transform(
        d["target"].ptr, d["weight"].ptr, d["poses"].ptr, d["disps"].ptr, d["intr"].ptr,
        d["ii"].ptr, d["jj"].ptr, o["Hs"].ptr, o["vs"].ptr, o["Eii"].ptr, o["Eij"].ptr,
        o["Cii"].ptr, o["bz"].ptr, M, 24, 32, None))
    slk.hip().sync()
    ref = orc.ba_linearize(p["target"], p["weight"], p["poses"], p["disps"], p["intr"], p["ii"],
                           p["jj"], 24, 32)
    for name, r in zip(("Hs", "vs", "Eii", "Eij", "Cii", "bz"), ref):
        assert_close_rel(o[name].to_host().reshape(r.shape), r, tol=1e-5, what=name)


def test_schur_stage_kernels(slk):
    pin = Pins(slk)
    rng = np.random.default_rng(7)
    D, NE, NK = 300, 5, 3
    E = rng.normal(size=(NE, 6, D)).astype(np.float32)
    C = rng.uniform(0.5, 2.0, (NK, D)).astype(np.float32)
    eta = rng.uniform(0, 1, (7, D)).astype(np.float32)
    kf_map = np.array([6, 2, 4], np.int32)
    w = rng.normal(size=(NK, D)).astype(np.float32)
    dE = slk.DeviceArray.from_host(E)
    dC = slk.DeviceArray.from_host(C)
    dQ = slk.DeviceArray((NK, D))
    lib = slk.lib()
    slk.check(lib.slk_ba_damping_q(dC.ptr, pin(eta),
                                   pin(kf_map), dQ.ptr, NK, D, 1e-7, None))
    slk.hip().sync()
    Cref = C.astype(np.float64) + 0.2 * eta[kf_map] + 1e-7
    assert_close_rel(dC.to_host(), Cref, tol=1e-6)
    Q = dQ.to_host()
    assert_close_rel(Q, 1.0 / Cref, tol=1e-6)
    idx = np.array([[0, 1, 0], [2, 2, 1], [4, 3, 2]], np.int32)
    S = slk.DeviceArray((3, 36))
    slk.check(lib.slk_ba_eet6x6(dE.ptr, dQ.ptr, pin(idx), S.ptr, D, 3,
                                None))
    v = slk.DeviceArray.from_host(np.ones((NE, 6), np.float32))
    ev_idx = np.array([0, 0, 1, 2, 2], np.int32)
    dw = slk.DeviceArray.from_host(w)
    slk.check(lib.slk_ba_ev6x1(dE.ptr, dQ.ptr, dw.ptr, pin(ev_idx), v.ptr,
                               D, NE, None))
    x = rng.normal(size=(4, 6)).astype(np.float32)
    evt_idx = np.array([0, 3, 1, -1, 2], np.int32)
    wout = slk.DeviceArray((NE, D))
    wout.zero()
    slk.check(lib.slk_ba_evt6x1(dE.ptr, pin(x),
                                pin(evt_idx), wout.ptr, D, NE, 4, None))
    slk.hip().sync()
    E64, Q64 = E.astype(np.float64), Q.astype(np.float64)
    for k, (a, b_, c) in enumerate(idx):
        assert_close_rel(S.to_host()[k].reshape(6, 6), (E64[a] * Q64[c]) @ E64[b_].T, tol=1e-5)
    vref = 1.0 + np.stack([(E64[r] * Q64[ev_idx[r]] * w[ev_idx[r]]).sum(-1) for r in range(NE)])
    assert_close_rel(v.to_host(), vref, tol=1e-5)
    wref = np.stack([x[evt_idx[r]].astype(np.float64) @ E64[r] if evt_idx[r] >= 0 else np.zeros(D)
                     for r in range(NE)])
    assert_close_rel(wout.to_host(), wref, tol=1e-5)
    # accum / accum_add (CSR gather-sum) and depth_update
    ptrs = np.array([0, 2, 2, 5], np.int32)
    idxs = np.array([4, 0, 1, 3, 2], np.int32)
    src = rng.normal(size=(5, D)).astype(np.float32)
    out = slk.DeviceArray.from_host(np.full((3, D), 2.0, np.float32))
    for add in (0, 1):
        slk.check(lib.slk_ba_accum(pin(src),
                                   pin(ptrs),
                                   pin(idxs), out.ptr, 3, D, add, None))
    slk.hip().sync()
    acc = np.stack([src[idxs[ptrs[r]:ptrs[r + 1]]].astype(np.float64).sum(0) for r in range(3)])
    assert_close_rel(out.to_host(), 2 * acc, tol=1e-6)
    disps = rng.uniform(0.5, 1, (7, D)).astype(np.float32)
    dd = slk.DeviceArray.from_host(disps)
    dwv = rng.normal(size=(NK, D)).astype(np.float32)
    slk.check(lib.slk_ba_depth_update(dQ.ptr, dw.ptr, pin(dwv), dd.ptr,
                                      pin(kf_map), NK, D, None))
    slk.hip().sync()
    want = disps.astype(np.float64).copy()
    want[kf_map] += Q64 * (w.astype(np.float64) - dwv)
    assert_close_rel(dd.to_host(), want, tol=1e-6)
