"""Pins the CPU oracle's SE3 functions, projmap, frame distance and bundle
adjustment (oracle/oracle.c) against mathematics that does not restate it:

* SE3: scipy.linalg.expm of the 4x4 twist (exp map, retraction = exp(xi)*T),
  quaternion rotation matrices (act, rel), the adjoint identity
  <adj(T, X), xi> = <X, Ad_T xi> with Ad_T xi = log(T exp(xi) T^-1);
* projmap: an independent fp64 pinhole reprojection (workloads.project);
* BA linearization: central finite differences of that reprojection give Ji,
  Jj and Jz, read back through vs / bz with a single unit-residual pixel;
* one BA iteration: a brute-force dense fp64 assembly of the full pose+depth
  normal equations from finite-difference Jacobians, Schur-reduced with the
  reference's damping (depth: C + 0.2 eta + 1e-7; poses: S_ii += ep + lm S_ii
  after the Schur step), compared on S, b, dx, dz, poses and disps;
* the Cholesky solve against numpy.linalg.solve, and an indefinite matrix.
"""
import numpy as np
import pytest
from scipy.linalg import expm, logm

from oracle import oracle as orc
import workloads as wl


@pytest.fixture(scope="module", autouse=True)
def _build():
    orc.build()


def skew(v):
    return np.array([[0, -v[2], v[1]], [v[2], 0, -v[0]], [-v[1], v[0], 0]])


def twist(xi):
    T = np.zeros((4, 4))
    T[:3, :3] = skew(xi[3:])
    T[:3, 3] = xi[:3]
    return T


def pose_mat(t, q):
    T = np.eye(4)
    T[:3, :3] = wl.quat_to_matrix(np.asarray(q, np.float64))
    T[:3, 3] = t
    return T


def mat_pose(T):
    from scipy.spatial.transform import Rotation
    q = Rotation.from_matrix(T[:3, :3]).as_quat()  # xyzw
    return T[:3, 3].copy(), q


def rand_pose(rng, rot=0.5, trans=1.0):
    q = wl.quat_from_rotvec(rng.normal(0, rot, 3))
    return rng.normal(0, trans, 3), q


@pytest.mark.parametrize("scale", [1.0, 1e-3, 1e-5, 0.0])
def test_exp_se3_matches_expm(scale):
    rng = np.random.default_rng(0)
    for _ in range(20):
        xi = rng.normal(0, 1, 6) * scale
        t, q = orc.exp_se3(xi)
        T = expm(twist(xi))
        np.testing.assert_allclose(pose_mat(t, q), T, atol=1e-9)
        assert abs(np.linalg.norm(q) - 1) < 1e-12


def test_act_rel_retr():
    rng = np.random.default_rng(1)
    for _ in range(20):
        ti, qi = rand_pose(rng)
        tj, qj = rand_pose(rng)
        X = np.append(rng.normal(0, 1, 3), rng.uniform(0.2, 2))
        Y = orc.act_se3(ti, qi, X)
        Ti = pose_mat(ti, qi)
        np.testing.assert_allclose(Y, Ti @ X, atol=1e-12)  # homogeneous action
        tij, qij = orc.rel_se3(ti, qi, tj, qj)
        np.testing.assert_allclose(pose_mat(tij, qij), pose_mat(tj, qj) @ np.linalg.inv(Ti),
                                   atol=1e-12)
        xi = rng.normal(0, 0.3, 6)
        t1, q1 = orc.retr_se3(xi, ti, qi)
        np.testing.assert_allclose(pose_mat(t1, q1), expm(twist(xi)) @ Ti, atol=1e-10)
        # retr(-xi) o retr(xi) = identity
        t2, q2 = orc.retr_se3(-xi, t1, q1)
        np.testing.assert_allclose(pose_mat(t2, q2), Ti, atol=1e-10)


def test_adj_is_adjoint_transpose():
    rng = np.random.default_rng(2)
    for _ in range(10):
        t, q = rand_pose(rng)
        T = pose_mat(t, q)
        X = rng.normal(0, 1, 6)
        Y = orc.adj_se3(t, q, X)
        for n in range(6):
            xi = np.zeros(6)
            xi[n] = 1.0
            L = np.real(logm(T @ expm(twist(1e-3 * xi)) @ np.linalg.inv(T))) / 1e-3
            ad_xi = np.array([L[0, 3], L[1, 3], L[2, 3], L[2, 1], L[0, 2], L[1, 0]])
            # Y_n = <adj(T,X), e_n> = <X, Ad_T e_n>
            assert abs(Y[n] - X @ ad_xi) < 1e-5 * (1 + np.abs(X).sum())


def test_projmap_matches_pinhole():
    p = wl.ba_problem(n=5, h=12, w=16, ii=np.array([0, 1, 2, 4]), jj=np.array([1, 3, 0, 2]),
                      seed=4)
    coords, valid = orc.projmap(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], 12, 16)
    ref, depth = wl.project(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], 12, 16)
    np.testing.assert_allclose(coords.reshape(4, -1, 2).transpose(0, 2, 1), ref, rtol=1e-6,
                               atol=1e-4)
    # valid = Z_j > 0.25 in the reprojection (depth scaled by disparity)
    zs = depth * p["disps"][p["ii"]].reshape(4, -1)
    np.testing.assert_array_equal(valid.reshape(4, -1), (zs > 0.25).astype(np.float32))


def test_pose_retr_and_disp_retr():
    rng = np.random.default_rng(3)
    poses = np.zeros((5, 7), np.float32)
    for k in range(5):
        t, q = rand_pose(rng)
        poses[k, :3], poses[k, 3:] = t, q
    dx = rng.normal(0, 0.1, (3, 6)).astype(np.float32)
    out = orc.pose_retr(poses, dx, 1, 4)
    np.testing.assert_array_equal(out[[0, 4]], poses[[0, 4]])
    for k in range(1, 4):
        want = expm(twist(dx[k - 1].astype(np.float64))) @ pose_mat(poses[k, :3], poses[k, 3:])
        np.testing.assert_allclose(pose_mat(out[k, :3], out[k, 3:]), want, atol=1e-6)
    d = rng.uniform(0.1, 1, (4, 6)).astype(np.float32)
    dz = rng.normal(0, 0.5, (2, 6)).astype(np.float32)
    r = orc.disp_retr(d, dz, np.array([3, 1], np.int32))
    want = d.copy()
    want[3] = np.maximum(d[3] + dz[0], 0.001)
    want[1] = np.maximum(d[1] + dz[1], 0.001)
    np.testing.assert_array_equal(r, want)


def test_frame_distance_formula():
    p = wl.ba_problem(n=4, h=6, w=8, ii=np.array([0, 1, 2]), jj=np.array([1, 0, 3]), seed=6)
    beta = 0.3
    got = orc.frame_distance(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], 6, 8, beta)
    full, depth = wl.project(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], 6, 8)
    # translation-only reprojection: same with the rotation removed
    tposes = p["poses"].copy()
    ref = []
    for e, (i, j) in enumerate(zip(p["ii"], p["jj"])):
        Ti = pose_mat(p["poses"][i, :3], p["poses"][i, 3:])
        Tj = pose_mat(p["poses"][j, :3], p["poses"][j, 3:])
        tij = (Tj @ np.linalg.inv(Ti))[:3, 3]
        tposes[:] = [0, 0, 0, 0, 0, 0, 1]
        tposes[j, :3] = tij
        tr, tdepth = wl.project(tposes, p["disps"], p["intr"], [i], [j], 6, 8)
        grid = wl.grid_coords(6, 8)
        d1 = np.hypot(*(full[e] - grid))
        d2 = np.hypot(*(tr[0] - grid))
        z1 = depth[e] * p["disps"][i].reshape(-1)
        z2 = tdepth[0] * p["disps"][i].reshape(-1)
        acc = beta * d1[z1 > 0.25].sum() + (1 - beta) * d2[z2 > 0.25].sum()
        val = beta * (z1 > 0.25).sum() + (1 - beta) * (z2 > 0.25).sum()
        tot = 48.0
        ref.append(1000.0 if val / (tot + 1e-8) < 0.75 else acc / val)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------- BA ---
def proj_pixel(poses64, disp, intr, i, j, u, v, stereo=False):
    """Reprojection of pixel (u,v) of frame i into j with inverse depth disp."""
    fx, fy, cx, cy = intr
    if stereo:
        Tij = np.eye(4)
        Tij[0, 3] = -0.1
    else:
        Tij = poses64[j] @ np.linalg.inv(poses64[i])
    Xh = np.array([(u - cx) / fx, (v - cy) / fy, 1.0, disp])
    Y = Tij @ Xh
    return np.array([fx * Y[0] / Y[2] + cx, fy * Y[1] / Y[2] + cy]), Y[2]


def fd_jacobians(poses64, disp, intr, i, j, u, v, h=1e-6):
    Ji, Jj = np.zeros((2, 6)), np.zeros((2, 6))
    for n in range(6):
        e = np.zeros(6)
        e[n] = h
        for k, J in ((i, Ji), (j, Jj)):
            pp, pm = [P.copy() for P in poses64], [P.copy() for P in poses64]
            pp[k] = expm(twist(e)) @ poses64[k]
            pm[k] = expm(twist(-e)) @ poses64[k]
            J[:, n] = (proj_pixel(pp, disp, intr, i, j, u, v)[0] -
                       proj_pixel(pm, disp, intr, i, j, u, v)[0]) / (2 * h)
    Jz = (proj_pixel(poses64, disp + h, intr, i, j, u, v)[0] -
          proj_pixel(poses64, disp - h, intr, i, j, u, v)[0]) / (2 * h)
    return Ji, Jj, Jz


def poses_to_mats(poses):
    return [pose_mat(p[:3].astype(np.float64), p[3:].astype(np.float64)) for p in poses]


def test_ba_linearize_jacobians_finite_difference():
    h, w = 6, 8
    p = wl.ba_problem(n=3, h=h, w=w, ii=np.array([0, 2]), jj=np.array([1, 1]), seed=7)
    mats = poses_to_mats(p["poses"])
    intr = p["intr"].astype(np.float64)
    for comp in (0, 1):
        for k in (0, 13, 47):
            u, v = k % w, k // w
            weight = np.zeros_like(p["weight"])
            target = p["target"].copy()
            for e, (i, j) in enumerate(zip(p["ii"], p["jj"])):
                weight[e, comp, k] = 1000.0  # 0.001*weight = 1
                pr, _ = proj_pixel(mats, float(p["disps"][i].reshape(-1)[k]), intr, i, j, u, v)
                target[e, comp, k] = np.float32(pr[comp] + 1.0)  # unit residual
            Hs, vs, Eii, Eij, Cii, bz = orc.ba_linearize(target, weight, p["poses"], p["disps"],
                                                         p["intr"], p["ii"], p["jj"], h, w)
            for e, (i, j) in enumerate(zip(p["ii"], p["jj"])):
                d = float(p["disps"][i].reshape(-1)[k])
                Ji, Jj, Jz = fd_jacobians(mats, d, intr, i, j, u, v)
                pr, _ = proj_pixel(mats, d, intr, i, j, u, v)
                r = float(target[e, comp, k]) - pr[comp]
                np.testing.assert_allclose(vs[0, e], r * Ji[comp], rtol=1e-5, atol=1e-6)
                np.testing.assert_allclose(vs[1, e], r * Jj[comp], rtol=1e-5, atol=1e-6)
                np.testing.assert_allclose(bz[e, k], r * Jz[comp], rtol=1e-5, atol=1e-6)
                np.testing.assert_allclose(Cii[e, k], Jz[comp] ** 2, rtol=1e-5, atol=1e-6)
                np.testing.assert_allclose(Hs[0, e], np.outer(Ji[comp], Ji[comp]), rtol=1e-5,
                                           atol=1e-5)
                np.testing.assert_allclose(Hs[1, e], np.outer(Ji[comp], Jj[comp]), rtol=1e-5,
                                           atol=1e-5)
                np.testing.assert_allclose(Hs[2, e], np.outer(Jj[comp], Ji[comp]), rtol=1e-5,
                                           atol=1e-5)
                np.testing.assert_allclose(Hs[3, e], np.outer(Jj[comp], Jj[comp]), rtol=1e-5,
                                           atol=1e-5)
                np.testing.assert_allclose(Eii[e, :, k], Jz[comp] * Ji[comp], rtol=1e-5,
                                           atol=1e-6)
                np.testing.assert_allclose(Eij[e, :, k], Jz[comp] * Jj[comp], rtol=1e-5,
                                           atol=1e-6)


def brute_force_step(p, lm, ep, motion_only=False):
    """Dense fp64 GN step assembled from finite-difference Jacobians."""
    poses, disps, intr = p["poses"], p["disps"], p["intr"].astype(np.float64)
    ii, jj, t0, t1, H, W = p["ii"], p["jj"], p["t0"], p["t1"], p["h"], p["w"]
    HW = H * W
    P = t1 - t0
    mats = poses_to_mats(poses)
    kfs = sorted(set(int(i) for i in ii))
    dcol = {kf: 6 * P + n * HW for n, kf in enumerate(kfs)}
    nvar = 6 * P + (0 if motion_only else len(kfs) * HW)
    Hm = np.zeros((nvar, nvar))
    g = np.zeros(nvar)
    for e, (i, j) in enumerate(zip(ii, jj)):
        i, j = int(i), int(j)
        for k in range(HW):
            u, v = k % W, k // W
            d = float(disps[i].reshape(-1)[k])
            pr, z = proj_pixel(mats, d, intr, i, j, u, v, stereo=(i == j))
            if z < 0.25:
                continue
            if i == j:
                Ji = Jj = np.zeros((2, 6))
                Jz = (proj_pixel(mats, d + 1e-6, intr, i, j, u, v, True)[0] -
                      proj_pixel(mats, d - 1e-6, intr, i, j, u, v, True)[0]) / 2e-6
            else:
                Ji, Jj, Jz = fd_jacobians(mats, d, intr, i, j, u, v)
            for comp in (0, 1):
                wgt = 0.001 * float(p["weight"][e, comp].reshape(-1)[k])
                r = float(p["target"][e, comp].reshape(-1)[k]) - pr[comp]
                row = np.zeros(nvar)
                if t0 <= i < t1:
                    row[6 * (i - t0):6 * (i - t0) + 6] += Ji[comp]
                if t0 <= j < t1:
                    row[6 * (j - t0):6 * (j - t0) + 6] += Jj[comp]
                if not motion_only:
                    row[dcol[i] + k] = Jz[comp]
                Hm += wgt * np.outer(row, row)
                g += wgt * r * row
    npo = 6 * P
    S = Hm[:npo, :npo].copy()
    b = g[:npo].copy()
    if not motion_only:
        C = np.diag(Hm)[npo:].copy()
        eta = np.concatenate([p["eta"][kf].reshape(-1) for kf in kfs]).astype(np.float64)
        C += 0.2 * eta + 1e-7
        Epd = Hm[:npo, npo:]
        S -= Epd @ (Epd / C).T
        b -= Epd @ (g[npo:] / C)
    S += np.diag(ep + lm * np.diag(S))
    dx = np.linalg.solve(S, b)
    dz = None
    if not motion_only:
        dz = (g[npo:] - Epd.T @ dx.astype(np.float32).astype(np.float64)) / C
    return S, b, dx, dz, kfs


@pytest.mark.parametrize("motion_only", [False, True])
def test_ba_iterate_matches_brute_force(motion_only):
    # 4 frames of 3x4 px, pose 0 fixed, one stereo edge, a duplicate edge and
    # a frame (3) that never appears in ii
    ii = np.array([0, 1, 2, 1, 2, 0, 1, 2], np.int32)
    jj = np.array([1, 2, 3, 0, 1, 2, 1, 3], np.int32)
    p = wl.ba_problem(n=4, h=3, w=4, ii=ii, jj=jj, seed=8, fixed=1, noise_px=0.5)
    p["eta"] = np.random.default_rng(9).uniform(0, 1e-3, p["eta"].shape).astype(np.float32)
    lm, ep = 1e-4, 0.1
    res = orc.ba_iterate(p["poses"], p["disps"], p["intr"], p["target"], p["weight"], p["eta"],
                         ii, jj, 3, 4, p["t0"], p["t1"], lm, ep, motion_only)
    assert res["status"] == 0
    S, b, dx, dz, kfs = brute_force_step(p, lm, ep, motion_only)
    np.testing.assert_allclose(res["S"], S, rtol=1e-6, atol=1e-6 * np.abs(S).max())
    np.testing.assert_allclose(res["b"], b, rtol=1e-6, atol=1e-6 * np.abs(b).max())
    np.testing.assert_allclose(res["dx"], dx, rtol=1e-5, atol=1e-6 * np.abs(dx).max())
    want_poses = orc.pose_retr(p["poses"], dx.astype(np.float32).reshape(-1, 6), 1, 4)
    np.testing.assert_allclose(res["poses"], want_poses, atol=1e-6)
    if motion_only:
        np.testing.assert_array_equal(res["disps"], p["disps"])
    else:
        HW = 12
        for n, kf in enumerate(kfs):
            np.testing.assert_allclose(res["dz"][kf], dz[n * HW:(n + 1) * HW], rtol=1e-5,
                                       atol=1e-6 * np.abs(dz).max())
        np.testing.assert_array_equal(res["disps"][3], p["disps"][3])  # not in ii
        np.testing.assert_allclose(res["disps"][kfs].reshape(len(kfs), -1),
                                   p["disps"][kfs].reshape(len(kfs), -1) + dz.reshape(len(kfs), -1),
                                   rtol=1e-5, atol=1e-6)


def test_ba_zero_residual_fixed_point():
    p = wl.ba_problem(n=4, h=6, w=8, seed=10, fixed=2, noise_px=0.0)
    proj, _ = wl.project(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], 6, 8)
    res = orc.ba_iterate(p["poses"], p["disps"], p["intr"], proj.astype(np.float32), p["weight"],
                         p["eta"], p["ii"], p["jj"], 6, 8, 2, 4, 1e-4, 0.1)
    assert res["status"] == 0
    assert np.abs(res["dx"]).max() < 1e-4
    assert np.abs(res["dz"]).max() < 1e-4


def test_ba_cost_decreases():
    p = wl.ba_problem(n=6, h=12, w=16, seed=11, fixed=2, noise_px=0.5)

    def cost(poses, disps):
        proj, depth = wl.project(poses, disps, p["intr"], p["ii"], p["jj"], 12, 16)
        r = p["target"].reshape(proj.shape) - proj
        return float((p["weight"].reshape(proj.shape) * r * r).sum())

    poses, disps = p["poses"], p["disps"]
    c0 = cost(poses, disps)
    for _ in range(3):
        res = orc.ba_iterate(poses, disps, p["intr"], p["target"], p["weight"], p["eta"],
                             p["ii"], p["jj"], 12, 16, 2, 6, 1e-4, 0.1)
        poses, disps = res["poses"], res["disps"]
    assert cost(poses, disps) < 0.9 * c0


def test_cholesky_solve_and_not_spd():
    rng = np.random.default_rng(12)
    A = rng.normal(size=(30, 30))
    S = A @ A.T + 30 * np.eye(30)
    b = rng.normal(size=30)
    st, x = orc.cholesky_solve(S, b)
    assert st == 0
    np.testing.assert_allclose(x, np.linalg.solve(S, b), rtol=1e-10)
    S[5, 5] = -1.0
    st, _ = orc.cholesky_solve(S, b)
    assert st == 3


# ------------------------------------------- frame distance: known answers ---
# Hand-derived values of frame_distance_kernel's rule (se3.cuh:209-277): per
# pixel a beta-weighted full reprojection term and a (1 - beta)-weighted
# translation-only term, each counted when its depth Z > 0.25; the mean over
# the counted weights, or 1000 when they are under 0.75 of all the weights.
# Intrinsics fx = fy = 10, cx = cy = 0, frame i at the identity, so that the
# relative pose is frame j's own and every flow below is closed-form.
_INTR = np.array([10.0, 10.0, 0.0, 0.0], np.float32)


def _fd(pose_j, disp_row, beta, H=1):
    poses = np.array([[0, 0, 0, 0, 0, 0, 1], pose_j], np.float32)
    disps = np.zeros((2, H, len(disp_row) // H), np.float32)
    disps[0] = np.asarray(disp_row, np.float32).reshape(H, -1)
    return float(orc.frame_distance(poses, disps, _INTR, np.array([0]), np.array([1]), H,
                                    len(disp_row) // H, beta)[0])


def test_frame_distance_translation_is_beta_independent():
    # tx = 0.2, disparity 0.5: every pixel moves by fx * d * tx = 1 px in both terms
    for beta in (0.0, 0.3, 1.0):
        assert _fd([0.2, 0, 0, 0, 0, 0, 1], [0.5] * 6, beta, H=2) == pytest.approx(1.0, rel=1e-6)


def test_frame_distance_rotation_weights_the_full_term_by_beta():
    # one pixel at the principal point, rotation by theta about y: the full term
    # moves it by fx * tan(theta), the translation-only term not at all, so the
    # distance is beta * fx * tan(theta) (a swapped mix would give (1 - beta) * ...)
    th = 0.1
    q = [0.0, np.sin(th / 2), 0.0, np.cos(th / 2)]
    got = _fd([0, 0, 0] + q, [0.7], 0.3)
    assert got == pytest.approx(0.3 * 10.0 * np.tan(th), rel=1e-5)
    assert _fd([0, 0, 0] + q, [0.7], 1.0) == pytest.approx(10.0 * np.tan(th), rel=1e-5)
    assert _fd([0, 0, 0] + q, [0.7], 0.0) == 0.0


def test_frame_distance_depth_mask_and_coverage():
    # tz = -0.5 along a row u = 0..W-1: Z = 1 - 0.5 d, and a counted pixel moves
    # from u to u / Z, i.e. by u when d = 1 (Z = 0.5)
    tz = [0, 0, -0.5, 0, 0, 0, 1]
    # 4 of 5 counted (d = 10 gives Z = -4): coverage 0.8, mean flow (0+1+2+3)/4
    assert _fd(tz, [1, 1, 1, 1, 10], 0.3) == pytest.approx(1.5, rel=1e-6)
    # 3 of 5 counted: coverage 0.6 < 0.75
    assert _fd(tz, [1, 1, 1, 10, 10], 0.3) == 1000.0
    # d = 1.5 gives Z = 0.25 exactly, which is not counted (Z > 0.25 strictly);
    # coverage 3/4 = 0.75 is enough (the test is < 0.75): mean (0+1+2)/3. A
    # mask of Z >= 0.25 would count u = 3 (flow 3/0.25 - 3 = 9): mean 3.
    assert _fd(tz, [1, 1, 1, 1.5], 0.3) == pytest.approx(1.0, rel=1e-6)


def test_disp_retr_known_answers():
    # fmaxf(d + dz, 0.001) per pixel of the listed frames (se3.cuh:195-206);
    # fmaxf returns the number when the sum is NaN (IEEE maxNum), unlike np.maximum
    d = np.array([[0.5, 0.5, 0.5, 0.5], [2.0, 2.0, 2.0, 2.0], [1.0, 1.0, 1.0, 1.0]],
                 np.float32)
    dz = np.array([[0.25, -0.75, -0.9995, np.nan], [-1.0, 0.5, 0.0, -2.0]], np.float32)
    r = orc.disp_retr(d, dz, np.array([2, 0], np.int32))
    np.testing.assert_array_equal(r[1], d[1])  # not listed
    np.testing.assert_array_equal(r[2], np.float32([1.25, 0.25, 0.001, 0.001]))
    np.testing.assert_array_equal(r[0], np.float32([0.001, 1.0, 0.5, 0.001]))
