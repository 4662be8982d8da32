"""Seeded synthetic workloads for the DROID-SLAM per-edge update path.

One generator feeds the GPU path, the CPU oracle and the CPU baseline, so all
three see identical inputs (the identical-inputs pattern of the reference's
verify_slam.py:82-136). numpy's PCG64 (`default_rng(seed)`) is deterministic
across machines.

Configs follow the benchmark definitions of this build:
  corr_single  -- one edge, 128x48x64 fp32 N(0,1) features, coords = grid+U(-8,8)
  corr_window  -- 12 frames, 48 directed edges, same feature/coord law
  ba_window    -- BA on the same 12-frame window (poses 0,1 fixed, 3 iterations)
  backend      -- 200 keyframes, ~2000 edges, 198 free poses
  highres      -- 16 frames of 128x54x96, 64 edges

Edge rule for the 12/16-frame windows: the cyclic rule
{(i, (i+d) mod n), (i, (i-d) mod n) : d in {1, 2}}, giving 4n directed edges
with 1 <= |i-j| <= 2 up to wrap-around (48 edges at n=12, 64 at n=16).
"""
from __future__ import annotations

import numpy as np

C_FEAT = 128
CORR_ALPHA_REF = 1.0 / 16.0  # cuda_slam/main.cu:1506,1572 (DROID-SLAM: fmap/4 on both sides)


def frames(n, C=C_FEAT, h=48, w=64, seed=0):
    """n feature maps [n, C, h, w] fp32, i.i.d. N(0,1) (instance-normed fnet)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, C, h, w), dtype=np.float32)


def cyclic_edges(n, dmax=2):
    ii, jj = [], []
    for i in range(n):
        for d in range(1, dmax + 1):
            ii += [i, i]
            jj += [(i + d) % n, (i - d) % n]
    return np.asarray(ii, np.int32), np.asarray(jj, np.int32)


def grid_coords(h, w):
    """[2, h*w]: x plane then y plane (main.cu:1941-1946)."""
    ys, xs = np.meshgrid(np.arange(h, dtype=np.float32), np.arange(w, dtype=np.float32),
                         indexing="ij")
    return np.stack([xs.reshape(-1), ys.reshape(-1)])


def flow_coords(B, h, w, seed=1, amp=8.0):
    """[B, 2, h*w] = pixel grid + U(-amp, amp) per component."""
    rng = np.random.default_rng(seed)
    g = grid_coords(h, w)[None]
    return (g + rng.uniform(-amp, amp, size=(B, 2, h * w))).astype(np.float32)


def quat_from_rotvec(v):
    v = np.asarray(v, np.float64)
    th = np.linalg.norm(v, axis=-1, keepdims=True)
    s = np.where(th > 1e-12, np.sin(th / 2) / np.maximum(th, 1e-300), 0.5)
    return np.concatenate([v * s, np.cos(th / 2)], axis=-1)


def quat_to_matrix(q):
    x, y, z, w = q
    return np.array([
        [1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
        [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
        [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)],
    ])


def project(poses, disps, intr, ii, jj, h, w):
    """Reprojection of frame ii's pixel grid into frame jj, fp64, written from
    the pinhole model with world->camera poses [t, q(xyzw)]:
    X_j = R_j R_i^T (X_i - t_i) + t_j, with X_i = [(u-cx)/fx, (v-cy)/fy, 1]/disp.
    Returns [M, 2, h*w] (x plane, y plane) and the camera-j depth [M, h*w]."""
    fx, fy, cx, cy = [float(v) for v in intr]
    ys, xs = np.meshgrid(np.arange(h, dtype=np.float64), np.arange(w, dtype=np.float64),
                         indexing="ij")
    xs, ys = xs.reshape(-1), ys.reshape(-1)
    out = np.zeros((len(ii), 2, h * w))
    depth = np.zeros((len(ii), h * w))
    for e, (i, j) in enumerate(zip(ii, jj)):
        Ri = quat_to_matrix(poses[i, 3:].astype(np.float64))
        Rj = quat_to_matrix(poses[j, 3:].astype(np.float64))
        ti = poses[i, :3].astype(np.float64)
        tj = poses[j, :3].astype(np.float64)
        d = disps[i].reshape(-1).astype(np.float64)
        Xi = np.stack([(xs - cx) / fx, (ys - cy) / fy, np.ones_like(xs)]) / d
        Xw = Ri.T @ (Xi - ti[:, None])
        Xj = Rj @ Xw + tj[:, None]
        out[e, 0] = fx * Xj[0] / Xj[2] + cx
        out[e, 1] = fy * Xj[1] / Xj[2] + cy
        depth[e] = Xj[2]
    return out, depth


def ba_problem(n=12, h=48, w=64, ii=None, jj=None, seed=3, fixed=2, noise_px=0.5,
               rot_sigma=0.05, trans_sigma=0.1, tz_step=0.0, disp_range=(0.2, 2.0)):
    """BA window: poses near identity, inverse depth U(0.2, 2.0), intrinsics
    fx=fy=60, cx=32, cy=24 scaled to (h, w) about the 48x64 base, targets =
    exact reprojection + N(0, noise_px) (clipped to +-1e6 px, which only
    points near a camera plane reach), weights U(0,1)^2, eta = 1e-6 (the
    reference's initial damping, main.cu:745-748). tz_step moves the free
    frames forward: frame k's camera centre advances by tz_step * k along
    the optical axis (translation z -= tz_step * k for k >= fixed), which puts
    near points of forward edges behind MIN_DEPTH; disp_range replaces the
    inverse-depth law's bounds. The defaults draw the same numbers as
    always."""
    rng = np.random.default_rng(seed)
    if ii is None:
        ii, jj = cyclic_edges(n)
    poses = np.zeros((n, 7), np.float64)
    poses[:, 3:] = quat_from_rotvec(rng.normal(0.0, rot_sigma, size=(n, 3)))
    poses[:, :3] = rng.normal(0.0, trans_sigma, size=(n, 3))
    poses[:fixed] = [0, 0, 0, 0, 0, 0, 1]
    if tz_step:
        poses[fixed:, 2] -= tz_step * np.arange(fixed, n)
    poses = poses.astype(np.float32)
    disps = rng.uniform(disp_range[0], disp_range[1], size=(n, h, w)).astype(np.float32)
    intr = np.array([60.0 * w / 64, 60.0 * h / 48, 32.0 * w / 64, 24.0 * h / 48], np.float32)
    proj, depth = project(poses, disps, intr, ii, jj, h, w)
    target = np.clip(proj + rng.normal(0.0, noise_px, size=proj.shape), -1e6, 1e6)
    if tz_step:
        # a pixel behind MIN_DEPTH (homogeneous depth = depth * disp < 0.25,
        # ba.cuh:117-122) keeps its weight but aims at its own grid position,
        # so a step that brings it back in front has a residual of pixels,
        # not of the exploding projection
        zh = depth * disps[np.asarray(ii)].reshape(len(ii), -1)
        grid = grid_coords(h, w)[None].astype(np.float64)
        target = np.where((zh < 0.25)[:, None, :], grid + (target - proj), target)
    target = target.astype(np.float32)
    weight = (rng.uniform(0.0, 1.0, size=proj.shape) ** 2).astype(np.float32)
    eta = np.full((n, h, w), 1e-6, np.float32)
    return dict(poses=poses, disps=disps, intr=intr, ii=np.asarray(ii, np.int32),
                jj=np.asarray(jj, np.int32), target=target, weight=weight, eta=eta,
                t0=fixed, t1=n, h=h, w=w)


def backend_edges(n=200, target_edges=2000, seed=5):
    """Temporal |i-j| <= 2 (both directions) plus distinct random long-range
    directed pairs with |i-j| > 2 up to `target_edges`."""
    ii, jj = [], []
    for d in (1, 2):
        for i in range(n - d):
            ii += [i, i + d]
            jj += [i + d, i]
    rng = np.random.default_rng(seed)
    have = set(zip(ii, jj))
    while len(ii) < target_edges:
        i, j = (int(v) for v in rng.integers(0, n, size=2))
        if abs(i - j) <= 2 or (i, j) in have:
            continue
        have.add((i, j))
        ii.append(i)
        jj.append(j)
    return np.asarray(ii, np.int32), np.asarray(jj, np.int32)


CONFIGS = {
    "corr_single": dict(frames=2, h=48, w=64, edges=1),
    "corr_window": dict(frames=12, h=48, w=64, edges=48),
    "ba_window": dict(frames=12, h=48, w=64, edges=48, iters=3, lm=1e-4, ep=0.1),
    "backend": dict(frames=200, h=48, w=64, edges=2000, iters=5, lm=1e-5, ep=1e-2),
    "highres": dict(frames=16, h=54, w=96, edges=64, iters=3, lm=1e-4, ep=0.1),
}
