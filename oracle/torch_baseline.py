"""PyTorch-CPU restatement of the per-edge update path: the CPU baseline that
bench.py reports beside the GPU figures.

TEST AND BASELINE INFRASTRUCTURE, NOT PRODUCT CODE. It is imported only by
bench.py's cpu_baseline leg (run in a child process, CPU tensors only) and by
tests/test_torch_baseline.py, which checks it against the C oracle
(oracle.c) on the same seeded inputs. The library never loads it.

The ops are the PyTorch-CPU equivalents of the reference's GPU calls:
  * correlation: torch.bmm in fp32 of the two [C, h*w] feature maps, times
    alpha (the cublasGemmBatchedEx of cuda_slam/main.cu:1573-1581);
  * pyramid: F.avg_pool2d(2, 2) three times (avg_pool_2x2_kernel,
    main.cu:1150-1170: floor sizes, mean of 4);
  * lookup: an explicit 8x8 gather of the window around floor(x*2^-l) - 3,
    zero outside the level, combined bilinearly into channel l*49 + a*7 + b
    with a the x offset (batch_corr_sample_kernel, main.cu:1175-1217);
  * BA: vectorised Jacobians (projective_transform_kernel, ba.cuh:39-221),
    einsum Hessian blocks, index_add_ into the dense pose system
    (ba.cuh:520-548), the Schur complement over the inverse depths of the
    keyframes in ii with E rows keyed by (pose, keyframe) (ba.cuh:566-743),
    LM damping after the Schur step (ba.cuh:749-750), torch.linalg.cholesky +
    cholesky_solve in float64 (cholesky_solve_double, ba.cuh:416-445), pose
    retraction on the fp32-rounded step and depth back-substitution
    (ba.cuh:757-783). All BA arithmetic is float64.
"""
from __future__ import annotations

import json
import os
import sys
import time

import torch
import torch.nn.functional as F

MIN_DEPTH = 0.25  # se3.cuh:6


# ------------------------------------------------------------------ correlation
def corr_lookup(fmaps, ii, jj, coords, alpha, levels=4, r=3):
    """fmaps [n, C, h, w] fp32, ii/jj [B] long, coords [B, 2, h*w] fp32 ->
    [B, levels*49, h*w] fp32."""
    assert r == 3
    n, C, h, w = fmaps.shape
    B, HW = len(ii), h * w
    fi = fmaps[ii].reshape(B, C, HW)
    fj = fmaps[jj].reshape(B, C, HW)
    vol = torch.bmm(fi.transpose(1, 2), fj).mul_(alpha)  # [B, HW(src), HW(tgt)]
    lev = vol.view(B * HW, 1, h, w)
    out = torch.zeros(B, levels * 49, HW, dtype=torch.float32)
    ar = torch.arange(8)
    for l in range(levels):
        if l > 0:
            lev = F.avg_pool2d(lev, 2, 2)
        H2, W2 = lev.shape[-2:]
        flat = lev.reshape(B * HW, H2 * W2)
        scale = 1.0 / (1 << l)
        x0 = coords[:, 0].reshape(-1) * scale  # fp32, like main.cu:1189-1190
        y0 = coords[:, 1].reshape(-1) * scale
        fx, fy = torch.floor(x0), torch.floor(y0)
        # a non-finite coordinate reads no cell (its window is all outside);
        # its weights are set to 0 so that 0 * NaN does not reach the output
        fin = torch.isfinite(x0) & torch.isfinite(y0)
        dx = torch.where(fin, x0 - fx, torch.zeros_like(x0))[:, None, None]
        dy = torch.where(fin, y0 - fy, torch.zeros_like(y0))[:, None, None]
        # window cell (i, j) = (x0 - 3 + i, y0 - 3 + j), i the x offset
        fxl = torch.nan_to_num(fx, nan=-1e9).clamp(-1e9, 1e9).long()
        fyl = torch.nan_to_num(fy, nan=-1e9).clamp(-1e9, 1e9).long()
        xs = fxl[:, None] - 3 + ar[None, :]  # [N, 8] (i)
        ys = fyl[:, None] - 3 + ar[None, :]  # [N, 8] (j)
        ok = ((xs >= 0) & (xs < W2))[:, :, None] & ((ys >= 0) & (ys < H2))[:, None, :]
        idx = (ys[:, None, :] * W2 + xs[:, :, None]).clamp(0, H2 * W2 - 1)
        win = torch.gather(flat, 1, idx.reshape(-1, 64)).reshape(-1, 8, 8)
        win = torch.where(ok, win, torch.zeros((), dtype=win.dtype))
        o = ((1 - dx) * (1 - dy) * win[:, :7, :7] + dx * (1 - dy) * win[:, 1:, :7]
             + (1 - dx) * dy * win[:, :7, 1:] + dx * dy * win[:, 1:, 1:])
        out[:, l * 49:(l + 1) * 49] = o.reshape(B, HW, 49).transpose(1, 2)
    return out


# -------------------------------------------------------------------------- SE3
def _act_so3(q, X):
    """q [..., 4] (x, y, z, w), X [..., 3] (se3.cuh:8-17)."""
    qv, qw = q[..., :3], q[..., 3:]
    uv = 2.0 * torch.cross(qv, X, dim=-1)
    return X + qw * uv + torch.cross(qv, uv, dim=-1)


def _rel_se3(ti, qi, tj, qj):
    """Tij = Tj * Ti^-1 (se3.cuh:43-54)."""
    x1, y1, z1, w1 = qi.unbind(-1)
    x2, y2, z2, w2 = qj.unbind(-1)
    qij = torch.stack([-w2 * x1 + x2 * w1 - y2 * z1 + z2 * y1,
                       -w2 * y1 + y2 * w1 - z2 * x1 + x2 * z1,
                       -w2 * z1 + z2 * w1 - x2 * y1 + y2 * x1,
                       w2 * w1 + x2 * x1 + y2 * y1 + z2 * z1], -1)
    return tj - _act_so3(qij, ti), qij


def _adj_se3(t, q, X):
    """se3.cuh:28-41 applied to X [..., 6]."""
    qinv = torch.cat([-q[..., :3], q[..., 3:]], -1)
    a = _act_so3(qinv, X[..., :3])
    b = _act_so3(qinv, X[..., 3:]) + _act_so3(qinv, torch.cross(X[..., :3], t, dim=-1))
    return torch.cat([a, b], -1)


def _retr_se3(xi, t, q):
    """T <- exp(xi) * T (se3.cuh:85-114), xi [..., 6] = [tau, phi]."""
    tau, phi = xi[..., :3], xi[..., 3:]
    th2 = (phi * phi).sum(-1, keepdim=True)
    th = th2.sqrt()
    small = th2 < 1e-8
    imag = torch.where(small, 0.5 - th2 / 48.0 + th2 * th2 / 3840.0,
                       torch.sin(0.5 * th) / torch.where(small, torch.ones_like(th), th))
    real = torch.where(small, 1.0 - th2 / 8.0 + th2 * th2 / 384.0, torch.cos(0.5 * th))
    dq = torch.cat([imag * phi, real], -1)
    big = th > 1e-4
    safe2 = torch.where(big, th2, torch.ones_like(th2))
    safe = torch.where(big, th, torch.ones_like(th))
    c1 = torch.cross(phi, tau, dim=-1)
    c2 = torch.cross(phi, c1, dim=-1)
    a = (1.0 - torch.cos(safe)) / safe2
    b = (safe - torch.sin(safe)) / (safe * safe2)
    dt = tau + torch.where(big, a * c1 + b * c2, torch.zeros_like(c1))
    x1, y1, z1, w1 = dq.unbind(-1)
    x2, y2, z2, w2 = q.unbind(-1)
    q1 = torch.stack([w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                      w1 * y2 + y1 * w2 + z1 * x2 - x1 * z2,
                      w1 * z2 + z1 * w2 + x1 * y2 - y1 * x2,
                      w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2], -1)
    return _act_so3(dq, t) + dt, q1


# --------------------------------------------------------------------------- BA
def ba_iterate(poses, disps, intr, target, weight, eta, ii, jj, h, w, t0, t1, lm, ep,
               motion_only=False):
    """One Gauss-Newton step on CPU tensors (poses [N,7], disps [N,h*w] or
    [N,h,w], target/weight [M,2,h*w], eta [N,h*w] fp32; ii/jj [M] long).
    Returns (poses, disps, info) with the updated fp32 poses and inverse
    depths and info = {S, b, dx, status}."""
    f64 = torch.float64
    N = poses.shape[0]
    HW = h * w
    M = len(ii)
    P = t1 - t0
    n = 6 * P
    disps = disps.reshape(N, HW)
    pose = poses.to(f64)
    fx, fy, cx, cy = (float(v) for v in intr)
    tij, qij = _rel_se3(pose[ii, :3], pose[ii, 3:], pose[jj, :3], pose[jj, 3:])
    stereo = ii == jj
    tij = torch.where(stereo[:, None], torch.tensor([-0.1, 0.0, 0.0], dtype=f64), tij)
    qij = torch.where(stereo[:, None], torch.tensor([0.0, 0.0, 0.0, 1.0], dtype=f64), qij)
    v, u = torch.meshgrid(torch.arange(h, dtype=f64), torch.arange(w, dtype=f64), indexing="ij")
    xn = ((u.reshape(-1) - cx) / fx).expand(M, HW)
    yn = ((v.reshape(-1) - cy) / fy).expand(M, HW)
    dsp = disps[ii].to(f64)
    T = tij[:, None, :]
    Q = qij[:, None, :].expand(M, HW, 4)
    Xr = _act_so3(Q, torch.stack([xn, yn, torch.ones_like(xn)], -1)) + dsp[..., None] * T
    X, Y, Z = Xr.unbind(-1)
    Hh = dsp
    bad = Z < MIN_DEPTH
    d = torch.where(bad, torch.zeros_like(Z), 1.0 / Z)
    d2 = d * d
    wt = weight.to(f64)
    tg = target.to(f64)
    wu = torch.where(bad, torch.zeros_like(Z), 0.001 * wt[:, 0])
    wv = torch.where(bad, torch.zeros_like(Z), 0.001 * wt[:, 1])
    ru = tg[:, 0] - (fx * d * X + cx)
    rv = tg[:, 1] - (fy * d * Y + cy)
    zero = torch.zeros_like(Z)
    Jjx = torch.stack([fx * Hh * d, zero, -fx * X * Hh * d2, -fx * X * Y * d2,
                       fx * (1 + X * X * d2), -fx * Y * d], -1)
    Jjy = torch.stack([zero, fy * Hh * d, -fy * Y * Hh * d2, fy * (-1 - Y * Y * d2),
                       fy * X * Y * d2, fy * X * d], -1)
    Jzx = fx * (T[..., 0] * d - T[..., 2] * X * d2)
    Jzy = fy * (T[..., 1] * d - T[..., 2] * Y * d2)
    Tx = T.expand(M, HW, 3)
    Jix = -_adj_se3(Tx, Q, Jjx)
    Jiy = -_adj_se3(Tx, Q, Jjy)
    keep = (~stereo).to(f64)[:, None]
    wue, wve = wu * keep, wv * keep
    Jx = torch.cat([Jix, Jjx], -1)
    Jy = torch.cat([Jiy, Jjy], -1)
    Hs = (torch.einsum("mk,mka,mkb->mab", wue, Jx, Jx)
          + torch.einsum("mk,mka,mkb->mab", wve, Jy, Jy))
    vs = torch.einsum("mk,mka->ma", wue * ru, Jx) + torch.einsum("mk,mka->ma", wve * rv, Jy)
    Eii = (wue * Jzx)[..., None] * Jix + (wve * Jzy)[..., None] * Jiy  # [M, HW, 6]
    Eij = (wue * Jzx)[..., None] * Jjx + (wve * Jzy)[..., None] * Jjy
    Cii = wu * Jzx * Jzx + wv * Jzy * Jzy
    bz = wu * ru * Jzx + wv * rv * Jzy

    pi, pj = ii - t0, jj - t0
    iv = (pi >= 0) & (pi < P)
    jv = (pj >= 0) & (pj < P)
    both = iv & jv
    S4 = torch.zeros(P * P, 6, 6, dtype=f64)
    S4.index_add_(0, (pi * P + pi)[iv], Hs[iv, :6, :6])
    S4.index_add_(0, (pi * P + pj)[both], Hs[both, :6, 6:])
    S4.index_add_(0, (pj * P + pi)[both], Hs[both, 6:, :6])
    S4.index_add_(0, (pj * P + pj)[jv], Hs[jv, 6:, 6:])
    b6 = torch.zeros(P, 6, dtype=f64)
    b6.index_add_(0, pi[iv], vs[iv, :6])
    b6.index_add_(0, pj[jv], vs[jv, 6:])

    if not motion_only:
        kf, kc = torch.unique(ii, sorted=True, return_inverse=True)
        nkf = len(kf)
        # E rows keyed by (pose, keyframe)
        key_i = pi * N + ii
        key_j = pj * N + ii
        keys = torch.unique(torch.cat([key_i[iv], key_j[jv]]))
        NE = len(keys)
        row_i = torch.searchsorted(keys, key_i)
        row_j = torch.searchsorted(keys, key_j)
        E = torch.zeros(NE, HW, 6, dtype=f64)
        E.index_add_(0, row_i[iv], Eii[iv])
        E.index_add_(0, row_j[jv], Eij[jv])
        row_pose = keys // N
        row_kf = torch.searchsorted(kf, keys % N)
        Cq = torch.zeros(nkf, HW, dtype=f64).index_add_(0, kc, Cii)
        wq = torch.zeros(nkf, HW, dtype=f64).index_add_(0, kc, bz)
        Qd = 1.0 / (Cq + 0.2 * eta.reshape(N, HW)[kf].to(f64) + 1e-7)
        # all pairs of E rows that share a keyframe
        same = row_kf[:, None] == row_kf[None, :]
        r1, r2 = torch.nonzero(same, as_tuple=True)
        blk = torch.einsum("phA,ph,phB->pAB", E[r1], Qd[row_kf[r1]], E[r2])
        S4.index_add_(0, row_pose[r1] * P + row_pose[r2], -blk)
        ev = torch.einsum("rh,rhA->rA", Qd[row_kf] * wq[row_kf], E)
        b6.index_add_(0, row_pose, -ev)
    S = S4.view(P, P, 6, 6).permute(0, 2, 1, 3).reshape(n, n)
    b = b6.reshape(n)
    S = S + torch.diag(ep + lm * torch.diagonal(S))
    info = {"S": S.clone(), "b": b.clone(), "status": 0}
    L, bad_ = torch.linalg.cholesky_ex(S)
    poses_out = poses.clone()
    disps_out = disps.clone()
    if int(bad_) != 0:
        info["status"] = 3
        return poses_out, disps_out, info
    dx = torch.cholesky_solve(b[:, None], L)[:, 0]
    info["dx"] = dx
    dxf = dx.to(torch.float32).to(f64).reshape(P, 6)
    t_new, q_new = _retr_se3(dxf, pose[t0:t1, :3], pose[t0:t1, 3:])
    poses_out[t0:t1, :3] = t_new.to(torch.float32)
    poses_out[t0:t1, 3:] = q_new.to(torch.float32)
    if not motion_only and NE > 0:
        dwr = torch.einsum("rhA,rA->rh", E, dxf[row_pose])
        dw = torch.zeros(nkf, HW, dtype=f64).index_add_(0, row_kf, dwr)
        dz = Qd * (wq - dw)
        disps_out[kf] = (disps[kf].to(f64) + dz).to(torch.float32)
    return poses_out, disps_out, info


# ------------------------------------------------------------------- timing
def _time_window(n, h, w, B, iters, lm, ep, edges, reps, chunk):
    """Times the window step (corr + lookup of `edges` of the B edges, in
    chunks, and `iters` BA iterations on the full window) on this host's
    cores; inputs from workloads.py with bench.py's seeds."""
    here = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, os.path.join(os.path.dirname(here), "slam-hands_amd"))
    import workloads as wl
    import numpy as np
    fm = torch.from_numpy(wl.frames(n, 128, h, w, seed=0))
    ii_np, jj_np = wl.cyclic_edges(n)
    ii = torch.from_numpy(ii_np.astype(np.int64))
    jj = torch.from_numpy(jj_np.astype(np.int64))
    coords = torch.from_numpy(wl.flow_coords(B, h, w, seed=1))
    p = wl.ba_problem(n=n, h=h, w=w, ii=ii_np, jj=jj_np, seed=3)
    tp = {k: torch.from_numpy(np.ascontiguousarray(p[k])) for k in
          ("poses", "disps", "intr", "target", "weight", "eta")}

    def corr():
        for c0 in range(0, edges, chunk):
            sl = slice(c0, min(edges, c0 + chunk))
            corr_lookup(fm, ii[sl], jj[sl], coords[sl], 1.0 / 16.0)

    def ba():
        poses, disps = tp["poses"], tp["disps"]
        for _ in range(iters):
            poses, disps, info = ba_iterate(poses, disps, tp["intr"], tp["target"],
                                            tp["weight"], tp["eta"], ii, jj, h, w,
                                            p["t0"], p["t1"], lm, ep)
            assert info["status"] == 0

    corr()
    ba()
    tc, tb = [], []
    for _ in range(reps):
        t = time.perf_counter()
        corr()
        tc.append(time.perf_counter() - t)
        t = time.perf_counter()
        ba()
        tb.append(time.perf_counter() - t)
    tc.sort()
    tb.sort()
    corr_s_edge = tc[len(tc) // 2] / edges
    ba_s_iter = tb[len(tb) // 2] / iters
    return corr_s_edge, ba_s_iter


def main():
    import argparse
    ap = argparse.ArgumentParser()
    ap.add_argument("--frames", type=int, default=12)
    ap.add_argument("--h", type=int, default=48)
    ap.add_argument("--w", type=int, default=64)
    ap.add_argument("--edges", type=int, default=48)
    ap.add_argument("--sample-edges", type=int, default=48)
    ap.add_argument("--iters", type=int, default=3)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--chunk", type=int, default=8)
    a = ap.parse_args()
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    corr_s, ba_s = _time_window(a.frames, a.h, a.w, a.edges, a.iters, 1e-4, 0.1,
                                a.sample_edges, a.reps, a.chunk)
    step_s = a.edges * corr_s + a.iters * ba_s
    print(json.dumps({"corr_s_per_edge": corr_s, "ba_s_per_iter": ba_s,
                      "edges_per_s": a.edges / step_s, "threads": torch.get_num_threads(),
                      "os_cpu_count": os.cpu_count(), "affinity_cpus": threads,
                      "torch": torch.__version__}), flush=True)


if __name__ == "__main__":
    main()
