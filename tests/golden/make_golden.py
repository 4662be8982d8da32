#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/*.npz: seeded inputs of the
per-edge path at small sizes and the expected outputs computed by the CPU
oracle (oracle/, C with fp64 accumulation), after the oracle itself has been
pinned by tests/test_oracle_*.py (closed forms, finite differences, brute-force
solves, scipy). The reference ships no fixtures for this path and cannot be
built here (CUDA), so these are the build's own vectors; they freeze the
expected outputs so that a change to either the oracle or the GPU path shows
up as a fixture mismatch.

Files (numpy .npz, no pickled objects):
  corr_window.npz    4 frames [32, 8, 8] fp32 N(0,1), 8 cyclic edges, flow
                     coords, alpha 1/16 -> lookup [8, 196, 64]
  corr_integer.npz   the same with integer features in [-3, 3] and coords
                     that are multiples of 8: every output is exact
  se3.npz            projmap, pose_retr, frame_distance on a 5-frame window
  ba_iter.npz        one BundleAdjustment::iterate on 5 frames of 6x8 pixels
                     (2 fixed poses): S, b, dx and the updated poses/disps

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "slam-hands_amd"))

from oracle import oracle as orc  # noqa: E402
import workloads as wl  # noqa: E402

ALPHA = np.float32(1.0 / 16.0)


def corr_window():
    n, C, h, w = 4, 32, 8, 8
    f = wl.frames(n, C=C, h=h, w=w, seed=900)
    ii, jj = wl.cyclic_edges(n, dmax=1)
    coords = wl.flow_coords(len(ii), h, w, seed=901, amp=4.0)
    out = orc.corr_batch(f, ii, jj, coords, float(ALPHA))
    return dict(fmaps=f, ii=ii, jj=jj, coords=coords, alpha=ALPHA, out=out)


def corr_integer():
    n, C, h, w = 4, 32, 8, 8
    rng = np.random.default_rng(902)
    f = rng.integers(-3, 4, size=(n, C, h, w)).astype(np.float32)
    ii, jj = wl.cyclic_edges(n, dmax=1)
    g = wl.grid_coords(h, w)[None]
    coords = (g // 8 * 8 + 8 * rng.integers(-1, 2, size=(len(ii), 2, h * w))).astype(np.float32)
    out = orc.corr_batch(f, ii, jj, coords, float(ALPHA))
    return dict(fmaps=f, ii=ii, jj=jj, coords=coords, alpha=ALPHA, out=out)


def se3():
    h, w = 6, 8
    p = wl.ba_problem(n=5, h=h, w=w, seed=903)
    coords, valid = orc.projmap(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], h, w)
    rng = np.random.default_rng(904)
    dx = rng.normal(0.0, 0.05, size=(3, 6)).astype(np.float32)
    retr = orc.pose_retr(p["poses"], dx, 2, 5)
    beta = np.float32(0.7)
    dist = orc.frame_distance(p["poses"], p["disps"], p["intr"], p["ii"], p["jj"], h, w,
                              float(beta))
    return dict(poses=p["poses"], disps=p["disps"], intr=p["intr"], ii=p["ii"], jj=p["jj"],
                h=np.int32(h), w=np.int32(w), coords=coords, valid=valid, dx=dx,
                t0=np.int32(2), t1=np.int32(5), poses_retr=retr, beta=beta, dist=dist)


def ba_iter():
    h, w = 6, 8
    p = wl.ba_problem(n=5, h=h, w=w, seed=905)
    lm, ep = np.float32(1e-4), np.float32(0.1)
    r = orc.ba_iterate(p["poses"], p["disps"], p["intr"], p["target"], p["weight"], p["eta"],
                       p["ii"], p["jj"], h, w, p["t0"], p["t1"], float(lm), float(ep))
    assert r["status"] == 0
    return dict(poses=p["poses"], disps=p["disps"], intr=p["intr"], target=p["target"],
                weight=p["weight"], eta=p["eta"], ii=p["ii"], jj=p["jj"], h=np.int32(h),
                w=np.int32(w), t0=np.int32(p["t0"]), t1=np.int32(p["t1"]), lm=lm, ep=ep,
                S=r["S"], b=r["b"], dx=r["dx"], poses_out=r["poses"], disps_out=r["disps"])


MAKERS = {"corr_window": corr_window, "corr_integer": corr_integer, "se3": se3,
          "ba_iter": ba_iter}


def main():
    orc.build()
    for name, fn in MAKERS.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {os.path.relpath(path, ROOT)} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
