"""The PyTorch-CPU baseline (oracle/torch_baseline.py) computes the same
thing as the C oracle: checked on the same seeded inputs at small sizes, so
the CPU figure bench.py reports is for the path's own arithmetic. Corr and
lookup (fp32 torch vs fp64-accumulated C): helpers.TOL relative to
max(|r|, rms); BA (both fp64): S, b, dx to 1e-8 normwise, poses and
inverse depths to 1e-6."""
import numpy as np
import pytest

from helpers import assert_close_rel, norm_rel
from oracle import oracle as orc
import workloads as wl

torch = pytest.importorskip("torch")
from oracle import torch_baseline as tb  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


@pytest.mark.parametrize("h,w", [(12, 16), (9, 14)])
def test_corr_lookup_matches_oracle(h, w):
    f = wl.frames(4, C=32, h=h, w=w, seed=5)
    ii, jj = wl.cyclic_edges(4, dmax=1)
    coords = wl.flow_coords(len(ii), h, w, seed=6)
    coords[0, 0, 3] = np.nan  # non-finite and far coordinates give zeros
    coords[1, 1, 5] = 1e9
    got = tb.corr_lookup(torch.from_numpy(f), torch.from_numpy(ii.astype(np.int64)),
                         torch.from_numpy(jj.astype(np.int64)), torch.from_numpy(coords),
                         1.0 / 16.0).numpy()
    ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
    assert_close_rel(got, ref, what="torch corr+lookup")
    assert not got[0, :, 3].any() and not got[1, :, 5].any()


def test_integer_coords_are_window_copies():
    """Integer coordinates: every level-0 channel is a plain copy of a volume
    cell, so the torch gather's channel order (a = x offset) is pinned
    exactly against the oracle."""
    h, w = 10, 12
    rng = np.random.default_rng(3)
    f = rng.integers(-3, 4, size=(2, 16, h, w)).astype(np.float32)
    coords = (wl.grid_coords(h, w)[None] + rng.integers(-4, 5, (1, 2, h * w))).astype(np.float32)
    ii, jj = np.array([0], np.int32), np.array([1], np.int32)
    got = tb.corr_lookup(torch.from_numpy(f), torch.tensor([0]), torch.tensor([1]),
                         torch.from_numpy(coords), 1.0 / 16.0).numpy()
    ref = orc.corr_batch(f, ii, jj, coords, 1.0 / 16.0)
    np.testing.assert_array_equal(got[:, :49], ref[:, :49])


@pytest.mark.parametrize("motion_only", [False, True])
def test_ba_iterate_matches_oracle(motion_only):
    ii = np.array([0, 1, 2, 3, 1, 2, 4, 2, 0], np.int32)
    jj = np.array([1, 2, 3, 4, 0, 1, 3, 2, 3], np.int32)  # (2, 2): a stereo edge
    p = wl.ba_problem(n=5, h=8, w=10, ii=ii, jj=jj, seed=7, fixed=1)
    p["eta"] = np.random.default_rng(8).uniform(0, 1e-3, p["eta"].shape).astype(np.float32)
    T = {k: torch.from_numpy(np.ascontiguousarray(p[k])) for k in
         ("poses", "disps", "intr", "target", "weight", "eta")}
    poses, disps, info = tb.ba_iterate(T["poses"], T["disps"], T["intr"], T["target"],
                                       T["weight"], T["eta"], torch.from_numpy(ii.astype(np.int64)),
                                       torch.from_numpy(jj.astype(np.int64)), 8, 10, p["t0"],
                                       p["t1"], 1e-4, 0.1, motion_only)
    ref = orc.ba_iterate(p["poses"], p["disps"], p["intr"], p["target"], p["weight"], p["eta"],
                         ii, jj, 8, 10, p["t0"], p["t1"], 1e-4, 0.1, motion_only=motion_only)
    assert info["status"] == 0 and ref["status"] == 0
    assert norm_rel(info["S"].numpy(), ref["S"]) < 1e-8
    assert norm_rel(info["b"].numpy(), ref["b"]) < 1e-8
    assert norm_rel(info["dx"].numpy(), ref["dx"]) < 1e-8
    np.testing.assert_allclose(poses.numpy(), ref["poses"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(disps.numpy().reshape(ref["disps"].shape), ref["disps"], rtol=1e-6,
                               atol=1e-7)


def test_ba_not_spd_reported():
    p = wl.ba_problem(n=4, h=6, w=8, seed=2)
    T = {k: torch.from_numpy(np.ascontiguousarray(p[k])) for k in
         ("poses", "disps", "intr", "target", "eta")}
    zero_w = torch.zeros_like(torch.from_numpy(p["weight"]))
    poses, disps, info = tb.ba_iterate(T["poses"], T["disps"], T["intr"], T["target"], zero_w,
                                       T["eta"], torch.from_numpy(p["ii"].astype(np.int64)),
                                       torch.from_numpy(p["jj"].astype(np.int64)), 6, 8, p["t0"],
                                       p["t1"], 0.0, 0.0)
    assert info["status"] != 0
    np.testing.assert_array_equal(poses.numpy(), p["poses"])
