"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the CPU oracle: the oracle must still
reproduce every expected output it once wrote. The oracle is fp64 inside and
deterministic; outputs agree to the last fp32 bit except where a summation
order over threads may differ (then within 1e-6 relative)."""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module", autouse=True)
def _build():
    orc.build()


def test_fixture_files_present():
    for n in ("corr_window", "corr_integer", "se3", "ba_iter"):
        assert os.path.exists(os.path.join(GOLD, n + ".npz")), n
    assert os.path.exists(os.path.join(GOLD, "make_golden.py"))


@pytest.mark.parametrize("name", ["corr_window", "corr_integer"])
def test_oracle_reproduces_corr(name):
    g = load(name)
    out = orc.corr_batch(g["fmaps"], g["ii"], g["jj"], g["coords"], float(g["alpha"]))
    assert out.shape == g["out"].shape == (len(g["ii"]), 196, g["coords"].shape[-1])
    if name == "corr_integer":
        np.testing.assert_array_equal(out, g["out"])
    else:
        np.testing.assert_allclose(out, g["out"], rtol=1e-6, atol=1e-6)


def test_oracle_reproduces_se3():
    g = load("se3")
    h, w = int(g["h"]), int(g["w"])
    coords, valid = orc.projmap(g["poses"], g["disps"], g["intr"], g["ii"], g["jj"], h, w)
    np.testing.assert_allclose(coords, g["coords"], rtol=1e-6, atol=1e-5)
    np.testing.assert_array_equal(valid, g["valid"])
    retr = orc.pose_retr(g["poses"], g["dx"], int(g["t0"]), int(g["t1"]))
    np.testing.assert_allclose(retr, g["poses_retr"], rtol=1e-6, atol=1e-7)
    dist = orc.frame_distance(g["poses"], g["disps"], g["intr"], g["ii"], g["jj"], h, w,
                              float(g["beta"]))
    np.testing.assert_allclose(dist, g["dist"], rtol=1e-6)


def test_oracle_reproduces_ba_iteration():
    g = load("ba_iter")
    r = orc.ba_iterate(g["poses"], g["disps"], g["intr"], g["target"], g["weight"], g["eta"],
                       g["ii"], g["jj"], int(g["h"]), int(g["w"]), int(g["t0"]), int(g["t1"]),
                       float(g["lm"]), float(g["ep"]))
    assert r["status"] == 0
    np.testing.assert_allclose(r["S"], g["S"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r["dx"], g["dx"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(r["poses"], g["poses_out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(r["disps"], g["disps_out"], rtol=1e-6, atol=1e-7)
