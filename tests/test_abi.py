"""CPU checks of the drop-in boundary: libslk.so loads, exports exactly the
entry points include/slk.h declares, rejects bad arguments before touching
the GPU, and the host-side plumbing (workload generator) is deterministic."""
import os
import re
import subprocess

import numpy as np
import pytest

import slk
import workloads as wl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "slk.h")).read()
    return sorted(set(re.findall(r"\b(slk_[a-z0-9_]+)\s*\(", src)))


def test_header_matches_binding_list():
    assert declared() == sorted(slk.EXPORTS)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(slk.LIB_PATH), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", slk.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (slk_\w+)", out))
    missing = [s for s in declared() if s not in exported]
    assert not missing, missing
    lib = slk.lib()  # loads with ctypes and binds every signature
    for s in declared():
        assert hasattr(lib, s)


def test_argument_errors_need_no_gpu():
    lib = slk.lib()
    import ctypes
    p = ctypes.c_void_p()
    assert lib.slk_create(ctypes.byref(p), 48, 64, 128, 48, 4, 2, 0.0625) == slk.SLK_E_ARG
    assert b"radius" in lib.slk_last_error()
    assert lib.slk_create(ctypes.byref(p), 48, 64, 127, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    assert lib.slk_create(ctypes.byref(p), 4, 64, 128, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    assert lib.slk_create(None, 48, 64, 128, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    # h*w at 2^21 would overflow the batched path's 32-bit window offsets
    assert lib.slk_create(ctypes.byref(p), 1024, 2048, 128, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    assert b"2^21" in lib.slk_last_error()
    assert lib.slk_create(ctypes.byref(p), 2048, 1024, 128, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    assert lib.slk_create(ctypes.byref(p), 8, 65537, 128, 48, 4, 3, 0.0625) == slk.SLK_E_ARG
    assert lib.slk_ba_iterate(None, *([None] * 10), 1, 0, 1, 1e-4, 0.1, 0, None) == slk.SLK_E_ARG
    assert lib.slk_corr_sample_level(None, None, None, 1, 2, 4, 4, 4, 4, 16, 1.0, 0,
                                     None) == slk.SLK_E_ARG
    # empty work is a no-op, not an error
    assert lib.slk_projmap(None, None, None, None, None, None, None, 0, 4, 4, None) == slk.SLK_OK


def test_workloads_are_deterministic():
    a = wl.frames(2, h=6, w=8, seed=1)
    b = wl.frames(2, h=6, w=8, seed=1)
    np.testing.assert_array_equal(a, b)
    ii, jj = wl.cyclic_edges(12)
    assert len(ii) == 48 and len(set(zip(ii, jj))) == 48
    d = np.abs(ii - jj)
    assert np.all((np.minimum(d, 12 - d) >= 1) & (np.minimum(d, 12 - d) <= 2))
    ii, jj = wl.backend_edges(200, 2000)
    assert len(ii) == 2000 and len(set(zip(ii, jj))) == 2000
    p = wl.ba_problem()
    assert p["target"].shape == (48, 2, 48 * 64) and p["t0"] == 2 and p["t1"] == 12
    np.testing.assert_array_equal(p["poses"][:2], [[0, 0, 0, 0, 0, 0, 1]] * 2)


def test_oldest_edges_mask_host_helper_matches_oracle():
    """slk_oldest_edges_mask runs on the host only: compared with the oracle's
    step-5 selection (main.cu:1762-1769) on random ages with many ties."""
    import ctypes
    import numpy as np
    from oracle import oracle as orc
    orc.build()
    rng = np.random.default_rng(5)
    for n, k in [(1, 1), (7, 3), (48, 10), (64, 70), (30, 0)]:
        age = rng.integers(0, 6, n).astype(np.int32)
        got = np.zeros(n, np.uint8)
        slk.lib().slk_oldest_edges_mask(age.ctypes.data_as(ctypes.c_void_p), n, k,
                                        got.ctypes.data_as(ctypes.c_void_p))
        np.testing.assert_array_equal(got, orc.oldest_mask(age, k))


def test_write_poses_bin_matches_the_reference_file(tmp_path):
    """slk_write_poses_bin (host-only) writes the file of main.cu:2924-2937,
    bytewise equal to the oracle's, with and without the camera-to-world
    inversion; a bad path is an error."""
    import slk
    from oracle import encoder_oracle as eo
    rng = np.random.default_rng(3)
    q = rng.normal(size=(6, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    poses = np.concatenate([rng.normal(0, 2, (6, 3)), q], 1).astype(np.float32)
    ts = np.array([0, 4, 9, 15, 22, 30], np.int32)
    for c2w in (False, True):
        path = os.path.join(tmp_path, f"p{int(c2w)}.bin")
        slk.write_poses_bin(path, ts, poses, c2w)
        with open(path, "rb") as f:
            assert f.read() == eo.poses_bin_bytes(ts, poses, c2w)
    with pytest.raises(slk.SlkError):
        slk.write_poses_bin(os.path.join(tmp_path, "no", "such", "dir.bin"), ts, poses)
