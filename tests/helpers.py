"""Shared tolerances and GPU helpers for the parity tests."""
import numpy as np
import pytest

# Floating-point parity bar: elementwise |g - r| <= TOL * max(|r|, rms(r)),
# TOL = 1e-4 (fp32 north-star tolerance), so near-zero correlation entries are
# judged against the scale of their row rather than their own magnitude.
TOL = 1e-4


def assert_close_rel(got, ref, tol=TOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    rms = np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
    bound = tol * np.maximum(np.abs(ref), rms) + 1e-30
    with np.errstate(invalid="ignore"):
        err = np.abs(got - ref)
        same = (got == ref) | (np.isnan(got) & np.isnan(ref))
        bad = ~same & ~(err <= bound)  # a NaN where the reference is finite fails
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, np.nan_to_num(err / bound, nan=np.inf),
                                                -1.0)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} outside tol {tol}; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} (rms {rms:.3g})")


def norm_rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.linalg.norm(ref)
    return np.linalg.norm(got - ref) / (d if d > 0 else 1.0)


def gpu_or_fail():
    """GPU tests run only where a GPU exists; there they must find the HIP
    library (no fallback)."""
    import slk
    if slk.hip().device_count() < 1:
        pytest.skip("no GPU visible")
    slk.lib()
    return slk


def announce(msg):
    """Names the case before a GPU step, so a run that dies mid-way says where."""
    print(f"[gpu-test] {msg}", flush=True)


class Pins:
    """Uploads host arrays and keeps the device copies alive for the whole
    test, so a pointer handed to a kernel never outlives its buffer."""

    def __init__(self, slk):
        self.slk = slk
        self.bufs = []

    def __call__(self, arr):
        d = self.slk.DeviceArray.from_host(arr)
        self.bufs.append(d)
        return d.ptr


def assert_valid_mask(valid, poses, disps, intr, ii, jj, h, w, band=1e-5):
    """projmap's valid mask (se3.cuh:174: homogeneous Z > 0.25) must match
    exactly, except for pixels whose Z lies within `band` of 0.25 (where fp32
    rounding of the projection decides). Z is the camera-j depth of the
    independent fp64 pinhole model (workloads.project) times frame ii's
    inverse depth, i.e. the homogeneous Z the kernel tests."""
    import workloads as wl
    valid = np.asarray(valid).reshape(len(ii), h * w)
    _, depth = wl.project(poses, disps, intr, ii, jj, h, w)
    z = depth * np.asarray(disps, np.float64).reshape(len(poses), h * w)[np.asarray(ii)]
    want = (z > 0.25).astype(np.float32)
    near = np.abs(z - 0.25) < band
    bad = (valid != want) & ~near
    if bad.any():
        idx = np.argwhere(bad)[:10].tolist()
        raise AssertionError(f"valid mask: {int(bad.sum())} entries differ outside the "
                             f"|Z - 0.25| < {band} band; first (edge, pixel): {idx}")
    assert np.all((valid == 0.0) | (valid == 1.0))
    return int(near.sum())
