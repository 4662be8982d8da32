"""GPU parity of the update operator (UpdateModule / ConvGRU,
cuda_slam/main.cu:385-667) through the C ABI against the float64 oracle
(oracle/update_oracle.py) on the same seeded weights and inputs.

Bar: every output (new state, delta, weight, agg_conv1, eta) elementwise
within 5e-3 * max(|r|, rms(r)) and normwise within 2e-3. The reference
rounds every activation to fp16 (2^-11 relative), and the GPU accumulates
its fp16-operand products in fp32 where the oracle is exact, so a small
fraction of roundings land one fp16 step apart and propagate through the
following layers; a float32-accumulation model of the same network stays
within 3e-3 of the oracle elementwise.
"""
import os

import numpy as np
import pytest

from helpers import announce, assert_close_rel, gpu_or_fail, norm_rel
from oracle import update_oracle as uo

pytestmark = pytest.mark.gpu
TOL_EL = 5e-3
TOL_NORM = 2e-3


@pytest.fixture(scope="module")
def slk():
    return gpu_or_fail()


def run_gpu(slk, P, corr, motion, net, inp, agg_kf=None, max_batch=None, via_dir=None):
    N, _, h, w = corr.shape
    um = slk.UpdateModule(max_batch or N, h, w)
    if via_dir:
        um.load_dir(via_dir)
    else:
        um.set_weights(P)
    D = slk.DeviceArray.from_host
    dc, dm, dn, di = D(corr), D(motion), D(net), D(inp)
    dd = slk.DeviceArray((N, 3, h, w))
    dw = slk.DeviceArray((N, 3, h, w))
    da = slk.DeviceArray((N, 128, h, w))
    um.forward(dc, dm, dn, di, dd, dw, da, N)
    out = {"net": None, "delta": None, "weight": None, "agg": None, "eta": None}
    if agg_kf is not None:
        dk = D(agg_kf)
        de = slk.DeviceArray((agg_kf.shape[0], 1, h, w))
        um.compute_eta(dk, de, agg_kf.shape[0])
    slk.hip().sync()
    out.update(net=dn.to_host(), delta=dd.to_host(), weight=dw.to_host(), agg=da.to_host())
    if agg_kf is not None:
        out["eta"] = de.to_host()
        out["agg_kf_rounded"] = dk.to_host()
    um.close()
    return out


def check(got, ref, what):
    assert np.all(np.isfinite(got)), what
    assert_close_rel(got, ref, tol=TOL_EL, what=what)
    rel = norm_rel(got, ref)
    assert rel < TOL_NORM, (what, rel)
    return rel


def test_update_small_ragged_tiles(slk):
    """3 edges of 12 x 20 maps: tiles cut by both image borders."""
    announce("update operator 3 edges 12x20")
    P = uo.seeded_weights(10)
    corr, motion, net, inp = uo.seeded_inputs(3, 12, 20, seed=11)
    agg_kf = np.random.default_rng(12).uniform(0, 2, (2, 128, 12, 20)).astype(np.float32)
    g = run_gpu(slk, P, corr, motion, net, inp, agg_kf)
    rn, rd, rw, ra = uo.update_forward(P, corr, motion, net, inp)
    re = uo.compute_eta(P, agg_kf)
    for name, ref in (("net", rn), ("delta", rd), ("weight", rw), ("agg", ra), ("eta", re)):
        check(g[name], ref, name)
    # the in-place rounding of compute_eta's input (main.cu:659)
    np.testing.assert_array_equal(g["agg_kf_rounded"], uo.round16(agg_kf).astype(np.float32))
    # outputs the reference rounds are fp16-valued
    for name in ("net", "delta", "weight", "agg"):
        np.testing.assert_array_equal(g[name], g[name].astype(np.float16).astype(np.float32))


def test_update_window_48_edges(slk):
    """The 48-edge 48x64 window in one call; six edges checked against the
    oracle (edges are independent: every tensor is per edge)."""
    announce("update operator 48 edges 48x64")
    P = uo.seeded_weights(20)
    corr, motion, net, inp = uo.seeded_inputs(48, 48, 64, seed=21)
    agg_kf = np.random.default_rng(22).uniform(0, 2, (12, 128, 48, 64)).astype(np.float32)
    g = run_gpu(slk, P, corr, motion, net, inp, agg_kf)
    pick = [0, 9, 18, 27, 36, 47]
    rn, rd, rw, ra = uo.update_forward(P, corr[pick], motion[pick], net[pick], inp[pick])
    for name, ref in (("net", rn), ("delta", rd), ("weight", rw), ("agg", ra)):
        rel = check(g[name][pick], ref, name)
        print(f"[update window] {name} normwise {rel:.2e}", flush=True)
    re = uo.compute_eta(P, agg_kf[[0, 5, 11]])
    check(g["eta"][[0, 5, 11]], re, "eta")


def test_weights_from_reference_tensor_files(slk, tmp_path):
    """slk_update_load_dir reads the reference's exported tensor files
    (<name>_weight.bin / _bias.bin: int32 ndim, dims, float32 data) and gives
    bitwise the results of setting the same weights directly; a batch above
    max_batch and a missing file are rejected."""
    announce("update operator weights from .bin files")
    P = uo.seeded_weights(30)
    for name, (w, b) in P.items():
        uo.save_bin(os.path.join(tmp_path, name + "_weight.bin"), w)
        uo.save_bin(os.path.join(tmp_path, name + "_bias.bin"), b)
    corr, motion, net, inp = uo.seeded_inputs(2, 8, 40, seed=31)
    a = run_gpu(slk, P, corr, motion, net, inp)
    b = run_gpu(slk, None, corr, motion, net, inp, via_dir=str(tmp_path))
    for name in ("net", "delta", "weight", "agg"):
        np.testing.assert_array_equal(a[name], b[name])
    um = slk.UpdateModule(2, 8, 40)
    um.set_weights(P)
    x = slk.DeviceArray((4, 196, 8, 40))
    with pytest.raises(slk.SlkError):
        um.forward(x, x, x, x, x, x, x, 3)
    os.remove(os.path.join(tmp_path, "update_gru_convq_bias.bin"))
    with pytest.raises(slk.SlkError):
        um.load_dir(str(tmp_path))
    um.close()
    fresh = slk.UpdateModule(1, 8, 40)
    with pytest.raises(slk.SlkError):  # no weights set
        fresh.forward(x, x, x, x, x, x, x, 1)
    fresh.close()


@pytest.mark.parametrize("f16", [False, True])
def test_motion_filter(slk, f16):
    """compute_motion_gru (main.cu:1934-1983): the single-edge correlation of
    (last keyframe, current frame) sampled at the identity grid, one update
    step from the keyframe's state with zero motion, then the mean flow
    magnitude of delta; against the oracle lookup + update operator, and the
    keyframe's state is left unchanged. fp16 fmaps are the reference's
    storage (main.cu:677)."""
    from oracle import oracle as orc
    import workloads as wl
    orc.build()
    announce(f"motion filter 48x64 fp16={f16}")
    h, w = 48, 64
    P = uo.seeded_weights(40)
    f = wl.frames(2, C=128, h=h, w=w, seed=41)
    if f16:
        f = f.astype(np.float16)
    _, _, net, inp = uo.seeded_inputs(1, h, w, seed=42)
    ctx = slk.Context(h, w, C=128, max_batch=1, corr_scale=wl.CORR_ALPHA_REF)
    um = slk.UpdateModule(1, h, w)
    um.set_weights(P)
    D = slk.DeviceArray.from_host
    d0, d1, dn, di = D(f[0]), D(f[1]), D(net[0]), D(inp[0])
    dt = slk.SLK_F16 if f16 else slk.SLK_F32
    got = um.motion_filter(ctx, d0, d1, dn, di, dtype=dt)
    np.testing.assert_array_equal(dn.to_host(), net[0])
    ctx.close()
    um.close()
    grid = wl.grid_coords(h, w)[None].astype(np.float32)
    corr = orc.corr_batch(f.astype(np.float32), np.array([0], np.int32), np.array([1], np.int32),
                          grid, wl.CORR_ALPHA_REF)
    _, delta, _, _ = uo.update_forward(P, corr.reshape(1, 196, h, w),
                                       np.zeros((1, 4, h, w), np.float32), net, inp)
    mag = np.sqrt(delta[0, 0] ** 2 + delta[0, 1] ** 2).astype(np.float32).reshape(-1)
    ref = float(np.cumsum(mag, dtype=np.float32)[-1] / np.float32(h * w))
    assert abs(got - ref) <= 2e-3 * abs(ref), (got, ref)
