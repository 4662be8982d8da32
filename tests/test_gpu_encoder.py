"""GPU parity of the front of the pipe through the C ABI: the fp16 encoders
(HalfBasicEncoder, cuda_slam/main.cu:236-381), encode_frame (:1465-1497),
preprocess_image_kernel (:1062-1075) and the decode conversions (:944-1058),
against oracle/encoder_oracle.py on the same seeded weights and frames.

Bars:
  * encoders: every output elementwise within 2e-2 * max(|r|, rms(r)) and
    normwise within 4e-3 of the float64-accumulation oracle. The reference
    rounds every activation to fp16 and accumulates in fp32, so some
    roundings land one fp16 step (2^-11) apart from the exact-sum oracle and
    propagate through the 16 layers. A float32-accumulation model of the
    same network (numpy, another summation order) is 9.4e-3 elementwise and
    1.5e-3 normwise from the oracle on the fmap of the 384 x 512 frame; the
    bars are about twice that;
  * the same network with one power-of-two tap per output channel makes
    every sum exact, so there the GPU must match bitwise (tap, stride,
    channel and residual indexing);
  * preprocess and the decode conversions: bitwise (float32 expressions in
    the reference's order, contraction off on both sides).
"""
import os

import numpy as np
import pytest

from helpers import announce, assert_close_rel, gpu_or_fail, norm_rel
from oracle import encoder_oracle as eo
from oracle import update_oracle as uo

pytestmark = pytest.mark.gpu
TOL_EL = 2e-2
TOL_NORM = 4e-3


@pytest.fixture(scope="module")
def slk():
    return gpu_or_fail()


def check(got, ref, what):
    assert np.all(np.isfinite(got)), what
    assert_close_rel(got, ref, tol=TOL_EL, what=what)
    rel = norm_rel(got, ref)
    print(f"[encoder] {what}: normwise {rel:.2e}, max |d| {np.abs(got - ref).max():.3g}",
          flush=True)
    assert rel < TOL_NORM, (what, rel)


@pytest.mark.parametrize("prefix,out_dim,norm", [("fnet", 128, True), ("cnet", 256, False)])
def test_encoder_forward_batch(slk, prefix, out_dim, norm):
    """HalfBasicEncoder::forward on 2 images of 64 x 96 (8 x 12 features):
    tiles cut by the borders at every stage; the output is fp16."""
    announce(f"encoder {prefix} 2 x 64x96")
    P = eo.seeded_weights(prefix, out_dim, seed=50)
    img = np.random.default_rng(51).standard_normal((2, 3, 64, 96)).astype(np.float32)
    enc = slk.Encoder(64, 96, out_dim, norm, max_batch=2)
    enc.set_weights(P, prefix)
    d_in = slk.DeviceArray.from_host(img)
    d_out = slk.DeviceArray((2, out_dim, 8, 12), np.float16)
    enc.forward(d_in, d_out, batch=2)
    slk.hip().sync()
    got = d_out.to_host().astype(np.float64)
    enc.close()
    ref = eo.encoder(uo.round16(img), P, prefix, norm)
    check(got, ref, f"{prefix} 64x96")


def test_encode_frame_full_size(slk):
    """encode_frame on a 384 x 512 BGR frame (the 48 x 64 feature maps of
    the headline window): fmap fp16, net = tanh, inp = relu."""
    announce("encode_frame 384x512")
    H, W = 384, 512
    Pf = eo.seeded_weights("fnet", 128, seed=60)
    Pc = eo.seeded_weights("cnet", 256, seed=61)
    bgr = eo.seeded_frame(H, W, seed=62)
    fnet = slk.Encoder(H, W, 128, True)
    cnet = slk.Encoder(H, W, 256, False)
    fnet.set_weights(Pf, "fnet")
    cnet.set_weights(Pc, "cnet")
    d_bgr = slk.DeviceArray.from_host(bgr)
    fmap = slk.DeviceArray((128, H // 8, W // 8), np.float16)
    net = slk.DeviceArray((128, H // 8, W // 8))
    inp = slk.DeviceArray((128, H // 8, W // 8))
    slk.encode_frame(fnet, cnet, d_bgr, fmap, net, inp)
    slk.hip().sync()
    got = fmap.to_host().astype(np.float64), net.to_host(), inp.to_host()
    fnet.close()
    cnet.close()
    ref = eo.encode_frame(bgr, Pf, Pc)
    for name, g, r in zip(("fmap", "net", "inp"), got, ref):
        check(g, r, name)


def single_tap_weights(prefix, out_dim, seed):
    """Each output channel reads one input channel at one tap with weight
    +-1 or +-0.5; biases random. Every convolution sum is one exact
    product, so the only roundings are the reference's own."""
    rng = np.random.default_rng(seed)
    P = {}
    for suffix, co, ci, k, _ in eo.LAYERS:
        co = out_dim if co is None else co
        w = np.zeros((co, ci, k, k), np.float32)
        for o in range(co):
            w[o, rng.integers(ci), rng.integers(k), rng.integers(k)] = rng.choice([1, -1, 0.5, -0.5])
        P[f"{prefix}_{suffix}"] = (w, rng.normal(0, 0.5, co).astype(np.float32))
    return P


def test_cnet_single_tap_weights_bitwise(slk):
    """cnet (no instance norm) with single-tap weights on 2 images of
    48 x 80: bitwise equal to the oracle."""
    announce("encoder cnet single-tap 2 x 48x80")
    P = single_tap_weights("cnet", 256, seed=55)
    img = np.random.default_rng(56).uniform(-4, 4, (2, 3, 48, 80)).astype(np.float32)
    enc = slk.Encoder(48, 80, 256, False, max_batch=2)
    enc.set_weights(P, "cnet")
    d_in = slk.DeviceArray.from_host(img)
    d_out = slk.DeviceArray((2, 256, 6, 10), np.float16)
    enc.forward(d_in, d_out, batch=2)
    slk.hip().sync()
    got = d_out.to_host().astype(np.float64)
    enc.close()
    ref = eo.encoder(uo.round16(img), P, "cnet", False)
    assert np.count_nonzero(ref) > ref.size // 4
    np.testing.assert_array_equal(got, ref)


def test_encoder_weights_from_files_and_errors(slk, tmp_path):
    """slk_encoder_load_dir reads <prefix>_<suffix>_weight.bin / _bias.bin
    (export_weights.py's tensor files) and gives bitwise the results of
    setting the same weights; bad shapes and missing files are rejected."""
    announce("encoder weights from .bin files")
    P = eo.seeded_weights("fnet", 128, seed=70)
    for name, (w, b) in P.items():
        uo.save_bin(os.path.join(tmp_path, name + "_weight.bin"), w)
        uo.save_bin(os.path.join(tmp_path, name + "_bias.bin"), b)
    img = np.random.default_rng(71).standard_normal((1, 3, 32, 64)).astype(np.float32)
    outs = []
    for via_dir in (False, True):
        enc = slk.Encoder(32, 64, 128, True)
        if via_dir:
            enc.load_dir(str(tmp_path), "fnet")
        else:
            enc.set_weights(P, "fnet")
        d_in = slk.DeviceArray.from_host(img)
        d_out = slk.DeviceArray((1, 128, 4, 8), np.float16)
        enc.forward(d_in, d_out)
        slk.hip().sync()
        outs.append(d_out.to_host())
        enc.close()
    np.testing.assert_array_equal(outs[0], outs[1])
    enc = slk.Encoder(32, 64, 128, True)
    x = slk.DeviceArray((2, 3, 32, 64))
    with pytest.raises(slk.SlkError):  # no weights
        enc.forward(x, x)
    enc.set_weights(P, "fnet")
    with pytest.raises(slk.SlkError):  # batch above max_batch
        enc.forward(x, x, batch=2)
    os.remove(os.path.join(tmp_path, "fnet_layer3_0_downsample_0_bias.bin"))
    with pytest.raises(slk.SlkError):
        enc.load_dir(str(tmp_path), "fnet")
    enc.close()
    for args in ((30, 64, 128, True), (32, 64, 100, True), (32, 64, 512, False)):
        with pytest.raises(slk.SlkError):
            slk.Encoder(*args)


def test_preprocess_bitwise(slk):
    announce("preprocess 48x80")
    bgr = eo.seeded_frame(48, 80, seed=80)
    d = slk.DeviceArray.from_host(bgr)
    out = slk.DeviceArray((3, 48, 80))
    slk.preprocess_image(d, out, 48, 80)
    slk.hip().sync()
    np.testing.assert_array_equal(out.to_host(), eo.preprocess(bgr))


@pytest.mark.parametrize("src,dst", [((1920, 1080), (512, 288)), ((64, 48), (160, 96)),
                                     ((50, 30), (50, 30))])
def test_decode_conversions_bitwise(slk, src, dst):
    """NV12, P010 and 8-bit BGR sources with padded row strides, down- and
    upsampled and at identity size, bitwise against the float32 oracle."""
    (sw, sh), (dw, dh) = src, dst
    announce(f"decode {sw}x{sh} -> {dw}x{dh}")
    rng = np.random.default_rng(sw + dh)
    pad = 64
    y = rng.integers(0, 256, (sh, sw + pad), dtype=np.uint8)
    uv = rng.integers(0, 256, (sh // 2, sw + pad), dtype=np.uint8)
    out = slk.DeviceArray((dh, dw, 3))
    dy, duv = slk.DeviceArray.from_host(y), slk.DeviceArray.from_host(uv)
    slk.nv12_to_bgr(dy, duv, out, sw, sh, sw + pad, sw + pad, dw, dh)
    slk.hip().sync()
    np.testing.assert_array_equal(out.to_host(), eo.nv12_to_bgr(y, uv, sw, sh, dw, dh))
    y16 = (rng.integers(0, 1024, (sh, sw + pad)) << 6).astype(np.uint16)
    uv16 = (rng.integers(0, 1024, (sh // 2, sw + pad)) << 6).astype(np.uint16)
    dy16, duv16 = slk.DeviceArray.from_host(y16), slk.DeviceArray.from_host(uv16)
    slk.p010_to_bgr(dy16, duv16, out, sw, sh, 2 * (sw + pad), 2 * (sw + pad), dw, dh)
    slk.hip().sync()
    np.testing.assert_array_equal(out.to_host(), eo.p010_to_bgr(y16, uv16, sw, sh, dw, dh))
    bgr = rng.integers(0, 256, (sh, sw * 3 + pad), dtype=np.uint8)
    db = slk.DeviceArray.from_host(bgr)
    slk.bgr8_to_bgrf(db, out, sw, sh, sw * 3 + pad, dw, dh)
    slk.hip().sync()
    src3 = bgr[:, :sw * 3].reshape(sh, sw, 3)
    np.testing.assert_array_equal(out.to_host(), eo.bgr8_to_bgrf(src3, sw, sh, dw, dh))
