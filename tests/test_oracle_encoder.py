"""Pins of the front-of-pipe oracle (oracle/encoder_oracle.py), the checker
of the GPU encoders (HalfBasicEncoder, cuda_slam/main.cu:236-381), the
frame preprocessing (:1062-1075), the decode conversions (:944-1058) and the
pose file (:2893-2937):
  * the strided convolution against a direct loop and against the stride-1
    convolution of the update oracle subsampled (same padding k//2);
  * the encoder's wiring with the roundings off against torch float64
    modules of the published BasicEncoder architecture (conv 7x7/2, instance
    norm, three stages of two residual blocks with 1x1 downsample branches,
    conv 1x1), so a dropped branch, a wrong stride or norm shows;
  * the rounding sequence on a case whose convolutions reduce to their
    biases, by hand;
  * preprocess at hand-picked pixels; the resize at identity size and on
    linear ramps (bilinear interpolation reproduces them); BT.709 against the
    forward transform of its definition; P010 against NV12 on shifted data;
  * the pose inversion against SE3 composition with scipy's rotations.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.spatial.transform import Rotation

from oracle import encoder_oracle as eo
from oracle import update_oracle as uo


def _loop_conv(x, w, s):
    N, Ci, H, W = x.shape
    Co, _, k, _ = w.shape
    p = k // 2
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    out = np.zeros((N, Co, Ho, Wo))
    for n in range(N):
        for o in range(Co):
            for yy in range(Ho):
                for xx in range(Wo):
                    acc = 0.0
                    for c in range(Ci):
                        for ky in range(k):
                            for kx in range(k):
                                y2, x2 = s * yy + ky - p, s * xx + kx - p
                                if 0 <= y2 < H and 0 <= x2 < W:
                                    acc += w[o, c, ky, kx] * x[n, c, y2, x2]
                    out[n, o, yy, xx] = acc
    return out


@pytest.mark.parametrize("k,s", [(1, 1), (1, 2), (3, 1), (3, 2), (7, 2)])
def test_conv_sum_matches_direct_loop(k, s):
    rng = np.random.default_rng(10 * k + s)
    x = uo.round16(rng.standard_normal((2, 3, 9, 12)))
    w = uo.round16(rng.standard_normal((4, 3, k, k)))
    np.testing.assert_allclose(eo.conv_sum(x, w, s), _loop_conv(x, w, s), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("k", [1, 3, 7])
def test_stride2_is_stride1_subsampled(k):
    rng = np.random.default_rng(k)
    x = uo.round16(rng.standard_normal((1, 5, 16, 20)))
    w = uo.round16(rng.standard_normal((6, 5, k, k)))
    s1 = uo.conv2d(x, w, np.zeros(6))
    np.testing.assert_allclose(eo.conv_sum(x, w, 2), s1[:, :, ::2, ::2], rtol=1e-12, atol=1e-12)


def _torch_encoder(img, Q, norm, out_dim):
    """The published BasicEncoder of DROID-SLAM (norm 'instance' or 'none')
    written with torch modules, float64, no rounding."""
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731

    def conv(x, name, stride):
        w, b = Q[name]
        return F.conv2d(x, t(w), t(b), stride=stride, padding=w.shape[-1] // 2)

    def nrm(x):
        return F.instance_norm(x, eps=1e-5) if norm else x

    x = torch.relu(nrm(conv(t(img), "conv1", 2)))
    for name, stride in [("layer1_0", 1), ("layer1_1", 1), ("layer2_0", 2), ("layer2_1", 1),
                         ("layer3_0", 2), ("layer3_1", 1)]:
        y = torch.relu(nrm(conv(x, name + "_conv1", stride)))
        y = torch.relu(nrm(conv(y, name + "_conv2", 1)))
        if name + "_downsample_0" in Q:
            x = nrm(conv(x, name + "_downsample_0", stride))
        x = torch.relu(x + y)
    return conv(x, "conv2", 1).numpy()


@pytest.mark.parametrize("prefix,out_dim,norm", [("fnet", 128, True), ("cnet", 256, False)])
def test_encoder_wiring_matches_torch_modules(prefix, out_dim, norm):
    P = eo.seeded_weights(prefix, out_dim, seed=3)
    img = np.random.default_rng(4).standard_normal((2, 3, 32, 48))
    got = eo.encoder(img, P, prefix, norm, r=lambda v: v)
    Q = {k[len(prefix) + 1:]: v for k, v in P.items()}
    want = _torch_encoder(img, Q, norm, out_dim)
    assert got.shape == (2, out_dim, 4, 6)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-9)


def test_instance_norm_matches_torch():
    y = np.random.default_rng(5).normal(3.0, 2.0, (2, 4, 7, 9))
    got = eo.instance_norm(y, r=lambda v: v)
    want = F.instance_norm(torch.from_numpy(y), eps=1e-5).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_rounding_sequence_by_hand():
    """cnet with zero weights: every conv returns round16(f32(round16(0) +
    b)) = round16(b); the blocks then add relu(b2) to their input (or to the
    downsample's bias) and apply relu, rounding each sum once."""
    P = {}
    biases = {}
    for i, (suffix, co, ci, k, _) in enumerate(eo.LAYERS):
        co = 256 if co is None else co
        b = 0.1 * (i + 1) * (-1) ** i + 1.0 / 3.0
        biases[suffix] = b
        P["cnet_" + suffix] = (np.zeros((co, ci, k, k), np.float32), np.full(co, b, np.float32))
    r16 = uo.round16
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    B = {k: r16(f32(v)) for k, v in biases.items()}
    x = max(B["conv1"], 0.0)
    for name, _ in eo.BLOCKS:
        y = max(B[name + "_conv2"], 0.0)
        res = B[name + "_downsample_0"] if name + "_downsample_0" in B else x
        x = max(r16(y + res), 0.0)
    want = B["conv2"]  # the last conv sees only its bias
    out = eo.encoder(np.zeros((1, 3, 16, 16)), P, "cnet", False)
    np.testing.assert_array_equal(out, np.full(out.shape, want))
    # the value entering conv2 is x: check it through a 1x1 conv2 of ones
    P2 = dict(P)
    P2["cnet_conv2"] = (np.ones((256, 128, 1, 1), np.float32), np.zeros(256, np.float32))
    out2 = eo.encoder(np.zeros((1, 3, 16, 16)), P2, "cnet", False)
    np.testing.assert_array_equal(out2, np.full(out2.shape, r16(128 * x)))


def test_preprocess_known_pixels():
    bgr = np.array([[[255.0, 0.0, 128.0], [10.0, 20.0, 30.0]]], np.float32)
    out = eo.preprocess(bgr)
    assert out.shape == (3, 1, 2)
    mean = {"R": 0.485, "G": 0.456, "B": 0.406}
    std = {"R": 0.229, "G": 0.224, "B": 0.225}
    for px, (b, g, r) in enumerate([(255, 0, 128), (10, 20, 30)]):
        for ch, (name, v) in enumerate([("R", r), ("G", g), ("B", b)]):
            assert out[ch, 0, px] == pytest.approx((v / 255 - mean[name]) / std[name], abs=1e-6)


def test_resize_identity_and_ramps():
    rng = np.random.default_rng(6)
    bgr = rng.integers(0, 256, (10, 14, 3), dtype=np.uint8)
    np.testing.assert_array_equal(eo.bgr8_to_bgrf(bgr, 14, 10, 14, 10), bgr.astype(np.float32))
    # a linear ramp in x is reproduced by bilinear sampling away from the
    # clamped border: value = 2*x + 3 at x = sx
    xs = np.arange(40)
    ramp = np.broadcast_to((2 * xs + 3)[None, :, None], (6, 40, 3)).astype(np.uint8)
    out = eo.bgr8_to_bgrf(np.ascontiguousarray(ramp), 40, 6, 16, 6)
    sx = (np.arange(16) + 0.5) * 40 / 16 - 0.5
    inner = (sx >= 0) & (sx <= 39)
    np.testing.assert_allclose(out[0, inner, 0], 2 * sx[inner] + 3, atol=1e-4)
    # upsampling: edges clamp to the border pixel
    up = eo.bgr8_to_bgrf(np.ascontiguousarray(ramp), 40, 6, 80, 12)
    assert up[0, 0, 0] == ramp[0, 0, 0] and up[0, -1, 0] == ramp[0, -1, 0]


def _rgb_to_yuv709(r, g, b):
    """The forward BT.709 transform (Kr = 0.2126, Kb = 0.0722)."""
    y = 0.2126 * r + 0.7152 * g + 0.0722 * b
    return y, (b - y) / 1.8556, (r - y) / 1.5748


def test_bt709_inverts_the_forward_transform():
    rng = np.random.default_rng(7)
    rgb = rng.uniform(40, 215, (200, 3))
    y, u, v = _rgb_to_yuv709(rgb[:, 0], rgb[:, 1], rgb[:, 2])
    bgr = eo._yuv_to_bgr(y.astype(np.float32), u.astype(np.float32), v.astype(np.float32))
    np.testing.assert_allclose(bgr[:, ::-1], rgb, atol=0.02)


def test_nv12_constant_gray_and_p010_matches_nv12():
    H, W = 8, 12
    y = np.full((H, W), 77, np.uint8)
    uv = np.full((H // 2, W), 128, np.uint8)
    out = eo.nv12_to_bgr(y, uv, W, H, 6, 4)
    np.testing.assert_array_equal(out, np.full((4, 6, 3), 77, np.float32))
    rng = np.random.default_rng(8)
    y = rng.integers(0, 256, (H, W), dtype=np.uint8)
    uv = rng.integers(0, 256, (H // 2, W), dtype=np.uint8)
    a = eo.nv12_to_bgr(y, uv, W, H, 10, 7)
    b = eo.p010_to_bgr(y.astype(np.uint16) << 8, uv.astype(np.uint16) << 8, W, H, 10, 7)
    np.testing.assert_array_equal(a, b)


def test_pose_inversion_is_the_se3_inverse():
    rng = np.random.default_rng(9)
    q = Rotation.random(5, random_state=10).as_quat()  # x, y, z, w
    t = rng.normal(0, 2, (5, 3))
    poses = np.concatenate([t, q], 1).astype(np.float32)
    inv = eo.invert_poses(poses)
    for i in range(5):
        R = Rotation.from_quat(poses[i, 3:].astype(np.float64))
        Ri = Rotation.from_quat(inv[i, 3:].astype(np.float64))
        # (R, t) o (Ri, ti) = identity
        np.testing.assert_allclose((R * Ri).as_rotvec(), 0, atol=1e-6)
        np.testing.assert_allclose(R.apply(inv[i, :3].astype(np.float64)) + poses[i, :3], 0,
                                   atol=1e-5)
    blob = eo.poses_bin_bytes([4, 9, 11, 20, 31], poses, True)
    assert len(blob) == 4 + 5 * 4 + 5 * 28
    assert np.frombuffer(blob[:4], np.int32)[0] == 5
