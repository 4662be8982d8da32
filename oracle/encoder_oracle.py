"""CPU restatement (numpy) of the front of the DROID-SLAM pipe: the fp16
feature / context encoders HalfBasicEncoder with HalfResBlock
(cuda_slam/main.cu:236-381), CudaDroid::encode_frame (:1465-1497) with
preprocess_image_kernel (:1062-1075), the decode-side conversions to float
BGR (:944-1058) and the keyframe pose file (:2893-2937).

TEST INFRASTRUCTURE, NOT PRODUCT CODE: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it, as the checker.

Numerics restated:
  * HalfConvLayer::forward (nn.cuh:737-790): fp16 weights and activations,
    the product formed exactly here (float64), the sum written as fp16
    (round16), then the fp32 bias added in fp32 and rounded to fp16 again
    (bias_add_half_kernel, nn.cuh:657-665);
  * instance_norm_half_kernel (nn.cuh:609-654): mean and biased variance per
    (image, channel) over h*w, eps 1e-5, (x - mean) * rsqrt(var + eps)
    rounded to fp16; evaluated in float64 here;
  * relu of fp16 is exact, add_half_kernel rounds the sum once;
  * the decode conversions and the preprocessing are float32 expressions
    evaluated in the reference's operation order, every operation rounded
    once (numpy float32 arithmetic is IEEE), which is what the GPU kernels
    compute with contraction switched off.

Every function is pinned in tests/test_oracle_encoder.py (direct loops,
the stride-1 convolution subsampled, torch float64 modules of the same
architecture, hand-worked values, closed forms of the resize and colour
conversion, the SE3 inverse).
"""
from __future__ import annotations

import numpy as np

from oracle.update_oracle import round16

# (suffix, co, ci, k, stride); co of conv2 is the encoder's output_dim
# (HalfBasicEncoder::init, main.cu:316-353; HalfResBlock::init :245-266)
LAYERS = [
    ("conv1", 32, 3, 7, 2),
    ("layer1_0_conv1", 32, 32, 3, 1), ("layer1_0_conv2", 32, 32, 3, 1),
    ("layer1_1_conv1", 32, 32, 3, 1), ("layer1_1_conv2", 32, 32, 3, 1),
    ("layer2_0_conv1", 64, 32, 3, 2), ("layer2_0_conv2", 64, 64, 3, 1),
    ("layer2_0_downsample_0", 64, 32, 1, 2),
    ("layer2_1_conv1", 64, 64, 3, 1), ("layer2_1_conv2", 64, 64, 3, 1),
    ("layer3_0_conv1", 128, 64, 3, 2), ("layer3_0_conv2", 128, 128, 3, 1),
    ("layer3_0_downsample_0", 128, 64, 1, 2),
    ("layer3_1_conv1", 128, 128, 3, 1), ("layer3_1_conv2", 128, 128, 3, 1),
    ("conv2", None, 128, 1, 1),
]

# stride and presence of a downsample branch of the six blocks (main.cu:329-349)
BLOCKS = [("layer1_0", 1), ("layer1_1", 1), ("layer2_0", 2), ("layer2_1", 1),
          ("layer3_0", 2), ("layer3_1", 1)]


def f32(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float64)


def conv_sum(x, w, stride, round_operands=True):
    """The convolution sum (no bias) of fp16-rounded operands, exact:
    stride s, padding k//2, cross-correlation (cudnnSetConvolution2dDescriptor
    with CUDNN_CROSS_CORRELATION, nn.cuh:704-705). x [N, Ci, H, W],
    w [Co, Ci, k, k] -> [N, Co, (H + 2p - k)//s + 1, ...]. With
    round_operands=False the operands are taken as given."""
    x = round16(x) if round_operands else np.asarray(x, np.float64)
    w = round16(w) if round_operands else np.asarray(w, np.float64)
    N, Ci, H, W = x.shape
    Co, _, k, _ = w.shape
    p = k // 2
    Ho, Wo = (H + 2 * p - k) // stride + 1, (W + 2 * p - k) // stride + 1
    xp = np.zeros((N, Ci, H + 2 * p, W + 2 * p))
    xp[:, :, p:p + H, p:p + W] = x
    out = np.zeros((N, Co, Ho * Wo))
    for ky in range(k):
        for kx in range(k):
            patch = xp[:, :, ky:ky + stride * (Ho - 1) + 1:stride,
                       kx:kx + stride * (Wo - 1) + 1:stride].reshape(N, Ci, Ho * Wo)
            out += np.einsum("oc,ncp->nop", w[:, :, ky, kx], patch, optimize=True)
    return out.reshape(N, Co, Ho, Wo)


def half_conv(x, w, b, stride, r=round16):
    """HalfConvLayer::forward + bias_add_half_kernel: round16(f32(round16(sum)
    + b)). With r = identity: the plain float64 convolution plus bias."""
    rounded = r is round16
    s = conv_sum(x, w, stride, round_operands=rounded)
    bb = np.asarray(b, np.float64)[None, :, None, None]
    return round16(f32(round16(s) + bb)) if rounded else s + bb


def instance_norm(y, r=round16, eps=1e-5):
    """instance_norm_half_kernel (nn.cuh:609-654) per (image, channel)."""
    mean = y.mean(axis=(2, 3), keepdims=True)
    var = ((y - mean) ** 2).mean(axis=(2, 3), keepdims=True)
    return r((y - mean) / np.sqrt(var + eps))


def relu(x):
    return np.maximum(x, 0.0)


def res_block(x, P, name, stride, norm, r=round16):
    """HalfResBlock::forward (main.cu:268-290)."""
    has_ds = (name + "_downsample_0") in P
    t = half_conv(x, *P[name + "_conv1"], stride, r=r)
    if norm:
        t = instance_norm(t, r)
    t = relu(t)
    y = half_conv(t, *P[name + "_conv2"], 1, r=r)
    if norm:
        y = instance_norm(y, r)
    y = relu(y)
    if has_ds:
        res = half_conv(x, *P[name + "_downsample_0"], stride, r=r)
        if norm:
            res = instance_norm(res, r)
    else:
        res = x
    return relu(r(y + res))


def encoder(img, P, prefix, norm, r=round16):
    """HalfBasicEncoder::forward (main.cu:357-380): img [N, 3, H, W] (fp16
    values, float_to_half of the input) -> [N, out_dim, H/8, W/8] fp16
    values. P maps '<prefix>_<suffix>' to (w, b)."""
    Q = {k[len(prefix) + 1:]: v for k, v in P.items() if k.startswith(prefix + "_")}
    x = half_conv(img, *Q["conv1"], 2, r=r)
    if norm:
        x = instance_norm(x, r)
    x = relu(x)
    for name, stride in BLOCKS:
        x = res_block(x, Q, name, stride, norm, r=r)
    return half_conv(x, *Q["conv2"], 1, r=r)


def preprocess(bgr):
    """preprocess_image_kernel (main.cu:1062-1075): bgr [H, W, 3] (0..255)
    -> rgb [3, H, W] float32: (bgr / 255 - mean) / std, channel c of BGR to
    RGB channel 2 - c."""
    bgr = np.asarray(bgr, np.float32)
    mean = np.array([0.406, 0.456, 0.485], np.float32)
    std = np.array([0.225, 0.224, 0.229], np.float32)
    v = (bgr / np.float32(255.0) - mean) / std
    return np.ascontiguousarray(v[:, :, ::-1].transpose(2, 0, 1))


def encode_frame(bgr, Pf, Pc):
    """CudaDroid::encode_frame (main.cu:1465-1497): fmap [128, h, w] (fp16
    values), net = tanh(cmap[:128]), inp = relu(cmap[128:]) (fp32 of fp16
    values)."""
    img = round16(preprocess(bgr)[None])
    fmap = encoder(img, Pf, "fnet", True)[0]
    cmap = encoder(img, Pc, "cnet", False)[0]
    return fmap, np.tanh(cmap[:128]), relu(cmap[128:])


def seeded_weights(prefix, out_dim, seed=0):
    """Random weights of the encoder's shapes: N(0, 1/fan_in) (He-style, the
    activations stay O(1) through the ReLU blocks), biases N(0, 0.1).
    {prefix_suffix: (w, b)} float32."""
    rng = np.random.default_rng(seed)
    out = {}
    for suffix, co, ci, k, _ in LAYERS:
        co = out_dim if co is None else co
        w = rng.standard_normal((co, ci, k, k)) / np.sqrt(ci * k * k)
        b = rng.normal(0.0, 0.1, co)
        out[f"{prefix}_{suffix}"] = (w.astype(np.float32), b.astype(np.float32))
    return out


def seeded_frame(H, W, seed=0):
    """A BGR frame [H, W, 3] in 0..255 with image-like structure: smooth
    gradients, a few rectangles and per-pixel noise."""
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:H, 0:W].astype(np.float32)
    img = np.stack([127 + 100 * np.sin(x / 17.0 + c) * np.cos(y / 23.0 - c) for c in range(3)], -1)
    for _ in range(6):
        y0, x0 = rng.integers(0, H - 8), rng.integers(0, W - 8)
        img[y0:y0 + rng.integers(4, H // 3), x0:x0 + rng.integers(4, W // 3)] = rng.uniform(0, 255, 3)
    img += rng.normal(0, 8, img.shape)
    return np.clip(img, 0, 255).astype(np.float32)


# ---------------------------------------------------------------- decoding
_F = np.float32


def _bilin(src_w, src_h, dst_w, dst_h):
    """Source positions of the output grid (main.cu:957-962), float32."""
    dx = np.arange(dst_w, dtype=_F)
    dy = np.arange(dst_h, dtype=_F)
    sx = (dx + _F(0.5)) * _F(src_w) / _F(dst_w) - _F(0.5)
    sy = (dy + _F(0.5)) * _F(src_h) / _F(dst_h) - _F(0.5)
    x0 = np.floor(sx).astype(np.int64)
    y0 = np.floor(sy).astype(np.int64)
    wx = sx - x0.astype(_F)
    wy = sy - y0.astype(_F)
    x1 = np.minimum(x0 + 1, src_w - 1)
    y1 = np.minimum(y0 + 1, src_h - 1)
    x0 = np.maximum(x0, 0)
    y0 = np.maximum(y0, 0)
    return sx, sy, x0, x1, y0, y1, wx, wy


def _lerp(plane, g):
    """(1-wy)*((1-wx)*v00 + wx*v01) + wy*((1-wx)*v10 + wx*v11), float32 in
    that order."""
    _, _, x0, x1, y0, y1, wx, wy = g
    wx = wx[None, :]
    wy = wy[:, None]
    v = lambda yy, xx: plane[yy[:, None], xx[None, :]].astype(_F)  # noqa: E731
    one = _F(1)
    return (one - wy) * ((one - wx) * v(y0, x0) + wx * v(y0, x1)) + \
        wy * ((one - wx) * v(y1, x0) + wx * v(y1, x1))


def _uv_index(g, src_w, src_h):
    sx, sy = g[0], g[1]
    ux = ((sx + _F(0.5)).astype(np.int64) // 2) * 2
    uy = (sy + _F(0.5)).astype(np.int64) // 2
    return np.clip(ux, 0, src_w - 2), np.clip(uy, 0, src_h // 2 - 1)


def _yuv_to_bgr(Y, U, V):
    R = Y + _F(1.5748) * V
    G = Y - _F(0.1873) * U - _F(0.4681) * V
    B = Y + _F(1.8556) * U
    return np.clip(np.stack([B, G, R], -1), _F(0), _F(255)).astype(_F)


def nv12_to_bgr(y_plane, uv_plane, src_w, src_h, dst_w, dst_h):
    """nv12_to_bgr_resize_kernel (main.cu:947-985). y_plane [src_h, >=src_w]
    uint8, uv_plane [src_h/2, >=src_w] uint8 (U, V interleaved)."""
    g = _bilin(src_w, src_h, dst_w, dst_h)
    Y = _lerp(y_plane, g)
    ux, uy = _uv_index(g, src_w, src_h)
    U = uv_plane[uy[:, None], ux[None, :]].astype(_F) - _F(128)
    V = uv_plane[uy[:, None], ux[None, :] + 1].astype(_F) - _F(128)
    return _yuv_to_bgr(Y, U, V)


def p010_to_bgr(y_plane, uv_plane, src_w, src_h, dst_w, dst_h):
    """p010_to_bgr_resize_kernel (main.cu:988-1027): uint16 planes with the
    10 significant bits on top, scaled to 0..255 as (v >> 6) / 4."""
    yv = (y_plane >> 6).astype(_F) / _F(4)
    g = _bilin(src_w, src_h, dst_w, dst_h)
    Y = _lerp(yv, g)
    ux, uy = _uv_index(g, src_w, src_h)
    U = (uv_plane[uy[:, None], ux[None, :]] >> 6).astype(_F) / _F(4) - _F(128)
    V = (uv_plane[uy[:, None], ux[None, :] + 1] >> 6).astype(_F) / _F(4) - _F(128)
    return _yuv_to_bgr(Y, U, V)


def bgr8_to_bgrf(bgr, src_w, src_h, dst_w, dst_h):
    """bgr8_to_bgrf_resize_kernel (main.cu:1030-1058): bgr [src_h, src_w, 3]
    uint8 -> [dst_h, dst_w, 3] float32."""
    g = _bilin(src_w, src_h, dst_w, dst_h)
    return np.stack([_lerp(bgr[:, :, c], g) for c in range(3)], -1).astype(_F)


def invert_poses(poses):
    """world->camera to camera->world in the reference's float arithmetic
    (main.cu:2896-2914): q^-1 = conjugate, t^-1 = -(q^-1 applied to t)."""
    p = np.array(poses, _F).reshape(-1, 7)
    out = p.copy()
    two = _F(2)
    for i in range(p.shape[0]):
        qi = np.array([-p[i, 3], -p[i, 4], -p[i, 5], p[i, 6]], _F)
        t = -p[i, :3]
        uv = np.array([two * (qi[1] * t[2] - qi[2] * t[1]),
                       two * (qi[2] * t[0] - qi[0] * t[2]),
                       two * (qi[0] * t[1] - qi[1] * t[0])], _F)
        out[i, 0] = t[0] + qi[3] * uv[0] + (qi[1] * uv[2] - qi[2] * uv[1])
        out[i, 1] = t[1] + qi[3] * uv[1] + (qi[2] * uv[0] - qi[0] * uv[2])
        out[i, 2] = t[2] + qi[3] * uv[2] + (qi[0] * uv[1] - qi[1] * uv[0])
        out[i, 3:] = qi
    return out


def poses_bin_bytes(timestamps, poses, cam_to_world):
    """The file of main.cu:2924-2937: [nk: i32][timestamps: i32 x nk]
    [poses: f32 x nk x 7]."""
    ts = np.asarray(timestamps, np.int32)
    p = invert_poses(poses) if cam_to_world else np.asarray(poses, _F).reshape(-1, 7)
    return np.int32(ts.shape[0]).tobytes() + ts.tobytes() + p.astype(_F).tobytes()
