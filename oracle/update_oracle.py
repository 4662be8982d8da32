"""CPU restatement (numpy, float64) of the DROID-SLAM update operator:
UpdateModule::forward and UpdateModule::compute_eta with ConvGRU::forward
(cuda_slam/main.cu:385-667), the layer that turns the 196-channel correlation
lookup into delta / weight (the BA targets), the new hidden state and the
GraphAgg features.

TEST INFRASTRUCTURE, NOT PRODUCT CODE: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it, as the checker.

Numerics restated:
  * Every convolution is cuDNN with CUDNN_TENSOR_OP_MATH on fp32 tensors
    (nn.cuh:146), i.e. tensor-core products of operands rounded to a 10-bit
    mantissa with fp32 accumulation. The oracle rounds both operands (weights
    and inputs) to fp16, which keeps that 10-bit mantissa, and forms the dot
    products exactly in float64; the bias is added after the convolution
    (cudnnAddTensor, nn.cuh:232-238).
  * round16(x) is round_to_fp16 (nn.cuh:563-569): round to nearest even
    fp16, back to float. It is applied exactly where the reference applies it.
  * sigmoid, tanh and 0.01 * log(1 + exp(x)) are evaluated in float64
    (nn.cuh:274-292).

Parity of this module is pinned in tests/test_oracle_update.py: conv2d
against a direct loop over taps and scipy.signal.correlate on small shapes,
the GRU elementwise steps against hand-worked values, and the composition
against the call order of main.cu:606-667 on a small case.
"""
from __future__ import annotations

import numpy as np

# layer order of the weight table (name -> (Co, Ci, k)); the names are the
# reference's weight files without the _weight/_bias suffix (main.cu:552-603,
# 396-425)
LAYERS = [
    ("update_corr_encoder_0", 128, 196, 1),
    ("update_corr_encoder_2", 128, 128, 3),
    ("update_flow_encoder_0", 128, 4, 7),
    ("update_flow_encoder_2", 64, 128, 3),
    ("update_gru_convz", 128, 448, 3),
    ("update_gru_convr", 128, 448, 3),
    ("update_gru_convq", 128, 448, 3),
    ("update_gru_convz_glo", 128, 128, 1),
    ("update_gru_convr_glo", 128, 128, 1),
    ("update_gru_convq_glo", 128, 128, 1),
    ("update_gru_w", 128, 128, 1),
    ("update_weight_0", 128, 128, 3),
    ("update_weight_2", 3, 128, 3),
    ("update_delta_0", 128, 128, 3),
    ("update_delta_2", 3, 128, 3),
    ("update_agg_conv1", 128, 128, 3),
    ("update_agg_conv2", 128, 128, 3),
    ("update_agg_eta_0", 1, 128, 3),
]
LAYER_INDEX = {name: i for i, (name, _, _, _) in enumerate(LAYERS)}


def round16(x):
    """round_to_fp16 (nn.cuh:563-569): nearest-even fp16, then back."""
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def conv2d(x, w, b):
    """ConvLayer::forward (nn.cuh:196-240): stride 1, padding k//2, the
    tensor-op product of fp16-rounded operands, exact accumulation, then the
    bias. x [N, Ci, H, W], w [Co, Ci, k, k], b [Co] -> [N, Co, H, W]."""
    x = round16(x)
    w = round16(w)
    N, Ci, H, W = x.shape
    Co, _, k, _ = w.shape
    p = k // 2
    xp = np.zeros((N, Ci, H + 2 * p, W + 2 * p))
    xp[:, :, p:p + H, p:p + W] = x
    out = np.zeros((N, Co, H * W))
    for ky in range(k):
        for kx in range(k):
            patch = xp[:, :, ky:ky + H, kx:kx + W].reshape(N, Ci, H * W)
            out += np.einsum("oc,ncp->nop", w[:, :, ky, kx], patch, optimize=True)
    return out.reshape(N, Co, H, W) + np.asarray(b, np.float64)[None, :, None, None]


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def relu(x):
    return np.maximum(x, 0.0)


def conv_gru(P, net, inp, corr, flow):
    """ConvGRU::forward (main.cu:454-530). net, inp [N,128,H,W]; corr
    [N,128,H,W], flow [N,64,H,W]. Returns the new net (fp16-valued)."""
    L = lambda name: P[name]  # noqa: E731
    net = round16(net)                                            # :464
    cat = np.concatenate([net, inp, corr, flow], axis=1)           # :467-471
    gate = round16(conv2d(net, *L("update_gru_w")))                # :474-475
    gate = round16(sigmoid(gate))                                  # :476-477
    gate = round16(gate * net)                                     # :479-480
    glo = gate.mean(axis=(2, 3), keepdims=True)                    # :482-486
    z = round16(conv2d(cat, *L("update_gru_convz")))               # :490-491
    zg = round16(conv2d(glo, *L("update_gru_convz_glo")))          # :492-493
    z = round16(sigmoid(z + zg))                                   # :494-496
    r = round16(conv2d(cat, *L("update_gru_convr")))               # :499-500
    rg = round16(conv2d(glo, *L("update_gru_convr_glo")))          # :501-502
    r = round16(sigmoid(r + rg))                                   # :503-505
    rnet = net * r                                                 # :509-511
    gin = np.concatenate([rnet, inp, corr, flow], axis=1)          # :513-517
    q = round16(conv2d(gin, *L("update_gru_convq")))               # :520-521
    qg = round16(conv2d(glo, *L("update_gru_convq_glo")))          # :522-523
    q = round16(np.tanh(q + qg))                                   # :524-526
    net = (1.0 - z) * net + z * q                                  # :529
    return round16(net)                                            # :532


def update_forward(P, corr, motion, net, inp):
    """UpdateModule::forward (main.cu:606-650). corr [N,196,H,W] (the
    lookup), motion [N,4,H,W], net/inp [N,128,H,W]. Returns (net, delta
    [N,3,H,W], weight [N,3,H,W], agg_conv1 [N,128,H,W])."""
    L = lambda name: P[name]  # noqa: E731
    c = round16(relu(conv2d(corr, *L("update_corr_encoder_0"))))   # :612-614
    c = round16(relu(conv2d(c, *L("update_corr_encoder_2"))))      # :615-617
    f = round16(relu(conv2d(motion, *L("update_flow_encoder_0"))))  # :620-622
    f = round16(relu(conv2d(f, *L("update_flow_encoder_2"))))      # :623-625
    net = conv_gru(P, net, inp, c, f)                              # :628
    t = round16(relu(conv2d(net, *L("update_delta_0"))))           # :631-633
    delta = round16(conv2d(t, *L("update_delta_2")))               # :634-635
    t = round16(relu(conv2d(net, *L("update_weight_0"))))          # :638-640
    weight = round16(sigmoid(conv2d(t, *L("update_weight_2"))))    # :641-643
    agg = round16(relu(conv2d(net, *L("update_agg_conv1"))))       # :647-649
    return net, delta, weight, agg


def compute_eta(P, agg):
    """UpdateModule::compute_eta (main.cu:654-667): agg [K,128,H,W] (the
    scatter-mean features) -> eta [K,1,H,W]."""
    agg = round16(agg)                                                         # :659
    t = round16(relu(conv2d(agg, *P["update_agg_conv2"])))                     # :660-662
    e = round16(conv2d(t, *P["update_agg_eta_0"]))                             # :663-664
    return 0.01 * np.log1p(np.exp(e))                                          # :665


def seeded_weights(seed=0):
    """Random weights of the reference's shapes, He-style scale
    N(0, 1/fan_in) per layer, biases N(0, 0.1): a plausible trained-network
    range (no checkpoint is available here). float32 numpy arrays,
    {name: (w [Co,Ci,k,k], b [Co])}."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, co, ci, k in LAYERS:
        w = rng.standard_normal((co, ci, k, k)) / np.sqrt(ci * k * k)
        b = rng.normal(0.0, 0.1, co)
        out[name] = (w.astype(np.float32), b.astype(np.float32))
    return out


def seeded_inputs(N, H, W, seed=1):
    """Update-operator inputs of realistic ranges: corr ~ N(0,1) (lookup
    values at alpha = 1/16), motion = clamped flow/residual in [-8, 8] px,
    net = a GRU state in [-1, 1], inp ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    corr = rng.standard_normal((N, 196, H, W)).astype(np.float32)
    motion = rng.uniform(-8.0, 8.0, (N, 4, H, W)).astype(np.float32)
    net = rng.uniform(-1.0, 1.0, (N, 128, H, W)).astype(np.float32)
    inp = rng.standard_normal((N, 128, H, W)).astype(np.float32)
    return corr, motion, net, inp


def save_bin(path, arr):
    """The reference's tensor file (export_weights.py:14-22, read by
    load_tensor nn.cuh:91-107): int32 ndim, int32 dims, float32 data."""
    a = np.ascontiguousarray(arr, np.float32)
    with open(path, "wb") as f:
        np.array([a.ndim] + list(a.shape), np.int32).tofile(f)
        a.tofile(f)
