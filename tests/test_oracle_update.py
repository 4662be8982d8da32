"""Pins of the update-operator oracle (oracle/update_oracle.py), the checker
of the GPU UpdateModule / ConvGRU (cuda_slam/main.cu:385-667):
  * conv2d: an explicit loop over output pixels, channels and taps on small
    shapes (stride 1, padding k//2, cross-correlation like cuDNN's
    CUDNN_CROSS_CORRELATION, nn.cuh:145), scipy's correlate2d, and exact
    integer cases where operand rounding changes nothing;
  * round16: round-to-nearest-even fp16 at hand-picked ties;
  * the GRU and head arithmetic: a case whose convolutions reduce to their
    biases, evaluated by hand from the reference's sequence of roundings;
  * compute_eta's 0.01 * softplus at known points.
"""
import numpy as np
import pytest
from scipy.signal import correlate2d

from oracle import update_oracle as uo


def test_round16_ties_and_range():
    x = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -2.0 - 2.0 ** -10, 65504.0, 1e-8])
    want = np.array([1.0, 1.0 + 2.0 ** -9, -2.0, 65504.0, 0.0])
    np.testing.assert_array_equal(uo.round16(x), want)


def _conv_loop(x, w, b):
    N, Ci, H, W = x.shape
    Co, _, k, _ = w.shape
    p = k // 2
    out = np.zeros((N, Co, H, W))
    for n in range(N):
        for o in range(Co):
            for yy in range(H):
                for xx in range(W):
                    s = 0.0
                    for c in range(Ci):
                        for ky in range(k):
                            for kx in range(k):
                                y2, x2 = yy + ky - p, xx + kx - p
                                if 0 <= y2 < H and 0 <= x2 < W:
                                    s += w[o, c, ky, kx] * x[n, c, y2, x2]
                    out[n, o, yy, xx] = s + b[o]
    return out


@pytest.mark.parametrize("k", [1, 3, 7])
def test_conv2d_matches_direct_loop(k):
    rng = np.random.default_rng(k)
    x = uo.round16(rng.standard_normal((2, 3, 5, 6)))
    w = uo.round16(rng.standard_normal((4, 3, k, k)))
    b = rng.standard_normal(4)
    np.testing.assert_allclose(uo.conv2d(x, w, b), _conv_loop(x, w, b), rtol=1e-12, atol=1e-12)


def test_conv2d_matches_scipy_correlate():
    rng = np.random.default_rng(5)
    x = uo.round16(rng.standard_normal((1, 2, 9, 7)))
    w = uo.round16(rng.standard_normal((3, 2, 3, 3)))
    b = np.zeros(3)
    got = uo.conv2d(x, w, b)
    for o in range(3):
        ref = sum(correlate2d(x[0, c], w[o, c], mode="same", boundary="fill") for c in range(2))
        np.testing.assert_allclose(got[0, o], ref, rtol=1e-12, atol=1e-12)


def test_conv2d_rounds_operands_to_fp16():
    """The tensor-op product sees 10-bit-mantissa operands: an input of
    1 + 2^-12 acts as 1, a weight of 1 + 3*2^-11 as 1 + 2^-9."""
    x = np.full((1, 1, 1, 1), 1.0 + 2.0 ** -12)
    w = np.full((1, 1, 1, 1), 1.0 + 3 * 2.0 ** -11)
    assert uo.conv2d(x, w, [0.0])[0, 0, 0, 0] == 1.0 + 2.0 ** -9


def _bias_only_weights(bias):
    """Zero weights and the given scalar bias per layer name."""
    P = {}
    for name, co, ci, k in uo.LAYERS:
        P[name] = (np.zeros((co, ci, k, k)), np.full(co, bias.get(name, 0.0)))
    return P


def test_gru_and_heads_by_hand():
    """With all weights zero, every conv returns its bias, so one pixel's
    outputs follow from the reference's sequence (main.cu:464-532, 612-649)
    by hand."""
    bias = {"update_gru_convz": 0.3, "update_gru_convz_glo": -0.1,
            "update_gru_convr": 0.7, "update_gru_convq": 0.25,
            "update_gru_convq_glo": 0.5, "update_delta_2": 1.0 / 3.0,
            "update_weight_2": 0.2, "update_agg_conv1": 0.4,
            "update_delta_0": 0.1, "update_agg_eta_0": -0.6}
    P = _bias_only_weights(bias)
    r16 = uo.round16
    net0 = 0.123456
    corr, motion, _, inp = uo.seeded_inputs(1, 2, 3, seed=4)
    net = np.full((1, 128, 2, 3), net0)
    net1, delta, weight, agg = uo.update_forward(P, corr, motion, net, inp)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))  # noqa: E731
    z = r16(sig(r16(0.3) + r16(-0.1)))
    q = r16(np.tanh(r16(0.25) + r16(0.5)))
    n0 = r16(net0)
    want = r16((1 - z) * n0 + z * q)
    np.testing.assert_array_equal(net1, want)
    np.testing.assert_array_equal(delta, r16(1.0 / 3.0))
    np.testing.assert_array_equal(weight, r16(sig(0.2)))
    np.testing.assert_array_equal(agg, r16(0.4))
    eta = uo.compute_eta(P, agg)
    np.testing.assert_allclose(eta, 0.01 * np.log1p(np.exp(r16(-0.6))), rtol=1e-15)


def test_gate_and_pool_feed_the_global_terms():
    """A nonzero w bias changes z only through the pooled global term when
    convz_glo has weights: z = sigmoid(bz + round16(Wg . mean(gate))) with
    gate = round16(round16(sigmoid(round16(bw))) * net) per pixel."""
    bias = {"update_gru_w": 0.8, "update_gru_convz": 0.1}
    P = _bias_only_weights(bias)
    wz = np.zeros((128, 128, 1, 1))
    wz[:, 0, 0, 0] = 0.5  # every output channel reads channel 0 of the pooled vector
    P["update_gru_convz_glo"] = (wz, np.zeros(128))
    net = np.zeros((1, 128, 2, 2))
    net[0, 0] = [[0.5, -0.25], [0.75, 1.0]]
    corr, motion, _, inp = uo.seeded_inputs(1, 2, 2, seed=6)
    z_seen = {}
    orig = uo.sigmoid

    def spy(v):
        out = orig(v)
        z_seen.setdefault("calls", []).append(np.array(v))
        return out
    uo.sigmoid = spy
    try:
        uo.update_forward(P, corr, motion, net, inp)
    finally:
        uo.sigmoid = orig
    r16 = uo.round16
    g = r16(r16(orig(r16(0.8))) * net[0, 0])
    glo = g.mean()
    zpre = r16(0.1) + r16(0.5 * r16(glo))
    # calls: gate sigmoid, z sigmoid, r sigmoid, weight-head sigmoid
    np.testing.assert_allclose(z_seen["calls"][1][0, :, 0, 0], zpre, rtol=1e-15)


def test_forward_shapes_and_ranges():
    P = uo.seeded_weights(0)
    corr, motion, net, inp = uo.seeded_inputs(2, 6, 8, seed=2)
    net1, delta, weight, agg = uo.update_forward(P, corr, motion, net, inp)
    assert net1.shape == (2, 128, 6, 8) and delta.shape == (2, 3, 6, 8)
    assert weight.shape == (2, 3, 6, 8) and agg.shape == (2, 128, 6, 8)
    assert np.all(np.abs(net1) <= 1.0) and np.all((weight >= 0) & (weight <= 1))
    assert np.all(agg >= 0)
    for a in (net1, delta, weight, agg):
        np.testing.assert_array_equal(a, uo.round16(a))  # fp16-valued outputs
    eta = uo.compute_eta(P, agg[:1])
    assert eta.shape == (1, 1, 6, 8) and np.all(eta > 0)
