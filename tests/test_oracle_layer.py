"""Pins of the layer oracle (oracle/layer.py) against facts that do not come
from retyping its formulas: shifts, an independent per-element loop, the tail
rules, segment invariance, the reference's own worked example for the L2
modes, softplus/sigmoid identities, and the epilogue's scale invariance."""
import numpy as np
import pytest

from oracle import layer as ol
from oracle.gdn import l2_normalize, round_bf16


def rng(seed=0):
    return np.random.default_rng(seed)


def test_conv_one_hot_weights_shift_the_input():
    """weight[:, j] = 1 (else 0) gives y_t = silu(x_{t - (K-1) + j}): tap K-1
    is the current input, tap 0 the oldest, reaching into the tail."""
    r = rng(1)
    x = r.standard_normal((2, 9, 5)).astype(np.float32)
    tail = r.standard_normal((2, 3, 5)).astype(np.float32)
    ext = np.concatenate([tail, x], axis=1)
    for j in range(4):
        w = np.zeros((5, 4), np.float32)
        w[:, j] = 1
        y, _ = ol.short_convolution(x, tail, w)
        shift = 3 - j
        np.testing.assert_allclose(y, ol.silu(ext[:, 3 - shift:3 - shift + 9]), rtol=1e-6, atol=1e-7)


def test_conv_matches_an_independent_loop():
    r = rng(2)
    x = r.standard_normal((1, 6, 3)).astype(np.float64)
    tail = r.standard_normal((1, 2, 3)).astype(np.float64)
    w = r.standard_normal((3, 3))
    y, new_tail = ol.short_convolution(x, tail, w)
    for t in range(6):
        for c in range(3):
            acc = 0.0
            for j in range(3):
                src = t - 2 + j  # token index of tap j
                val = tail[0, 2 + src, c] if src < 0 else x[0, src, c]
                acc += w[c, j] * val
            assert abs(y[0, t, c] - acc / (1 + np.exp(-acc))) < 1e-12
    np.testing.assert_array_equal(new_tail, x[:, -2:])


def test_conv_tail_rules():
    """T < K-1: the new tail keeps part of the old one; K = 1: the tail is
    empty; no weight: SiLU only and the tail is returned unchanged."""
    r = rng(3)
    x = r.standard_normal((1, 2, 4)).astype(np.float32)
    tail = r.standard_normal((1, 3, 4)).astype(np.float32)
    _, new_tail = ol.short_convolution(x, tail, np.ones((4, 4), np.float32))
    np.testing.assert_array_equal(new_tail, np.concatenate([tail[:, 2:], x], axis=1))
    y, t1 = ol.short_convolution(x, np.zeros((1, 0, 4), np.float32), 2 * np.ones((4, 1), np.float32))
    np.testing.assert_allclose(y, ol.silu(2 * x), rtol=1e-6)
    assert t1.shape == (1, 0, 4)
    y, t2 = ol.short_convolution(x, tail, None)
    np.testing.assert_allclose(y, ol.silu(x), rtol=1e-6)
    assert t2 is tail


def test_conv_segments_with_carried_tail_equal_one_pass():
    r = rng(4)
    x = r.standard_normal((2, 50, 6)).astype(np.float64)
    tail = r.standard_normal((2, 3, 6))
    w = r.standard_normal((6, 4))
    y, t_end = ol.short_convolution(x, tail, w)
    y1, t1 = ol.short_convolution(x[:, :17], tail, w)
    y2, t2 = ol.short_convolution(x[:, 17:18], t1, w)
    y3, t3 = ol.short_convolution(x[:, 18:], t2, w)
    np.testing.assert_allclose(np.concatenate([y1, y2, y3], axis=1), y, rtol=1e-12, atol=1e-13)
    np.testing.assert_array_equal(t3, t_end)


def test_conv_rounds_the_tail_through_the_input_dtype():
    """cat(tail.to(x.dtype), x): with bf16 inputs the fp32 tail enters (and
    leaves, as the new tail) rounded to bf16."""
    tail = np.full((1, 3, 2), 1 + 2.0 ** -12, np.float32)  # not a bf16 value
    x = np.zeros((1, 1, 2), np.float32)
    _, new_tail = ol.short_convolution(x, tail, np.ones((2, 4), np.float32), x_dtype="bf16")
    np.testing.assert_array_equal(new_tail[:, :2], round_bf16(tail[:, 1:]))
    assert not np.array_equal(new_tail[:, :2], tail[:, 1:])


def test_l2_modes_on_the_reference_example():
    """gated_deltanet.py:62-64: [1e-4, 0] -> [1, 0] ('max') vs [0.0995, 0] ('hf')."""
    x = np.array([1e-4, 0.0], np.float32)
    np.testing.assert_allclose(l2_normalize(x, "max"), [1.0, 0.0], rtol=1e-6)
    np.testing.assert_allclose(l2_normalize(x, "hf"), [0.0995, 0.0], rtol=1e-3)
    big = rng(5).standard_normal((7, 128)).astype(np.float32)
    for mode in ("max", "hf"):
        np.testing.assert_allclose(np.linalg.norm(l2_normalize(big, mode), axis=-1), 1.0, rtol=1e-5)
    assert not l2_normalize(np.zeros(4, np.float32), "max").any()


def test_gates_identities():
    hv = 3
    a_log = np.log(np.array([1.0, 2.0, 0.5], np.float32))
    dt_bias = np.zeros(hv, np.float32)
    a = np.array([[0.0, 25.0, -3.0]], np.float32)
    b = np.array([[0.0, 4.0, -4.0]], np.float32)
    g, beta = ol.gates(np.concatenate([a, b], axis=-1), a_log, dt_bias)
    assert g[0, 0] == pytest.approx(-np.log(2.0), rel=1e-6)          # softplus(0) = ln 2
    assert g[0, 1] == pytest.approx(-2.0 * 25.0, rel=1e-7)           # above the threshold: x
    assert g[0, 2] == pytest.approx(-0.5 * np.log1p(np.exp(-3.0)), rel=1e-6)
    assert beta[0, 0] == 0.5 and beta[0, 1] + beta[0, 2] == pytest.approx(1.0, abs=1e-7)
    x = rng(6).standard_normal((4, 2 * hv)).astype(np.float32) * 30
    g, beta = ol.gates(x, a_log, dt_bias)
    assert (g <= 0).all() and ((beta > 0) & (beta < 1) | (np.abs(x[:, hv:]) > 15)).all()


def test_epilogue_scale_invariance_and_unit_rms():
    r = rng(7)
    o = r.standard_normal((2, 5, 3, 16)).astype(np.float64)
    gate = r.standard_normal((2, 5, 48))
    o_norm = r.standard_normal(16)
    out = ol.layer_epilogue(o, gate, o_norm, eps=0.0)
    np.testing.assert_allclose(ol.layer_epilogue(7.5 * o, gate, o_norm, eps=0.0), out, rtol=1e-12)
    unit = ol.layer_epilogue(o, np.full_like(gate, 50.0), np.ones(16), eps=0.0) / 50.0  # silu(50) = 50
    rms = np.sqrt(np.mean(np.square(unit.reshape(2, 5, 3, 16)), axis=-1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-12)
    assert not ol.layer_epilogue(o, np.zeros_like(gate), o_norm).any()  # silu(0) = 0


def test_prologue_splits_and_normalises_per_head():
    r = rng(8)
    heads, dk, vheads, dv = 2, 8, 4, 8
    ch = 2 * heads * dk + vheads * dv
    qkv = r.standard_normal((1, 10, ch)).astype(np.float32)
    decay = r.standard_normal((1, 10, 2 * vheads)).astype(np.float32)
    tail = r.standard_normal((1, 3, ch)).astype(np.float32)
    w = r.standard_normal((ch, 4)).astype(np.float32)
    q, k, v, g, beta, new_tail = ol.layer_prologue(qkv, decay, tail, w, np.zeros(vheads, np.float32),
                                                   np.zeros(vheads, np.float32), heads, dk, vheads, dv)
    y, t2 = ol.short_convolution(qkv, tail, w)
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(q[0, 3, 1], y[0, 3, dk:2 * dk] / np.linalg.norm(y[0, 3, dk:2 * dk]), rtol=1e-5)
    np.testing.assert_allclose(k[0, 3, 0], y[0, 3, 2 * dk:3 * dk] / np.linalg.norm(y[0, 3, 2 * dk:3 * dk]),
                               rtol=1e-5)
    np.testing.assert_array_equal(v[0, 3, 2], y[0, 3, 2 * heads * dk + 2 * dv:2 * heads * dk + 3 * dv])
    np.testing.assert_array_equal(new_tail, t2)
    assert g.shape == beta.shape == (1, 10, vheads)
