"""CPU oracle for the layer-side work around the recurrence (numpy).

TEST INFRASTRUCTURE ONLY, like `oracle/gdn.py`: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it; the `pseudobrain_amd` package never does.

It restates, from `pseudobrain/gated_deltanet.py`:

* the short causal depthwise convolution with a carried tail, then SiLU
  (`short_convolution`, :314-338);
* the q/k L2 normalisation (`l2_normalize`, :59-70; restated in `gdn.py`);
* the decay and beta gates of the layer (:425-427):
  g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b);
* the layer prologue that feeds the operator (:415-429): split of the
  projection into [q | k | v | gate | a | b], convolution of q, k, v, the
  normalisation of q and k per key head, the gates;
* the epilogue (:439-441): per-head RMSNorm (eps 1e-5), times o_norm, times
  SiLU(gate).

Arithmetic is float32 (float64 when the inputs are float64). Inputs that are
bf16/fp16 in the real layer are float32 arrays holding representable values;
`x_dtype` names their type where the reference rounds through it (the tail is
cast to the input's dtype before the convolution, :333).

How each function is pinned (tests/test_oracle_layer.py): the convolution by
one-hot weights (a pure shift of the input), by a per-element loop written
independently, by the tail rules for short inputs and by segment invariance
(two calls with the carried tail equal one call); the normalisation by the
reference's own worked example ([1e-4, 0] -> [1, 0] 'max', [0.0995, 0] 'hf',
:62-64); the gates by softplus's threshold (x > 20 gives x), softplus(0) =
ln 2 and sigmoid's symmetry; the epilogue by scale invariance and unit RMS at
eps = 0 and by SiLU(0) = 0.
"""
from __future__ import annotations

import numpy as np

from oracle.gdn import _compute_dtype, l2_normalize, round_bf16, round_fp16

NORM_EPS = 1e-5          # gated_deltanet.py:72
SOFTPLUS_THRESHOLD = 20.0  # torch.nn.functional.softplus default (beta=1)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to 'bf16' / 'fp16' (float32 out), or leave 'fp32'/'fp64'."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "fp16":
        return round_fp16(x)
    return x


def sigmoid(x: np.ndarray) -> np.ndarray:
    """1 / (1 + exp(-x)) without overflow for large |x|."""
    e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1 / (1 + e), e / (1 + e)).astype(x.dtype)


def silu(x: np.ndarray) -> np.ndarray:
    """x sigmoid(x) (F.silu)."""
    return x * sigmoid(x)


def softplus(x: np.ndarray) -> np.ndarray:
    """log(1 + exp(x)), and x itself above the threshold 20 (F.softplus)."""
    return np.where(x > SOFTPLUS_THRESHOLD, x, np.log1p(np.exp(np.minimum(x, SOFTPLUS_THRESHOLD)))).astype(x.dtype)


def short_convolution(x, tail, weight, x_dtype: str = "fp32"):
    """Causal depthwise convolution over time with a carried tail, then SiLU
    (gated_deltanet.py:314-338).

    x [B,T,C]; tail [B,K-1,C] (the last K-1 inputs before x); weight [C,K]
    (weight[:, -1] multiplies the current input) or None (SiLU only). The tail
    is rounded to x's dtype before it joins x (:333). Returns (y [B,T,C],
    new tail [B,K-1,C] = the last K-1 inputs of tail ++ x)."""
    dtype = _compute_dtype(x)
    if weight is None:
        return silu(np.asarray(x, dtype=dtype)), tail
    size = weight.shape[1]
    length = x.shape[1]
    if size > 1:
        t = np.asarray(tail)
        t = round_to(t.astype(np.float32), x_dtype) if x_dtype in ("bf16", "fp16") else t
        extended = np.concatenate((t.astype(x.dtype), x), axis=1)
        new_tail = extended[:, extended.shape[1] - (size - 1):]
    else:
        extended, new_tail = x, tail
    extended = extended.astype(dtype)
    w = np.asarray(weight, dtype=dtype)
    y = extended[:, :length] * w[:, 0]
    for j in range(1, size):
        y = y + extended[:, j:j + length] * w[:, j]
    return silu(y), new_tail


def gates(decay, a_log, dt_bias):
    """g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) with a, b the
    two halves of the last axis of `decay` [B,T,2Hv] (gated_deltanet.py:425-427)."""
    dtype = np.float64 if np.asarray(decay).dtype == np.float64 else np.float32
    d = np.asarray(decay, dtype=dtype)
    a, b = np.split(d, 2, axis=-1)
    g = -np.exp(np.asarray(a_log, dtype=dtype)) * softplus(a + np.asarray(dt_bias, dtype=dtype))
    return g, sigmoid(b)


def layer_prologue(qkv, decay, tail, weight, a_log, dt_bias, heads: int, key_dim: int, value_heads: int,
                   value_dim: int, l2norm: str = "max", x_dtype: str = "fp32"):
    """The layer steps between the input projection and the operator
    (gated_deltanet.py:415-429), before the GQA repeat (which the kernels do by
    head index): qkv [B,T,2 H dk + Hv dv] and decay [B,T,2 Hv] are slices of
    the projection. Returns q, k [B,T,H,dk], v [B,T,Hv,dv], g, beta [B,T,Hv],
    new tail."""
    batch, length, _ = qkv.shape
    y, new_tail = short_convolution(qkv, tail, weight, x_dtype)
    qk = heads * key_dim
    q = l2_normalize(y[..., :qk].reshape(batch, length, heads, key_dim), l2norm)
    k = l2_normalize(y[..., qk:2 * qk].reshape(batch, length, heads, key_dim), l2norm)
    v = y[..., 2 * qk:].reshape(batch, length, value_heads, value_dim)
    g, beta = gates(decay, a_log, dt_bias)
    return q, k, v, g, beta, new_tail


def layer_epilogue(o, gate, o_norm, eps: float = NORM_EPS):
    """o * rsqrt(mean(o^2) + eps) per head, times o_norm, times SiLU(gate)
    (gated_deltanet.py:439-441). o [B,T,Hv,dv]; gate [B,T,Hv dv]; returns
    [B,T,Hv dv] in o's compute dtype."""
    o = np.asarray(o)
    dtype = _compute_dtype(o)
    o = o.astype(dtype)
    batch, length, heads, dv = o.shape
    o = o / np.sqrt(np.mean(np.square(o), axis=-1, keepdims=True) + dtype(eps))
    o = o * np.asarray(o_norm, dtype=dtype) * silu(np.asarray(gate, dtype=dtype).reshape(batch, length, heads, dv))
    return o.reshape(batch, length, heads * dv)
