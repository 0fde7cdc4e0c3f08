"""CPU oracle for the Gated DeltaNet recurrence (numpy).

TEST INFRASTRUCTURE ONLY. This module is the checker, never the product: only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import it. The `pseudobrain_amd` package never imports it and has no CPU path.

It restates the reference algorithms of `pseudobrain/gated_deltanet.py` from the
mathematics, in numpy:

    S_t = a_t S_{t-1} + k_t u_t^T,  u_t = b_t (v_t - a_t S_{t-1}^T k_t),
    o_t = S_t^T (q_t * scale),      a_t = exp(g_t)            (gated_deltanet.py:9-11)

with S stored [d_k, d_v] per head. Layouts follow the reference: q, k [B,T,H,K],
v [B,T,H,V], g, beta [B,T,H], h0 [B,H,K,V]; results (o [B,T,H,V], S_T [B,H,K,V]).
Arithmetic is float32, or float64 when the inputs are float64
(`_compute_dtype`, gated_deltanet.py:78-80). bf16 inputs are represented as
float32 arrays holding bf16-representable values (`round_bf16`).

How each function is pinned (tests/test_oracle.py): the sequential recurrence
by the closed form of one step written in the Householder form
a (I - b k k^T) S + b k v^T, by a scalar (K=1) recurrence solved in closed form,
by beta=0 pure decay, and by exact retrieval with orthonormal keys; the chunked
algorithm by equality with the sequential one for chunk sizes 1..128, padding
and segment invariance, and linearity in (V, S0). GQA, varlen and streaming by
their definitions (repeat_interleave, per-sequence calls, state carry). The
residuals gc and A (chunk_residuals) by scipy's unit lower-triangular solve of
I + a with a built by loops (decays as sums of g), by A (I + a) = I, by the
identity for orthogonal keys, by the two-token closed form and by gc against
per-chunk sums, and by mutants those pins catch.
"""
from __future__ import annotations

import numpy as np

CHUNK = 64            # gated_deltanet.py:49
L2_EPS = 1e-6         # gated_deltanet.py:56


def _compute_dtype(*arrays) -> np.dtype:
    """float64 when any input is float64, else float32 (gated_deltanet.py:78-80)."""
    return np.float64 if any(np.asarray(a).dtype == np.float64 for a in arrays) else np.float32


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32.

    Inf/NaN are not expected in the workloads and are not special-cased."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = (bits + (np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)
    return rounded.view(np.float32)


def round_fp16(x: np.ndarray) -> np.ndarray:
    """Round to IEEE half precision (numpy's float16 rounds to nearest even); float32 out."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def l2_normalize(x: np.ndarray, mode: str = "max", eps: float = L2_EPS) -> np.ndarray:
    """q/k normalisation over the last axis (gated_deltanet.py:59-70).

    'max': x / max(||x||, eps) (F.normalize); 'hf': x * rsqrt(sum x^2 + eps) in fp32."""
    if mode == "max":
        norm = np.sqrt(np.sum(np.square(x, dtype=np.float64), axis=-1, keepdims=True)).astype(x.dtype)
        return x / np.maximum(norm, np.asarray(eps, dtype=x.dtype))
    if mode == "hf":
        xf = x.astype(np.float32)
        return (xf / np.sqrt(np.sum(xf * xf, axis=-1, keepdims=True) + np.float32(eps))).astype(x.dtype)
    raise ValueError("l2 normalization mode must be one of ('max', 'hf')")


def repeat_heads(x: np.ndarray, heads: int, axis: int = 2) -> np.ndarray:
    """GQA: value head h reads query/key head h // (heads // Hk) (repeat_interleave,
    gated_deltanet.py:422-424)."""
    groups = heads // x.shape[axis]
    if groups * x.shape[axis] != heads:
        raise ValueError("value heads must be a multiple of the key heads")
    return np.repeat(x, groups, axis=axis) if groups > 1 else x


def _prepare(q, k, v, g, beta, h0):
    dtype = _compute_dtype(q, k, v, g, beta, h0)
    heads = v.shape[2]
    q = repeat_heads(np.asarray(q), heads).astype(dtype)
    k = repeat_heads(np.asarray(k), heads).astype(dtype)
    return dtype, q, k, np.asarray(v, dtype), np.asarray(g, dtype), np.asarray(beta, dtype), \
        np.asarray(h0, dtype)


def delta_rule_sequential(q, k, v, g, beta, scale, h0):
    """Per-step recurrence (gated_deltanet.py:93-107).

    Per token: S <- a S; u = b (v - S^T k); S <- S + k u^T; o = S^T (q scale)."""
    dtype, q, k, v, g, beta, state = _prepare(q, k, v, g, beta, h0)
    q = q * dtype(scale)
    decay = np.exp(g)
    rows = []
    for t in range(q.shape[1]):
        state = state * decay[:, t, :, None, None]
        kt = k[:, t]
        u = (v[:, t] - np.einsum("bhkv,bhk->bhv", state, kt)) * beta[:, t, :, None]
        state = state + kt[..., None] * u[..., None, :]
        rows.append(np.einsum("bhkv,bhk->bhv", state, q[:, t]))
    if not rows:
        return np.zeros(v.shape, dtype), state
    return np.stack(rows, 1), state


def unit_lower_inverse(a: np.ndarray) -> np.ndarray:
    """(I + a)^-1 for strictly lower-triangular a [..., C, C], by forward
    substitution row by row (the unitriangular solve of gated_deltanet.py:147-149)."""
    size = a.shape[-1]
    inv = np.zeros_like(a)
    for t in range(size):
        row = -np.einsum("...i,...ij->...j", a[..., t, :t], inv[..., :t, :])
        row[..., t] = 1.0
        inv[..., t, :] = row
    return inv


def chunk_residuals(k, g, beta, chunk: int = CHUNK):
    """The residuals gc and A of the reference's fla op (gated_deltanet.py:
    200-217, 64-token chunks), as delta_rule_chunked forms them
    (:141-149): gc = the inclusive cumsum of g within each chunk (:141), and
    A [B,T,H,chunk], row t of its chunk's T = (I + strict_lower(b_t (k_t.k_i)
    exp(gc_t - gc_i)))^-1 (:145-149). k [B,T,Hk,K] (repeated to the H value
    heads of g), g and beta [B,T,H]. A chunk shorter than `chunk` (the last)
    is padded with k = g = b = 0, which leaves its rows unchanged."""
    k = np.asarray(k)
    g = np.asarray(g)
    beta = np.asarray(beta)
    dtype = _compute_dtype(k, g, beta)
    batch, length, heads = g.shape
    k = repeat_heads(k.astype(dtype), heads)
    gc = np.empty((batch, length, heads), dtype)
    a_out = np.empty((batch, length, heads, chunk), dtype)
    strict = np.tril(np.ones((chunk, chunk), dtype=bool), -1)
    for t0 in range(0, length, chunk):
        n = min(chunk, length - t0)
        for b in range(batch):
            for h in range(heads):
                c = np.cumsum(g[b, t0:t0 + n, h].astype(dtype), dtype=dtype)
                kk = np.zeros((chunk, k.shape[-1]), dtype)
                kk[:n] = k[b, t0:t0 + n, h]
                cc = np.zeros(chunk, dtype)
                cc[:n] = c
                cc[n:] = c[-1] if n else 0
                bb = np.zeros(chunk, dtype)
                bb[:n] = beta[b, t0:t0 + n, h]
                decay = np.exp(np.where(strict, cc[:, None] - cc[None, :], -np.inf))
                a = np.where(strict, bb[:, None] * (kk @ kk.T) * decay, 0.0).astype(dtype)
                gc[b, t0:t0 + n, h] = c
                a_out[b, t0:t0 + n, h] = unit_lower_inverse(a)[:n]
    return gc, a_out


def _chunked_head(q, k, v, c, beta, state, scale, size):
    """One (batch, head) of delta_rule_chunked on chunk-shaped arrays:
    q, k [n,C,K], v [n,C,V], c (cumsum of g) and beta [n,C], state [K,V]."""
    dtype = q.dtype.type
    inclusive = np.tril(np.ones((size, size), dtype=bool))
    strict = np.tril(inclusive, -1)
    decay = np.exp(np.where(inclusive, c[:, :, None] - c[:, None, :], -np.inf)).astype(q.dtype)
    a = np.where(strict, beta[:, :, None] * (k @ np.swapaxes(k, -1, -2)) * decay, 0.0).astype(q.dtype)
    solve = unit_lower_inverse(a)
    gamma = np.exp(c)
    w = solve @ (k * (beta * gamma)[..., None])
    u0 = solve @ (v * beta[..., None])
    qs = q * dtype(scale)
    qk = (qs @ np.swapaxes(k, -1, -2)) * decay
    qg = qs * gamma[..., None]
    tail = np.exp(c[:, -1:] - c)[..., None] * k
    last = gamma[:, -1]
    out = np.empty(v.shape, q.dtype)
    for n in range(q.shape[0]):
        u = u0[n] - w[n] @ state
        out[n] = qg[n] @ state + qk[n] @ u
        state = state * last[n] + tail[n].T @ u
    return out, state


def delta_rule_chunked(q, k, v, g, beta, scale, h0, chunk: int | None = None):
    """Chunkwise WY algorithm (gated_deltanet.py:110-165).

    Pads T up to a multiple of C with k = v = g = beta = 0 (identity steps, :127,
    :134-136); C = min(chunk, T) (:125); in-chunk inclusive cumsum c of g (:141);
    D_ti = exp(c_t - c_i) for i <= t (:145); A = strict_lower(b_t (k_t.k_i) D_ti)
    (:146); T = (I + A)^-1 (:147-149); W = T (K * b exp(c)), U' = T (V * b) (:151-152);
    then chunk by chunk: U = U' - W S; O = (Q exp(c)) S + (Q K^T * D) U;
    S <- exp(c_C) S + (exp(c_C - c_i) k_i)^T U (:158-163). Heads are independent
    and are evaluated one at a time (the reference batches them)."""
    dtype, q, k, v, g, beta, h0 = _prepare(q, k, v, g, beta, h0)
    batch, length, heads, dk = q.shape
    dv = v.shape[-1]
    if length == 0:
        return np.zeros(v.shape, dtype), h0.copy()
    size = min(CHUNK if chunk is None else chunk, length)
    pad = (-length) % size
    count = (length + pad) // size
    out = np.empty((batch, heads, count * size, dv), dtype)
    final = np.empty_like(h0)

    def chunks(x, width):
        x = np.pad(x, ((0, pad),) + ((0, 0),) * (x.ndim - 1)) if pad else x
        return np.ascontiguousarray(x).reshape((count, size) + ((width,) if width else ()))

    for b in range(batch):
        for h in range(heads):
            qh, kh = chunks(q[b, :, h], dk), chunks(k[b, :, h], dk)
            vh = chunks(v[b, :, h], dv)
            c = np.cumsum(chunks(g[b, :, h], 0), axis=-1, dtype=dtype)
            bh = chunks(beta[b, :, h], 0)
            o, final[b, h] = _chunked_head(qh, kh, vh, c, bh, h0[b, h], scale, size)
            out[b, h] = o.reshape(count * size, dv)
    return out[:, :, :length].transpose(0, 2, 1, 3), final


KERNELS = {"sequential": delta_rule_sequential, "chunked": delta_rule_chunked}


def gated_delta_rule(q, k, v, g, beta, scale, h0, kernel: str = "chunked"):
    """Kernel dispatch of gated_deltanet.py:300-308 (CPU kernels only)."""
    if kernel not in KERNELS:
        raise ValueError(f"gated delta rule kernel must be one of {tuple(KERNELS)}")
    return KERNELS[kernel](q, k, v, g, beta, scale, h0)


def varlen(q, k, v, g, beta, scale, h0, cu_seqlens, kernel: str = "chunked"):
    """Packed sequences [1, sum T, ...] with boundaries cu_seqlens [N+1] and per-sequence
    initial states h0 [N,H,K,V]: one call per sequence with its own h0 (the reference
    has no cu_seqlens; a packed batch is a loop of independent calls).
    Returns (o [1, sum T, H, V], final states [N,H,K,V])."""
    cu = [int(x) for x in np.asarray(cu_seqlens)]
    outs, finals = [], []
    for n in range(len(cu) - 1):
        lo, hi = cu[n], cu[n + 1]
        o, s = gated_delta_rule(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], g[:, lo:hi],
                                beta[:, lo:hi], scale, h0[n:n + 1], kernel)
        outs.append(o)
        finals.append(s[0])
    return np.concatenate(outs, axis=1), np.stack(finals, 0)


def streamed(q, k, v, g, beta, scale, h0, segment: int, kernel: str = "chunked"):
    """One sequence processed as consecutive segments of `segment` tokens, the final
    state of each fed as the initial state of the next (transplant.py:1254-1271,
    scripts/eval/recall_eval.py:67-77). Yields (o_segment, state_after) per segment."""
    state = h0
    for lo in range(0, q.shape[1], segment):
        hi = min(lo + segment, q.shape[1])
        o, state = gated_delta_rule(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], g[:, lo:hi],
                                    beta[:, lo:hi], scale, state, kernel)
        yield o, state


def gated_delta_rule_backward(q, k, v, g, beta, scale, h0, do, dht):
    """Gradients of (o, S_T) = gated_delta_rule(q, k, v, g, beta, scale, h0)
    with respect to every input, given do [B,T,H,V] and dht [B,H,K,V]: what
    the reference's pseudobrain::gated_delta_chunk_backward op returns
    (gated_deltanet.py:230-277, fla's chunk backward; parity unpinned against
    fla itself, which is absent here). Reverse mode through the per-token
    recurrence (gated_deltanet.py:9-11, :93-107), states kept from a forward
    pass; q, k may be un-repeated [B,T,Hk,K], and their gradients are then
    summed over the value heads that read them.

    Per token, reversed, with P = a_t S_{t-1}, r = v_t - P^T k_t, u = b_t r:
        dS += q_t do_t^T scale          dq_t = S_t do_t scale
        dk_t = dS u,  du = dS^T k_t     db_t = du . r,  dr = b_t du,  dv_t = dr
        dP = dS - k_t dr^T              dk_t -= P dr
        dg_t = a_t <dP, S_{t-1}>        dS = a_t dP
    Returns (dq, dk, dv, dg, dbeta, dh0) in the compute dtype."""
    dtype, qr, kr, v, g, beta, state = _prepare(q, k, v, g, beta, h0)
    do = np.asarray(do, dtype)
    ds = np.asarray(dht, dtype).copy()
    length = v.shape[1]
    decay = np.exp(g)
    states = [state]
    for t in range(length):  # forward, keeping S_{t-1} for every t
        p = states[-1] * decay[:, t, :, None, None]
        r = v[:, t] - np.einsum("bhkv,bhk->bhv", p, kr[:, t])
        states.append(p + kr[:, t, :, :, None] * (r * beta[:, t, :, None])[:, :, None, :])
    dq, dk, dv = np.zeros_like(qr), np.zeros_like(kr), np.zeros_like(v)
    dg, db = np.zeros_like(g), np.zeros_like(beta)
    sc = dtype(scale)
    for t in reversed(range(length)):
        prev, cur = states[t], states[t + 1]
        kt, qt, a, b = kr[:, t], qr[:, t], decay[:, t, :, None, None], beta[:, t, :, None]
        ds = ds + sc * qt[..., None] * do[:, t, :, None, :]
        dq[:, t] = sc * np.einsum("bhkv,bhv->bhk", cur, do[:, t])
        p = prev * a
        r = v[:, t] - np.einsum("bhkv,bhk->bhv", p, kt)
        u = b * r
        dk[:, t] = np.einsum("bhkv,bhv->bhk", ds, u)
        du = np.einsum("bhkv,bhk->bhv", ds, kt)
        db[:, t] = np.sum(du * r, axis=-1)
        dr = b * du
        dv[:, t] = dr
        dp = ds - kt[..., None] * dr[:, :, None, :]
        dk[:, t] -= np.einsum("bhkv,bhv->bhk", p, dr)
        dg[:, t] = decay[:, t] * np.sum(dp * prev, axis=(-2, -1))
        ds = dp * a
    heads_k = np.asarray(q).shape[2]
    if heads_k != v.shape[2]:  # GQA: sum over the value heads of each key head
        groups = v.shape[2] // heads_k
        dq = dq.reshape(*dq.shape[:2], heads_k, groups, dq.shape[-1]).sum(3)
        dk = dk.reshape(*dk.shape[:2], heads_k, groups, dk.shape[-1]).sum(3)
    return dq, dk, dv, dg, db, ds


def rel_inf_error(x, ref) -> float:
    """Infinity-norm relative error max|x - ref| / max|ref| (the tolerance measure)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(x - ref))) if ref.size else 0.0
    return err / denom if denom > 0 else err
