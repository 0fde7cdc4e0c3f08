"""Pins of the CPU oracle (oracle/gdn.py) against what the mathematics fixes.

The reference ships no tests, fixtures or golden vectors for this path, so the
oracle is pinned by closed forms, special cases and invariants written
independently of its code, plus mutation checks showing that plausible
mistakes planted in the oracle fail those pins.
"""
import inspect

import numpy as np
import pytest

from oracle import gdn

RNG = np.random.default_rng(1234)


def rand_inputs(batch, length, heads, dk, dv, *, hk=None, rng=RNG, unit=True, h0_std=0.3,
                dtype=np.float64, g_scale=1.0):
    hk = heads if hk is None else hk
    q = rng.standard_normal((batch, length, hk, dk))
    k = rng.standard_normal((batch, length, hk, dk))
    if unit:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((batch, length, heads, dv))
    beta = 1 / (1 + np.exp(-rng.standard_normal((batch, length, heads))))
    g = -np.log1p(np.exp(rng.standard_normal((batch, length, heads)))) * g_scale
    h0 = rng.standard_normal((batch, heads, dk, dv)) * h0_std
    return tuple(x.astype(dtype) for x in (q, k, v, g, beta, h0))


def close(a, b, tol):
    return gdn.rel_inf_error(a, b) < tol


# ---------------------------------------------------------------------------
# Sequential recurrence (gated_deltanet.py:93-107)
# ---------------------------------------------------------------------------
def householder_step(q, k, v, g, beta, scale, s0):
    """One step in the Householder form of the module docstring
    (gated_deltanet.py:12): S1 = a (I - b k k^T) S0 + b k v^T, o = S1^T q scale.
    Shapes for one head: q, k [K], v [V], s0 [K,V]."""
    a = np.exp(g)
    eye = np.eye(k.shape[0])
    s1 = a * (eye - beta * np.outer(k, k)) @ s0 + beta * np.outer(k, v)
    return s1.T @ q * scale, s1


@pytest.mark.parametrize("unit", [True, False])
def test_sequential_one_step_closed_form(unit):
    q, k, v, g, beta, h0 = rand_inputs(2, 1, 3, 8, 5, unit=unit)
    o, s = gdn.delta_rule_sequential(q, k, v, g, beta, 0.7, h0)
    for b in range(2):
        for h in range(3):
            o_ref, s_ref = householder_step(q[b, 0, h], k[b, 0, h], v[b, 0, h], g[b, 0, h],
                                            beta[b, 0, h], 0.7, h0[b, h])
            np.testing.assert_allclose(o[b, 0, h], o_ref, rtol=1e-12, atol=1e-12)
            np.testing.assert_allclose(s[b, h], s_ref, rtol=1e-12, atol=1e-12)


def test_sequential_many_steps_householder_product():
    """T steps = the product of T Householder steps (one head, K=6, V=4)."""
    q, k, v, g, beta, h0 = rand_inputs(1, 9, 1, 6, 4)
    o, s = gdn.delta_rule_sequential(q, k, v, g, beta, 0.5, h0)
    state = h0[0, 0]
    for t in range(9):
        o_t, state = householder_step(q[0, t, 0], k[0, t, 0], v[0, t, 0], g[0, t, 0],
                                      beta[0, t, 0], 0.5, state)
        np.testing.assert_allclose(o[0, t, 0], o_t, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s[0, 0], state, rtol=1e-12, atol=1e-12)


def test_scalar_recurrence_closed_form():
    """K = V = 1: S_t = m_t S_{t-1} + b_t k_t v_t with m_t = a_t (1 - b_t k_t^2), so
    S_t = (prod_{s<=t} m_s) S_0 + sum_{j<=t} (prod_{j<s<=t} m_s) b_j k_j v_j."""
    rng = np.random.default_rng(7)
    length = 12
    q, k, v, g, beta, h0 = rand_inputs(1, length, 1, 1, 1, unit=False, rng=rng)
    o, s = gdn.delta_rule_sequential(q, k, v, g, beta, 1.3, h0)
    a = np.exp(g[0, :, 0])
    kk, vv, bb, qq = k[0, :, 0, 0], v[0, :, 0, 0], beta[0, :, 0], q[0, :, 0, 0]
    m = a * (1 - bb * kk * kk)
    for t in range(length):
        state = np.prod(m[: t + 1]) * h0[0, 0, 0, 0]
        for j in range(t + 1):
            state += np.prod(m[j + 1: t + 1]) * bb[j] * kk[j] * vv[j]
        assert abs(o[0, t, 0, 0] - state * qq[t] * 1.3) < 1e-12
    assert abs(s[0, 0, 0, 0] - state) < 1e-12


@pytest.mark.parametrize("kernel", ["sequential", "chunked"])
def test_beta_zero_is_pure_decay(kernel):
    """beta = 0: S_t = exp(c_t) S_0 and o_t = exp(c_t) S_0^T q_t scale, c = cumsum g."""
    q, k, v, g, beta, h0 = rand_inputs(1, 70, 2, 8, 8)
    beta[:] = 0
    o, s = gdn.gated_delta_rule(q, k, v, g, beta, 0.9, h0, kernel)
    c = np.cumsum(g, axis=1)
    o_ref = np.exp(c)[..., None] * np.einsum("bhkv,bthk->bthv", h0, q) * 0.9
    np.testing.assert_allclose(o, o_ref, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(s, np.exp(c[:, -1])[..., None, None] * h0, rtol=1e-10, atol=1e-14)


@pytest.mark.parametrize("kernel", ["sequential", "chunked"])
def test_orthonormal_keys_retrieve_exactly(kernel):
    """g = 0, beta = 1, S_0 = 0, orthonormal keys: S_T^T k_j = v_j (the delta rule
    writes exactly), and a query equal to an earlier key reads its value."""
    rng = np.random.default_rng(3)
    dk, dv, length = 16, 5, 10
    basis, _ = np.linalg.qr(rng.standard_normal((dk, dk)))
    k = basis[:length][None, :, None, :]
    q = k.copy()
    v = rng.standard_normal((1, length, 1, dv))
    g = np.zeros((1, length, 1))
    beta = np.ones((1, length, 1))
    h0 = np.zeros((1, 1, dk, dv))
    o, s = gdn.gated_delta_rule(q, k, v, g, beta, 1.0, h0, kernel)
    np.testing.assert_allclose(s[0, 0].T @ k[0, :, 0].T, v[0, :, 0].T, atol=1e-12)
    np.testing.assert_allclose(o[0, :, 0], v[0, :, 0], atol=1e-12)


def test_rewriting_a_key_replaces_its_value():
    """beta = 1, unit key written twice: the second value replaces the first."""
    dk = 4
    key = np.zeros(dk)
    key[1] = 1.0
    k = np.stack([key, key])[None, :, None, :]
    v = np.array([[1.0, 2.0], [5.0, -3.0]])[None, :, None, :]
    g = np.zeros((1, 2, 1))
    beta = np.ones((1, 2, 1))
    o, s = gdn.delta_rule_sequential(k, k, v, g, beta, 1.0, np.zeros((1, 1, dk, 2)))
    np.testing.assert_allclose(s[0, 0].T @ key, [5.0, -3.0], atol=1e-14)


# ---------------------------------------------------------------------------
# Chunked algorithm (gated_deltanet.py:110-165)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("chunk", [1, 16, 32, 64, 128])
@pytest.mark.parametrize("length", [1, 5, 63, 64, 65, 200])
def test_chunked_equals_sequential(chunk, length):
    q, k, v, g, beta, h0 = rand_inputs(2, length, 2, 16, 8)
    o1, s1 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.25, h0, chunk=chunk)
    o2, s2 = gdn.delta_rule_sequential(q, k, v, g, beta, 0.25, h0)
    assert close(o1, o2, 1e-10) and close(s1, s2, 1e-10)


def test_wide_heads_chunked_equals_sequential_and_zero_padding_is_exact():
    """At 256-wide keys the chunked algorithm still equals the recurrence, and
    zero-padding the head widths (K 200 -> 256 in q, k, h0; V 80 -> 96 in v,
    h0, as the device path pads them) leaves the original block of o and of
    the final state unchanged and the padded parts zero."""
    q, k, v, g, beta, h0 = rand_inputs(1, 130, 2, 256, 64)
    o1, s1 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.0625, h0)
    o2, s2 = gdn.delta_rule_sequential(q, k, v, g, beta, 0.0625, h0)
    assert close(o1, o2, 1e-10) and close(s1, s2, 1e-10)
    q, k, v, g, beta, h0 = rand_inputs(1, 100, 2, 200, 80)
    o, s = gdn.delta_rule_chunked(q, k, v, g, beta, 0.07, h0)
    pk = ((0, 0), (0, 0), (0, 0), (0, 56))
    hp = np.pad(h0, ((0, 0), (0, 0), (0, 56), (0, 16)))
    op, sp = gdn.delta_rule_chunked(np.pad(q, pk), np.pad(k, pk), np.pad(v, ((0, 0), (0, 0), (0, 0), (0, 16))),
                                    g, beta, 0.07, hp)
    assert close(op[..., :80], o, 1e-12) and close(sp[..., :200, :80], s, 1e-12)
    assert not op[..., 80:].any() and not sp[..., 200:, :].any() and not sp[..., :, 80:].any()


def test_chunked_low_decay_long_range():
    """Slow decay (g scaled by 0.01): the initial state stays visible for hundreds
    of steps; chunked still equals sequential."""
    q, k, v, g, beta, h0 = rand_inputs(1, 300, 2, 16, 16, g_scale=0.01)
    o1, s1 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.25, h0)
    o2, s2 = gdn.delta_rule_sequential(q, k, v, g, beta, 0.25, h0)
    assert close(o1, o2, 1e-10) and close(s1, s2, 1e-10)
    assert np.abs(np.exp(np.cumsum(g, 1))[0, -1]).min() > 1e-2  # the carry is not negligible


def test_segment_invariance():
    """Any split of T with the state carried equals one pass (gated_deltanet.py:26)."""
    q, k, v, g, beta, h0 = rand_inputs(1, 250, 2, 16, 8)
    o_full, s_full = gdn.delta_rule_chunked(q, k, v, g, beta, 0.3, h0)
    outs, state = [], h0
    for lo, hi in ((0, 37), (37, 101), (101, 250)):
        o, state = gdn.delta_rule_chunked(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], g[:, lo:hi],
                                          beta[:, lo:hi], 0.3, state)
        outs.append(o)
    assert close(np.concatenate(outs, 1), o_full, 1e-11) and close(state, s_full, 1e-11)
    streamed = list(gdn.streamed(q, k, v, g, beta, 0.3, h0, 64))
    assert close(np.concatenate([o for o, _ in streamed], 1), o_full, 1e-11)
    assert close(streamed[-1][1], s_full, 1e-11)


def test_linearity_in_values_and_state():
    """For fixed q, k, g, beta the map (V, S_0) -> (O, S_T) is linear."""
    q, k, v1, g, beta, h1 = rand_inputs(1, 90, 2, 8, 8)
    v2 = RNG.standard_normal(v1.shape)
    h2 = RNG.standard_normal(h1.shape)
    oa, sa = gdn.delta_rule_chunked(q, k, v1, g, beta, 0.5, h1)
    ob, sb = gdn.delta_rule_chunked(q, k, v2, g, beta, 0.5, h2)
    oc, sc = gdn.delta_rule_chunked(q, k, 2 * v1 - 3 * v2, g, beta, 0.5, 2 * h1 - 3 * h2)
    assert close(oc, 2 * oa - 3 * ob, 1e-11) and close(sc, 2 * sa - 3 * sb, 1e-11)


def test_gqa_equals_repeat_interleave():
    q, k, v, g, beta, h0 = rand_inputs(1, 40, 4, 8, 8, hk=2)
    o1, s1 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.5, h0)
    rq, rk = np.repeat(q, 2, axis=2), np.repeat(k, 2, axis=2)
    o2, s2 = gdn.delta_rule_sequential(rq, rk, v, g, beta, 0.5, h0)
    assert close(o1, o2, 1e-11) and close(s1, s2, 1e-11)
    # head 1 reads key head 0, head 2 reads key head 1 (not head 1 -> 1)
    o3, _ = gdn.delta_rule_sequential(rq[:, :, 1:2], rk[:, :, 1:2], v[:, :, 1:2], g[:, :, 1:2],
                                      beta[:, :, 1:2], 0.5, h0[:, 1:2])
    o4, _ = gdn.delta_rule_sequential(q[:, :, 0:1], k[:, :, 0:1], v[:, :, 1:2], g[:, :, 1:2],
                                      beta[:, :, 1:2], 0.5, h0[:, 1:2])
    assert close(o3, o4, 1e-13)


def test_varlen_is_a_loop_of_calls():
    q, k, v, g, beta, _ = rand_inputs(1, 150, 2, 8, 8)
    h0 = RNG.standard_normal((4, 2, 8, 8))
    cu = np.array([0, 40, 40, 107, 150])  # includes an empty sequence
    o, finals = gdn.varlen(q, k, v, g, beta, 0.5, h0, cu)
    for n in range(4):
        lo, hi = cu[n], cu[n + 1]
        o_n, s_n = gdn.delta_rule_sequential(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], g[:, lo:hi],
                                             beta[:, lo:hi], 0.5, h0[n:n + 1])
        assert close(o[:, lo:hi], o_n, 1e-11) if hi > lo else True
        assert close(finals[n], s_n[0], 1e-11)
    np.testing.assert_array_equal(finals[1], h0[1])  # the empty sequence keeps its state


def test_fp32_oracle_tracks_fp64():
    q, k, v, g, beta, h0 = rand_inputs(1, 300, 2, 64, 64)
    o64, s64 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.125, h0)
    o32, s32 = gdn.delta_rule_chunked(*(x.astype(np.float32) for x in (q, k, v, g, beta)), 0.125,
                                      h0.astype(np.float32))
    assert o32.dtype == np.float32
    assert close(o32, o64, 1e-5) and close(s32, s64, 1e-5)


def test_unknown_kernel_raises():
    q, k, v, g, beta, h0 = rand_inputs(1, 4, 1, 4, 4)
    with pytest.raises(ValueError):
        gdn.gated_delta_rule(q, k, v, g, beta, 1.0, h0, "fla")


# ---------------------------------------------------------------------------
# l2 normalisation (gated_deltanet.py:59-70): the reference docstring's
# known answers, [1e-4, 0] -> [1, 0] ('max') vs [0.0995, 0] ('hf').
# ---------------------------------------------------------------------------
def test_l2_normalize_known_answers():
    x = np.array([[1e-4, 0.0]], dtype=np.float32)
    np.testing.assert_allclose(gdn.l2_normalize(x, "max"), [[1.0, 0.0]], rtol=1e-6)
    np.testing.assert_allclose(gdn.l2_normalize(x, "hf"), [[0.0995, 0.0]], rtol=1e-3)
    y = RNG.standard_normal((5, 7)).astype(np.float32)
    np.testing.assert_allclose(np.linalg.norm(gdn.l2_normalize(y), axis=-1), 1.0, rtol=1e-6)
    with pytest.raises(ValueError):
        gdn.l2_normalize(y, "l1")


def test_round_bf16_and_fp16():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 1e-30], dtype=np.float32)
    # ties to even at bf16's 2^-7 spacing
    np.testing.assert_array_equal(gdn.round_bf16(x)[:3], [1.0, 1.0, 1.0 + 2 ** -6])
    assert gdn.round_bf16(x)[3] == -2.5
    np.testing.assert_array_equal(gdn.round_fp16(np.array([1 + 2 ** -12], np.float32)), [1.0])


# ---------------------------------------------------------------------------
# Mutation checks: a plausible mistake planted in the oracle fails a pin above.
# ---------------------------------------------------------------------------
def _mutant(fn, old, new):
    src = inspect.getsource(fn)
    assert old in src, old
    namespace = dict(vars(gdn))
    exec(compile(src.replace(old, new), gdn.__file__, "exec"), namespace)  # noqa: S102
    return namespace[fn.__name__]


SEQUENTIAL_MUTANTS = [
    ("state = state * decay[:, t, :, None, None]", "state = state"),                      # dropped decay
    ("(v[:, t] - np.einsum", "(v[:, t] + np.einsum"),                                      # wrong sign
    ('np.einsum("bhkv,bhk->bhv", state, kt)', 'np.einsum("bhvk,bhk->bhv", state, kt)'),  # transposed S
    ("state = state + kt[..., None] * u[..., None, :]", "state = state + kt[..., None] * u[..., None, :] * 0.999"),
]


@pytest.mark.parametrize("old,new", SEQUENTIAL_MUTANTS)
def test_sequential_pins_catch_mutants(old, new, monkeypatch):
    bad = _mutant(gdn.delta_rule_sequential, old, new)
    q, k, v, g, beta, h0 = rand_inputs(1, 1, 1, 6, 6)
    o, s = bad(q, k, v, g, beta, 0.7, h0)
    o_ref, s_ref = householder_step(q[0, 0, 0], k[0, 0, 0], v[0, 0, 0], g[0, 0, 0], beta[0, 0, 0],
                                    0.7, h0[0, 0])
    assert not (close(o[0, 0, 0], o_ref, 1e-9) and close(s[0, 0], s_ref, 1e-9))


CHUNKED_MUTANTS = [
    ("inclusive = np.tril(np.ones((size, size), dtype=bool))",
     "inclusive = np.tril(np.ones((size, size), dtype=bool), -1)"),          # exclusive decay mask
    ("c[:, :, None] - c[:, None, :]", "c[:, None, :] - c[:, :, None]"),     # decay exponent sign
    ("w = solve @ (k * (beta * gamma)[..., None])", "w = solve @ (k * beta[..., None])"),  # dropped gamma
    ("state = state * last[n] + tail[n].T @ u", "state = state + tail[n].T @ u"),          # no carry decay
    ("tail = np.exp(c[:, -1:] - c)[..., None] * k", "tail = k"),                            # no tail decay
    ("u = u0[n] - w[n] @ state", "u = u0[n] - w[n] @ state.T"),                             # transposed S
]


@pytest.mark.parametrize("old,new", CHUNKED_MUTANTS)
def test_chunked_pins_catch_mutants(old, new, monkeypatch):
    bad_head = _mutant(gdn._chunked_head, old, new)
    monkeypatch.setattr(gdn, "_chunked_head", bad_head)
    q, k, v, g, beta, h0 = rand_inputs(1, 100, 1, 8, 8)
    o1, s1 = gdn.delta_rule_chunked(q, k, v, g, beta, 0.5, h0)
    o2, s2 = gdn.delta_rule_sequential(q, k, v, g, beta, 0.5, h0)
    assert not (close(o1, o2, 1e-6) and close(s1, s2, 1e-6))


# ---------------------------------------------------------------------------
# Backward (gated_deltanet.py:230-277): gradients of <do, o> + <dht, S_T>
# ---------------------------------------------------------------------------
def numeric_gradients(inputs, scale, do, dht, eps=1e-6):
    """Central differences of L = <do, o> + <dht, S_T> (float64, sequential
    kernel) with respect to every element of every input."""
    def loss(args):
        o, s = gdn.delta_rule_sequential(*args[:5], scale, args[5])
        return float(np.sum(o * do) + np.sum(s * dht))
    grads = []
    for i in range(6):
        grad = np.zeros_like(inputs[i])
        for idx in np.ndindex(inputs[i].shape):
            args = [x.copy() for x in inputs]
            args[i][idx] += eps
            up = loss(args)
            args[i][idx] -= 2 * eps
            grad[idx] = (up - loss(args)) / (2 * eps)
        grads.append(grad)
    return grads


def fd_case(seed=7):
    rng = np.random.default_rng(seed)
    q, k, v, g, beta, h0 = rand_inputs(1, 6, 2, 3, 2, hk=1, rng=rng, unit=False)
    do = rng.standard_normal(v.shape)
    dht = rng.standard_normal(h0.shape)
    return (q, k, v, g, beta, h0), do, dht


def test_backward_matches_finite_differences():
    """Every gradient (GQA: q, k summed over their two value heads) equals
    central differences of the loss through the sequential recurrence."""
    inputs, do, dht = fd_case()
    got = gdn.gated_delta_rule_backward(*inputs[:5], 0.8, inputs[5], do, dht)
    want = numeric_gradients(list(inputs), 0.8, do, dht)
    names = ("dq", "dk", "dv", "dg", "dbeta", "dh0")
    for name, a, b in zip(names, got, want):
        assert a.shape == b.shape, name
        assert close(a, b, 1e-7), f"{name}: {gdn.rel_inf_error(a, b):.2e}"


def test_backward_of_the_chunked_kernel_is_the_same():
    """The chunked kernel computes the same function, so central differences
    through it give the same gradients (a second route to the same numbers)."""
    inputs, do, dht = fd_case(8)
    q, k, v, g, beta, h0 = inputs
    eps = 1e-6
    got = gdn.gated_delta_rule_backward(q, k, v, g, beta, 0.6, h0, do, dht)

    def loss(gv):
        o, s = gdn.delta_rule_chunked(q, k, v, gv, beta, 0.6, h0, chunk=4)
        return float(np.sum(o * do) + np.sum(s * dht))
    dg = np.zeros_like(g)
    for idx in np.ndindex(g.shape):
        up, down = g.copy(), g.copy()
        up[idx] += eps
        down[idx] -= eps
        dg[idx] = (loss(up) - loss(down)) / (2 * eps)
    assert close(got[3], dg, 1e-7)


BACKWARD_MUTANTS = [
    ("ds = dp * a", "ds = dp"),                                                        # dropped decay of the adjoint
    ("dk[:, t] -= np.einsum", "dk[:, t] += np.einsum"),                                # wrong sign
    ("dg[:, t] = decay[:, t] * np.sum(dp * prev", "dg[:, t] = decay[:, t] * np.sum(ds * prev"),  # dS for dP
    ("db[:, t] = np.sum(du * r, axis=-1)", "db[:, t] = np.sum(du * u, axis=-1)"),      # u for r
    ("dq[:, t] = sc * np.einsum(\"bhkv,bhv->bhk\", cur,", "dq[:, t] = sc * np.einsum(\"bhkv,bhv->bhk\", prev,"),
]


@pytest.mark.parametrize("old,new", BACKWARD_MUTANTS)
def test_backward_pins_catch_mutants(old, new):
    bad = _mutant(gdn.gated_delta_rule_backward, old, new)
    inputs, do, dht = fd_case()
    got = bad(*inputs[:5], 0.8, inputs[5], do, dht)
    want = numeric_gradients(list(inputs), 0.8, do, dht)
    assert not all(close(a, b, 1e-7) for a, b in zip(got, want))


# ---------------------------------------------------------------------------
# fla's residuals of the chunk forward (gated_deltanet.py:200-217, :141-149)
# ---------------------------------------------------------------------------
def brute_a(k, g, beta, t0, n):
    """strict_lower(b_t (k_t.k_s) exp(g_{s+1} + ... + g_t)) of the chunk at t0
    (n tokens) of one head, by loops: the decay as the sum of the decays
    between the two tokens, not a difference of cumulative sums."""
    a = np.zeros((n, n))
    for t in range(n):
        for s in range(t):
            a[t, s] = beta[t0 + t] * (k[t0 + t] @ k[t0 + s]) * np.exp(np.sum(g[t0 + s + 1:t0 + t + 1]))
    return a


def test_residuals_invert_i_plus_a():
    """Each chunk's rows of A are the inverse of I + a (a built by loops), as
    scipy's unit lower-triangular solve gives it; GQA 1 -> 2, a short last chunk."""
    from scipy.linalg import solve_triangular
    _, k, _, g, beta, _ = rand_inputs(1, 150, 2, 16, 4, hk=1)
    gc, a = gdn.chunk_residuals(k, g, beta)
    assert a.shape == (1, 150, 2, 64) and gc.shape == (1, 150, 2)
    for h in range(2):
        for t0 in (0, 64, 128):
            n = min(64, 150 - t0)
            m = np.eye(n) + brute_a(k[0, :, 0], g[0, :, h], beta[0, :, h], t0, n)
            inv = solve_triangular(m, np.eye(n), lower=True, unit_diagonal=True)
            rows = a[0, t0:t0 + n, h]
            assert close(rows[:, :n], inv, 1e-12)
            assert np.all(rows[:, n:] == 0)
            assert close(rows[:, :n] @ m, np.eye(n), 1e-12)


def test_residuals_gc_restarts_at_each_chunk():
    _, k, _, g, beta, _ = rand_inputs(2, 200, 1, 4, 4)
    gc, _ = gdn.chunk_residuals(k, g, beta)
    for b in range(2):
        for t in range(200):
            assert abs(gc[b, t, 0] - np.sum(g[b, 64 * (t // 64):t + 1, 0])) < 1e-12


def test_residuals_orthogonal_keys_give_the_identity():
    """Keys orthogonal within each chunk: a = 0, so every chunk's T is I."""
    rng = np.random.default_rng(5)
    basis = np.linalg.qr(rng.standard_normal((64, 64)))[0]
    k = np.concatenate([basis, basis[:36]])[None, :, None, :]
    g = -rng.random((1, 100, 1))
    beta = rng.random((1, 100, 1))
    _, a = gdn.chunk_residuals(k, g, beta)
    for t in range(100):
        expect = np.zeros(64)
        expect[t % 64] = 1.0
        assert np.allclose(a[0, t, 0], expect, atol=1e-12)


def test_residuals_two_tokens_closed_form():
    """T = 2: T = [[1, 0], [-b_1 (k_1.k_0) e^{g_1}, 1]]."""
    _, k, _, g, beta, _ = rand_inputs(1, 2, 1, 5, 5)
    gc, a = gdn.chunk_residuals(k, g, beta)
    assert np.allclose(gc[0, :, 0], [g[0, 0, 0], g[0, 0, 0] + g[0, 1, 0]], atol=1e-15)
    assert np.allclose(a[0, 0, 0, :2], [1.0, 0.0]) and np.allclose(a[0, 1, 0, 1], 1.0)
    assert np.isclose(a[0, 1, 0, 0], -beta[0, 1, 0] * (k[0, 1, 0] @ k[0, 0, 0]) * np.exp(g[0, 1, 0]))


RESIDUAL_MUTANTS = [
    ("cc[:, None] - cc[None, :]", "cc[None, :] - cc[:, None]"),           # decay exponent sign
    ("bb[:, None] * (kk @ kk.T)", "bb[None, :] * (kk @ kk.T)"),           # beta of the column
    ("unit_lower_inverse(a)[:n]", "unit_lower_inverse(-a)[:n]"),          # (I - a)^-1
    ("np.cumsum(g[b, t0:t0 + n, h].astype(dtype), dtype=dtype)",
     "np.cumsum(g[b, t0:t0 + n, h].astype(dtype), dtype=dtype) + g[b, :t0, h].sum()"),  # no restart
]


@pytest.mark.parametrize("old,new", RESIDUAL_MUTANTS)
def test_residual_pins_catch_mutants(old, new):
    bad = _mutant(gdn.chunk_residuals, old, new)
    _, k, _, g, beta, _ = rand_inputs(1, 100, 1, 8, 4)
    gc, a = bad(k, g, beta)
    rows_ok = all(close(a[0, t0:t0 + n, 0, :n] @ (np.eye(n) + brute_a(k[0, :, 0], g[0, :, 0], beta[0, :, 0], t0, n)),
                        np.eye(n), 1e-9) for t0, n in ((0, 64), (64, 36)))
    gc_ok = all(abs(gc[0, t, 0] - np.sum(g[0, 64 * (t // 64):t + 1, 0])) < 1e-9 for t in range(100))
    assert not (rows_ok and gc_ok)
