"""Parity of the chunk backward (pbgdn_chunk_bwd, the gradients of
pseudobrain::gated_delta_chunk_backward, gated_deltanet.py:230-277) with the
oracle's reverse mode through the per-token recurrence
(oracle/gdn.py: gated_delta_rule_backward, itself pinned by central
differences in tests/test_oracle.py), on the same input values.

Tolerances (infinity-norm relative error against the float64 oracle): 2e-4 for
everything computed and returned in float32 (dg, a float32 dbeta, dh0, and all
gradients of float32 inputs: the kernels run float32 sums of up to 128 terms
through every chunk); 1e-2 for gradients returned in bf16 or fp16 (their rounding)."""
import numpy as np
import pytest
import torch

from oracle import gdn
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import generate, to_numpy
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32_TOL = 2e-4
BF16_TOL = 1e-2
NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")


def make(batch, length, hk, hv, dk, dv, dtype, seed, h0=True, dht=True):
    q, k, v, g, beta, state = generate(batch, length, hk, hv, dk, dv, dtype, 0.05, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    do = (torch.randn(batch, length, hv, dv, generator=gen) * 0.1).to(dtype)
    dht_ = torch.randn(batch, hv, dk, dv, generator=gen) * 0.1 if dht else None
    return q, k, v, g, beta, state if h0 else None, do, dht_


def oracle_grads(q, k, v, g, beta, scale, h0, do, dht):
    f64 = [to_numpy(x.double()) for x in (q, k, v, g, beta, do)]
    shape = (q.shape[0], v.shape[2], q.shape[3], v.shape[3])
    h = np.zeros(shape) if h0 is None else to_numpy(h0.double())
    d = np.zeros(shape) if dht is None else to_numpy(dht.double())
    return gdn.gated_delta_rule_backward(*f64[:5], scale, h, f64[5], d)


def check(name, got, ref, dtypes):
    errs = {n: rel_err(x, r) for n, x, r in zip(NAMES, got, ref)}
    print(f"[{name}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, x in zip(NAMES, got):
        tol = BF16_TOL if x.dtype in (torch.bfloat16, torch.float16) else F32_TOL
        assert errs[n] <= tol, f"{name}: {n} error {errs[n]:.3e} > {tol}"
        assert x.dtype == dtypes[n], f"{name}: {n} is {x.dtype}"


@pytest.mark.parametrize("batch,length,hk,hv,dk,dv,dtype", [
    (2, 150, 2, 2, 64, 64, torch.float32),       # three chunks, the last one padded
    (1, 64, 1, 1, 128, 128, torch.float32),      # exactly one chunk
    (1, 333, 1, 4, 128, 64, torch.bfloat16),     # GQA 1 -> 4, bf16 inputs
    (2, 200, 2, 4, 64, 128, torch.bfloat16),
    (1, 1000, 2, 2, 128, 128, torch.float32),    # 16 chunks
    (1, 260, 2, 2, 128, 128, torch.float16),     # fp16 inputs
])
def test_backward_matches_the_oracle(batch, length, hk, hv, dk, dv, dtype):
    name = f"bwd B={batch} T={length} {hk}->{hv} K={dk} V={dv} {dtype}"
    print(f"[{name}]", flush=True)
    q, k, v, g, beta, h0, do, dht = make(batch, length, hk, hv, dk, dv, dtype, seed=length + dk)
    scale = dk ** -0.5
    got = gd.chunk_bwd(*[x.to(DEV) for x in (q, k, v, g, beta)], scale, h0.to(DEV), do.to(DEV), dht.to(DEV))
    torch.cuda.synchronize()
    ref = oracle_grads(q, k, v, g, beta, scale, h0, do, dht)
    check(name, got, ref, dict(dq=dtype, dk=dtype, dv=dtype, dg=torch.float32, dbeta=torch.float32,
                               dh0=torch.float32))


def test_backward_without_initial_state_or_final_gradient():
    """h0 and dht absent (zeros), a bf16 beta (its gradient comes back bf16)."""
    q, k, v, g, beta, _, do, _ = make(1, 130, 2, 2, 64, 64, torch.bfloat16, seed=5, h0=False, dht=False)
    beta = beta.to(torch.bfloat16)
    got = gd.chunk_bwd(*[x.to(DEV) for x in (q, k, v, g, beta)], 0.125, None, do.to(DEV), None)
    torch.cuda.synchronize()
    ref = oracle_grads(q, k, v, g, beta, 0.125, None, do, None)
    check("bwd no h0/dht", got, ref, dict(dq=torch.bfloat16, dk=torch.bfloat16, dv=torch.bfloat16,
                                          dg=torch.float32, dbeta=torch.bfloat16, dh0=torch.float32))


def test_slow_decay_long_range():
    """g near 0 (the state carries across all 8 chunks) and strong writes."""
    q, k, v, g, beta, h0, do, dht = make(1, 512, 1, 2, 64, 64, torch.float32, seed=9)
    g = g * 0.01
    got = gd.chunk_bwd(*[x.to(DEV) for x in (q, k, v, g, beta)], 0.125, h0.to(DEV), do.to(DEV), dht.to(DEV))
    torch.cuda.synchronize()
    ref = oracle_grads(q, k, v, g, beta, 0.125, h0, do, dht)
    check("bwd slow decay", got, ref, dict(dq=torch.float32, dk=torch.float32, dv=torch.float32, dg=torch.float32,
                                           dbeta=torch.float32, dh0=torch.float32))


def test_autograd_through_the_operator():
    """torch.autograd through gated_delta_rule(..., 'hip') (the custom op with
    its registered backward) gives the oracle's gradients of a loss on o and
    the final state, each in its input's dtype."""
    q, k, v, g, beta, h0, do, dht = make(2, 100, 2, 4, 128, 128, torch.bfloat16, seed=11)
    leaves = [x.to(DEV).requires_grad_() for x in (q, k, v, g, beta, h0)]
    o, final = gd.gated_delta_rule(*leaves[:5], 128 ** -0.5, leaves[5], "hip")
    loss = (o * do.to(DEV).float()).sum() + (final * dht.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    got = [x.grad for x in leaves]
    ref = oracle_grads(q, k, v, g, beta, 128 ** -0.5, h0, do.float(), dht)
    check("autograd", got, ref, dict(dq=torch.bfloat16, dk=torch.bfloat16, dv=torch.bfloat16, dg=torch.float32,
                                     dbeta=torch.float32, dh0=torch.float32))


@pytest.mark.parametrize("dtype,dk,dv", [(torch.bfloat16, 128, 128), (torch.float32, 96, 64)])
def test_autograd_through_packed_sequences(dtype, dk, dv):
    """A packed training call (cu_seqlens, one h0 per sequence, an empty
    sequence among them) through gated_delta_rule(..., 'hip'): the backward
    runs sequence by sequence and gives the oracle's gradients of each."""
    from pseudobrain_amd.workloads import cu_seqlens_of
    lengths = [70, 0, 130, 5, 64]
    n, total = len(lengths), sum(lengths)
    q, k, v, g, beta, h0 = generate(1, total, 2, 4, dk, dv, dtype, 0.05, seed=21, nstates=n)
    gen = torch.Generator().manual_seed(22)
    do = (torch.randn(1, total, 4, dv, generator=gen) * 0.1).to(dtype)
    dht = torch.randn(n, 4, dk, dv, generator=gen) * 0.1
    cu = cu_seqlens_of(lengths)
    leaves = [x.to(DEV).requires_grad_() for x in (q, k, v, g, beta, h0)]
    o, final = gd.gated_delta_rule(*leaves[:5], dk ** -0.5, leaves[5], "hip", cu_seqlens=cu.to(DEV))
    loss = (o * do.to(DEV).float()).sum() + (final * dht.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    got = [x.grad for x in leaves]
    parts, dh0 = [], []
    bounds = cu.tolist()
    for i in range(n):
        sl = slice(bounds[i], bounds[i + 1])
        if bounds[i + 1] == bounds[i]:
            dh0.append(to_numpy(dht[i].double()))
            continue
        r = oracle_grads(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], dk ** -0.5, h0[i:i + 1],
                         do[:, sl].float(), dht[i:i + 1])
        parts.append(r[:5])
        dh0.append(r[5][0])
    ref = [np.concatenate([p_[j] for p_ in parts], axis=1) for j in range(5)] + [np.stack(dh0)]
    check(f"packed autograd {dtype} K={dk} V={dv}", got, ref,
          dict(dq=dtype, dk=dtype, dv=dtype, dg=torch.float32, dbeta=torch.float32, dh0=torch.float32))
    assert torch.equal(got[5][1].cpu(), dht[1])  # the empty sequence: its final state is its h0


def test_zero_length_gives_the_final_gradient_as_dh0():
    q, k, v, g, beta, h0, do, dht = make(1, 0, 1, 1, 64, 64, torch.float32, seed=3)
    got = gd.chunk_bwd(*[x.to(DEV) for x in (q, k, v, g, beta)], 0.125, h0.to(DEV), do.to(DEV), dht.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(got[5].cpu(), dht)
    assert got[0].numel() == 0 and got[3].numel() == 0


def test_full_size_gradients_are_linear_in_the_output_gradients():
    """At the prefill shape (B=1, T=32768, Hk=16, Hv=32, K=V=128, bf16), too
    large for the oracle: every gradient is linear in (dO, dht), so the
    gradients for (dO1 + dO2, dht1 + dht2) equal the sum of the two calls'.
    dO1 and dO2 live on the even and the odd tokens, so their sum is exact in
    bf16. Float32 results within 1e-4 of the largest magnitude, bf16 results
    within their rounding (1e-2)."""
    from pseudobrain_amd.workloads import workload
    q, k, v, g, beta, h0 = (x.to(DEV) for x in workload("prefill_qwen3next", seed=0))
    gen = torch.Generator().manual_seed(21)
    length = q.shape[1]
    do = (torch.randn(1, length, v.shape[2], v.shape[3], generator=gen) * 0.05).to(torch.bfloat16)
    even = (torch.arange(length) % 2 == 0).view(1, length, 1, 1)
    do1, do2 = (do * even).to(DEV), (do * ~even).to(DEV)
    d1, d2 = [(torch.randn(h0.shape, generator=gen) * 0.05).to(DEV) for _ in range(2)]
    scale = q.shape[-1] ** -0.5
    ga = [x.float().cpu() for x in gd.chunk_bwd(q, k, v, g, beta, scale, h0, do1, d1)]
    gb = [x.float().cpu() for x in gd.chunk_bwd(q, k, v, g, beta, scale, h0, do2, d2)]
    gs = gd.chunk_bwd(q, k, v, g, beta, scale, h0, do.to(DEV), d1 + d2)
    torch.cuda.synchronize()
    for name, a, b2, s in zip(NAMES, ga, gb, gs):
        err = rel_err(s, to_numpy(a + b2))
        tol = BF16_TOL if s.dtype == torch.bfloat16 else 1e-4
        print(f"[full-size linearity] {name} rel_inf={err:.2e}", flush=True)
        assert err <= tol, f"{name}: {err:.3e}"


@pytest.mark.parametrize("case", range(8))
def test_random_backward(case):
    """Randomised shapes against the oracle: head widths, GQA ratio, batch,
    length (padding), input dtype, beta in float32 or q's dtype, h0 and dht
    present or absent; drawn from a fixed seed."""
    rng = np.random.default_rng(3000 + case)
    pick = lambda xs: xs[int(rng.integers(len(xs)))]  # noqa: E731
    dk, dv = pick([64, 128]), pick([64, 128])
    hk = pick([1, 2])
    hv = hk * pick([1, 2, 4])
    dtype = pick([torch.float32, torch.bfloat16, torch.float16])
    batch, length = int(rng.integers(1, 3)), int(rng.integers(1, 300))
    with_h0, with_dht = bool(rng.integers(2)), bool(rng.integers(2))
    q, k, v, g, beta, h0, do, dht = make(batch, length, hk, hv, dk, dv, dtype, seed=40 + case, h0=with_h0,
                                         dht=with_dht)
    if dtype != torch.float32 and bool(rng.integers(2)):
        beta = beta.to(dtype)
    name = (f"random bwd {case}: B={batch} T={length} {hk}->{hv} K={dk} V={dv} {dtype} beta {beta.dtype} "
            f"h0={with_h0} dht={with_dht}")
    print(f"[{name}]", flush=True)
    scale = dk ** -0.5
    got = gd.chunk_bwd(*[x.to(DEV) for x in (q, k, v, g, beta)], scale, None if h0 is None else h0.to(DEV),
                       do.to(DEV), None if dht is None else dht.to(DEV))
    torch.cuda.synchronize()
    ref = oracle_grads(q, k, v, g, beta, scale, h0, do, dht)
    check(name, got, ref, dict(dq=dtype, dk=dtype, dv=dtype, dg=torch.float32, dbeta=beta.dtype,
                               dh0=torch.float32))
