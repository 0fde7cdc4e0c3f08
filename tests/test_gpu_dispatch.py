"""The reference's kernel selection and entry point on device tensors
(select_kernel / gated_delta_rule, gated_deltanet.py:189-197, :288-308;
set_scan_backend's "fused" backend, scan.py:100, :143-161), checked against the
oracle: every name select_kernel returns for a device tensor runs, every head
width up to 256 runs (zero-padded to the kernels' widths, or through the
recurrent kernel for float32 inputs with K > 128), and gradients either flow (compared with the
oracle's reverse mode) or the call raises.

Tolerances: outputs 2e-2 and final states 1e-3 (infinity-norm relative, against
the fp32 oracle on the same inputs); gradients as tests/test_gpu_backward.py
(2e-4 float32, 1e-2 for 16-bit results)."""
import numpy as np
import pytest
import torch

from oracle import gdn
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import cu_seqlens_of, generate, to_numpy
from tests.gpu_util import assert_parity, oracle, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(*xs):
    return [None if x is None else x.to(DEV) for x in xs]


def inputs(batch, length, hk, hv, dk, dv, dtype=torch.bfloat16, seed=0, h0_std=0.02, nstates=None):
    return generate(batch, length, hk, hv, dk, dv, dtype, h0_std, seed=seed, nstates=nstates)


@pytest.mark.parametrize("length,expect", [(300, "hip"), (3, "sequential"), (4, "sequential"), (5, "hip")])
def test_fused_backend_selects_and_runs_the_device_kernel(length, expect):
    """The layer's call (gated_deltanet.py:433-438): select_kernel with the
    'fused' backend on device tensors, state first, then gated_delta_rule with
    the name it returned; the result matches the oracle."""
    q, k, v, g, beta, h0 = inputs(1, length, 2, 4, 128, 128, seed=length)
    dq, dk, dv, dg, db, dh = to_dev(q, k, v, g, beta, h0)
    name = gd.select_kernel("fused", False, length, dh, dq)
    assert name == expect
    assert gd.select_kernel("reference", False, length, dh, dq) == ("sequential" if length <= 4 else "chunked")
    assert gd.select_kernel("fused", True, length, dh, dq) == "sequential"
    o, s = gd.gated_delta_rule(dq, dk, dv, dg, db, 128 ** -0.5, dh, kernel=name)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and s.dtype == torch.float32
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0, "sequential" if name == "sequential" else "chunked")
    assert_parity(f"select {name} T={length}", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dk,dv,hk,hv,length,dtype", [
    (256, 256, 1, 2, 150, torch.bfloat16),  # K 256: the chunk kernel for 256-wide keys
    (256, 64, 2, 2, 70, torch.bfloat16),
    (200, 100, 1, 1, 90, torch.float16),    # K 200 -> 256, V 100 -> 128 (a multiple of 32)
    (256, 64, 1, 2, 70, torch.float32),     # float32 above K 128: the recurrent kernel over every token
    (200, 100, 1, 1, 90, torch.float32),    # K 200 -> 256, V 100 -> 128 on the recurrent path
    (64, 48, 2, 4, 200, torch.bfloat16),    # V a multiple of 16 the kernels do not pad
    (96, 40, 1, 2, 130, torch.bfloat16),    # both widths padded (K 96 -> 128, V 40 -> 48)
    (32, 16, 2, 2, 100, torch.bfloat16),    # K 32 -> 64
])
@pytest.mark.parametrize("kernel", ["hip", "chunked"])
def test_every_head_width_up_to_256_runs(dk, dv, hk, hv, length, dtype, kernel):
    q, k, v, g, beta, h0 = inputs(1, length, hk, hv, dk, dv, dtype=dtype, seed=dk + dv)
    dq, dk_, dv_, dg, db, dh = to_dev(q, k, v, g, beta, h0)
    # the gate admits what runs chunkwise: K <= 128, and K <= 256 for 16-bit
    # inputs; float32 inputs wider than 128 would run token by token, so in the
    # reference's wiring fla or chunked keeps them
    chunkwise = dk <= 128 or dtype != torch.float32
    assert gd.hip_usable(dh, dq) == chunkwise
    assert gd.select_kernel("fused", False, length, dh, dq) == ("hip" if chunkwise else "chunked")
    o, s = gd.gated_delta_rule(dq, dk_, dv_, dg, db, dk ** -0.5, dh, kernel=kernel)
    torch.cuda.synchronize()
    assert o.shape == (1, length, hv, dv) and s.shape == (1, hv, dk, dv)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0)
    assert_parity(f"{kernel} K={dk} V={dv}", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dk,dv", [(256, 256), (40, 100)])
def test_sequential_at_odd_widths(dk, dv):
    q, k, v, g, beta, h0 = inputs(2, 3, 1, 2, dk, dv, dtype=torch.float32, seed=7)
    o, s = gd.gated_delta_rule(*to_dev(q, k, v, g, beta), dk ** -0.5, h0.to(DEV), kernel="sequential")
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0, "sequential")
    assert_parity(f"sequential K={dk} V={dv}", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_sequences_with_k256(dtype):
    """cu_seqlens at K = 256 (bfloat16: the chunk kernel for 256-wide keys;
    float32: the recurrent route, one call per sequence), an empty sequence
    keeping its initial state."""
    lengths = [70, 0, 130, 5]
    q, k, v, g, beta, h0 = inputs(1, sum(lengths), 1, 2, 256, 128, dtype=dtype, seed=3, nstates=len(lengths))
    cu = cu_seqlens_of(lengths)
    o, s = gd.gated_delta_rule(*to_dev(q, k, v, g, beta), 256 ** -0.5, h0.to(DEV), kernel="hip",
                               cu_seqlens=cu.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 256 ** -0.5, h0, cu_seqlens=cu)
    assert_parity(f"packed K=256 {dtype}", o, o_ref, s, s_ref)
    assert torch.equal(s[1].cpu(), h0[1])


def _grads(kernel, q, k, v, g, beta, h0, do, dht, scale):
    leaves = [x.to(DEV).detach().requires_grad_(True) for x in (q, k, v, g, beta, h0)]
    o, s = gd.gated_delta_rule(*leaves[:5], scale, leaves[5], kernel=kernel)
    assert o.requires_grad and s.requires_grad
    loss = (o * do.to(DEV).float()).sum() + (s * dht.to(DEV)).sum()
    loss.backward()
    torch.cuda.synchronize()
    return [x.grad for x in leaves]


@pytest.mark.parametrize("kernel,length,dk,dv,hk,hv,dtype", [
    ("sequential", 3, 128, 128, 1, 2, torch.float32),   # T <= SEQUENTIAL_MAX in training: the chunk op's backward
    ("sequential", 1, 64, 64, 2, 2, torch.bfloat16),
    ("hip", 150, 96, 40, 1, 2, torch.float32),          # padded widths keep their gradients
    ("chunked", 90, 64, 128, 2, 4, torch.float32),
])
def test_training_calls_carry_gradients(kernel, length, dk, dv, hk, hv, dtype):
    """A grad-requiring call through gated_delta_rule returns tensors with a
    graph, and backward gives the oracle's gradients (float64 reverse mode
    through the per-token recurrence, pinned by central differences)."""
    q, k, v, g, beta, h0 = inputs(1, length, hk, hv, dk, dv, dtype=dtype, seed=length, h0_std=0.05)
    gen = torch.Generator().manual_seed(99)
    do = torch.randn(1, length, hv, dv, generator=gen) * 0.1
    dht = torch.randn(1, hv, dk, dv, generator=gen) * 0.1
    scale = dk ** -0.5
    got = _grads(kernel, q, k, v, g, beta, h0, do, dht, scale)
    # the chunk backward receives grad_o in q's dtype (the reference casts it, :272)
    do_ref = do.to(dtype).double()
    ref = gdn.gated_delta_rule_backward(*(to_numpy(x.double()) for x in (q, k, v, g, beta)), scale,
                                        to_numpy(h0.double()), to_numpy(do_ref), to_numpy(dht.double()))
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), got, ref):
        tol = 1e-2 if x.dtype in (torch.bfloat16, torch.float16) else 2e-4
        e = rel_err(x, r)
        print(f"[grad {kernel} T={length} K={dk} V={dv}] {name} {e:.2e}", flush=True)
        assert np.isfinite(e) and e <= tol, f"{name}: {e:.3e} > {tol}"


def test_training_call_without_a_device_backward_raises():
    q, k, v, g, beta, h0 = inputs(1, 100, 1, 2, 256, 64, seed=1)
    leaves = [x.to(DEV).requires_grad_(x.is_floating_point()) for x in (q, k, v, g, beta, h0)]
    with pytest.raises(RuntimeError, match="backward"):
        gd.gated_delta_rule(*leaves[:5], 0.0625, leaves[5], kernel="hip")
    # under no_grad the same call is inference and runs
    with torch.no_grad():
        o, _ = gd.gated_delta_rule(*leaves[:5], 0.0625, leaves[5], kernel="hip")
    assert not o.requires_grad
    # the gate sends such calls (K = 256, above the chunk backward's keys) to
    # the reference's path when a gradient is wanted, and takes them (16-bit
    # inputs, the chunk kernel for 256-wide keys) for inference
    assert not gd.hip_usable(leaves[5], leaves[0])
    assert gd.select_kernel("fused", False, 100, leaves[5], leaves[0]) == "chunked"
    with torch.no_grad():
        assert gd.hip_usable(leaves[5], leaves[0])
    # a value width the chunk kernel takes but its backward does not: usable for
    # inference only
    wide_v = torch.zeros(1, 2, 64, 256, device=DEV, requires_grad=True)
    assert not gd.hip_usable(wide_v, leaves[0])
    with torch.no_grad():
        assert gd.hip_usable(wide_v, leaves[0])


def test_entry_points_without_backward_refuse_grad():
    q, k, v, g, beta, h0 = to_dev(*inputs(1, 10, 1, 2, 64, 64, seed=2))
    v.requires_grad_(True)
    with pytest.raises(RuntimeError, match="no backward"):
        gd.chunk_fwd(q, k, v, g, beta, 0.125, h0)
    with pytest.raises(RuntimeError, match="no backward"):
        gd.recurrent_fwd(q, k, v, g, beta, 0.125, h0)
    with torch.no_grad():
        o, s = gd.chunk_fwd(q, k, v, g, beta, 0.125, h0)
    assert not o.requires_grad


def test_recurrent_fwd_keeps_unwritten_slots_and_checks_out():
    """state_out=None with slots: the new pool starts as a copy of state_in, so
    slots the call does not name (and a -1 slot) keep their values; a wrong
    `out` is refused before any launch."""
    q, k, v, g, beta, _ = inputs(3, 1, 1, 2, 64, 64, seed=4)
    pool = torch.randn(6, 2, 64, 64) * 0.1
    idx = torch.tensor([4, -1, 1], dtype=torch.int32)
    with torch.no_grad():
        o, out_pool = gd.recurrent_fwd(*to_dev(q, k, v, g, beta), 0.125, pool.to(DEV), None, idx.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q[[0, 2]], k[[0, 2]], v[[0, 2]], g[[0, 2]], beta[[0, 2]], 0.125, pool[[4, 1]],
                          "sequential")
    assert_parity("slots", o.cpu()[[0, 2]], o_ref, out_pool.cpu()[[4, 1]], s_ref)
    assert torch.equal(out_pool.cpu()[[0, 2, 3, 5]], pool[[0, 2, 3, 5]])
    assert torch.count_nonzero(o.cpu()[1]) == 0
    with pytest.raises(ValueError, match="out must be"):
        gd.recurrent_fwd(*to_dev(q, k, v, g, beta), 0.125, pool.to(DEV), None, idx.to(DEV),
                         out=torch.empty(3, 1, 2, 32, device=DEV))


def test_overlong_cu_seqlens_is_clamped_to_the_tokens():
    """cu_seqlens whose last entry runs past T: the last sequence ends at T
    (the kernels clamp every bound to [0, T]) and nothing outside the buffers
    is touched: the result equals the call with the bound at T."""
    q, k, v, g, beta, h0 = inputs(1, 200, 2, 4, 128, 128, seed=5, nstates=2)
    over = torch.tensor([0, 100, 5000], dtype=torch.int32)
    exact = torch.tensor([0, 100, 200], dtype=torch.int32)
    with torch.no_grad():
        o1, s1 = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV), over.to(DEV))
        o2, s2 = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV), exact.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0, cu_seqlens=exact)
    assert_parity("clamped cu_seqlens", o1, o_ref, s1, s_ref)
