"""Parity of the chunkwise prefill for 256-wide keys (chunk_k256.hip with the
prep kernel at K = 256) with the fp32 oracle (delta_rule_chunked,
gated_deltanet.py:110-165), through the C ABI.

Tolerances as the other chunk tests (infinity-norm relative error vs the fp32
reference on the same inputs): outputs 2e-2, final states 1e-3. The cases
cover both workgroup widths (2 waves, and 4 waves where the workgroups fill
the CUs), chunk-edge lengths, packed sequences with empty and one-token
members, state slots with has_initial_state and a bf16 pool, GQA with an odd
group, float32 outputs, the X range scaling (|v| ~ 1e3), strong decay, and key
and value widths the caller pads (K 200 -> 256, V 80 -> 96), and the layer
core (the operator, then the epilogue kernel). At the full
32,768-token shape with 32 heads: the whole call against the oracle, and the
two-call identity (a split at a chunk boundary, the state carried in fp32,
equals one call bit for bit)."""
import numpy as np
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import cu_seqlens_of, generate, workload
from tests.gpu_util import assert_parity, oracle, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 256 ** -0.5


def to_dev(*xs):
    return [None if x is None else x.to(DEV) for x in xs]


def run(q, k, v, g, beta, h0, cu=None, out_dtype=None, scale=SCALE):
    o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), scale, None if h0 is None else h0.to(DEV),
                        None if cu is None else cu.to(DEV), out_dtype=out_dtype)
    torch.cuda.synchronize()
    return o, s


@pytest.mark.parametrize("length", [1, 17, 63, 64, 65, 130, 300])
@pytest.mark.parametrize("dv", [32, 64, 256])
def test_lengths_and_value_widths(length, dv):
    print(f"[k256] T={length} V={dv}", flush=True)
    q, k, v, g, beta, h0 = generate(1, length, 2, 4, 256, dv, torch.bfloat16, 0.02, seed=length + dv)
    o, s = run(q, k, v, g, beta, h0)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert o.dtype == torch.bfloat16
    assert_parity(f"k256 T={length} V={dv}", o, o_ref, s, s_ref)


def test_four_wave_workgroups():
    """Enough (sequence, value head, 64-column group) workgroups to cover the
    CUs: the 4-wave kernel takes the call (2 x 32 x 4 = 256)."""
    q, k, v, g, beta, h0 = generate(2, 200, 16, 32, 256, 256, torch.bfloat16, 0.02, seed=5)
    o, s = run(q, k, v, g, beta, h0)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert_parity("k256 4-wave B=2 T=200 Hv=32", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_float32_output_and_fp16_inputs(dtype):
    q, k, v, g, beta, h0 = generate(1, 257, 1, 3, 256, 64, dtype, 0.02, seed=9)  # GQA 1 -> 3 (odd group)
    o, s = run(q, k, v, g, beta, h0, out_dtype=torch.float32)
    assert o.dtype == torch.float32
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert_parity(f"k256 {dtype} -> f32 GQA 1->3", o, o_ref, s, s_ref)


def test_zero_initial_state_and_no_final_state():
    q, k, v, g, beta, _ = generate(2, 150, 2, 2, 256, 128, torch.bfloat16, 0.0, seed=3)
    o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), SCALE, None, output_final_state=False)
    torch.cuda.synchronize()
    assert s is None
    o_ref, _ = oracle(q, k, v, g, beta, SCALE, torch.zeros(2, 2, 256, 128))
    assert rel_err(o, o_ref) <= 2e-2


def test_large_values_and_strong_decay():
    """|v| ~ 1e3 (X beyond the fp16 operand range: the per-tile power-of-two
    scaling) and gates down to exp(-20) per token."""
    q, k, v, g, beta, h0 = generate(1, 200, 2, 4, 256, 64, torch.bfloat16, 0.02, seed=11)
    v = (v.float() * 1000).to(torch.bfloat16)
    g = g * 8
    o, s = run(q, k, v, g, beta, h0)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert_parity("k256 |v|~1e3, strong decay", o, o_ref, s, s_ref)


def test_packed_sequences():
    lengths = [0, 1, 64, 65, 300, 7, 128]
    total = sum(lengths)
    q, k, v, g, beta, h0 = generate(1, total, 2, 4, 256, 64, torch.bfloat16, 0.02, seed=21,
                                    nstates=len(lengths))
    cu = cu_seqlens_of(lengths)
    o, s = run(q, k, v, g, beta, h0, cu)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, cu_seqlens=cu)
    assert_parity("k256 packed", o, o_ref, s, s_ref)


def test_many_short_sequences():
    """200 packed sequences of 1 to 130 tokens (one workgroup per sequence,
    value head and column group, most of them a chunk or less)."""
    gen = torch.Generator().manual_seed(61)
    lengths = torch.randint(1, 131, (200,), generator=gen).tolist()
    q, k, v, g, beta, h0 = generate(1, sum(lengths), 1, 2, 256, 64, torch.bfloat16, 0.02, seed=62,
                                    nstates=len(lengths))
    cu = cu_seqlens_of(lengths)
    o, s = run(q, k, v, g, beta, h0, cu)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, cu_seqlens=cu)
    assert_parity("k256 200 short sequences", o, o_ref, s, s_ref)


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_state_slots(pool_dtype):
    """chunk_fwd_slots: sequences start from pool slots (zeros where
    has_initial_state is False) and write their final states back in place."""
    lengths = [70, 1, 200]
    total = sum(lengths)
    q, k, v, g, beta, h0 = generate(1, total, 2, 2, 256, 64, torch.bfloat16, 0.02, seed=31, nstates=3)
    cu = cu_seqlens_of(lengths)
    pool = (torch.randn(6, 2, 256, 64) * 0.02).to(pool_dtype)
    idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    has = torch.tensor([True, False, True])
    start = torch.stack([pool[4].float(), torch.zeros(2, 256, 64), pool[2].float()])
    dpool = pool.to(DEV)
    o = gd.chunk_fwd_slots(*to_dev(q, k, v, g, beta), SCALE, dpool, idx.to(DEV), cu.to(DEV), has.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, start, cu_seqlens=cu)
    got = dpool.cpu().float()
    s = torch.stack([got[4], got[0], got[2]])
    s_tol = 1e-3 if pool_dtype == torch.float32 else 8e-3  # a bf16 pool rounds the state to 8 bits
    assert_parity(f"k256 slots {pool_dtype}", o, o_ref, s, s_ref, s_tol=s_tol)
    untouched = [1, 3, 5]
    assert torch.equal(got[untouched], pool[untouched].float())


@pytest.mark.parametrize("dk,dv,dtype", [(200, 80, torch.bfloat16), (256, 256, torch.float16), (160, 100, torch.bfloat16)])
def test_operator_pads_key_and_value_widths(dk, dv, dtype):
    """gated_delta_rule's device path (delta_rule_hip) zero-pads K to 256 and V
    to a multiple of 32 and takes the chunk kernel."""
    q, k, v, g, beta, h0 = generate(1, 190, 1, 2, dk, dv, dtype, 0.02, seed=dk)
    dq, dk_, dv_, dg, db, dh = to_dev(q, k, v, g, beta, h0)
    assert gd.hip_usable(dh, dq)
    o, s = gd.gated_delta_rule(dq, dk_, dv_, dg, db, dk ** -0.5, dh, kernel="hip")
    torch.cuda.synchronize()
    assert o.shape == (1, 190, 2, dv) and s.shape == (1, 2, dk, dv)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0)
    assert_parity(f"k256 operator K={dk} V={dv}", o, o_ref, s, s_ref)


def test_full_shape_against_the_oracle():
    """The 256-wide workload (B=1, T=32,768, Hk=16 -> Hv=32, K=V=256) in full."""
    q, k, v, g, beta, h0 = workload("prefill_k256", seed=41)
    o, s = run(q, k, v, g, beta, h0)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert_parity("k256 T=32768 Hv=32", o, o_ref, s, s_ref)


def test_full_shape_split_equals_one_call():
    """T = 32,768 at the 256-wide shape: two calls split at token 16,384 (a
    chunk boundary), the second from the first's final state, give the one
    call's outputs and final state bit for bit."""
    q, k, v, g, beta, h0 = to_dev(*workload("prefill_k256", seed=43))
    o, s = gd.chunk_fwd(q, k, v, g, beta, SCALE, h0)
    half = 16384
    o1, s1 = gd.chunk_fwd(q[:, :half], k[:, :half], v[:, :half], g[:, :half], beta[:, :half], SCALE, h0)
    o2, s2 = gd.chunk_fwd(q[:, half:], k[:, half:], v[:, half:], g[:, half:], beta[:, half:], SCALE, s1)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(s).all()
    assert torch.equal(o[:, :half], o1) and torch.equal(o[:, half:], o2)
    assert torch.equal(s, s2)


def test_layer_core_two_pass():
    """chunk_layer_fwd at K = 256 (the operator for 256-wide keys, then the
    epilogue kernel) against the oracle operator and the oracle epilogue."""
    from oracle import layer as ol
    from pseudobrain_amd.layer import chunk_layer_fwd
    from pseudobrain_amd.workloads import to_numpy
    eps = 1e-5
    q, k, v, g, beta, h0 = generate(2, 200, 2, 4, 256, 128, torch.bfloat16, 0.02, seed=51)
    gen = torch.Generator().manual_seed(52)
    z = torch.randn(2, 200, 3 * 4 * 128, generator=gen).to(torch.bfloat16)
    gate = z[..., 4 * 128:2 * 4 * 128]  # a column slice of the projection, as the layer has it
    o_norm = torch.rand(128, generator=gen) + 0.5
    dev = to_dev(q, k, v, g, beta, h0, gate, o_norm)
    with torch.no_grad():
        hs, s = chunk_layer_fwd(*dev[:5], SCALE, dev[5], dev[6], dev[7], eps)
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    hs_ref = ol.layer_epilogue(o_ref, to_numpy(gate.float()), to_numpy(o_norm), eps)
    assert hs.shape == gate.shape
    assert rel_err(hs, hs_ref.reshape(hs.shape)) <= 2e-2
    assert rel_err(s, s_ref) <= 1e-3
