"""Parity of the wide prefill scan (chunk_wide.hip: 128 value columns of a
(sequence, value head) per workgroup) with the fp32 oracle, at shapes that
select it: 16-bit inputs and outputs, K = 128, V a multiple of 128, and at
least 128 of its workgroups (sequences x value heads x V/128).

Tolerances as tests/test_gpu_chunk.py: outputs 2e-2, final states 1e-3
(infinity-norm relative error against the fp32 oracle on the same inputs)."""
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import cu_seqlens_of, generate
from tests.gpu_util import assert_parity, oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(*xs):
    return [None if x is None else x.to(DEV) for x in xs]


@pytest.mark.parametrize("batch,length,hk,hv,dtype", [
    (4, 300, 16, 32, torch.bfloat16),   # Qwen3-Next heads, a padded last chunk
    (4, 130, 32, 32, torch.float16),    # no GQA, fp16
    (4, 64, 8, 32, torch.bfloat16),     # 4 value heads per key head, exactly one chunk
    (8, 1, 16, 32, torch.bfloat16),     # one token
])
def test_wide_batch(batch, length, hk, hv, dtype):
    q, k, v, g, beta, h0 = generate(batch, length, hk, hv, 128, 128, dtype, 0.02, seed=length + hk)
    assert batch * hv >= 128  # the wide scan's workgroups
    with torch.no_grad():
        o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0)
    assert_parity(f"wide B={batch} T={length} Hk={hk}", o, o_ref, s, s_ref)


def test_wide_two_column_groups_per_head():
    """V = 256: two 128-column groups per value head (column offset 128, and
    2 Hv / Hk workgroups per key head in the XCD grouping), 128 workgroups."""
    q, k, v, g, beta, h0 = generate(2, 200, 16, 32, 128, 256, torch.bfloat16, 0.02, seed=11)
    with torch.no_grad():
        o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0)
    assert_parity("wide V=256", o, o_ref, s, s_ref)


def test_wide_packed_sequences_with_empty_and_ragged_lengths():
    lengths = [200, 0, 1, 63, 64, 65, 129, 10]
    q, k, v, g, beta, h0 = generate(1, sum(lengths), 16, 32, 128, 128, torch.bfloat16, 0.02, seed=7,
                                    nstates=len(lengths))
    cu = cu_seqlens_of(lengths)
    with torch.no_grad():
        o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0, cu_seqlens=cu)
    assert_parity("wide packed", o, o_ref, s, s_ref)
    assert torch.equal(s[1].cpu(), h0[1])  # the empty sequence keeps its initial state


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_wide_state_slots(state_dtype):
    """Slot-indexed states (vLLM's chunked prefill), a new request without an
    initial state, a -1 slot; the pool in float32 or bf16."""
    lengths = [100, 70, 0, 150]
    n = len(lengths)
    q, k, v, g, beta, h0 = generate(1, sum(lengths), 16, 32, 128, 128, torch.bfloat16, 0.02, seed=3, nstates=n)
    pool = (torch.randn(9, 32, 128, 128) * 0.02).to(state_dtype)
    slots = torch.tensor([5, 0, 7, -1], dtype=torch.int32)
    has_init = torch.tensor([1, 0, 1, 1], dtype=torch.uint8)
    cu = cu_seqlens_of(lengths)
    dpool = pool.to(DEV)
    with torch.no_grad():
        o = gd.chunk_fwd_slots(*to_dev(q, k, v, g, beta), 128 ** -0.5, dpool, slots.to(DEV), cu.to(DEV),
                               has_init.to(DEV))
    torch.cuda.synchronize()
    init = torch.stack([pool[5].float(), torch.zeros(32, 128, 128), pool[7].float(), torch.zeros(32, 128, 128)])
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, init, cu_seqlens=cu)
    s_tol = 1e-3 if state_dtype == torch.float32 else 1e-2
    got = dpool.cpu().float()
    assert_parity(f"wide slots {state_dtype}", o, o_ref, got[[5, 0, 7]], s_ref[:3], s_tol=s_tol)
    untouched = [1, 2, 3, 4, 6, 8]
    assert torch.equal(dpool.cpu()[untouched], pool[untouched])


def test_wide_matches_the_narrow_scan_on_long_sequences():
    """Four sequences of 2,048 tokens (128 wide workgroups): against the
    oracle, and the same call split into one-sequence calls (narrow scan)
    agrees within the tolerance."""
    q, k, v, g, beta, h0 = generate(4, 2048, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=11)
    with torch.no_grad():
        o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), 128 ** -0.5, h0.to(DEV))
        parts = [gd.chunk_fwd(*to_dev(q[b:b + 1], k[b:b + 1], v[b:b + 1], g[b:b + 1], beta[b:b + 1]), 128 ** -0.5,
                              h0[b:b + 1].to(DEV)) for b in range(4)]
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0)
    assert_parity("wide 4x2048", o, o_ref, s, s_ref)
    assert_parity("narrow 1x2048 each", torch.cat([p[0] for p in parts]), o_ref, torch.cat([p[1] for p in parts]),
                  s_ref)
