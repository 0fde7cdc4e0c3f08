"""Parity of the fused recurrent (decode) kernel with the fp32 oracle
(delta_rule_sequential, gated_deltanet.py:93-107), through the C ABI."""
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import generate, workload
from tests.gpu_util import assert_parity, oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5


def to_dev(*xs):
    return [x.to(DEV) for x in xs]


def test_decode_b64_one_step():
    """64 sequences x 1 token, Hk=16 -> Hv=32, K=V=128, bf16, state [64,32,128,128]."""
    q, k, v, g, beta, h0 = workload("decode_b64", seed=11)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, "sequential")
    dq, dk, dv, dg, db, state = to_dev(q, k, v, g, beta, h0)
    o = torch.ops.pbgdn.recurrent_step_(dq, dk, dv, dg, db, state, None, SCALE)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == (64, 1, 32, 128)
    assert_parity("decode_b64 step", o, o_ref, state, s_ref)


@pytest.mark.parametrize("batch,state_dtype", [(100, torch.float32), (128, torch.float32), (200, torch.bfloat16)])
def test_decode_step_streamed_past_the_cache(batch, state_dtype):
    """Steps that move more than 192 MiB of state at the Qwen3-Next head shape
    stream it past the cache: B=100 float32 and B=200 bf16 with one workgroup
    per head state, B=128 float32 (4,096 head states) with each state's columns
    split over two workgroups. Same results as the oracle."""
    q, k, v, g, beta, h0 = generate(batch, 1, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=batch)
    h0 = h0.to(state_dtype)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0.float(), "sequential")
    dq, dk, dv, dg, db, state = to_dev(q, k, v, g, beta, h0)
    o = torch.ops.pbgdn.recurrent_step_(dq, dk, dv, dg, db, state, None, SCALE)
    torch.cuda.synchronize()
    s_tol = 1e-3 if state_dtype == torch.float32 else 1e-2
    assert_parity(f"decode B={batch} {state_dtype} streamed", o, o_ref, state.float(), s_ref, s_tol=s_tol)


@pytest.mark.parametrize("batch,state_dtype,dk", [(64, torch.float32, 128), (128, torch.float32, 128),
                                                  (64, torch.bfloat16, 128), (256, torch.float32, 64)])
def test_decode_state_policy_sets_cache_bits_only(batch, state_dtype, dk):
    """The state's cache policy is the caller's (PBGDN_STATE_STREAM, the default,
    or PBGDN_STATE_RESIDENT) and changes cache bits only: the same step under
    either policy gives the same output and state bit for bit, twice in a row
    (no call history), for whole-state and split (4,096+ head states) launches
    and for a resident call small enough to be kept cached (B = 256 at K = 64:
    128 MiB). Both match the oracle."""
    q, k, v, g, beta, h0 = generate(batch, 1, 16, 32, dk, 128, torch.bfloat16, 0.02, seed=batch + dk)
    h0 = h0.to(state_dtype)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0.float(), "sequential")
    dq, dk_, dv, dg, db, base = to_dev(q, k, v, g, beta, h0)
    results = []
    for resident in (False, True, True, False):
        state = base.clone()
        o = torch.ops.pbgdn.recurrent_step_(dq, dk_, dv, dg, db, state, None, dk ** -0.5, resident)
        torch.cuda.synchronize()
        results.append((o, state))
    for o, state in results[1:]:
        assert torch.equal(o, results[0][0]) and torch.equal(state, results[0][1])
    s_tol = 1e-3 if state_dtype == torch.float32 else 1e-2
    assert_parity(f"decode B={batch} K={dk} {state_dtype} either policy", results[0][0], o_ref,
                  results[0][1].float(), s_ref, s_tol=s_tol)


def test_stream_probe_copies():
    """pbgdn_stream_probe copies every byte (64 MiB plus a 16-byte tail piece)."""
    from pseudobrain_amd import _lib
    n = (64 << 20) + 16
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=DEV)
    dst = torch.zeros_like(src)
    _lib.check(_lib.lib().pbgdn_stream_probe(src.data_ptr(), dst.data_ptr(), n,
                                             torch.cuda.current_stream().cuda_stream), "pbgdn_stream_probe")
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


def test_decode_chained_in_place_steps():
    """8 chained in-place steps with fresh tokens equal 8 oracle steps."""
    q, k, v, g, beta, h0 = generate(8, 8, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=5)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, "sequential")
    dq, dk, dv, dg, db, state = to_dev(q, k, v, g, beta, h0)
    outs = []
    for t in range(8):
        sl = slice(t, t + 1)
        outs.append(torch.ops.pbgdn.recurrent_step_(dq[:, sl], dk[:, sl], dv[:, sl], dg[:, sl],
                                                    db[:, sl], state, None, SCALE))
    torch.cuda.synchronize()
    assert_parity("decode 8 chained steps", torch.cat(outs, 1), o_ref, state, s_ref)


def test_state_slots_via_state_idx():
    """state_idx picks the slot each sequence reads and writes; other slots keep their values."""
    q, k, v, g, beta, _ = generate(4, 1, 2, 4, 64, 64, torch.bfloat16, 0.0, seed=9)
    pool = torch.randn(10, 4, 64, 64) * 0.1
    idx = torch.tensor([7, 2, 9, 0], dtype=torch.int32)
    o_ref, s_ref = oracle(q, k, v, g, beta, 0.125, pool[idx.long()], "sequential")
    dq, dk, dv, dg, db, dpool, didx = to_dev(q, k, v, g, beta, pool.clone(), idx)
    o = torch.ops.pbgdn.recurrent_step_(dq, dk, dv, dg, db, dpool, didx, 0.125)
    torch.cuda.synchronize()
    assert_parity("state_idx", o, o_ref, dpool.cpu()[idx.long()], s_ref)
    untouched = [i for i in range(10) if i not in idx.tolist()]
    assert torch.equal(dpool.cpu()[untouched], pool[untouched])


@pytest.mark.parametrize("dk,dv", [(32, 32), (64, 128), (128, 64), (256, 256), (128, 32)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_sequential_kernel_multi_token(dk, dv, dtype):
    """T = 3 tokens through delta_rule_sequential's device kernel; fp32 o."""
    q, k, v, g, beta, h0 = generate(2, 3, 2, 4, dk, dv, dtype, 0.05, seed=dk + dv)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0, "sequential")
    o, s = gd.gated_delta_rule(*to_dev(q, k, v, g, beta), dk ** -0.5, h0.to(DEV), kernel="sequential")
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    assert_parity(f"sequential K={dk} V={dv} {dtype}", o, o_ref, s, s_ref, o_tol=1e-4, s_tol=1e-4)


def test_already_repeated_heads_and_bf16_beta():
    """Hk == Hv (q/k repeated by the caller, the reference's layout) and beta in q's dtype."""
    q, k, v, g, beta, h0 = generate(3, 2, 8, 8, 128, 128, torch.bfloat16, 0.02, seed=4)
    beta = beta.to(torch.bfloat16)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, "sequential")
    o, s = gd.delta_rule_sequential(*to_dev(q, k, v, g, beta), SCALE, h0.to(DEV))
    torch.cuda.synchronize()
    assert_parity("Hk == Hv, bf16 beta", o, o_ref, s, s_ref, o_tol=1e-4, s_tol=1e-4)


def test_speculative_verify_keeps_the_state_after_every_token():
    """Verify mode: 6 sequences x 4 tokens (one accepted + 3 drafts) from
    pooled starting slots; the state after token t lands in its own slot and
    equals the oracle's state after the first t+1 tokens; o matches the
    sequential oracle; slots not named are untouched, a -1 token slot is
    skipped, and a -1 starting slot gives zero output and writes nothing."""
    batch, length, hk, hv, dk, dv = 6, 4, 16, 32, 128, 128
    q, k, v, g, beta, _ = generate(batch, length, hk, hv, dk, dv, torch.bfloat16, 0.0, seed=21)
    pool = torch.randn(40, hv, dk, dv, generator=torch.Generator().manual_seed(22)) * 0.02
    start = torch.tensor([3, 11, 0, 39, -1, 7], dtype=torch.int32)
    slots = torch.arange(12, 12 + batch * length, dtype=torch.int32).view(batch, length)
    slots[1, 2] = -1  # a draft position whose state is not kept
    dq, dk_, dv_, dg, db, dpool, dstart, dslots = to_dev(q, k, v, g, beta, pool.clone(), start, slots)
    o, states = gd.recurrent_fwd(dq, dk_, dv_, dg, db, SCALE, dpool, dpool, dstart,
                                 out_dtype=torch.bfloat16, token_state_idx=dslots)
    torch.cuda.synchronize()
    states = states.cpu()
    live = [b for b in range(batch) if start[b] >= 0]
    h0 = pool[start[live].long()]
    o_ref, _ = oracle(q[live], k[live], v[live], g[live], beta[live], SCALE, h0, "sequential")
    for t in range(length):
        _, s_t = oracle(q[live, :t + 1], k[live, :t + 1], v[live, :t + 1], g[live, :t + 1],
                        beta[live, :t + 1], SCALE, h0, "sequential")
        for i, b in enumerate(live):
            if slots[b, t] >= 0:
                assert_parity(f"verify b={b} t={t}", o[b:b + 1, t:t + 1], o_ref[i:i + 1, t:t + 1],
                              states[slots[b, t]][None], s_t[i:i + 1])
    named = set(slots[slots >= 0].tolist()) | set(start[start >= 0].tolist())
    assert torch.equal(states[[s for s in range(40) if s not in named]], pool[[s for s in range(40) if s not in named]])
    assert torch.equal(states[start[start >= 0].long()], pool[start[start >= 0].long()])  # starting slots are only read
    assert torch.equal(states[slots[4].long()], pool[slots[4].long()])  # the -1 start writes nothing
    assert not o[4].float().abs().any()
    # the last kept state equals the plain recurrent call's final state, bit for bit
    _, final = gd.recurrent_fwd(dq, dk_, dv_, dg, db, SCALE, dpool.clone(), None, dstart, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for b in live:
        assert torch.equal(states[slots[b, -1]], final.cpu()[start[b]])
