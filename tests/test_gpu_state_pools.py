"""States held the way a serving cache holds them: pools of slots in float32,
bfloat16 or float16 (vLLM keeps the recurrent state in the model's dtype unless
told otherwise, serving/pb27_vllm/pb27_vllm/universal_models.py:137-165), read
and written in place by slot index, for decode, speculative verify and prefill.

The arithmetic stays float32; a 16-bit state is widened when it is read and
rounded to nearest even when it is written. So a 16-bit state written once must
equal the fp32 oracle's state rounded to that format, to within one unit in the
last place (the kernel's fp32 result and the oracle's differ by ~1e-6 relative,
which can move a value across a rounding boundary) plus 1e-5 of the largest
magnitude; o keeps the usual 2e-2 (bf16) bound against the oracle run from the
widened starting values. The prefill's fp32 state carries its own error
against the oracle (within 1e-3 of the largest magnitude, its usual bound), so
there the 16-bit state gets that allowance on top of the ulp, and must equal
the kernel's own fp32 result rounded to nearest even, bit for bit."""
import numpy as np
import pytest
import torch

from oracle import gdn
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import generate, to_numpy
from tests.gpu_util import S_TOL, assert_parity, oracle, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5
ROUND = {torch.bfloat16: gdn.round_bf16, torch.float16: gdn.round_fp16}
MANTISSA = {torch.bfloat16: 7, torch.float16: 10}   # explicit significand bits
UNIT = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}  # unit roundoff


def to_dev(*xs):
    return [x.to(DEV) for x in xs]


def ulp(x, dtype):
    """Spacing of `dtype` at |x| (fp16 subnormal spacing below 2^-14)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-38)))
    if dtype == torch.float16:
        e = np.maximum(e, -14)
    return 2.0 ** (e - MANTISSA[dtype])


def assert_rounded(name, got, ref, dtype, tol=1e-5):
    """got (a 16-bit state) == ref (fp32) rounded to dtype, within one ulp + tol max|ref|
    (tol: the fp32 path's own error against the oracle)."""
    got = to_numpy(got.float()).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = ulp(ref, dtype) + tol * np.abs(ref).max()
    excess = np.abs(got - ROUND[dtype](ref.astype(np.float32))) - bound
    exact = np.mean(got == ROUND[dtype](ref.astype(np.float32)))
    print(f"[{name}] worst excess over 1 ulp {excess.max():.3e}; exactly rounded {100 * exact:.2f}%", flush=True)
    assert excess.max() <= 0, f"{name}: a state value is off by more than one {dtype} ulp"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_16bit_state_slots(dtype):
    """Decode at the Qwen3-Next head shape (64 sequences, Hk=16, Hv=32, K=V=128)
    from a 16-bit pool of 80 slots, through permuted slots: one call of 3
    tokens (one rounding) against the oracle, then 3 chained in-place one-token
    calls against the oracle rounded after each step."""
    batch, hk, hv, dk, dv = 64, 16, 32, 128, 128
    q, k, v, g, beta, _ = generate(batch, 3, hk, hv, dk, dv, torch.bfloat16, 0.0, seed=61)
    pool = (torch.randn(80, hv, dk, dv, generator=torch.Generator().manual_seed(62)) * 0.02).to(dtype)
    idx = torch.randperm(80, generator=torch.Generator().manual_seed(63))[:batch].to(torch.int32)
    h0 = pool[idx.long()].float()
    dq, dk_, dv_, dg, db, didx = to_dev(q, k, v, g, beta, idx)

    dpool = pool.to(DEV)
    o, _ = gd.recurrent_fwd(dq, dk_, dv_, dg, db, SCALE, dpool, dpool, didx, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, "sequential")
    assert_parity(f"decode T=3 {dtype} state: o", o, o_ref)
    assert_rounded(f"decode T=3 {dtype} state", dpool.cpu()[idx.long()], s_ref, dtype)
    others = [i for i in range(80) if i not in set(idx.tolist())]
    assert torch.equal(dpool.cpu()[others], pool[others])

    dpool = pool.to(DEV)
    ref = to_numpy(h0)
    for t in range(3):
        sl = slice(t, t + 1)
        o_t = torch.ops.pbgdn.recurrent_step_(dq[:, sl], dk_[:, sl], dv_[:, sl], dg[:, sl], db[:, sl], dpool,
                                              didx, SCALE)
        o_ref, ref = oracle(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], SCALE, torch.from_numpy(ref),
                            "sequential")
        ref = ROUND[dtype](ref.astype(np.float32))  # the pool holds the rounded state between calls
        assert_parity(f"decode chained step {t} {dtype} state: o", o_t, o_ref)
    torch.cuda.synchronize()
    err = rel_err(dpool.cpu()[idx.long()], ref)
    print(f"[decode 3 chained steps {dtype} state] S rel_inf={err:.3e}", flush=True)
    assert err <= S_TOL + 3 * UNIT[dtype]  # at most one rounding-boundary flip per stored step


def test_verify_bf16_state_slots():
    """Speculative verify with a bf16 pool: the state after every token, each
    written once, equals the oracle's prefix state rounded to bf16."""
    batch, length, hk, hv, dk, dv = 4, 4, 16, 32, 128, 128
    q, k, v, g, beta, _ = generate(batch, length, hk, hv, dk, dv, torch.bfloat16, 0.0, seed=64)
    pool = (torch.randn(24, hv, dk, dv, generator=torch.Generator().manual_seed(65)) * 0.02).to(torch.bfloat16)
    start = torch.tensor([1, 0, 3, 2], dtype=torch.int32)
    slots = torch.arange(8, 8 + batch * length, dtype=torch.int32).view(batch, length)
    dq, dk_, dv_, dg, db, dpool, dstart, dslots = to_dev(q, k, v, g, beta, pool, start, slots)
    o, states = gd.recurrent_fwd(dq, dk_, dv_, dg, db, SCALE, dpool, dpool, dstart, out_dtype=torch.bfloat16,
                                 token_state_idx=dslots)
    torch.cuda.synchronize()
    states = states.cpu()
    h0 = pool[start.long()].float()
    o_ref, _ = oracle(q, k, v, g, beta, SCALE, h0, "sequential")
    assert_parity("verify bf16 state: o", o, o_ref)
    for t in range(length):
        _, s_t = oracle(q[:, :t + 1], k[:, :t + 1], v[:, :t + 1], g[:, :t + 1], beta[:, :t + 1], SCALE, h0,
                        "sequential")
        assert_rounded(f"verify bf16 state after token {t}", states[slots[:, t].long()], s_t, torch.bfloat16)
    assert torch.equal(states[:8], pool[:8])  # starting slots (and slots 4..7) are only read


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_state_slots(dtype):
    """Packed prefill against a pool of 12 slots (vLLM's chunked prefill with
    ssm_state_indices and has_initial_state): sequence 0 continues slot 5,
    sequence 1 is a new request in slot 0 (stale data, has_initial_state 0),
    the empty sequence 2 keeps slot 9, sequence 3 has no slot (-1: zero start,
    no write). Other slots are untouched."""
    lengths = [300, 64, 0, 1000]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    hk, hv, dk, dv = 16, 32, 128, 128
    q, k, v, g, beta, _ = generate(1, int(cu[-1]), hk, hv, dk, dv, torch.bfloat16, 0.0, seed=66)
    pool = (torch.randn(12, hv, dk, dv, generator=torch.Generator().manual_seed(67)) * 0.02).to(dtype)
    idx = torch.tensor([5, 0, 9, -1], dtype=torch.int32)
    has_init = torch.tensor([True, False, True, True])
    h0 = torch.zeros(4, hv, dk, dv)
    h0[0], h0[2] = pool[5].float(), pool[9].float()
    dpool = pool.to(DEV)
    o = gd.chunk_fwd_slots(*to_dev(q, k, v, g, beta), SCALE, dpool, idx.to(DEV), cu.to(DEV), has_init.to(DEV))
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, cu_seqlens=cu)
    assert_parity(f"prefill slots {dtype}: o", o, o_ref)
    got = dpool.cpu()
    if dtype == torch.float32:
        assert_parity("prefill slots fp32: states", o, o_ref, got[[5, 0]], s_ref[[0, 1]])
    else:
        assert_rounded(f"prefill slots {dtype}: states", got[[5, 0]], s_ref[[0, 1]], dtype, tol=S_TOL)
        f32pool = pool.float().to(DEV)  # the same values held in float32: the same arithmetic
        gd.chunk_fwd_slots(*to_dev(q, k, v, g, beta), SCALE, f32pool, idx.to(DEV), cu.to(DEV), has_init.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(got, f32pool.cpu().to(dtype)), "a 16-bit state is the fp32 state rounded to nearest even"
    assert torch.equal(got[9], pool[9])  # the empty sequence writes its starting state back unchanged
    untouched = [i for i in range(12) if i not in (5, 0, 9)]
    assert torch.equal(got[untouched], pool[untouched])

    # the same call through chunk_fwd with the gathered starting states: the same o, bit for bit
    o2, final = gd.chunk_fwd(*to_dev(q, k, v, g, beta), SCALE, h0.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(o.cpu(), o2.cpu())
    if dtype == torch.float32:
        assert torch.equal(got[[5, 0]], final.cpu()[[0, 1]])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_zero_tokens_copy_the_state(dtype):
    """T = 0: no input is read (the input tensors are empty); each named state
    is copied to state_out unchanged."""
    q, k, v, g, beta, _ = generate(3, 0, 2, 4, 64, 64, torch.bfloat16, 0.0, seed=68)
    pool = (torch.randn(5, 4, 64, 64, generator=torch.Generator().manual_seed(69)) * 0.1).to(dtype)
    idx = torch.tensor([4, 1, 2], dtype=torch.int32)
    dpool = pool.to(DEV)
    out = torch.full_like(dpool, 7.0)
    o, _ = gd.recurrent_fwd(*to_dev(q, k, v, g, beta), 0.125, dpool, out, idx.to(DEV))
    torch.cuda.synchronize()
    assert o.shape == (3, 0, 4, 64)
    assert torch.equal(out.cpu()[idx.long()], pool[idx.long()])
    assert (out.cpu()[[0, 3]] == 7.0).all()
