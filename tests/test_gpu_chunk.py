"""Parity of the chunkwise prefill kernel with the fp32 oracle
(delta_rule_chunked, gated_deltanet.py:110-165), through the C ABI.

Tolerances (infinity-norm relative error vs the fp32 reference on the same
inputs): outputs 2e-2, final states 1e-3. At the full sizes of the varlen
(262,144 packed tokens) and million-token (16 x 65,536 streamed) workloads the
oracle runs one key head (its two value heads) over every token, carrying its
own state, and the device run of all heads is compared with it sequence by
sequence and segment by segment; beside that, size-independent properties
(packing == separate calls, streaming == one pass bit for bit)."""
import numpy as np
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import (STREAM_SEGMENT, generate, varlen_workload, workload)
from oracle import gdn
from tests.gpu_util import assert_parity, oracle, rel_err, summarize

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 128 ** -0.5


def to_dev(*xs):
    return [x.to(DEV) for x in xs]


def to_np(t):
    return t.float().cpu().numpy()


def run(q, k, v, g, beta, scale, h0, cu=None):
    o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), scale, None if h0 is None else h0.to(DEV),
                        None if cu is None else cu.to(DEV))
    torch.cuda.synchronize()
    return o, s


def test_prefill_small_fp32_inputs():
    """B=1, T=2048, H=4, K=V=64, fp32 inputs, zero initial state."""
    q, k, v, g, beta, h0 = workload("prefill_small", seed=0)
    o_ref, s_ref = oracle(q, k, v, g, beta, 64 ** -0.5, h0)
    o, s = gd.gated_delta_rule(*to_dev(q, k, v, g, beta), 64 ** -0.5, h0.to(DEV), kernel="chunked")
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and s.dtype == torch.float32
    # U = Tb X from fp16 high/low pairs for float32 inputs: S 2.9e-4 (6.6e-4 with
    # single fp16 operands), held to half the 1e-3 bound
    assert_parity("prefill_small", o, o_ref, s, s_ref, s_tol=5e-4)


@pytest.mark.parametrize("length", [4096])
def test_prefill_qwen3next_shape(length):
    """Hk=16 -> Hv=32, K=V=128, bf16 in, fp32 state, seeded h0."""
    q, k, v, g, beta, h0 = workload("prefill_qwen3next", seed=1, length=length)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    o, s = run(q, k, v, g, beta, SCALE, h0)
    assert o.dtype == torch.bfloat16
    assert_parity(f"qwen3next T={length}", o, o_ref, s, s_ref)


def test_prefill_qwen3next_full_length():
    """The full T=32768 prefill against the oracle."""
    q, k, v, g, beta, h0 = workload("prefill_qwen3next", seed=2)
    o, s = run(q, k, v, g, beta, SCALE, h0)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    assert_parity("qwen3next T=32768", o, o_ref, s, s_ref)


@pytest.mark.parametrize("length", [1, 2, 17, 63, 64, 65, 130, 200])
def test_padding_and_short_sequences(length):
    """T not a multiple of 64 (padded steps are the identity) and T < 64."""
    q, k, v, g, beta, h0 = generate(2, length, 2, 4, 128, 32, torch.bfloat16, 0.05, seed=length)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    o, s = run(q, k, v, g, beta, SCALE, h0)
    assert_parity(f"T={length}", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_input_dtypes_and_zero_state(dtype):
    q, k, v, g, beta, _ = generate(1, 500, 4, 4, 64, 64, dtype, 0.0, seed=3)
    o_ref, s_ref = oracle(q, k, v, g, beta, 0.125, torch.zeros(1, 4, 64, 64))
    o, s = run(q, k, v, g, beta, 0.125, None)
    assert_parity(f"dtype {dtype}, h0=None", o, o_ref, s, s_ref)


def test_slow_decay_long_range():
    """g scaled by 0.01: the state is carried over hundreds of chunks."""
    q, k, v, g, beta, h0 = generate(1, 8192, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=6,
                                    g_scale=0.01)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    o, s = run(q, k, v, g, beta, SCALE, h0)
    assert_parity("slow decay", o, o_ref, s, s_ref)


@pytest.mark.parametrize("case", ["strong_decay", "no_decay", "beta_zero", "beta_one"])
def test_gate_extremes(case):
    """Gates at their edges: g about 30x the usual log decay (in-chunk decays
    underflow to zero; nothing may become NaN or inf), g = 0 (no decay), beta = 0
    (pure decay: S_t = exp(c_t) S_0) and beta = 1."""
    q, k, v, g, beta, h0 = generate(1, 1000, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=31,
                                    g_scale=30.0 if case == "strong_decay" else 1.0)
    if case == "no_decay":
        g = torch.zeros_like(g)
    if case == "beta_zero":
        beta = torch.zeros_like(beta)
    if case == "beta_one":
        beta = torch.ones_like(beta)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    o, s = run(q, k, v, g, beta, SCALE, h0)
    assert torch.isfinite(o.float()).all() and torch.isfinite(s).all()
    assert_parity(f"gates {case}", o, o_ref, s, s_ref)


def test_beta_in_input_dtype_and_fp32_output():
    q, k, v, g, beta, h0 = generate(1, 300, 2, 4, 128, 64, torch.bfloat16, 0.02, seed=8)
    beta = beta.to(torch.bfloat16)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0)
    o, s = gd.chunk_fwd(*to_dev(q, k, v, g, beta), SCALE, h0.to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32
    assert_parity("bf16 beta, fp32 o", o, o_ref, s, s_ref)


@pytest.mark.parametrize("dk,dv,hk,hv", [(64, 16, 1, 8), (128, 48, 2, 2), (128, 256, 1, 4), (64, 256, 2, 4)])
def test_value_widths_and_gqa_groups(dk, dv, hk, hv):
    """Every value width the ABI takes (multiples of 16: one to sixteen column
    tiles per head), eight value heads on one key head, B = 2 without
    cu_seqlens, a length that is not a multiple of the chunk."""
    q, k, v, g, beta, h0 = generate(2, 300, hk, hv, dk, dv, torch.bfloat16, 0.02, seed=dk + dv + hv)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, h0)
    o, s = run(q, k, v, g, beta, dk ** -0.5, h0)
    assert_parity(f"K={dk} V={dv} {hk}->{hv}", o, o_ref, s, s_ref)


def test_varlen_small():
    """8 packed sequences (ragged, one empty, lengths not multiples of 64)."""
    lengths = [700, 64, 0, 1, 1500, 333, 129, 2000]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    q, k, v, g, beta, h0 = generate(1, int(cu[-1]), 16, 32, 128, 128, torch.bfloat16, 0.02, seed=12,
                                    nstates=len(lengths))
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, cu_seqlens=cu)
    o, s = run(q, k, v, g, beta, SCALE, h0, cu)
    assert_parity("varlen small", o, o_ref, s, s_ref)
    assert torch.equal(s[2].cpu(), h0[2])  # the empty sequence returns its initial state


@pytest.mark.parametrize("nseq,hk,hv,dv", [(300, 2, 4, 64), (40, 16, 32, 128)])
def test_many_short_sequences(nseq, hk, hv, dv):
    """Serving-style packing: many short sequences (0 to 150 tokens, some
    empty), each from its own initial state. A workgroup of the scan runs a
    group of sequences back to back (16 groups of ~19 sequences for the small
    heads, one group of all 40 at the Qwen3-Next heads), swapping states at
    every boundary."""
    lengths = torch.randint(0, 151, (nseq,), generator=torch.Generator().manual_seed(nseq)).tolist()
    lengths[3] = 0
    lengths[nseq - 1] = 0
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    q, k, v, g, beta, h0 = generate(1, int(cu[-1]), hk, hv, 128, dv, torch.bfloat16, 0.02, seed=nseq + 1,
                                    nstates=nseq)
    o_ref, s_ref = oracle(q, k, v, g, beta, SCALE, h0, cu_seqlens=cu)
    o, s = run(q, k, v, g, beta, SCALE, h0, cu)
    assert_parity(f"{nseq} short sequences", o, o_ref, s, s_ref)
    for i in (3, nseq - 1):  # empty sequences return their initial states
        assert torch.equal(s[i].cpu(), h0[i])


def test_varlen_full_size_against_the_oracle():
    """The full varlen workload (8 packed sequences, 262,144 tokens, seeded
    per-sequence initial states; the wide scan, 512 of its workgroups): o and
    the final state of every sequence match the oracle's varlen path (one call
    per sequence from its own h0) for key head 0 and its two value heads over
    all 262,144 tokens; and the packed call agrees with one call per sequence
    (the narrow scan) for every head."""
    q, k, v, g, beta, h0, cu = varlen_workload(seed=0)
    o, s = run(q, k, v, g, beta, SCALE, h0, cu)
    bounds = cu.tolist()
    group = v.shape[2] // q.shape[2]
    hq, hv = slice(0, 1), slice(0, group)
    args = [to_np(x[:, :, hq]) for x in (q, k)] + [to_np(x[:, :, hv]) for x in (v, g, beta)]
    o_ref, s_ref = gdn.varlen(*args, SCALE, to_np(h0[:, hv]), np.asarray(bounds))
    o_h, s_h = to_np(o[:, :, hv]), to_np(s[:, hv])
    errs = []
    for n in range(len(bounds) - 1):
        lo, hi = bounds[n], bounds[n + 1]
        errs.append((hi - lo, rel_err(o_h[:, lo:hi], o_ref[:, lo:hi]), rel_err(s_h[n:n + 1], s_ref[n:n + 1])))
    summarize("varlen 8 x ~32K (262,144 tokens), key head 0, per sequence (T: o / S): "
              + ", ".join(f"{t}: {eo:.1e} / {es:.1e}" for t, eo, es in errs))
    for n in range(len(bounds) - 1):
        lo, hi = bounds[n], bounds[n + 1]
        assert_parity(f"varlen sequence {n} (T={hi - lo}), key head 0 vs oracle", o_h[:, lo:hi], o_ref[:, lo:hi],
                      s_h[n:n + 1], s_ref[n:n + 1])
    dq, dk, dv, dg, db, dh = to_dev(q, k, v, g, beta, h0)
    for n in range(len(bounds) - 1):
        lo, hi = bounds[n], bounds[n + 1]
        o_n, s_n = gd.chunk_fwd(dq[:, lo:hi], dk[:, lo:hi], dv[:, lo:hi], dg[:, lo:hi], db[:, lo:hi],
                                SCALE, dh[n:n + 1])
        assert_parity(f"packed vs separate, sequence {n} (T={hi - lo})", o[:, lo:hi], to_np(o_n),
                      s[n:n + 1], to_np(s_n))


def test_streamed_segments_small():
    """16 segments of 1024 tokens, the final state of each fed to the next; the
    output and state after every segment match the oracle's streamed run."""
    seg = 1024
    q, k, v, g, beta, h0 = workload("stream_1m", seed=21, length=16 * seg)
    dq, dk, dv, dg, db = to_dev(q, k, v, g, beta)
    state = h0.to(DEV)
    ref = gdn.streamed(*(to_np(x) for x in (q, k, v, g, beta)), SCALE, to_np(h0), seg)
    for i, (o_ref, s_ref) in enumerate(ref):
        sl = slice(i * seg, (i + 1) * seg)
        o, state = gd.chunk_fwd(dq[:, sl], dk[:, sl], dv[:, sl], dg[:, sl], db[:, sl], SCALE, state)
        torch.cuda.synchronize()
        assert_parity(f"segment {i}", o, o_ref, state, s_ref)


@pytest.mark.parametrize("g_scale", [1.0, 0.01])
def test_streamed_million_tokens_against_the_oracle(g_scale):
    """The million-token stream (16 segments of 65,536 tokens, all 32 heads,
    the final state of each segment fed to the next) against the oracle
    carrying its own state through the same 1,048,576 tokens for key head 0
    and its two value heads: o and the state after every segment, at the
    workload's decay and at g x 0.01 (memory over hundreds of tokens, where
    rounding in the carried state would show first)."""
    nseg, seg = 16, STREAM_SEGMENT
    state = ref_state = None
    errs = []
    for i in range(nseg):
        q, k, v, g, beta, h0 = workload("stream_1m", seed=1000 + i, length=seg, g_scale=g_scale, device=DEV)
        if i == 0:  # the stream's initial state: segment 0's draw
            state, ref_state = h0, to_np(h0[:, :2])
        o, state = gd.chunk_fwd(q, k, v, g, beta, SCALE, state)
        torch.cuda.synchronize()
        args = [to_np(x[:, :, :1]) for x in (q, k)] + [to_np(x[:, :, :2]) for x in (v, g, beta)]
        o_ref, ref_state = gdn.gated_delta_rule(*args, SCALE, ref_state)
        errs.append((rel_err(o[:, :, :2], o_ref), rel_err(state[:, :2], ref_state)))
        if i == nseg - 1:
            summarize(f"stream 16 x 65,536, g x {g_scale}, key head 0, per segment (o / S): "
                      + ", ".join(f"{eo:.1e} / {es:.1e}" for eo, es in errs))
        assert_parity(f"g x {g_scale}: segment {i}, key head 0 vs oracle", o[:, :, :2], o_ref, state[:, :2],
                      ref_state)
        del q, k, v, g, beta, o


def test_streamed_million_tokens_equals_one_pass():
    """1,048,576 tokens as 16 x 65,536 segments with state carry equal one pass
    over all tokens bit for bit. Inputs are drawn on the device (16 GiB of them)."""
    nseg, seg = 16, STREAM_SEGMENT
    segments = [workload("stream_1m", seed=1000 + i, length=seg, device=DEV) for i in range(nseg)]
    h0 = segments[0][5]
    state = h0
    last_rows = []
    for q, k, v, g, beta, _ in segments:
        o_b, state = gd.chunk_fwd(q, k, v, g, beta, SCALE, state)
        last_rows.append(o_b[:, -8:].clone())
    torch.cuda.synchronize()
    # One pass over the concatenation (B=1, T=2^20) reproduces the carried run.
    cat = [torch.cat([s[j] for s in segments], 1) for j in range(5)]
    del segments
    o_all, s_all = gd.chunk_fwd(*cat, SCALE, h0)
    torch.cuda.synchronize()
    assert torch.equal(s_all, state)
    for i in range(nseg):
        end = (i + 1) * seg
        assert torch.equal(o_all[:, end - 8:end], last_rows[i])
