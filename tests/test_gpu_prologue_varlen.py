"""Parity of the packed-sequence layer prologue (pbgdn_prologue_varlen_fwd:
N sequences back to back, each convolving against its own conv tail held in a
slot pool, the layout a serving engine's prefill batch uses) with the fp32
oracle run one sequence at a time (oracle/layer.py: layer_prologue, after
pseudobrain/gated_deltanet.py:314-338, :415-429).

Tolerances as for the single-sequence prologue (infinity-norm relative error):
outputs rounded to bf16/fp16 1e-2, float32 outputs 1e-5, gates 1e-5; the new
tails are copies of input values and must match exactly (rounded to the
pool's dtype, which keeps them), and slots no sequence names must be left
untouched."""
import numpy as np
import pytest
import torch

from oracle import layer as ol
from pseudobrain_amd.layer import layer_prologue_varlen
from pseudobrain_amd.workloads import cu_seqlens_of, to_numpy
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
LOW_TOL = 1e-2
F32_TOL = 1e-5
DT_NAME = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}


def run_case(name, lengths, heads, dk, vheads, dv, conv, seed, dtype=torch.bfloat16, tail_dtype=torch.float32,
             out_dtype=None, l2norm="max", extra_slots=3, invalid=(), no_initial=(), channel_major=False,
             separate_out=False, padded_rows=False):
    gen = torch.Generator().manual_seed(seed)
    channels = 2 * heads * dk + vheads * dv
    nseq = len(lengths)
    total = sum(lengths)
    z = torch.randn(total, channels + vheads * dv + 2 * vheads, generator=gen).to(dtype)
    nslots = nseq + extra_slots
    pool = None
    if conv > 1:
        if channel_major:  # [S, C, conv-1] storage seen as [S, conv-1, C]
            pool = torch.randn(nslots, channels, conv - 1, generator=gen).to(tail_dtype).transpose(1, 2)
        else:
            pool = torch.randn(nslots, conv - 1, channels, generator=gen).to(tail_dtype)
    weight = (torch.rand(channels, conv, generator=gen) * 2 - 1) / conv ** 0.5 if conv else None
    a_log = torch.empty(vheads).uniform_(0, 16, generator=gen).log()
    dt_bias = torch.randn(vheads, generator=gen) - 4
    slots = torch.randperm(nslots, generator=gen)[:nseq].tolist()
    for i in invalid:
        slots[i] = -1 if i % 2 == 0 else nslots + i
    has_init = [i not in no_initial for i in range(nseq)]
    cu = cu_seqlens_of(lengths)
    print(f"[{name}] lengths={lengths} slots={slots}", flush=True)

    dpool = store = None
    if pool is not None:
        dpool = pool.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) if channel_major else pool.to(DEV)
        if padded_rows:  # rows 3 elements apart from a multiple of 8: no whole-vector access
            store = torch.full((nslots, conv - 1, channels + 3), 5.0, dtype=tail_dtype, device=DEV)
            store[..., :channels] = dpool
            dpool = store[..., :channels]
    dout = None
    if separate_out and pool is not None:
        dout = torch.full_like(dpool, 7.0)
    q, k, v, g, beta, gate = layer_prologue_varlen(
        z.to(DEV), cu.to(DEV), dpool, None if weight is None else weight.to(DEV), a_log.to(DEV), dt_bias.to(DEV),
        heads, dk, vheads, dv, torch.tensor(slots, dtype=torch.int32, device=DEV),
        torch.tensor(has_init, device=DEV), l2norm, out_dtype=out_dtype, tail_out=dout)
    torch.cuda.synchronize()
    assert q.shape == (1, total, heads, dk) and v.shape == (1, total, vheads, dv)
    assert gate.shape == (1, total, vheads * dv)

    zn = to_numpy(z.float())
    tol = F32_TOL if q.dtype == torch.float32 else LOW_TOL
    written = {}
    for s, (lo, hi) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        valid = 0 <= slots[s] < nslots
        tail = None
        if conv > 1:
            tail = (to_numpy(pool[slots[s]].float()) if valid and has_init[s]
                    else np.zeros((conv - 1, channels), np.float32))[None]
        seg = zn[None, lo:hi]
        rq, rk, rv, rg, rb, rt = ol.layer_prologue(
            seg[..., :channels], seg[..., channels + vheads * dv:], tail,
            None if weight is None else to_numpy(weight), to_numpy(a_log), to_numpy(dt_bias), heads, dk, vheads, dv,
            l2norm, x_dtype=DT_NAME[dtype])
        if hi > lo:
            errs = {"q": rel_err(q[:, lo:hi], rq), "k": rel_err(k[:, lo:hi], rk), "v": rel_err(v[:, lo:hi], rv),
                    "g": rel_err(g[:, lo:hi], rg), "beta": rel_err(beta[:, lo:hi], rb)}
            for n in ("q", "k", "v"):
                assert errs[n] <= tol, f"{name} seq {s}: {n} error {errs[n]:.3e} > {tol}"
            for n in ("g", "beta"):
                assert errs[n] <= F32_TOL, f"{name} seq {s}: {n} error {errs[n]:.3e}"
        if conv > 1 and valid:
            written[slots[s]] = rt[0]
    if padded_rows:
        assert store[..., channels:].eq(5.0).all(), f"{name}: the padding between pool rows changed"
    if conv > 1:
        got = (dout if dout is not None else dpool).cpu()
        for slot, rt in written.items():
            # the pool keeps the new tail in its own dtype
            want = ol.round_to(rt.astype(np.float32), DT_NAME[tail_dtype])
            np.testing.assert_array_equal(to_numpy(got[slot].float()), want, err_msg=f"{name}: tail of slot {slot}")
        others = [i for i in range(nslots) if i not in written]
        expect = torch.full_like(pool, 7.0) if dout is not None else pool
        assert torch.equal(got[others], expect[others]), f"{name}: a slot no sequence names changed"


def test_varlen_qwen3next_serving_batch():
    """The Qwen3-Next layer shape (Hk=16, Hv=32, K=V=128, conv 4), a bf16
    projection of 12 packed sequences (with empty and one- to three-token
    sequences shorter than the tail), an fp32 tail pool updated in place."""
    run_case("varlen qwen3next", [300, 0, 1, 2, 3, 64, 65, 129, 5, 700, 17, 1], 16, 128, 32, 128, 4, seed=1,
             no_initial=(4, 9))


@pytest.mark.parametrize("conv", [0, 1, 2, 3, 4])
def test_varlen_conv_widths(conv):
    run_case(f"varlen conv={conv}", [0, 1, 2, 3, 40, 77], 2, 64, 4, 64, conv, seed=10 + conv,
             dtype=torch.float32, no_initial=(3,))


def test_varlen_invalid_slots_and_new_sequences():
    """Padded (-1) and out-of-pool slots start from a zero tail and write
    nothing; sequences without an initial state start from zeros and still
    write their new tail."""
    run_case("varlen invalid slots", [9, 1, 30, 2, 0, 66], 2, 128, 4, 64, 4, seed=20, invalid=(0, 3, 4),
             no_initial=(1, 5))


def test_varlen_channel_major_bf16_pool_hf():
    """vLLM's channel-major [S, C, conv-1] conv-state pool in bf16, 'hf' L2
    mode, fp16 projection with float32 outputs."""
    run_case("varlen channel-major", [2, 130, 1, 45], 4, 128, 8, 128, 4, seed=30, dtype=torch.float16,
             tail_dtype=torch.bfloat16, out_dtype=torch.float32, l2norm="hf", channel_major=True)


def test_varlen_pool_with_padded_rows():
    """A pool whose rows are not whole 8-element vectors apart (a view into
    wider storage) goes element by element and leaves the padding alone."""
    run_case("varlen padded pool rows", [4, 0, 90, 1, 2], 2, 64, 4, 64, 4, seed=35, padded_rows=True,
             no_initial=(2,), invalid=(4,))


@pytest.mark.parametrize("dtype,tail_dtype,out_dtype", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32, torch.bfloat16),
    (torch.float16, torch.float32, torch.float16)])
def test_varlen_dtypes_separate_output_pool(dtype, tail_dtype, out_dtype):
    run_case(f"varlen {dtype} tail {tail_dtype} out {out_dtype}", [3, 1, 200, 0, 31], 2, 128, 4, 128, 4,
             seed=40, dtype=dtype, tail_dtype=tail_dtype, out_dtype=out_dtype, separate_out=True)


def test_varlen_matches_batched_prologue_on_equal_lengths():
    """Sequences of equal length through the packed path equal the batched
    single-call prologue of the same inputs (same kernels' arithmetic), so the
    two entry points agree bit for bit."""
    from pseudobrain_amd.layer import layer_prologue
    heads, dk, vheads, dv, conv, batch, length = 4, 128, 8, 128, 4, 3, 150
    gen = torch.Generator().manual_seed(50)
    channels = 2 * heads * dk + vheads * dv
    z = torch.randn(batch, length, channels + vheads * dv + 2 * vheads, generator=gen).to(torch.bfloat16).to(DEV)
    tail = torch.randn(batch, conv - 1, channels, generator=gen).to(DEV)
    weight = ((torch.rand(channels, conv, generator=gen) * 2 - 1) / 2).to(DEV)
    a_log = torch.empty(vheads).uniform_(0, 16, generator=gen).log().to(DEV)
    dt_bias = (torch.randn(vheads, generator=gen) - 4).to(DEV)
    ref = layer_prologue(z, tail.clone(), weight, a_log, dt_bias, heads, dk, vheads, dv)
    pool = tail.clone()
    got = layer_prologue_varlen(z.reshape(batch * length, -1), cu_seqlens_of([length] * batch).to(DEV), pool,
                                weight, a_log, dt_bias, heads, dk, vheads, dv)
    torch.cuda.synchronize()
    for a, b in zip(ref[:5], got[:5]):
        assert torch.equal(a.reshape(b.shape), b)
    assert torch.equal(ref[6], pool)
