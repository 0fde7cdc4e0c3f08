"""Parity of the fused layer prologue and epilogue kernels with the fp32 oracle
(oracle/layer.py: short_convolution, l2_normalize, the gates and the
epilogue of pseudobrain/gated_deltanet.py:314-338, :415-441).

Tolerances (infinity-norm relative error vs the fp32 oracle on the same
input values): outputs rounded to bf16/fp16 1e-2 (a few units of the output
format's rounding), float32 outputs 1e-5; the new tail is a copy of input
values and must match exactly."""
import numpy as np
import pytest
import torch

from oracle import gdn, layer as ol
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.layer import layer_epilogue, layer_prologue
from pseudobrain_amd.workloads import to_numpy
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
LOW_TOL = 1e-2
F32_TOL = 1e-5
DT_NAME = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}


def make_layer_inputs(batch, length, heads, dk, vheads, dv, conv, dtype, seed, tail_dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    channels = 2 * heads * dk + vheads * dv
    z = torch.randn(batch, length, channels + vheads * dv + 2 * vheads, generator=gen).to(dtype)
    tail = (torch.randn(batch, max(conv - 1, 0), channels, generator=gen).to(tail_dtype) if conv > 1 else None)
    weight = (torch.rand(channels, conv, generator=gen) * 2 - 1) / conv ** 0.5 if conv else None
    a_log = torch.empty(vheads).uniform_(0, 16, generator=gen).log()
    dt_bias = torch.randn(vheads, generator=gen) - 4
    return z, tail, weight, a_log, dt_bias


def oracle_prologue(z, tail, weight, a_log, dt_bias, heads, dk, vheads, dv, l2norm):
    channels = 2 * heads * dk + vheads * dv
    zn = to_numpy(z.float())
    qkv, decay = zn[..., :channels], zn[..., channels + vheads * dv:]
    tn = None if tail is None else to_numpy(tail.float())
    wn = None if weight is None else to_numpy(weight)
    return ol.layer_prologue(qkv, decay, tn, wn, to_numpy(a_log), to_numpy(dt_bias), heads, dk, vheads, dv,
                             l2norm, x_dtype=DT_NAME[z.dtype])


def check_prologue(name, z, tail, weight, a_log, dt_bias, heads, dk, vheads, dv, l2norm="max", out_dtype=None):
    dev = [None if x is None else x.to(DEV) for x in (z, tail, weight, a_log, dt_bias)]
    q, k, v, g, beta, gate, new_tail = layer_prologue(*dev, heads, dk, vheads, dv, l2norm, out_dtype=out_dtype)
    torch.cuda.synchronize()
    rq, rk, rv, rg, rb, rt = oracle_prologue(z, tail, weight, a_log, dt_bias, heads, dk, vheads, dv, l2norm)
    tol = F32_TOL if q.dtype == torch.float32 else LOW_TOL
    errs = {"q": rel_err(q, rq), "k": rel_err(k, rk), "v": rel_err(v, rv), "g": rel_err(g, rg),
            "beta": rel_err(beta, rb)}
    print(f"[{name}] " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n in ("q", "k", "v"):
        assert errs[n] <= tol, f"{name}: {n} error {errs[n]:.3e} > {tol}"
    for n in ("g", "beta"):
        assert errs[n] <= F32_TOL, f"{name}: {n} error {errs[n]:.3e} > {F32_TOL}"
    if tail is not None:
        np.testing.assert_array_equal(to_numpy(new_tail.float()), rt.astype(np.float32))
        assert new_tail.dtype == tail.dtype
    assert gate.shape == (z.shape[0], z.shape[1], vheads * dv)
    return q, k, v, g, beta, gate, new_tail


@pytest.mark.parametrize("l2norm", ["max", "hf"])
def test_prologue_qwen3next_shape(l2norm):
    """Hk=16, Hv=32, K=V=128, conv 4, bf16 projection, fp32 tail."""
    args = make_layer_inputs(1, 1000, 16, 128, 32, 128, 4, torch.bfloat16, seed=1)
    check_prologue(f"prologue qwen3next {l2norm}", *args, 16, 128, 32, 128, l2norm)


@pytest.mark.parametrize("conv", [0, 1, 2, 3, 4])
def test_prologue_conv_widths(conv):
    args = make_layer_inputs(2, 77, 2, 128, 4, 64, conv, torch.bfloat16, seed=2 + conv)
    check_prologue(f"prologue conv={conv}", *args, 2, 128, 4, 64)


@pytest.mark.parametrize("length", [1, 2, 3, 129])
def test_prologue_short_inputs_keep_part_of_the_tail(length):
    """T < conv-1: the new tail is the old tail's last rows followed by the inputs."""
    args = make_layer_inputs(3, length, 1, 64, 2, 128, 4, torch.float32, seed=10 + length)
    check_prologue(f"prologue T={length}", *args, 1, 64, 2, 128, "hf")


@pytest.mark.parametrize("dtype,tail_dtype,out_dtype", [
    (torch.float32, torch.float32, None),
    (torch.float16, torch.float32, None),
    (torch.bfloat16, torch.bfloat16, torch.float32),
])
def test_prologue_dtypes(dtype, tail_dtype, out_dtype):
    args = make_layer_inputs(2, 200, 4, 64, 8, 128, 4, dtype, seed=20, tail_dtype=tail_dtype)
    check_prologue(f"prologue {dtype} tail {tail_dtype} out {out_dtype}", *args, 4, 64, 8, 128,
                   out_dtype=out_dtype)


def test_prologue_segments_equal_one_pass():
    """Two calls with the tail carried equal one call, bit for bit."""
    z, tail, w, a_log, dtb = [None if x is None else x.to(DEV)
                              for x in make_layer_inputs(2, 500, 16, 128, 32, 128, 4, torch.bfloat16, seed=30)]
    whole = layer_prologue(z, tail, w, a_log, dtb, 16, 128, 32, 128)
    first = layer_prologue(z[:, :321], tail, w, a_log, dtb, 16, 128, 32, 128)
    second = layer_prologue(z[:, 321:], first[6], w, a_log, dtb, 16, 128, 32, 128)
    for i in range(5):
        assert torch.equal(torch.cat([first[i], second[i]], dim=1), whole[i]), i
    assert torch.equal(second[6], whole[6])


@pytest.mark.parametrize("length", [1, 2, 200])
def test_prologue_tail_in_place(length):
    """tail_out = tail: the tail is updated in place and every output equals
    the call with a separate new tail, bit for bit (short inputs keep part of
    the old tail)."""
    z, tail, w, a_log, dtb = [None if x is None else x.to(DEV)
                              for x in make_layer_inputs(3, length, 4, 128, 8, 128, 4, torch.bfloat16, seed=31)]
    ref = layer_prologue(z, tail, w, a_log, dtb, 4, 128, 8, 128)
    pool = tail.clone()
    got = layer_prologue(z, pool, w, a_log, dtb, 4, 128, 8, 128, tail_out=pool)
    torch.cuda.synchronize()
    for i in range(5):
        assert torch.equal(got[i], ref[i]), i
    assert got[6] is pool and torch.equal(pool, ref[6])


@pytest.mark.parametrize("dv,o_dtype,gate_dtype,out_dtype", [
    (128, torch.bfloat16, torch.bfloat16, torch.float32),
    (128, torch.float32, torch.bfloat16, torch.bfloat16),
    (64, torch.float16, torch.float32, torch.float32),
])
def test_epilogue(dv, o_dtype, gate_dtype, out_dtype):
    gen = torch.Generator().manual_seed(40 + dv)
    batch, length, hv = 2, 300, 8
    o = (torch.randn(batch, length, hv, dv, generator=gen) * 0.3).to(o_dtype)
    z = torch.randn(batch, length, 3 * hv * dv, generator=gen).to(gate_dtype)
    gate = z[..., hv * dv:2 * hv * dv]  # a strided column slice, as in the layer
    o_norm = torch.rand(dv, generator=gen) + 0.5
    out = layer_epilogue(o.to(DEV), gate.to(DEV), o_norm.to(DEV), 1e-5, out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = ol.layer_epilogue(to_numpy(o.float()), to_numpy(gate.float()), to_numpy(o_norm), 1e-5)
    err = rel_err(out, ref)
    tol = F32_TOL if out_dtype == torch.float32 else LOW_TOL
    print(f"[epilogue dv={dv} {o_dtype} {gate_dtype} -> {out_dtype}] rel_inf={err:.2e}", flush=True)
    assert out.shape == (batch, length, hv * dv) and out.dtype == out_dtype
    assert err <= tol


def test_epilogue_streamed_matches_cached():
    """A call moving more than 192 MiB (8,192 tokens x 32 heads x 128: 256 MiB
    of o, gate and output) streams with non-temporal hints; its halves, below
    that size, keep the cacheable path. Same arithmetic: equal bit for bit,
    and within the tolerance of the oracle."""
    gen = torch.Generator().manual_seed(44)
    length, hv, dv = 8192, 32, 128
    o = (torch.randn(1, length, hv, dv, generator=gen) * 0.3).to(torch.bfloat16)
    z = torch.randn(1, length, 2 * hv * dv, generator=gen).to(torch.bfloat16)
    gate = z[..., hv * dv:]
    o_norm = torch.rand(dv, generator=gen) + 0.5
    do, dz, dn = o.to(DEV), z.to(DEV), o_norm.to(DEV)
    whole = layer_epilogue(do, dz[..., hv * dv:], dn, 1e-5, out_dtype=torch.float32)
    halves = torch.cat([layer_epilogue(do[:, s], dz[:, s].contiguous()[..., hv * dv:], dn, 1e-5,
                                       out_dtype=torch.float32)
                        for s in (slice(0, length // 2), slice(length // 2, length))], dim=1)
    torch.cuda.synchronize()
    assert torch.equal(whole, halves)
    ref = ol.layer_epilogue(to_numpy(o.float()), to_numpy(gate.float()), to_numpy(o_norm), 1e-5)
    err = rel_err(whole, ref)
    print(f"[epilogue streamed T={length}] rel_inf={err:.2e}", flush=True)
    assert err <= F32_TOL


def test_prologue_past_2gib_equals_two_calls():
    """98,304 tokens of the Qwen3-Next projection (24,704 bytes a row: 2.4 GB,
    past 32-bit byte offsets from the sequence's start) in one call equal two
    calls with the tail carried, bit for bit; its last tokens match the oracle
    run on them with the rows before them as the tail."""
    heads, dk, vheads, dv, conv = 16, 128, 32, 128, 4
    length = 98304
    channels = 2 * heads * dk + vheads * dv
    gen = torch.Generator(device=DEV).manual_seed(60)
    z = torch.randn(1, length, channels + vheads * dv + 2 * vheads, device=DEV, generator=gen).to(torch.bfloat16)
    assert z.shape[1] * z.stride(1) * 2 > 2 ** 31
    _, tail, w, a_log, dtb = make_layer_inputs(1, 1, heads, dk, vheads, dv, conv, torch.bfloat16, seed=61)
    tail, w, a_log, dtb = [x.to(DEV) for x in (tail, w, a_log, dtb)]
    whole = layer_prologue(z, tail, w, a_log, dtb, heads, dk, vheads, dv)
    half = length // 2
    first = layer_prologue(z[:, :half], tail, w, a_log, dtb, heads, dk, vheads, dv)
    second = layer_prologue(z[:, half:], first[6], w, a_log, dtb, heads, dk, vheads, dv)
    torch.cuda.synchronize()
    for i in range(5):
        assert torch.equal(torch.cat([first[i], second[i]], dim=1), whole[i]), i
    assert torch.equal(second[6], whole[6])
    last = 8
    zs = z[:, length - last:].cpu()
    ts = z[:, length - last - (conv - 1):length - last, :channels].float().cpu()
    rq, rk, rv, rg, rb, rt = oracle_prologue(zs, ts, w.cpu(), a_log.cpu(), dtb.cpu(), heads, dk, vheads, dv, "max")
    got = [x[:, length - last:] for x in whole[:5]]
    errs = [rel_err(g_, r_) for g_, r_ in zip(got, (rq, rk, rv, rg, rb))]
    print(f"[prologue T={length}] last tokens " + " ".join(f"{e:.2e}" for e in errs), flush=True)
    assert max(errs[:3]) <= LOW_TOL and max(errs[3:]) <= F32_TOL
    np.testing.assert_array_equal(to_numpy(whole[6].float()), rt.astype(np.float32))


def test_epilogue_past_2gib_equals_two_calls():
    """270,336 tokens x 32 heads x 128 (o 2.2 GB in bf16, past 32-bit byte
    offsets from its start) in one call equal two calls, bit for bit; the last
    rows match the oracle."""
    length, hv, dv = 270336, 32, 128
    gen = torch.Generator(device=DEV).manual_seed(62)
    o = (torch.randn(1, length, hv, dv, device=DEV, generator=gen) * 0.3).to(torch.bfloat16)
    gate = torch.randn(1, length, hv * dv, device=DEV, generator=gen).to(torch.bfloat16)
    o_norm = torch.rand(dv, device=DEV, generator=gen) + 0.5
    assert o.numel() * 2 > 2 ** 31
    whole = layer_epilogue(o, gate, o_norm, 1e-5, out_dtype=torch.float32)
    half = length // 2
    parts = torch.cat([layer_epilogue(o[:, :half], gate[:, :half], o_norm, 1e-5, out_dtype=torch.float32),
                       layer_epilogue(o[:, half:], gate[:, half:], o_norm, 1e-5, out_dtype=torch.float32)], dim=1)
    torch.cuda.synchronize()
    assert torch.equal(whole, parts)
    del parts
    last = 16
    ref = ol.layer_epilogue(to_numpy(o[:, length - last:].float()), to_numpy(gate[:, length - last:].float()),
                            to_numpy(o_norm), 1e-5)
    err = rel_err(whole[:, length - last:], ref)
    print(f"[epilogue T={length}] last rows rel_inf={err:.2e}", flush=True)
    assert err <= F32_TOL


def test_layer_prologue_operator_epilogue_against_the_oracle():
    """The whole GatedDeltaNetLayer core (gated_deltanet.py:415-441) at the
    Qwen3-Next head shape: fused prologue -> chunk operator -> fused epilogue
    against prologue -> delta_rule_chunked -> epilogue of the oracle."""
    heads, dk, vheads, dv = 16, 128, 32, 128
    z, tail, w, a_log, dtb = make_layer_inputs(1, 600, heads, dk, vheads, dv, 4, torch.bfloat16, seed=50)
    o_norm = torch.rand(dv, generator=torch.Generator().manual_seed(51)) + 0.5
    h0 = torch.randn(1, vheads, dk, dv, generator=torch.Generator().manual_seed(52)) * 0.02
    dz, dtail, dw, da, ddt, dn, dh = [x.to(DEV) for x in (z, tail, w, a_log, dtb, o_norm, h0)]
    q, k, v, g, beta, gate, new_tail = layer_prologue(dz, dtail, dw, da, ddt, heads, dk, vheads, dv)
    o, s = gd.gated_delta_rule(q, k, v, g, beta, dk ** -0.5, dh, kernel="hip")
    hs = layer_epilogue(o, gate, dn)
    torch.cuda.synchronize()
    rq, rk, rv, rg, rb, _ = oracle_prologue(z, tail, w, a_log, dtb, heads, dk, vheads, dv, "max")
    # the operator reads q, k, v at the projection's precision (bf16), as the reference's fla path does
    rq, rk, rv = (gdn.round_bf16(x.astype(np.float32)) for x in (rq, rk, rv))
    rq, rk = gdn.repeat_heads(rq, vheads), gdn.repeat_heads(rk, vheads)
    ro, rs = gdn.gated_delta_rule(rq, rk, rv, rg, rb, dk ** -0.5, to_numpy(h0), "chunked")
    rhs = ol.layer_epilogue(ro, to_numpy(gate.float()), to_numpy(o_norm))
    e_hs, e_s = rel_err(hs, rhs), rel_err(s, rs)
    print(f"[layer core T=600] hs rel_inf={e_hs:.2e} S rel_inf={e_s:.2e}", flush=True)
    assert e_hs <= 2e-2 and e_s <= 1e-3
