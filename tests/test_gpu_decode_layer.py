"""Parity of the fused decode step (pbgdn_decode_layer_fwd: one token per
sequence through GatedDeltaNetLayer.forward, gated_deltanet.py:415-441) with
the oracle: oracle/layer.py's prologue (conv against the carried tail, SiLU,
L2 norms, gates) -> oracle/gdn.py's sequential recurrence with q, k, v kept
float32 (the reference's sequential path casts nothing) -> the epilogue.

Tolerances (infinity-norm relative error vs the fp32 oracle): hs 1e-4 in
float32 (SiLU on v_exp/v_rcp and a different summation order, ~1e-6 in
practice) and 1e-2 in bf16; a float32 state 1e-4; a bf16 state the oracle's
rounded to bf16 within one unit in the last place; the conv tails exactly
(they are copies of input values)."""
import numpy as np
import pytest
import torch

from oracle import gdn, layer as ol
from pseudobrain_amd.layer import decode_layer_step
from pseudobrain_amd.workloads import to_numpy
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
DT_NAME = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}


def make(batch, slots, heads, dk, vheads, dv, conv, seed, z_dtype=torch.bfloat16, conv_dtype=torch.float32,
         state_dtype=torch.float32, channel_major=False):
    gen = torch.Generator().manual_seed(seed)
    channels = 2 * heads * dk + vheads * dv
    z = torch.randn(batch, channels + vheads * dv + 2 * vheads, generator=gen).to(z_dtype)
    if conv > 1:
        if channel_major:  # vLLM's layout [S, C, conv-1], seen as [S, conv-1, C]
            pool = torch.randn(slots, channels, conv - 1, generator=gen).to(conv_dtype).transpose(1, 2)
        else:
            pool = torch.randn(slots, conv - 1, channels, generator=gen).to(conv_dtype)
    else:
        pool = None
    weight = (torch.rand(channels, conv, generator=gen) * 2 - 1) / conv ** 0.5 if conv else None
    a_log = torch.empty(vheads).uniform_(0, 16, generator=gen).log()
    dt_bias = torch.randn(vheads, generator=gen) - 4
    state = (torch.randn(slots, vheads, dk, dv, generator=gen) * 0.05).to(state_dtype)
    o_norm = torch.rand(dv, generator=gen) + 0.5
    return z, pool, weight, a_log, dt_bias, state, o_norm


def oracle_step(z, pool, weight, a_log, dt_bias, state, o_norm, idx, heads, dk, vheads, dv, l2norm, eps=1e-5):
    """hs, new states and new tails of the sequences whose slot is valid (in idx order)."""
    channels = 2 * heads * dk + vheads * dv
    zn = to_numpy(z.float())[:, None]
    qkv, gate, decay = zn[..., :channels], zn[..., channels:channels + vheads * dv], zn[..., channels + vheads * dv:]
    tail = None if pool is None else to_numpy(pool.float())[idx]
    q, k, v, g, beta, new_tail = ol.layer_prologue(qkv, decay, tail, None if weight is None else to_numpy(weight),
                                                   to_numpy(a_log), to_numpy(dt_bias), heads, dk, vheads, dv, l2norm,
                                                   x_dtype=DT_NAME[z.dtype])
    rq, rk = gdn.repeat_heads(q, vheads), gdn.repeat_heads(k, vheads)
    o, s = gdn.gated_delta_rule(rq, rk, v, g, beta, dk ** -0.5, to_numpy(state.float())[idx], "sequential")
    hs = ol.layer_epilogue(o, gate, to_numpy(o_norm), eps)[:, 0]
    return hs, s, new_tail


def run_and_check(name, args, idx, heads, dk, vheads, dv, l2norm="max", out_dtype=torch.float32):
    z, pool, weight, a_log, dt_bias, state, o_norm = args
    dpool = None if pool is None else pool.to(DEV)
    if pool is not None and not pool.is_contiguous():  # keep the channel-major storage on the device
        dpool = pool.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    dstate = state.to(DEV)
    hs = decode_layer_step(z.to(DEV), dpool, None if weight is None else weight.to(DEV), a_log.to(DEV),
                           dt_bias.to(DEV), dstate, o_norm.to(DEV), heads, dk, vheads, dv,
                           torch.tensor(idx, dtype=torch.int32, device=DEV), l2norm, out_dtype=out_dtype)
    torch.cuda.synchronize()
    live = [b for b, s in enumerate(idx) if 0 <= s < state.shape[0]]
    slots = [idx[b] for b in live]
    rhs, rs, rtail = oracle_step(z[live], pool, weight, a_log, dt_bias, state, o_norm, slots, heads, dk, vheads,
                                 dv, l2norm)
    e_hs = rel_err(hs[live], rhs)
    got_state = dstate.cpu()[slots]
    print(f"[{name}] hs rel_inf={e_hs:.2e} S rel_inf={rel_err(got_state, rs):.2e}", flush=True)
    assert e_hs <= (1e-4 if out_dtype == torch.float32 else 1e-2)
    if state.dtype == torch.float32:
        assert rel_err(got_state, rs) <= 1e-4
    else:
        rounded = gdn.round_bf16(rs.astype(np.float32)) if state.dtype == torch.bfloat16 else \
            gdn.round_fp16(rs.astype(np.float32))
        spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(rs), 1e-38))) - (7 if state.dtype == torch.bfloat16 else 10))
        assert (np.abs(to_numpy(got_state.float()) - rounded) <= spacing + 1e-5 * np.abs(rs).max()).all()
    dead = [b for b in range(len(idx)) if b not in live]
    assert not hs[dead].float().abs().any()
    others = [s for s in range(state.shape[0]) if s not in slots]
    assert torch.equal(dstate.cpu()[others], state[others])
    if pool is not None:
        got_pool = dpool.cpu()
        np.testing.assert_array_equal(to_numpy(got_pool[slots].float()), rtail.astype(np.float32))
        assert torch.equal(got_pool[others], pool[others])
    return hs


def test_decode_step_qwen3next_b64():
    """64 sequences of the Qwen3-Next layer shape (Hk=16, Hv=32, K=V=128,
    conv 4), bf16 projection, fp32 conv pool and state pool of 80 slots,
    permuted slots with one padded (-1) entry."""
    args = make(64, 80, 16, 128, 32, 128, 4, seed=71)
    idx = torch.randperm(80, generator=torch.Generator().manual_seed(72))[:64].tolist()
    idx[5] = -1
    run_and_check("decode layer B=64", args, idx, 16, 128, 32, 128)


def test_decode_step_bf16_pools_channel_major_hf():
    """bf16 state and conv pools, the conv pool stored channel-major (vLLM's
    [S, C, conv-1]), 'hf' L2 mode, bf16 output."""
    args = make(8, 12, 4, 128, 8, 128, 4, seed=73, conv_dtype=torch.bfloat16, state_dtype=torch.bfloat16,
                channel_major=True)
    run_and_check("decode layer bf16 pools", args, [3, 0, 11, 7, 1, 9, 4, 2], 4, 128, 8, 128, "hf",
                  out_dtype=torch.bfloat16)


def test_decode_step_qwen3next_bf16_tail():
    """The Qwen3-Next shape with the conv pool in bf16, row-major, as a
    serving cache holds it (the kernel's bf16 path: typed loads, the tail
    shifted by copying bits; the new tail is checked bit for bit), fp32 state,
    a padded (-1) entry."""
    args = make(64, 70, 16, 128, 32, 128, 4, seed=75, conv_dtype=torch.bfloat16)
    idx = torch.randperm(70, generator=torch.Generator().manual_seed(76))[:64].tolist()
    idx[9] = -1
    run_and_check("decode layer B=64 bf16 tail", args, idx, 16, 128, 32, 128)


@pytest.mark.parametrize("conv", [0, 1, 2])
@pytest.mark.parametrize("dk,dv,heads,vheads", [(64, 64, 2, 2), (64, 128, 2, 8), (128, 64, 4, 8)])
def test_decode_step_shapes(conv, dk, dv, heads, vheads):
    args = make(5, 6, heads, dk, vheads, dv, conv, seed=74 + conv + dk + dv, z_dtype=torch.float32,
                state_dtype=torch.float16 if dk == 64 else torch.float32)
    run_and_check(f"decode layer conv={conv} K={dk} V={dv} {heads}->{vheads}", args, [5, 1, 0, 3, 2], heads, dk,
                  vheads, dv)


def test_decode_steps_chain():
    """Three fused steps in a row (state and tail carried in the pools) equal
    three oracle steps."""
    heads, dk, vheads, dv = 4, 128, 8, 128
    z, pool, weight, a_log, dt_bias, state, o_norm = make(6, 6, heads, dk, vheads, dv, 4, seed=80)
    gen = torch.Generator().manual_seed(81)
    zs = [z] + [torch.randn(z.shape, generator=gen).to(z.dtype) for _ in range(2)]
    idx = [4, 2, 0, 5, 1, 3]
    dpool, dstate = pool.to(DEV), state.to(DEV)
    rpool, rstate = pool.clone(), state.clone()
    didx = torch.tensor(idx, dtype=torch.int32, device=DEV)
    for step, zt in enumerate(zs):
        hs = decode_layer_step(zt.to(DEV), dpool, weight.to(DEV), a_log.to(DEV), dt_bias.to(DEV), dstate,
                               o_norm.to(DEV), heads, dk, vheads, dv, didx)
        rhs, rs, rtail = oracle_step(zt, rpool, weight, a_log, dt_bias, rstate, o_norm, idx, heads, dk, vheads, dv,
                                     "max")
        rstate[idx] = torch.from_numpy(rs.astype(np.float32))
        rpool[idx] = torch.from_numpy(rtail.astype(np.float32))
        torch.cuda.synchronize()
        e = rel_err(hs, rhs)
        print(f"[decode layer chain step {step}] hs rel_inf={e:.2e}", flush=True)
        assert e <= 1e-4
    assert rel_err(dstate.cpu()[idx], to_numpy(rstate[idx])) <= 1e-4
    np.testing.assert_array_equal(to_numpy(dpool.cpu()), to_numpy(rpool))


def test_decode_step_state_policy_sets_cache_bits_only():
    """The fused step under the default (streamed) and the resident state
    policy: hs, the state pool and the conv pool equal bit for bit."""
    heads, dk, vheads, dv = 16, 128, 32, 128
    z, pool, weight, a_log, dt_bias, state, o_norm = make(64, 64, heads, dk, vheads, dv, 4, seed=90)
    dz, dw, da, db, dn = z.to(DEV), weight.to(DEV), a_log.to(DEV), dt_bias.to(DEV), o_norm.to(DEV)
    runs = []
    for resident in (False, True):
        dpool, dstate = pool.to(DEV), state.to(DEV)
        hs = decode_layer_step(dz, dpool, dw, da, db, dstate, dn, heads, dk, vheads, dv, state_resident=resident)
        torch.cuda.synchronize()
        runs.append((hs, dstate, dpool))
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
