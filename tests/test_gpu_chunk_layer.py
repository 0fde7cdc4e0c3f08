"""Parity of the prefill layer core, chunk_layer_fwd (pbgdn_chunk_layer_fwd:
the operator followed by the RMSNorm x o_norm x SiLU(gate) epilogue of
gated_deltanet.py:437-441), with the fp32 oracle: gdn.gated_delta_rule (or
gdn.varlen) for o and the final states, then oracle/layer.py's
layer_epilogue on that o.

Shapes that the wide scan takes (16-bit inputs, K = V = 128, at least 128
(sequence, value head) pairs) run the epilogue inside the scan; the others
(one or a few long sequences on the narrow scan, chained short sequences,
V = 64, a gate in another dtype) write o and run the epilogue kernel after
it. Tolerances: hs 2e-2 and final states 1e-3 (infinity-norm relative error
against the oracle), as the operator's outputs."""
import numpy as np
import pytest
import torch

from oracle import layer as ol
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.layer import chunk_layer_fwd, chunk_layer_fwd_slots, layer_epilogue
from pseudobrain_amd.workloads import cu_seqlens_of, generate, to_numpy
from tests.gpu_util import O_TOL, S_TOL, oracle, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-5


def layer_case(batch, length, hk, hv, dv, dtype, seed, *, gate_dtype=None, nstates=None, v_scale=1.0):
    q, k, v, g, beta, h0 = generate(batch, length, hk, hv, 128, dv, dtype, 0.02, seed=seed, nstates=nstates)
    if v_scale != 1.0:
        v = (v.float() * v_scale).to(dtype)
    gen = torch.Generator().manual_seed(seed + 1)
    # the gate as the layer has it: a column slice of the projection
    z = torch.randn(batch, length, 3 * hv * dv, generator=gen).to(gate_dtype or dtype)
    gate = z[..., hv * dv:2 * hv * dv]
    o_norm = torch.rand(dv, generator=gen) + 0.5
    return q, k, v, g, beta, h0, gate, o_norm


def check(name, case, cu=None, out_dtype=torch.float32):
    q, k, v, g, beta, h0, gate, o_norm = case
    dev = [x.to(DEV) for x in (q, k, v, g, beta, h0, gate, o_norm)]
    with torch.no_grad():
        hs, s = chunk_layer_fwd(*dev[:5], 128 ** -0.5, dev[5], dev[6], dev[7], EPS,
                                None if cu is None else cu.to(DEV), out_dtype=out_dtype)
    torch.cuda.synchronize()
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, h0, cu_seqlens=cu)
    hs_ref = ol.layer_epilogue(o_ref, to_numpy(gate.float()), to_numpy(o_norm), EPS)
    e_hs, e_s = rel_err(hs, hs_ref.reshape(hs.shape)), rel_err(s, s_ref)
    print(f"[{name}] hs rel_inf={e_hs:.2e} S rel_inf={e_s:.2e}", flush=True)
    assert hs.dtype == out_dtype and hs.shape == gate.shape
    assert np.isfinite(e_hs) and e_hs <= O_TOL, f"{name}: hs error {e_hs:.3e}"
    assert np.isfinite(e_s) and e_s <= S_TOL, f"{name}: state error {e_s:.3e}"
    return hs, s


@pytest.mark.parametrize("batch,length,hk,dtype,out_dtype", [
    (4, 300, 16, torch.bfloat16, torch.float32),   # Qwen3-Next heads, a padded last chunk
    (4, 300, 16, torch.bfloat16, torch.bfloat16),  # hs in the inputs' dtype
    (4, 130, 32, torch.float16, torch.float16),    # no GQA, fp16
    (4, 130, 32, torch.float16, torch.float32),
    (8, 1, 16, torch.bfloat16, torch.float32),     # one token
])
def test_fused_in_the_wide_scan(batch, length, hk, dtype, out_dtype):
    check(f"fused B={batch} T={length} Hk={hk} {dtype}->{out_dtype}",
          layer_case(batch, length, hk, 32, 128, dtype, seed=length + hk), out_dtype=out_dtype)


def test_fused_packed_sequences_with_empty_and_ragged_lengths():
    lengths = [200, 0, 1, 63, 64, 65, 129, 10]
    case = layer_case(1, sum(lengths), 16, 32, 128, torch.bfloat16, seed=7, nstates=len(lengths))
    hs, s = check("fused packed", case, cu=cu_seqlens_of(lengths))
    assert torch.equal(s[1].cpu(), case[5][1])  # the empty sequence keeps its initial state


def test_fused_with_range_scaled_chunks():
    """v x 1000 in bf16: chunks whose V - gamma K S leaves the fp16 range are
    scaled inside the scan; the epilogue sees the restored O."""
    check("fused v x 1e3", layer_case(4, 200, 16, 32, 128, torch.bfloat16, seed=5, v_scale=1e3))


def test_fused_matches_operator_then_epilogue():
    """The fused call against gated_delta_rule's output (rounded to bf16) run
    through layer_epilogue: equal up to that rounding of o."""
    q, k, v, g, beta, h0, gate, o_norm = [x.to(DEV) for x in layer_case(4, 500, 16, 32, 128, torch.bfloat16, 9)]
    with torch.no_grad():
        hs, s = chunk_layer_fwd(q, k, v, g, beta, 128 ** -0.5, h0, gate, o_norm, EPS)
        o, s2 = gd.chunk_fwd(q, k, v, g, beta, 128 ** -0.5, h0)
        hs2 = layer_epilogue(o, gate, o_norm, EPS)
    torch.cuda.synchronize()
    assert torch.equal(s, s2)  # the state path is the same kernel
    err = rel_err(hs, to_numpy(hs2.float()))
    print(f"[fused vs two passes] rel_inf={err:.2e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("batch,length,dtype,out_dtype", [
    (1, 1000, torch.bfloat16, torch.float32),   # one sequence, a padded last chunk
    (1, 1000, torch.bfloat16, torch.bfloat16),  # hs in the inputs' dtype
    (1, 640, torch.float16, torch.float16),     # fp16, whole chunks
    (1, 640, torch.float16, torch.float32),
    (1, 1, torch.bfloat16, torch.float32),      # one token
    (2, 2100, torch.bfloat16, torch.float32),   # two sequences, a workgroup each
])
def test_narrow_scan_then_epilogue(batch, length, dtype, out_dtype):
    check(f"narrow scan + epilogue B={batch} T={length} {dtype}->{out_dtype}",
          layer_case(batch, length, 16, 32, 128, dtype, seed=length + batch), out_dtype=out_dtype)


def test_narrow_scan_then_epilogue_with_range_scaled_chunks():
    check("narrow scan + epilogue v x 1e3", layer_case(1, 500, 16, 32, 128, torch.bfloat16, seed=6, v_scale=1e3))


def test_narrow_scan_layer_call_is_operator_then_epilogue():
    """One sequence: chunk_layer_fwd runs the same two kernels as chunk_fwd
    followed by layer_epilogue, so hs and the final states are equal bit for
    bit."""
    q, k, v, g, beta, h0, gate, o_norm = [x.to(DEV) for x in layer_case(1, 3000, 16, 32, 128, torch.bfloat16, 19)]
    with torch.no_grad():
        hs, s = chunk_layer_fwd(q, k, v, g, beta, 128 ** -0.5, h0, gate, o_norm, EPS)
        o, s2 = gd.chunk_fwd(q, k, v, g, beta, 128 ** -0.5, h0)
        hs2 = layer_epilogue(o, gate, o_norm, EPS)
    torch.cuda.synchronize()
    assert torch.equal(s, s2)
    assert torch.equal(hs, hs2)


@pytest.mark.parametrize("batch,length,dv,gate_dtype", [
    (4, 200, 64, None),                 # V = 64
    (4, 200, 128, torch.float32),       # a float32 gate with bf16 operator inputs
    (1, 700, 128, None),                # chained sequences (cu_seqlens below): o, then the epilogue kernel
])
def test_two_pass_shapes(batch, length, dv, gate_dtype):
    cu = cu_seqlens_of([300, 0, 400]) if length == 700 else None  # too few for the wide scan, one group
    check(f"two-pass B={batch} T={length} V={dv} gate={gate_dtype}",
          layer_case(batch, length, 16, 32, dv, torch.bfloat16, seed=length + dv, gate_dtype=gate_dtype,
                     nstates=None if cu is None else 3), cu=cu)


def test_float32_inputs():
    """float32 q, k, v go through chunk_fwd's range scaling and layer_epilogue."""
    check("fp32 inputs", layer_case(2, 150, 16, 32, 128, torch.float32, seed=12, v_scale=1e4))


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
def test_fused_with_state_slots(state_dtype):
    """chunk_layer_fwd_slots: sequences start from their slots of a pool (a new
    request without an initial state, a -1 slot) and write their final states
    back in the pool's dtype; the other slots keep their contents."""
    lengths = [100, 70, 0, 150]
    n = len(lengths)
    q, k, v, g, beta, _, gate, o_norm = layer_case(1, sum(lengths), 16, 32, 128, torch.bfloat16, 21, nstates=n)
    pool = (torch.randn(9, 32, 128, 128, generator=torch.Generator().manual_seed(22)) * 0.02).to(state_dtype)
    slots = torch.tensor([5, 0, 7, -1], dtype=torch.int32)
    has_init = torch.tensor([1, 0, 1, 1], dtype=torch.uint8)
    cu = cu_seqlens_of(lengths)
    dpool = pool.to(DEV)
    dev = [x.to(DEV) for x in (q, k, v, g, beta, gate, o_norm)]
    with torch.no_grad():
        hs = chunk_layer_fwd_slots(*dev[:5], 128 ** -0.5, dpool, slots.to(DEV), dev[5], dev[6], EPS, cu.to(DEV),
                                   has_init.to(DEV))
    torch.cuda.synchronize()
    init = torch.stack([pool[5].float(), torch.zeros(32, 128, 128), pool[7].float(), torch.zeros(32, 128, 128)])
    o_ref, s_ref = oracle(q, k, v, g, beta, 128 ** -0.5, init, cu_seqlens=cu)
    hs_ref = ol.layer_epilogue(o_ref, to_numpy(gate.float()), to_numpy(o_norm), EPS)
    got = dpool.cpu().float()
    e_hs, e_s = rel_err(hs, hs_ref.reshape(hs.shape)), rel_err(got[[5, 0, 7]], s_ref[:3])
    s_tol = S_TOL if state_dtype == torch.float32 else 1e-2
    print(f"[fused slots {state_dtype}] hs rel_inf={e_hs:.2e} S rel_inf={e_s:.2e}", flush=True)
    assert e_hs <= O_TOL and e_s <= s_tol
    untouched = [1, 2, 3, 4, 6, 8]
    assert torch.equal(dpool.cpu()[untouched], pool[untouched])


def test_no_tokens_carries_the_initial_states():
    """T = 0 with 8 sequences (a batch the wide scan would take): hs is empty
    and the final states are the initial ones."""
    q, k, v, g, beta, h0, gate, o_norm = [x.to(DEV) for x in layer_case(8, 0, 16, 32, 128, torch.bfloat16, 30)]
    with torch.no_grad():
        hs, s = chunk_layer_fwd(q, k, v, g, beta, 128 ** -0.5, h0, gate, o_norm, EPS)
    torch.cuda.synchronize()
    assert hs.shape == (8, 0, 32 * 128)
    assert torch.equal(s, h0)
