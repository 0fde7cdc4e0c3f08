"""The reference's own op pair (pseudobrain::gated_delta_chunk and its
backward, gated_deltanet.py:200-277), with fla's residuals gc and A:
pbgdn_chunk_residuals against the oracle's chunk_residuals (gc to float32
rounding of the same sequential sum, A within 1e-4 in float32 and 1e-2 of its
largest entry in bf16), pbgdn_chunk_decumulate as gc's inverse, the ops
pbgdn::gated_delta_chunk_fla and pseudobrain::gated_delta_chunk (defined by
register_reference_ops) against the operator and its backward."""
import numpy as np
import pytest
import torch

from oracle import gdn
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import generate, to_numpy

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("batch,length,hk,hv,dk,dtype", [
    (1, 130, 2, 4, 64, torch.bfloat16),    # GQA 2 -> 4, a short last chunk
    (2, 64, 1, 1, 128, torch.float32),     # one whole chunk per sequence
    (1, 1, 1, 2, 128, torch.float16),      # one token
    (1, 1000, 16, 32, 128, torch.bfloat16),  # the Qwen3-Next heads
])
def test_residuals_match_the_oracle(batch, length, hk, hv, dk, dtype):
    _, k, _, g, beta, _ = generate(batch, length, hk, hv, dk, 64, dtype, 0.02, seed=length + hv)
    print(f"[residuals B={batch} T={length} {hk}->{hv} K={dk} {dtype}]", flush=True)
    with torch.no_grad():
        gc, a = gd.chunk_residuals(k.to(DEV), g.to(DEV), beta.to(DEV))
    torch.cuda.synchronize()
    assert a.dtype == dtype and a.shape == (batch, length, hv, 64) and gc.shape == (batch, length, hv)
    gc_ref, a_ref = gdn.chunk_residuals(to_numpy(k.float()), to_numpy(g), to_numpy(beta.float()))
    gc_err = np.abs(gc.cpu().numpy() - gc_ref).max()
    a_err = np.abs(a.float().cpu().numpy() - a_ref).max() / np.abs(a_ref).max()
    print(f"[residuals] gc max abs {gc_err:.2e}, A max abs / max |A| {a_err:.2e}", flush=True)
    assert gc_err <= 1e-6 * max(1.0, np.abs(gc_ref).max())
    assert a_err <= (1e-4 if dtype == torch.float32 else 1e-2)


def test_decumulate_inverts_the_cumulative_sums():
    _, k, _, g, beta, _ = generate(2, 300, 1, 2, 64, 64, torch.bfloat16, 0.02, seed=4)
    with torch.no_grad():
        gc, _ = gd.chunk_residuals(k.to(DEV), g.to(DEV), beta.to(DEV))
        back = gd.chunk_decumulate(gc)
    torch.cuda.synchronize()
    err = (back.cpu() - g).abs().max().item()
    print(f"[decumulate] max abs {err:.2e}", flush=True)
    assert err <= 4 * torch.finfo(torch.float32).eps * gc.abs().max().item()


def fla_case(seed, dtype=torch.bfloat16):
    q, k, v, g, beta, h0 = generate(1, 200, 1, 2, 64, 64, dtype, 0.02, seed=seed)
    return [x.to(DEV) for x in (q, k, v, g, beta, h0)]


@pytest.mark.parametrize("reference_names", [False, True])
def test_op_returns_the_operator_and_its_residuals(reference_names):
    q, k, v, g, beta, h0 = fla_case(8)
    op = gd.register_reference_ops()[0] if reference_names else torch.ops.pbgdn.gated_delta_chunk_fla
    if reference_names:
        assert torch.ops.pseudobrain.gated_delta_chunk is not None
    with torch.no_grad():
        o, final, gc, a = op(q, k, v, g, beta, h0, 0.125)
        o2, final2 = gd.chunk_fwd(q, k, v, g, beta, 0.125, h0)
        gc2, a2 = gd.chunk_residuals(k, g, beta)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(final, final2) and torch.equal(gc, gc2) and torch.equal(a, a2)


def test_autograd_through_the_op_is_the_operator_backward():
    """Gradients through pbgdn::gated_delta_chunk_fla (whose backward recovers
    g from gc) against chunk_bwd with the original g."""
    q, k, v, g, beta, h0 = fla_case(9)
    leaves = [x.detach().float().requires_grad_(True) for x in (q, k, v, g, beta, h0)]
    ins = [leaves[0].to(q.dtype), leaves[1].to(k.dtype), leaves[2].to(v.dtype), leaves[3], leaves[4], leaves[5]]
    o, final, _, _ = torch.ops.pbgdn.gated_delta_chunk_fla(*ins, 0.125)
    gen = torch.Generator(device=DEV).manual_seed(3)
    do = torch.randn(o.shape, generator=gen, device=DEV).to(o.dtype)
    dht = torch.randn(final.shape, generator=gen, device=DEV)
    torch.autograd.backward([o, final], [do, dht])
    with torch.no_grad():
        ref = gd.chunk_bwd(q, k, v, g, beta, 0.125, h0, do, dht)
    torch.cuda.synchronize()
    for name, got, want in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), [x.grad for x in leaves], ref):
        err = ((got.float() - want.float()).abs().max() / want.float().abs().max().clamp_min(1e-30)).item()
        print(f"[fla op autograd] {name} {err:.2e}", flush=True)
        assert err <= 1e-3, name
