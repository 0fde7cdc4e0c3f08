"""Randomised parity sweep of the prefill and decode paths against the fp32
oracle (delta_rule_chunked / delta_rule_sequential, gated_deltanet.py:93-165):
each case draws its own shapes (batch or packed sequences with empty ones,
GQA ratio, head widths, input dtype, beta dtype, initial states or none,
state slots, state dtype, output dtype) from a fixed seed, so the sweep is
reproducible and covers combinations the targeted tests do not.

Tolerances as everywhere: o within 2e-2 (1e-4 for float32 inputs through the
sequential kernel), float32 states within 1e-3, relative infinity norm; a
16-bit state within one unit in the last place of the rounded oracle plus the
float32 bound."""
import numpy as np
import pytest
import torch

from oracle import gdn
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import cu_seqlens_of, generate, to_numpy
from tests.gpu_util import O_TOL, S_TOL, assert_parity, oracle, rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def draw(rng, choices):
    return choices[int(rng.integers(len(choices)))]


def check_state(name, got, ref, dtype, tol):
    if dtype == torch.float32:
        err = rel_err(got, ref)
        assert err <= tol, f"{name}: state error {err:.3e}"
        return
    rounded = (gdn.round_bf16 if dtype == torch.bfloat16 else gdn.round_fp16)(ref.astype(np.float32))
    mant = 7 if dtype == torch.bfloat16 else 10
    spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-38))) - mant)
    excess = np.abs(to_numpy(got.float()) - rounded) - spacing - tol * np.abs(ref).max()
    assert excess.max() <= 0, f"{name}: 16-bit state off by more than an ulp"


@pytest.mark.parametrize("case", range(12))
def test_random_prefill(case):
    rng = np.random.default_rng(1000 + case)
    dk = draw(rng, [64, 128])
    dv = draw(rng, [16, 32, 64, 128])
    hk = draw(rng, [1, 2, 4])
    hv = hk * draw(rng, [1, 2, 4])
    dtype = draw(rng, DTYPES)
    packed = bool(rng.integers(2))
    state_dtype = draw(rng, DTYPES) if packed else torch.float32
    if packed:
        lengths = [int(x) for x in rng.integers(0, 400, size=int(rng.integers(1, 12)))]
        batch, length = 1, sum(lengths)
        nseq = len(lengths)
    else:
        batch, length = int(rng.integers(1, 4)), int(rng.integers(1, 700))
        nseq = batch
    q, k, v, g, beta, h0 = generate(batch, length, hk, hv, dk, dv, dtype, 0.05, seed=case, nstates=nseq)
    if bool(rng.integers(2)):
        beta = beta.to(dtype)
    name = (f"case {case}: {'packed ' + str(lengths) if packed else f'B={batch} T={length}'} K={dk} V={dv} "
            f"{hk}->{hv} {dtype} state {state_dtype}")
    print(f"[{name}]", flush=True)
    scale = dk ** -0.5
    if not packed:
        o_ref, s_ref = oracle(q, k, v, g, beta, scale, h0)
        o, s = gd.chunk_fwd(*[x.to(DEV) for x in (q, k, v, g, beta)], scale, h0.to(DEV))
        torch.cuda.synchronize()
        assert_parity(name, o, o_ref, s, s_ref)
        return
    # packed sequences against a pool of state slots (some sequences new)
    cu = cu_seqlens_of(lengths)
    slots = rng.permutation(nseq + 3)[:nseq]
    has_init = rng.integers(0, 2, size=nseq).astype(bool)
    pool = (torch.randn(nseq + 3, hv, dk, dv, generator=torch.Generator().manual_seed(case)) * 0.05).to(state_dtype)
    h0 = torch.zeros(nseq, hv, dk, dv)
    for i in range(nseq):
        if has_init[i]:
            h0[i] = pool[slots[i]].float()
    o_ref, s_ref = oracle(q, k, v, g, beta, scale, h0, cu_seqlens=cu)
    dpool = pool.to(DEV)
    o = gd.chunk_fwd_slots(*[x.to(DEV) for x in (q, k, v, g, beta)], scale, dpool,
                           torch.tensor(slots, dtype=torch.int32, device=DEV), cu.to(DEV),
                           torch.tensor(has_init, device=DEV))
    torch.cuda.synchronize()
    assert_parity(name, o, o_ref)
    check_state(name, dpool.cpu()[slots], s_ref, state_dtype, S_TOL)
    others = [i for i in range(nseq + 3) if i not in set(slots.tolist())]
    assert torch.equal(dpool.cpu()[others], pool[others])


@pytest.mark.parametrize("case", range(8))
def test_random_decode(case):
    rng = np.random.default_rng(2000 + case)
    dk = draw(rng, [32, 64, 128, 256])
    dv = draw(rng, [32, 64, 128, 256])
    hk = draw(rng, [1, 2, 4])
    hv = hk * draw(rng, [1, 2])
    dtype = draw(rng, DTYPES)
    state_dtype = draw(rng, DTYPES)
    batch, length = int(rng.integers(1, 9)), int(rng.integers(1, 5))
    q, k, v, g, beta, _ = generate(batch, length, hk, hv, dk, dv, dtype, 0.0, seed=100 + case)
    nslots = batch + 2
    pool = (torch.randn(nslots, hv, dk, dv, generator=torch.Generator().manual_seed(case)) * 0.05).to(state_dtype)
    slots = rng.permutation(nslots)[:batch]
    name = f"case {case}: B={batch} T={length} K={dk} V={dv} {hk}->{hv} {dtype} state {state_dtype}"
    print(f"[{name}]", flush=True)
    o_ref, s_ref = oracle(q, k, v, g, beta, dk ** -0.5, pool[slots].float(), "sequential")
    dpool = pool.to(DEV)
    o, _ = gd.recurrent_fwd(*[x.to(DEV) for x in (q, k, v, g, beta)], dk ** -0.5, dpool, dpool,
                            torch.tensor(slots, dtype=torch.int32, device=DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else O_TOL
    assert_parity(name, o, o_ref, o_tol=tol)
    check_state(name, dpool.cpu()[slots], s_ref, state_dtype, 1e-4)
