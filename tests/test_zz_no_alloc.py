"""The no-allocation prefill entry point (pbgdn_chunk_fwd_noalloc) against the
existing one (pbgdn_chunk_fwd with a caller workspace), both through the C ABI:
the same kernels run on the same inputs, so outputs and final states must be
equal bit for bit, on two calls in a row, the second smaller than the first
(the scratch keeps the first call's records, which the second must not see).
A call larger than the scratch is refused and launches nothing."""
import pytest
import torch

from pseudobrain_amd import _lib
from pseudobrain_amd.workloads import cu_seqlens_of, generate
from tests.gpu_util import assert_parity, oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def call(noalloc, q, k, v, g, beta, h0, cu, hk, hv, dk, dv, scale):
    """One prefill through the C ABI; returns (o in q's dtype, final states fp32)."""
    batch, length = q.shape[:2]
    nseq = batch if cu is None else cu.numel() - 1
    o = torch.full((batch, length, hv, dv), float("nan"), dtype=q.dtype, device=DEV)
    ht = torch.full((nseq, hv, dk, dv), float("nan"), dtype=torch.float32, device=DEV)
    lib = _lib.lib()
    codes = _lib.DTYPE_CODES
    common = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta), _lib.F32,
              _lib.ptr(h0), _lib.ptr(ht), _lib.F32, None, None, 0, _lib.ptr(cu), nseq, _lib.ptr(o), codes[o.dtype],
              batch, length, hk, hv, dk, dv, scale, 64)
    stream = _lib.stream_handle(torch.device(DEV))
    if noalloc:
        status = lib.pbgdn_chunk_fwd_noalloc(*common, stream)
    else:
        ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq, _lib.DTYPE_CODES[q.dtype])
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        status = lib.pbgdn_chunk_fwd(*common, _lib.ptr(ws), ws_bytes, stream)
    _lib.check(status, "noalloc" if noalloc else "chunk_fwd")
    torch.cuda.synchronize()
    return o, ht


def case(length, hk, hv, dk, dv, seed, lengths=None, dtype=torch.bfloat16, v_scale=1.0):
    nseq = 1 if lengths is None else len(lengths)
    q, k, v, g, beta, h0 = generate(1, length, hk, hv, dk, dv, dtype, 0.02, seed=seed, nstates=nseq)
    cu = None if lengths is None else cu_seqlens_of(lengths)
    return q, k, v * v_scale, g, beta, h0 * v_scale, cu


@pytest.mark.parametrize("first,second", [
    # the Qwen3-Next head shape: a 4,096-token call, then a 1,000-token one
    ((4096, 16, 32, 128, 128, 1, None), (1000, 16, 32, 128, 128, 2, None)),
    # packed sequences, then fewer and shorter ones with other heads
    ((3000, 4, 8, 128, 64, 3, [1000, 64, 0, 1936]), (700, 2, 4, 64, 128, 4, [300, 400])),
    # float32 inputs (the range scale of v and h0 is reduced into the scratch's
    # tail): v x 1e3, then a smaller call with v x 1e5 and other heads
    ((2048, 4, 4, 64, 64, 5, None, torch.float32, 1e3), (900, 2, 4, 128, 64, 6, [500, 400], torch.float32, 1e5)),
    # 256-wide keys (the prep kernel at K = 256, then the scan for such keys)
    ((2000, 2, 4, 256, 128, 7, None), (600, 1, 2, 256, 64, 8, [250, 350])),
])
def test_noalloc_equals_the_workspace_entry_point(first, second):
    for length, hk, hv, dk, dv, seed, lengths, *more in (first, second):
        q, k, v, g, beta, h0, cu = case(length, hk, hv, dk, dv, seed, lengths, *more)
        dev = [None if x is None else x.to(DEV) for x in (q, k, v, g, beta, h0, cu)]
        scale = dk ** -0.5
        print(f"[noalloc] T={length} Hk={hk} Hv={hv} K={dk} V={dv} seqs={lengths}", flush=True)
        o_ref, s_ref = call(False, *dev, hk, hv, dk, dv, scale)
        o, s = call(True, *dev, hk, hv, dk, dv, scale)
        assert torch.equal(o, o_ref), "outputs differ from pbgdn_chunk_fwd"
        assert torch.equal(s, s_ref), "final states differ from pbgdn_chunk_fwd"
        if length <= 1000 or q.dtype == torch.float32:  # and both meet the oracle
            o_or, s_or = oracle(q, k, v, g, beta, scale, h0, cu_seqlens=cu)
            assert_parity(f"noalloc T={length}", o, o_or, s, s_or)


def test_noalloc_refuses_a_call_beyond_its_scratch():
    q, k, v, g, beta, h0, _ = case(16384, 16, 32, 128, 128, 5)
    dev = [x.to(DEV) for x in (q, k, v, g, beta, h0)]
    o = torch.zeros(1, 16384, 32, 128, dtype=torch.bfloat16, device=DEV)
    lib = _lib.lib()
    assert lib.pbgdn_chunk_workspace_size(1, 16384, 32, 1, _lib.BF16) > _lib.NOALLOC_SCRATCH_BYTES
    status = lib.pbgdn_chunk_fwd_noalloc(
        *(_lib.ptr(x) for x in dev[:3]), _lib.BF16, _lib.ptr(dev[3]), _lib.ptr(dev[4]), _lib.F32,
        _lib.ptr(dev[5]), None, _lib.F32, None, None, 0, None, 1, _lib.ptr(o), _lib.BF16, 1, 16384, 16, 32, 128,
        128, 128 ** -0.5, 64, _lib.stream_handle(torch.device(DEV)))
    torch.cuda.synchronize()
    assert status == _lib.ERR_SCRATCH
    assert torch.count_nonzero(o) == 0  # nothing ran
