"""Seeded synthetic inputs of the operator's five workloads.

Draw order per call is fixed: q, k, v, beta logits, g logits, h0; each drawn in
float32 from a torch.Generator seeded with `seed`, then cast. q and k are drawn
~ N(0,1) and L2-normalised per head in float32 ('max' mode: x / max(||x||, 1e-6),
gated_deltanet.py:59-70) before the cast; v ~ N(0,1); beta = sigmoid(N(0,1));
g = -softplus(N(0,1)) (log decay <= 0); h0 ~ N(0, 0.02) or zeros.

Workloads (name: shapes):
  prefill_small   B=1, T=2048, H=4, K=V=64, float32 inputs, zero h0
  prefill_qwen3next  B=1, T=32768, Hk=16 -> Hv=32, K=V=128, bf16 q/k/v, h0 [32,128,128]
  decode_b64      64 sequences x 1 token, Hk=16, Hv=32, K=V=128, bf16, state [64,32,128,128]
  varlen_8seq     8 packed sequences, lengths U[1024, 65536] rescaled to sum 262144
  stream_1m       1,048,576 tokens as 16 segments of 65,536 (state carried)
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class Shape:
    batch: int
    length: int
    hk: int
    hv: int
    dk: int
    dv: int
    dtype: torch.dtype
    h0_std: float  # 0 -> zero initial state


WORKLOADS = {
    "prefill_small": Shape(1, 2048, 4, 4, 64, 64, torch.float32, 0.0),
    "prefill_qwen3next": Shape(1, 32768, 16, 32, 128, 128, torch.bfloat16, 0.02),
    "decode_b64": Shape(64, 1, 16, 32, 128, 128, torch.bfloat16, 0.02),
    "varlen_8seq": Shape(1, 262144, 16, 32, 128, 128, torch.bfloat16, 0.02),
    "stream_1m": Shape(1, 1048576, 16, 32, 128, 128, torch.bfloat16, 0.02),
    # the prefill shape with 256-wide key and value heads (the widest the
    # reference's device gate admits, gated_deltanet.py:189-197)
    "prefill_k256": Shape(1, 32768, 16, 32, 256, 256, torch.bfloat16, 0.02),
}
STREAM_SEGMENT = 65536
VARLEN_SEQS = 8


def l2norm_max(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return F.normalize(x, dim=-1, eps=eps)


def generate(batch, length, hk, hv, dk, dv, dtype, h0_std, seed, *, nstates=None,
             g_scale: float = 1.0, device="cpu"):
    """Inputs (q, k, v, g, beta, h0) with the documented draw order.

    nstates: leading size of h0 (default batch); g_scale multiplies g (values
    below 1 give slow decay, for long-range stress cases)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))
    f32 = dict(dtype=torch.float32, device=device, generator=gen)
    q = torch.randn(batch, length, hk, dk, **f32)
    k = torch.randn(batch, length, hk, dk, **f32)
    v = torch.randn(batch, length, hv, dv, **f32)
    beta = torch.sigmoid(torch.randn(batch, length, hv, **f32))
    g = -F.softplus(torch.randn(batch, length, hv, **f32)) * g_scale
    nstates = batch if nstates is None else nstates
    if h0_std > 0:
        h0 = torch.randn(nstates, hv, dk, dv, **f32) * h0_std
    else:
        h0 = torch.zeros(nstates, hv, dk, dv, dtype=torch.float32, device=device)
    q = l2norm_max(q).to(dtype)
    k = l2norm_max(k).to(dtype)
    return q, k, v.to(dtype), g, beta, h0


def workload(name: str, seed: int = 0, *, length: int | None = None, batch: int | None = None,
             g_scale: float = 1.0, device="cpu"):
    """Inputs of a named workload; `length`/`batch` shrink it for tests."""
    s = WORKLOADS[name]
    return generate(s.batch if batch is None else batch, s.length if length is None else length,
                    s.hk, s.hv, s.dk, s.dv, s.dtype, s.h0_std, seed, g_scale=g_scale, device=device)


def varlen_lengths(total: int = 262144, nseq: int = VARLEN_SEQS, lo: int = 1024, hi: int = 65536,
                   seed: int = 0) -> list[int]:
    """nseq lengths drawn uniform in [lo, hi] and rescaled to sum `total`
    (the remainder goes to the last sequence)."""
    gen = torch.Generator().manual_seed(int(seed))
    raw = torch.randint(lo, hi + 1, (nseq,), generator=gen).double()
    lengths = [max(1, int(x)) for x in (raw * (total / raw.sum())).floor().tolist()]
    lengths[-1] += total - sum(lengths)
    return lengths


def cu_seqlens_of(lengths) -> torch.Tensor:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    return torch.tensor(cu, dtype=torch.int32)


def varlen_workload(seed: int = 0, total: int = 262144, nseq: int = VARLEN_SEQS, *,
                    lo: int = 1024, hi: int = 65536, device="cpu"):
    """Packed varlen inputs: (q, k, v, g, beta, h0 [N,...], cu_seqlens)."""
    s = WORKLOADS["varlen_8seq"]
    lengths = varlen_lengths(total, nseq, lo, hi, seed)
    q, k, v, g, beta, h0 = generate(1, total, s.hk, s.hv, s.dk, s.dv, s.dtype, s.h0_std, seed,
                                    nstates=nseq, device=device)
    return q, k, v, g, beta, h0, cu_seqlens_of(lengths).to(device)


def sha256(t: torch.Tensor) -> str:
    """SHA-256 of a tensor's bytes (CPU copy), for logging the exact inputs."""
    x = t.detach().contiguous().cpu()
    if x.dtype == torch.bfloat16:
        x = x.view(torch.int16)
    return hashlib.sha256(x.numpy().tobytes()).hexdigest()


def to_numpy(t: torch.Tensor):
    """float32/float64 numpy copy (bf16/fp16 widened exactly)."""
    x = t.detach().cpu()
    if x.dtype in (torch.bfloat16, torch.float16):
        x = x.float()
    return x.numpy()
