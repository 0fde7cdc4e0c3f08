"""Gated DeltaNet recurrence on MI355X: the device-side kernels behind the
reference's operator API (pseudobrain/gated_deltanet.py:74-308).

    S_t = a_t S_{t-1} + k_t u_t^T,   u_t = b_t (v_t - a_t S_{t-1}^T k_t)
    o_t = S_t^T q_t * scale,         a_t = exp(g_t)          (gated_deltanet.py:9-11)

Tensors follow the reference layouts: q, k [B,T,Hk,K]; v [B,T,Hv,V]; g, beta
[B,T,Hv] (g <= 0 is the log decay); h0 [B,Hv,K,V] fp32 with S stored [K, V].
Hk may equal Hv (q/k already repeated, as the reference passes them) or divide
it (GQA without the repeat: value head h reads key head h // (Hv // Hk), the
repeat_interleave mapping of gated_deltanet.py:422-424).

Kernels (all run on the GPU; there is no CPU path in this package):
  * "hip"         chunkwise prefill kernel (pbgdn_chunk_fwd), the replacement of
                  fla's chunk kernels (delta_rule_fla, :280-285)
  * "chunked"     the same chunk kernel: the device counterpart of the
                  reference's PyTorch delta_rule_chunked (:110-165)
  * "sequential"  fused recurrent kernel (pbgdn_recurrent_fwd), the device
                  counterpart of delta_rule_sequential (:93-107), used for decode
                  and T <= SEQUENTIAL_MAX as select_kernel does (:291-297)
Every entry returns (o float32 [B,T,Hv,V], final state float32 [B,Hv,K,V]) like
the reference. cu_seqlens (int32 [N+1], B == 1) packs N independent sequences
with h0 / final states [N,Hv,K,V].
"""
from __future__ import annotations

import torch

from . import _lib

CHUNK = 64            # gated_deltanet.py:49
SEQUENTIAL_MAX = 4    # gated_deltanet.py:54
KERNELS = ("sequential", "chunked", "hip")
CHUNK_HEAD_DIMS = (64, 128)               # key widths the chunk kernel is built for
RECURRENT_HEAD_DIMS = (32, 64, 128, 256)  # key and value widths of the recurrent kernel


# ----------------------------------------------------------------------------
# Argument checks (ValueError, as the reference raises for bad shapes/names).
# ----------------------------------------------------------------------------
def _shapes(q, k, v, g, beta):
    if q.ndim != 4 or k.shape != q.shape or v.ndim != 4:
        raise ValueError("expected q, k [B,T,Hk,K] of one shape and v [B,T,Hv,V]")
    batch, length, hk, dk = q.shape
    if v.shape[:2] != (batch, length):
        raise ValueError("v must share q's batch and time axes")
    hv, dv = v.shape[2], v.shape[3]
    if hk < 1 or hv % hk:
        raise ValueError("gated deltanet value heads must be a multiple of the key heads")
    if g.shape != (batch, length, hv) or beta.shape != (batch, length, hv):
        raise ValueError(f"g and beta must be [B,T,Hv] = {(batch, length, hv)}")
    return batch, length, hk, hv, dk, dv


def _require_device(*tensors):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "pbgdn kernels run on ROCm devices only (got a tensor on "
            f"'{dev}'); this package has no CPU path")
    for t in tensors:
        if t is not None and t.device != dev:
            raise ValueError("all tensors must be on one device")
    return dev


def _operands(q, k, v, g, beta):
    """q, k, v in one dtype (q's, as the fla path casts v and beta to q.dtype,
    gated_deltanet.py:284); g float32; beta float32 or q's dtype."""
    if q.dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"unsupported q dtype {q.dtype}")
    k = _aligned(k.to(q.dtype).contiguous(), 16)
    v = _aligned(v.to(q.dtype).contiguous(), 16)
    q = _aligned(q.contiguous(), 16)
    g = _aligned(g.to(torch.float32).contiguous(), 4)
    if beta.dtype not in (torch.float32, q.dtype):
        beta = beta.to(torch.float32)
    return q, k, v, g, _aligned(beta.contiguous(), 4)


def _aligned(x: torch.Tensor, nbytes: int) -> torch.Tensor:
    """x, or a copy of it when a view leaves it off the alignment the kernels read in."""
    return x if x.data_ptr() % nbytes == 0 else x.clone()


# ----------------------------------------------------------------------------
# Chunk kernel.
# ----------------------------------------------------------------------------
def chunk_fwd(q, k, v, g, beta, scale: float, h0=None, cu_seqlens=None, *,
              out_dtype: torch.dtype | None = None, output_final_state: bool = True,
              out: torch.Tensor | None = None):
    """Launch pbgdn_chunk_fwd. Returns (o [B,T,Hv,V] in out_dtype (default q's dtype),
    final [N,Hv,K,V] fp32 or None). `out` may supply the output buffer."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    if out_dtype is not None and out_dtype not in (torch.float32, q.dtype):
        raise ValueError(f"chunk kernel writes o as float32 or q's dtype ({q.dtype}), not {out_dtype}")
    dev = _require_device(q, k, v, g, beta, h0, cu_seqlens)
    if dk not in CHUNK_HEAD_DIMS or dv % 16:
        raise ValueError(f"chunk kernel supports K in {CHUNK_HEAD_DIMS} and V a multiple of 16")
    q, k, v, g, beta = _operands(q, k, v, g, beta)
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError("cu_seqlens needs B == 1 (sequences packed along T)")
        if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 1:
            raise ValueError("cu_seqlens must be a 1-D tensor [N+1]")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
        nseq = cu_seqlens.numel() - 1
    else:
        nseq = batch
    if h0 is not None:
        if h0.shape != (nseq, hv, dk, dv):
            raise ValueError(f"initial state must be [N,Hv,K,V] = {(nseq, hv, dk, dv)}")
        h0 = h0.to(torch.float32).contiguous()
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty(batch, length, hv, dv, dtype=out_dtype, device=dev)
    elif out.shape != (batch, length, hv, dv) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B,T,Hv,V] tensor of out_dtype")
    final = torch.empty(nseq, hv, dk, dv, dtype=torch.float32, device=dev) if output_final_state else None
    lib = _lib.lib()
    ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    codes = _lib.DTYPE_CODES
    status = lib.pbgdn_chunk_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta),
        codes[beta.dtype], _lib.ptr(h0), _lib.ptr(final), _lib.F32, None, None, 0, _lib.ptr(cu_seqlens), nseq,
        _lib.ptr(out), codes[out_dtype], batch, length, hk, hv, dk, dv, float(scale), CHUNK,
        _lib.ptr(workspace), ws_bytes, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_fwd")
    return out, final


def _state_pool(states, hv, dk, dv):
    if (states.ndim != 4 or states.shape[1:] != (hv, dk, dv) or states.dtype not in _lib.DTYPE_CODES
            or not states.is_contiguous()):
        raise ValueError(f"states must be a contiguous [S,{hv},{dk},{dv}] float32, bfloat16 or float16 tensor")


def chunk_fwd_slots(q, k, v, g, beta, scale: float, states, state_idx, cu_seqlens=None,
                    has_initial_state=None, *, out_dtype: torch.dtype | None = None,
                    out: torch.Tensor | None = None):
    """Prefill against a pool of state slots, the way a serving cache holds
    them (vLLM's per-request slots, serving/pb27_vllm/pb27_vllm/universal_models.py:147-165):
    sequence n starts from states[state_idx[n]] (zeros where has_initial_state[n]
    is False, or where the slot is outside the pool) and its final state is
    written back to that slot, in the pool's dtype (float32, bfloat16 or
    float16; the arithmetic is float32). Slots must be distinct. One call of
    pbgdn_chunk_fwd; no gather or scatter copies. Returns o [B,T,Hv,V]."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    if out_dtype is not None and out_dtype not in (torch.float32, q.dtype):
        raise ValueError(f"chunk kernel writes o as float32 or q's dtype ({q.dtype}), not {out_dtype}")
    dev = _require_device(q, k, v, g, beta, states, state_idx, cu_seqlens, has_initial_state)
    if dk not in CHUNK_HEAD_DIMS or dv % 16:
        raise ValueError(f"chunk kernel supports K in {CHUNK_HEAD_DIMS} and V a multiple of 16")
    _state_pool(states, hv, dk, dv)
    q, k, v, g, beta = _operands(q, k, v, g, beta)
    if cu_seqlens is not None:
        if batch != 1:
            raise ValueError("cu_seqlens needs B == 1 (sequences packed along T)")
        if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 1:
            raise ValueError("cu_seqlens must be a 1-D tensor [N+1]")
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
        nseq = cu_seqlens.numel() - 1
    else:
        nseq = batch
    if state_idx.shape != (nseq,):
        raise ValueError(f"state_idx must be [N] = [{nseq}]")
    state_idx = state_idx.to(torch.int32).contiguous()
    if has_initial_state is not None:
        if has_initial_state.shape != (nseq,):
            raise ValueError(f"has_initial_state must be [N] = [{nseq}]")
        has_initial_state = has_initial_state.to(torch.uint8).contiguous()
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty(batch, length, hv, dv, dtype=out_dtype, device=dev)
    elif out.shape != (batch, length, hv, dv) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B,T,Hv,V] tensor of out_dtype")
    lib = _lib.lib()
    ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    codes = _lib.DTYPE_CODES
    status = lib.pbgdn_chunk_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta),
        codes[beta.dtype], _lib.ptr(states), _lib.ptr(states), codes[states.dtype], _lib.ptr(state_idx),
        _lib.ptr(has_initial_state), states.shape[0], _lib.ptr(cu_seqlens), nseq, _lib.ptr(out),
        codes[out_dtype], batch, length, hk, hv, dk, dv, float(scale), CHUNK, _lib.ptr(workspace), ws_bytes,
        _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_fwd")
    return out


def recurrent_fwd(q, k, v, g, beta, scale: float, state_in, state_out=None, state_idx=None, *,
                  out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
                  token_state_idx: torch.Tensor | None = None):
    """Launch pbgdn_recurrent_fwd: all T tokens through the per-step recurrence.
    state_out may be state_in (in place) or None (a new tensor). state_idx [B]
    int32 maps sequences to state slots (distinct; a slot outside the state
    tensor, e.g. -1, is skipped and its o is zero). The states may be float32,
    bfloat16 or float16 (state_out in state_in's dtype); the arithmetic is
    float32. Returns (o, state_out).

    token_state_idx [B,T] int32 selects the speculative-verify form
    (pbgdn_recurrent_verify_fwd): sequence b starts from slot state_idx[b] and
    the state after its token t is written to slot token_state_idx[b, t] of
    state_out (skipped when outside the state tensor); nothing else is
    written."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    dev = _require_device(q, k, v, g, beta, state_in, state_out, state_idx)
    if dk not in RECURRENT_HEAD_DIMS or dv not in RECURRENT_HEAD_DIMS:
        raise ValueError(f"recurrent kernel supports K, V in {RECURRENT_HEAD_DIMS}")
    q, k, v, g, beta = _operands(q, k, v, g, beta)
    _state_pool(state_in, hv, dk, dv)
    if state_idx is None:
        if state_in.shape[0] != batch:
            raise ValueError("without state_idx the state batch must equal B")
    else:
        if state_idx.shape != (batch,):
            raise ValueError("state_idx must be [B]")
        state_idx = state_idx.to(torch.int32).contiguous()
    if state_out is None:
        state_out = torch.empty_like(state_in)
    elif state_out.shape != state_in.shape or state_out.dtype != state_in.dtype or not state_out.is_contiguous():
        raise ValueError("state_out must match state_in")
    if out is None:
        out = torch.empty(batch, length, hv, dv, dtype=out_dtype, device=dev)
    codes = _lib.DTYPE_CODES
    if token_state_idx is not None:
        if token_state_idx.shape != (batch, length):
            raise ValueError("token_state_idx must be [B,T]")
        token_state_idx = token_state_idx.to(torch.int32).contiguous()
        status = _lib.lib().pbgdn_recurrent_verify_fwd(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta),
            codes[beta.dtype], _lib.ptr(state_in), _lib.ptr(state_out), codes[state_in.dtype], _lib.ptr(state_idx),
            _lib.ptr(token_state_idx), state_in.shape[0], _lib.ptr(out), codes[out.dtype], batch, length, hk,
            hv, dk, dv, float(scale), _lib.stream_handle(dev))
        _lib.check(status, "pbgdn_recurrent_verify_fwd")
        return out, state_out
    status = _lib.lib().pbgdn_recurrent_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta),
        codes[beta.dtype], _lib.ptr(state_in), _lib.ptr(state_out), codes[state_in.dtype], _lib.ptr(state_idx),
        state_in.shape[0], _lib.ptr(out), codes[out.dtype], batch, length, hk, hv, dk, dv, float(scale),
        _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_recurrent_fwd")
    return out, state_out


BACKWARD_HEAD_DIMS = (64, 128)


def chunk_bwd(q, k, v, g, beta, scale: float, h0, do, dht=None):
    """Launch pbgdn_chunk_bwd: the gradients of (o, final) = chunk_fwd(q, k, v,
    g, beta, scale, h0) given do [B,T,Hv,V] and dht [B,Hv,K,V] (None: zeros),
    as the reference's gated_delta_chunk_backward returns them
    (gated_deltanet.py:230-277). Returns (dq, dk [B,T,Hk,K], dv [B,T,Hv,V] in
    q's dtype, dg [B,T,Hv] float32, dbeta in beta's operand dtype, dh0
    [B,Hv,K,V] float32)."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    dev = _require_device(q, k, v, g, beta, h0, do, dht)
    if dk not in BACKWARD_HEAD_DIMS or dv not in BACKWARD_HEAD_DIMS:
        raise ValueError(f"chunk backward supports K and V in {BACKWARD_HEAD_DIMS}")
    q, k, v, g, beta = _operands(q, k, v, g, beta)
    if do.shape != (batch, length, hv, dv):
        raise ValueError(f"grad of o must be [B,T,Hv,V] = {(batch, length, hv, dv)}")
    do = _aligned(do.to(q.dtype).contiguous(), 16)  # the reference passes grad_o.to(q.dtype) (:272)
    state_shape = (batch, hv, dk, dv)
    if h0 is not None:
        if h0.shape != state_shape:
            raise ValueError(f"initial state must be [B,Hv,K,V] = {state_shape}")
        h0 = h0.to(torch.float32).contiguous()
    if dht is not None:
        if dht.shape != state_shape:
            raise ValueError(f"grad of the final state must be [B,Hv,K,V] = {state_shape}")
        dht = dht.to(torch.float32).contiguous()
    dq, dk_ = torch.empty_like(q), torch.empty_like(k)
    dv_ = torch.empty_like(v)
    dg = torch.empty(batch, length, hv, dtype=torch.float32, device=dev)
    dbeta = torch.empty_like(beta)
    dh0 = torch.empty(state_shape, dtype=torch.float32, device=dev)
    lib = _lib.lib()
    ws_bytes = lib.pbgdn_chunk_bwd_workspace_size(batch, length, hk, hv, dk, dv)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    codes = _lib.DTYPE_CODES
    status = lib.pbgdn_chunk_bwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta), codes[beta.dtype],
        _lib.ptr(h0), _lib.ptr(do), codes[do.dtype], _lib.ptr(dht), _lib.ptr(dq), _lib.ptr(dk_), _lib.ptr(dv_),
        _lib.ptr(dg), _lib.ptr(dbeta), _lib.ptr(dh0), _lib.ptr(workspace), ws_bytes, batch, length, hk, hv, dk, dv,
        float(scale), _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_bwd")
    return dq, dk_, dv_, dg, dbeta, dh0


# ----------------------------------------------------------------------------
# torch custom ops (functional prefill, mutating decode step) with fake impls,
# the form of pseudobrain::gated_delta_chunk (gated_deltanet.py:200-227).
# ----------------------------------------------------------------------------
@torch.library.custom_op("pbgdn::gated_delta_chunk", mutates_args=(),
                         schema="(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor? h0, "
                                "Tensor? cu_seqlens, float scale) -> (Tensor, Tensor)")
def gated_delta_chunk(q, k, v, g, beta, h0, cu_seqlens, scale):
    """(o [B,T,Hv,V] in q's dtype, final state fp32 [N,Hv,K,V])."""
    return chunk_fwd(q, k, v, g, beta, scale, h0, cu_seqlens)


@gated_delta_chunk.register_fake
def _(q, k, v, g, beta, h0, cu_seqlens, scale):
    batch, length, _, dk = q.shape
    hv, dv = v.shape[2], v.shape[3]
    nseq = batch if cu_seqlens is None else cu_seqlens.shape[0] - 1
    return (q.new_empty(batch, length, hv, dv),
            q.new_empty(nseq, hv, dk, dv, dtype=torch.float32))


@torch.library.custom_op("pbgdn::gated_delta_chunk_backward", mutates_args=(),
                         schema="(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor? h0, "
                                "Tensor grad_o, Tensor? grad_final, float scale) "
                                "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
def gated_delta_chunk_backward(q, k, v, g, beta, h0, grad_o, grad_final, scale):
    """(dq, dk, dv, dg fp32, dbeta, dh0 fp32): pseudobrain::gated_delta_chunk_backward
    (gated_deltanet.py:230-256) without fla's saved gc and A (recomputed)."""
    return chunk_bwd(q, k, v, g, beta, scale, h0, grad_o, grad_final)


@gated_delta_chunk_backward.register_fake
def _(q, k, v, g, beta, h0, grad_o, grad_final, scale):
    beta_dtype = beta.dtype if beta.dtype in (torch.float32, q.dtype) else torch.float32
    batch, hv, dk, dv = q.shape[0], v.shape[2], q.shape[3], v.shape[3]
    return (torch.empty_like(q), q.new_empty(k.shape), q.new_empty(v.shape),
            g.new_empty(g.shape, dtype=torch.float32), beta.new_empty(beta.shape, dtype=beta_dtype),
            q.new_empty(batch, hv, dk, dv, dtype=torch.float32))


def _chunk_setup(ctx, inputs, output):
    q, k, v, g, beta, h0, cu_seqlens, scale = inputs
    ctx.save_for_backward(q, k, v, g, beta, h0)
    ctx.scale = scale
    ctx.packed = cu_seqlens is not None


def _chunk_grad(ctx, grad_o, grad_final):
    """The reference's _fla_grad (gated_deltanet.py:266-275): zeros for a
    missing output gradient, each gradient in its input's dtype."""
    if ctx.packed:
        raise NotImplementedError("the chunk backward takes [B,T] batches; packed sequences (cu_seqlens) "
                                  "have no backward here")
    q, k, v, g, beta, h0 = ctx.saved_tensors
    if grad_o is None:
        grad_o = torch.zeros(*q.shape[:2], v.shape[2], v.shape[3], dtype=q.dtype, device=q.device)
    dq, dk, dv, dg, dbeta, dh0 = gated_delta_chunk_backward(q, k, v, g, beta, h0, grad_o, grad_final, ctx.scale)
    return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
            None if h0 is None else dh0.to(h0.dtype), None, None)


gated_delta_chunk.register_autograd(_chunk_grad, setup_context=_chunk_setup)


@torch.library.custom_op("pbgdn::recurrent_step_", mutates_args=("state",),
                         schema="(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor(a!) state, "
                                "Tensor? state_idx, float scale) -> Tensor")
def recurrent_step_(q, k, v, g, beta, state, state_idx, scale):
    """Decode step(s) updating `state` [S,Hv,K,V] in place; o in q's dtype."""
    out, _ = recurrent_fwd(q, k, v, g, beta, scale, state, state, state_idx, out_dtype=q.dtype)
    return out


@recurrent_step_.register_fake
def _(q, k, v, g, beta, state, state_idx, scale):
    return q.new_empty(q.shape[0], q.shape[1], v.shape[2], v.shape[3])


@torch.library.custom_op("pbgdn::chunk_slots_", mutates_args=("states",),
                         schema="(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor(a!) states, "
                                "Tensor state_idx, Tensor? cu_seqlens, Tensor? has_initial_state, "
                                "float scale) -> Tensor")
def chunk_slots_(q, k, v, g, beta, states, state_idx, cu_seqlens, has_initial_state, scale):
    """Prefill against state slots (chunk_fwd_slots), updating `states` in place; o in q's dtype."""
    return chunk_fwd_slots(q, k, v, g, beta, scale, states, state_idx, cu_seqlens, has_initial_state)


@chunk_slots_.register_fake
def _(q, k, v, g, beta, states, state_idx, cu_seqlens, has_initial_state, scale):
    return q.new_empty(q.shape[0], q.shape[1], v.shape[2], v.shape[3])


# ----------------------------------------------------------------------------
# The reference's kernel-level API.
# ----------------------------------------------------------------------------
def delta_rule_hip(q, k, v, g, beta, scale, h0, cu_seqlens=None):
    """Chunk kernel with the fla path's conventions (gated_deltanet.py:280-285):
    q/k/v at their own precision, fp32 state and decay; returns (o.float(), final)."""
    o, final = gated_delta_chunk(q, k, v, g, beta, h0, cu_seqlens, float(scale))
    return o.float(), final


def delta_rule_sequential(q, k, v, g, beta, scale, h0):
    """Per-step recurrence on the device (gated_deltanet.py:93-107); the state is
    returned, not mutated. o is float32."""
    batch = q.shape[0]
    hv, dk, dv = v.shape[2], q.shape[3], v.shape[3]
    if h0.shape != (batch, hv, dk, dv):
        raise ValueError(f"initial state must be [B,Hv,K,V] = {(batch, hv, dk, dv)}")
    state = h0.to(torch.float32).contiguous()
    return recurrent_fwd(q, k, v, g, beta, scale, state, None, out_dtype=torch.float32)


def hip_usable(*tensors: torch.Tensor) -> bool:
    """The chunk kernel applies (the fla_usable gate, gated_deltanet.py:189-197):
    device tensors and head widths this library has kernels for. tensors[0] is the
    matrix state [..., K, V]. Raises if the tensors are on a GPU but the library
    is missing: a GPU caller never silently loses the kernel."""
    if not tensors or not all(t.is_cuda for t in tensors):
        return False
    state = tensors[0]
    if state.ndim < 2 or state.shape[-2] not in CHUNK_HEAD_DIMS or state.shape[-1] % 16:
        return False
    _lib.lib()
    return True


def select_kernel(backend: str, serial: bool, length: int, *tensors: torch.Tensor) -> str:
    """Kernel for one call (gated_deltanet.py:291-297), with "hip" in fla's place:
    sequential for serial calls and T <= SEQUENTIAL_MAX, the chunk kernel for the
    'fused' backend when usable, else "chunked"."""
    if serial or length <= SEQUENTIAL_MAX:
        return "sequential"
    if backend == "fused" and hip_usable(*tensors):
        return "hip"
    return "chunked"


def gated_delta_rule(q, k, v, g, beta, scale, h0, kernel: str = "chunked", cu_seqlens=None):
    """The recurrence with the given kernel (gated_deltanet.py:300-308)."""
    if kernel == "sequential":
        if cu_seqlens is not None:
            raise ValueError("cu_seqlens applies to the chunk kernel")
        return delta_rule_sequential(q, k, v, g, beta, scale, h0)
    if kernel in ("hip", "chunked"):
        return delta_rule_hip(q, k, v, g, beta, scale, h0, cu_seqlens)
    raise ValueError(f"gated delta rule kernel must be one of {KERNELS}")
