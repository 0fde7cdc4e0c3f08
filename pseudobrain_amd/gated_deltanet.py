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
  * "chunked"     the same device path: the counterpart of the reference's
                  PyTorch delta_rule_chunked (:110-165) for device tensors
  * "sequential"  fused recurrent kernel (pbgdn_recurrent_fwd), the device
                  counterpart of delta_rule_sequential (:93-107), used for decode
                  and T <= SEQUENTIAL_MAX as select_kernel does (:291-297)
Every entry returns (o float32 [B,T,Hv,V], final state float32 [B,Hv,K,V]) like
the reference. cu_seqlens (int32 [N+1], B == 1) packs N independent sequences
with h0 / final states [N,Hv,K,V].

Head widths. Every device call with K, V <= 256 (fla_usable's bound, :189-197)
runs: widths between the kernels' instantiations are zero-padded, which leaves
the recurrence exact (a zero key or query dimension never enters a product, and
zero value columns start and stay zero); K above 128 runs on the chunk kernel
for 256-wide keys with 16-bit inputs, and token by token through the
recurrent kernel with float32 inputs.

Gradients. gated_delta_rule's device paths are differentiable through the chunk
operator's backward (pbgdn::gated_delta_chunk, for K, V <= 128; a packed
call's backward runs sequence by sequence); a training call through
"sequential" (T <= SEQUENTIAL_MAX) takes the
same operator. The lower-level entry points (chunk_fwd, chunk_fwd_slots,
recurrent_fwd, the decode and slot ops, the layer kernels in
pseudobrain_amd.layer) have no backward: with grad mode on and an input that
requires grad they raise instead of returning tensors cut from the graph.
"""
from __future__ import annotations

import torch

from . import _lib

CHUNK = 64            # gated_deltanet.py:49
SEQUENTIAL_MAX = 4    # gated_deltanet.py:54
KERNELS = ("sequential", "chunked", "hip")
CHUNK_HEAD_DIMS = (64, 128, 256)          # key widths the chunk kernels are built for
CHUNK_WIDE_KEY = 256                      # 16-bit inputs only, V a multiple of 32 (chunk_k256.hip)
RECURRENT_HEAD_DIMS = (32, 64, 128, 256)  # key and value widths of the recurrent kernel
BACKWARD_HEAD_DIMS = (64, 128)            # key and value widths of the chunk backward
MAX_HEAD_DIM = 256                        # widest head a device path takes (fla_usable, :189-197)


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


def grad_needed(*tensors) -> bool:
    """Autograd would want gradients of a result computed from these tensors."""
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


def require_no_grad(where: str, *tensors) -> None:
    """Raise when `where`, which has no backward, is called with grad mode on and
    an input that requires grad: its results would silently leave the graph."""
    if grad_needed(*tensors):
        raise RuntimeError(
            f"{where} has no backward: call it under torch.no_grad() (inference), or use "
            "gated_delta_rule(..., kernel='hip'), whose chunk operator has one")


def _head_bound(dk: int, dv: int) -> None:
    if dk > MAX_HEAD_DIM or dv > MAX_HEAD_DIM:
        raise ValueError(f"no device kernel for head widths above {MAX_HEAD_DIM} (got K={dk}, V={dv}); "
                         "fla_usable has the same bound and the reference runs such heads on delta_rule_chunked")


def _width_at_least(d: int, widths) -> int:
    return next(w for w in widths if w >= d)


def _pad_last(x: torch.Tensor | None, width: int) -> torch.Tensor | None:
    if x is None or x.shape[-1] == width:
        return x
    return torch.nn.functional.pad(x, (0, width - x.shape[-1]))


def _pad_state(h: torch.Tensor | None, dk: int, dv: int) -> torch.Tensor | None:
    if h is None or h.shape[-2:] == (dk, dv):
        return h
    return torch.nn.functional.pad(h, (0, dv - h.shape[-1], 0, dk - h.shape[-2]))


def _chunk_widths(dk: int, dv: int, grad: bool) -> tuple[int, int]:
    """(K, V) a chunk-kernel call of these head widths runs at: K in
    CHUNK_HEAD_DIMS, V a multiple of 16, of 32 at K = 256 (in
    BACKWARD_HEAD_DIMS when a backward may follow)."""
    if grad:
        return _width_at_least(dk, BACKWARD_HEAD_DIMS), _width_at_least(dv, BACKWARD_HEAD_DIMS)
    kp = _width_at_least(dk, CHUNK_HEAD_DIMS)
    step = 32 if kp == CHUNK_WIDE_KEY else 16
    return kp, -(-dv // step) * step


def _chunk_shape_ok(dk: int, dv: int, dtype: torch.dtype) -> bool:
    """The chunk kernels take these widths and input dtype: K 64 or 128 with V
    a multiple of 16, or K 256 with 16-bit inputs and V a multiple of 32."""
    if dk == CHUNK_WIDE_KEY:
        return dtype in (torch.bfloat16, torch.float16) and dv % 32 == 0
    return dk in CHUNK_HEAD_DIMS and dv % 16 == 0


_CHUNK_SHAPES = ("chunk kernel supports K 64 or 128 with V a multiple of 16, and K 256 with bfloat16 or "
                 "float16 inputs and V a multiple of 32")


# ----------------------------------------------------------------------------
# Chunk kernel.
# ----------------------------------------------------------------------------
def chunk_fwd(q, k, v, g, beta, scale: float, h0=None, cu_seqlens=None, *,
              out_dtype: torch.dtype | None = None, output_final_state: bool = True,
              out: torch.Tensor | None = None):
    """Launch pbgdn_chunk_fwd. Returns (o [B,T,Hv,V] in out_dtype (default q's dtype),
    final [N,Hv,K,V] fp32 or None). `out` may supply the output buffer.
    Inference only (no backward; see gated_delta_chunk for the differentiable op)."""
    require_no_grad("chunk_fwd", q, k, v, g, beta, h0)
    return _chunk_fwd(q, k, v, g, beta, scale, h0, cu_seqlens, out_dtype=out_dtype,
                      output_final_state=output_final_state, out=out)


def _chunk_args(q, k, v, g, beta, h0, cu_seqlens):
    """Checked operands of a chunk-kernel call: (shapes, device, q, k, v, g, beta,
    h0 as contiguous fp32 or None, cu_seqlens as int32 or None, N)."""
    shapes = _shapes(q, k, v, g, beta)
    batch, length, hk, hv, dk, dv = shapes
    dev = _require_device(q, k, v, g, beta, h0, cu_seqlens)
    if not _chunk_shape_ok(dk, dv, q.dtype):
        raise ValueError(_CHUNK_SHAPES)
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
    return shapes, dev, q, k, v, g, beta, h0, cu_seqlens, nseq


def _chunk_fwd(q, k, v, g, beta, scale: float, h0=None, cu_seqlens=None, *,
               out_dtype: torch.dtype | None = None, output_final_state: bool = True,
               out: torch.Tensor | None = None):
    if out_dtype is not None and out_dtype not in (torch.float32, q.dtype):
        raise ValueError(f"chunk kernel writes o as float32 or q's dtype ({q.dtype}), not {out_dtype}")
    shapes, dev, q, k, v, g, beta, h0, cu_seqlens, nseq = _chunk_args(q, k, v, g, beta, h0, cu_seqlens)
    batch, length, hk, hv, dk, dv = shapes
    # (float32 inputs: the library scales v and h0 into its products' range
    # on the device and the results back, include/pbgdn.h)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty(batch, length, hv, dv, dtype=out_dtype, device=dev)
    elif out.shape != (batch, length, hv, dv) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B,T,Hv,V] tensor of out_dtype")
    final = torch.empty(nseq, hv, dk, dv, dtype=torch.float32, device=dev) if output_final_state else None
    lib = _lib.lib()
    ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq, _lib.DTYPE_CODES[q.dtype])
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
    pbgdn_chunk_fwd; no gather or scatter copies. Returns o [B,T,Hv,V].
    Inference only (no backward)."""
    require_no_grad("chunk_fwd_slots", q, k, v, g, beta, states)
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    if out_dtype is not None and out_dtype not in (torch.float32, q.dtype):
        raise ValueError(f"chunk kernel writes o as float32 or q's dtype ({q.dtype}), not {out_dtype}")
    dev = _require_device(q, k, v, g, beta, states, state_idx, cu_seqlens, has_initial_state)
    if not _chunk_shape_ok(dk, dv, q.dtype):
        raise ValueError(_CHUNK_SHAPES)
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
    ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq, _lib.DTYPE_CODES[q.dtype])
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
                  token_state_idx: torch.Tensor | None = None, state_resident: bool = False):
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
    written. With state_out None the new tensor starts as a copy of state_in,
    so the slots a call does not write keep their values there.

    state_resident: the caller steps this state pool again before much else
    passes through the GPU's 256 MB last-level cache (one layer stepped in a
    loop), so a one-token step keeps it cacheable (PBGDN_STATE_RESIDENT); the
    default streams it past the cache, as suits a model whose layers each keep
    a pool. Cache bits only: the results are the same.
    Inference only (no backward)."""
    require_no_grad("recurrent_fwd", q, k, v, g, beta, state_in)
    return _recurrent_fwd(q, k, v, g, beta, scale, state_in, state_out, state_idx, out_dtype=out_dtype, out=out,
                          token_state_idx=token_state_idx, state_resident=state_resident)


def _recurrent_fwd(q, k, v, g, beta, scale: float, state_in, state_out=None, state_idx=None, *,
                   out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
                   token_state_idx: torch.Tensor | None = None, state_resident: bool = False):
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
        # every slot the kernel leaves alone (unnamed, out-of-pool, and in verify
        # mode all but the token slots) keeps state_in's value
        partial = state_idx is not None or token_state_idx is not None or state_in.shape[0] != batch
        state_out = state_in.clone() if partial else torch.empty_like(state_in)
    elif state_out.shape != state_in.shape or state_out.dtype != state_in.dtype or not state_out.is_contiguous():
        raise ValueError("state_out must match state_in")
    if out is None:
        out = torch.empty(batch, length, hv, dv, dtype=out_dtype, device=dev)
    elif (out.shape != (batch, length, hv, dv) or out.dtype not in _lib.DTYPE_CODES or not out.is_contiguous()
          or out.device != dev):
        raise ValueError(f"out must be a contiguous [B,T,Hv,V] = {(batch, length, hv, dv)} float32, bfloat16 or "
                         "float16 tensor on the inputs' device")
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
        _lib.STATE_RESIDENT if state_resident else _lib.STATE_STREAM, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_recurrent_fwd")
    return out, state_out



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
    return _chunk_fwd(q, k, v, g, beta, scale, h0, cu_seqlens)


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
    ctx.save_for_backward(q, k, v, g, beta, h0, cu_seqlens)
    ctx.scale = scale


def _packed_backward(q, k, v, g, beta, h0, cu_seqlens, grad_o, grad_final, scale):
    """The backward of a packed call ([1, sum T] with cu_seqlens): each
    sequence's slice through the batched backward (its own h0 and final-state
    gradient), the gradients written back into the packed layout. An empty
    sequence's final state is its h0, so its dh0 is its final-state gradient."""
    bounds = [min(max(int(x), 0), q.shape[1]) for x in cu_seqlens.tolist()]
    nseq = len(bounds) - 1
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dg = torch.zeros(g.shape, dtype=torch.float32, device=g.device)
    dbeta = torch.zeros(beta.shape, dtype=beta.dtype if beta.dtype in (torch.float32, q.dtype) else torch.float32,
                        device=beta.device)
    dh0 = torch.zeros(nseq, v.shape[2], q.shape[3], v.shape[3], dtype=torch.float32, device=q.device)
    for n in range(nseq):
        lo, hi = bounds[n], max(bounds[n], bounds[n + 1])
        if hi == lo:
            if grad_final is not None:
                dh0[n] = grad_final[n]
            continue
        sl = slice(lo, hi)
        r = gated_delta_chunk_backward(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl],
                                       None if h0 is None else h0[n:n + 1], grad_o[:, sl],
                                       None if grad_final is None else grad_final[n:n + 1], scale)
        dq[:, sl], dk[:, sl], dv[:, sl], dg[:, sl], dbeta[:, sl] = r[0], r[1], r[2], r[3], r[4]
        dh0[n] = r[5][0]
    return dq, dk, dv, dg, dbeta, dh0


def _chunk_grad(ctx, grad_o, grad_final):
    """The reference's _fla_grad (gated_deltanet.py:266-275): zeros for a
    missing output gradient, each gradient in its input's dtype. A packed call
    (cu_seqlens) takes the batched backward sequence by sequence."""
    q, k, v, g, beta, h0, cu_seqlens = ctx.saved_tensors
    if grad_o is None:
        grad_o = torch.zeros(*q.shape[:2], v.shape[2], v.shape[3], dtype=q.dtype, device=q.device)
    if cu_seqlens is not None:
        dq, dk, dv, dg, dbeta, dh0 = _packed_backward(q, k, v, g, beta, h0, cu_seqlens, grad_o, grad_final,
                                                      ctx.scale)
    else:
        dq, dk, dv, dg, dbeta, dh0 = gated_delta_chunk_backward(q, k, v, g, beta, h0, grad_o, grad_final,
                                                                ctx.scale)
    return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
            None if h0 is None else dh0.to(h0.dtype), None, None)


gated_delta_chunk.register_autograd(_chunk_grad, setup_context=_chunk_setup)


def chunk_residuals(k, g, beta, *, a_dtype: torch.dtype | None = None):
    """Launch pbgdn_chunk_residuals: the gc and A that the reference's
    pseudobrain::gated_delta_chunk returns beside o and the final state
    (gated_deltanet.py:200-217, fla's residuals for 64-token chunks): gc
    [B,T,Hv] float32, the inclusive cumulative sum of g within each chunk, and
    A [B,T,Hv,64] in a_dtype (k's by default), row t of its chunk's
    T = (I + strict_lower(beta_t k_t.k_s exp(gc_t - gc_s)))^-1 (the `solve` of
    delta_rule_chunked, :141-149). k [B,T,Hk,K], g and beta [B,T,Hv]."""
    if k.ndim != 4 or g.ndim != 3 or g.shape[:2] != k.shape[:2] or beta.shape != g.shape:
        raise ValueError("expected k [B,T,Hk,K] and g, beta [B,T,Hv]")
    batch, length, hk, dk = k.shape
    hv = g.shape[2]
    if hk < 1 or hv % hk:
        raise ValueError("gated deltanet value heads must be a multiple of the key heads")
    dev = _require_device(k, g, beta)
    codes = _lib.DTYPE_CODES
    a_dtype = k.dtype if a_dtype is None else a_dtype
    if k.dtype not in codes or a_dtype not in codes:
        raise ValueError("k and A must be float32, bfloat16 or float16")
    k = k.contiguous()
    g = g.to(torch.float32).contiguous()
    beta = (beta if beta.dtype in codes else beta.to(torch.float32)).contiguous()
    gc = torch.empty(batch, length, hv, dtype=torch.float32, device=dev)
    a = torch.empty(batch, length, hv, CHUNK, dtype=a_dtype, device=dev)
    status = _lib.lib().pbgdn_chunk_residuals(
        _lib.ptr(k), codes[k.dtype], _lib.ptr(g), _lib.ptr(beta), codes[beta.dtype], _lib.ptr(gc), _lib.ptr(a),
        codes[a_dtype], batch, length, hk, hv, dk, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_residuals")
    return gc, a


def chunk_decumulate(gc):
    """Launch pbgdn_chunk_decumulate: g [B,T,Hv] float32 from the chunk-local
    cumulative sums gc that chunk_residuals returns."""
    if gc.ndim != 3:
        raise ValueError("expected gc [B,T,Hv]")
    dev = _require_device(gc)
    gc = gc.to(torch.float32).contiguous()
    g = torch.empty_like(gc)
    status = _lib.lib().pbgdn_chunk_decumulate(_lib.ptr(gc), _lib.ptr(g), gc.shape[0], gc.shape[1], gc.shape[2],
                                                _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_decumulate")
    return g


# The reference's own op pair, schemas and all (gated_deltanet.py:200-277):
# the forward returns fla's residuals gc and A beside o and the final state,
# and the backward takes them back. Here A is informational (the backward
# recomputes everything from g, which it recovers from gc).
_FLA_FWD_SCHEMA = ("(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor h0, float scale) "
                   "-> (Tensor, Tensor, Tensor, Tensor)")
_FLA_BWD_SCHEMA = ("(Tensor q, Tensor k, Tensor v, Tensor gc, Tensor beta, Tensor a, Tensor h0, Tensor grad_o, "
                   "Tensor grad_final, float scale) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")


def _fla_forward(q, k, v, g, beta, h0, scale):
    """(o [B,T,Hv,V] in q's dtype, final state fp32, gc, A) as _fla_chunk_op
    (gated_deltanet.py:205-216) returns them."""
    o, final = _chunk_fwd(q, k, v, g, beta, scale, h0, None)
    gc, a = chunk_residuals(k, g, beta)
    return o, final, gc, a


def _fla_forward_fake(q, k, v, g, beta, h0, scale):
    batch, length, _, dk = q.shape
    hv, dv = v.shape[2], v.shape[3]
    return (q.new_empty(batch, length, hv, dv), h0.new_empty(batch, hv, dk, dv, dtype=torch.float32),
            g.new_empty(batch, length, hv, dtype=torch.float32), k.new_empty(batch, length, hv, CHUNK))


def _fla_backward(q, k, v, gc, beta, a, h0, grad_o, grad_final, scale):
    """(dq, dk, dv, dg fp32, dbeta, dh0) in the dtypes _fla_chunk_backward_op
    returns (gated_deltanet.py:235-249); a is not read."""
    dq, dk, dv, dg, dbeta, dh0 = chunk_bwd(q, k, v, chunk_decumulate(gc), beta, scale, h0, grad_o, grad_final)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.float(), dbeta.to(beta.dtype), dh0.to(h0.dtype)


def _fla_backward_fake(q, k, v, gc, beta, a, h0, grad_o, grad_final, scale):
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            torch.empty_like(gc, dtype=torch.float32), torch.empty_like(beta), torch.empty_like(h0))


def _define_fla_ops(name: str):
    """The forward op `name` and its backward `name`_backward with the
    reference's schemas and autograd (_fla_setup, _fla_grad:
    gated_deltanet.py:259-277)."""
    fwd = torch.library.custom_op(name, _fla_forward, mutates_args=(), schema=_FLA_FWD_SCHEMA)
    bwd = torch.library.custom_op(f"{name}_backward", _fla_backward, mutates_args=(), schema=_FLA_BWD_SCHEMA)
    fwd.register_fake(_fla_forward_fake)
    bwd.register_fake(_fla_backward_fake)

    def setup(ctx, inputs, output):
        q, k, v, _g, beta, h0, scale = inputs
        _o, _final, gc, a = output
        ctx.save_for_backward(q, k, v, gc, beta, a, h0)
        ctx.scale = scale

    def grad(ctx, grad_o, grad_final, _grad_gc, _grad_a):
        q, k, v, gc, beta, a, h0 = ctx.saved_tensors
        if grad_o is None:
            grad_o = torch.zeros(*q.shape[:2], v.shape[2], v.shape[3], dtype=q.dtype, device=q.device)
        if grad_final is None:
            grad_final = torch.zeros(h0.shape, dtype=torch.float32, device=h0.device)
        dq, dk, dv, dg, dbeta, dh0 = bwd(q, k, v, gc, beta, a, h0, grad_o.to(q.dtype), grad_final.float(), ctx.scale)
        return dq, dk, dv, dg, dbeta, dh0, None

    fwd.register_autograd(grad, setup_context=setup)
    return fwd, bwd


# pbgdn::gated_delta_chunk_fla and pbgdn::gated_delta_chunk_fla_backward: the
# reference's schemas under this package's namespace, always defined.
gated_delta_chunk_fla, gated_delta_chunk_fla_backward = _define_fla_ops("pbgdn::gated_delta_chunk_fla")
_REFERENCE_OPS = {}


def register_reference_ops():
    """Define pseudobrain::gated_delta_chunk and
    pseudobrain::gated_delta_chunk_backward, the reference's op names and
    schemas (gated_deltanet.py:200-277), on these kernels, for code that calls
    torch.ops.pseudobrain.* in a process without the reference module (which
    defines them itself, on fla). Returns the two ops; a second call returns
    the same ones. Raises RuntimeError when the names exist already."""
    if not _REFERENCE_OPS:
        if hasattr(torch.ops.pseudobrain, "gated_delta_chunk"):
            raise RuntimeError("pseudobrain::gated_delta_chunk is already defined (is the reference module imported?)")
        _REFERENCE_OPS["ops"] = _define_fla_ops("pseudobrain::gated_delta_chunk")
    return _REFERENCE_OPS["ops"]


@torch.library.custom_op("pbgdn::recurrent_step_", mutates_args=("state",),
                         schema="(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor(a!) state, "
                                "Tensor? state_idx, float scale, bool state_resident=False) -> Tensor")
def recurrent_step_(q, k, v, g, beta, state, state_idx, scale, state_resident=False):
    """Decode step(s) updating `state` [S,Hv,K,V] in place; o in q's dtype.
    state_resident as recurrent_fwd's (the state's cache policy)."""
    out, _ = _recurrent_fwd(q, k, v, g, beta, scale, state, state, state_idx, out_dtype=q.dtype,
                            state_resident=state_resident)
    return out


@recurrent_step_.register_fake
def _(q, k, v, g, beta, state, state_idx, scale, state_resident=False):
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
    """The device prefill with the fla path's conventions (gated_deltanet.py:280-285):
    q/k/v at their own precision, fp32 state and decay; returns (o.float(), final).

    The chunk kernels through pbgdn::gated_delta_chunk, the head widths
    zero-padded to theirs: K <= 128 for every input dtype (differentiable for
    [B,T] batches with K, V <= 128), and 128 < K <= 256 for bfloat16 and
    float16 inputs (K padded to 256, no backward). float32 inputs with
    128 < K <= 256 run the recurrent kernel over every token (no backward)."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    _require_device(q, k, v, g, beta, h0, cu_seqlens)
    _head_bound(dk, dv)
    grad = grad_needed(q, k, v, g, beta, h0)
    if grad:
        if dk > BACKWARD_HEAD_DIMS[-1] or dv > BACKWARD_HEAD_DIMS[-1]:
            raise RuntimeError(f"the chunk backward is built for K, V <= {BACKWARD_HEAD_DIMS[-1]} "
                               f"(got K={dk}, V={dv}); call under torch.no_grad()")
    if dk > CHUNK_HEAD_DIMS[-2] and q.dtype not in (torch.bfloat16, torch.float16):
        return _recurrent_prefill(q, k, v, g, beta, scale, h0, cu_seqlens)
    kp, vp = _chunk_widths(dk, dv, grad)
    o, final = gated_delta_chunk(_pad_last(q, kp), _pad_last(k, kp), _pad_last(v, vp), g, beta,
                                 _pad_state(h0, kp, vp), cu_seqlens, float(scale))
    if (kp, vp) != (dk, dv):
        o, final = o[..., :dv], final[..., :dk, :dv].contiguous()
    return o.float(), final


def _recurrent_prefill(q, k, v, g, beta, scale, h0, cu_seqlens):
    """Prefill of key widths above the chunk kernel's (up to 256) through the
    recurrent kernel, every token in order (one workgroup per sequence and value
    head holds the state in registers for the whole sequence). Packed sequences
    run one call each."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    kp, vp = _width_at_least(dk, RECURRENT_HEAD_DIMS), _width_at_least(dv, RECURRENT_HEAD_DIMS)
    qp, kq, vq = _pad_last(q, kp), _pad_last(k, kp), _pad_last(v, vp)
    nseq = batch if cu_seqlens is None else cu_seqlens.numel() - 1
    if h0 is None:
        state = torch.zeros(nseq, hv, kp, vp, dtype=torch.float32, device=q.device)
    else:
        if h0.shape != (nseq, hv, dk, dv):
            raise ValueError(f"initial state must be [N,Hv,K,V] = {(nseq, hv, dk, dv)}")
        state = _pad_state(h0.to(torch.float32), kp, vp).contiguous().clone()
    o = torch.empty(batch, length, hv, vp, dtype=torch.float32, device=q.device)
    if cu_seqlens is None:
        _recurrent_fwd(qp, kq, vq, g, beta, scale, state, state, out=o)
    else:
        if batch != 1:
            raise ValueError("cu_seqlens needs B == 1 (sequences packed along T)")
        bounds = [min(max(int(x), 0), length) for x in cu_seqlens.tolist()]
        for n in range(nseq):
            lo, hi = bounds[n], max(bounds[n], bounds[n + 1])
            if hi == lo:
                continue
            sl = slice(lo, hi)
            idx = torch.full((1,), n, dtype=torch.int32, device=q.device)
            _recurrent_fwd(qp[:, sl], kq[:, sl], vq[:, sl], g[:, sl], beta[:, sl], scale, state, state, idx,
                           out=o[:, sl])
    return o[..., :dv].contiguous() if vp != dv else o, state[..., :dk, :dv].contiguous()


def delta_rule_sequential(q, k, v, g, beta, scale, h0):
    """Per-step recurrence on the device (gated_deltanet.py:93-107); the state is
    returned, not mutated. o is float32. With grad mode on and an input that
    requires grad the call goes through the chunk operator, which computes the
    same recurrence for any T and has a backward (K, V <= 128)."""
    batch, length, hk, hv, dk, dv = _shapes(q, k, v, g, beta)
    if h0.shape != (batch, hv, dk, dv):
        raise ValueError(f"initial state must be [B,Hv,K,V] = {(batch, hv, dk, dv)}")
    _require_device(q, k, v, g, beta, h0)
    _head_bound(dk, dv)
    if grad_needed(q, k, v, g, beta, h0):
        return delta_rule_hip(q, k, v, g, beta, scale, h0)
    kp, vp = _width_at_least(dk, RECURRENT_HEAD_DIMS), _width_at_least(dv, RECURRENT_HEAD_DIMS)
    state = _pad_state(h0.to(torch.float32), kp, vp).contiguous()
    o, final = _recurrent_fwd(_pad_last(q, kp), _pad_last(k, kp), _pad_last(v, vp), g, beta, scale, state, None,
                              out_dtype=torch.float32)
    if (kp, vp) != (dk, dv):
        o, final = o[..., :dv].contiguous(), final[..., :dk, :dv].contiguous()
    return o, final


def hip_usable(*tensors: torch.Tensor) -> bool:
    """The chunkwise device prefill applies (the fla_usable gate,
    gated_deltanet.py:189-197, which select_kernel consults only for calls
    longer than SEQUENTIAL_MAX tokens): every tensor on the device, a dtype
    the kernels read (float32, bfloat16, float16), head widths K, V <= 256,
    and a key width K <= 128 unless every other floating-point tensor is
    bfloat16 or float16 (the chunk kernel for 128 < K <= 256 takes 16-bit
    inputs; float32 ones would run token by token on the recurrent kernel, so
    fla or the reference's chunked path keeps them); when a gradient will be
    wanted, K, V <= 128 (the chunk backward's widths), so that a training call
    the device cannot differentiate stays on the reference's PyTorch path.
    tensors[0] is the matrix state [..., K, V]. Raises if the tensors are on a
    GPU but the library is missing: a GPU caller never silently loses the
    kernel."""
    if not tensors or not all(t.is_cuda for t in tensors):
        return False
    if not all(t.dtype in _lib.DTYPE_CODES for t in tensors if t.is_floating_point()):
        return False
    state = tensors[0]
    dv = state.shape[-1]
    dk = state.shape[-2] if state.ndim >= 2 else 0
    if dk > CHUNK_HEAD_DIMS[-1] or dv > MAX_HEAD_DIM:
        return False
    if grad_needed(*tensors) and (dk > BACKWARD_HEAD_DIMS[-1] or dv > BACKWARD_HEAD_DIMS[-1]):
        return False
    if dk > CHUNK_HEAD_DIMS[-2] and not all(t.dtype in (torch.bfloat16, torch.float16)
                                            for t in tensors[1:] if t.is_floating_point()):
        return False
    _lib.lib()
    return True


def select_kernel(backend: str, serial: bool, length: int, *tensors: torch.Tensor) -> str:
    """Kernel for one call (gated_deltanet.py:291-297), with "hip" in fla's place:
    sequential for serial calls and T <= SEQUENTIAL_MAX, the device prefill for
    the 'fused' backend when usable, else "chunked". On device tensors every
    name it returns runs here; "chunked" on CPU tensors is the reference's own
    PyTorch path (this package has none)."""
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
