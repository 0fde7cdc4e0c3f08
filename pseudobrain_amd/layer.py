"""The layer-side work around the recurrence on MI355X: the fused prologue and
epilogue of GatedDeltaNetLayer.forward (pseudobrain/gated_deltanet.py:403-441).

    z = proj(norm(x))                                 [q | k | v | gate | a | b]
    layer_prologue(z, tail, ...)  ->  q, k, v, g, beta, gate, new tail   (:415-427)
        one kernel (pbgdn_prologue_fwd): causal depthwise convolution over
        tail ++ [q | k | v] then SiLU (short_convolution, :314-338), q/k L2
        normalisation per key head (l2_normalize, :59-70), the gates
        g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
    o, S = gated_delta_rule(q, k, v, g, beta, K ** -0.5, S, "hip")    (:433-438)
    layer_epilogue(o, gate, o_norm, eps)  ->  hs                      (:439-441)
        one kernel (pbgdn_epilogue_fwd): per-head RMSNorm x o_norm x SiLU(gate)

For prefill, chunk_layer_fwd runs the operator and the epilogue as one call
(pbgdn_chunk_layer_fwd): where the wide scan takes the call, the scan applies
the epilogue to each chunk's output and writes hs directly.

For decode (one token per sequence), decode_layer_step does all of it in one
kernel (pbgdn_decode_layer_fwd), against slot pools of conv tails and states
updated in place, the way a serving cache holds them.

q and k come out [B,T,Hk,K] without the GQA repeat (:422-424): the operator
maps value head h to key head h // (Hv // Hk) itself. Both kernels run on the
GPU only; a missing library or a CPU tensor raises. They are inference
kernels: none has a backward, so each raises when grad mode is on and an input
(the projection, the tails, conv_weight, A_log, dt_bias, o_norm, the state)
requires grad, rather than returning results cut from the graph; training
keeps the reference's differentiable PyTorch layer around the operator.
"""
from __future__ import annotations

import torch

from . import _lib
from .gated_deltanet import (CHUNK, _chunk_args, _chunk_fwd, _require_device, _state_pool, chunk_fwd_slots,
                             require_no_grad)

NORM_EPS = 1e-5           # gated_deltanet.py:72
L2_MODES = ("max", "hf")  # gated_deltanet.py:57
PROLOGUE_KEY_DIMS = (64, 128)
EPILOGUE_VALUE_DIMS = (64, 128)
DECODE_HEAD_DIMS = (64, 128)
MAX_CONV = 4


def _dense_rows(x: torch.Tensor) -> bool:
    """Token rows of one stride across the batch, unit column stride (a column
    or token slice of a contiguous [B,T,C] tensor; with B = 1 the batch stride
    is not used, so a token slice of one batch row qualifies, and an empty
    tensor addresses no rows at all)."""
    if x.numel() == 0:  # no rows are addressed
        return True
    return x.stride(-1) == 1 and (x.shape[0] <= 1 or x.stride(0) == x.shape[1] * x.stride(1))


def _rows(x: torch.Tensor, name: str) -> int:
    """Row stride (elements per token) of a [B,T,C] tensor or column slice of one."""
    if x.ndim != 3 or not _dense_rows(x):
        raise ValueError(f"{name} must be a [B,T,C] tensor with unit column stride and dense rows "
                         "(a column slice of a contiguous projection is fine)")
    return x.stride(1)


def layer_prologue(z: torch.Tensor, tail: torch.Tensor | None, conv_weight: torch.Tensor | None,
                   A_log: torch.Tensor, dt_bias: torch.Tensor, heads: int, key_dim: int, value_heads: int,
                   value_dim: int, l2norm: str = "max", *, out_dtype: torch.dtype | None = None,
                   tail_out: torch.Tensor | None = None):
    """GatedDeltaNetLayer.forward from the projection to the operator's inputs
    (gated_deltanet.py:415-427) in one kernel.

    z [B,T,2*heads*key_dim + 2*value_heads*value_dim + 2*value_heads], split as
    the reference splits it (qkv, gate, decay); tail [B,conv-1,channels] (the
    last conv-1 inputs of q|k|v; any float dtype, kept); conv_weight
    [channels, conv] or None (SiLU only); A_log, dt_bias [value_heads].

    Returns (q [B,T,heads,key_dim], k, v [B,T,value_heads,value_dim] in
    out_dtype (default z's dtype, the operator's matmul precision), g, beta
    [B,T,value_heads] float32, gate (the [B,T,value_heads*value_dim] view of z
    the epilogue takes), new tail [B,conv-1,channels] in the tail's dtype,
    written to tail_out when given: a contiguous tensor of the tail's shape
    and dtype, which may be the tail itself)."""
    require_no_grad("layer_prologue", z, tail, conv_weight, A_log, dt_bias)
    if l2norm not in L2_MODES:
        raise ValueError(f"l2 normalization mode must be one of {L2_MODES}")
    if heads < 1 or value_heads % heads:
        raise ValueError("gated deltanet value heads must be a multiple of the key heads")
    if key_dim not in PROLOGUE_KEY_DIMS or value_dim % 8:
        raise ValueError(f"layer_prologue supports key widths {PROLOGUE_KEY_DIMS} and value widths "
                         "that are multiples of 8")
    channels = 2 * heads * key_dim + value_heads * value_dim
    vwidth = value_heads * value_dim
    if z.ndim != 3 or z.shape[-1] != channels + vwidth + 2 * value_heads:
        raise ValueError(f"z must be [B,T,{channels + vwidth + 2 * value_heads}] "
                         "([q | k | v | gate | a | b])")
    if not _dense_rows(z):
        z = z.contiguous()  # the kernel addresses token rows of one stride across the batch
    qkv, gate, decay = z.split((channels, vwidth, 2 * value_heads), dim=-1)
    batch, length, _ = z.shape
    dev = z.device
    if dev.type != "cuda":
        raise RuntimeError(f"pbgdn kernels run on ROCm devices only (got a tensor on '{dev}'); "
                           "this package has no CPU path")
    conv = 0 if conv_weight is None else conv_weight.shape[1]
    if conv_weight is not None:
        if conv_weight.shape != (channels, conv) or not 1 <= conv <= MAX_CONV:
            raise ValueError(f"conv_weight must be [{channels}, conv] with 1 <= conv <= {MAX_CONV}")
        conv_weight = conv_weight.to(device=dev, dtype=torch.float32).contiguous()
    tail_rows = max(conv - 1, 0)
    new_tail = tail
    if tail_rows:
        if tail is None or tail.shape != (batch, tail_rows, channels):
            raise ValueError(f"tail must be [B, conv-1, channels] = {(batch, tail_rows, channels)}")
        if tail_out is not None and tail_out.data_ptr() == tail.data_ptr() and not tail.is_contiguous():
            raise ValueError("an in-place tail must be contiguous")
        tail = tail.contiguous()
        if tail_out is None:
            new_tail = torch.empty_like(tail)
        else:
            if tail_out.shape != tail.shape or tail_out.dtype != tail.dtype or not tail_out.is_contiguous():
                raise ValueError("tail_out must be a contiguous tensor of the tail's shape and dtype")
            new_tail = tail_out
    out_dtype = z.dtype if out_dtype is None else out_dtype
    codes = _lib.DTYPE_CODES
    if z.dtype not in codes or out_dtype not in codes or (tail_rows and tail.dtype not in codes):
        raise ValueError("z, the tail and out_dtype must be float32, bfloat16 or float16")
    q = torch.empty(batch, length, heads, key_dim, dtype=out_dtype, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(batch, length, value_heads, value_dim, dtype=out_dtype, device=dev)
    g = torch.empty(batch, length, value_heads, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    a_log = A_log.to(device=dev, dtype=torch.float32).contiguous()
    dtb = dt_bias.to(device=dev, dtype=torch.float32).contiguous()
    if a_log.shape != (value_heads,) or dtb.shape != (value_heads,):
        raise ValueError(f"A_log and dt_bias must be [{value_heads}]")
    if _rows(qkv, "z") % 8 or qkv.data_ptr() % 16:  # the kernel reads 16-byte row pieces
        qkv = qkv.contiguous()
    status = _lib.lib().pbgdn_prologue_fwd(
        _lib.ptr(qkv), _rows(qkv, "z"), _lib.ptr(decay), _rows(decay, "z"), codes[z.dtype],
        _lib.ptr(tail) if tail_rows else None, _lib.ptr(new_tail) if tail_rows else None,
        codes[tail.dtype] if tail_rows else _lib.F32, _lib.ptr(conv_weight), conv, _lib.ptr(a_log),
        _lib.ptr(dtb), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[out_dtype], _lib.ptr(g), _lib.ptr(beta),
        batch, length, heads, value_heads, key_dim, value_dim, L2_MODES.index(l2norm), _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_prologue_fwd")
    return q, k, v, g, beta, gate, new_tail


def layer_prologue_varlen(z: torch.Tensor, cu_seqlens: torch.Tensor, tail_pool: torch.Tensor | None,
                          conv_weight: torch.Tensor | None, A_log: torch.Tensor, dt_bias: torch.Tensor, heads: int,
                          key_dim: int, value_heads: int, value_dim: int, slot_idx: torch.Tensor | None = None,
                          has_initial_state: torch.Tensor | None = None, l2norm: str = "max", *,
                          out_dtype: torch.dtype | None = None, tail_out: torch.Tensor | None = None):
    """layer_prologue over packed sequences, the way a serving engine batches
    prefill: z [T, width] (or [1, T, width]) holds N sequences back to back
    (cu_seqlens int32 [N+1]); sequence n convolves against its own tail,
    tail_pool[slot_idx[n]] ([S, conv-1, channels], any strides, e.g. a
    channel-major pool viewed as that), or a zero tail when
    has_initial_state[n] is False or the slot is outside the pool. The new
    tails go to tail_out (default: the pool itself, updated in place).
    Returns (q [1,T,heads,key_dim], k, v [1,T,value_heads,value_dim] in
    out_dtype, g, beta [1,T,value_heads] float32, gate view of z)."""
    require_no_grad("layer_prologue_varlen", z, tail_pool, conv_weight, A_log, dt_bias)
    if l2norm not in L2_MODES:
        raise ValueError(f"l2 normalization mode must be one of {L2_MODES}")
    if heads < 1 or value_heads % heads:
        raise ValueError("gated deltanet value heads must be a multiple of the key heads")
    if key_dim not in PROLOGUE_KEY_DIMS or value_dim % 8:
        raise ValueError(f"layer_prologue supports key widths {PROLOGUE_KEY_DIMS} and value widths "
                         "that are multiples of 8")
    if z.ndim == 3:
        if z.shape[0] != 1:
            raise ValueError("packed sequences: z must be [T, width] or [1, T, width]")
        z = z[0]
    channels = 2 * heads * key_dim + value_heads * value_dim
    vwidth = value_heads * value_dim
    if z.ndim != 2 or z.shape[-1] != channels + vwidth + 2 * value_heads:
        raise ValueError(f"z must be [T, {channels + vwidth + 2 * value_heads}] ([q | k | v | gate | a | b])")
    if z.stride(-1) != 1 or z.stride(0) % 8 or z.data_ptr() % 16:
        z = z.contiguous()
    dev = z.device
    if dev.type != "cuda":
        raise RuntimeError(f"pbgdn kernels run on ROCm devices only (got a tensor on '{dev}'); "
                           "this package has no CPU path")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D tensor [N+1]")
    cu = cu_seqlens.to(device=dev, dtype=torch.int32).contiguous()
    nseq = cu.numel() - 1
    length = z.shape[0]
    conv = 0 if conv_weight is None else conv_weight.shape[1]
    if conv_weight is not None:
        if conv_weight.shape != (channels, conv) or not 1 <= conv <= MAX_CONV:
            raise ValueError(f"conv_weight must be [{channels}, conv] with 1 <= conv <= {MAX_CONV}")
        conv_weight = conv_weight.to(device=dev, dtype=torch.float32).contiguous()
    codes = _lib.DTYPE_CODES
    strides = (0, 0, 0)
    nslots = 0
    if conv > 1:
        if (tail_pool is None or tail_pool.ndim != 3 or tail_pool.shape[1:] != (conv - 1, channels)
                or tail_pool.dtype not in codes):
            raise ValueError(f"tail_pool must be [S, conv-1, channels] = [S, {conv - 1}, {channels}]")
        tail_out = tail_pool if tail_out is None else tail_out
        if tail_out.shape != tail_pool.shape or tail_out.stride() != tail_pool.stride() or \
                tail_out.dtype != tail_pool.dtype:
            raise ValueError("tail_out must have the tail pool's shape, strides and dtype")
        strides = tail_pool.stride()
        nslots = tail_pool.shape[0]
    else:
        tail_pool = tail_out = None
    if slot_idx is not None:
        if slot_idx.shape != (nseq,):
            raise ValueError(f"slot_idx must be [N] = [{nseq}]")
        slot_idx = slot_idx.to(device=dev, dtype=torch.int32).contiguous()
    elif conv > 1 and nslots < nseq:
        raise ValueError("without slot_idx the tail pool needs a slot per sequence")
    if has_initial_state is not None:
        if has_initial_state.shape != (nseq,):
            raise ValueError(f"has_initial_state must be [N] = [{nseq}]")
        has_initial_state = has_initial_state.to(device=dev, dtype=torch.uint8).contiguous()
    out_dtype = z.dtype if out_dtype is None else out_dtype
    if z.dtype not in codes or out_dtype not in codes:
        raise ValueError("z and out_dtype must be float32, bfloat16 or float16")
    qkv, gate, decay = z.split((channels, vwidth, 2 * value_heads), dim=-1)
    q = torch.empty(1, length, heads, key_dim, dtype=out_dtype, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(1, length, value_heads, value_dim, dtype=out_dtype, device=dev)
    g = torch.empty(1, length, value_heads, dtype=torch.float32, device=dev)
    beta = torch.empty_like(g)
    a_log = A_log.to(device=dev, dtype=torch.float32).contiguous()
    dtb = dt_bias.to(device=dev, dtype=torch.float32).contiguous()
    if a_log.shape != (value_heads,) or dtb.shape != (value_heads,):
        raise ValueError(f"A_log and dt_bias must be [{value_heads}]")
    status = _lib.lib().pbgdn_prologue_varlen_fwd(
        _lib.ptr(qkv), z.stride(0), _lib.ptr(decay), z.stride(0), codes[z.dtype], _lib.ptr(cu), nseq,
        _lib.ptr(tail_pool), _lib.ptr(tail_out), codes[tail_pool.dtype] if tail_pool is not None else _lib.F32,
        *strides, _lib.ptr(slot_idx), _lib.ptr(has_initial_state), nslots, _lib.ptr(conv_weight), conv,
        _lib.ptr(a_log), _lib.ptr(dtb), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[out_dtype], _lib.ptr(g),
        _lib.ptr(beta), length, heads, value_heads, key_dim, value_dim, L2_MODES.index(l2norm),
        _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_prologue_varlen_fwd")
    return q, k, v, g, beta, gate[None]


def layer_epilogue(o: torch.Tensor, gate: torch.Tensor, o_norm: torch.Tensor, eps: float = NORM_EPS, *,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """hs = o rsqrt(mean(o^2) + eps) o_norm SiLU(gate) per (token, value head),
    reshaped to [B,T,Hv*V] in out_dtype (the reference's hidden dtype), as
    gated_deltanet.py:439-441 computes it, in one kernel. o [B,T,Hv,V] (the
    operator's output, any float dtype); gate [B,T,Hv*V] (the projection's
    gate columns, e.g. the view layer_prologue returns); o_norm [V]."""
    require_no_grad("layer_epilogue", o, gate, o_norm)
    if o.ndim != 4:
        raise ValueError("o must be [B,T,Hv,V]")
    batch, length, hv, dv = o.shape
    if dv not in EPILOGUE_VALUE_DIMS:
        raise ValueError(f"layer_epilogue supports value widths {EPILOGUE_VALUE_DIMS}")
    if gate.shape != (batch, length, hv * dv):
        raise ValueError(f"gate must be [B,T,Hv*V] = {(batch, length, hv * dv)}")
    if not eps >= 0:
        raise ValueError("eps must be >= 0")
    dev = o.device
    if dev.type != "cuda":
        raise RuntimeError(f"pbgdn kernels run on ROCm devices only (got a tensor on '{dev}'); "
                           "this package has no CPU path")
    codes = _lib.DTYPE_CODES
    if o.dtype not in codes or gate.dtype not in codes or out_dtype not in codes:
        raise ValueError("o, gate and out_dtype must be float32, bfloat16 or float16")
    o = o.contiguous()
    norm = o_norm.to(device=dev, dtype=torch.float32).contiguous()
    if norm.shape != (dv,):
        raise ValueError(f"o_norm must be [{dv}]")
    out = torch.empty(batch, length, hv * dv, dtype=out_dtype, device=dev)
    # one row stride across the batch, 16-byte row pieces
    if not _dense_rows(gate) or gate.stride(1) % 8 or gate.data_ptr() % 16:
        gate = gate.contiguous()
    status = _lib.lib().pbgdn_epilogue_fwd(
        _lib.ptr(o), codes[o.dtype], _lib.ptr(gate), _rows(gate, "gate"), codes[gate.dtype], _lib.ptr(norm),
        float(eps), _lib.ptr(out), codes[out_dtype], batch, length, hv, dv, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_epilogue_fwd")
    return out


def chunk_layer_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                    scale: float, h0: torch.Tensor | None, gate: torch.Tensor, o_norm: torch.Tensor,
                    eps: float = NORM_EPS, cu_seqlens: torch.Tensor | None = None, *,
                    out_dtype: torch.dtype = torch.float32, output_final_state: bool = True):
    """The layer core of a prefill (gated_deltanet.py:437-441): o, S =
    gated_delta_rule(q, k, v, g, beta, scale, h0) followed by hs = o rsqrt(mean
    (o^2) + eps) o_norm SiLU(gate), in one call (pbgdn_chunk_layer_fwd).
    Arguments as chunk_fwd and layer_epilogue; returns (hs [B,T,Hv*V] in
    out_dtype, final states [N,Hv,K,V] fp32 or None).

    With bf16/fp16 q, k, v at K = V = 128 and enough (sequence, value head)
    pairs for the wide scan, the epilogue is applied inside the scan (no o is
    written or re-read); otherwise the operator writes o and the epilogue runs
    as its own kernel. float32 inputs go through chunk_fwd (which scales them
    into the kernels' range) and layer_epilogue."""
    require_no_grad("chunk_layer_fwd", q, k, v, g, beta, h0, gate, o_norm)
    _epilogue_dtypes(gate, out_dtype)
    if q.dtype == torch.float32:
        o, final = _chunk_fwd(q, k, v, g, beta, scale, h0, cu_seqlens, output_final_state=output_final_state)
        return layer_epilogue(o, gate, o_norm, eps, out_dtype=out_dtype), final
    shapes, dev, q, k, v, g, beta, h0, cu_seqlens, nseq = _chunk_args(q, k, v, g, beta, h0, cu_seqlens)
    batch, length, hk, hv, dk, dv = shapes
    final = torch.empty(nseq, hv, dk, dv, dtype=torch.float32, device=dev) if output_final_state else None
    hs = _chunk_layer(shapes, dev, q, k, v, g, beta, scale, cu_seqlens, nseq, gate, o_norm, eps, out_dtype,
                      h0, final, _lib.F32, None, None, 0)
    return hs, final


def chunk_layer_fwd_slots(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                          scale: float, states: torch.Tensor, state_idx: torch.Tensor, gate: torch.Tensor,
                          o_norm: torch.Tensor, eps: float = NORM_EPS, cu_seqlens: torch.Tensor | None = None,
                          has_initial_state: torch.Tensor | None = None, *,
                          out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """chunk_layer_fwd against a pool of state slots, as chunk_fwd_slots
    (vLLM's per-request slots): sequence n starts from states[state_idx[n]]
    (zeros where has_initial_state[n] is False or the slot is outside the
    pool) and its final state goes back to that slot in the pool's dtype.
    Returns hs [B,T,Hv*V] in out_dtype."""
    require_no_grad("chunk_layer_fwd_slots", q, k, v, g, beta, states, gate, o_norm)
    _epilogue_dtypes(gate, out_dtype)
    if q.dtype == torch.float32:
        o = chunk_fwd_slots(q, k, v, g, beta, scale, states, state_idx, cu_seqlens, has_initial_state)
        return layer_epilogue(o, gate, o_norm, eps, out_dtype=out_dtype)
    shapes, dev, q, k, v, g, beta, _, cu_seqlens, nseq = _chunk_args(q, k, v, g, beta, None, cu_seqlens)
    batch, length, hk, hv, dk, dv = shapes
    _require_device(states, state_idx, has_initial_state)
    _state_pool(states, hv, dk, dv)
    if states.device != dev:
        raise ValueError("states must be on the device of q")
    if state_idx.shape != (nseq,):
        raise ValueError(f"state_idx must be [N] = [{nseq}]")
    state_idx = state_idx.to(device=dev, dtype=torch.int32).contiguous()
    if has_initial_state is not None:
        if has_initial_state.shape != (nseq,):
            raise ValueError(f"has_initial_state must be [N] = [{nseq}]")
        has_initial_state = has_initial_state.to(device=dev, dtype=torch.uint8).contiguous()
    return _chunk_layer(shapes, dev, q, k, v, g, beta, scale, cu_seqlens, nseq, gate, o_norm, eps, out_dtype,
                        states, states, _lib.DTYPE_CODES[states.dtype], state_idx, has_initial_state,
                        states.shape[0])


def _epilogue_dtypes(gate, out_dtype):
    codes = _lib.DTYPE_CODES
    if out_dtype not in codes or gate.dtype not in codes:
        raise ValueError("gate and out_dtype must be float32, bfloat16 or float16")


def _chunk_layer(shapes, dev, q, k, v, g, beta, scale, cu_seqlens, nseq, gate, o_norm, eps, out_dtype,
                 h0, ht, state_code, state_idx, has_initial_state, num_states):
    """pbgdn_chunk_layer_fwd on checked operands; returns hs."""
    batch, length, hk, hv, dk, dv = shapes
    if dv not in EPILOGUE_VALUE_DIMS:
        raise ValueError(f"the epilogue supports value widths {EPILOGUE_VALUE_DIMS}")
    if gate.shape != (batch, length, hv * dv):
        raise ValueError(f"gate must be [B,T,Hv*V] = {(batch, length, hv * dv)}")
    if not eps >= 0:
        raise ValueError("eps must be >= 0")
    if gate.device != dev:
        raise ValueError("gate must be on the device of q")
    norm = o_norm.to(device=dev, dtype=torch.float32).contiguous()
    if norm.shape != (dv,):
        raise ValueError(f"o_norm must be [{dv}]")
    # one row stride across the batch, 16-byte row pieces
    if not _dense_rows(gate) or gate.stride(1) % 8 or gate.data_ptr() % 16:
        gate = gate.contiguous()
    codes = _lib.DTYPE_CODES
    hs = torch.empty(batch, length, hv * dv, dtype=out_dtype, device=dev)
    lib = _lib.lib()
    # o only where the epilogue runs as a pass of its own (the wide scan writes hs itself)
    gate_stride = _rows(gate, "gate")
    fuses = lib.pbgdn_chunk_layer_fuses(codes[q.dtype], codes[gate.dtype], codes[out_dtype], gate_stride, nseq, hv,
                                        dk, dv)
    o = None if fuses == 1 else torch.empty(batch, length, hv, dv, dtype=q.dtype, device=dev)
    ws_bytes = lib.pbgdn_chunk_workspace_size(batch, length, hv, nseq, _lib.DTYPE_CODES[q.dtype])
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    status = lib.pbgdn_chunk_layer_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), codes[q.dtype], _lib.ptr(g), _lib.ptr(beta), codes[beta.dtype],
        _lib.ptr(h0), _lib.ptr(ht), state_code, _lib.ptr(state_idx), _lib.ptr(has_initial_state), num_states,
        _lib.ptr(cu_seqlens), nseq, _lib.ptr(gate), gate_stride, codes[gate.dtype], _lib.ptr(norm),
        float(eps), _lib.ptr(hs), codes[out_dtype], _lib.ptr(o), batch, length, hk, hv, dk, dv, float(scale),
        CHUNK, _lib.ptr(workspace), ws_bytes, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_chunk_layer_fwd")
    return hs


def decode_layer_step(z: torch.Tensor, conv_state: torch.Tensor | None, conv_weight: torch.Tensor | None,
                      A_log: torch.Tensor, dt_bias: torch.Tensor, state: torch.Tensor, o_norm: torch.Tensor,
                      heads: int, key_dim: int, value_heads: int, value_dim: int,
                      state_idx: torch.Tensor | None = None, l2norm: str = "max", eps: float = NORM_EPS, *,
                      scale: float | None = None, out_dtype: torch.dtype = torch.float32,
                      state_resident: bool = False) -> torch.Tensor:
    """One decode token per sequence through GatedDeltaNetLayer.forward from the
    projection to hs (gated_deltanet.py:415-441) in one kernel: the short
    convolution against the carried tail, SiLU, q/k L2 norms, the gates, the
    recurrent step (delta_rule_sequential, :93-107, with q, k, v kept float32
    as on that path), and the RMSNorm x o_norm x SiLU(gate) epilogue.

    z [B, 2*heads*key_dim + 2*value_heads*value_dim + 2*value_heads] (or
    [B, 1, ...]) is the projection of the token; conv_state [S, conv-1,
    channels] is the pool of tails (any strides: a channel-major pool viewed as
    [S, conv-1, channels] works) and state [S, Hv, K, V] the pool of recurrent
    states (float32, bfloat16 or float16), both updated in place at slot
    state_idx[b] (int32 [B], or None for slot b; a slot outside the pools
    touches nothing and gives zeros). Returns hs [B, value_heads*value_dim] in
    out_dtype. state_resident: the state's cache policy, as recurrent_fwd's
    (the default streams it, as a model whose layers each keep a pool needs)."""
    require_no_grad("decode_layer_step", z, conv_state, conv_weight, A_log, dt_bias, state, o_norm)
    if l2norm not in L2_MODES:
        raise ValueError(f"l2 normalization mode must be one of {L2_MODES}")
    if heads < 1 or value_heads % heads:
        raise ValueError("gated deltanet value heads must be a multiple of the key heads")
    if key_dim not in DECODE_HEAD_DIMS or value_dim not in DECODE_HEAD_DIMS:
        raise ValueError(f"decode_layer_step supports key and value widths {DECODE_HEAD_DIMS}")
    if z.ndim == 3 and z.shape[1] == 1:
        z = z[:, 0]
    channels = 2 * heads * key_dim + value_heads * value_dim
    width = channels + value_heads * value_dim + 2 * value_heads
    if z.ndim != 2 or z.shape[1] != width:
        raise ValueError(f"z must be [B, {width}] ([q | k | v | gate | a | b] of one token)")
    if z.stride(1) != 1:
        z = z.contiguous()
    dev = z.device
    if dev.type != "cuda":
        raise RuntimeError(f"pbgdn kernels run on ROCm devices only (got a tensor on '{dev}'); "
                           "this package has no CPU path")
    codes = _lib.DTYPE_CODES
    batch = z.shape[0]
    if (state.ndim != 4 or state.shape[1:] != (value_heads, key_dim, value_dim) or state.dtype not in codes
            or not state.is_contiguous()):
        raise ValueError(f"state must be a contiguous [S,{value_heads},{key_dim},{value_dim}] float32, bfloat16 "
                         "or float16 pool")
    conv = 0 if conv_weight is None else conv_weight.shape[1]
    if conv_weight is not None:
        if conv_weight.shape != (channels, conv) or not 1 <= conv <= MAX_CONV:
            raise ValueError(f"conv_weight must be [{channels}, conv] with 1 <= conv <= {MAX_CONV}")
        conv_weight = conv_weight.to(device=dev, dtype=torch.float32).contiguous()
    if conv > 1:
        if (conv_state is None or conv_state.ndim != 3 or conv_state.shape[1:] != (conv - 1, channels)
                or conv_state.shape[0] != state.shape[0] or conv_state.dtype not in codes):
            raise ValueError(f"conv_state must be a [S, conv-1, channels] = [{state.shape[0]}, {conv - 1}, "
                             f"{channels}] pool with the state pool's slots")
        strides = conv_state.stride()
    else:
        conv_state, strides = None, (0, 0, 0)
    if state_idx is None:
        if state.shape[0] < batch:
            raise ValueError("without state_idx the pools need a slot per sequence")
    else:
        if state_idx.shape != (batch,):
            raise ValueError("state_idx must be [B]")
        state_idx = state_idx.to(device=dev, dtype=torch.int32).contiguous()
    if z.dtype not in codes or out_dtype not in codes:
        raise ValueError("z and out_dtype must be float32, bfloat16 or float16")
    a_log = A_log.to(device=dev, dtype=torch.float32).contiguous()
    dtb = dt_bias.to(device=dev, dtype=torch.float32).contiguous()
    norm = o_norm.to(device=dev, dtype=torch.float32).contiguous()
    if a_log.shape != (value_heads,) or dtb.shape != (value_heads,) or norm.shape != (value_dim,):
        raise ValueError(f"A_log and dt_bias must be [{value_heads}], o_norm [{value_dim}]")
    if not eps >= 0:
        raise ValueError("eps must be >= 0")
    hs = torch.empty(batch, value_heads * value_dim, dtype=out_dtype, device=dev)
    status = _lib.lib().pbgdn_decode_layer_fwd(
        _lib.ptr(z), z.stride(0), codes[z.dtype], _lib.ptr(conv_state),
        codes[conv_state.dtype] if conv_state is not None else _lib.F32, *strides, _lib.ptr(conv_weight), conv,
        _lib.ptr(a_log), _lib.ptr(dtb), L2_MODES.index(l2norm), _lib.ptr(state), codes[state.dtype],
        _lib.ptr(state_idx), state.shape[0], _lib.ptr(norm), float(eps), _lib.ptr(hs), codes[out_dtype], batch,
        heads, value_heads, key_dim, value_dim, float(key_dim ** -0.5 if scale is None else scale),
        _lib.STATE_RESIDENT if state_resident else _lib.STATE_STREAM, _lib.stream_handle(dev))
    _lib.check(status, "pbgdn_decode_layer_fwd")
    return hs
