"""Host-side logic of pseudobrain_amd.gated_deltanet (no GPU): dispatch, argument
checks and the custom ops' shape inference. The package has no CPU compute path:
CPU tensors are refused."""
import pytest
import torch

from pseudobrain_amd import gated_deltanet as gd


def inputs(batch=1, length=8, hk=2, hv=4, dk=64, dv=64, dtype=torch.bfloat16):
    q = torch.randn(batch, length, hk, dk).to(dtype)
    k = torch.randn(batch, length, hk, dk).to(dtype)
    v = torch.randn(batch, length, hv, dv).to(dtype)
    g = -torch.rand(batch, length, hv)
    beta = torch.rand(batch, length, hv)
    h0 = torch.zeros(batch, hv, dk, dv)
    return q, k, v, g, beta, h0


def test_select_kernel_mirrors_the_reference_rules():
    q, k, v, g, beta, h0 = inputs()
    assert gd.select_kernel("fused", True, 100, h0, q) == "sequential"
    assert gd.select_kernel("fused", False, gd.SEQUENTIAL_MAX, h0, q) == "sequential"
    # CPU tensors: the chunk kernel does not apply, as fla_usable on CPU tensors
    assert gd.select_kernel("fused", False, 100, h0, q) == "chunked"
    assert gd.select_kernel("reference", False, 100, h0, q) == "chunked"
    assert not gd.hip_usable(h0, q)
    assert not gd.hip_usable()


def test_unknown_kernel_raises_value_error():
    with pytest.raises(ValueError, match="kernel must be one of"):
        gd.gated_delta_rule(*inputs()[:5], 0.1, inputs()[5], kernel="fla")


@pytest.mark.parametrize("kernel", ["hip", "chunked", "sequential"])
def test_cpu_tensors_are_refused(kernel):
    q, k, v, g, beta, h0 = inputs()
    with pytest.raises(RuntimeError, match="ROCm devices only"):
        gd.gated_delta_rule(q, k, v, g, beta, 0.125, h0, kernel=kernel)


def test_shape_errors():
    q, k, v, g, beta, h0 = inputs()
    with pytest.raises(ValueError, match="multiple of the key heads"):
        gd.chunk_fwd(q, k, v[:, :, :3], g[:, :, :3], beta[:, :, :3], 0.1)
    with pytest.raises(ValueError, match=r"\[B,T,Hv\]"):
        gd.chunk_fwd(q, k, v, g[:, :4], beta, 0.1)
    with pytest.raises(ValueError):
        gd.chunk_fwd(q, k[:, :4], v, g, beta, 0.1)
    with pytest.raises(ValueError, match="initial state"):
        gd.delta_rule_sequential(q, k, v, g, beta, 0.1, h0[:, :2])
    with pytest.raises(ValueError, match="float32 or q's dtype"):
        gd.chunk_fwd(q, k, v, g, beta, 0.1, out_dtype=torch.float16 if q.dtype != torch.float16 else torch.bfloat16)


def test_custom_ops_are_registered_with_shape_inference():
    from torch._subclasses.fake_tensor import FakeTensorMode
    assert hasattr(torch.ops.pbgdn, "gated_delta_chunk")
    assert hasattr(torch.ops.pbgdn, "recurrent_step_")
    assert hasattr(torch.ops.pbgdn, "chunk_slots_")
    with FakeTensorMode():
        q, k, v, g, beta, h0 = inputs(batch=1, length=300, hk=2, hv=4, dk=128, dv=64)
        cu = torch.zeros(4, dtype=torch.int32)
        o, final = torch.ops.pbgdn.gated_delta_chunk(q, k, v, g, beta, h0[:1].expand(3, -1, -1, -1),
                                                     cu, 0.1)
        assert o.shape == (1, 300, 4, 64) and o.dtype == torch.bfloat16
        assert final.shape == (3, 4, 128, 64) and final.dtype == torch.float32
        state = torch.zeros(5, 4, 128, 64)
        o2 = torch.ops.pbgdn.recurrent_step_(q[:, :1], k[:, :1], v[:, :1], g[:, :1], beta[:, :1],
                                             state, None, 0.1)
        assert o2.shape == (1, 1, 4, 64)
        pool = torch.zeros(6, 4, 128, 64, dtype=torch.bfloat16)
        o3 = torch.ops.pbgdn.chunk_slots_(q, k, v, g, beta, pool, torch.zeros(1, dtype=torch.int32), None, None,
                                          0.1)
        assert o3.shape == (1, 300, 4, 64) and o3.dtype == torch.bfloat16


def test_reference_schema_ops_infer_the_reference_shapes():
    """pbgdn::gated_delta_chunk_fla and its backward have the reference's
    schemas (gated_deltanet.py:200-256) and its fake outputs: o, final fp32,
    gc fp32 [B,T,H], A [B,T,H,64] in k's dtype; the backward's gradients like
    its inputs."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    assert "(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor h0, float scale)" in str(
        torch.ops.pbgdn.gated_delta_chunk_fla.default._schema)
    assert "Tensor gc, Tensor beta, Tensor a, Tensor h0, Tensor grad_o, Tensor grad_final, float scale" in str(
        torch.ops.pbgdn.gated_delta_chunk_fla_backward.default._schema)
    with FakeTensorMode():
        q, k, v, g, beta, h0 = inputs(batch=2, length=100, hk=4, hv=4, dk=64, dv=64)
        o, final, gc, a = torch.ops.pbgdn.gated_delta_chunk_fla(q, k, v, g, beta, h0, 0.125)
        assert o.shape == (2, 100, 4, 64) and final.shape == (2, 4, 64, 64) and final.dtype == torch.float32
        assert gc.shape == (2, 100, 4) and gc.dtype == torch.float32
        assert a.shape == (2, 100, 4, 64) and a.dtype == k.dtype
        grads = torch.ops.pbgdn.gated_delta_chunk_fla_backward(q, k, v, gc, beta, a, h0, o, final, 0.125)
        assert [x.shape for x in grads] == [q.shape, k.shape, v.shape, gc.shape, beta.shape, h0.shape]
        assert grads[3].dtype == torch.float32


def test_entry_points_without_backward_refuse_grad_before_anything_runs():
    """With grad mode on, a grad-requiring input to an entry point that has no
    backward raises (before any device work) instead of silently detaching."""
    from pseudobrain_amd import layer
    q, k, v, g, beta, h0 = inputs()
    v.requires_grad_(True)
    for fn in (lambda: gd.chunk_fwd(q, k, v, g, beta, 0.1, h0),
               lambda: gd.recurrent_fwd(q, k, v, g, beta, 0.1, h0),
               lambda: gd.chunk_fwd_slots(q, k, v, g, beta, 0.1, h0, torch.zeros(1, dtype=torch.int32))):
        with pytest.raises(RuntimeError, match="no backward"):
            fn()
    z = torch.randn(1, 4, 2 * 2 * 64 + 2 * 4 * 64 + 8, requires_grad=True)
    with pytest.raises(RuntimeError, match="layer_prologue has no backward"):
        layer.layer_prologue(z, None, None, torch.zeros(4), torch.zeros(4), 2, 64, 4, 64)
    weight = torch.randn(2 * 2 * 64 + 4 * 64, 4, requires_grad=True)
    with pytest.raises(RuntimeError, match="no backward"):
        layer.layer_prologue(z.detach(), torch.zeros(1, 3, weight.shape[0]), weight, torch.zeros(4),
                             torch.zeros(4), 2, 64, 4, 64)
    o = torch.randn(1, 4, 4, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match="layer_epilogue has no backward"):
        layer.layer_epilogue(o, torch.randn(1, 4, 256), torch.ones(64))
    with pytest.raises(RuntimeError, match="decode_layer_step has no backward"):
        layer.decode_layer_step(z[:, 0], None, None, torch.zeros(4), torch.zeros(4),
                                torch.zeros(1, 4, 64, 64), torch.ones(64, requires_grad=True), 2, 64, 4, 64)
    gate = torch.randn(q.shape[0], q.shape[1], v.shape[2] * v.shape[3])
    with pytest.raises(RuntimeError, match="chunk_layer_fwd has no backward"):
        layer.chunk_layer_fwd(q, k, v, g, beta, 0.1, h0, gate, torch.ones(v.shape[3]))
    with pytest.raises(RuntimeError, match="chunk_layer_fwd_slots has no backward"):
        layer.chunk_layer_fwd_slots(q, k, v, g, beta, 0.1, h0, torch.zeros(1, dtype=torch.int32), gate,
                                    torch.ones(v.shape[3]))
    # under no_grad the guard is silent (and the CPU tensors are then refused)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm devices only"):
        gd.chunk_fwd(q, k, v, g, beta, 0.1, h0)


def test_head_widths_route_to_kernels_that_run():
    """The widths a call runs at: the chunk kernels' K in {64, 128} with V a
    multiple of 16, and K 256 (16-bit inputs) with V a multiple of 32 (the
    backward's {64, 128} when grad is wanted); float32 keys above 128 go to
    the recurrent kernel; above 256 there is no device path."""
    assert gd._chunk_widths(128, 128, False) == (128, 128)
    assert gd._chunk_widths(200, 100, False) == (256, 128)
    assert gd._chunk_widths(256, 80, False) == (256, 96)
    assert gd._chunk_shape_ok(256, 96, torch.bfloat16) and gd._chunk_shape_ok(256, 64, torch.float16)
    assert not gd._chunk_shape_ok(256, 64, torch.float32) and not gd._chunk_shape_ok(256, 48, torch.bfloat16)
    assert gd._chunk_shape_ok(128, 48, torch.float32) and not gd._chunk_shape_ok(96, 64, torch.bfloat16)
    assert gd._chunk_widths(96, 40, False) == (128, 48)
    assert gd._chunk_widths(32, 16, False) == (64, 16)
    assert gd._chunk_widths(96, 40, True) == (128, 64)
    assert gd._chunk_widths(64, 100, True) == (64, 128)
    assert gd._width_at_least(200, gd.RECURRENT_HEAD_DIMS) == 256
    with pytest.raises(ValueError, match="above 256"):
        gd._head_bound(300, 64)
    # zero padding of the state: the original block is kept, the rest is zero
    h = torch.randn(2, 3, 5, 7)
    p = gd._pad_state(h, 8, 16)
    assert p.shape == (2, 3, 8, 16) and torch.equal(p[..., :5, :7], h)
    assert torch.count_nonzero(p[..., 5:, :]) == 0 and torch.count_nonzero(p[..., :, 7:]) == 0
    # float64 (the reference's check precision) is not a device dtype: the gate says so
    assert not gd.hip_usable(torch.zeros(1, 2, 64, 64, dtype=torch.float64))


def test_layer_row_stride_accepts_token_slices_of_one_batch_row():
    """The layer kernels address token rows of one stride across the batch:
    a token slice of a single batch row keeps the full tensor's batch stride,
    which a batch of one never uses, so it passes; with B = 2 it does not."""
    from pseudobrain_amd.layer import _rows
    z = torch.empty(1, 100, 64)
    assert _rows(z[:, 10:60], "z") == 64
    assert _rows(z[:, 10:60, 16:48], "z") == 64  # a column slice as well
    with pytest.raises(ValueError, match="dense rows"):
        _rows(torch.empty(2, 100, 64)[:, 10:60], "z")
