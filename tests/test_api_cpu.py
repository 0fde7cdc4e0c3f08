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
