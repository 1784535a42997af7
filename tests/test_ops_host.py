"""Host-side behaviour of the torch layer that needs no GPU."""

import pytest
import torch

import kotodama_amd
from kotodama_amd import ops
from kotodama_amd.flash_attn_res import phase_1_batched_attention_triton_op


class Norm(torch.nn.Module):
    def __init__(self, d):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(d))
        self.eps = 1e-5


def test_cpu_tensors_raise_no_fallback():
    buf = torch.randn(3, 1, 4, 64)
    with torch.no_grad():
        with pytest.raises(RuntimeError, match="no CPU path"):
            kotodama_amd.route_static(buf, torch.zeros(64), Norm(64), torch.ones(3, dtype=torch.bool), 3)
        with pytest.raises(RuntimeError, match="no CPU path"):
            phase_1_batched_attention_triton_op(buf, torch.zeros(2, 64), 1e-5)


def test_forward_only_guards():
    # the weights helper and the arena engine have no backward
    buf = torch.randn(3, 1, 4, 64, requires_grad=True)
    q = torch.zeros(64, requires_grad=True)
    with pytest.raises(NotImplementedError, match="forward-only"):
        kotodama_amd.route_weights(buf, 3, q, Norm(64))
    with pytest.raises(NotImplementedError, match="forward-only"):
        ops.check_forward_only(buf)


def test_single_query_routing_is_differentiable_up_to_the_device_check():
    # route_static with requires_grad reaches the device check (no forward-only guard)
    buf = torch.randn(3, 1, 4, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kotodama_amd.route_static(buf, torch.zeros(64, requires_grad=True), Norm(64), torch.ones(3, dtype=torch.bool), 3)


def test_fake_kernels_give_reference_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        buf = torch.empty(8, 2, 16, 128, dtype=torch.bfloat16, device="cuda")
        q = torch.empty(3, 128, dtype=torch.bfloat16, device="cuda")
        out, w, lse, inv, lg = torch.ops.attnres_hip.route(buf, 5, q, None, 1e-5, torch.bfloat16, True, True)
        assert out.shape == (3, 2, 16, 128) and out.dtype == torch.bfloat16
        assert w.shape == (3, 5, 2, 16) and lse.shape == (3, 2, 16)
        assert inv.shape == (2, 16, 5) and lg.shape == (3, 2, 16, 5)
        gb, gq, gg = torch.ops.attnres_hip.route_bwd(buf, 5, q[0], None, 1e-5, out[0], None)
        assert gb.shape == buf.shape and gq.shape == (128,) and gg.numel() == 0
        gl, gq2, gg2 = torch.ops.attnres_hip.route_list_bwd([buf[0], buf[1]], q[0], q[1], 1e-5, out[0], lse[0])
        assert len(gl) == 2 and gl[0].shape == buf[0].shape and gg2.shape == (128,)
        gb3, gq3, _ = torch.ops.attnres_hip.route_bwd(buf, 5, q, None, 1e-5, out, lse)
        assert gq3.shape == (3, 128)
        gp, gq4, gi, glse = torch.ops.attnres_hip.merge_bwd(buf[0], q[0], out[0], lse[0], 1e-5, out[0])
        assert gp.shape == buf[0].shape and gi.shape == out[0].shape and glse.shape == lse[0].shape
        arena = torch.empty(9, 4, 1, 128, dtype=torch.bfloat16, device="cuda")
        o, w2, l2 = torch.ops.attnres_hip.block_step(arena, 3, True, arena[0], q[0], None, 1e-5, True)
        assert o.shape == (4, 1, 128) and w2.shape == (5, 4, 1)


def test_dtype_codes():
    assert ops.dtype_code(torch.bfloat16) == 1 and ops.dtype_code(torch.float32) == 0
    with pytest.raises(TypeError):
        ops.dtype_code(torch.float16)
