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


def test_forward_only_guard():
    buf = torch.randn(3, 1, 4, 64)
    q = torch.zeros(64, requires_grad=True)
    with pytest.raises(NotImplementedError, match="forward-only"):
        kotodama_amd.route_static(buf, q, Norm(64), torch.ones(3, dtype=torch.bool), 3)


def test_fake_kernels_give_reference_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        buf = torch.empty(8, 2, 16, 128, dtype=torch.bfloat16, device="cuda")
        q = torch.empty(3, 128, dtype=torch.bfloat16, device="cuda")
        out, w, lse, inv, lg = torch.ops.attnres_hip.route(buf, 5, q, None, 1e-5, torch.bfloat16, True, True)
        assert out.shape == (3, 2, 16, 128) and out.dtype == torch.bfloat16
        assert w.shape == (3, 5, 2, 16) and lse.shape == (3, 2, 16)
        assert inv.shape == (2, 16, 5) and lg.shape == (3, 2, 16, 5)
        arena = torch.empty(9, 4, 1, 128, dtype=torch.bfloat16, device="cuda")
        o, w2, l2 = torch.ops.attnres_hip.block_step(arena, 3, True, arena[0], q[0], None, 1e-5, True)
        assert o.shape == (4, 1, 128) and w2.shape == (5, 4, 1)


def test_dtype_codes():
    assert ops.dtype_code(torch.bfloat16) == 1 and ops.dtype_code(torch.float32) == 0
    with pytest.raises(TypeError):
        ops.dtype_code(torch.float16)
