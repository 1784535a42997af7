"""torch.compile and torch.library.opcheck over the attnres_hip ops (GPU).

The reference compiles its model for training (src/training/train.py:314-324)
and builds ``_route_static`` so that "torch.compile [can] trace a single graph
without breaks" (llama.py:615-616).  Here:

* ``torch.library.opcheck`` on every registered op (route, route_list,
  route_bwd, route_list_bwd, merge, merge_bwd, block_step): schema and
  mutation annotations, the autograd registration, the fake (meta) kernels
  against the real outputs, and AOT dispatch with dynamic shapes;
* the reference-shaped training loop (pad + stack before each routing call,
  ``route_static`` swapped in) under ``torch.compile(fullgraph=True)`` —
  Dynamo + AOTAutograd with the ops' fake kernels (``aot_eager``) and the
  reference's default backend (``inductor``) — forward and backward, against
  the eager run and the float64 restatement of the same loop.
"""

import copy

import pytest
import torch

import kotodama_amd
from kotodama_amd import ops

from ._tiny_model import TinyModel, training_forward

pytestmark = pytest.mark.gpu


def _src(gpu, shape, dtype, seed, grad=False):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=gpu)).to(dtype).requires_grad_(grad)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_opcheck_forward_ops(gpu, dtype):
    d = 256
    buf = _src(gpu, (4, 2, 8, d), dtype, 1, grad=True)
    q = (_src(gpu, (d,), dtype, 2) * 0.1).requires_grad_(True)
    gain = (1 + 0.1 * _src(gpu, (d,), dtype, 3)).requires_grad_(True)
    qs = (_src(gpu, (3, d), dtype, 4) * 0.1).requires_grad_(True)
    torch.library.opcheck(ops.route, (buf, 3, q, gain, 1e-5, dtype, True, True))
    torch.library.opcheck(ops.route, (buf, 4, qs, None, 1e-5, torch.bfloat16, True, False))
    srcs = [_src(gpu, (2, 8, d), dtype, 10 + i, grad=True) for i in range(3)]
    torch.library.opcheck(ops.route_list, (srcs, q, gain, 1e-5, dtype, True, False))
    p = _src(gpu, (2, 8, d), dtype, 20, grad=True)
    inter = _src(gpu, (2, 8, d), dtype, 21, grad=True)
    lse = _src(gpu, (2, 8), torch.float32, 22, grad=True)
    torch.library.opcheck(ops.merge, (p, q, inter, lse, 1e-5))


def test_opcheck_backward_ops(gpu):
    d, dt = 256, torch.bfloat16
    buf = _src(gpu, (4, 2, 8, d), dt, 1)
    q = _src(gpu, (d,), dt, 2) * 0.1
    gain = 1 + 0.1 * _src(gpu, (d,), dt, 3)
    go = _src(gpu, (2, 8, d), dt, 4)
    gl = _src(gpu, (2, 8), torch.float32, 5)
    torch.library.opcheck(ops.route_bwd, (buf, 3, q, gain, 1e-5, go, gl, True))
    torch.library.opcheck(ops.route_bwd, (buf, 4, q, None, 1e-5, go, None, True))
    srcs = [_src(gpu, (2, 8, d), dt, 10 + i) for i in range(3)]
    torch.library.opcheck(ops.route_list_bwd, (srcs, q, gain, 1e-5, go, gl))
    p, inter = _src(gpu, (2, 8, d), dt, 20), _src(gpu, (2, 8, d), dt, 21)
    torch.library.opcheck(ops.merge_bwd, (p, q, inter, gl, 1e-5, go))


def test_opcheck_block_step(gpu):
    # the arena op mutates its arena (declared in the schema)
    d, dt = 256, torch.bfloat16
    arena = _src(gpu, (4, 2, 8, d), dt, 1)
    delta = _src(gpu, (2, 8, d), dt, 2)
    q, gain = _src(gpu, (d,), dt, 3) * 0.1, 1 + 0.1 * _src(gpu, (d,), dt, 4)
    torch.library.opcheck(ops.block_step, (arena, 1, False, delta, q, gain, 1e-5, True))
    torch.library.opcheck(ops.block_step, (arena, 1, True, delta, q, gain, 1e-5, False))


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_compiled_training_loop_matches_eager_and_float64(gpu, backend):
    # llama.py:666-716's loop with route_static, compiled as one graph
    # (fullgraph=True: any graph break fails), forward and backward
    from oracle.torch_cpu_path import route_static_cpu

    torch._dynamo.reset()
    model = TinyModel(d=512, num_layers=4, boundaries=(0, 2), seed=21)
    ref_model = copy.deepcopy(model).double()
    g = torch.Generator().manual_seed(22)
    embed = torch.randn((2, 16, 512), generator=g)
    G = torch.randn((2, 16, 512), generator=g)
    out_ref = training_forward(ref_model, embed.double(),
                                lambda buf, q, norm, mask, n: route_static_cpu(buf, q * norm.weight, norm.eps, mask))
    (out_ref * G.double()).sum().backward()

    m_eager = model.to(gpu)
    m_comp = copy.deepcopy(m_eager)
    e, Gg = embed.to(gpu), G.to(gpu)
    (training_forward(m_eager, e, kotodama_amd.route_static) * Gg).sum().backward()

    step = torch.compile(lambda m, x: training_forward(m, x, kotodama_amd.route_static), backend=backend,
                         fullgraph=True)
    for it in range(2):  # the second call runs the cached graph
        m_comp.zero_grad(set_to_none=True)
        out = step(m_comp, e)
        loss = (out * Gg).sum()
        loss.backward()
        torch.cuda.synchronize()
        for (name, p), (_, pe), (_, pr) in zip(m_comp.named_parameters(), m_eager.named_parameters(),
                                               ref_model.named_parameters()):
            got = p.grad.double().cpu()
            want = pr.grad
            tol = 2e-4 * want.abs().max().item() + 1e-7
            assert (got - want).abs().max().item() <= tol, f"{backend} it={it} {name}: vs float64"
            tol_e = 2e-4 * pe.grad.abs().max().item() + 1e-7
            assert (p.grad - pe.grad).abs().max().item() <= tol_e, f"{backend} it={it} {name}: vs eager"
        torch.testing.assert_close(out.detach().double().cpu(), out_ref.detach(), rtol=2e-4, atol=2e-4)


def test_compiled_stack_free_training_matches_eager_and_float64(gpu):
    # the stack-free caller (forward_attn_res under autograd: route_list with a
    # list of block tensors per routing point, INTEGRATION's training drop-in)
    # compiled as one graph with the reference's default backend, forward and
    # backward, against the eager run and the reference's pad-and-stack loop in
    # float64; two calls (the second runs the cached graph)
    from oracle.torch_cpu_path import route_static_cpu

    torch._dynamo.reset()
    model = TinyModel(d=512, num_layers=4, boundaries=(0, 2), seed=25)
    ref_model = copy.deepcopy(model).double()
    g = torch.Generator().manual_seed(26)
    embed = torch.randn((2, 16, 512), generator=g)
    G = torch.randn((2, 16, 512), generator=g)
    out_ref = training_forward(ref_model, embed.double(),
                                lambda buf, q, norm, mask, n: route_static_cpu(buf, q * norm.weight, norm.eps, mask))
    loss_ref = (out_ref * G.double()).sum()
    loss_ref.backward()

    m_eager = model.to(gpu)
    m_comp = copy.deepcopy(m_eager)
    e, Gg = embed.to(gpu), G.to(gpu)
    (kotodama_amd.forward_attn_res(m_eager, e) * Gg).sum().backward()
    step = torch.compile(lambda m, x: kotodama_amd.forward_attn_res(m, x), backend="inductor", fullgraph=True)
    for it in range(2):
        m_comp.zero_grad(set_to_none=True)
        out = step(m_comp, e)
        loss = (out * Gg).sum()
        loss.backward()
        torch.cuda.synchronize()
        assert abs(loss.item() - loss_ref.item()) <= 1e-4 * abs(loss_ref.item()) + 1e-3, f"it={it}: loss"
        torch.testing.assert_close(out.detach().double().cpu(), out_ref.detach(), rtol=2e-4, atol=2e-4)
        checked = 0
        for (name, p), (_, pe), (_, pr) in zip(m_comp.named_parameters(), m_eager.named_parameters(),
                                               ref_model.named_parameters()):
            want = pr.grad
            tol = 2e-4 * want.abs().max().item() + 1e-7
            assert (p.grad.double().cpu() - want).abs().max().item() <= tol, f"it={it} {name}: vs float64"
            tol_e = 2e-4 * pe.grad.abs().max().item() + 1e-7
            assert (p.grad - pe.grad).abs().max().item() <= tol_e, f"it={it} {name}: vs eager"
            checked += 1
        assert checked == len(list(m_comp.parameters()))


def test_compiled_training_with_eager_points_defers(gpu, monkeypatch):
    # kotodama_amd.engine.defer_under_compile: the reference's torch.compile(model)
    # (no fullgraph) with the routing points run eagerly as graph breaks, so the
    # blocks' gradients are deferred (attnres_route_bwd_defer per point, segment
    # sums at the commits) while the sublayers are compiled by inductor; bf16 at
    # hidden 3072 over 8 layers, two calls, against the reference loop in float64
    # at the bar of the eager deferred loop test (2x the error of the reference's
    # own op sequence evaluated in bf16, plus 2^-9 of the largest magnitude)
    from kotodama_amd import engine
    from oracle.torch_cpu_path import route_static_cpu

    d = 3072
    model = TinyModel(d=d, num_layers=8, boundaries=(0, 2, 4, 6), seed=31, elementwise=True)
    model = model.to(torch.bfloat16).float()
    gen = torch.Generator().manual_seed(32)
    embed = (torch.randn((2, 32, d), generator=gen) * 2).to(torch.bfloat16).float()
    G = torch.randn((2, 32, d), generator=gen).to(torch.bfloat16).float()

    def einsum(buf, q, norm, mask, n):
        return route_static_cpu(buf, q * norm.weight, norm.eps, mask)

    def run(m, e, fwd):
        e = e.clone().requires_grad_(True)
        out = fwd(m, e)
        (out.float() * G.to(e.device)).sum().backward()
        grads = {n: p.grad.double().cpu() for n, p in m.named_parameters()}
        grads["embed"] = e.grad.double().cpu()
        return out.detach().double().cpu(), grads

    ref = run(copy.deepcopy(model).double(), embed.double(), lambda m, e: training_forward(m, e, einsum))
    tb = run(copy.deepcopy(model).to(gpu).to(torch.bfloat16), embed.to(gpu).to(torch.bfloat16),
             lambda m, e: training_forward(m, e, einsum))
    deferred = []
    real = ops._route_rows_backward_defer

    def counting(*a, **k):
        r = real(*a, **k)
        deferred.append(r is not None)
        return r

    monkeypatch.setattr(ops, "_route_rows_backward_defer", counting)
    torch._dynamo.reset()
    step = torch.compile(lambda m, x: kotodama_amd.forward_attn_res(m, x), backend="inductor", fullgraph=False)
    m_comp = copy.deepcopy(model).to(gpu).to(torch.bfloat16)
    engine.defer_under_compile(True)
    try:
        for it in range(2):
            deferred.clear()
            m_comp.zero_grad(set_to_none=True)
            ours = run(m_comp, embed.to(gpu).to(torch.bfloat16), step)
            torch.cuda.synchronize()
            # every point with a committed block deferred its blocks' gradients
            assert deferred and all(deferred), f"it={it}: the points did not defer ({deferred})"

            def worst(a, b):
                return (a - b).abs().max().item()

            assert worst(ours[0], ref[0]) <= 2 * worst(tb[0], ref[0]) + 2.0**-9 * ref[0].abs().max().item(), \
                f"it={it}: output"
            for name, want in ref[1].items():
                e_ours, e_tb = worst(ours[1][name], want), worst(tb[1][name], want)
                assert e_ours <= 2 * e_tb + 2.0**-9 * want.abs().max().item(), \
                    f"it={it} {name}: err {e_ours:.3e}, torch bf16 op sequence {e_tb:.3e}"
    finally:
        engine.defer_under_compile(False)
        torch._dynamo.reset()
