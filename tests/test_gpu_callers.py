"""Caller-level drop-ins on a reference-shaped model (GPU): the prefill forward
(llama.py:666-716), the KV-cache forward (llama.py:718-763) and the serve fast
path (serve.py:113-164), against a float64 restatement of the reference loop."""

import copy

import pytest
import torch

from kotodama_amd import forward_attn_res, forward_attn_res_cached
from kotodama_amd.serving import FastAttnResContext, fast_forward_attn_res

from ._tiny_model import TinyModel, reference_forward_f64

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("boundaries", [(0, 2), (0, 1, 3), (1, 3)])
def test_prefill_forward_matches_reference_loop(gpu, boundaries):
    model = TinyModel(d=512, num_layers=4, boundaries=boundaries, seed=1)
    embed = torch.randn((2, 48, 512), generator=torch.Generator().manual_seed(2))
    ref = reference_forward_f64(copy.deepcopy(model), embed)
    m = model.to(gpu)
    with torch.no_grad():
        out = forward_attn_res(m, embed.to(gpu))
    torch.testing.assert_close(out.double().cpu(), ref, rtol=2e-4, atol=2e-4)


def test_kv_cache_forward_returns_same_hidden_and_kv(gpu):
    model = TinyModel(d=1024, num_layers=3, boundaries=(0, 1), seed=3).to(gpu)
    embed = torch.randn((3, 1, 1024), device=gpu)
    with torch.no_grad():
        h1 = forward_attn_res(model, embed)
        h2, kv = forward_attn_res_cached(model, embed)
    assert torch.equal(h1, h2) and len(kv) == 3


def test_serve_fast_path_matches_stack_free_forward_bf16(gpu):
    model = TinyModel(d=512, num_layers=4, boundaries=(0, 2), seed=5).to(gpu).to(torch.bfloat16)
    embed = torch.randn((2, 64, 512), device=gpu).to(torch.bfloat16)
    with torch.no_grad():
        fast = fast_forward_attn_res(FastAttnResContext(model), embed)
        slow = forward_attn_res(model, embed)
    assert fast.dtype == torch.bfloat16
    # the fast path rounds each phase-1 result to bf16 before merging (as the reference's)
    rel = (fast.float() - slow.float()).norm() / slow.float().norm()
    assert rel < 1e-2, f"relative difference {rel:.3e}"


def _training_forward(model, embed, route_fn):
    """The training loop of llama.py:666-716 (pad + stack before every routing call,
    out-of-place partial updates), with the routing function swapped in."""
    from kotodama_amd import AttnResSchedule

    sched = AttnResSchedule.build(model.config.num_layers, boundaries=sorted(model._attn_res_boundary_set))
    masks = sched.masks(embed.device)
    counts = sched.active_counts
    committed, partial = [], embed
    zero = torch.zeros_like(embed)

    def pad_and_stack():
        sources = committed + [partial]
        sources += [zero] * (sched.max_sources - len(sources))
        return torch.stack(sources, dim=0)

    for i, layer in enumerate(model.layers):
        h = route_fn(pad_and_stack(), layer.attn_res_query, layer.attn_res_norm, masks[2 * i], counts[2 * i])
        if i in model._attn_res_boundary_set:
            committed.append(partial.clone())
            partial = zero.clone()
        partial = partial + layer.attn(layer.attn_norm(h), None, None)
        h = route_fn(pad_and_stack(), layer.mlp_res_query, layer.mlp_res_norm, masks[2 * i + 1], counts[2 * i + 1])
        partial = partial + layer.ffn(layer.ffn_norm(h))
    x = route_fn(pad_and_stack(), model.final_res_query, model.final_res_norm, masks[-1], counts[-1])
    return model.norm(x)


def test_training_step_gradients_match_float64_reference(gpu):
    # the reference's training forward with _route_static swapped for the HIP op:
    # loss and every parameter gradient (routing queries and gains, sublayer
    # weights upstream of the routing calls) against the same loop in float64
    # on the CPU with the einsum branch's op sequence
    from kotodama_amd import route_static
    from oracle.torch_cpu_path import route_static_cpu

    model = TinyModel(d=512, num_layers=4, boundaries=(0, 2), seed=21)
    ref_model = copy.deepcopy(model).double()
    g = torch.Generator().manual_seed(22)
    embed = torch.randn((2, 16, 512), generator=g)
    G = torch.randn((2, 16, 512), generator=g)

    out_ref = _training_forward(ref_model, embed.double(),
                                lambda buf, q, norm, mask, n: route_static_cpu(buf, q * norm.weight, norm.eps, mask))
    loss_ref = (out_ref * G.double()).sum()
    loss_ref.backward()

    m = model.to(gpu)
    out = _training_forward(m, embed.to(gpu), route_static)
    loss = (out * G.to(gpu)).sum()
    loss.backward()
    torch.cuda.synchronize()
    assert abs(loss.item() - loss_ref.item()) <= 1e-4 * abs(loss_ref.item()) + 1e-3
    checked = 0
    for (name, p), (_, pr) in zip(m.named_parameters(), ref_model.named_parameters()):
        if pr.grad is None:
            continue
        got, want = p.grad.double().cpu(), pr.grad
        tol = 2e-4 * want.abs().max().item() + 1e-7
        assert (got - want).abs().max().item() <= tol, f"{name}: max err {(got - want).abs().max().item():.3e}"
        checked += 1
    assert checked == len(list(m.parameters()))  # every parameter is upstream of the loss


def test_stack_free_forward_trains_like_the_reference_loop(gpu):
    # forward_attn_res under autograd (list-based routing, no stacks) against the
    # reference's pad-and-stack loop in float64: loss and every parameter gradient
    from oracle.torch_cpu_path import route_static_cpu

    model = TinyModel(d=512, num_layers=4, boundaries=(1, 3), seed=23)
    ref_model = copy.deepcopy(model).double()
    g = torch.Generator().manual_seed(24)
    embed = torch.randn((2, 16, 512), generator=g)
    G = torch.randn((2, 16, 512), generator=g)
    out_ref = _training_forward(ref_model, embed.double(),
                                lambda buf, q, norm, mask, n: route_static_cpu(buf, q * norm.weight, norm.eps, mask))
    (out_ref * G.double()).sum().backward()
    m = model.to(gpu)
    out = forward_attn_res(m, embed.to(gpu))
    (out * G.to(gpu)).sum().backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(out.detach().double().cpu(), out_ref.detach(), rtol=2e-4, atol=2e-4)
    for (name, p), (_, pr) in zip(m.named_parameters(), ref_model.named_parameters()):
        got, want = p.grad.double().cpu(), pr.grad
        tol = 2e-4 * want.abs().max().item() + 1e-7
        assert (got - want).abs().max().item() <= tol, f"{name}: max err {(got - want).abs().max().item():.3e}"
    # without autograd the same call takes the fused arena path and agrees
    with torch.no_grad():
        out2 = forward_attn_res(m, embed.to(gpu))
    torch.testing.assert_close(out2, out.detach(), rtol=1e-5, atol=1e-5)


def test_eager_calls_skip_the_dispatcher_only_when_nothing_is_recorded(gpu, monkeypatch):
    # the drop-ins launch the op's implementation directly in eager no-grad
    # use (same values as the op), and go through the op when autograd or a
    # dispatch mode must see the call
    from kotodama_amd import ops, routing

    d = 1024
    g = torch.Generator(device=gpu).manual_seed(31)
    buf = torch.randn((4, 2, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    query = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    norm = torch.nn.Module()
    norm.weight = torch.nn.Parameter((1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16))
    norm.eps = 1e-5
    mask = torch.ones(4, dtype=torch.bool, device=gpu)
    via_op = ops.route(buf, 3, query, norm.weight, 1e-5, torch.bfloat16, False, False)[0][0]
    partial = torch.randn((2, 16, d), generator=g, device=gpu).to(torch.bfloat16)
    lse = torch.randn((2, 16), generator=g, device=gpu)
    merged_op = ops.merge(partial, query, buf[0], lse, 1e-5)[0]

    calls = []
    real_route, real_merge = ops.route, ops.merge
    monkeypatch.setattr(ops, "route", lambda *a: calls.append("route") or real_route(*a))
    monkeypatch.setattr(ops, "merge", lambda *a: calls.append("merge") or real_merge(*a))
    with torch.no_grad():
        h = routing.route_static(buf, query, norm, mask, 3)
        m = ops.merge_call(partial, query, buf[0], lse, 1e-5)
    assert calls == [] and torch.equal(h, via_op) and torch.equal(m, merged_op)
    # a parameter that requires grad under autograd: the op (and its backward) runs
    h2 = routing.route_static(buf, query, norm, mask, 3)
    assert calls == ["route"] and h2.requires_grad and torch.equal(h2.detach(), via_op)
    calls.clear()

    class PassThrough(torch.utils._python_dispatch.TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with torch.no_grad(), PassThrough():
        h3 = routing.route_static(buf, query, norm, mask, 3)
    assert calls == ["route"] and torch.equal(h3, via_op)
