"""The accumulating training path's autograd plumbing, on the CPU.

``forward_attn_res`` under autograd sums each committed block's gradient over
the routing calls that read it inside the backward kernel
(``ops.route_point`` + ``ops.GradSlot`` + the commit node).  Here the
kernel launches (``ops._route_rows_forward`` / ``_route_rows_step`` / ``_route_rows_backward``)
are replaced by float64 torch restatements of the reference op sequence
(llama.py:640-644) that honour the same contract — ``grads[s]`` receives
dL/dsource_s plus ``adds[s]`` when that is given — so the test checks what
the host side decides: which calls write a block's gradient fresh and which
add to it, that the commit node returns the sum after every reader has run,
and that a second backward pass (retained graph, or a pass that did not reach
the commit nodes) starts over.  The losses and every gradient are compared
with plain autograd through the reference's pad-and-stack loop.
"""

import copy

import pytest
import torch

from kotodama_amd import engine, ops
from oracle.torch_cpu_path import route_static_cpu

from ._tiny_model import TinyModel, training_forward


def _ref_route(buf, q, norm, mask, n):
    return route_static_cpu(buf, q * norm.weight, norm.eps, mask)


@pytest.fixture
def cpu_kernels(monkeypatch):
    calls = []

    def fwd(sources, query, gain, eps, out_dtype):
        buf = torch.stack([s.detach() for s in sources]).double()
        qw = query.detach().double() * (gain.detach().double() if gain is not None else 1.0)
        mask = torch.ones(len(sources), dtype=torch.bool)
        return route_static_cpu(buf, qw, eps, mask).to(out_dtype)

    def bwd(sources, grads, adds, query, gain, eps, grad_out):
        xs = [s.detach().double().requires_grad_(True) for s in sources]
        q = query.detach().double().requires_grad_(True)
        g = gain.detach().double().requires_grad_(True) if gain is not None else None
        mask = torch.ones(len(sources), dtype=torch.bool)
        with torch.enable_grad():  # autograd runs backward functions with grad mode off
            qw = q * g if g is not None else q
            route_static_cpu(torch.stack(xs), qw, eps, mask).backward(grad_out.double())
        vals = [x.grad + (a.double() if a is not None else 0.0) for x, a in zip(xs, adds)]
        for gr, v in zip(grads, vals):
            gr.copy_(v)
        calls.append([("add" if a is not None else "write") for a in adds])
        return q.grad.to(query.dtype), (g.grad.to(gain.dtype) if g is not None else None)

    def step(committed, partial, delta, query, gain, eps, out_dtype):
        new_partial = partial.detach() + delta.detach()
        return fwd(list(committed) + [new_partial], query, gain, eps, out_dtype), new_partial

    monkeypatch.setattr(ops, "_route_rows_forward", fwd)
    monkeypatch.setattr(ops, "_route_rows_step", step)
    monkeypatch.setattr(ops, "_route_rows_backward", bwd)
    return calls


def _grads(model, embed):
    out = {n: p.grad.clone() for n, p in model.named_parameters()}
    out["embed"] = embed.grad.clone()
    return out


@pytest.mark.parametrize("boundaries", [(0, 2), (1, 3), (0, 1, 2, 3)])
def test_accumulated_gradients_equal_plain_autograd(cpu_kernels, boundaries):
    model = TinyModel(d=64, num_layers=4, boundaries=boundaries, seed=3).double()
    ref = copy.deepcopy(model)
    g = torch.Generator().manual_seed(4)
    embed = torch.randn((2, 5, 64), generator=g, dtype=torch.float64)
    G = torch.randn((2, 5, 64), generator=g, dtype=torch.float64)
    e1 = embed.clone().requires_grad_(True)
    loss = (engine.forward_attn_res(model, e1) * G).sum()
    loss.backward()
    e2 = embed.clone().requires_grad_(True)
    loss_ref = (training_forward(ref, e2, _ref_route) * G).sum()
    loss_ref.backward()
    torch.testing.assert_close(loss, loss_ref, rtol=1e-12, atol=1e-12)
    got, want = _grads(model, e1), _grads(ref, e2)
    for k in want:
        torch.testing.assert_close(got[k], want[k], rtol=1e-10, atol=1e-12, msg=lambda m, k=k: f"{k}: {m}")
    # every committed block's gradient is written once (by the last routing call
    # that reads it, whose backward runs first) and added to by every earlier reader
    n_blocks = len(boundaries)
    writes = [0] * n_blocks
    adds = [0] * n_blocks
    for c in cpu_kernels:
        for b, kind in enumerate(c[:-1]):
            (writes if kind == "write" else adds)[b] += 1
    assert writes == [1] * n_blocks
    uses = [sum(1 for c in cpu_kernels if len(c) - 1 > b) for b in range(n_blocks)]
    assert adds == [u - 1 for u in uses]
    # the routed partial's gradient: the final point's (first backward call) is
    # its routing gradient alone; every other point adds the gradient of the
    # partial the next point routes (or, at a commit, the block's summed gradient)
    assert len(cpu_kernels) == 2 * len(model.layers) + 1
    assert cpu_kernels[0][-1] == "write" and all(c[-1] == "add" for c in cpu_kernels[1:])


def test_retained_graph_and_partial_backward_start_over(cpu_kernels):
    model = TinyModel(d=32, num_layers=4, boundaries=(0, 2), seed=5).double()
    ref = copy.deepcopy(model)
    g = torch.Generator().manual_seed(6)
    embed = torch.randn((1, 4, 32), generator=g, dtype=torch.float64)
    G = torch.randn((1, 4, 32), generator=g, dtype=torch.float64)
    e1 = embed.clone().requires_grad_(True)
    out = engine.forward_attn_res(model, e1)
    loss = (out * G).sum()
    # a pass that stops short of the commit nodes (only one query's gradient)
    # leaves a partial sum in the blocks' slots; the next passes must not add to it
    (gq,) = torch.autograd.grad(loss, [model.layers[3].mlp_res_query], retain_graph=True)
    loss.backward(retain_graph=True)
    loss.backward()
    e2 = embed.clone().requires_grad_(True)
    loss_ref = (training_forward(ref, e2, _ref_route) * G).sum()
    loss_ref.backward(retain_graph=True)
    loss_ref.backward()
    torch.testing.assert_close(gq, ref.layers[3].mlp_res_query.grad / 2, rtol=1e-10, atol=1e-12)
    got, want = _grads(model, e1), _grads(ref, e2)
    for k in want:
        torch.testing.assert_close(got[k], want[k], rtol=1e-10, atol=1e-12, msg=lambda m, k=k: f"{k}: {m}")


def test_blocks_without_grad_and_plain_calls_mix(cpu_kernels, monkeypatch):
    # an embedding that does not require grad (its block's gradient is not
    # needed) and routing points whose output dtype differs from the blocks'
    # (those take route_list and return the blocks' gradients through autograd,
    # which the commit node adds to the slot's sum)
    model = TinyModel(d=32, num_layers=4, boundaries=(0, 1, 3), seed=7).double()
    ref = copy.deepcopy(model)
    g = torch.Generator().manual_seed(8)
    embed = torch.randn((1, 3, 32), generator=g, dtype=torch.float64)
    G = torch.randn((1, 3, 32), generator=g, dtype=torch.float64)

    def fake_list_call(sources, query, gain, eps, out_dtype, *a, **k):
        mask = torch.ones(len(sources), dtype=torch.bool)
        qw = query * gain if gain is not None else query
        return (route_static_cpu(torch.stack(list(sources)), qw, eps, mask).unsqueeze(0),)

    monkeypatch.setattr(ops, "route_list_call", fake_list_call)
    real_ok = ops.accumulating_path_ok
    state = {"n": 0}

    def every_other(*t):
        state["n"] += 1
        return real_ok(*t) and (len(t) == 1 or state["n"] % 2 == 0)

    monkeypatch.setattr(ops, "accumulating_path_ok", every_other)
    loss = (engine.forward_attn_res(model, embed) * G).sum()
    loss.backward()
    loss_ref = (training_forward(ref, embed, _ref_route) * G).sum()
    loss_ref.backward()
    torch.testing.assert_close(loss, loss_ref, rtol=1e-12, atol=1e-12)
    for (n, p), (_, pr) in zip(model.named_parameters(), ref.named_parameters()):
        torch.testing.assert_close(p.grad, pr.grad, rtol=1e-10, atol=1e-12, msg=lambda m, n=n: f"{n}: {m}")


@pytest.mark.parametrize("backend", ["eager", "aot_eager"])
def test_points_run_eagerly_under_compile(cpu_kernels, backend):
    # engine.defer_under_compile: under torch.compile (no fullgraph) each routing
    # point, commit and sublayer-output step is a graph break run eagerly, so the
    # accumulating path (its slots and commit nodes) is the one that runs, with
    # the sublayers between the points compiled; gradients as plain autograd,
    # the same write / add pattern as in eager mode, on two compiled calls
    model = TinyModel(d=32, num_layers=4, boundaries=(0, 2), seed=7).double()
    ref = copy.deepcopy(model)
    g = torch.Generator().manual_seed(8)
    embed = torch.randn((2, 3, 32), generator=g, dtype=torch.float64)
    G = torch.randn((2, 3, 32), generator=g, dtype=torch.float64)
    torch._dynamo.reset()
    fwd = torch.compile(lambda m, e: engine.forward_attn_res(m, e), backend=backend, fullgraph=False)
    engine.defer_under_compile(True)
    try:
        for rep in range(2):
            cpu_kernels.clear()
            model.zero_grad(set_to_none=True)
            e1 = embed.clone().requires_grad_(True)
            loss = (fwd(model, e1) * G).sum()
            loss.backward()
            ref.zero_grad(set_to_none=True)
            e2 = embed.clone().requires_grad_(True)
            loss_ref = (training_forward(ref, e2, _ref_route) * G).sum()
            loss_ref.backward()
            torch.testing.assert_close(loss, loss_ref, rtol=1e-12, atol=1e-12)
            got, want = _grads(model, e1), _grads(ref, e2)
            for k in want:
                torch.testing.assert_close(got[k], want[k], rtol=1e-10, atol=1e-12,
                                           msg=lambda m, k=k, rep=rep: f"call {rep} {k}: {m}")
            assert len(cpu_kernels) == 2 * len(model.layers) + 1, f"call {rep}: the accumulating path did not run"
            assert cpu_kernels[0][-1] == "write" and all(c[-1] == "add" for c in cpu_kernels[1:])
    finally:
        engine.defer_under_compile(False)
        torch._dynamo.reset()
