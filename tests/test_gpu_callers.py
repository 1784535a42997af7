"""Caller-level drop-ins on a reference-shaped model (GPU): the prefill forward
(llama.py:666-716) and the KV-cache forward with decode steps (llama.py:718-763)
against float64 restatements of the reference loops, and the serve fast path
(serve.py:113-164) point by point against the oracle's two-phase restatement."""

import copy

import numpy as np
import pytest
import torch

from kotodama_amd import forward_attn_res, forward_attn_res_cached
from oracle import attnres_oracle as O

from ._tiny_model import TinyModel, reference_forward_f64, training_forward

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


def np64(t):
    return t.detach().float().cpu().double().numpy()


def bf16_ulp(x):
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 2.0**-126))) - 7)


@pytest.mark.parametrize("boundaries", [(0, 2), (1, 3), (0, 1, 2, 3)])
def test_kv_cache_decode_threads_past_kv_like_the_reference(gpu, boundaries):
    # llama.py:718-763 as the serve engine drives it (serve.py:357-380): a prefill, then
    # T=1 decode steps with each call's KV list passed to the next, against the same
    # sequence of calls restated in float64 (routing through the oracle); the decoded
    # positions also equal one cached forward over the whole sequence
    from ._tiny_model import reference_cached_forward_f64

    d, B, T0, steps = 1024, 3, 8, 4
    model = TinyModel(d=d, num_layers=4, boundaries=boundaries, seed=41)
    ref_model = copy.deepcopy(model).double()
    tokens = torch.randn((B, T0 + steps, d), generator=torch.Generator().manual_seed(42))
    m = model.to(gpu)

    def close(got, want, what):
        torch.testing.assert_close(got.double().cpu(), want, rtol=2e-4, atol=2e-4, msg=lambda e: f"{what}: {e}")

    with torch.no_grad():
        h, kv = forward_attn_res_cached(m, tokens[:, :T0].to(gpu))
        h_ref, kv_ref = reference_cached_forward_f64(ref_model, tokens[:, :T0])
        close(h, h_ref, "prefill")
        decoded = []
        for t in range(steps):
            x = tokens[:, T0 + t: T0 + t + 1]
            h, kv = forward_attn_res_cached(m, x.to(gpu), past_kv=kv)
            h_ref, kv_ref = reference_cached_forward_f64(ref_model, x, past_kv=kv_ref)
            close(h, h_ref, f"decode step {t}")
            assert len(kv) == 4 and all(k.shape == (B, T0 + t + 1, d) for k, _ in kv)
            for i in range(4):
                close(kv[i][0], kv_ref[i][0], f"decode step {t} layer {i} keys")
            decoded.append(h)
        full, _ = forward_attn_res_cached(m, tokens.to(gpu))
    torch.testing.assert_close(torch.cat(decoded, dim=1), full[:, T0:], rtol=1e-4, atol=1e-4)


# (num_layers, boundaries): uniform blocks; the DD-v1 proxy's non-uniform blocks
# (configs/openwebtext-ddv1.yaml:10); a set that does not start at layer 0, whose
# leading sublayers serve.py:121-126 never runs
SERVE_CASES = [(4, (0, 2)), (28, (0, 3, 7, 12, 21, 25)), (6, (1, 3, 4))]


@pytest.mark.parametrize("L,boundaries", SERVE_CASES, ids=["uniform", "dd-v1", "no-layer-0"])
def test_serve_fast_path_matches_two_phase_oracle(gpu, L, boundaries):
    # fast_forward_attn_res (serve.py:113-164) with sublayers that record their routed
    # input and return given outputs, point by point against the oracle's restatement of
    # the same loop in bf16: phase-1 output rounded to bf16 and lse kept in fp32, merge
    # output rounded to bf16, running blocks added in bf16.  Bar per element:
    # max(2e-2, 1 bf16 ulp) for phase-1 outputs; for merged points the same plus
    # (1 - pi) ulp(inter), the phase-1 input's own one-ulp rounding difference carried
    # through the merge, which weights the phase-1 row by 1 - pi; and >= 98% of the
    # elements equal to the correctly rounded oracle.
    from kotodama_amd.serving import FastAttnResContext, fast_forward_attn_res

    d, B, T = 512, 2, 32
    N = B * T
    g = torch.Generator(device=gpu).manual_seed(L * 100 + len(boundaries))
    embed = (torch.randn((B, T, d), generator=g, device=gpu) * 2).to(torch.bfloat16)
    deltas = [(torch.randn((B, T, d), generator=g, device=gpu) * (0.25 + 0.05 * (j % 7))).to(torch.bfloat16)
              for j in range(2 * L)]
    q = (torch.randn((2 * L + 1, d), generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    gain = (1 + 0.1 * torch.randn((2 * L + 1, d), generator=g, device=gpu)).to(torch.bfloat16)
    pq = q * gain  # folded in the parameter dtype, as serve.py:85-92
    seen = {}

    def sublayer(j):
        def run(x):
            seen[j] = x.clone()
            return deltas[j]
        return run

    ctx = FastAttnResContext.from_parts(pq, [2 * b for b in sorted(boundaries)], [sublayer(j) for j in range(2 * L)],
                                        1e-5)
    with torch.no_grad():
        final = fast_forward_attn_res(ctx, embed)
    torch.cuda.synchronize()
    ref = O.two_phase_forward(np64(embed).reshape(N, d), [np64(x).reshape(N, d) for x in deltas],
                              [np64(pq[j]) for j in range(2 * L + 1)], 1e-5, L, set(boundaries), dtype="bf16")
    assert sorted(seen) == sorted(ref["h"])
    worst, exact, total = 0.0, 0, 0
    points = [(j, np64(seen[j]).reshape(N, d), ref["h"][j]) for j in sorted(seen)]
    points.append((2 * L, np64(final).reshape(N, d), ref["final"]))
    for j, got, want in points:
        tol = np.maximum(2e-2, bf16_ulp(want))
        if j in ref["pi"]:
            tol = tol + (1 - ref["pi"][j])[:, None] * bf16_ulp(ref["inter"][j])
        err = np.abs(got - want)
        assert (err <= tol).all(), f"point {j}: worst err {err.max():.3e}"
        big = np.abs(want) >= 1.0  # where the ulp term, not the 2e-2 floor, sets the bar
        if big.any():
            worst = max(worst, float((err[big] / bf16_ulp(want[big])).max()))
        exact += int((got == want).sum())
        total += got.size
    print(f"serve L={L} boundaries={boundaries}: max err {worst:.2f} bf16 ulp where |ref| >= 1, "
          f"{exact / total:.4%} of {total} elements equal to the rounded oracle")
    assert exact >= 0.98 * total


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

    out_ref = training_forward(ref_model, embed.double(),
                                lambda buf, q, norm, mask, n: route_static_cpu(buf, q * norm.weight, norm.eps, mask))
    loss_ref = (out_ref * G.double()).sum()
    loss_ref.backward()

    m = model.to(gpu)
    out = training_forward(m, embed.to(gpu), route_static)
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
    out_ref = training_forward(ref_model, embed.double(),
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


@pytest.mark.parametrize("path", ["stack_free", "stacked"])
def test_bf16_training_loop_sixteen_layers(gpu, path):
    # a bf16 model (the reference trains in bf16, train.py:237) of 16 layers in 4
    # blocks (S = 1..5), sublayers without matrix products: loss, output and every
    # parameter gradient (routing queries and gains, sublayer parameters, the
    # embedding) against the reference loop in float64.  Bar per tensor: the
    # worst error within 2x that of the reference's own op sequence
    # (llama.py:640-644, the einsum branch) evaluated in bf16 on the same bf16
    # model, plus 2^-9 of the largest reference magnitude (sublayer roundings
    # alone move bf16 values by that much).  path: forward_attn_res under
    # autograd (list routing) or the pad-and-stack loop with route_static.
    from kotodama_amd import route_static
    from oracle.torch_cpu_path import route_static_cpu

    L, bounds, d = 16, (0, 4, 8, 12), 1024
    model = TinyModel(d=d, num_layers=L, boundaries=bounds, seed=51, elementwise=True)
    model = model.to(torch.bfloat16).float()  # bf16-exact parameters shared by every run
    assert model._attn_res_max_sources == 5
    gen = torch.Generator().manual_seed(52)
    embed = (torch.randn((2, 32, d), generator=gen) * 2).to(torch.bfloat16).float()
    G = torch.randn((2, 32, d), generator=gen).to(torch.bfloat16).float()

    def einsum(buf, q, norm, mask, n):
        return route_static_cpu(buf, q * norm.weight, norm.eps, mask)

    def run(m, e, fwd):
        e = e.clone().requires_grad_(True)
        out = fwd(m, e)
        loss = (out.float() * G.to(e.device)).sum()
        loss.backward()
        grads = {n: p.grad.double().cpu() for n, p in m.named_parameters()}
        grads["embed"] = e.grad.double().cpu()
        return loss.item(), out.detach().double().cpu(), grads

    ref = run(copy.deepcopy(model).double(), embed.double(), lambda m, e: training_forward(m, e, einsum))
    tb = run(copy.deepcopy(model).to(gpu).to(torch.bfloat16), embed.to(gpu).to(torch.bfloat16),
             lambda m, e: training_forward(m, e, einsum))
    if path == "stack_free":
        fwd = forward_attn_res
    else:
        def fwd(m, e):
            return training_forward(m, e, route_static)
    ours = run(copy.deepcopy(model).to(gpu).to(torch.bfloat16), embed.to(gpu).to(torch.bfloat16), fwd)
    torch.cuda.synchronize()

    def worst(a, b):
        return (a - b).abs().max().item()

    loss_bar = 2 * abs(tb[0] - ref[0]) + 2.0**-9 * abs(ref[0])
    print(f"bf16 L=16 {path}: loss err {abs(ours[0] - ref[0]):.3e} (torch bf16 {abs(tb[0] - ref[0]):.3e})", flush=True)
    assert abs(ours[0] - ref[0]) <= loss_bar
    floor = 2.0**-9 * ref[1].abs().max().item()
    assert worst(ours[1], ref[1]) <= 2 * worst(tb[1], ref[1]) + floor, "output"
    ratios = []
    for name, want in ref[2].items():
        e_ours, e_tb = worst(ours[2][name], want), worst(tb[2][name], want)
        bar = 2 * e_tb + 2.0**-9 * want.abs().max().item()
        ratios.append(e_ours / max(e_tb, 1e-30))
        assert e_ours <= bar, f"{name}: err {e_ours:.3e}, torch bf16 op sequence {e_tb:.3e}"
    print(f"bf16 L=16 {path}: {len(ratios)} gradients, error / torch-bf16 error: median "
          f"{float(np.median(ratios)):.2f}, max {max(ratios):.2f}", flush=True)
