"""The whole-training-step model (kotodama_amd.lmstep) on the GPU.

Its AttnRes residual stream runs through this package's kernels
(engine.forward_attn_res); here it is checked on the same model and batch against
the reference's caller loop with the reference's routing ops (llama.py:630-644,
666-716, restated in torch below) run in float64: the loss within five times
the error of that loop run in fp32, and every parameter's gradient within five
times that loop's fp32 error plus 2e-4 of the gradient's largest element.  Per
routing call both fp32 paths land within ~1e-6 (relative) of float64; through
a few layers of attention and SwiGLU either path's rounding is amplified
differently, up to ~1e-4 of the gradient's size where a gradient sums
cancelling terms.  A misrouted source or gradient is off by about the
gradient's own size.  A bf16 step of each residual stream, with the optimizer,
gives finite losses and gradients (attention on SDPA's fused kernels only).
"""

import copy

import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from kotodama_amd import lmstep, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _route_reference(buf, query, norm, mask, num_active):
    qw = query * norm.weight
    rsqrt = torch.rsqrt(buf.pow(2).mean(-1) + norm.eps)
    logits = (buf * qw).sum(-1) * rsqrt
    logits = logits.masked_fill(~mask.view(-1, 1, 1), float("-inf"))
    return (F.softmax(logits, dim=0).unsqueeze(-1) * buf).sum(0)


def _reference_loop(model, embed):
    return workloads.stacked_training_forward(model, embed, _route_reference)


def _grads(model):
    return {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}


@pytest.mark.parametrize("hidden,layers,blocks", [(512, 4, 2), (1024, 5, 3)], ids=["d512-L4", "d1024-L5"])
def test_attnres_step_matches_reference_loop_fp32(hidden, layers, blocks):
    lmstep.compile_sublayers(False)
    c = lmstep.LMConfig("t", hidden, layers, 4, 2, 128, 384, vocab_size=1000, attn_res_n_blocks=blocks,
                        batch=2, seq=64)
    model = lmstep.LanguageModel(c, DEV, dtype=torch.float32, seed=5)
    g = torch.Generator(device=DEV).manual_seed(6)
    with torch.no_grad():  # queries and gains away from their zero / one start, so routing is not uniform
        for name, p in model.named_parameters():
            if "res_query" in name:
                p.copy_(torch.randn(p.shape, generator=g, device=DEV) * 0.2)
            elif "res_norm" in name:
                p.add_(torch.randn(p.shape, generator=g, device=DEV) * 0.1)
    ids, labels = lmstep.make_batch(c, DEV, seed=7)
    print(f"lmstep fp32 D={hidden} L={layers} blocks={blocks}", flush=True)

    model.zero_grad(set_to_none=True)
    loss = model(ids, labels, "attnres")
    loss.backward()
    got = _grads(model)
    model.zero_grad(set_to_none=True)
    ref_loss = model(ids, labels, _reference_loop)
    ref_loss.backward()
    ref = _grads(model)
    exact = copy.deepcopy(model).double()  # the reference loop in float64: the error scale of fp32
    exact.zero_grad(set_to_none=True)
    exact_loss = exact(ids, labels, _reference_loop)
    exact_loss.backward()
    want = _grads(exact)

    # bar: five times the fp32 reference loop's own error against float64, plus 1e-6 of the gradient's size
    assert abs(loss.item() - exact_loss.item()) <= 5 * abs(ref_loss.item() - exact_loss.item()) + 1e-6
    assert got.keys() == want.keys() == ref.keys() and len(want) == len(list(model.parameters()))
    worst = []
    for name, w in want.items():
        scale = w.abs().max().item()
        err = (got[name].double() - w).abs().max().item()
        ref_err = (ref[name].double() - w).abs().max().item()
        bar = 5 * ref_err + 2e-4 * scale
        worst.append((err / bar if bar > 0 else (0.0 if err == 0 else float("inf")), name, err, ref_err, scale))
    worst.sort(reverse=True)
    for row in worst[:8]:
        print("ratio %.3f %s err %.3e ref_err %.3e scale %.3e" % row, flush=True)
    assert worst[0][0] <= 1.0, worst[0]


def test_bf16_steps_of_each_residual_stream():
    lmstep.compile_sublayers(False)
    c = lmstep.LMConfig("t", 512, 4, 4, 2, 128, 384, vocab_size=1000, attn_res_n_blocks=2, batch=2, seq=128)
    model = lmstep.LanguageModel(c, DEV, seed=8)
    opt = lmstep.optimizer(model)
    ids, labels = lmstep.make_batch(c, DEV, seed=9)
    for residual in ("standard", "attnres", _reference_loop):
        print(f"lmstep bf16 residual={getattr(residual, '__name__', residual)}", flush=True)
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):  # fused kernels only
                loss = model(ids, labels, residual)
                loss.backward()
            assert torch.isfinite(loss).item()
            assert all(torch.isfinite(p.grad).all().item() for p in model.parameters() if p.grad is not None)
            opt.step()
