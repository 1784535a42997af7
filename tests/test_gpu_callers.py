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
