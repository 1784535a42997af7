"""Host-side checks of the whole-training-step model (kotodama_amd.lmstep), on the CPU.

The routing schedule the model carries must be the reference's (llama.py:545-571:
boundaries from ``attn_res_n_blocks`` or an explicit list, per-point masks and
source counts), the presets must be configs/model.yaml's shapes, and the standard
residual stream and the reference caller loop must run (forward, loss, backward)
on a tiny model, and bench.py's compiled comparator loop must equal the reference
loop.  The AttnRes stream through this package's kernels needs the GPU
(tests/test_gpu_lmstep.py).
"""

import math

import pytest
import torch
import torch.nn.functional as F

from kotodama_amd import lmstep, workloads
from kotodama_amd.schedule import AttnResSchedule


def _route_reference(buf, query, norm, mask, num_active):
    qw = query * norm.weight
    rsqrt = torch.rsqrt(buf.pow(2).mean(-1) + norm.eps)
    logits = ((buf * qw).sum(-1) * rsqrt).masked_fill(~mask.view(-1, 1, 1), float("-inf"))
    return (F.softmax(logits, dim=0).unsqueeze(-1) * buf).sum(0)


def test_presets_are_the_reference_models():
    # configs/model.yaml: hidden, layers, heads, KV heads, head dim, SwiGLU width; 49152 vocabulary
    want = {"proxy": (512, 28, 4, 2, 128, 1408), "1b": (1024, 28, 8, 4, 128, 2816),
            "3b": (3072, 28, 24, 8, 128, 8192), "8b": (4096, 32, 32, 8, 128, 14336)}
    for name, shape in want.items():
        c = lmstep.PRESETS[name]
        assert (c.hidden_size, c.num_layers, c.num_attention_heads, c.num_kv_heads, c.head_dim,
                c.intermediate_size) == shape
        assert c.vocab_size == 49152 and c.norm_eps == 1e-5 and c.rope_theta == 500000.0
    # the proxy's parameter count is the brief's "108M params" (tied embedding, no biases)
    c = lmstep.PRESETS["proxy"]
    per_layer = (c.hidden_size * c.head_dim * (2 * c.num_attention_heads + 2 * c.num_kv_heads)
                 + 3 * c.hidden_size * c.intermediate_size)
    assert round((c.num_layers * per_layer + c.vocab_size * c.hidden_size) / 1e6) == 108


@pytest.mark.parametrize("name", ["proxy", "1b", "3b", "8b"])
def test_model_schedule_matches_the_reference_rule(name):
    c = lmstep.PRESETS[name]
    small = lmstep.LMConfig("s", 32, c.num_layers, 2, 1, 16, 48, vocab_size=64,
                            attn_res_n_blocks=c.attn_res_n_blocks, attn_res_boundaries=c.attn_res_boundaries,
                            batch=1, seq=8)
    model = lmstep.LanguageModel(small, "cpu", torch.float32)
    if c.attn_res_boundaries is None:
        step = math.ceil(c.num_layers / c.attn_res_n_blocks)
        sched = AttnResSchedule.build(c.num_layers, n_blocks=c.attn_res_n_blocks)
        assert model._attn_res_boundary_set == frozenset(range(0, c.num_layers, step))
    else:
        sched = AttnResSchedule.build(c.num_layers, boundaries=c.attn_res_boundaries)
    assert model._attn_res_boundary_set == sched.boundary_set
    assert model._attn_res_max_sources == sched.max_sources
    assert tuple(model._attn_res_active_counts) == sched.active_counts
    masks = model._attn_res_masks
    for j, n in enumerate(sched.active_counts):
        assert masks[j].tolist() == [k < n for k in range(sched.max_sources)]
    assert {"proxy": 8, "1b": 7, "3b": 8, "8b": 9}[name] == sched.max_sources


def test_standard_and_reference_loop_steps_run_on_cpu():
    lmstep.compile_sublayers(False)
    c = lmstep.LMConfig("t", 64, 3, 4, 2, 16, 96, vocab_size=128, attn_res_n_blocks=2, batch=2, seq=16)
    model = lmstep.LanguageModel(c, "cpu", torch.float32, seed=1)
    ids, labels = lmstep.make_batch(c, "cpu")
    opt = lmstep.optimizer(model)
    for residual, used in (("standard", 35), (lambda m, x: workloads.stacked_training_forward(m, x, _route_reference),
                                              49)):
        opt.zero_grad(set_to_none=True)
        loss = model(ids, labels, residual)
        loss.backward()
        # a uniform-at-start model: the loss is near log(vocab)
        assert abs(loss.item() - math.log(c.vocab_size)) < 0.5
        assert sum(p.grad is not None for p in model.parameters()) == used
        opt.step()
    with pytest.raises(ValueError):
        model(ids, labels, "no-such-stream")


def test_pre_norms_run_inside_the_sublayer_functions():
    # attn(attn_norm(h)) equals attention(rms(h) * w) with the module's own weight
    lmstep.compile_sublayers(False)
    c = lmstep.LMConfig("t", 64, 1, 4, 2, 16, 96, vocab_size=128, batch=1, seq=8)
    model = lmstep.LanguageModel(c, "cpu", torch.float64, seed=2)
    layer = model.layers[0]
    with torch.no_grad():
        layer.attn_norm.weight.normal_()
        layer.ffn_norm.weight.normal_()
    h = torch.randn(1, 8, 64, dtype=torch.float64)
    assert torch.equal(layer.attn_norm(h), h)
    a = layer.attn(layer.attn_norm(h), model.rope_cos, model.rope_sin, None)
    normed = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + c.norm_eps) * layer.attn_norm.weight
    q = F.linear(normed, layer.attn.wq).view(1, 8, 4, 16).transpose(1, 2)
    k = F.linear(normed, layer.attn.wk).view(1, 8, 2, 16).transpose(1, 2)
    v = F.linear(normed, layer.attn.wv).view(1, 8, 2, 16).transpose(1, 2)
    qn = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + c.norm_eps) * layer.attn.q_norm.weight
    kn = k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + c.norm_eps) * layer.attn.k_norm.weight

    def rope(x):
        rot = torch.cat((-x[..., 8:], x[..., :8]), -1)
        return x * model.rope_cos + rot * model.rope_sin

    o = F.scaled_dot_product_attention(rope(qn), rope(kn), v, is_causal=True, enable_gqa=True)
    want = F.linear(o.transpose(1, 2).reshape(1, 8, 64), layer.attn.wo)
    torch.testing.assert_close(a, want, rtol=1e-12, atol=1e-12)
    f = layer.ffn(layer.ffn_norm(h))
    normed = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + c.norm_eps) * layer.ffn_norm.weight
    want = F.linear(F.silu(F.linear(normed, layer.ffn.wg)) * F.linear(normed, layer.ffn.wu), layer.ffn.wd)
    torch.testing.assert_close(f, want, rtol=1e-12, atol=1e-12)


def test_bench_comparator_loop_is_the_reference_loop():
    # bench.py's comparator (the reference's loop and routing ops, compiled by inductor with the
    # padded stack inside the compiled function) gives the reference loop's loss and gradients
    import copy
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench

    lmstep.compile_sublayers(False)
    c = lmstep.LMConfig("t", 64, 3, 4, 2, 16, 96, vocab_size=128, attn_res_n_blocks=2, batch=2, seq=16)
    model = lmstep.LanguageModel(c, "cpu", torch.float64, seed=3)
    with torch.no_grad():  # routing away from uniform
        for name, p in model.named_parameters():
            if "res_query" in name:
                p.normal_(0.0, 0.3)
    ids, labels = lmstep.make_batch(c, "cpu", seed=4)
    other = copy.deepcopy(model)
    loss = model(ids, labels, bench.reference_routing_loop())
    loss.backward()
    ref = other(ids, labels, lambda m, x: workloads.stacked_training_forward(m, x, _route_reference))
    ref.backward()
    torch.testing.assert_close(loss, ref, rtol=1e-12, atol=1e-12)
    for (name, p), q in zip(model.named_parameters(), other.parameters()):
        assert (p.grad is None) == (q.grad is None), name
        if p.grad is not None:
            torch.testing.assert_close(p.grad, q.grad, rtol=1e-9, atol=1e-12, msg=name)
