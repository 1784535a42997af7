"""A small model with the reference's AttnRes attribute layout (llama.py:446-551),
for testing the caller-level drop-ins.  Sublayers are cheap deterministic maps,
not attention/FFN; only the routing path around them matters here."""

import math

import numpy as np
import torch
from torch import nn

from oracle import attnres_oracle as O


class TinyNorm(nn.Module):
    def __init__(self, d, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


class TinyAttn(nn.Module):
    """A causal stand-in for attention with a KV cache: position t adds the mean of the
    keys of every position up to t (the cached ones first) to a projection of x_t, so a
    decode step depends on ``layer_past`` and decoding with the cache equals recomputing
    the whole sequence (the contract of the reference's attention, llama.py:384-401)."""

    def __init__(self, d):
        super().__init__()
        self.proj = nn.Linear(d, d, bias=False)
        self.kproj = nn.Linear(d, d, bias=False)

    def forward(self, x, rope_cos, rope_sin, mask=None, layer_past=None, use_cache=False):
        k = torch.tanh(self.kproj(x)) * 0.5
        k_all = torch.cat([layer_past[0], k], dim=-2) if layer_past is not None else k
        t = x.shape[-2]
        t0 = k_all.shape[-2] - t
        pos = torch.arange(t0 + 1, t0 + t + 1, device=x.device).to(x.dtype).unsqueeze(-1)
        ctx = torch.cumsum(k_all, dim=-2)[..., t0:, :] / pos
        y = torch.tanh(self.proj(x) + ctx) * 0.5
        if use_cache:
            return y, (k_all, k_all)
        return y


class TinyFFN(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.proj = nn.Linear(d, d, bias=False)

    def forward(self, x):
        return torch.sin(self.proj(x)) * 0.5


class TinyElementwise(nn.Module):
    """A sublayer without matrix products: tanh(x * a + b) / 2 with (D,) parameters a, b
    (for bf16 models: no batched bf16 products anywhere in the step)."""

    def __init__(self, d):
        super().__init__()
        self.a = nn.Parameter(torch.ones(d))
        self.b = nn.Parameter(torch.zeros(d))

    def forward(self, x, rope_cos=None, rope_sin=None, mask=None, layer_past=None, use_cache=False):
        y = torch.tanh(x * self.a + self.b) * 0.5
        if use_cache:
            return y, (x, x)
        return y


class TinyLayer(nn.Module):
    def __init__(self, d, eps, elementwise=False):
        super().__init__()
        self.attn_norm = TinyNorm(d, eps)
        self.attn = TinyElementwise(d) if elementwise else TinyAttn(d)
        self.ffn_norm = TinyNorm(d, eps)
        self.ffn = TinyElementwise(d) if elementwise else TinyFFN(d)
        self.attn_res_query = nn.Parameter(torch.zeros(d))
        self.attn_res_norm = TinyNorm(d, eps)
        self.mlp_res_query = nn.Parameter(torch.zeros(d))
        self.mlp_res_norm = TinyNorm(d, eps)


class Cfg:
    def __init__(self, num_layers, norm_eps):
        self.num_layers = num_layers
        self.norm_eps = norm_eps


class TinyModel(nn.Module):
    def __init__(self, d=512, num_layers=4, boundaries=(0, 2), eps=1e-5, seed=0, elementwise=False):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.config = Cfg(num_layers, eps)
        self.layers = nn.ModuleList([TinyLayer(d, eps, elementwise) for _ in range(num_layers)])
        self.final_res_query = nn.Parameter(torch.zeros(d))
        self.final_res_norm = TinyNorm(d, eps)
        self.norm = TinyNorm(d, eps)
        self._attn_res_boundary_set = frozenset(boundaries)
        # the schedule the reference precomputes at init (llama.py:545-571)
        from kotodama_amd import AttnResSchedule

        sched = AttnResSchedule.build(num_layers, boundaries=sorted(boundaries))
        self._attn_res_max_sources = sched.max_sources
        self._attn_res_active_counts = list(sched.active_counts)
        self.register_buffer("_attn_res_masks", sched.masks(), persistent=False)
        self.register_buffer("rope_cos", torch.zeros(1))
        self.register_buffer("rope_sin", torch.zeros(1))
        with torch.no_grad():
            for p in self.parameters():
                if p.dim() == 2:
                    p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[1]))
            for layer in self.layers:
                for sub in (layer.attn, layer.ffn):
                    if isinstance(sub, TinyElementwise):
                        sub.a.copy_(1 + 0.2 * torch.randn(d, generator=g))
                        sub.b.copy_(0.1 * torch.randn(d, generator=g))
                for q in (layer.attn_res_query, layer.mlp_res_query):
                    q.copy_(torch.randn(d, generator=g) * 0.1)
                for n in (layer.attn_res_norm, layer.mlp_res_norm):
                    n.weight.copy_(1 + 0.1 * torch.randn(d, generator=g))
            self.final_res_query.copy_(torch.randn(d, generator=g) * 0.1)


def reference_forward_f64(model, embed):
    """llama.py:666-716 in float64 on the CPU, routing through the oracle."""
    m = model.double().cpu() if next(model.parameters()).dtype != torch.float64 else model
    x = embed.double().cpu()
    shape = x.shape
    d = shape[-1]

    def route(srcs, q, norm):
        qw = (q.detach() * norm.weight.detach()).numpy()
        r = O.route(np.stack([s.reshape(-1, d).numpy() for s in srcs]), qw, norm.eps)
        return torch.from_numpy(r["out"][0]).reshape(shape)

    committed, partial = [], x
    with torch.no_grad():
        for i, layer in enumerate(m.layers):
            h = route(committed + [partial], layer.attn_res_query, layer.attn_res_norm)
            if i in m._attn_res_boundary_set:
                committed.append(partial.clone())
                partial = torch.zeros_like(partial)
            partial = partial + layer.attn(layer.attn_norm(h), None, None)
            h = route(committed + [partial], layer.mlp_res_query, layer.mlp_res_norm)
            partial = partial + layer.ffn(layer.ffn_norm(h))
        h = route(committed + [partial], m.final_res_query, m.final_res_norm)
        return m.norm(h)


def reference_cached_forward_f64(model, embed, past_kv=None):
    """llama.py:718-763 in float64 on the CPU, routing through the oracle: the KV-cache
    engine's forward (a prefill, or a decode step with ``past_kv`` from the previous
    call); returns (hidden, new_kv_list).  ``model`` is a float64 CPU copy."""
    x = embed.double().cpu()
    shape = x.shape
    d = shape[-1]

    def route(srcs, q, norm):
        qw = (q.detach() * norm.weight.detach()).numpy()
        r = O.route(np.stack([s.reshape(-1, d).numpy() for s in srcs]), qw, norm.eps)
        return torch.from_numpy(r["out"][0]).reshape(shape)

    committed, partial, new_kv = [], x, []
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            h = route(committed + [partial], layer.attn_res_query, layer.attn_res_norm)
            if i in model._attn_res_boundary_set:
                committed.append(partial.clone())
                partial = torch.zeros_like(partial)
            layer_past = past_kv[i] if past_kv is not None else None
            attn_out, kv = layer.attn(layer.attn_norm(h), None, None, None, layer_past, use_cache=True)
            new_kv.append(kv)
            partial = partial + attn_out
            h = route(committed + [partial], layer.mlp_res_query, layer.mlp_res_norm)
            partial = partial + layer.ffn(layer.ffn_norm(h))
        h = route(committed + [partial], model.final_res_query, model.final_res_norm)
        return model.norm(h), new_kv


def training_forward(model, embed, route_fn):
    """The training loop of llama.py:666-716 (pad + stack before every routing call,
    out-of-place partial updates, the schedule's masks and counts precomputed at init),
    with the routing function swapped in: ``route_fn(buf, query, norm, mask, num_active)``."""
    masks = model._attn_res_masks
    counts = model._attn_res_active_counts
    max_s = model._attn_res_max_sources
    committed, partial = [], embed
    zero = torch.zeros_like(embed)

    def pad_and_stack():
        sources = committed + [partial]
        sources += [zero] * (max_s - len(sources))
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
