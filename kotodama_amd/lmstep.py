"""A Llama-family language model for timing AttnRes routing inside a whole training step.

The reference's own numbers for this path are training-step numbers: its
28-layer proxy model (hidden 512) trained at 117K tok/s with AttnRes against
256K tok/s with the standard residual stream on one B200, both under
torch.compile (docs/attnres-performance-brief.md:53-59); "<4%" wall-clock at
3B (README.md:81); "AttnRes routing softmax ~8%" of CUDA time (README.md:141).
This module builds the model those numbers come from, in bf16 as train.py:237
casts it, so one training step (forward, loss, backward, optimizer step) can
be timed with the residual stream as the only difference:

* ``standard`` — ``x = x + f(norm(x))`` per sublayer (llama.py:783-796);
* ``attnres`` — the routing points through this package's kernels
  (:func:`kotodama_amd.engine.forward_attn_res`: fused routing steps forward,
  deferred block gradients and their segment sums backward);
* any other caller loop ``fn(model, embed)`` of the reference's form
  (llama.py:666-716).

Layers (llama.py): RMSNorm ``x * rsqrt(mean(x^2) + eps) * w`` (:143-153); RoPE
with full-width cos/sin tables (:155-192); GQA attention with RMSNorm on the
query and key heads (qk_norm, train.py:226) and causal SDPA (:300-346); SwiGLU
``down(silu(gate(x)) * up(x))`` (:412-441); tied embeddings; cross-entropy on
the shifted logits plus ``z_loss_weight * mean(logsumexp^2)`` (:823-847).
Shapes are configs/model.yaml's (:PRESETS cites the lines).  The
AttnRes queries start at zero and the gains at one (llama.py:461-464, 542-543).

The dense work (projections, attention, SwiGLU, norms, loss) is torch on ROCm
(hipBLASLt GEMMs, SDPA's fused attention kernel).  :func:`compile_sublayers`
compiles those functions with inductor once for every layer (the layers share
shapes, so one graph serves them all); the routing loop around them stays
eager, which is where this package's kernels run.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import engine


@dataclass(frozen=True)
class LMConfig:
    """configs/model.yaml's model entries (hidden, layers, heads, KV heads, head dim, SwiGLU width)."""

    name: str
    hidden_size: int
    num_layers: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int = 49152
    rope_theta: float = 500000.0
    norm_eps: float = 1e-5
    z_loss_weight: float = 1e-5
    attn_res_n_blocks: int = 7
    attn_res_boundaries: Optional[tuple] = None
    batch: int = 4
    seq: int = 2048

    @property
    def tokens(self) -> int:
        return self.batch * self.seq


# configs/model.yaml (the 3B model :8-14, proxy :41-47, 8b :50-56, intermediate :59-65);
# micro-batch, sequence and blocks from configs/proxy-benchmark.yaml:5-6 (train.py:991's
# default of 7 blocks), 1b-intermediate.yaml:5-6,30, canary-3b.yaml:6-7,30 and
# canary-8b.yaml:7-8,31.
PRESETS = {
    "proxy": LMConfig("proxy", 512, 28, 4, 2, 128, 1408, batch=4, seq=2048),
    "1b": LMConfig("1b", 1024, 28, 8, 4, 128, 2816, attn_res_boundaries=(0, 3, 7, 12, 21, 25),
                   batch=4, seq=2048),
    "3b": LMConfig("3b", 3072, 28, 24, 8, 128, 8192, attn_res_n_blocks=8, batch=4, seq=4096),
    "8b": LMConfig("8b", 4096, 32, 32, 8, 128, 14336, attn_res_n_blocks=8, batch=2, seq=4096),
}


# ------------------------------------------------------------------ functions --


def _rms(x: Tensor, w: Tensor, eps: float) -> Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


def _attention(x: Tensor, an: Tensor, wq: Tensor, wk: Tensor, wv: Tensor, wo: Tensor, qn: Tensor, kn: Tensor,
               cos: Tensor, sin: Tensor, heads: int, kv_heads: int, head_dim: int, eps: float) -> Tensor:
    b, t, _ = x.shape
    x = _rms(x, an, eps)
    q = F.linear(x, wq).view(b, t, heads, head_dim).transpose(1, 2)
    k = F.linear(x, wk).view(b, t, kv_heads, head_dim).transpose(1, 2)
    v = F.linear(x, wv).view(b, t, kv_heads, head_dim).transpose(1, 2)
    q = _rope(_rms(q, qn, eps), cos, sin)
    k = _rope(_rms(k, kn, eps), cos, sin)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    return F.linear(o.transpose(1, 2).reshape(b, t, heads * head_dim), wo)


def _swiglu(x: Tensor, fn: Tensor, wg: Tensor, wu: Tensor, wd: Tensor, eps: float) -> Tensor:
    x = _rms(x, fn, eps)
    return F.linear(F.silu(F.linear(x, wg)) * F.linear(x, wu), wd)


def _standard_layer(x: Tensor, an: Tensor, wq: Tensor, wk: Tensor, wv: Tensor, wo: Tensor, qn: Tensor,
                    kn: Tensor, fn: Tensor, wg: Tensor, wu: Tensor, wd: Tensor, cos: Tensor, sin: Tensor,
                    heads: int, kv_heads: int, head_dim: int, eps: float) -> Tensor:
    x = x + _attention(x, an, wq, wk, wv, wo, qn, kn, cos, sin, heads, kv_heads, head_dim, eps)
    return x + _swiglu(x, fn, wg, wu, wd, eps)


def _loss(x: Tensor, fw: Tensor, emb: Tensor, labels: Tensor, eps: float, z_weight: float) -> Tensor:
    logits = F.linear(_rms(x, fw, eps), emb)
    shift = logits[:, :-1, :].reshape(-1, logits.shape[-1])
    target = labels[:, 1:].reshape(-1)
    loss = F.cross_entropy(shift, target)
    if z_weight > 0:
        loss = loss + z_weight * torch.logsumexp(shift.float(), dim=-1).pow(2).mean()
    return loss


_EAGER = {"rms": _rms, "attention": _attention, "swiglu": _swiglu, "standard_layer": _standard_layer,
          "loss": _loss}
_FN = dict(_EAGER)


def compile_sublayers(enabled: bool = True) -> None:
    """Run the dense functions compiled by inductor (``enabled``) or eagerly."""
    _FN.clear()
    if enabled:
        _FN.update({k: torch.compile(f, dynamic=False) for k, f in _EAGER.items()})
    else:
        _FN.update(_EAGER)


# -------------------------------------------------------------------- modules --


class _Norm(nn.Module):
    def __init__(self, dim: int, eps: float, device, dtype) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return _FN["rms"](x, self.weight, self.eps)


class _PreNorm(_Norm):
    """A sublayer's input RMSNorm (``attn_norm`` / ``ffn_norm``).  Its weight is
    applied inside the sublayer's function, in the same compiled graph as the
    projections that read it (as the standard layer's graph does), so the module
    itself passes its input through."""

    def forward(self, x: Tensor) -> Tensor:
        return x


def _linear(n_in: int, n_out: int, device, dtype, gen: torch.Generator) -> nn.Parameter:
    return nn.Parameter(torch.empty((n_out, n_in), device=device, dtype=dtype).normal_(0.0, 0.02, generator=gen))


class _Attention(nn.Module):
    def __init__(self, c: LMConfig, pre_norm: _PreNorm, device, dtype, gen: torch.Generator) -> None:
        super().__init__()
        self.c = c
        object.__setattr__(self, "pre_norm", pre_norm)  # owned (and registered) by the layer
        inner, kv = c.num_attention_heads * c.head_dim, c.num_kv_heads * c.head_dim
        self.wq = _linear(c.hidden_size, inner, device, dtype, gen)
        self.wk = _linear(c.hidden_size, kv, device, dtype, gen)
        self.wv = _linear(c.hidden_size, kv, device, dtype, gen)
        self.wo = _linear(inner, c.hidden_size, device, dtype, gen)
        self.q_norm = _Norm(c.head_dim, c.norm_eps, device, dtype)
        self.k_norm = _Norm(c.head_dim, c.norm_eps, device, dtype)

    def forward(self, x: Tensor, rope_cos: Tensor, rope_sin: Tensor, mask: Optional[Tensor] = None) -> Tensor:
        if mask is not None:
            raise ValueError("the training step runs causal attention without a mask")
        c = self.c
        return _FN["attention"](x, self.pre_norm.weight, self.wq, self.wk, self.wv, self.wo, self.q_norm.weight,
                                self.k_norm.weight, rope_cos, rope_sin, c.num_attention_heads, c.num_kv_heads,
                                c.head_dim, c.norm_eps)


class _SwiGLU(nn.Module):
    def __init__(self, c: LMConfig, pre_norm: _PreNorm, device, dtype, gen: torch.Generator) -> None:
        super().__init__()
        self.eps = c.norm_eps
        object.__setattr__(self, "pre_norm", pre_norm)  # owned (and registered) by the layer
        self.wg = _linear(c.hidden_size, c.intermediate_size, device, dtype, gen)
        self.wu = _linear(c.hidden_size, c.intermediate_size, device, dtype, gen)
        self.wd = _linear(c.intermediate_size, c.hidden_size, device, dtype, gen)

    def forward(self, x: Tensor) -> Tensor:
        return _FN["swiglu"](x, self.pre_norm.weight, self.wg, self.wu, self.wd, self.eps)


class _Layer(nn.Module):
    def __init__(self, c: LMConfig, device, dtype, gen: torch.Generator) -> None:
        super().__init__()
        self.attn_norm = _PreNorm(c.hidden_size, c.norm_eps, device, dtype)
        self.attn = _Attention(c, self.attn_norm, device, dtype, gen)
        self.ffn_norm = _PreNorm(c.hidden_size, c.norm_eps, device, dtype)
        self.ffn = _SwiGLU(c, self.ffn_norm, device, dtype, gen)
        self.attn_res_query = nn.Parameter(torch.zeros(c.hidden_size, device=device, dtype=dtype))
        self.attn_res_norm = _Norm(c.hidden_size, c.norm_eps, device, dtype)
        self.mlp_res_query = nn.Parameter(torch.zeros(c.hidden_size, device=device, dtype=dtype))
        self.mlp_res_norm = _Norm(c.hidden_size, c.norm_eps, device, dtype)

    def standard(self, x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
        a, f, c = self.attn, self.ffn, self.attn.c
        return _FN["standard_layer"](x, self.attn_norm.weight, a.wq, a.wk, a.wv, a.wo, a.q_norm.weight,
                                     a.k_norm.weight, self.ffn_norm.weight, f.wg, f.wu, f.wd, cos, sin,
                                     c.num_attention_heads, c.num_kv_heads, c.head_dim, c.norm_eps)


class _FinalNorm(nn.Module):
    """The model's last RMSNorm; it is applied inside the loss function so that
    inductor fuses it with the LM head's input."""

    def __init__(self, dim: int, eps: float, device, dtype) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return x


class LanguageModel(nn.Module):
    """The reference's LuxiaBaseModel shape (llama.py:446-551) with the attributes
    :func:`engine.forward_attn_res` reads; ``forward`` returns the training loss."""

    def __init__(self, c: LMConfig, device, dtype=torch.bfloat16, seed: int = 0) -> None:
        super().__init__()
        gen = torch.Generator(device=device).manual_seed(seed)
        self.config = c
        self.embed = nn.Parameter(torch.empty((c.vocab_size, c.hidden_size), device=device,
                                              dtype=dtype).normal_(0.0, 0.02, generator=gen))
        self.layers = nn.ModuleList([_Layer(c, device, dtype, gen) for _ in range(c.num_layers)])
        self.norm = _FinalNorm(c.hidden_size, c.norm_eps, device, dtype)
        self.final_res_query = nn.Parameter(torch.zeros(c.hidden_size, device=device, dtype=dtype))
        self.final_res_norm = _Norm(c.hidden_size, c.norm_eps, device, dtype)
        if c.attn_res_boundaries is not None:
            self._attn_res_boundary_set = frozenset(c.attn_res_boundaries)
        else:
            step = math.ceil(c.num_layers / c.attn_res_n_blocks)
            self._attn_res_boundary_set = frozenset(range(0, c.num_layers, step))
        self._attn_res_max_sources = len(self._attn_res_boundary_set) + 1
        masks = torch.zeros((2 * c.num_layers + 1, self._attn_res_max_sources), dtype=torch.bool)
        n = 0
        for i in range(c.num_layers):
            masks[2 * i, :n + 1] = True
            n += i in self._attn_res_boundary_set
            masks[2 * i + 1, :n + 1] = True
        masks[-1, :n + 1] = True
        self._attn_res_active_counts = [int(m.sum()) for m in masks]
        self.register_buffer("_attn_res_masks", masks.to(device), persistent=False)
        freqs = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, dtype=torch.float64) / c.head_dim))
        ang = torch.outer(torch.arange(c.seq, dtype=torch.float64), freqs)
        self.register_buffer("rope_cos", torch.cat((ang.cos(), ang.cos()), -1).to(device=device, dtype=dtype),
                             persistent=False)
        self.register_buffer("rope_sin", torch.cat((ang.sin(), ang.sin()), -1).to(device=device, dtype=dtype),
                             persistent=False)

    def hidden_states(self, input_ids: Tensor, residual) -> Tensor:
        """The last layer's output before the final norm.  ``residual`` is
        "standard", "attnres", or a caller loop ``fn(model, embed)`` in the
        form of llama.py:666-716."""
        x = F.embedding(input_ids, self.embed)
        if residual == "standard":
            for layer in self.layers:
                x = layer.standard(x, self.rope_cos, self.rope_sin)
            return x
        if residual == "attnres":
            return engine.forward_attn_res(self, x)
        if callable(residual):
            return residual(self, x)
        raise ValueError(f"unknown residual stream {residual!r}")

    def forward(self, input_ids: Tensor, labels: Tensor, residual="attnres") -> Tensor:
        x = self.hidden_states(input_ids, residual)
        c = self.config
        return _FN["loss"](x, self.norm.weight, self.embed, labels, c.norm_eps, c.z_loss_weight)


def make_batch(c: LMConfig, device, seed: int = 1) -> tuple[Tensor, Tensor]:
    g = torch.Generator(device=device).manual_seed(seed)
    ids = torch.randint(0, c.vocab_size, (c.batch, c.seq), generator=g, device=device)
    return ids, ids.clone()


def optimizer(model: nn.Module) -> torch.optim.Optimizer:
    """AdamW with the reference's AdamW settings (configs/proxy-benchmark.yaml: lr 6e-4,
    betas 0.9/0.95, weight decay 0.1), over every parameter; the fused
    implementation (a few launches for all parameters) on the GPU."""
    fused = next(model.parameters()).is_cuda
    return torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1,
                             foreach=None if fused else True, fused=fused or None)
