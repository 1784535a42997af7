"""Synthetic routing workloads at the shapes of the 3B / 8B models.

Five configurations (the benchmark's and the parity tests' cases):

1. ``cfg1``  fp32 anchor: D=3072, B=1, T=512, S=3; x ~ N(0,1), w ~ N(0,0.02),
   gains = 1, eps = 1e-6.
2. ``cfg2``  3B prefill sweep, bf16: D=3072, B=8, T=4096, 28 layers with
   ``attn_res_n_blocks=8`` -> boundaries {0,4,...,24}, 57 routing points with
   S = 1..8; source k ~ N(0,1) * s_k, s_k ~ logU[0.5, 4]; w ~ N(0,0.05);
   gains ~ 1 + N(0,0.1); eps = 1e-5.
3. ``cfg3``  8B deepest routing, bf16: D=4096, B=4, T=4096, S=9 (8 calls);
   s_k ~ logU[0.1, 10]; w ~ N(0,0.1); gains ~ 1 + N(0,0.1).
4. ``cfg4``  8B decode step, bf16: T=1, B=256, D=4096, 32 layers in blocks of
   4 -> 65 routing points with S = 1..9, sublayer outputs ~ N(0,1) given.
5. ``cfg5``  3B data-driven blocks, bf16: D=3072, B=2, T=4096, boundaries
   {0,3,7,12,18,23} (block ends 3,7,12,18,23,28), S up to 7; token 0 of every
   source 20x larger (BOS sink); w ~ N(0,0.2).

Sources of the sweep configurations are a pool laid out like the reference's
stacked buffer: ``(max_S, B, T, D)``; routing point j reads its first S_j
slots.  Everything is generated on the device from a seeded generator.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from .schedule import AttnResSchedule


@dataclass(frozen=True)
class Workload:
    name: str
    hidden: int
    batch: int
    seq: int
    dtype: torch.dtype
    schedule: Optional[AttnResSchedule]  # None: a single routing point
    sources: int  # S for single-point configs; max_S for scheduled ones
    calls: tuple  # S of every routing call of one step
    scale_lo: float
    scale_hi: float
    w_std: float
    gain_std: float
    eps: float
    bos_scale: float = 1.0

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    @property
    def elem_bytes(self) -> int:
        return torch.tensor([], dtype=self.dtype).element_size()

    def call_bytes(self, s: int) -> int:
        """Algorithmic HBM bytes of one routing call over s sources: s rows read + 1 written."""
        return (s + 1) * self.tokens * self.hidden * self.elem_bytes

    def step_bytes(self) -> int:
        return sum(self.call_bytes(s) for s in self.calls)


def _sched_3b() -> AttnResSchedule:
    return AttnResSchedule.build(28, n_blocks=8)


def _sched_8b() -> AttnResSchedule:
    return AttnResSchedule.build(32, n_blocks=8)


def _sched_dd() -> AttnResSchedule:
    return AttnResSchedule.build(28, boundaries=[0, 3, 7, 12, 18, 23])


def get(name: str) -> Workload:
    if name == "cfg1":
        return Workload("cfg1", 3072, 1, 512, torch.float32, None, 3, (3,), 1.0, 1.0, 0.02, 0.0, 1e-6)
    if name == "cfg2":
        s = _sched_3b()
        return Workload("cfg2", 3072, 8, 4096, torch.bfloat16, s, s.max_sources, s.active_counts, 0.5, 4.0, 0.05, 0.1, 1e-5)
    if name == "cfg3":
        return Workload("cfg3", 4096, 4, 4096, torch.bfloat16, None, 9, (9,) * 8, 0.1, 10.0, 0.1, 0.1, 1e-5)
    if name == "cfg4":
        s = _sched_8b()
        return Workload("cfg4", 4096, 256, 1, torch.bfloat16, s, s.max_sources, s.active_counts, 1.0, 1.0, 0.1, 0.1, 1e-5)
    if name == "cfg1btrain":
        # the reference's 1B intermediate model (configs/1b-intermediate.yaml: hidden 1024, 28 layers,
        # DD-v1 boundaries 0,3,7,12,21,25, sequence 2048, micro-batch 4)
        s = AttnResSchedule.build(28, boundaries=[0, 3, 7, 12, 21, 25])
        return Workload("cfg1btrain", 1024, 4, 2048, torch.bfloat16, s, s.max_sources, s.active_counts, 0.5, 4.0, 0.05,
                        0.1, 1e-5)
    if name == "cfg3train":
        # the 8B model's whole routing loop (32 layers, 8 blocks, 65 points, S up to 9) at config 3's shape
        s = _sched_8b()
        return Workload("cfg3train", 4096, 4, 4096, torch.bfloat16, s, s.max_sources, s.active_counts, 0.1, 10.0, 0.1,
                        0.1, 1e-5)
    if name == "cfg5":
        s = _sched_dd()
        return Workload(
            "cfg5", 3072, 2, 4096, torch.bfloat16, s, s.max_sources, s.active_counts, 0.5, 4.0, 0.2, 0.1, 1e-5, 20.0
        )
    raise KeyError(name)


ALL = ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5")


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_pool(w: Workload, device, seed: int, tokens: Optional[tuple] = None) -> torch.Tensor:
    """(max_S, B, T, D) source pool in the workload dtype.

    Source k is N(0,1) * s_k with s_k log-uniform in [scale_lo, scale_hi];
    with ``bos_scale`` != 1, token 0 of every sequence is multiplied by it.
    ``tokens=(B, T)`` overrides the batch shape (smaller test sizes).
    """
    b, t = tokens if tokens is not None else (w.batch, w.seq)
    g = _gen(device, seed)
    pool = torch.empty((w.sources, b, t, w.hidden), dtype=w.dtype, device=device)
    lo, hi = math.log(w.scale_lo), math.log(w.scale_hi)
    u = torch.rand((w.sources,), generator=g, device=device, dtype=torch.float32)
    scales = torch.exp(lo + (hi - lo) * u)
    for k in range(w.sources):
        x = torch.randn((b, t, w.hidden), generator=g, device=device, dtype=torch.float32)
        x.mul_(scales[k])
        if w.bos_scale != 1.0:
            x[:, 0, :].mul_(w.bos_scale)
        pool[k].copy_(x)
        del x
    return pool


def make_params(w: Workload, device, seed: int, count: int, param_dtype: Optional[torch.dtype] = None):
    """``count`` (query, gain) pairs: query ~ N(0, w_std), gain ~ 1 + N(0, gain_std)."""
    pdt = param_dtype or w.dtype
    g = _gen(device, seed + 1000)
    q = (torch.randn((count, w.hidden), generator=g, device=device) * w.w_std).to(pdt)
    gain = (1.0 + torch.randn((count, w.hidden), generator=g, device=device) * w.gain_std).to(pdt)
    return q, gain


def make_deltas(w: Workload, device, seed: int, count: int, tokens: Optional[tuple] = None) -> torch.Tensor:
    """(count, B, T, D) sublayer outputs ~ N(0,1) for the arena / decode configs."""
    b, t = tokens if tokens is not None else (w.batch, w.seq)
    g = _gen(device, seed + 2000)
    return torch.randn((count, b, t, w.hidden), generator=g, device=device, dtype=torch.float32).to(w.dtype)


# ------------------------------------------------------------ training step --


class _HalfSublayer(torch.nn.Module):
    """Stand-in for attention / the MLP in the training-step workload: ``x * 0.5``,
    one elementwise kernel each way, so the step's time is the routing side."""

    def forward(self, x: torch.Tensor, *args, **kwargs) -> torch.Tensor:
        return x * 0.5


class _RoutingNorm(torch.nn.Module):
    """The routing points' RMSNorm as the routing path uses it (llama.py:143-153):
    a gain parameter and ``eps``; its ``forward`` is never called on the path."""

    def __init__(self, gain: torch.Tensor, eps: float) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(gain)
        self.eps = eps


class _TrainingLayer(torch.nn.Module):
    def __init__(self, q_attn, g_attn, q_mlp, g_mlp, eps: float) -> None:
        super().__init__()
        self.attn_norm = torch.nn.Identity()
        self.attn = _HalfSublayer()
        self.ffn_norm = torch.nn.Identity()
        self.ffn = _HalfSublayer()
        self.attn_res_query = torch.nn.Parameter(q_attn)
        self.attn_res_norm = _RoutingNorm(g_attn, eps)
        self.mlp_res_query = torch.nn.Parameter(q_mlp)
        self.mlp_res_norm = _RoutingNorm(g_mlp, eps)


class _Cfg:
    def __init__(self, num_layers: int, norm_eps: float) -> None:
        self.num_layers = num_layers
        self.norm_eps = norm_eps


class TrainingModel(torch.nn.Module):
    """A model with the attributes the reference's AttnRes forward reads
    (llama.py:446-551, 545-571): ``layers[i].{attn_norm, attn, ffn_norm, ffn,
    attn_res_query, attn_res_norm, mlp_res_query, mlp_res_norm}``,
    ``final_res_query`` / ``final_res_norm``, ``norm``, ``rope_cos/sin``,
    ``_attn_res_boundary_set`` and the schedule tables (``_attn_res_max_sources``,
    ``_attn_res_masks``, ``_attn_res_active_counts``).  The routing queries and
    gains are the workload's (``make_params``), in its dtype and trainable; the
    sublayers are ``x * 0.5`` and the norms around them identities, so a
    training step of it is the routing calls, the caller loop's own tensor
    traffic (stacks, partial sums, commits) and autograd's gradient sums."""

    def __init__(self, w: Workload, device, seed: int) -> None:
        super().__init__()
        sched = w.schedule
        L = sched.num_layers
        q, gain = make_params(w, device, seed, sched.num_points)
        self.config = _Cfg(L, w.eps)
        self.layers = torch.nn.ModuleList(
            [_TrainingLayer(q[2 * i].clone(), gain[2 * i].clone(), q[2 * i + 1].clone(), gain[2 * i + 1].clone(), w.eps)
             for i in range(L)])
        self.final_res_query = torch.nn.Parameter(q[-1].clone())
        self.final_res_norm = _RoutingNorm(gain[-1].clone(), w.eps)
        self.norm = torch.nn.Identity()
        self._attn_res_boundary_set = frozenset(sched.boundary_set)
        self._attn_res_max_sources = sched.max_sources
        self._attn_res_active_counts = list(sched.active_counts)
        self.register_buffer("_attn_res_masks", sched.masks().to(device), persistent=False)
        self.register_buffer("rope_cos", torch.zeros(1, device=device))
        self.register_buffer("rope_sin", torch.zeros(1, device=device))


def stacked_training_forward(model, embed: torch.Tensor, route_fn) -> torch.Tensor:
    """The reference's training forward (llama.py:666-716) as it runs after the
    routing function alone is swapped: before every routing call the committed
    blocks and the partial are zero-padded to max_S and stacked (llama.py:690-695),
    a commit clones the partial and restarts from a cloned zero block
    (llama.py:701-703), and sublayer outputs are added out of place
    (llama.py:706, 712).  ``route_fn(buf, query, norm, mask, num_active)``."""
    masks = model._attn_res_masks
    counts = model._attn_res_active_counts
    max_s = model._attn_res_max_sources
    boundaries = model._attn_res_boundary_set
    committed: list = []
    partial = embed
    zero = torch.zeros_like(embed)

    def stacked():
        srcs = committed + [partial]
        srcs += [zero] * (max_s - len(srcs))
        return torch.stack(srcs, dim=0)

    for i, layer in enumerate(model.layers):
        h = route_fn(stacked(), layer.attn_res_query, layer.attn_res_norm, masks[2 * i], counts[2 * i])
        if i in boundaries:
            committed.append(partial.clone())
            partial = zero.clone()
        partial = partial + layer.attn(layer.attn_norm(h), model.rope_cos, model.rope_sin, None)
        h = route_fn(stacked(), layer.mlp_res_query, layer.mlp_res_norm, masks[2 * i + 1], counts[2 * i + 1])
        partial = partial + layer.ffn(layer.ffn_norm(h))
    L = len(model.layers)
    x = route_fn(stacked(), model.final_res_query, model.final_res_norm, masks[2 * L], counts[2 * L])
    return model.norm(x)
