"""Stack-free routing over a preallocated block arena (prefill and decode).

The reference's caller loops (``_forward_attn_res``, llama.py:666-716, and
``_forward_attn_res_cached``, llama.py:718-763) keep the committed blocks in a
Python list and, before each of the 2L+1 routing calls, zero-pad and
``torch.stack`` them into a fresh ``(max_S, B, T, D)`` buffer; a commit
clones the partial and starts a zero one; every sublayer output is added to
the partial out of place.

Here the blocks live in one arena ``(max_S, *batch, D)`` allocated once per
forward: slots ``0..n_committed-1`` are committed blocks and slot
``n_committed`` is the running partial.  One ``attnres_hip::block_step``
call per routing point adds the previous sublayer's output to the partial
(or, right after a commit, starts the new partial from it), writes it back,
and routes — a commit is only an index bump.  Per routing point this moves
(S+3) rows instead of the reference's stack (max_S writes + S reads), route
and separate add.

Under autograd (training) the same loop runs with differentiable list-based
routing calls instead (no arena mutation, still no stacked copy).
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence

import torch
from torch import Tensor

from . import ops
from .schedule import AttnResSchedule


class BlockArena:
    """The committed blocks and the partial block of one forward."""

    def __init__(self, max_sources: int, batch_shape: Sequence[int], hidden: int, dtype: torch.dtype, device) -> None:
        self.buf = torch.empty((max_sources, *batch_shape, hidden), dtype=dtype, device=device)
        self.n_committed = 0

    @property
    def max_sources(self) -> int:
        return self.buf.shape[0]

    def start(self, embed: Tensor) -> None:
        """Begin a forward: the embedding is the first partial block."""
        self.buf[0].copy_(embed)
        self.n_committed = 0

    @property
    def partial(self) -> Tensor:
        return self.buf[self.n_committed]

    @property
    def committed(self) -> Tensor:
        return self.buf[: self.n_committed]

    def step(
        self,
        query: Tensor,
        gain: Optional[Tensor],
        eps: float,
        delta: Optional[Tensor] = None,
        commit: bool = False,
        want_weights: bool = False,
    ):
        """One routing point: optional commit, partial update, route.

        Returns the routed ``(*batch, D)`` row block, or ``(out, weights,
        lse)`` when ``want_weights``.
        """
        out, w, lse = ops.block_step_call(self.buf, self.n_committed, commit, delta, query, gain, eps, want_weights)
        if commit:
            self.n_committed += 1
        return (out, w, lse) if want_weights else out


class AttnResRouter:
    """The routing side of one AttnRes forward over a :class:`BlockArena`.

    ``queries[j]`` / ``gains[j]`` are the pseudo-query and RMSNorm gain of
    routing point j in the reference's order ``[attn_0, mlp_0, attn_1, ...,
    final]`` (serve.py:85-92); ``sublayer(j, h)`` returns the residual update
    of sublayer j (attention for even j, MLP for odd j) given its routed input.
    """

    def __init__(
        self,
        schedule: AttnResSchedule,
        queries: Sequence[Tensor],
        gains: Sequence[Optional[Tensor]],
        eps: float,
    ) -> None:
        if len(queries) != schedule.num_points or len(gains) != schedule.num_points:
            raise ValueError(f"need {schedule.num_points} queries and gains")
        self.schedule = schedule
        self.queries = list(queries)
        self.gains = list(gains)
        self.eps = float(eps)

    def new_arena(self, batch_shape: Sequence[int], hidden: int, dtype: torch.dtype, device) -> BlockArena:
        return BlockArena(self.schedule.max_sources, batch_shape, hidden, dtype, device)

    def forward(
        self,
        embed: Tensor,
        sublayer: Callable[[int, Tensor], Tensor],
        arena: Optional[BlockArena] = None,
    ) -> Tensor:
        """Run all 2L+1 routing points; returns the final aggregation (before the final norm)."""
        if arena is None:
            arena = self.new_arena(embed.shape[:-1], embed.shape[-1], embed.dtype, embed.device)
        arena.start(embed)
        sched = self.schedule
        delta = None
        h = embed
        last = sched.num_points - 1
        for j in range(sched.num_points):
            h = arena.step(self.queries[j], self.gains[j], self.eps, delta=delta, commit=sched.commit_before[j])
            if j < last:
                delta = sublayer(j, h)
        return h


def _model_schedule(model) -> AttnResSchedule:
    sched = getattr(model, "_kotodama_amd_schedule", None)
    if sched is None:
        sched = AttnResSchedule.build(model.config.num_layers, boundaries=sorted(model._attn_res_boundary_set))
        model._kotodama_amd_schedule = sched
    return sched


def _model_router(model) -> AttnResRouter:
    sched = _model_schedule(model)
    queries, gains = [], []
    for layer in model.layers:
        queries += [layer.attn_res_query, layer.mlp_res_query]
        gains += [layer.attn_res_norm.weight, layer.mlp_res_norm.weight]
    queries.append(model.final_res_query)
    gains.append(model.final_res_norm.weight)
    return AttnResRouter(sched, queries, gains, model.final_res_norm.eps)


def _grad_needed(model, embed: Tensor) -> bool:
    return torch.is_grad_enabled() and (embed.requires_grad or any(p.requires_grad for p in model.parameters()))


_DEFER_UNDER_COMPILE = False


def defer_under_compile(enabled: bool = True) -> None:
    """Under ``torch.compile`` without ``fullgraph`` (the reference compiles its
    model with ``torch.compile(model)``, train.py:314-324), run each routing
    point of the training loop eagerly, as a graph break, so that the blocks'
    gradients are deferred and summed in the segment kernels as in eager mode;
    the sublayers between the points are still compiled.  Off by default: with
    ``fullgraph=True`` a graph break is an error, and the points are then
    ``attnres_hip::route_list`` calls with torch adds that inductor fuses."""
    global _DEFER_UNDER_COMPILE
    _DEFER_UNDER_COMPILE = bool(enabled)


class _PointLoop:
    """The routing side of the caller loop of llama.py:697-715 under autograd:
    the committed blocks, their gradient slots, the partial block and the
    sublayer output not yet added to it.

    Every routing point passes the committed blocks and the partial as
    separate tensors (one pointer per source, no padded ``(max_S, B, T, D)``
    copy, differentiable through the backward kernels).  A commit appends the
    partial itself (nothing mutates it later) and the new partial starts as
    the next sublayer output, which is what ``zero.clone() + attn_out`` gives.

    In eager mode each point is one ``ops.route_point``: the partial's update
    ``partial + sublayer output`` is formed by the routing kernel into a new
    tensor (attnres_route_step), and in the backward the gradients are summed
    inside the routing backward kernels — each committed block's over the
    points that read it (``ops.GradSlot``, handed back by the block's commit
    node; the points between two commits summed into all their blocks at
    once, ``ops.GradSegments``) and the partial's routing gradient with the
    gradient of the partial that the next point routes — so autograd adds no
    gradients and the loop launches no adds.  Under torch.compile (unless the
    points run eagerly, :func:`defer_under_compile`), and at points whose
    output dtype or sublayer output dtype differs from the blocks', the point
    is an ``attnres_hip::route_list`` call with torch adds, and autograd sums.
    """

    def __init__(self, embed: Tensor) -> None:
        self.committed: list[Tensor] = []
        self.slots: list[ops.GradSlot] = []
        self.segments = ops.GradSegments()  # the blocks' deferred gradients, summed segment by segment
        self.dt = embed.dtype
        self.fused = ops.accumulating_path_ok(embed)
        self.partial: Optional[Tensor] = embed
        self.pending: Optional[Tensor] = None  # the sublayer output not yet added to the partial

    def point(self, query: Tensor, norm) -> Tensor:
        gain = norm.weight
        dt = self.dt
        out_dtype = torch.promote_types(dt, torch.promote_types(query.dtype, gain.dtype))
        pending = self.pending
        if (self.fused and out_dtype == dt and (pending is None or pending.dtype == dt)
                and ops.accumulating_path_ok(query, gain, self.partial, pending)):
            h, self.partial = ops.route_point(self.committed, self.slots, self.partial, pending, query, gain,
                                              float(norm.eps), out_dtype)
        else:
            if pending is not None:
                self.partial = self.partial + pending
            h = ops.route_list_call(self.committed + [self.partial], query, gain, float(norm.eps), out_dtype)[0]
            h = h.squeeze(0)
        self.pending = None
        return h

    def commit(self) -> None:
        if self.fused:
            slot = ops.GradSlot(self.segments)
            self.committed.append(ops.commit_block(self.partial, slot))
            self.slots.append(slot)
        else:
            self.committed.append(self.partial)
        self.partial = None

    def add(self, d: Tensor) -> None:
        """The sublayer output ``d``: the new partial right after a commit, else pending."""
        if self.partial is None:
            self.partial = d.to(torch.promote_types(self.dt, d.dtype))
        else:
            self.pending = d


# The same steps as graph breaks: torch.compile runs them eagerly.
@torch.compiler.disable
def _eager_loop(embed: Tensor) -> _PointLoop:
    return _PointLoop(embed)


@torch.compiler.disable
def _eager_point(loop: _PointLoop, query: Tensor, norm) -> Tensor:
    return loop.point(query, norm)


@torch.compiler.disable
def _eager_commit(loop: _PointLoop) -> None:
    loop.commit()


@torch.compiler.disable
def _eager_add(loop: _PointLoop, d: Tensor) -> None:
    loop.add(d)


def _route_points_autograd(model, embed: Tensor, sublayer: Callable[[int, Tensor], Tensor]) -> Tensor:
    """The caller loop of llama.py:697-715 under autograd, without the stacks
    (:class:`_PointLoop`); under torch.compile with :func:`defer_under_compile`
    its routing steps run eagerly between the compiled sublayers."""
    if torch.compiler.is_compiling() and _DEFER_UNDER_COMPILE:
        loop = _eager_loop(embed)
        point, commit, add = _eager_point, _eager_commit, _eager_add
    else:
        loop = _PointLoop(embed)
        point, commit, add = _PointLoop.point, _PointLoop.commit, _PointLoop.add
    boundaries = model._attn_res_boundary_set
    for i, layer in enumerate(model.layers):
        h = point(loop, layer.attn_res_query, layer.attn_res_norm)
        if i in boundaries:
            commit(loop)
        add(loop, sublayer(2 * i, h))
        h = point(loop, layer.mlp_res_query, layer.mlp_res_norm)
        add(loop, sublayer(2 * i + 1, h))
    return point(loop, model.final_res_query, model.final_res_norm)


def forward_attn_res(model, embed: Tensor, mask: Optional[Tensor] = None) -> Tensor:
    """Drop-in for ``LuxiaBaseModel._forward_attn_res`` (llama.py:666-716).

    ``model`` has the reference's attributes (``layers[i].attn``, ``attn_norm``,
    ``ffn``, ``ffn_norm``, the AttnRes queries and norms, ``final_res_*``,
    ``norm``, ``rope_cos/sin``, ``_attn_res_boundary_set``).  All AttnRes
    norms are built with the same ``config.norm_eps`` (llama.py:462,464,543),
    so one eps serves every routing point.  Without autograd the routing
    points run as fused block steps over one arena; when gradients are needed
    (training) they run as differentiable list-based routing calls.
    """
    rope_cos, rope_sin = model.rope_cos, model.rope_sin
    layers = model.layers

    def sublayer(j: int, h: Tensor) -> Tensor:
        layer = layers[j // 2]
        if j % 2 == 0:
            return layer.attn(layer.attn_norm(h), rope_cos, rope_sin, mask)
        return layer.ffn(layer.ffn_norm(h))

    if _grad_needed(model, embed):
        return model.norm(_route_points_autograd(model, embed, sublayer))
    return model.norm(_model_router(model).forward(embed, sublayer))


def forward_attn_res_cached(model, embed: Tensor, mask: Optional[Tensor] = None, past_kv=None):
    """Drop-in for ``_forward_attn_res_cached`` (llama.py:718-763): the KV-cache
    engine's forward (prefill, and T=1 decode steps), returning
    ``(hidden, new_kv_list)``; differentiable like :func:`forward_attn_res`."""
    rope_cos, rope_sin = model.rope_cos, model.rope_sin
    layers = model.layers
    new_kv: list = []

    def sublayer(j: int, h: Tensor) -> Tensor:
        i = j // 2
        layer = layers[i]
        if j % 2 == 0:
            layer_past = past_kv[i] if past_kv is not None else None
            out, kv = layer.attn(layer.attn_norm(h), rope_cos, rope_sin, mask, layer_past, use_cache=True)
            new_kv.append(kv)
            return out
        return layer.ffn(layer.ffn_norm(h))

    if _grad_needed(model, embed):
        x = _route_points_autograd(model, embed, sublayer)
    else:
        x = _model_router(model).forward(embed, sublayer)
    return model.norm(x), new_kv
