"""The serving engine's two-phase AttnRes forward (serve.py:78-164) over the HIP ops.

``FastAttnResContext`` / ``fast_forward_attn_res`` keep the reference's
structure: per block of sublayers, one phase-1 call routes all of the block's
pseudo-queries over the committed blocks at once (each committed row read once
for the whole block), then every sublayer after the block's first merges the
running intra-block partial in with one phase-2 call.  Differences from the
reference: the committed blocks are passed to phase 1 as a list of pointers
(no ``torch.stack`` per block), and everything runs on the gfx950 kernels.

As in the reference, the effective queries are folded in the parameter dtype
and stacked in the order ``[attn_0, mlp_0, ..., final]``; sublayer ranges
start at ``2 * boundary``, so sublayers before the first boundary are skipped
when the boundaries do not include layer 0 (serve.py:121-126 behaves the same).
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch
from torch import Tensor

from . import ops


class FastAttnResContext:
    """Pre-computed state of the two-phase forward (serve.py:78-110)."""

    def __init__(self, model) -> None:
        self.eps = float(model.config.norm_eps)
        effective: list[Tensor] = []
        for layer in model.layers:
            effective.append(layer.attn_res_query * layer.attn_res_norm.weight)
            effective.append(layer.mlp_res_query * layer.mlp_res_norm.weight)
        effective.append(model.final_res_query * model.final_res_norm.weight)
        self.pseudo_queries = torch.stack(effective, dim=0).detach()  # (2L+1, D)
        self.sublayer_boundaries = [2 * b for b in sorted(model._attn_res_boundary_set)]
        rope_cos, rope_sin = model.rope_cos, model.rope_sin
        self.sublayers: list[Callable[[Tensor], Tensor]] = []
        for layer in model.layers:
            self.sublayers.append(lambda x, ly=layer: ly.attn(ly.attn_norm(x), rope_cos, rope_sin))
            self.sublayers.append(lambda x, ly=layer: ly.ffn(ly.ffn_norm(x)))
        self.final_norm = model.norm

    @classmethod
    def from_parts(
        cls,
        pseudo_queries: Tensor,
        sublayer_boundaries: Sequence[int],
        sublayers: Sequence[Callable[[Tensor], Tensor]],
        eps: float,
        final_norm: Callable[[Tensor], Tensor] = lambda x: x,
    ) -> "FastAttnResContext":
        """Build from already-folded queries and sublayer callables (no model object)."""
        ctx = cls.__new__(cls)
        ctx.eps = float(eps)
        ctx.pseudo_queries = pseudo_queries
        ctx.sublayer_boundaries = list(sublayer_boundaries)
        ctx.sublayers = list(sublayers)
        ctx.final_norm = final_norm
        return ctx


def _phase_1(blocks: list[Tensor], queries: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """(out (Q, B, T, D) bf16, lse (Q, B, T)) over a list of committed blocks."""
    out, _, lse, _, _ = ops.route_list_call(blocks, queries, None, eps, torch.bfloat16, want_lse=True)
    return out, lse


def fast_forward_attn_res(ctx: FastAttnResContext, embed: Tensor) -> Tensor:
    """Two-phase forward with variable block sizes (serve.py:113-164); returns the normed hidden state."""
    ops.check_forward_only(embed)
    blocks = [embed]
    pq = ctx.pseudo_queries
    eps = ctx.eps
    n_sub = len(ctx.sublayers)
    bounds = ctx.sublayer_boundaries
    ranges = [(start, bounds[i + 1] if i + 1 < len(bounds) else n_sub) for i, start in enumerate(bounds)]
    for start, end in ranges:
        nq = end - start
        p1_out, p1_lse = _phase_1(blocks, pq[start : start + nq], eps)
        curr = None
        for qo in range(nq):
            j = start + qo
            if qo == 0:
                curr = ctx.sublayers[j](p1_out[0])
            else:
                merged = ops.merge_call(curr, pq[j], p1_out[qo], p1_lse[qo], eps)
                curr = curr + ctx.sublayers[j](merged)
        blocks.append(curr)
    final_out, _ = _phase_1(blocks, pq[-1:], eps)
    return ctx.final_norm(final_out[0].to(embed.dtype))
