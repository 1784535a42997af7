"""Phase 2: online-softmax merge of the intra-block partial (ops/phase_2.py:8-71 contract).

Given the phase-1 result over the committed blocks (``inter``, with its
``lse``) and the running partial ``p`` of the current block, the merged
routing over committed blocks + partial is

    logit = (p . q) * rsqrt(mean(p^2) + eps)
    pi    = sigmoid(logit - lse)
    out   = inter + pi * (p - inter)

(kernels/phase_2.py:40-57).  Output dtype = ``inter``'s (ops/phase_2.py:41-45).
Differentiable in all four tensor inputs (the phase-2 backward,
ops/phase_2.py:211-261); the logit and inverse-RMS outputs are not, as in the
reference.
"""

from __future__ import annotations

from torch import Tensor

from ... import ops


def phase_2_online_softmax_merge_forward_with_aux(
    intrablock_partial_sum: Tensor,
    pseudo_query: Tensor,
    interblock_normalized_output: Tensor,
    interblock_lse: Tensor,
    eps: float,
) -> tuple[Tensor, Tensor, Tensor]:
    """(merged (B,T,D), intrablock_logit (B,T), intrablock_inverse_rms_norm (B,T))."""
    return ops.merge(intrablock_partial_sum, pseudo_query, interblock_normalized_output, interblock_lse, float(eps))


def phase_2_online_softmax_merge(
    intrablock_partial_sum: Tensor,
    pseudo_query: Tensor,
    interblock_normalized_output: Tensor,
    interblock_lse: Tensor,
    eps: float,
) -> Tensor:
    """Merged routing output (B, T, D) — ops/phase_2.py:8-24."""
    return ops.merge_call(intrablock_partial_sum, pseudo_query, interblock_normalized_output, interblock_lse, float(eps))


# The reference's name for the same entry point (ops/phase_2.py:8).
phase_2_online_softmax_merge_triton_op = phase_2_online_softmax_merge
