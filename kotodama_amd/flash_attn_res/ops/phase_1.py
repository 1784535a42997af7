"""Phase 1: batched inter-block depth softmax (ops/phase_1.py:11-85 contract).

For Q pseudo-queries (already folded with their norm gains, serve.py:85-92)
and a ``(S, B, T, D)`` stack of block representations, every token gets Q
routed rows — the committed blocks are read once for all Q queries.

Contract kept from the reference:
* output ``(Q, B, T, D)`` is always bfloat16 (ops/phase_1.py:26-30);
* ``lse`` ``(Q, B, T)`` float32 is the log-sum-exp of the Q logit vectors
  (kernels/phase_1.py:98-101), the input of the phase-2 merge;
* ``num_active=None`` means every slot is active (ops/phase_1.py:75-76);
  otherwise the first ``num_active`` slots are (a prefix, as the Triton
  kernel's ``source < num_active`` mask at kernels/phase_1.py:31-33);
* differentiable (ops/phase_1.py:160-290) in the blocks and the queries, with
  the aux outputs non-differentiable as in the reference's backward
  (ops/phase_1.py:235-241).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from ... import ops


def phase_1_batched_attention_forward_with_aux(
    block_representations: Tensor,
    pseudo_queries: Tensor,
    eps: float,
    num_active: int,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(out bf16 (Q,B,T,D), lse (Q,B,T), inverse_rms_norms (B,T,S), attention_logits (Q,B,T,S)).

    Slots at or beyond ``num_active`` carry 0 in the two aux outputs (the
    reference leaves them unwritten).
    """
    s_total = block_representations.shape[0]
    out, _, lse, inv_rms, logits = ops.route_call(
        block_representations, int(num_active), pseudo_queries, None, float(eps), torch.bfloat16, want_aux=True,
        want_lse=True,
    )
    if num_active < s_total:
        pad = (0, s_total - int(num_active))
        inv_rms = F.pad(inv_rms, pad)
        logits = F.pad(logits, pad)
    return out, lse, inv_rms, logits


def phase_1_batched_attention(
    block_representations: Tensor,
    pseudo_queries: Tensor,
    eps: float,
    num_active: Optional[int] = None,
) -> tuple[Tensor, Tensor]:
    """(out (Q, B, T, D) bf16, lse (Q, B, T) fp32) — ops/phase_1.py:69-85."""
    if num_active is None:
        num_active = block_representations.shape[0]
    out, _, lse, _, _ = ops.route_call(
        block_representations, int(num_active), pseudo_queries, None, float(eps), torch.bfloat16, want_lse=True
    )
    return out, lse


# The reference's name for the same entry point (ops/phase_1.py:69).
phase_1_batched_attention_triton_op = phase_1_batched_attention
