"""The reference's CPU routing path, restated in torch — TEST/BENCH INFRASTRUCTURE ONLY.

Used by ``bench.py``'s ``cpu_baseline`` leg (timed on the host cores) and by
tests as a second, independent float32 implementation next to the float64
numpy oracle.  The product never imports it.

On CPU tensors ``LuxiaBaseModel._route_static`` takes the einsum branch
(llama.py:633 is false), and ``_forward_attn_res`` rebuilds the padded
``(max_S, B, T, D)`` buffer with ``torch.stack`` before every call
(llama.py:690-695).  The op sequence timed here is that path, step for step:

1. ``pow -> mean(-1) -> + eps -> rsqrt``             (llama.py:640)
2. ``mul(qw) -> sum(-1) -> * rsqrt``                 (llama.py:641)
3. ``masked_fill(~mask, -inf)``                      (llama.py:642)
4. ``softmax(dim=0)``                                (llama.py:643)
5. ``mul -> sum(0)``                                 (llama.py:644)

over all max_S slots (zero padding included), in float32: the reference
only casts the model to bf16 on CUDA (serve.py:209-211).
"""

from __future__ import annotations

import torch


def pad_and_stack(sources: list[torch.Tensor], max_sources: int) -> torch.Tensor:
    """Zero-pad a source list to max_S and stack it (llama.py:690-695)."""
    zero = torch.zeros_like(sources[0])
    padded = list(sources) + [zero] * (max_sources - len(sources))
    return torch.stack(padded, dim=0)


def route_static_cpu(buf: torch.Tensor, qw: torch.Tensor, eps: float, active_mask: torch.Tensor) -> torch.Tensor:
    """One routing call over a padded buffer on CPU (llama.py:640-644 op order)."""
    r = torch.rsqrt(buf.pow(2).mean(-1) + eps)
    logits = (buf * qw).sum(-1) * r
    logits = logits.masked_fill(~active_mask.view(-1, 1, 1), float("-inf"))
    w = torch.softmax(logits, dim=0)
    return (w.unsqueeze(-1) * buf).sum(0)


def route_weights_cpu(buf: torch.Tensor, qw: torch.Tensor, eps: float, active_mask: torch.Tensor) -> torch.Tensor:
    """The softmax weights (max_S, B, T) of the same op sequence."""
    r = torch.rsqrt(buf.pow(2).mean(-1) + eps)
    logits = (buf * qw).sum(-1) * r
    logits = logits.masked_fill(~active_mask.view(-1, 1, 1), float("-inf"))
    return torch.softmax(logits, dim=0)
