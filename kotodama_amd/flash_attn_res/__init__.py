"""Import-path mirror of the reference's ``src/model/flash_attn_res`` package.

``from kotodama_amd.flash_attn_res import phase_1_batched_attention_triton_op,
phase_2_online_softmax_merge_triton_op`` resolves to the gfx950 HIP kernels,
with the reference's names and signatures (ops/phase_1.py:69-85,
ops/phase_2.py:8-24).  The ``_triton_op`` names are kept so existing callers
(serve.py:39-40) switch by changing only the package they import from.
"""

from .ops.phase_1 import (
    phase_1_batched_attention,
    phase_1_batched_attention_forward_with_aux,
    phase_1_batched_attention_triton_op,
)
from .ops.phase_2 import (
    phase_2_online_softmax_merge,
    phase_2_online_softmax_merge_forward_with_aux,
    phase_2_online_softmax_merge_triton_op,
)

__all__ = [
    "phase_1_batched_attention",
    "phase_1_batched_attention_forward_with_aux",
    "phase_1_batched_attention_triton_op",
    "phase_2_online_softmax_merge",
    "phase_2_online_softmax_merge_forward_with_aux",
    "phase_2_online_softmax_merge_triton_op",
]
