"""kotodama_amd — MI355X (gfx950) Block Attention Residual routing.

Hand-written HIP kernels behind a C ABI (``include/attnres.h``,
``lib/libattnres_hip.so``), registered as ``torch.library`` ops
(``attnres_hip::*``), with drop-ins for the reference's routing entry points:

* :func:`kotodama_amd.routing.route_static`  — ``LuxiaBaseModel._route_static``
* :func:`kotodama_amd.routing.block_attn_res_from_list` — ``_block_attn_res_from_list``
* :mod:`kotodama_amd.flash_attn_res` — ``phase_1_batched_attention_triton_op`` /
  ``phase_2_online_softmax_merge_triton_op``
* :func:`kotodama_amd.engine.forward_attn_res` / ``forward_attn_res_cached`` —
  the prefill / KV-cache caller loops over a preallocated block arena
* :mod:`kotodama_amd.checkpoint` — routing weights from trained checkpoints
  (safe loading only)
"""

from . import ops  # noqa: F401  (registers the attnres_hip ops)
from .checkpoint import RoutingWeights, load_checkpoint_registry, load_routing_weights
from .engine import AttnResRouter, BlockArena, forward_attn_res, forward_attn_res_cached
from .routing import block_attn_res_from_list, route_static, route_weights
from .schedule import AttnResSchedule

__all__ = [
    "AttnResRouter",
    "AttnResSchedule",
    "BlockArena",
    "RoutingWeights",
    "block_attn_res_from_list",
    "forward_attn_res",
    "forward_attn_res_cached",
    "load_checkpoint_registry",
    "load_routing_weights",
    "route_static",
    "route_weights",
]
