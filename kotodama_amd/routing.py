"""Drop-ins for the reference's routing entry points in ``src/model/llama.py``.

* :func:`route_static` — ``LuxiaBaseModel._route_static(buf, query, norm,
  active_mask, num_active=0)`` (llama.py:605-644): same arguments, same
  result, computed by the gfx950 kernel.  ``norm`` is anything with
  ``.weight`` and ``.eps`` (the reference's RMSNorm, llama.py:143-153).
* :func:`block_attn_res_from_list` — ``_block_attn_res_from_list(sources,
  query, norm)`` (llama.py:646-664), without padding or stacking: the kernel
  takes one pointer per source.

Result dtype follows the reference's einsum branch (llama.py:640-644): the
promotion of the sources' dtype with ``query * norm.weight``'s.  The kernels
accumulate in fp32 and round the output once.  There is no CPU path: CPU
tensors raise.  :func:`route_static` and :func:`block_attn_res_from_list` are
differentiable (gradients of the sources, the query and the norm gain come
from the backward kernels); :func:`route_weights` is forward-only.
"""

from __future__ import annotations

from typing import Sequence

import torch
from torch import Tensor

from . import ops


def _out_dtype(src: torch.dtype, query: Tensor, gain: Tensor) -> torch.dtype:
    return torch.promote_types(src, torch.promote_types(query.dtype, gain.dtype))


def route_static(
    buf: Tensor,
    query: Tensor,
    norm,
    active_mask: Tensor,
    num_active: int = 0,
) -> Tensor:
    """Block AttnRes routing over a padded ``(max_S, B, T, D)`` buffer.

    ``num_active > 0`` means the first ``num_active`` slots are the active
    ones (the prefix masks of llama.py:555-569, which every caller passes);
    with ``num_active == 0`` the mask is read on the host (a device sync, as
    the reference's ``active_mask.sum().item()`` at llama.py:636) and any set
    of active slots is routed by passing their pointers.
    """
    gain = norm.weight
    out_dtype = _out_dtype(buf.dtype, query, gain)
    if num_active:
        n = int(num_active)
        res = ops.route_call(buf, n, query, gain, float(norm.eps), out_dtype)
        return res[0].squeeze(0)
    idx = [i for i, a in enumerate(active_mask.reshape(-1).tolist()) if a]
    if idx == list(range(len(idx))):
        res = ops.route_call(buf, len(idx), query, gain, float(norm.eps), out_dtype)
    else:
        res = ops.route_list_call([buf[i] for i in idx], query, gain, float(norm.eps), out_dtype)
    return res[0].squeeze(0)


def block_attn_res_from_list(sources: Sequence[Tensor], query: Tensor, norm) -> Tensor:
    """Routing over a variable-length list of ``(B, T, D)`` sources (llama.py:646-664).

    The reference pads the list to max_S with zeros and masks the padding to
    -inf; the padded slots get weight exactly 0, so routing over the list
    itself gives the same result without building the padded buffer.
    """
    gain = norm.weight
    out_dtype = _out_dtype(sources[0].dtype, query, gain)
    res = ops.route_list_call(list(sources), query, gain, float(norm.eps), out_dtype)
    return res[0].squeeze(0)


def route_weights(buf: Tensor, num_active: int, query: Tensor, norm) -> tuple[Tensor, Tensor, Tensor]:
    """(out, weights (S, B, T), lse (B, T)) — the routing result plus the
    depth-softmax weights the reference's monitors recompute
    (src/monitoring/geometric.py:501-507)."""
    gain = norm.weight
    ops.check_forward_only(buf, query, gain)
    out_dtype = _out_dtype(buf.dtype, query, gain)
    out, w, lse, _, _ = ops.route_call(buf, int(num_active), query, gain, float(norm.eps), out_dtype, True)
    return out[0], w[0], lse[0]
