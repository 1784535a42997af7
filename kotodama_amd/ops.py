"""torch.library registration of the routing ops (namespace ``attnres_hip``).

Each op is a thin shim over the C ABI (``_capi``): it validates tensors,
allocates outputs on torch's caching allocator, and launches on the current
HIP stream of the inputs' device.  Fake (meta) implementations give shapes
for ``torch.compile``.  Inputs must be ROCm device tensors: there is no CPU
path.  ``route``, ``route_list`` and ``merge`` are differentiable (the backward kernels of ``attnres_route_bwd`` /
``attnres_merge_bwd``); ``block_step`` is forward-only.

Ops
---
``attnres_hip::route(buf, num_sources, query, gain, eps, out_dtype, want_weights, want_aux)``
    Routing over the first ``num_sources`` slots of a stacked ``(max_S, *batch, D)``
    buffer (``llama.py:605-644``; phase-1 ``ops/phase_1.py:11-66`` for
    ``query`` of shape ``(Q, D)``).
``attnres_hip::route_list(sources, query, gain, eps, out_dtype, want_weights, want_aux)``
    Same over a list of ``(*batch, D)`` tensors, with no stacked copy.
``attnres_hip::merge(partial, query, inter, inter_lse, eps)``
    Phase-2 merge (``ops/phase_2.py:27-71``).
``attnres_hip::block_step(arena, n_committed, commit, delta, query, gain, eps, want_weights)``
    One routing point over a block arena with the partial update fused in
    (the body of ``llama.py:697-715`` / ``742-762``); mutates ``arena``.
``attnres_hip::route_bwd`` / ``attnres_hip::route_list_bwd`` / ``attnres_hip::merge_bwd``
    Backward of ``route`` / ``route_list``: gradients of the sources, the
    query (one row per query) and the gain from dL/dout and dL/dlse
    (``ops/phase_1.py:88-284``, ``kernels/phase_1.py:104-280``).  The weights
    and the aux outputs (inv_rms, logits) are non-differentiable outputs, as
    in the reference, whose backward ignores their gradients
    (``ops/phase_1.py:235-241``).  ``merge_bwd`` is the phase-2 backward
    (``ops/phase_2.py:74-255``); its logit / inv_rms outputs are likewise
    non-differentiable.

Returned tuples always have the same arity; outputs that were not requested
are empty tensors.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
from torch import Tensor

from . import _capi

_DTYPE_CODES = {torch.float32: _capi.DTYPE_F32, torch.bfloat16: _capi.DTYPE_BF16}
_CODE_DTYPES = {v: k for k, v in _DTYPE_CODES.items()}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise TypeError(f"attnres_hip supports float32 and bfloat16 tensors, got {dt}") from None


def _require_device(*tensors: Optional[Tensor]) -> torch.device:
    first = None
    idx = -1
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"attnres_hip runs on ROCm device tensors only (got a {t.device.type} tensor); there is no CPU path"
            )
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise RuntimeError(f"attnres_hip: tensors on different devices ({first.device} vs {t.device})")
    assert first is not None
    return first.device


_WS_BYTES: dict = {}


def _bwd_workspace(device: torch.device, n: int, d: int) -> Tensor:
    """The routing backward's workspace for ``n`` rows of ``d`` on ``device``
    (the current device; its size, which depends on the device's CU count,
    asked of the library once per shape)."""
    key = (device.index, n, d)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        nbytes = _WS_BYTES[key] = _capi.route_bwd_workspace_size(n, d)
    return torch.empty(max(1, nbytes // 4), device=device, dtype=torch.float32)


def _no_grad_needed(*tensors: Optional[Tensor]) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(
            "this attnres_hip path (the block-arena engine / the routing-weights helper) is forward-only: "
            "run it under torch.no_grad()/inference_mode or detach the inputs; for training route through "
            "route_static / block_attn_res_from_list, which are differentiable"
        )


class _DeviceStream:
    """Make ``dev`` current for the C-ABI call and give its current stream."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev: torch.device) -> None:
        self.dev = dev
        self.prev = None

    def __enter__(self) -> int:
        idx = self.dev.index if self.dev.index is not None else torch.cuda.current_device()
        cur = torch.cuda.current_device()
        if cur != idx:
            self.prev = cur
            torch.cuda.set_device(idx)
        return torch._C._cuda_getCurrentRawStream(idx)

    def __exit__(self, *exc) -> None:
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def _fold_query(query: Tensor, gain: Optional[Tensor]) -> tuple[Tensor, Optional[Tensor], int]:
    """(query, gain, param dtype code) for the kernel.

    The kernel folds ``query * gain`` itself and rounds the product to the
    parameter dtype; when the two differ in dtype the fold is done here, in
    the promoted dtype, exactly as ``query * norm.weight`` would be.
    """
    if gain is not None and gain.dtype != query.dtype:
        query = query * gain
        gain = None
    query = query.contiguous()
    if gain is not None:
        gain = gain.contiguous()
    return query, gain, dtype_code(query.dtype)


def _outputs(
    device: torch.device,
    out_dtype: torch.dtype,
    nq: int,
    s: int,
    batch: Sequence[int],
    d: int,
    want_weights: bool,
    want_aux: bool,
    placeholders: bool = True,
    want_lse: Optional[bool] = None,
) -> tuple:
    f32 = torch.float32
    # every returned tensor is its own allocation: custom ops may not return
    # aliases.  Without placeholders (the dispatcher-free eager path) outputs
    # that were not requested are None.
    def alloc(shape, wanted):
        if not wanted and not placeholders:
            return None
        return torch.empty(shape if wanted else (0,), device=device, dtype=f32)

    out = torch.empty((nq, *batch, d), device=device, dtype=out_dtype)
    weights = alloc((nq, s, *batch), want_weights)
    lse = alloc((nq, *batch), want_weights if want_lse is None else want_lse)
    inv_rms = alloc((*batch, s), want_aux)
    logits = alloc((nq, *batch, s), want_aux)
    return out, weights, lse, inv_rms, logits


def _launch_route(
    ptrs: list[int],
    src_ld: int,
    src_dtype: torch.dtype,
    batch: Sequence[int],
    d: int,
    device: torch.device,
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    out_dtype: torch.dtype,
    want_weights: bool,
    want_aux: bool,
    placeholders: bool = True,
    want_lse: Optional[bool] = None,
) -> tuple:
    if query.dim() == 1:
        query = query.unsqueeze(0)
    if query.dim() != 2 or query.shape[1] != d:
        raise ValueError(f"attnres_hip: query must be (D,) or (Q, D) with D={d}, got {tuple(query.shape)}")
    if gain is not None and gain.shape != (d,):
        raise ValueError(f"attnres_hip: gain must be ({d},), got {tuple(gain.shape)}")
    query, gain, pcode = _fold_query(query, gain)
    nq = query.shape[0]
    s = len(ptrs)
    n = 1
    for b in batch:
        n *= b
    outs = _outputs(device, out_dtype, nq, s, batch, d, want_weights, want_aux, placeholders, want_lse)
    out, weights, lse, inv_rms, logits = outs

    def p(t: Optional[Tensor]) -> Optional[int]:
        return t.data_ptr() if t is not None and t.numel() else None

    with _DeviceStream(device) as stream:
        _capi.route_fwd(
            _capi.pointer_array(ptrs),
            s,
            n,
            d,
            src_ld,
            dtype_code(src_dtype),
            query.data_ptr(),
            gain.data_ptr() if gain is not None else None,
            nq,
            pcode,
            float(eps),
            out.data_ptr() if out.numel() else None,
            dtype_code(out_dtype),
            d,
            n * d,
            p(weights),
            p(lse),
            p(inv_rms),
            p(logits),
            stream,
        )
    return outs


# ------------------------------------------------------------------ route --


def _route_impl(buf, num_sources, query, gain, eps, out_dtype, want_weights, want_aux, placeholders=True,
                want_lse=None):
    device = _require_device(buf, query, gain)
    if buf.dim() < 2:
        raise ValueError("attnres_hip::route: buf must be (max_S, *batch, D)")
    if not 0 <= num_sources <= buf.shape[0]:
        raise ValueError(f"attnres_hip::route: num_sources={num_sources} outside [0, {buf.shape[0]}]")
    if not buf.is_contiguous():
        buf = buf.contiguous()
    d = buf.shape[-1]
    batch = tuple(buf.shape[1:-1])
    slot = buf[0].numel() if buf.shape[0] else 0
    es = buf.element_size()
    base = buf.data_ptr()
    ptrs = [base + i * slot * es for i in range(num_sources)]
    return _launch_route(ptrs, d, buf.dtype, batch, d, device, query, gain, eps, out_dtype, want_weights, want_aux,
                         placeholders, want_lse)


@torch.library.custom_op("attnres_hip::route", mutates_args=())
def route(
    buf: Tensor,
    num_sources: int,
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    out_dtype: torch.dtype,
    want_weights: bool,
    want_aux: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return _route_impl(buf, num_sources, query, gain, eps, out_dtype, want_weights, want_aux)


@route.register_fake
def _route_fake(buf, num_sources, query, gain, eps, out_dtype, want_weights, want_aux):
    nq = 1 if query.dim() == 1 else query.shape[0]
    return _outputs(buf.device, out_dtype, nq, num_sources, tuple(buf.shape[1:-1]), buf.shape[-1], want_weights, want_aux)


def _route_list_impl(sources, query, gain, eps, out_dtype, want_weights, want_aux, placeholders=True,
                     want_lse=None):
    if len(sources) == 0:
        raise ValueError("attnres_hip::route_list: empty source list (use route with num_sources=0)")
    device = _require_device(*sources, query, gain)
    ref = sources[0]
    for t in sources[1:]:
        if t.shape != ref.shape or t.dtype != ref.dtype:
            raise ValueError("attnres_hip::route_list: sources must share shape and dtype")
    d = ref.shape[-1]
    # A temporary made contiguous here is freed on return; the caching
    # allocator reuses it only for later work on this same stream, which runs
    # after the kernel has read it.
    srcs = [t if t.is_contiguous() else t.contiguous() for t in sources]
    return _launch_route(
        [t.data_ptr() for t in srcs], d, ref.dtype, tuple(ref.shape[:-1]), d, device, query, gain, eps, out_dtype,
        want_weights, want_aux, placeholders, want_lse,
    )


@torch.library.custom_op("attnres_hip::route_list", mutates_args=())
def route_list(
    sources: list[Tensor],
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    out_dtype: torch.dtype,
    want_weights: bool,
    want_aux: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return _route_list_impl(sources, query, gain, eps, out_dtype, want_weights, want_aux)


@route_list.register_fake
def _route_list_fake(sources, query, gain, eps, out_dtype, want_weights, want_aux):
    ref = sources[0]
    nq = 1 if query.dim() == 1 else query.shape[0]
    return _outputs(ref.device, out_dtype, nq, len(sources), tuple(ref.shape[:-1]), ref.shape[-1], want_weights, want_aux)


# --------------------------------------------------------------- backward --


def _launch_route_bwd(
    ptrs: list[int],
    grad_ptrs: list[int],
    src_dtype: torch.dtype,
    n: int,
    d: int,
    device: torch.device,
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    grad_out: Tensor,
    grad_lse: Optional[Tensor],
    add_ptrs: Optional[list] = None,
) -> tuple[Tensor, Optional[Tensor]]:
    """Launch attnres_route_bwd (attnres_route_bwd_add when ``add_ptrs`` holds
    addend rows: ``None`` entries for none, the gradient's own pointer to add in
    place); returns (grad_query, grad_gain) in the parameter dtype.

    ``query``/``gain`` are the op's inputs; when their dtypes differ the fold
    is taken here (as in the forward) and the product rule applied in torch.
    """
    q = query.reshape(-1)
    mixed = gain is not None and gain.dtype != q.dtype
    kq, kg, pcode = _fold_query(q, gain)
    dq = torch.empty(d, device=device, dtype=kq.dtype)
    dg = torch.empty(d, device=device, dtype=kg.dtype) if kg is not None else None
    grad_out = grad_out.reshape(n, d).contiguous()
    if grad_lse is not None:
        grad_lse = grad_lse.reshape(n).to(torch.float32).contiguous()
    with _DeviceStream(device) as stream:
        ws = _bwd_workspace(device, n, d)
        head = (_capi.pointer_array(ptrs), len(ptrs), n, d, d, dtype_code(src_dtype), kq.data_ptr(),
                kg.data_ptr() if kg is not None else None, pcode, float(eps), grad_out.data_ptr(),
                dtype_code(grad_out.dtype), d, grad_lse.data_ptr() if grad_lse is not None else None,
                _capi.pointer_array(grad_ptrs))
        tail = (d, ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), dg.data_ptr() if dg is not None else None, stream)
        if add_ptrs is not None and any(a is not None for a in add_ptrs):
            _capi.route_bwd_add(*head, _capi.pointer_array(add_ptrs), *tail)
        else:
            _capi.route_bwd(*head, *tail)
    if mixed:
        # dq is dL/dqw for qw = query * gain taken in the promoted dtype
        return (dq * gain).to(query.dtype).reshape(query.shape), (dq * q).to(gain.dtype)
    return dq.reshape(query.shape), dg


def _launch_route_bwd_queries(
    ptrs: list[int],
    grad_ptrs: list[int],
    src_dtype: torch.dtype,
    n: int,
    d: int,
    device: torch.device,
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    grad_out: Tensor,
    grad_lse: Optional[Tensor],
) -> Optional[tuple[Tensor, Optional[Tensor]]]:
    """Launch attnres_route_bwd_queries for Q >= 2 queries; (grad_query (Q, D), grad_gain), or None
    when the library has no batched kernel for the shape (nothing was written)."""
    nq = query.shape[0]
    mixed = gain is not None and gain.dtype != query.dtype
    kq, kg, pcode = _fold_query(query, gain)
    dq = torch.empty((nq, d), device=device, dtype=kq.dtype)
    dg = torch.empty(d, device=device, dtype=kg.dtype) if kg is not None else None
    grad_out = grad_out.reshape(nq, n, d).contiguous()
    if grad_lse is not None:
        grad_lse = grad_lse.reshape(nq, n).to(torch.float32).contiguous()
    with _DeviceStream(device) as stream:
        nbytes = _capi.route_bwd_queries_workspace_size(n, d, len(ptrs), nq)
        ws = torch.empty(max(1, (nbytes + 3) // 4), device=device, dtype=torch.float32)
        code = _capi.route_bwd_queries(
            _capi.pointer_array(ptrs), len(ptrs), n, d, d, dtype_code(src_dtype), kq.data_ptr(),
            kg.data_ptr() if kg is not None else None, nq, pcode, float(eps), grad_out.data_ptr(),
            dtype_code(grad_out.dtype), d, n * d, grad_lse.data_ptr() if grad_lse is not None else None,
            _capi.pointer_array(grad_ptrs), d, ws.data_ptr(), ws.numel() * 4, dq.data_ptr(),
            dg.data_ptr() if dg is not None else None, stream,
        )
    if code != _capi.OK:
        return None
    if mixed:
        # dq is dL/dqw for qw = query * gain taken in the promoted dtype
        return (dq * gain).to(query.dtype), (dq * query).sum(0).to(gain.dtype)
    return dq, dg


def _bwd_args(grad_out: Optional[Tensor], n_out_shape, device, dt) -> Tensor:
    if grad_out is None:
        grad_out = torch.zeros(n_out_shape, device=device, dtype=dt)
    return grad_out


def _route_bwd_any(
    srcs: list[Tensor],
    grads: list[Tensor],
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    grad_out: Tensor,
    grad_lse: Optional[Tensor],
) -> tuple[Tensor, Optional[Tensor]]:
    """Backward over contiguous sources into the preallocated ``grads``.

    One query: one attnres_route_bwd call.  Q > 1 queries (the batched
    phase-1 call): attnres_route_bwd_queries, one pass over the sources for
    all queries (ops/phase_1.py:160-170 accumulates the same sum over
    queries); for shapes it does not cover, one attnres_route_bwd call per
    query on fp32 copies of the sources, the source gradients summed in fp32
    and rounded once, the query gradients stacked and the gain gradients
    summed.
    """
    device = srcs[0].device
    d = srcs[0].shape[-1]
    n = srcs[0].numel() // d
    if query.dim() == 1 or query.shape[0] == 1:
        return _launch_route_bwd(
            [t.data_ptr() for t in srcs], [g.data_ptr() for g in grads], srcs[0].dtype, n, d, device, query, gain,
            eps, grad_out, grad_lse,
        )
    nq = query.shape[0]
    res = _launch_route_bwd_queries(
        [t.data_ptr() for t in srcs], [g.data_ptr() for g in grads], srcs[0].dtype, n, d, device, query, gain, eps,
        grad_out, grad_lse,
    )
    if res is not None:
        return res
    if d > 4096:  # fp32 copies of these rows exceed the fp32 row limit
        raise RuntimeError(
            f"attnres_hip: the backward of {nq} queries over {len(srcs)} sources of {d} elements is not supported "
            "(no batched kernel for this shape, and fp32 rows are limited to 4096 elements)"
        )
    s32 = [t.float().contiguous() for t in srcs]
    acc = [torch.zeros(t.shape, device=device, dtype=torch.float32) for t in srcs]
    tmp = [torch.empty(t.shape, device=device, dtype=torch.float32) for t in srcs]
    go = grad_out.reshape(nq, n, d)
    gl = grad_lse.reshape(nq, n) if grad_lse is not None else None
    dqs, dg = [], None
    for j in range(nq):
        dq_j, dg_j = _launch_route_bwd(
            [t.data_ptr() for t in s32], [t.data_ptr() for t in tmp], torch.float32, n, d, device, query[j], gain,
            eps, go[j], gl[j] if gl is not None else None,
        )
        for a, t in zip(acc, tmp):
            a.add_(t)
        dqs.append(dq_j)
        if dg_j is not None:
            dg = dg_j.float() if dg is None else dg + dg_j.float()
    for g, a in zip(grads, acc):
        g.copy_(a)
    return torch.stack(dqs, 0), (dg.to(gain.dtype) if dg is not None else None)


@torch.library.custom_op("attnres_hip::route_bwd", mutates_args=())
def route_bwd(
    buf: Tensor,
    num_sources: int,
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    grad_out: Tensor,
    grad_lse: Optional[Tensor],
    zero_inactive: bool = True,
) -> tuple[Tensor, Tensor, Tensor]:
    """(grad_buf, grad_query, grad_gain) of ``route``.

    ``grad_buf`` is zero in slots at or beyond ``num_sources`` (left
    unwritten when ``zero_inactive`` is False: for a caller whose gradient
    of those slots is discarded); ``grad_gain`` is an empty tensor when
    ``gain`` is None.  With ``num_sources == 0`` the forward output is NaN and
    so are the gradients.
    """
    device = _require_device(buf, query, gain, grad_out, grad_lse)
    buf = buf.contiguous()
    d = buf.shape[-1]
    n = buf[0].numel() // d if buf.shape[0] else 0
    grad_buf = torch.empty_like(buf)
    if zero_inactive:
        grad_buf[num_sources:].zero_()
    gq_dtype = query.dtype
    gg = torch.empty((0,), device=device, dtype=gain.dtype if gain is not None else query.dtype)
    if num_sources == 0 or n == 0:
        fill = float("nan") if num_sources == 0 else 0.0
        grad_buf.fill_(fill)
        gq = torch.full_like(query, fill, dtype=gq_dtype)
        if gain is not None:
            gg = torch.full_like(gain, fill)
        return grad_buf, gq, gg
    gq, g2 = _route_bwd_any(list(buf[:num_sources]), list(grad_buf[:num_sources]), query, gain, eps, grad_out,
                            grad_lse)
    return grad_buf, gq.reshape(query.shape), g2 if g2 is not None else gg


@route_bwd.register_fake
def _route_bwd_fake(buf, num_sources, query, gain, eps, grad_out, grad_lse, zero_inactive=True):
    gg = torch.empty_like(gain) if gain is not None else query.new_empty((0,))
    return torch.empty_like(buf), torch.empty_like(query), gg


@torch.library.custom_op("attnres_hip::route_list_bwd", mutates_args=())
def route_list_bwd(
    sources: list[Tensor],
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    grad_out: Tensor,
    grad_lse: Optional[Tensor],
) -> tuple[list[Tensor], Tensor, Tensor]:
    """(grad_sources, grad_query, grad_gain) of ``route_list``."""
    device = _require_device(*sources, query, gain, grad_out, grad_lse)
    ref = sources[0]
    d = ref.shape[-1]
    n = ref.numel() // d
    srcs = [t if t.is_contiguous() else t.contiguous() for t in sources]
    grads = [torch.empty(t.shape, device=device, dtype=t.dtype) for t in srcs]
    gg = torch.empty((0,), device=device, dtype=gain.dtype if gain is not None else query.dtype)
    if n == 0:
        gq = torch.zeros_like(query)
        if gain is not None:
            gg = torch.zeros_like(gain)
        return grads, gq, gg
    gq, g2 = _route_bwd_any(srcs, grads, query, gain, eps, grad_out, grad_lse)
    return grads, gq.reshape(query.shape), g2 if g2 is not None else gg


@route_list_bwd.register_fake
def _route_list_bwd_fake(sources, query, gain, eps, grad_out, grad_lse):
    gg = torch.empty_like(gain) if gain is not None else query.new_empty((0,))
    return [torch.empty_like(t) for t in sources], torch.empty_like(query), gg


def _inactive_grads_discarded(buf: Tensor, num_sources: int) -> bool:
    """True when ``buf`` is a ``torch.stack`` whose inputs from ``num_sources`` on
    do not require grad (the reference's zero padding, llama.py:690-695):
    their gradient rows are then dropped by the stack's backward, so the
    routing backward need not write them (zeroing them costs one row write
    per padding slot per call).  Any other producer keeps the zero fill."""
    fn = buf.grad_fn
    if fn is None or fn.name() != "StackBackward0":
        return False
    if getattr(buf, "retains_grad", False) or getattr(buf, "_backward_hooks", None):
        return False  # the buffer's own gradient is observed
    nxt = fn.next_functions
    if len(nxt) != buf.shape[0]:
        return False
    return all(f is None for f, _ in nxt[num_sources:])


def _route_setup_context(ctx, inputs, output):
    buf, num_sources, query, gain, eps, out_dtype, _, _ = inputs
    out, weights, lse, inv_rms, logits = output
    ctx.mark_non_differentiable(weights, inv_rms, logits)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(buf, query, gain)
    ctx.zero_inactive = not _inactive_grads_discarded(buf, num_sources)
    ctx.num_sources = num_sources
    ctx.eps = eps
    ctx.out_shape = tuple(out.shape)
    ctx.out_dtype = out_dtype


def _route_backward(ctx, g_out, g_w, g_lse, g_inv, g_logits):
    buf, query, gain = ctx.saved_tensors
    if g_out is None and g_lse is None:
        return None, None, None, None, None, None, None, None
    g_out = _bwd_args(g_out, ctx.out_shape, buf.device, ctx.out_dtype)
    grad_buf, gq, gg = route_bwd(buf, ctx.num_sources, query, gain, ctx.eps, g_out, g_lse, ctx.zero_inactive)
    need = ctx.needs_input_grad
    return (
        grad_buf if need[0] else None,
        None,
        gq if need[2] else None,
        gg if (gain is not None and need[3]) else None,
        None,
        None,
        None,
        None,
    )


route.register_autograd(_route_backward, setup_context=_route_setup_context)


def _route_list_setup_context(ctx, inputs, output):
    sources, query, gain, eps, out_dtype, _, _ = inputs
    out, weights, lse, inv_rms, logits = output
    ctx.mark_non_differentiable(weights, inv_rms, logits)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(*sources, query, gain)
    ctx.num_sources = len(sources)
    ctx.eps = eps
    ctx.out_shape = tuple(out.shape)
    ctx.out_dtype = out_dtype


def _route_list_backward(ctx, g_out, g_w, g_lse, g_inv, g_logits):
    saved = ctx.saved_tensors
    sources = list(saved[: ctx.num_sources])
    query, gain = saved[ctx.num_sources], saved[ctx.num_sources + 1]
    if g_out is None and g_lse is None:
        return None, None, None, None, None, None, None
    g_out = _bwd_args(g_out, ctx.out_shape, query.device, ctx.out_dtype)
    grads, gq, gg = route_list_bwd(sources, query, gain, ctx.eps, g_out, g_lse)
    need = ctx.needs_input_grad
    return (
        list(grads) if need[0] else None,
        gq if need[1] else None,
        gg if (gain is not None and need[2]) else None,
        None,
        None,
        None,
        None,
    )


route_list.register_autograd(_route_list_backward, setup_context=_route_list_setup_context)


# ------------------------------------------------- summed block gradients --
#
# In the reference's training loop (llama.py:666-716) a committed block is a
# source of every later routing point, and autograd sums the gradients those
# calls return with one add kernel per use after the first (two rows read,
# one written).  On the accumulating path each routing call's gradient of a
# committed block is added into that block's gradient buffer inside the
# backward kernel (attnres_route_bwd_add: one row read more), and the block's
# commit node hands the sum to autograd once every routing call that read the
# block has run its backward (autograd runs a node after all of its
# consumers).  Eager only: under torch.compile the loop keeps the op path.


class GradSlot:
    """The gradient of one committed block, summed over the routing calls that
    read it during one backward pass: rows accumulated in place (``buf``,
    attnres_route_bwd_add) and deferred terms (``terms``: per call its output
    gradient, coefficient records and folded query, attnres_route_bwd_defer),
    which the block's commit node sums in one pass (attnres_route_bwd_gather).
    A slot that belongs to a ``GradSegments`` (the training loop's blocks in
    commit order) has its deferred terms summed segment by segment there."""

    __slots__ = ("buf", "task", "terms", "seg")

    def __init__(self, seg: Optional["GradSegments"] = None) -> None:
        self.buf: Optional[Tensor] = None
        self.task: Optional[int] = None
        self.terms: list = []
        self.seg = seg
        if seg is not None:
            seg.slots.append(self)

    def _join(self) -> None:
        """Start over when this is a new backward pass (autograd graph task):
        what an earlier pass left (one that did not reach the commit node) is
        not added to."""
        task = torch._C._current_graph_task_id()
        if self.task != task:
            self.buf, self.terms, self.task = None, [], task

    def target(self, like: Tensor) -> tuple[Tensor, bool]:
        """The buffer for one more call's gradient and whether to add to it."""
        self._join()
        if self.buf is None:
            self.buf = torch.empty(like.shape, device=like.device, dtype=like.dtype)
            return self.buf, False
        return self.buf, True

    def defer(self, grad_out: Tensor, coef: Tensor, index: int, qfold: Tensor) -> None:
        """Record one call's term: ``grad_out`` (n, D) rows, the call's
        (n, S-1, 4) coefficient records, this block's source index in the
        call and the call's folded query."""
        self._join()
        self.terms.append((grad_out, coef, index, qfold))

    def take(self) -> tuple[Optional[Tensor], list]:
        self._join()
        buf, terms = self.buf, self.terms
        self.buf, self.terms, self.task = None, [], None
        return buf, terms


class GradSegments:
    """The committed blocks of one training loop (their GradSlots in commit
    order) and the deferred terms of the routing points whose backward ran
    since the last commit node.  Those points read exactly the blocks committed
    before them, 0 .. k, where k is the block whose commit node runs next; that
    node sums their terms into every one of those blocks in one pass
    (attnres_route_bwd_gather_seg: each point's dL/dout row read once), keeping
    the running sums of blocks 0 .. k-1 (bf16 rows, fp32 per-token sums of the
    x coefficient) for the later segments and finishing block k's gradient."""

    __slots__ = ("slots", "task", "pending", "part", "csum")

    def __init__(self) -> None:
        self.slots: list[GradSlot] = []
        self.task: Optional[int] = None
        self.pending: list = []
        self.part: dict = {}
        self.csum: dict = {}

    def _join(self) -> None:
        task = torch._C._current_graph_task_id()
        if self.task != task:
            self.pending, self.part, self.csum, self.task = [], {}, {}, task

    def add(self, slots: Sequence[Optional[GradSlot]], grad_out: Tensor, coef: Tensor, qfold: Tensor) -> bool:
        """Keep one point's deferred term if it read blocks 0 .. len(slots)-1 of
        this loop in order; False (nothing kept) otherwise."""
        k = len(slots)
        if k == 0 or k > len(self.slots) or any(a is not b for a, b in zip(slots, self.slots)):
            return False
        self._join()
        self.pending.append((grad_out, coef, qfold, k))
        return True

    def flush(self, slot: GradSlot, x: Tensor, addend: Optional[Tensor]) -> Optional[Tensor]:
        """At ``slot``'s commit node: the block's gradient (plus ``addend``) with
        the pending terms summed into it and into the earlier blocks' running
        sums; None when no term is pending for it (nothing done)."""
        self._join()
        if not self.pending:
            return self._finish(slot, x, addend)
        k = next(i for i, s in enumerate(self.slots) if s is slot)
        terms, self.pending = self.pending, []
        if any(n != k + 1 for _, _, _, n in terms) or k + 1 > _capi.SEG_MAX_BLOCKS:
            # not one segment over blocks 0 .. k: per-block sums instead
            for g, coef, qfold, n in terms:
                for j in range(n):
                    self.slots[j].defer(g, coef, j, qfold)
            return self._finish(slot, x, addend)
        d = x.shape[-1]
        n_tok = x.numel() // d
        nb = k + 1
        part_in = [self.part.get(j) for j in range(nb)]
        csum_in = [self.csum.get(j) for j in range(nb)]
        part_out = [p if p is not None else torch.empty((n_tok, d), device=x.device, dtype=x.dtype)
                    for p in part_in[:k]]
        csum_out = [c if c is not None else torch.empty(n_tok, device=x.device, dtype=torch.float32)
                    for c in csum_in[:k]]
        out = addend if addend is not None else torch.empty(x.shape, device=x.device, dtype=x.dtype)
        last_csum = torch.empty(n_tok, device=x.device, dtype=torch.float32) if len(terms) > _capi.SEG_MAX_TERMS \
            else None
        with _DeviceStream(x.device) as stream:
            _capi.route_bwd_gather_seg(
                nb, n_tok, d, dtype_code(x.dtype), len(terms),
                _capi.pointer_array([g.data_ptr() for g, _, _, _ in terms]), d,
                _capi.pointer_array([c.data_ptr() for _, c, _, _ in terms]),
                _capi.int64_array([4 * c.shape[1] for _, c, _, _ in terms]),
                _capi.pointer_array([q.data_ptr() for _, _, q, _ in terms]),
                _capi.pointer_array([p.data_ptr() if p is not None else None for p in part_in]),
                _capi.pointer_array([c.data_ptr() if c is not None else None for c in csum_in]),
                _capi.pointer_array([p.data_ptr() for p in part_out] + [out.data_ptr()]),
                _capi.pointer_array([c.data_ptr() for c in csum_out] + [last_csum.data_ptr() if last_csum is not None
                                                                        else None]),
                x.data_ptr(), d, addend.data_ptr() if addend is not None else None, d, stream,
            )
        for j in range(k):
            self.part[j], self.csum[j] = part_out[j], csum_out[j]
        self.part.pop(k, None)
        self.csum.pop(k, None)
        return out

    def _finish(self, slot: GradSlot, x: Tensor, addend: Optional[Tensor]) -> Optional[Tensor]:
        """A block whose last segment had no pending term: its running sum (if
        any) plus ``addend``; None when it has neither."""
        k = next(i for i, s in enumerate(self.slots) if s is slot)
        part, csum = self.part.pop(k, None), self.csum.pop(k, None)
        if part is None:
            return None
        # the running sum still lacks its x term: csum * x
        out = part.float() + csum.view(*x.shape[:-1], 1) * x.float()
        if addend is not None:
            out += addend.float()
        return out.to(x.dtype)


def _gather_terms(x: Tensor, terms: list, addend: Optional[Tensor], out: Tensor) -> None:
    """attnres_route_bwd_gather: out = addend + the deferred terms' sum."""
    d = x.shape[-1]
    n = x.numel() // d
    with _DeviceStream(x.device) as stream:
        _capi.route_bwd_gather(
            x.data_ptr(), n, d, d, dtype_code(x.dtype), len(terms),
            _capi.pointer_array([g.data_ptr() for g, _, _, _ in terms]), d,
            _capi.pointer_array([c.data_ptr() + 16 * k for _, c, k, _ in terms]),
            _capi.int64_array([4 * c.shape[1] for _, c, _, _ in terms]),
            _capi.pointer_array([q.data_ptr() for _, _, _, q in terms]),
            addend.data_ptr() if addend is not None else None, out.data_ptr(), d, stream,
        )


class _Commit(torch.autograd.Function):
    """A block becoming committed (llama.py:701-702): the identity forward; the
    backward returns the gradient summed in the block's GradSlot, plus what
    autograd delivered from uses outside the accumulating calls."""

    @staticmethod
    def forward(ctx, block, slot):
        ctx.slot = slot
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(block)
        return block.view_as(block)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        acc, terms = ctx.slot.take()
        if acc is not None and grad is not None:
            acc.add_(grad)
        elif acc is None:
            acc = grad
        seg = ctx.slot.seg
        if not terms and (seg is None or (not seg.pending and not seg.part)):
            return acc, None
        (x,) = ctx.saved_tensors
        x = x if x.is_contiguous() else x.contiguous()
        if acc is not None and not acc.is_contiguous():
            acc = acc.contiguous()
        if acc is grad and acc is not None:
            acc = acc.clone()  # written in place below; autograd's own gradient is left as it is
        if seg is not None:
            out = seg.flush(ctx.slot, x, acc)
            if out is not None:
                acc = out
                _, terms = ctx.slot.take()  # a segment that fell back to per-block sums
        if not terms:
            return acc, None
        out = acc if acc is not None else torch.empty(x.shape, device=x.device, dtype=x.dtype)
        _gather_terms(x, terms, acc, out)
        return out, None


def commit_block(block: Tensor, slot: GradSlot) -> Tensor:
    """``block`` as a committed source whose routing gradients accumulate in ``slot``."""
    return _Commit.apply(block, slot)


def _route_rows_forward(sources, query, gain, eps, out_dtype) -> Tensor:
    out = _route_list_impl(list(sources), query, gain, eps, out_dtype, False, False, placeholders=False)[0]
    return out.view(out.shape[1:])


def _route_rows_backward(sources, grads, adds, query, gain, eps, grad_out) -> tuple[Tensor, Optional[Tensor]]:
    """attnres_route_bwd(_add) into ``grads``; ``adds[s]`` is None or the row block added to source s's gradient."""
    device = sources[0].device
    d = sources[0].shape[-1]
    n = sources[0].numel() // d
    return _launch_route_bwd(
        [t.data_ptr() for t in sources], [g.data_ptr() for g in grads], sources[0].dtype, n, d, device, query, gain,
        eps, grad_out, None, add_ptrs=[a.data_ptr() if a is not None else None for a in adds],
    )


def _route_rows_backward_defer(sources, query, gain, eps, grad_out, grad_add):
    """attnres_route_bwd_defer: (partial's gradient, (n, S-1, 4) coefficient
    records, folded query, grad_out as (n, D) rows, grad_query, grad_gain),
    or None when the library has no deferred kernel for the call."""
    p = sources[-1]
    device = p.device
    d = p.shape[-1]
    n = p.numel() // d
    q = query.reshape(-1)
    if p.dtype != torch.bfloat16 or d not in (512, 1024, 3072, 4096) or (gain is not None and gain.dtype != q.dtype):
        return None  # no deferred kernel (the library decides the rest)
    kq, kg, pcode = _fold_query(q, gain)
    grad_out = grad_out.reshape(n, d).contiguous()
    gp = torch.empty(p.shape, device=device, dtype=p.dtype)
    coef = torch.empty((n, len(sources) - 1, 4), device=device, dtype=torch.float32)
    qfold = torch.empty(d, device=device, dtype=kq.dtype)
    dq = torch.empty(d, device=device, dtype=kq.dtype)
    dg = torch.empty(d, device=device, dtype=kg.dtype) if kg is not None else None
    with _DeviceStream(device) as stream:
        ws = _bwd_workspace(device, n, d)
        code = _capi.route_bwd_defer(
            _capi.pointer_array([t.data_ptr() for t in sources]), len(sources), n, d, d, dtype_code(p.dtype),
            kq.data_ptr(), kg.data_ptr() if kg is not None else None, pcode, float(eps), grad_out.data_ptr(),
            dtype_code(grad_out.dtype), d, None, gp.data_ptr(), grad_add.data_ptr() if grad_add is not None else None,
            d, coef.data_ptr(), qfold.data_ptr(), ws.data_ptr(), ws.numel() * 4, dq.data_ptr(),
            dg.data_ptr() if dg is not None else None, stream,
        )
    if code != _capi.OK:
        return None
    return gp, coef, qfold, grad_out, dq.reshape(query.shape), dg


def _route_rows_step(committed, partial, delta, query, gain, eps, out_dtype) -> tuple[Tensor, Tensor]:
    """attnres_route_step: (routed rows, partial + delta in a new tensor)."""
    device = _require_device(*committed, partial, delta, query, gain)
    ref = partial
    for t in (*committed, delta):
        if t.shape != ref.shape or t.dtype != ref.dtype:
            raise ValueError("attnres_hip: blocks, partial and delta must share shape and dtype")
    d = ref.shape[-1]
    n = ref.numel() // d
    q = query.reshape(1, -1) if query.dim() == 1 else query
    kq, kg, pcode = _fold_query(q, gain)
    srcs = [t if t.is_contiguous() else t.contiguous() for t in committed]
    partial = partial if partial.is_contiguous() else partial.contiguous()
    delta = delta if delta.is_contiguous() else delta.contiguous()
    new_partial = torch.empty(ref.shape, device=device, dtype=ref.dtype)
    out = torch.empty(ref.shape, device=device, dtype=out_dtype)
    with _DeviceStream(device) as stream:
        _capi.route_step(
            _capi.pointer_array([t.data_ptr() for t in srcs]), len(srcs), partial.data_ptr(), delta.data_ptr(),
            new_partial.data_ptr(), n, d, dtype_code(ref.dtype), kq.data_ptr(),
            kg.data_ptr() if kg is not None else None, pcode, float(eps), out.data_ptr(), None, None, stream,
        )
    return out, new_partial


class _RoutePoint(torch.autograd.Function):
    """One routing point of the training loop, with the blocks' gradient sums
    inside the backward kernel.

    Inputs: the committed blocks (``slots[s]`` holds the GradSlot of block s,
    into which its gradient is added instead of being returned), the partial
    block before this point's update and ``delta``, the previous sublayer's
    output, or None when the partial is routed as it is.  Outputs: the routed
    rows and the partial block this point routed (``partial + delta`` in a new
    tensor, attnres_route_step; or the partial itself, as a view).  The
    backward forms the routed partial's gradient as the routing gradient plus
    the gradient of the partial output (that gradient as the kernel's addend),
    which is also the gradient of ``partial`` and of ``delta``: autograd adds
    nothing.  Where the library has a deferred kernel for the call
    (attnres_route_bwd_defer: bf16, hidden 512 / 1024 / 3072 / 4096) the committed blocks'
    gradients are not formed here: the call's output gradient and
    coefficients go to the blocks' GradSlots (their GradSegments), and the
    commit nodes sum them once (attnres_route_bwd_gather_seg, or
    attnres_route_bwd_gather per block); otherwise each block's gradient is
    added into its slot's rows (attnres_route_bwd_add)."""

    @staticmethod
    def forward(ctx, slots, eps, out_dtype, query, gain, delta, *sources):
        committed, partial = sources[:-1], sources[-1]
        if delta is None:
            out = _route_rows_forward(sources, query, gain, eps, out_dtype)
            routed = partial
            new_partial = partial.view_as(partial)
        else:
            out, new_partial = _route_rows_step(committed, partial, delta, query, gain, eps, out_dtype)
            routed = new_partial
        ctx.slots = slots
        ctx.eps = eps
        ctx.has_delta = delta is not None
        ctx.save_for_backward(query, gain, routed, *committed)
        ctx.set_materialize_grads(False)
        return out, new_partial

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g_out, g_partial):
        n_com = len(ctx.slots)
        need = ctx.needs_input_grad
        if g_out is None:
            # only the partial output is used downstream: its gradient passes through
            gp = g_partial
            return (None,) * 5 + (gp if ctx.has_delta and need[5] else None,) + (None,) * n_com + (
                gp if need[6 + n_com] else None,)
        query, gain, routed, *committed = ctx.saved_tensors
        sources = [t if t.is_contiguous() else t.contiguous() for t in (*committed, routed)]
        if g_partial is not None and not g_partial.is_contiguous():
            g_partial = g_partial.contiguous()
        com_need = need[6:6 + n_com]
        if n_com and any(com_need) and all(slot is not None or not nd for slot, nd in zip(ctx.slots, com_need)):
            # the committed blocks' gradients deferred to their commit nodes
            res = _route_rows_backward_defer(sources, query, gain, ctx.eps, g_out, g_partial)
            if res is not None:
                gp, coef, qfold, g_rows, dq, dg = res
                seg = ctx.slots[0].seg if ctx.slots[0] is not None else None
                if not (seg is not None and all(com_need) and seg.add(ctx.slots, g_rows, coef, qfold)):
                    for s_idx, (slot, nd) in enumerate(zip(ctx.slots, com_need)):
                        if nd:
                            slot.defer(g_rows, coef, s_idx, qfold)
                return ((None, None, None, dq if need[3] else None, dg if (gain is not None and need[4]) else None,
                         gp if ctx.has_delta and need[5] else None) + (None,) * n_com
                        + (gp if need[6 + n_com] else None,))
        grads, adds = [], []
        for src, slot, nd in zip(sources[:-1], ctx.slots, need[6:6 + n_com]):
            if slot is None or not nd:
                grads.append(torch.empty(src.shape, device=src.device, dtype=src.dtype))
                adds.append(None)
            else:
                buf, acc = slot.target(src)
                grads.append(buf)
                adds.append(buf if acc else None)
        p = sources[-1]
        gp = torch.empty(p.shape, device=p.device, dtype=p.dtype)
        grads.append(gp)
        adds.append(g_partial)
        dq, dg = _route_rows_backward(sources, grads, adds, query, gain, ctx.eps, g_out)
        res = [None, None, None, dq if need[3] else None, dg if (gain is not None and need[4]) else None,
               gp if ctx.has_delta and need[5] else None]
        for g, slot, nd in zip(grads[:-1], ctx.slots, need[6:6 + n_com]):
            res.append(g if (slot is None and nd) else None)
        res.append(gp if need[6 + n_com] else None)
        return tuple(res)


def accumulating_path_ok(*tensors: Optional[Tensor]) -> bool:
    """Whether the accumulating calls may run: eager autograd (no compile
    tracing, no dispatch or function modes, no functorch transforms) on plain
    tensors."""
    if (
        torch.compiler.is_compiling()
        or torch._C._len_torch_dispatch_stack()
        or torch._C._is_torch_function_mode_enabled()
        or torch._C._are_functorch_transforms_active()
    ):
        return False
    return all(t is None or type(t) in _PLAIN_TYPES for t in tensors)


def route_point(committed: Sequence[Tensor], slots: Sequence[Optional[GradSlot]], partial: Tensor,
                delta: Optional[Tensor], query: Tensor, gain: Optional[Tensor], eps: float,
                out_dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """One routing point of the training loop: (routed ``(*batch, D)`` rows, the
    partial block it routed).  The partial routed is ``partial + delta`` (a new
    tensor) or, with ``delta`` None, ``partial`` itself.  Under autograd the
    gradient of committed block s is added into ``slots[s]`` (blocks, partial,
    delta and ``out_dtype`` share one dtype)."""
    return _RoutePoint.apply(tuple(slots), float(eps), out_dtype, query, gain, delta, *committed, partial)


# ------------------------------------------------------------------ merge --


@torch.library.custom_op("attnres_hip::merge", mutates_args=())
def merge(partial: Tensor, query: Tensor, inter: Tensor, inter_lse: Tensor, eps: float) -> tuple[Tensor, Tensor, Tensor]:
    return _merge_impl(partial, query, inter, inter_lse, eps)


def _merge_impl(partial, query, inter, inter_lse, eps, aux=True):
    """Merged rows plus, with ``aux``, the fp32 logit and inverse RMS of the partial (kept for the backward)."""
    device = _require_device(partial, query, inter, inter_lse)
    d = partial.shape[-1]
    if inter.shape != partial.shape:
        raise ValueError("attnres_hip::merge: inter must have the partial's shape")
    if query.shape != (d,):
        raise ValueError(f"attnres_hip::merge: query must be ({d},)")
    if inter_lse.shape != partial.shape[:-1] or inter_lse.dtype != torch.float32:
        raise ValueError("attnres_hip::merge: inter_lse must be fp32 of shape partial.shape[:-1]")
    partial = partial.contiguous()
    inter = inter.contiguous()
    inter_lse = inter_lse.contiguous()
    query = query.contiguous()
    n = partial.numel() // d
    out = torch.empty_like(inter)
    logit = torch.empty(partial.shape[:-1], device=device, dtype=torch.float32) if aux else None
    inv_rms = torch.empty(partial.shape[:-1], device=device, dtype=torch.float32) if aux else None
    with _DeviceStream(device) as stream:
        _capi.merge_fwd(
            partial.data_ptr(),
            n,
            d,
            dtype_code(partial.dtype),
            query.data_ptr(),
            dtype_code(query.dtype),
            inter.data_ptr(),
            dtype_code(inter.dtype),
            inter_lse.data_ptr(),
            float(eps),
            out.data_ptr(),
            logit.data_ptr() if logit is not None and logit.numel() else None,
            inv_rms.data_ptr() if inv_rms is not None and inv_rms.numel() else None,
            stream,
        )
    return out, logit, inv_rms


@merge.register_fake
def _merge_fake(partial, query, inter, inter_lse, eps):
    shp = partial.shape[:-1]
    return (
        torch.empty_like(inter),
        partial.new_empty(shp, dtype=torch.float32),
        partial.new_empty(shp, dtype=torch.float32),
    )


# ------------------------------------------------------------ eager calls --
#
# Called through the dispatcher, each op costs ~24 us of host time per call
# (measured on an MI355X host: the dispatcher, four placeholder outputs, the ctypes call),
# several times the kernel of a small routing call.  The drop-ins go through
# the helpers below, which launch the same implementation directly when there
# is nothing to record: eager mode, no autograd graph to build, no tracing,
# no dispatch or function mode, plain tensors.  Otherwise they call the op.
# Outputs that were not requested are None on the direct path.

_PLAIN_TYPES = (torch.Tensor, torch.nn.Parameter)


def _eager_direct(*tensors: Optional[Tensor]) -> bool:
    if (
        torch.compiler.is_compiling()
        or torch._C._len_torch_dispatch_stack()
        or torch._C._is_torch_function_mode_enabled()
        or torch._C._are_functorch_transforms_active()
    ):
        return False
    grad = torch.is_grad_enabled()
    for t in tensors:
        if t is None:
            continue
        if type(t) not in _PLAIN_TYPES or (grad and t.requires_grad):
            return False
    return True


def route_call(buf, num_sources, query, gain, eps, out_dtype, want_weights=False, want_aux=False,
               want_lse=None) -> tuple:
    """:func:`route`, launched directly when nothing needs the dispatcher.

    ``want_lse`` asks for the lse without the weights (the op ties them).
    """
    if _eager_direct(buf, query, gain):
        return _route_impl(buf, num_sources, query, gain, eps, out_dtype, want_weights, want_aux, placeholders=False,
                           want_lse=want_lse)
    return route(buf, num_sources, query, gain, eps, out_dtype, want_weights or bool(want_lse), want_aux)


def route_list_call(sources, query, gain, eps, out_dtype, want_weights=False, want_aux=False,
                    want_lse=None) -> tuple:
    """:func:`route_list`, launched directly when nothing needs the dispatcher (``want_lse`` as in
    :func:`route_call`)."""
    if _eager_direct(query, gain, *sources):
        return _route_list_impl(sources, query, gain, eps, out_dtype, want_weights, want_aux, placeholders=False,
                                want_lse=want_lse)
    return route_list(list(sources), query, gain, eps, out_dtype, want_weights or bool(want_lse), want_aux)


def merge_call(partial, query, inter, inter_lse, eps) -> Tensor:
    """The merged rows of :func:`merge`, launched directly when nothing needs the dispatcher."""
    if _eager_direct(partial, query, inter, inter_lse):
        return _merge_impl(partial, query, inter, inter_lse, eps, aux=False)[0]
    return merge(partial, query, inter, inter_lse, eps)[0]


@torch.library.custom_op("attnres_hip::merge_bwd", mutates_args=())
def merge_bwd(
    partial: Tensor, query: Tensor, inter: Tensor, inter_lse: Tensor, eps: float, grad_out: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(grad_partial, grad_query, grad_inter, grad_inter_lse) of ``merge``."""
    device = _require_device(partial, query, inter, inter_lse, grad_out)
    d = partial.shape[-1]
    partial = partial.contiguous()
    inter = inter.contiguous()
    inter_lse = inter_lse.contiguous()
    query = query.contiguous()
    grad_out = grad_out.to(inter.dtype).contiguous()
    n = partial.numel() // d
    gp = torch.empty_like(partial)
    gi = torch.empty_like(inter)
    gl = torch.empty(partial.shape[:-1], device=device, dtype=torch.float32)
    gq = torch.zeros_like(query) if n == 0 else torch.empty_like(query)
    if n == 0:
        return gp, gq, gi, gl
    with _DeviceStream(device) as stream:
        ws = _bwd_workspace(device, n, d)
        _capi.merge_bwd(
            partial.data_ptr(),
            n,
            d,
            dtype_code(partial.dtype),
            query.data_ptr(),
            dtype_code(query.dtype),
            inter.data_ptr(),
            dtype_code(inter.dtype),
            inter_lse.data_ptr(),
            float(eps),
            grad_out.data_ptr(),
            gp.data_ptr(),
            gi.data_ptr(),
            gl.data_ptr(),
            ws.data_ptr(),
            ws.numel() * 4,
            gq.data_ptr(),
            stream,
        )
    return gp, gq, gi, gl


@merge_bwd.register_fake
def _merge_bwd_fake(partial, query, inter, inter_lse, eps, grad_out):
    return (
        torch.empty_like(partial),
        torch.empty_like(query),
        torch.empty_like(inter),
        partial.new_empty(partial.shape[:-1], dtype=torch.float32),
    )


def _merge_setup_context(ctx, inputs, output):
    partial, query, inter, inter_lse, eps = inputs
    _, logit, inv_rms = output
    ctx.mark_non_differentiable(logit, inv_rms)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(partial, query, inter, inter_lse)
    ctx.eps = eps


def _merge_backward(ctx, g_out, g_logit, g_inv):
    if g_out is None:
        return None, None, None, None, None
    partial, query, inter, inter_lse = ctx.saved_tensors
    gp, gq, gi, gl = merge_bwd(partial, query, inter, inter_lse, ctx.eps, g_out)
    need = ctx.needs_input_grad
    return (
        gp if need[0] else None,
        gq if need[1] else None,
        gi if need[2] else None,
        gl if need[3] else None,
        None,
    )


merge.register_autograd(_merge_backward, setup_context=_merge_setup_context)


# ------------------------------------------------------------- block step --


def _block_step_impl(arena, n_committed, commit, delta, query, gain, eps, want_weights, placeholders=True):
    device = _require_device(arena, delta, query, gain)
    if not arena.is_contiguous():
        raise ValueError("attnres_hip::block_step: the arena must be contiguous")
    d = arena.shape[-1]
    batch = tuple(arena.shape[1:-1])
    if delta is not None:
        if delta.shape != arena.shape[1:] or delta.dtype != arena.dtype:
            raise ValueError("attnres_hip::block_step: delta must match one arena slot in shape and dtype")
        delta = delta.contiguous()
    if query.shape != (d,):
        raise ValueError(f"attnres_hip::block_step: query must be ({d},)")
    query, gain, pcode = _fold_query(query, gain)
    s = n_committed + int(commit) + 1
    n = arena[0].numel() // d if arena.shape[0] else 0
    out = torch.empty((*batch, d), device=device, dtype=arena.dtype)
    f32 = torch.float32
    if want_weights:
        weights = torch.empty((s, *batch), device=device, dtype=f32)
        lse = torch.empty(batch, device=device, dtype=f32)
    elif placeholders:
        weights = torch.empty((0,), device=device, dtype=f32)
        lse = torch.empty((0,), device=device, dtype=f32)
    else:
        weights = lse = None
    with _DeviceStream(device) as stream:
        _capi.block_step(
            arena.data_ptr(),
            arena.shape[0],
            n * d,
            n_committed,
            int(commit),
            delta.data_ptr() if delta is not None else None,
            n,
            d,
            dtype_code(arena.dtype),
            query.data_ptr(),
            gain.data_ptr() if gain is not None else None,
            pcode,
            float(eps),
            out.data_ptr() if out.numel() else None,
            weights.data_ptr() if weights is not None and weights.numel() else None,
            lse.data_ptr() if lse is not None and lse.numel() else None,
            stream,
        )
    return out, weights, lse


@torch.library.custom_op("attnres_hip::block_step", mutates_args=("arena",))
def block_step(
    arena: Tensor,
    n_committed: int,
    commit: bool,
    delta: Optional[Tensor],
    query: Tensor,
    gain: Optional[Tensor],
    eps: float,
    want_weights: bool,
) -> tuple[Tensor, Tensor, Tensor]:
    return _block_step_impl(arena, n_committed, commit, delta, query, gain, eps, want_weights)


def block_step_call(arena, n_committed, commit, delta, query, gain, eps, want_weights=False) -> tuple:
    """:func:`block_step`, launched directly when nothing needs the dispatcher."""
    if _eager_direct(arena, delta, query, gain):
        return _block_step_impl(arena, n_committed, commit, delta, query, gain, eps, want_weights, placeholders=False)
    return block_step(arena, n_committed, commit, delta, query, gain, eps, want_weights)


@block_step.register_fake
def _block_step_fake(arena, n_committed, commit, delta, query, gain, eps, want_weights):
    s = n_committed + int(commit) + 1
    batch = tuple(arena.shape[1:-1])
    out = arena.new_empty((*batch, arena.shape[-1]))
    if want_weights:
        return out, arena.new_empty((s, *batch), dtype=torch.float32), arena.new_empty(batch, dtype=torch.float32)
    return out, arena.new_empty((0,), dtype=torch.float32), arena.new_empty((0,), dtype=torch.float32)


def check_forward_only(*tensors: Optional[Tensor]) -> None:
    """Raise if autograd would have to differentiate through the ops."""
    _no_grad_needed(*tensors)


__all__ = [
    "route",
    "route_list",
    "route_bwd",
    "route_list_bwd",
    "merge",
    "merge_bwd",
    "block_step",
    "dtype_code",
    "check_forward_only",
    "route_call",
    "route_list_call",
    "merge_call",
    "block_step_call",
]
