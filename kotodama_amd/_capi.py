"""ctypes binding of libattnres_hip.so (the C ABI in include/attnres.h).

``torch`` is imported before the library is opened: the library needs
``libamdhip64.so.7`` and the dynamic linker then binds it to the HIP runtime
torch has already loaded, so torch streams and device pointers are valid in
the library.  There is no fallback: if the library is missing, every call
raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: shares its HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libattnres_hip.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1

OK = 0
ERR_ARG = -1
ERR_UNSUPPORTED = -2
ERR_ALIGN = -3
ERR_HIP = -4

MAX_SOURCES = 16

POLICY_AUTO = 0
POLICY_WORKGROUP = 1
POLICY_STREAM = 2

_ERR_NAMES = {
    ERR_ARG: "ATTNRES_ERR_ARG",
    ERR_UNSUPPORTED: "ATTNRES_ERR_UNSUPPORTED",
    ERR_ALIGN: "ATTNRES_ERR_ALIGN",
    ERR_HIP: "ATTNRES_ERR_HIP",
}

# Exported symbols, in the order include/attnres.h declares them.
EXPORTS = (
    "attnres_version",
    "attnres_max_sources",
    "attnres_last_error",
    "attnres_set_kernel_policy",
    "attnres_route_kernel_name",
    "attnres_init",
    "attnres_route_fwd",
    "attnres_merge_fwd",
    "attnres_merge_kernel_name",
    "attnres_block_step",
    "attnres_route_step",
    "attnres_route_bwd_workspace_size",
    "attnres_route_bwd",
    "attnres_route_bwd_add",
    "attnres_route_bwd_defer",
    "attnres_route_bwd_gather",
    "attnres_route_bwd_gather_seg",
    "attnres_route_bwd_noalloc",
    "attnres_route_bwd_kernel_name",
    "attnres_route_bwd_queries_workspace_size",
    "attnres_route_bwd_queries",
    "attnres_route_bwd_queries_kernel_name",
    "attnres_merge_bwd",
)

_c_vp = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_float = ctypes.c_float

_SIGNATURES = {
    "attnres_version": ([], _c_int),
    "attnres_max_sources": ([], _c_int),
    "attnres_last_error": ([], ctypes.c_char_p),
    "attnres_init": ([], _c_int),
    "attnres_set_kernel_policy": ([_c_int], _c_int),
    "attnres_route_kernel_name": (
        [_c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.c_char_p, _c_int],
        _c_int,
    ),
    "attnres_route_fwd": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # num_queries
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # out
            _c_int,  # out_dtype
            _c_i64,  # out_ld
            _c_i64,  # out_qstride
            _c_vp,  # weights
            _c_vp,  # lse
            _c_vp,  # inv_rms
            _c_vp,  # logits
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_merge_fwd": (
        [
            _c_vp,  # partial
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_int,  # partial_dtype
            _c_vp,  # query
            _c_int,  # param_dtype
            _c_vp,  # inter
            _c_int,  # inter_dtype
            _c_vp,  # inter_lse
            _c_float,  # eps
            _c_vp,  # out
            _c_vp,  # logit
            _c_vp,  # inv_rms
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_block_step": (
        [
            _c_vp,  # arena
            _c_int,  # num_slots
            _c_i64,  # slot_stride
            _c_int,  # n_committed
            _c_int,  # commit
            _c_vp,  # delta
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_int,  # dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # out
            _c_vp,  # weights
            _c_vp,  # lse
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_workspace_size": ([_c_i64, _c_int, ctypes.POINTER(_c_i64)], _c_int),
    "attnres_route_bwd": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_int,  # grad_out_dtype
            _c_i64,  # grad_out_ld
            _c_vp,  # grad_lse
            ctypes.POINTER(_c_vp),  # grad_sources
            _c_i64,  # grad_ld
            _c_vp,  # workspace
            _c_i64,  # workspace_bytes
            _c_vp,  # grad_query
            _c_vp,  # grad_gain
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_step": (
        [
            ctypes.POINTER(_c_vp),  # committed
            _c_int,  # num_committed
            _c_vp,  # partial
            _c_vp,  # delta
            _c_vp,  # partial_out
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_int,  # dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # out
            _c_vp,  # weights
            _c_vp,  # lse
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_add": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_int,  # grad_out_dtype
            _c_i64,  # grad_out_ld
            _c_vp,  # grad_lse
            ctypes.POINTER(_c_vp),  # grad_sources
            ctypes.POINTER(_c_vp),  # grad_addend
            _c_i64,  # grad_ld
            _c_vp,  # workspace
            _c_i64,  # workspace_bytes
            _c_vp,  # grad_query
            _c_vp,  # grad_gain
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_defer": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_int,  # grad_out_dtype
            _c_i64,  # grad_out_ld
            _c_vp,  # grad_lse
            _c_vp,  # grad_partial
            _c_vp,  # grad_partial_addend
            _c_i64,  # grad_ld
            _c_vp,  # coef
            _c_vp,  # qfold
            _c_vp,  # workspace
            _c_i64,  # workspace_bytes
            _c_vp,  # grad_query
            _c_vp,  # grad_gain
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_gather": (
        [
            _c_vp,  # x
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # x_ld
            _c_int,  # dtype
            _c_int,  # num_terms
            ctypes.POINTER(_c_vp),  # grad_outs
            _c_i64,  # grad_out_ld
            ctypes.POINTER(_c_vp),  # coefs
            ctypes.POINTER(_c_i64),  # coef_lds
            ctypes.POINTER(_c_vp),  # qfolds
            _c_vp,  # addend
            _c_vp,  # out
            _c_i64,  # out_ld
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_gather_seg": (
        [
            _c_int,  # num_blocks
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_int,  # dtype
            _c_int,  # num_terms
            ctypes.POINTER(_c_vp),  # grad_outs
            _c_i64,  # grad_out_ld
            ctypes.POINTER(_c_vp),  # coefs
            ctypes.POINTER(_c_i64),  # coef_lds
            ctypes.POINTER(_c_vp),  # qfolds
            ctypes.POINTER(_c_vp),  # part_in
            ctypes.POINTER(_c_vp),  # csum_in
            ctypes.POINTER(_c_vp),  # part_out
            ctypes.POINTER(_c_vp),  # csum_out
            _c_vp,  # x
            _c_i64,  # x_ld
            _c_vp,  # addend
            _c_i64,  # out_ld
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_noalloc": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_int,  # grad_out_dtype
            _c_i64,  # grad_out_ld
            _c_vp,  # grad_lse
            ctypes.POINTER(_c_vp),  # grad_sources
            _c_i64,  # grad_ld
            _c_vp,  # grad_query
            _c_vp,  # grad_gain
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_route_bwd_queries_workspace_size": ([_c_i64, _c_int, _c_int, _c_int, ctypes.POINTER(_c_i64)], _c_int),
    "attnres_route_bwd_kernel_name": (
        [_c_int, _c_i64, _c_int, _c_int, _c_int, ctypes.c_char_p, _c_int],
        _c_int,
    ),
    "attnres_merge_kernel_name": (
        [_c_i64, _c_int, _c_int, _c_int, _c_int, ctypes.c_char_p, _c_int],
        _c_int,
    ),
    "attnres_route_bwd_queries_kernel_name": (
        [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.c_char_p, _c_int],
        _c_int,
    ),
    "attnres_route_bwd_queries": (
        [
            ctypes.POINTER(_c_vp),  # sources
            _c_int,  # num_sources
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_i64,  # src_ld
            _c_int,  # src_dtype
            _c_vp,  # query
            _c_vp,  # gain
            _c_int,  # num_queries
            _c_int,  # param_dtype
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_int,  # grad_out_dtype
            _c_i64,  # grad_out_ld
            _c_i64,  # grad_out_qstride
            _c_vp,  # grad_lse
            ctypes.POINTER(_c_vp),  # grad_sources
            _c_i64,  # grad_ld
            _c_vp,  # workspace
            _c_i64,  # workspace_bytes
            _c_vp,  # grad_query
            _c_vp,  # grad_gain
            _c_vp,  # stream
        ],
        _c_int,
    ),
    "attnres_merge_bwd": (
        [
            _c_vp,  # partial
            _c_i64,  # num_tokens
            _c_int,  # hidden
            _c_int,  # partial_dtype
            _c_vp,  # query
            _c_int,  # param_dtype
            _c_vp,  # inter
            _c_int,  # inter_dtype
            _c_vp,  # inter_lse
            _c_float,  # eps
            _c_vp,  # grad_out
            _c_vp,  # grad_partial
            _c_vp,  # grad_inter
            _c_vp,  # grad_inter_lse
            _c_vp,  # workspace
            _c_i64,  # workspace_bytes
            _c_vp,  # grad_query
            _c_vp,  # stream
        ],
        _c_int,
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class AttnResError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, fn: str, code: int, message: str) -> None:
        super().__init__(f"{fn} -> {_ERR_NAMES.get(code, code)}: {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: the MI355X routing kernels are not built "
                    "(run `python -m kotodama_amd.build` or __graft_entry__.build()); "
                    "there is no CPU fallback"
                )
            h = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            for name, (argtypes, restype) in _SIGNATURES.items():
                fn = getattr(h, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = h
    return _lib


def check(fn: str, code: int) -> None:
    if code != OK:
        msg = lib().attnres_last_error()
        raise AttnResError(fn, code, msg.decode() if msg else "")


def pointer_array(ptrs: list[int]):
    return (_c_vp * max(1, len(ptrs)))(*ptrs)


def int64_array(vals: list[int]):
    arr = (_c_i64 * max(1, len(vals)))()
    for i, v in enumerate(vals):
        arr[i] = v
    return arr


def route_fwd(*args) -> None:
    check("attnres_route_fwd", lib().attnres_route_fwd(*args))


def merge_fwd(*args) -> None:
    check("attnres_merge_fwd", lib().attnres_merge_fwd(*args))


def block_step(*args) -> None:
    check("attnres_block_step", lib().attnres_block_step(*args))


def route_bwd_workspace_size(num_tokens: int, hidden: int) -> int:
    """Bytes of workspace :func:`route_bwd` needs on the current device."""
    out = _c_i64(0)
    check("attnres_route_bwd_workspace_size", lib().attnres_route_bwd_workspace_size(num_tokens, hidden, ctypes.byref(out)))
    return int(out.value)


def route_bwd(*args) -> None:
    check("attnres_route_bwd", lib().attnres_route_bwd(*args))


def route_step(*args) -> None:
    """attnres_route_step: the partial update into a new buffer, then the routing over committed + it."""
    check("attnres_route_step", lib().attnres_route_step(*args))


def route_bwd_add(*args) -> None:
    """attnres_route_bwd with addend rows (grad_sources[s] += grad_addend[s] where non-NULL)."""
    check("attnres_route_bwd_add", lib().attnres_route_bwd_add(*args))


def route_bwd_defer(*args) -> int:
    """attnres_route_bwd_defer; returns its code (ERR_UNSUPPORTED: no deferred kernel for the call, nothing written)."""
    code = lib().attnres_route_bwd_defer(*args)
    if code not in (OK, ERR_UNSUPPORTED):
        check("attnres_route_bwd_defer", code)
    return code


def route_bwd_gather(*args) -> None:
    """attnres_route_bwd_gather: one source's gradient summed from the deferred terms of the calls that read it."""
    check("attnres_route_bwd_gather", lib().attnres_route_bwd_gather(*args))


def route_bwd_gather_seg(*args) -> None:
    """attnres_route_bwd_gather_seg: one segment's terms summed into blocks 0 .. num_blocks-1."""
    check("attnres_route_bwd_gather_seg", lib().attnres_route_bwd_gather_seg(*args))


def route_bwd_noalloc(*args) -> None:
    """attnres_route_bwd without a workspace (the library's fixed scratch array)."""
    check("attnres_route_bwd_noalloc", lib().attnres_route_bwd_noalloc(*args))


NOALLOC_SCRATCH_BYTES = 32 << 20  # ATTNRES_NOALLOC_SCRATCH_BYTES
SEG_MAX_BLOCKS = 8  # ATTNRES_SEG_MAX_BLOCKS
SEG_MAX_TERMS = 48  # ATTNRES_SEG_MAX_TERMS


def route_bwd_queries_workspace_size(num_tokens: int, hidden: int, num_sources: int, num_queries: int) -> int:
    """Bytes of workspace :func:`route_bwd_queries` needs on the current device."""
    out = _c_i64(0)
    check("attnres_route_bwd_queries_workspace_size",
          lib().attnres_route_bwd_queries_workspace_size(num_tokens, hidden, num_sources, num_queries,
                                                         ctypes.byref(out)))
    return out.value


def route_bwd_queries(*args) -> int:
    """attnres_route_bwd_queries; returns its code (ERR_UNSUPPORTED: no batched kernel for the shape)."""
    code = lib().attnres_route_bwd_queries(*args)
    if code not in (OK, ERR_UNSUPPORTED):
        check("attnres_route_bwd_queries", code)
    return code


def merge_bwd(*args) -> None:
    check("attnres_merge_bwd", lib().attnres_merge_bwd(*args))


def set_kernel_policy(policy: int) -> int:
    """Select the kernel family (POLICY_*); returns the previous policy."""
    prev = lib().attnres_set_kernel_policy(policy)
    if prev < 0:
        check("attnres_set_kernel_policy", prev)
    return prev
