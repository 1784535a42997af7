"""The C-ABI library: loads, exports every declared symbol, and rejects bad
arguments on the host before touching the GPU (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest

from kotodama_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "attnres.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(attnres_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == list(_capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _capi.lib()
    raw = ctypes.CDLL(str(_capi.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(raw, name), name
    assert lib.attnres_version() >= 10000
    assert lib.attnres_max_sources() == _capi.MAX_SOURCES == 16


# C parameter types of the header and the ctypes type each must be bound with
C_TO_CTYPES = {
    "int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float, "char*": ctypes.c_char_p,
    "const void*": ctypes.c_void_p, "void*": ctypes.c_void_p, "const float*": ctypes.c_void_p,
    "float*": ctypes.c_void_p, "const void* const*": ctypes.POINTER(ctypes.c_void_p),
    "void* const*": ctypes.POINTER(ctypes.c_void_p), "int64_t*": ctypes.POINTER(ctypes.c_int64),
    "const float* const*": ctypes.POINTER(ctypes.c_void_p), "const int64_t*": ctypes.POINTER(ctypes.c_int64),
    "float* const*": ctypes.POINTER(ctypes.c_void_p),
}


def test_binding_signatures_match_the_header_prototypes():
    # a parameter bound with the wrong width (int against int64_t, say) would
    # pass wrong values through the ABI without any error
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    protos = re.findall(r"^\s*((?:const\s+)?\w+\**)\s+(attnres_\w+)\s*\((.*?)\);", text, flags=re.M | re.S)
    assert [p[1] for p in protos] == list(_capi.EXPORTS)
    for ret, name, params in protos:
        ptypes = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p in ("", "void"):
                continue
            ptypes.append(C_TO_CTYPES[re.sub(r"\s*\w+$", "", p)])
        argtypes, restype = _capi._SIGNATURES[name]
        assert list(argtypes) == ptypes, f"{name}: binding argtypes differ from the header"
        assert restype == {"int": ctypes.c_int, "const char*": ctypes.c_char_p}[ret], f"{name}: return type"


FAKE = 0x7F0000000000  # never dereferenced: argument checks run first


def route(sources, S=None, N=16, D=64, ld=None, sdt=_capi.DTYPE_BF16, query=FAKE, Q=1, pdt=_capi.DTYPE_BF16,
          eps=1e-5, out=FAKE, odt=_capi.DTYPE_BF16, out_ld=None):
    S = len(sources) if S is None else S
    return _capi.lib().attnres_route_fwd(
        _capi.pointer_array(sources), S, N, D, ld if ld is not None else D, sdt, query, None, Q, pdt, eps, out, odt,
        out_ld if out_ld is not None else D, N * D, None, None, None, None, None)


def test_python_constants_match_the_kernel_parameters():
    # the ops layer chunks segment sums by these limits; they must be the C side's
    params = (ROOT / "kotodama_amd" / "csrc" / "attnres_params.h").read_text()
    for name, value in (("ATTNRES_SEG_MAX_BLOCKS", _capi.SEG_MAX_BLOCKS), ("ATTNRES_SEG_MAX_TERMS", _capi.SEG_MAX_TERMS)):
        m = re.search(rf"#define {name} (\d+)", params)
        assert m is not None and int(m.group(1)) == value, name
    # every (row KiB, block count) the host can ask for has a compiled segment kernel
    inst = re.findall(r"X\((\d+), (\d+), (\d+), (\d+), (\d+)\)", params)
    have = {(int(a), int(b)) for a, b, *_ in inst}
    assert have == {(nch, nb) for nch in (1, 2, 6, 8) for nb in range(1, _capi.SEG_MAX_BLOCKS + 1)}
    for nch, nb, cpw, depth, wpe in ((int(v) for v in t) for t in inst):
        assert nch % cpw == 0 and depth >= 2 and 1 <= wpe <= 4, (nch, nb)


def test_route_argument_errors():
    ok_src = [FAKE + 4096 * i for i in range(3)]
    assert route(ok_src, N=0) == _capi.OK  # empty launch: returns before any HIP call
    assert route([FAKE] * 17) == _capi.ERR_UNSUPPORTED
    assert route(ok_src, S=-1) == _capi.ERR_UNSUPPORTED
    assert route(ok_src, query=None) == _capi.ERR_ARG
    assert route(ok_src, out=None) == _capi.ERR_ARG
    assert route(ok_src, Q=0) == _capi.ERR_ARG
    assert route(ok_src, sdt=7) == _capi.ERR_ARG
    assert route(ok_src, D=12) == _capi.ERR_UNSUPPORTED  # not a multiple of 8 bf16
    assert route(ok_src, D=8192 + 8) == _capi.ERR_UNSUPPORTED  # wider than the largest row
    assert route(ok_src, D=64, ld=32) == _capi.ERR_ARG
    assert route([FAKE + 2, FAKE]) == _capi.ERR_ALIGN
    assert route(ok_src, out=FAKE + 4) == _capi.ERR_ALIGN
    assert route(ok_src, eps=float("nan")) == _capi.ERR_ARG
    assert route([FAKE, 0]) == _capi.ERR_ARG
    msg = _capi.lib().attnres_last_error().decode()
    assert "sources[1]" in msg
    with pytest.raises(_capi.AttnResError, match="ATTNRES_ERR_UNSUPPORTED"):
        _capi.check("attnres_route_fwd", route([FAKE] * 17))


def step(arena=FAKE, slots=9, stride=16 * 64, nc=0, commit=0, delta=None, N=16, D=64, dt=_capi.DTYPE_BF16):
    return _capi.lib().attnres_block_step(arena, slots, stride, nc, commit, delta, N, D, dt, FAKE, None,
                                          _capi.DTYPE_BF16, 1e-5, FAKE, None, None, None)


def test_block_step_argument_errors():
    assert step(N=0) == _capi.OK
    assert step(arena=None) == _capi.ERR_ARG
    assert step(commit=1) == _capi.ERR_ARG  # a commit needs the new partial
    assert step(nc=8, commit=1, delta=FAKE) == _capi.ERR_ARG  # partial slot 9 outside 9 slots
    assert step(nc=-1) == _capi.ERR_ARG
    assert step(commit=2) == _capi.ERR_ARG
    assert step(stride=100) == _capi.ERR_ARG
    assert step(slots=20, nc=16) == _capi.ERR_UNSUPPORTED


def test_merge_argument_errors():
    lib = _capi.lib()
    args = [FAKE, 16, 64, _capi.DTYPE_BF16, FAKE, _capi.DTYPE_BF16, FAKE, _capi.DTYPE_BF16, FAKE, 1e-5, FAKE, None,
            None, None]
    a = list(args)
    a[1] = 0
    assert lib.attnres_merge_fwd(*a) == _capi.OK
    a = list(args)
    a[8] = None
    assert lib.attnres_merge_fwd(*a) == _capi.ERR_ARG
    a = list(args)
    a[2] = 60
    assert lib.attnres_merge_fwd(*a) == _capi.ERR_UNSUPPORTED


def bwd(sources=None, S=None, N=16, D=64, ld=None, sdt=_capi.DTYPE_BF16, query=FAKE, gain=None,
        pdt=_capi.DTYPE_BF16, eps=1e-5, gout=FAKE, gdt=_capi.DTYPE_BF16, gld=None, grads=None, grad_ld=None,
        ws=FAKE, ws_bytes=1 << 30, dq=FAKE, dg=None):
    sources = [FAKE + 4096 * i for i in range(3)] if sources is None else sources
    grads = [FAKE + (1 << 20) + 4096 * i for i in range(len(sources))] if grads is None else grads
    S = len(sources) if S is None else S
    return _capi.lib().attnres_route_bwd(
        _capi.pointer_array(sources), S, N, D, ld if ld is not None else D, sdt, query, gain, pdt, eps, gout, gdt,
        gld if gld is not None else D, None, _capi.pointer_array(grads), grad_ld if grad_ld is not None else D, ws,
        ws_bytes, dq, dg, None)


def test_route_bwd_argument_errors():
    assert bwd(N=0) == _capi.OK  # no tokens: returns before any HIP call
    assert bwd(S=0) == _capi.ERR_UNSUPPORTED  # nothing to differentiate
    assert bwd(sources=[FAKE] * 17, grads=[FAKE] * 17) == _capi.ERR_UNSUPPORTED
    assert bwd(query=None) == _capi.ERR_ARG
    assert bwd(gout=None) == _capi.ERR_ARG
    assert bwd(dg=FAKE) == _capi.ERR_ARG  # grad_gain without gain
    assert bwd(gdt=5) == _capi.ERR_ARG
    assert bwd(D=12) == _capi.ERR_UNSUPPORTED
    assert bwd(D=8192 + 8) == _capi.ERR_UNSUPPORTED
    assert bwd(grad_ld=32) == _capi.ERR_ARG
    assert bwd(gout=FAKE + 4) == _capi.ERR_ALIGN
    assert bwd(grads=[FAKE, FAKE + 8, FAKE]) == _capi.ERR_ALIGN
    assert bwd(eps=float("inf")) == _capi.ERR_ARG
    assert bwd(grads=[FAKE, 0, FAKE]) == _capi.ERR_ARG
    assert "grad_sources[1]" in _capi.lib().attnres_last_error().decode()


def bwdq(sources=None, S=None, N=16, D=64, Q=3, sdt=_capi.DTYPE_BF16, gain=None, gld=None, gqs=None, ws=FAKE,
         dq=FAKE, dg=None):
    sources = [FAKE + 4096 * i for i in range(3)] if sources is None else sources
    grads = [FAKE + (1 << 20) + 4096 * i for i in range(len(sources))]
    S = len(sources) if S is None else S
    gld = D if gld is None else gld
    return _capi.lib().attnres_route_bwd_queries(
        _capi.pointer_array(sources), S, N, D, D, sdt, FAKE, gain, Q, _capi.DTYPE_BF16, 1e-5, FAKE,
        _capi.DTYPE_BF16, gld, N * gld if gqs is None else gqs, None, _capi.pointer_array(grads), D, ws, 1 << 30,
        dq, dg, None)


def test_route_bwd_queries_argument_errors():
    assert bwdq(N=0) == _capi.OK  # no tokens: returns before any HIP call
    assert bwdq(S=0) == _capi.ERR_UNSUPPORTED
    assert bwdq(Q=0) == _capi.ERR_ARG
    assert bwdq(dg=FAKE) == _capi.ERR_ARG  # grad_gain without gain
    assert bwdq(gqs=8) == _capi.ERR_ARG  # query blocks of grad_out overlap
    # bf16 sources, one chunk per thread: batched kernels up to S = 9
    srcs = [FAKE + 4096 * i for i in range(10)]
    assert bwdq(sources=srcs) == _capi.ERR_UNSUPPORTED
    assert "attnres_route_bwd once per query" in _capi.lib().attnres_last_error().decode()
    assert bwdq(D=12) == _capi.ERR_UNSUPPORTED


def test_merge_bwd_argument_errors():
    lib = _capi.lib()
    args = [FAKE, 16, 64, _capi.DTYPE_BF16, FAKE, _capi.DTYPE_BF16, FAKE, _capi.DTYPE_BF16, FAKE, 1e-5, FAKE,
            FAKE + 8192, FAKE + 16384, None, FAKE, 1 << 30, FAKE, None]
    a = list(args)
    a[1] = 0
    assert lib.attnres_merge_bwd(*a) == _capi.OK
    for i in (0, 4, 6, 8, 10, 11, 12):  # required pointers
        a = list(args)
        a[i] = None
        assert lib.attnres_merge_bwd(*a) == _capi.ERR_ARG, i
    a = list(args)
    a[2] = 60
    assert lib.attnres_merge_bwd(*a) == _capi.ERR_UNSUPPORTED
    a = list(args)
    a[11] = FAKE + 8
    assert lib.attnres_merge_bwd(*a) == _capi.ERR_ALIGN
    a = list(args)
    a[9] = float("nan")
    assert lib.attnres_merge_bwd(*a) == _capi.ERR_ARG


def test_kernel_name_argument_errors():
    lib = _capi.lib()
    buf = ctypes.create_string_buffer(8)
    assert lib.attnres_route_kernel_name(3, 16, 64, 1, 1, 1, 1, 0, 1, None, 0) == _capi.ERR_ARG
    assert lib.attnres_route_kernel_name(3, 16, 64, 1, 1, 9, 1, 0, 1, buf, 8) == _capi.ERR_ARG  # out dtype
    assert lib.attnres_route_kernel_name(17, 16, 64, 1, 1, 1, 1, 0, 1, buf, 8) == _capi.ERR_ARG
    assert lib.attnres_merge_kernel_name(16, 512, 1, 1, 1, None, 0) == _capi.ERR_ARG
    assert lib.attnres_merge_kernel_name(16, 512, 1, 7, 1, buf, 8) == _capi.ERR_ARG  # param dtype
    assert lib.attnres_merge_kernel_name(-1, 512, 1, 1, 1, buf, 8) == _capi.ERR_ARG  # negative rows
    # no rows: attnres_merge_fwd launches nothing, and the name is empty (no device needed)
    assert lib.attnres_merge_kernel_name(0, 512, 1, 1, 1, buf, 8) == _capi.OK and buf.value == b""
    assert lib.attnres_merge_kernel_name(16, 500, 1, 1, 1, buf, 8) == _capi.ERR_UNSUPPORTED  # not 16-byte chunks


def test_route_step_argument_errors():
    lib = _capi.lib()
    N, D = 16, 64
    blk = N * D * 2  # bytes of one bf16 row block
    com = _capi.pointer_array([FAKE, FAKE + blk])

    def step(committed=com, nc=2, partial=FAKE + 2 * blk, delta=FAKE + 3 * blk, pout=FAKE + 4 * blk, n=N, d=D,
             dt=_capi.DTYPE_BF16, query=FAKE, out=FAKE + 5 * blk):
        return lib.attnres_route_step(committed, nc, partial, delta, pout, n, d, dt, query, None, _capi.DTYPE_BF16,
                                      1e-5, out, None, None, None)

    assert step(n=0) == _capi.OK  # nothing to do: returns before any HIP call
    assert step(partial=None) == _capi.ERR_ARG
    assert step(delta=None) == _capi.ERR_ARG
    assert step(pout=None) == _capi.ERR_ARG
    assert step(nc=-1) == _capi.ERR_ARG
    assert step(committed=None) == _capi.ERR_ARG
    assert step(nc=16) == _capi.ERR_UNSUPPORTED  # 17 sources
    assert step(dt=7) == _capi.ERR_ARG
    # the new partial may not overlap an input: it would be read while written
    assert step(pout=FAKE + 2 * blk) == _capi.ERR_ARG
    assert step(pout=FAKE + 3 * blk + 64) == _capi.ERR_ARG
    assert step(pout=FAKE + blk // 2) == _capi.ERR_ARG
    assert step(pout=FAKE + 4 * blk + 8) == _capi.ERR_ALIGN  # route_launch's alignment check of partial_out
    assert step(query=None) == _capi.ERR_ARG


def test_route_bwd_add_argument_errors():
    lib = _capi.lib()
    N, D, S = 16, 64, 2
    srcs = _capi.pointer_array([FAKE, FAKE + 4096])
    grads = _capi.pointer_array([FAKE + 8192, FAKE + 12288])

    def call(adds, gdt=_capi.DTYPE_BF16, n=N):
        return lib.attnres_route_bwd_add(srcs, S, n, D, D, _capi.DTYPE_BF16, FAKE, None, _capi.DTYPE_BF16, 1e-5,
                                         FAKE, gdt, D, None, grads, adds, D, FAKE, 1 << 20, None, None, None)

    assert call(_capi.pointer_array([FAKE + 8192, None]), n=0) == _capi.OK
    assert call(_capi.pointer_array([FAKE + 8200, None]), n=0) == _capi.ERR_ALIGN
    # an addend needs grad_out in the source dtype (bf16 sources, fp32 dL/dout: no kernel)
    assert call(_capi.pointer_array([FAKE + 8192, None]), gdt=_capi.DTYPE_F32, n=0) == _capi.ERR_UNSUPPORTED
    # without any addend the call is attnres_route_bwd
    assert call(_capi.pointer_array([None, None]), gdt=_capi.DTYPE_F32, n=0) == _capi.OK
    assert call(None, gdt=_capi.DTYPE_F32, n=0) == _capi.OK


def test_route_bwd_defer_argument_errors():
    lib = _capi.lib()
    bf, f32 = _capi.DTYPE_BF16, _capi.DTYPE_F32

    def call(S=3, D=3072, n=0, sdt=bf, gdt=bf, pdt=bf, gp=FAKE + 65536, coef=FAKE + 131072, qfold=FAKE + 196608,
             add=None):
        srcs = _capi.pointer_array([FAKE + 4096 * s for s in range(S)])
        return lib.attnres_route_bwd_defer(srcs, S, n, D, D, sdt, FAKE, None, pdt, 1e-5, FAKE, gdt, D, None, gp, add,
                                           D, coef, qfold, FAKE, 1 << 20, None, None, None)

    # kernels: bf16 everywhere, hidden 512, 1024 or 3072 (2..8 sources) or 4096 (2..9); n = 0 returns
    # before any HIP call
    assert call() == _capi.OK
    assert call(S=8) == _capi.OK and call(S=9, D=4096) == _capi.OK
    assert call(S=8, D=1024) == _capi.OK and call(S=8, D=512) == _capi.OK
    assert call(S=9) == _capi.ERR_UNSUPPORTED and call(S=9, D=1024) == _capi.ERR_UNSUPPORTED
    assert call(S=1) == _capi.ERR_UNSUPPORTED  # no committed source to defer
    assert call(D=2048) == _capi.ERR_UNSUPPORTED
    assert call(sdt=f32) == _capi.ERR_UNSUPPORTED and call(gdt=f32) == _capi.ERR_UNSUPPORTED
    assert call(pdt=f32) == _capi.ERR_UNSUPPORTED
    assert call(S=17) == _capi.ERR_ARG
    assert call(gp=None) == _capi.ERR_ARG and call(coef=None) == _capi.ERR_ARG and call(qfold=None) == _capi.ERR_ARG
    assert call(coef=FAKE + 8) == _capi.ERR_ALIGN and call(add=FAKE + 4) == _capi.ERR_ALIGN
    assert call(add=FAKE + 65536) == _capi.OK  # the addend may be the gradient itself


def test_route_bwd_gather_argument_errors():
    lib = _capi.lib()
    bf = _capi.DTYPE_BF16

    def call(nt=2, D=3072, n=0, dt=bf, gouts=None, coefs=None, lds=None, qfs=None, x=FAKE, out=FAKE + 65536,
             add=None):
        gouts = gouts if gouts is not None else [FAKE + 4096 * j for j in range(nt)]
        coefs = coefs if coefs is not None else [FAKE + 1024 * j for j in range(nt)]
        lds = lds if lds is not None else [8] * nt
        qfs = qfs if qfs is not None else [FAKE] * nt
        return lib.attnres_route_bwd_gather(x, n, D, D, dt, nt, _capi.pointer_array(gouts), D,
                                            _capi.pointer_array(coefs), _capi.int64_array(lds),
                                            _capi.pointer_array(qfs), add, out, D, None)

    assert call() == _capi.OK and call(nt=0) == _capi.OK and call(D=4096, nt=60) == _capi.OK
    assert call(D=1024) == _capi.OK and call(D=512) == _capi.OK
    assert call(D=2048) == _capi.ERR_UNSUPPORTED and call(dt=_capi.DTYPE_F32) == _capi.ERR_UNSUPPORTED
    assert call(nt=-1) == _capi.ERR_ARG and call(x=None) == _capi.ERR_ARG and call(out=None) == _capi.ERR_ARG
    assert call(gouts=[FAKE, None]) == _capi.ERR_ARG
    assert call(lds=[8, 6]) == _capi.ERR_ARG and call(lds=[0, 8]) == _capi.ERR_ARG
    assert call(coefs=[FAKE, FAKE + 4]) == _capi.ERR_ALIGN and call(add=FAKE + 2) == _capi.ERR_ALIGN
    assert call(out=FAKE + 8) == _capi.ERR_ALIGN
