"""attnres_route_bwd_noalloc (GPU): the routing backward with its
query-gradient partials in the library's fixed device scratch array instead
of a caller workspace.

Two calls in a row through the C ABI — the second on a smaller input, so it
runs on whatever the first left in the shared array — each compared with
attnres_route_bwd on a torch-allocated workspace (bit-identical: same kernels,
same grid, same fixed-order reduction) and with the float64 oracle at the
backward bars of test_gpu_backward.  A repeat of the second call must leave
the device's free memory unchanged (the entry point allocates nothing).
"""

import numpy as np
import pytest
import torch

from kotodama_amd import _capi
from oracle import attnres_oracle as O

pytestmark = pytest.mark.gpu


def np64(t):
    return t.detach().float().cpu().double().numpy()


def bf16_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0**-126)))
    return 2.0 ** (e - 7)


def code(dtype):
    return _capi.DTYPE_BF16 if dtype == torch.bfloat16 else _capi.DTYPE_F32


def make_case(gpu, S, n, d, dt, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    src = torch.stack([torch.randn((n, d), generator=g, device=gpu) * (0.5 + s) for s in range(S)]).to(dt)
    q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(dt)
    gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(dt)
    gout = torch.randn((n, d), generator=g, device=gpu).to(dt)
    glse = torch.randn(n, generator=g, device=gpu) * 0.1
    return src, q, gain, gout, glse


def run(gpu, src, q, gain, gout, glse, noalloc):
    S, n, d = src.shape
    dt = src.dtype
    dsrc = torch.full_like(src, 3.0)
    dq = torch.full((d,), 3.0, device=gpu, dtype=dt)
    dg = torch.full((d,), 3.0, device=gpu, dtype=dt)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    srcs = _capi.pointer_array([src[s].data_ptr() for s in range(S)])
    dsrcs = _capi.pointer_array([dsrc[s].data_ptr() for s in range(S)])
    head = (srcs, S, n, d, d, code(dt), q.data_ptr(), gain.data_ptr(), code(dt), 1e-5, gout.data_ptr(), code(dt), d,
            glse.data_ptr(), dsrcs, d)
    if noalloc:
        _capi.route_bwd_noalloc(*head, dq.data_ptr(), dg.data_ptr(), stream)
    else:
        ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
        _capi.route_bwd(*head, ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), dg.data_ptr(), stream)
    torch.cuda.synchronize()
    return dsrc, dq, dg


def check_oracle(src, q, gain, gout, glse, dsrc, dq, dg):
    dt = src.dtype
    pdt = "bf16" if dt == torch.bfloat16 else "f32"
    qw = O.fold_query(np64(q), np64(gain), pdt)
    ref = O.route_backward(np64(src), qw, 1e-5, np64(gout), np64(glse))
    pairs = ((dsrc, ref["dx"], "dx"), (dq, ref["dqw"] * np64(gain), "dquery"), (dg, ref["dqw"] * np64(q), "dgain"))
    for got, want, name in pairs:
        scale = np.abs(want).max()
        if dt == torch.float32:
            tol = 1e-4 * np.abs(want) + 1e-5 * scale
        else:
            tol = bf16_ulp(want) + 1e-3 * scale
        err = np.abs(np64(got) - want)
        assert (err <= tol).all(), f"{name}: worst err {err.max():.3e}"


# the second case is smaller in every dimension than the first
CASES = [(6, 4096, 3072, torch.bfloat16, 11), (3, 200, 1024, torch.float32, 12)]


def test_noalloc_matches_workspace_entry(gpu):
    assert _capi.lib().attnres_init() == _capi.OK
    for S, n, d, dt, seed in CASES:
        print(f"noalloc case S={S} n={n} d={d} {dt}", flush=True)
        case = make_case(gpu, S, n, d, dt, seed)
        want = run(gpu, *case, noalloc=False)
        got = run(gpu, *case, noalloc=True)
        for a, b, name in zip(got, want, ("dsources", "dquery", "dgain")):
            assert torch.equal(a, b), f"S={S} n={n} d={d}: {name} differs from attnres_route_bwd"
        check_oracle(*case, *got)
    # a repeat of the last (smaller) call allocates nothing
    free0, _ = torch.cuda.mem_get_info(gpu)
    again = run(gpu, *case, noalloc=True)
    free1, _ = torch.cuda.mem_get_info(gpu)
    assert free0 == free1, f"device free memory changed by {free0 - free1} bytes"
    for a, b in zip(again, want):
        assert torch.equal(a, b)


def test_noalloc_rejects_bad_arguments(gpu):
    lib = _capi.lib()
    args = (_capi.pointer_array([0]), 1, 16, 64, 64, _capi.DTYPE_BF16, None, None, _capi.DTYPE_BF16, 1e-5, None,
            _capi.DTYPE_BF16, 64, None, _capi.pointer_array([0]), 64, None, None, None)
    assert lib.attnres_route_bwd_noalloc(*args) == _capi.ERR_ARG  # NULL query / grad_out / sources
    bad = list(args)
    bad[3] = 0
    assert lib.attnres_route_bwd_noalloc(*bad) == _capi.ERR_ARG  # hidden = 0


def _bwd_name(S, n, d, dt):
    import ctypes

    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_bwd_kernel_name",
                _capi.lib().attnres_route_bwd_kernel_name(S, n, d, code(dt), code(dt), buf, 128))
    return buf.value.decode()


# the row-per-wave backward (one 4-wave workgroup per CU: a different grid, so a
# different share of the scratch array), at 6 KiB rows with the source rows in
# registers and at 8 KiB rows with the first S - 6 rows kept in LDS
STREAM_CASES = [(8, 4096, 3072, 21, "attnres_route_bwd_stream_c6_s8"), (9, 2048, 4096, 22, "attnres_route_bwd_stream_c8_s9")]


def test_noalloc_row_per_wave_backward(gpu):
    assert _capi.lib().attnres_init() == _capi.OK
    prev = _capi.set_kernel_policy(_capi.POLICY_STREAM)
    try:
        for S, n, d, seed, kernel in STREAM_CASES:
            print(f"noalloc row-per-wave S={S} n={n} d={d}", flush=True)
            assert _bwd_name(S, n, d, torch.bfloat16) == kernel
            case = make_case(gpu, S, n, d, torch.bfloat16, seed)
            want = run(gpu, *case, noalloc=False)
            got = run(gpu, *case, noalloc=True)
            for a, b, name in zip(got, want, ("dsources", "dquery", "dgain")):
                assert torch.equal(a, b), f"S={S} d={d}: {name} differs from attnres_route_bwd"
            check_oracle(*case, *got)
    finally:
        _capi.set_kernel_policy(prev)


def test_noalloc_under_graph_capture(gpu):
    # after attnres_init(), one noalloc call captured in a HIP graph: every
    # replay (with eager work between them, including another noalloc call of a
    # different shape that overwrites the shared scratch array) equals the
    # workspace entry point's result
    assert _capi.lib().attnres_init() == _capi.OK
    S, n, d = 4, 2048, 3072
    case = make_case(gpu, S, n, d, torch.bfloat16, 31)
    want = run(gpu, *case, noalloc=False)
    src, q, gain, gout, glse = case
    dsrc = torch.empty_like(src)
    dq = torch.empty((d,), device=gpu, dtype=src.dtype)
    dg = torch.empty((d,), device=gpu, dtype=src.dtype)
    srcs = _capi.pointer_array([src[s].data_ptr() for s in range(S)])
    dsrcs = _capi.pointer_array([dsrc[s].data_ptr() for s in range(S)])

    def call(stream):
        return _capi.lib().attnres_route_bwd_noalloc(
            srcs, S, n, d, d, code(src.dtype), q.data_ptr(), gain.data_ptr(), code(src.dtype), 1e-5,
            gout.data_ptr(), code(src.dtype), d, glse.data_ptr(), dsrcs, d, dq.data_ptr(), dg.data_ptr(), stream)

    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):  # warm-up on the capture's kind of stream: kernel lookups happen here
        assert call(side.cuda_stream) == _capi.OK
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call(torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == _capi.OK
    other = make_case(gpu, 2, 300, 1024, torch.float32, 32)
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        for t in (dsrc, dq, dg):
            t.fill_(3.0)
        run(gpu, *other, noalloc=True)  # leaves other values in the scratch array
        graph.replay()
        torch.cuda.synchronize()
        for a, b, name in zip((dsrc, dq, dg), want, ("dsources", "dquery", "dgain")):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from attnres_route_bwd"
