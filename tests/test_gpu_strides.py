"""Row strides through the C ABI (GPU).

A caller binding ``attnres_route_fwd`` / ``attnres_route_bwd`` directly may
pass rows of wider buffers: ``src_ld``, ``out_ld`` and ``out_qstride`` (forward),
``grad_out_ld`` and ``grad_ld`` (backward) in elements.  Each case routes rows
that sit inside a canary-filled buffer and checks the results against the
float64 oracle and that no byte outside the rows was written.  The cases cover
every kernel family the host can pick: the row-per-workgroup kernel (few rows),
the streaming kernel (both its base+stride and pointer-table addressing), the
batched-query kernel (bf16 queries) and the per-query kernel (fp32 queries),
bf16 and fp32; and the training loop's deferred backward and per-block sum.
Tolerances as in test_gpu_parity / test_gpu_backward.
"""

import ctypes

import numpy as np
import pytest
import torch

from kotodama_amd import _capi
from oracle import attnres_oracle as O

pytestmark = pytest.mark.gpu

CANARY = 7.0  # exact in bf16; no routed value here equals it


def np64(t):
    return t.detach().float().cpu().double().numpy()


def bf16_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0**-126)))
    return 2.0 ** (e - 7)


def check_out(out, ref, dtype, label):
    got = np64(out)
    err = np.abs(got - ref)
    if dtype == torch.float32:
        tol = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max()
    else:
        tol = np.maximum(2e-2, bf16_ulp(ref))
    assert (err <= tol).all(), f"{label}: worst err {err.max():.3e}"


def code(dtype):
    return _capi.DTYPE_BF16 if dtype == torch.bfloat16 else _capi.DTYPE_F32


def kernel_name(s, n, d, src, par, out, q, equally_spaced=True):
    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_kernel_name",
                _capi.lib().attnres_route_kernel_name(s, n, d, code(src), code(par), code(out), q, 0,
                                                      int(equally_spaced), buf, 128))
    return buf.value.decode()


# (label, S, n, d, source dtype, query dtype, Q, separate allocations, expected kernel suffix)
FWD_CASES = [
    ("workgroup-bf16", 5, 96, 3072, torch.bfloat16, torch.bfloat16, 1, False, "_q1"),
    ("workgroup-f32", 3, 40, 1024, torch.float32, torch.float32, 1, False, "_q1"),
    ("stream-plain", 4, 4096, 2048, torch.bfloat16, torch.bfloat16, 1, False, "_plain"),
    ("stream-table", 4, 4096, 2048, torch.bfloat16, torch.bfloat16, 1, True, "_table"),
    ("batched-bf16", 6, 64, 1024, torch.bfloat16, torch.bfloat16, 5, False, "_qg"),
    ("per-query-f32q", 3, 64, 1024, torch.bfloat16, torch.float32, 3, False, "_qn"),
]


@pytest.mark.parametrize("label,S,n,d,sdt,qdt,Q,separate,suffix", FWD_CASES, ids=[c[0] for c in FWD_CASES])
def test_route_fwd_row_strides(gpu, label, S, n, d, sdt, qdt, Q, separate, suffix):
    # the kernel-name query takes the spacing of the source pointers, as the launch does
    assert kernel_name(S, n, d, sdt, qdt, sdt, Q, equally_spaced=not separate).endswith(suffix)
    g = torch.Generator(device=gpu).manual_seed(n + d + Q)
    src_ld, out_ld = d + 64, d + 32
    es = 2 if sdt == torch.bfloat16 else 4
    if separate:  # one allocation per source, in an order that is not equally spaced
        bufs = [torch.full((n, src_ld), CANARY, device=gpu, dtype=sdt) for _ in range(S + 2)]
        rows = [bufs[i] for i in (2, 0, 4, 1)][:S]
    else:
        big = torch.full((S, n, src_ld), CANARY, device=gpu, dtype=sdt)
        rows = [big[s] for s in range(S)]
    for s, r in enumerate(rows):
        r[:, :d] = (torch.randn((n, d), generator=g, device=gpu) * (0.5 + s)).to(sdt)
    qs = (torch.randn((Q, d), generator=g, device=gpu) * 0.05).to(qdt)
    qstride = n * out_ld + 64
    obuf = torch.full(((Q - 1) * qstride + n * out_ld,), CANARY, device=gpu, dtype=sdt)
    weights = torch.full((Q, S, n), CANARY, device=gpu)
    lse = torch.full((Q, n), CANARY, device=gpu)
    srcs_before = [r.clone() for r in rows]
    _capi.route_fwd(
        _capi.pointer_array([r.data_ptr() for r in rows]), S, n, d, src_ld, code(sdt), qs.data_ptr(), None, Q,
        code(qdt), 1e-5, obuf.data_ptr(), code(sdt), out_ld, qstride, weights.data_ptr(), lse.data_ptr(), None,
        None, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    ref = O.route(np.stack([np64(r[:, :d]) for r in rows]), np64(qs), 1e-5)
    for q in range(Q):
        view = obuf[q * qstride: q * qstride + n * out_ld].view(n, out_ld)
        check_out(view[:, :d], ref["out"][q], sdt, f"{label} q={q}")
        assert torch.all(view[:, d:] == CANARY), f"{label}: output row padding written"
        if q + 1 < Q:
            assert torch.all(obuf[q * qstride + n * out_ld: (q + 1) * qstride] == CANARY), f"{label}: gap written"
        assert np.abs(np64(weights[q]) - ref["weights"][q]).max() <= 1e-5
        np.testing.assert_allclose(np64(lse[q]), ref["lse"][q], rtol=1e-5, atol=1e-5)
    for a, b in zip(rows, srcs_before):
        assert torch.equal(a, b), f"{label}: a source was modified"


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("S", [3, 6])
def test_route_bwd_row_strides(gpu, sdt, S):
    _route_bwd_strided(gpu, sdt, S, 300, 2048)


@pytest.mark.parametrize("S,n", [(2, 777), (8, 1029)])
def test_route_bwd_row_per_wave_row_strides(gpu, S, n):
    # the row-per-wave backward (bf16, rows of 6 KiB) over padded rows and
    # separate gradient rows: its whole-row loads and stores stay inside each row
    kn = ctypes.create_string_buffer(128)
    prev = _capi.set_kernel_policy(_capi.POLICY_STREAM)
    try:
        _capi.check("attnres_route_bwd_kernel_name", _capi.lib().attnres_route_bwd_kernel_name(
            S, n, 3072, _capi.DTYPE_BF16, _capi.DTYPE_BF16, kn, 128))
        assert kn.value.decode() == f"attnres_route_bwd_stream_c6_s{S}"
        _route_bwd_strided(gpu, torch.bfloat16, S, n, 3072)
    finally:
        _capi.set_kernel_policy(prev)


def _route_bwd_strided(gpu, sdt, S, n, d):
    print(f"route_bwd strided {sdt} S={S} n={n} d={d}", flush=True)
    src_ld, gout_ld, grad_ld = d + 64, d + 128, d + 32
    g = torch.Generator(device=gpu).manual_seed(S * 7 + (sdt == torch.float32))
    big = torch.full((S, n, src_ld), CANARY, device=gpu, dtype=sdt)
    for s in range(S):
        big[s, :, :d] = (torch.randn((n, d), generator=g, device=gpu) * (0.5 + s)).to(sdt)
    qdt = sdt
    q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(qdt)
    gbuf = torch.full((n, gout_ld), CANARY, device=gpu, dtype=sdt)
    gbuf[:, :d] = torch.randn((n, d), generator=g, device=gpu).to(sdt)
    glse = torch.randn(n, generator=g, device=gpu) * 0.1
    dbig = torch.full((S, n, grad_ld), CANARY, device=gpu, dtype=sdt)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    dq = torch.empty(d, device=gpu, dtype=qdt)
    _capi.route_bwd(
        _capi.pointer_array([big[s].data_ptr() for s in range(S)]), S, n, d, src_ld, code(sdt), q.data_ptr(), None,
        code(qdt), 1e-5, gbuf.data_ptr(), code(sdt), gout_ld, glse.data_ptr(),
        _capi.pointer_array([dbig[s].data_ptr() for s in range(S)]), grad_ld, ws.data_ptr(), ws.numel() * 4,
        dq.data_ptr(), None, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    ref = O.route_backward(np64(big[:, :, :d]), np64(q), 1e-5, np64(gbuf[:, :d]), np64(glse))
    got = np64(dbig[:, :, :d])
    scale = np.abs(ref["dx"]).max()
    if sdt == torch.float32:
        tol = 1e-4 * np.abs(ref["dx"]) + 1e-5 * scale
    else:
        tol = bf16_ulp(ref["dx"]) + 1e-3 * scale
    assert (np.abs(got - ref["dx"]) <= tol).all(), f"dx worst err {np.abs(got - ref['dx']).max():.3e}"
    assert torch.all(dbig[:, :, d:] == CANARY), "gradient row padding written"
    dqr = ref["dqw"]
    tq = 1e-4 * np.abs(dqr) + 1e-5 * np.abs(dqr).max() if qdt == torch.float32 else \
        bf16_ulp(dqr) + 1e-3 * np.abs(dqr).max()
    assert (np.abs(np64(dq) - dqr) <= tq).all(), "query gradient"


@pytest.mark.parametrize("S,n,d", [(3, 777, 3072), (9, 515, 4096)])
def test_route_bwd_defer_and_gather_row_strides(gpu, S, n, d):
    # attnres_route_bwd_defer over padded source, dL/dout and gradient rows, with
    # dL/dlse; then attnres_route_bwd_gather of source 0's gradient from that
    # call's records over a padded block row and padded output rows: every
    # result against the oracle, no byte of the padding written
    print(f"route_bwd_defer + gather strided S={S} n={n} d={d}", flush=True)
    bf = torch.bfloat16
    src_ld, gout_ld, grad_ld = d + 64, d + 128, d + 32
    g = torch.Generator(device=gpu).manual_seed(S * 13 + n)
    big = torch.full((S, n, src_ld), CANARY, device=gpu, dtype=bf)
    for s in range(S):
        big[s, :, :d] = (torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.3 * s)).to(bf)
    q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(bf)
    gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(bf)
    gbuf = torch.full((n, gout_ld), CANARY, device=gpu, dtype=bf)
    gbuf[:, :d] = torch.randn((n, d), generator=g, device=gpu).to(bf)
    glse = torch.randn(n, generator=g, device=gpu) * 0.1
    gpart = torch.full((n, grad_ld), CANARY, device=gpu, dtype=bf)
    add = torch.full((n, grad_ld), CANARY, device=gpu, dtype=bf)
    add[:, :d] = (torch.randn((n, d), generator=g, device=gpu) * 0.01).to(bf)
    coef = torch.full((n, S - 1, 4), float("nan"), device=gpu)
    qfold = torch.empty(d, device=gpu, dtype=bf)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    dq = torch.empty(d, device=gpu, dtype=bf)
    st = torch.cuda.current_stream(gpu).cuda_stream
    rc = _capi.route_bwd_defer(
        _capi.pointer_array([big[s].data_ptr() for s in range(S)]), S, n, d, src_ld, _capi.DTYPE_BF16, q.data_ptr(),
        gain.data_ptr(), _capi.DTYPE_BF16, 1e-5, gbuf.data_ptr(), _capi.DTYPE_BF16, gout_ld, glse.data_ptr(),
        gpart.data_ptr(), add.data_ptr(), grad_ld, coef.data_ptr(), qfold.data_ptr(), ws.data_ptr(), ws.numel() * 4,
        dq.data_ptr(), None, st)
    _capi.check("attnres_route_bwd_defer", rc)
    torch.cuda.synchronize()
    qw = O.fold_query(np64(q), np64(gain), "bf16")
    ref = O.route_backward(np64(big[:, :, :d]), qw, 1e-5, np64(gbuf[:, :d]), np64(glse))
    want = ref["dx"][S - 1] + np64(add[:, :d])
    err = np.abs(np64(gpart[:, :d]) - want)
    assert (err <= bf16_ulp(want) + 1e-3 * np.abs(want).max()).all(), f"partial gradient worst err {err.max():.3e}"
    assert torch.all(gpart[:, d:] == CANARY), "partial gradient row padding written"
    dqr = ref["dqw"] * np64(gain)
    assert (np.abs(np64(dq) - dqr) <= bf16_ulp(dqr) + 1e-3 * np.abs(dqr).max()).all(), "query gradient"
    assert not torch.isnan(coef).any(), "a record was not written"
    # gather source 0's gradient from this call (one term) onto padded output rows
    out = torch.full((n, grad_ld), CANARY, device=gpu, dtype=bf)
    _capi.route_bwd_gather(
        big[0].data_ptr(), n, d, src_ld, _capi.DTYPE_BF16, 1, _capi.pointer_array([gbuf.data_ptr()]), gout_ld,
        _capi.pointer_array([coef.data_ptr()]), _capi.int64_array([4 * (S - 1)]),
        _capi.pointer_array([qfold.data_ptr()]), add.data_ptr(), out.data_ptr(), grad_ld, st)
    torch.cuda.synchronize()
    want0 = ref["dx"][0] + np64(add[:, :d])
    err = np.abs(np64(out[:, :d]) - want0)
    assert (err <= bf16_ulp(want0) + 1e-3 * np.abs(want0).max()).all(), f"gathered gradient worst err {err.max():.3e}"
    assert torch.all(out[:, d:] == CANARY), "gathered gradient row padding written"


@pytest.mark.parametrize("nb,P,n,d", [(3, 5, 700, 3072), (6, 4, 513, 4096), (8, 3, 301, 4096)])
def test_route_bwd_gather_seg_row_strides_in_place(gpu, nb, P, n, d):
    # P calls of attnres_route_bwd_defer over nb padded block rows and a
    # partial of their own, then one attnres_route_bwd_gather_seg with padded
    # dL/dout, block and output rows: blocks 0 .. nb-2 continue their running
    # sums in place (part_in = part_out, csum_in = csum_out), the last block
    # takes its addend in place (addend = its output).  The carried sums against
    # float64 sums of the records, the last block against the oracle; no byte
    # of the padding written
    print(f"route_bwd_gather_seg strided in place nb={nb} P={P} n={n} d={d}", flush=True)
    bf = torch.bfloat16
    src_ld, gout_ld, out_ld = d + 64, d + 128, d + 32
    g = torch.Generator(device=gpu).manual_seed(nb * 31 + P)
    big = torch.full((nb, n, src_ld), CANARY, device=gpu, dtype=bf)
    for j in range(nb):
        big[j, :, :d] = (torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.2 * j)).to(bf)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    gouts, coefs, qfolds, dx = [], [], [], []
    for p in range(P):
        own = torch.full((n, src_ld), CANARY, device=gpu, dtype=bf)
        own[:, :d] = torch.randn((n, d), generator=g, device=gpu).to(bf)
        q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(bf)
        gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(bf)
        gbuf = torch.full((n, gout_ld), CANARY, device=gpu, dtype=bf)
        gbuf[:, :d] = torch.randn((n, d), generator=g, device=gpu).to(bf)
        gpart = torch.empty((n, d), device=gpu, dtype=bf)
        coef = torch.full((n, nb, 4), float("nan"), device=gpu)
        qfold = torch.empty(d, device=gpu, dtype=bf)
        dq = torch.empty(d, device=gpu, dtype=bf)
        srcs = [big[j].data_ptr() for j in range(nb)] + [own.data_ptr()]
        rc = _capi.route_bwd_defer(
            _capi.pointer_array(srcs), nb + 1, n, d, src_ld, _capi.DTYPE_BF16, q.data_ptr(), gain.data_ptr(),
            _capi.DTYPE_BF16, 1e-5, gbuf.data_ptr(), _capi.DTYPE_BF16, gout_ld, None, gpart.data_ptr(), None, d,
            coef.data_ptr(), qfold.data_ptr(), ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), None, st)
        _capi.check("attnres_route_bwd_defer", rc)
        torch.cuda.synchronize()
        srcs64 = np.concatenate([np64(big[:, :, :d]), np64(own[:, :d])[None]])
        dx.append(O.route_backward(srcs64, O.fold_query(np64(q), np64(gain), "bf16"), 1e-5, np64(gbuf[:, :d]),
                                   None)["dx"])
        gouts.append(gbuf), coefs.append(coef), qfolds.append(qfold)
    # running sums of blocks 0 .. nb-2 from a later segment, updated in place
    part = torch.full((nb, n, out_ld), CANARY, device=gpu, dtype=bf)
    for j in range(nb - 1):
        part[j, :, :d] = (torch.randn((n, d), generator=g, device=gpu) * 0.1).to(bf)
    csum = torch.randn((nb, n), generator=g, device=gpu) * 0.01
    part[nb - 1, :, :d] = (torch.randn((n, d), generator=g, device=gpu) * 0.01).to(bf)  # the addend
    prev = np64(part[:, :, :d])
    prev_cs = np64(csum)
    rows = [part[j].data_ptr() for j in range(nb)]
    cs = [csum[j].data_ptr() for j in range(nb - 1)] + [None]
    _capi.route_bwd_gather_seg(
        nb, n, d, _capi.DTYPE_BF16, P, _capi.pointer_array([t.data_ptr() for t in gouts]), gout_ld,
        _capi.pointer_array([c.data_ptr() for c in coefs]), _capi.int64_array([4 * nb] * P),
        _capi.pointer_array([q.data_ptr() for q in qfolds]), _capi.pointer_array(rows[:-1] + [None]),
        _capi.pointer_array(cs), _capi.pointer_array(rows), _capi.pointer_array(cs), big[nb - 1].data_ptr(), src_ld,
        rows[-1], out_ld, st)
    torch.cuda.synchronize()
    recs = [(np64(c), np64(t[:, :d]), np64(q)) for c, t, q in zip(coefs, gouts, qfolds)]
    for j in range(nb - 1):
        want = prev[j] + sum(c[:, j, 0:1] * G + c[:, j, 1:2] * q[None, :] for c, G, q in recs)
        err = np.abs(np64(part[j, :, :d]) - want)
        assert (err <= bf16_ulp(want) + 1e-3 * np.abs(want).max()).all(), f"block {j} running sum worst err {err.max():.3e}"
        wc = prev_cs[j] + sum(c[:, j, 2] for c, _, _ in recs)
        assert (np.abs(np64(csum[j]) - wc) <= 1e-5 * np.abs(wc) + 1e-6 * np.abs(wc).max()).all(), f"block {j} csum"
    want = sum(x[nb - 1] for x in dx) + prev[nb - 1]
    err = np.abs(np64(part[nb - 1, :, :d]) - want)
    assert (err <= bf16_ulp(want) + 1e-3 * np.abs(want).max()).all(), f"last block worst err {err.max():.3e}"
    assert torch.all(part[:, :, d:] == CANARY), "output row padding written"
    assert torch.all(big[:, :, d:] == CANARY), "block row padding written"
