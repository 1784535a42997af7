"""Gradient sums inside the routing backward, and the fused training step (GPU).

``attnres_route_bwd_add`` writes grad_sources[s] = dL/dsource_s + grad_addend[s]
(fp32 sum, one rounding) for the sources given an addend, in place when the
addend is the gradient itself.  Checked through the C ABI on both kernel
families (row per wave, row per workgroup), bf16 and fp32, with a mix of
sources with and without addends:
* against the float64 oracle's gradient plus the addend, at the backward bars
  of test_gpu_backward (bf16: 1 ulp + 1e-3 max|ref|, >= 95% correctly rounded;
  fp32: 1e-4 |ref| + 1e-5 max|ref|);
* sources without an addend bit-identical to attnres_route_bwd (zeros compare
  equal to negative zeros), and the query / gain gradients bit-identical too;
* in place (addend == gradient) bit-identical to a separate addend buffer.
``attnres_route_step`` (partial + delta into a new buffer, then routing over
the committed blocks and it): the new partial exactly the rounded sum, the
inputs untouched, the routed rows at the forward bars against the oracle and
bit-identical to the arena's fused step on the same values.  Then the
training loop that uses both (forward_attn_res under autograd) against the
same loop with them switched off (route_list calls and torch adds; autograd
sums the gradients), fp32 and bf16.
"""

import copy
import ctypes

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops
from oracle import attnres_oracle as O

from ._tiny_model import TinyModel
from .test_gpu_backward import check_grad, np64

pytestmark = pytest.mark.gpu


def code(dt):
    return _capi.DTYPE_BF16 if dt == torch.bfloat16 else _capi.DTYPE_F32


def _bwd_name(S, n, d, dt):
    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_bwd_kernel_name",
                _capi.lib().attnres_route_bwd_kernel_name(S, n, d, code(dt), code(dt), buf, 128))
    return buf.value.decode()


def _case(gpu, S, n, d, dt, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    src = torch.stack([torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.5 * s) for s in range(S)]).to(dt)
    q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(dt)
    gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(dt)
    gout = torch.randn((n, d), generator=g, device=gpu).to(dt)
    addend = (torch.randn((S, n, d), generator=g, device=gpu) * 0.01).to(dt)
    return src, q, gain, gout, addend


def _call(gpu, src, q, gain, gout, grads, adds):
    S, n, d = src.shape
    dt = src.dtype
    dq = torch.empty(d, device=gpu, dtype=dt)
    dg = torch.empty(d, device=gpu, dtype=dt)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    head = (_capi.pointer_array([src[s].data_ptr() for s in range(S)]), S, n, d, d, code(dt), q.data_ptr(),
            gain.data_ptr(), code(dt), 1e-5, gout.data_ptr(), code(dt), d, None,
            _capi.pointer_array([grads[s].data_ptr() for s in range(S)]))
    tail = (d, ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), dg.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    if adds is None:
        _capi.route_bwd(*head, *tail)
    else:
        _capi.route_bwd_add(*head, _capi.pointer_array([a.data_ptr() if a is not None else None for a in adds]),
                            *tail)
    torch.cuda.synchronize()
    return dq, dg


# (S, rows, hidden, dtype, policy, kernel prefix)
CASES = [
    (1, 2048, 3072, torch.bfloat16, _capi.POLICY_STREAM, "attnres_route_bwd_stream_c6_s1"),
    (5, 2048, 3072, torch.bfloat16, _capi.POLICY_STREAM, "attnres_route_bwd_stream_c6_s5"),
    (8, 4096, 3072, torch.bfloat16, _capi.POLICY_STREAM, "attnres_route_bwd_stream_c6_s8"),
    (9, 1024, 4096, torch.bfloat16, _capi.POLICY_STREAM, "attnres_route_bwd_stream_c8_s9"),
    (3, 700, 3072, torch.bfloat16, _capi.POLICY_WORKGROUP, "attnres_route_bwd_bf_gbf_s3_v"),
    (8, 64, 8184, torch.bfloat16, _capi.POLICY_WORKGROUP, "attnres_route_bwd_bf_gbf_s8_v2"),
    (9, 600, 4096, torch.bfloat16, _capi.POLICY_WORKGROUP, "attnres_route_bwd_bf_gbf_s9_v1"),
    (12, 300, 1024, torch.bfloat16, _capi.POLICY_WORKGROUP, "attnres_route_bwd_bf_gbf_s12_v"),
    (4, 500, 2048, torch.float32, _capi.POLICY_AUTO, "attnres_route_bwd_f32_gf32_s4_v"),
    (9, 300, 1024, torch.float32, _capi.POLICY_AUTO, "attnres_route_bwd_f32_gf32_s9_v"),
]


@pytest.mark.parametrize("S,n,d,dt,policy,kernel", CASES, ids=[c[5].split("bwd_")[1] for c in CASES])
def test_route_bwd_add_matches_oracle_and_plain_backward(gpu, S, n, d, dt, policy, kernel):
    print(f"route_bwd_add S={S} n={n} d={d} {dt}", flush=True)
    prev = _capi.set_kernel_policy(policy)
    try:
        assert _bwd_name(S, n, d, dt).startswith(kernel)
        src, q, gain, gout, addend = _case(gpu, S, n, d, dt, 100 + S)
        # plain backward
        plain = torch.full_like(src, 3.0)
        dq0, dg0 = _call(gpu, src, q, gain, gout, plain, None)
        # every other source with a separate addend buffer
        has = [s % 2 == 0 for s in range(S)]
        sep = torch.full_like(src, 3.0)
        dq1, dg1 = _call(gpu, src, q, gain, gout, sep, [addend[s] if has[s] else None for s in range(S)])
        # the same in place: the addend is the gradient buffer itself
        inpl = torch.full_like(src, 3.0)
        for s in range(S):
            if has[s]:
                inpl[s].copy_(addend[s])
        dq2, dg2 = _call(gpu, src, q, gain, gout, inpl, [inpl[s] if has[s] else None for s in range(S)])
    finally:
        _capi.set_kernel_policy(prev)
    assert torch.equal(sep, inpl), "in-place accumulation differs from a separate addend"
    for a, b, name in ((dq0, dq1, "dquery"), (dg0, dg1, "dgain"), (dq0, dq2, "dquery in place")):
        assert torch.equal(a, b), f"{name} differs from attnres_route_bwd"
    for s in range(S):
        if not has[s]:
            assert torch.equal(sep[s], plain[s]), f"source {s} without addend differs from attnres_route_bwd"
    ref = O.route_backward(np64(src), O.fold_query(np64(q), np64(gain), "bf16" if dt == torch.bfloat16 else "f32"),
                           1e-5, np64(gout), None)
    want = ref["dx"] + np.stack([np64(addend[s]) if has[s] else np.zeros((n, d)) for s in range(S)])
    check_grad(sep, want, dt, "dsources + addend")


def test_route_bwd_add_rejects_mixed_dtypes(gpu):
    S, n, d = 2, 64, 512
    src, q, gain, gout, addend = _case(gpu, S, n, d, torch.bfloat16, 7)
    gout32 = gout.float()
    grads = torch.empty_like(src)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    rc = _capi.lib().attnres_route_bwd_add(
        _capi.pointer_array([src[0].data_ptr(), src[1].data_ptr()]), S, n, d, d, _capi.DTYPE_BF16, q.data_ptr(),
        gain.data_ptr(), _capi.DTYPE_BF16, 1e-5, gout32.data_ptr(), _capi.DTYPE_F32, d, None,
        _capi.pointer_array([grads[0].data_ptr(), grads[1].data_ptr()]),
        _capi.pointer_array([addend[0].data_ptr(), None]), d, ws.data_ptr(), ws.numel() * 4, None, None, None)
    assert rc == _capi.ERR_UNSUPPORTED
    # without any addend the call is attnres_route_bwd, which takes fp32 output gradients
    rc = _capi.lib().attnres_route_bwd_add(
        _capi.pointer_array([src[0].data_ptr(), src[1].data_ptr()]), S, n, d, d, _capi.DTYPE_BF16, q.data_ptr(),
        gain.data_ptr(), _capi.DTYPE_BF16, 1e-5, gout32.data_ptr(), _capi.DTYPE_F32, d, None,
        _capi.pointer_array([grads[0].data_ptr(), grads[1].data_ptr()]), _capi.pointer_array([None, None]), d,
        ws.data_ptr(), ws.numel() * 4, None, None, None)
    assert rc == _capi.OK
    torch.cuda.synchronize()


# (dtype, width, kernel policy): the row-per-workgroup kernels, and under POLICY_STREAM
# the row-per-wave ones (the `_fusedtable` forward and `_stream_c6_*_add` backward)
LOOP_CASES = [(torch.float32, 1024, _capi.POLICY_AUTO), (torch.bfloat16, 1024, _capi.POLICY_AUTO),
              (torch.bfloat16, 3072, _capi.POLICY_STREAM)]


@pytest.mark.parametrize("dtype,d,policy", LOOP_CASES, ids=["f32", "bf16", "bf16-row-per-wave"])
def test_training_loop_accumulating_equals_autograd_sums(gpu, dtype, d, policy, monkeypatch):
    # forward_attn_res under autograd: the blocks' gradients summed in the
    # backward kernels, against the same loop with that switched off (route_list
    # calls; autograd adds each use's gradient): every gradient.  fp32: to 1e-5
    # of each tensor's largest magnitude (the sums differ only in rounding);
    # bf16: autograd rounds each use's gradient and then each partial sum, the
    # kernel rounds each partial sum once, over up to 16 uses of a block, and
    # the differences travel upstream through the bf16 sublayers: within 4 bf16
    # ulps (2^-5) of each tensor's largest magnitude
    model = TinyModel(d=d, num_layers=8, boundaries=(0, 2, 4, 6), seed=61, elementwise=True).to(gpu).to(dtype)
    g = torch.Generator(device=gpu).manual_seed(62)
    embed = torch.randn((2, 64, d), generator=g, device=gpu).to(dtype)
    G = torch.randn((2, 64, d), generator=g, device=gpu).to(dtype)

    def run(m):
        e = embed.clone().requires_grad_(True)
        prev = _capi.set_kernel_policy(policy)
        try:
            (kotodama_amd.forward_attn_res(m, e).float() * G.float()).sum().backward()
            torch.cuda.synchronize()
        finally:
            _capi.set_kernel_policy(prev)
        out = {n: p.grad.float() for n, p in m.named_parameters()}
        out["embed"] = e.grad.float()
        return out

    calls = []
    real = ops.route_point

    def counting(*a, **k):
        calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(ops, "route_point", counting)
    m1 = copy.deepcopy(model)
    got = run(m1)
    assert len(calls) == 17  # every routing point took the accumulating path
    monkeypatch.setattr(ops, "accumulating_path_ok", lambda *t: False)
    want = run(copy.deepcopy(model))
    worst = 0.0
    for k, w in want.items():
        scale = w.abs().max().item()
        err = (got[k] - w).abs().max().item()
        tol = (1e-5 if dtype == torch.float32 else 2.0**-5) * scale + 1e-30
        worst = max(worst, err / max(scale, 1e-30))
        assert err <= tol, f"{k}: err {err:.3e}, max|grad| {scale:.3e}"
    print(f"accumulating vs autograd sums ({dtype}): worst err {worst:.2e} of max|grad|", flush=True)


# (committed blocks, rows, hidden, dtype, policy, kernel suffix)
STEP_CASES = [
    (0, 700, 3072, torch.bfloat16, _capi.POLICY_AUTO, "_s1_v2_q1"),
    (2, 4096, 3072, torch.bfloat16, _capi.POLICY_STREAM, "_c6_fusedtable"),
    (7, 4096, 3072, torch.bfloat16, _capi.POLICY_STREAM, "_c6_fusedtable"),
    (8, 2048, 4096, torch.bfloat16, _capi.POLICY_STREAM, "_c8_fusedtable"),
    (4, 500, 2048, torch.bfloat16, _capi.POLICY_WORKGROUP, "_s5_v1_q1"),
    (3, 300, 1024, torch.float32, _capi.POLICY_AUTO, "_s4_v1_q1"),
    (5, 300, 1024, torch.float32, _capi.POLICY_STREAM, "_c4_fusedtable"),
]


@pytest.mark.parametrize("nc,n,d,dt,policy,suffix", STEP_CASES, ids=[f"c{c[0]}-{c[5][1:]}" for c in STEP_CASES])
def test_route_step_matches_oracle_and_arena_step(gpu, nc, n, d, dt, policy, suffix):
    from .test_gpu_parity import check_bf16, check_f32

    print(f"route_step committed={nc} n={n} d={d} {dt}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(200 + nc)
    arena = torch.stack([torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.3 * s) for s in range(nc + 1)]).to(dt)
    delta = torch.randn((n, d), generator=g, device=gpu).to(dt)
    q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(dt)
    gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(dt)
    committed = [arena[s].clone() for s in range(nc)]  # separate allocations (not equally spaced)
    partial = arena[nc].clone()
    before = [t.clone() for t in (*committed, partial, delta)]
    prev = _capi.set_kernel_policy(policy)
    try:
        buf = ctypes.create_string_buffer(128)
        _capi.check("attnres_route_kernel_name", _capi.lib().attnres_route_kernel_name(
            nc + 1, n, d, code(dt), code(dt), code(dt), 1, 1, 0, buf, 128))
        assert buf.value.decode().endswith(suffix), buf.value.decode()
        out, new_partial = ops._route_rows_step(committed, partial, delta, q, gain, 1e-5, dt)
        # the arena's fused step on the same values (updates its partial slot in place)
        ref_arena = arena.clone()
        out2, _, _ = ops.block_step(ref_arena, nc, False, delta, q, gain, 1e-5, False)
        torch.cuda.synchronize()
    finally:
        _capi.set_kernel_policy(prev)
    for a, b in zip(before, (*committed, partial, delta)):
        assert torch.equal(a, b), "an input was modified"
    assert torch.equal(new_partial, (partial.float() + delta.float()).to(dt)), "partial + delta not rounded once"
    assert torch.equal(new_partial, ref_arena[nc]) and torch.equal(out, out2.reshape(out.shape))
    pd = "bf16" if dt == torch.bfloat16 else "f32"
    x = np.stack([np64(t) for t in (*committed, new_partial)])
    ref = O.route(x, O.fold_query(np64(q), np64(gain), pd), 1e-5)["out"][0]
    if dt == torch.bfloat16:
        check_bf16(out, ref, "route_step")
    else:
        check_f32(out, ref, "route_step")


def test_route_step_rejects_overlapping_output(gpu):
    n, d = 64, 512
    t = torch.randn((3, n, d), device=gpu).to(torch.bfloat16)
    q = torch.zeros(d, device=gpu, dtype=torch.bfloat16)
    out = torch.empty((n, d), device=gpu, dtype=torch.bfloat16)
    lib = _capi.lib()
    args = (_capi.pointer_array([t[0].data_ptr()]), 1, t[1].data_ptr(), t[2].data_ptr())
    tail = (n, d, _capi.DTYPE_BF16, q.data_ptr(), None, _capi.DTYPE_BF16, 1e-5, out.data_ptr(), None, None, None)
    assert lib.attnres_route_step(*args, t[1].data_ptr(), *tail) == _capi.ERR_ARG  # over the partial
    assert lib.attnres_route_step(*args, t[0].data_ptr(), *tail) == _capi.ERR_ARG  # over a committed block
    assert lib.attnres_route_step(*args, None, *tail) == _capi.ERR_ARG
