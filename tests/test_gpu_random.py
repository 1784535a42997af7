"""Seeded randomized parity sweep (GPU) over the routing entry points.

Each case draws its shape and options from a fixed seed: source count,
width (any multiple of the 16-byte chunk up to the largest supported row),
row count, source and parameter dtypes, gain or none, a flat or a peaky
softmax (query scale), and the kernel policy (row-per-wave or
row-per-workgroup).  It runs the drop-in forward and backward through
torch.autograd and checks outputs and gradients against the float64 oracle
at the bars of the other parity tests (check_bf16 / check_f32 for outputs,
check_grad for gradients).  Row counts are capped so that the float64 oracle
handles at most ~2M source elements per case.
"""

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops
from oracle import attnres_oracle as O

from .test_gpu_backward import Norm, check_grad, np64
from .test_gpu_parity import check_bf16, check_f32

pytestmark = pytest.mark.gpu

MAX_ELEMS = 2_000_000


def _policy(rng):
    return [_capi.POLICY_AUTO, _capi.POLICY_STREAM, _capi.POLICY_WORKGROUP][int(rng.integers(3))]


def _rows(rng, per_row):
    return int(max(1, min(int(rng.integers(1, 3000)), MAX_ELEMS // per_row)))


def _with_policy(pol, fn):
    prev = _capi.set_kernel_policy(pol)
    try:
        return fn()
    finally:
        _capi.set_kernel_policy(prev)


@pytest.mark.parametrize("seed", range(12))
def test_random_route_forward_backward(gpu, seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    vec = 8 if dtype == torch.bfloat16 else 4
    S = int(rng.integers(1, 17))
    D = vec * int(rng.integers(8, (8192 if dtype == torch.bfloat16 else 4096) // vec + 1))
    N = _rows(rng, S * D)
    pdt = dtype if dtype == torch.float32 else [torch.bfloat16, torch.float32][int(rng.integers(2))]
    with_gain = bool(rng.integers(2))
    qscale = [0.05, 0.5][int(rng.integers(2))]
    pol = _policy(rng)
    print(f"random route seed={seed}: {dtype} S={S} D={D} N={N} param={pdt} gain={with_gain} "
          f"qscale={qscale} policy={pol}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(2000 + seed)
    scales = torch.exp(torch.empty(S).uniform_(np.log(0.25), np.log(4.0), generator=g))
    buf = (torch.randn(S, 1, N, D, generator=g) * scales[:, None, None, None]).to(dtype).to(gpu).requires_grad_(True)
    query = (torch.randn(D, generator=g) * qscale).to(pdt).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(pdt).to(gpu) if with_gain else torch.ones(D, dtype=pdt).to(gpu)
    norm = Norm(gain.clone(), 1e-5)
    norm.weight.requires_grad_(with_gain)
    G = torch.randn(1, N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    mask = torch.ones(S, dtype=torch.bool, device=gpu)

    def run():
        out = kotodama_amd.route_static(buf, query, norm, mask, S)
        (out.float() * G).sum().backward()
        torch.cuda.synchronize()
        return out

    out = _with_policy(pol, run)
    pd = "bf16" if pdt == torch.bfloat16 else "f32"
    qw = O.fold_query(np64(query), np64(norm.weight), pd)
    x = np64(buf).reshape(S, N, D)
    ref = O.route(x, qw, 1e-5)["out"][0]
    # bf16 sources with fp32 parameters give an fp32 output (the einsum branch promotes)
    assert out.dtype == (torch.float32 if torch.float32 in (dtype, pdt) else torch.bfloat16)
    if out.dtype == torch.bfloat16:
        check_bf16(out.reshape(N, D), ref, f"seed {seed} out")
    else:
        check_f32(out.reshape(N, D), ref, f"seed {seed} out")
    b = O.route_backward(x, qw, 1e-5, np64(G).reshape(N, D), None)
    check_grad(buf.grad.reshape(S, N, D), b["dx"], dtype, f"seed {seed} dsources")
    check_grad(query.grad, b["dqw"] * np64(norm.weight), pdt, f"seed {seed} dquery")
    if with_gain:
        check_grad(norm.weight.grad, b["dqw"] * np64(query), pdt, f"seed {seed} dgain")


@pytest.mark.parametrize("seed", range(8))
def test_random_merge_forward_backward(gpu, seed):
    rng = np.random.default_rng(3000 + seed)
    pdt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    idt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    qdt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    vec = 8 if pdt == torch.bfloat16 else 4
    D = vec * int(rng.integers(8, (8192 if pdt == torch.bfloat16 else 4096) // vec + 1))
    if rng.integers(2):  # half the cases on widths the row-per-wave merge takes
        D = 512 * int(rng.integers(1, 9))
    N = _rows(rng, 2 * D)
    pol = _policy(rng)
    print(f"random merge seed={seed}: partial {pdt} inter {idt} query {qdt} D={D} N={N} policy={pol}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(4000 + seed)
    partial = torch.randn(N, D, generator=g).to(pdt).to(gpu).requires_grad_(True)
    inter = (0.5 * torch.randn(N, D, generator=g)).to(idt).to(gpu).requires_grad_(True)
    lse = (2 * torch.randn(N, generator=g)).to(gpu).requires_grad_(True)
    q = (torch.randn(D, generator=g) * [0.05, 0.5][int(rng.integers(2))]).to(qdt).to(gpu).requires_grad_(True)
    G = torch.randn(N, D, generator=g).to(torch.bfloat16).float().to(gpu)

    def run():
        merged, logit, inv = ops.merge(partial, q, inter, lse, 1e-5)
        (merged.float() * G).sum().backward()
        torch.cuda.synchronize()
        return merged, logit, inv

    merged, logit, inv = _with_policy(pol, run)
    ref = O.merge(np64(partial), np64(q), np64(inter), np64(lse), 1e-5)
    if idt == torch.bfloat16:
        check_bf16(merged, ref["out"], f"seed {seed} merged")
    else:
        check_f32(merged, ref["out"], f"seed {seed} merged")
    np.testing.assert_allclose(np64(logit), ref["logit"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(np64(inv), ref["inv_rms"], rtol=1e-5)
    b = O.merge_backward(np64(partial), np64(q), np64(inter), np64(lse), 1e-5, np64(G))
    check_grad(partial.grad, b["dpartial"], pdt, f"seed {seed} dpartial")
    check_grad(inter.grad, b["dinter"], idt, f"seed {seed} dinter")
    check_grad(lse.grad, b["dlse"], torch.float32, f"seed {seed} dlse")
    check_grad(q.grad, b["dq"], qdt, f"seed {seed} dquery")


@pytest.mark.parametrize("seed", range(8))
def test_random_batched_queries_forward_backward(gpu, seed):
    # the serving engine's phase-1 call: Q queries over one stack, bf16
    # output and fp32 lse, and its batched backward (matrix-core kernels for
    # S <= 8, Q <= 8, D <= 4096; the VALU kernel or per-query calls beyond)
    rng = np.random.default_rng(5000 + seed)
    S = int(rng.integers(1, 10))
    Q = int(rng.integers(2, 10))
    D = 8 * int(rng.integers(16, 513))
    N = _rows(rng, (S + Q) * D)
    with_gain = bool(rng.integers(2))
    print(f"random batched seed={seed}: S={S} Q={Q} D={D} N={N} gain={with_gain}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(6000 + seed)
    scales = torch.exp(torch.empty(S).uniform_(np.log(0.5), np.log(4.0), generator=g))
    buf = (torch.randn(S, 1, N, D, generator=g) * scales[:, None, None, None]).to(torch.bfloat16).to(gpu)
    buf.requires_grad_(True)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(torch.bfloat16).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu).requires_grad_(True) if with_gain else None
    G = torch.randn(Q, 1, N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    GL = torch.randn(Q, 1, N, generator=g).to(gpu)
    out, _, lse, _, _ = ops.route(buf, S, qs, gain, 1e-5, torch.bfloat16, True, False)
    (out.float() * G).sum().add_((lse * GL).sum()).backward()
    torch.cuda.synchronize()
    x = np64(buf).reshape(S, N, D)
    dx = np.zeros_like(x)
    dgain = np.zeros(D)
    for j in range(Q):
        qw = O.fold_query(np64(qs[j]), np64(gain) if with_gain else None, "bf16")
        r = O.route(x, qw, 1e-5)
        check_bf16(out[j].reshape(N, D), r["out"][0], f"seed {seed} out[{j}]")
        np.testing.assert_allclose(np64(lse[j]).reshape(-1), r["lse"][0], atol=2e-5, rtol=1e-6)
        b = O.route_backward(x, qw, 1e-5, np64(G[j]).reshape(N, D), np64(GL[j]).reshape(-1))
        dx += b["dx"]
        check_grad(qs.grad[j], b["dqw"] * (np64(gain) if with_gain else 1.0), torch.bfloat16, f"seed {seed} dquery[{j}]")
        dgain += b["dqw"] * np64(qs[j])
    check_grad(buf.grad.reshape(S, N, D), dx, torch.bfloat16, f"seed {seed} dsources")
    if with_gain:
        check_grad(gain.grad, dgain, torch.bfloat16, f"seed {seed} dgain")
