"""Seeded randomized parity sweep (GPU) over the routing entry points.

Each case draws its shape and options from a fixed seed: source count,
width (any multiple of the 16-byte chunk up to the largest supported row),
row count, source and parameter dtypes, gain or none, a flat or a peaky
softmax (query scale), and the kernel policy (row-per-wave or
row-per-workgroup).  It runs the drop-in forward and backward through
torch.autograd and checks outputs and gradients against the float64 oracle
at the bars of the other parity tests (check_bf16 for bf16 outputs,
check_grad for bf16 gradients; fp32 outputs with logits to 2 fp32 ulps of
their dot products' absolute sums and
fp32 gradients within 5x of the reference's op sequence differentiated in
fp32, see check_f32_logits and check_grad_f32).  Row counts are capped so that the float64 oracle
handles at most ~2M source elements per case.  ATTNRES_RANDOM_SEEDS=<n> runs n
seeds per family instead of the default 8-12.
"""

import os

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops
from oracle import attnres_oracle as O
from oracle import torch_cpu_path as TP

from .test_gpu_backward import Norm, check_grad, np64
from .test_gpu_parity import check_bf16, check_f32

pytestmark = pytest.mark.gpu

MAX_ELEMS = 2_000_000
# seeds per family; ATTNRES_RANDOM_SEEDS=<n> runs a longer sweep
SEEDS = int(os.environ.get("ATTNRES_RANDOM_SEEDS", "0"))


def check_f32_logits(out, ref, sens, dot_scale, label, ulps=2):
    """fp32 outputs, per row: |err| <= 1e-5 |ref| + 1e-6 max|ref| (the contract bar)
    + ulps * 2^-24 * dot_scale * sens.  `sens` ((N, D)) is the outputs' first-order
    response per unit of logit error; `dot_scale` ((N,)) the largest inv_rms *
    sum_d |x_d q_d| of the row's logits, the scale of an fp32 dot product's rounding
    error.  The last term matters on peaked rows (logits of 30-60 from thousands of
    terms, comparable weights), where any fp32 evaluation moves the output by a few
    times the contract bar."""
    got = np64(out)
    tol = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max() + ulps * 2.0**-24 * dot_scale[:, None] * sens
    e = float((np.abs(got - ref) / tol).max())
    assert e <= 1.0, f"{label}: {e:.2f}x the fp32 bar"


def route_sensitivity(x, qw, ref_out, r):
    """(sens, dot_scale) of a routing call from the float64 oracle's weights and
    inv_rms: d out / d logit_s = w_s (x_s - out)."""
    sens = np.einsum("sn,snd->nd", r["weights"][0], np.abs(x - ref_out[None]))
    dot_scale = (np.einsum("snd,d->ns", np.abs(x), np.abs(qw)) * r["inv_rms"]).max(1)
    return sens, dot_scale


def check_grad_f32(got, ref, ref32, label, factor=5.0):
    """fp32 gradients: the contract bar of check_grad (1e-4 |ref| + 1e-5 max|ref|), or
    within `factor` of the worst error of the reference's op sequence differentiated in
    fp32 (ref32) against the same float64 oracle: sums over tokens of products whose
    softmax part cancels (G.x_s - G.out) carry fp32 errors above the fixed bar.  Over
    186 fp32 gradient checks of a 100-seed sweep the kernels' worst error was 1.0x the
    fp32 reference's at the median, 2.0x at the 99th percentile and 4.2x at most, and
    one check exceeded the contract bar (1.14x)."""
    got = np64(got)
    tol = 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max()

    def ratio(err):  # err / tol, 0 where both are 0 (e.g. all-zero query gradients at S = 1)
        return float(np.where(err == 0, 0.0, err / np.maximum(tol, 1e-300)).max())

    e, e32 = ratio(np.abs(got - ref)), ratio(np.abs(ref32 - ref))
    print(f"[f32 grad] {label}: {e:.2f}x the bar (fp32 reference op sequence {e32:.2f}x)", flush=True)
    assert e <= max(1.0, factor * e32), f"{label}: {e:.2f}x the fp32 bar; the fp32 reference op sequence {e32:.2f}x"


def _route_f32_grads(x, query, gain, eps, G):
    """Gradients (sources, query, gain) of the reference's op sequence (llama.py:640-644) in
    fp32 on the CPU, through torch autograd; the gain fold is an fp32 product."""
    xt = torch.tensor(x, dtype=torch.float32).unsqueeze(1).requires_grad_(True)
    q = torch.tensor(query, dtype=torch.float32).requires_grad_(True)
    g = torch.tensor(gain, dtype=torch.float32).requires_grad_(True)
    mask = torch.ones(x.shape[0], dtype=torch.bool)
    out = TP.route_static_cpu(xt, q * g, eps, mask)
    (out * torch.tensor(G, dtype=torch.float32)).sum().backward()
    return xt.grad[:, 0].double().numpy(), q.grad.double().numpy(), g.grad.double().numpy()


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


@pytest.mark.parametrize("seed", range(SEEDS or 12))
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
        sens, lmax = route_sensitivity(x, qw, ref, O.route(x, qw, 1e-5))
        check_f32_logits(out.reshape(N, D), ref, sens, lmax, f"seed {seed} out")
    b = O.route_backward(x, qw, 1e-5, np64(G).reshape(N, D), None)
    f32 = None
    if torch.float32 in (dtype, pdt):
        f32 = _route_f32_grads(x, np64(query), np64(norm.weight), 1e-5, np64(G).reshape(N, D))
    if dtype == torch.float32:
        check_grad_f32(buf.grad.reshape(S, N, D), b["dx"], f32[0], f"seed {seed} dsources")
    else:
        check_grad(buf.grad.reshape(S, N, D), b["dx"], dtype, f"seed {seed} dsources")
    if pdt == torch.float32:
        check_grad_f32(query.grad, b["dqw"] * np64(norm.weight), f32[1], f"seed {seed} dquery")
        if with_gain:
            check_grad_f32(norm.weight.grad, b["dqw"] * np64(query), f32[2], f"seed {seed} dgain")
    else:
        check_grad(query.grad, b["dqw"] * np64(norm.weight), pdt, f"seed {seed} dquery")
        if with_gain:
            check_grad(norm.weight.grad, b["dqw"] * np64(query), pdt, f"seed {seed} dgain")


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_row_per_wave_backward(gpu, seed):
    # the row-per-wave backward's shapes (bf16, rows of 6 KiB with S <= 8 or 8 KiB with
    # S <= 9) with random row counts, parameter dtype, gain, softmax peakedness and dL/dlse
    rng = np.random.default_rng(9000 + seed)
    D = [3072, 4096][int(rng.integers(2))]
    S = int(rng.integers(1, (8 if D == 3072 else 9) + 1))
    N = _rows(rng, S * D)
    pdt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    with_gain = bool(rng.integers(2))
    # dL/dlse with bf16 parameters only (the fp32 comparator below has no lse term)
    with_lse = bool(rng.integers(2)) and pdt == torch.bfloat16
    qscale = [0.05, 0.5][int(rng.integers(2))]
    print(f"random row-per-wave backward seed={seed}: S={S} D={D} N={N} param={pdt} gain={with_gain} "
          f"lse={with_lse} qscale={qscale}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(9500 + seed)
    scales = torch.exp(torch.empty(S).uniform_(np.log(0.25), np.log(4.0), generator=g))
    buf = (torch.randn(S, 1, N, D, generator=g) * scales[:, None, None, None]).to(torch.bfloat16).to(gpu)
    buf.requires_grad_(True)
    query = (torch.randn(D, generator=g) * qscale).to(pdt).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(pdt).to(gpu) if with_gain else torch.ones(D, dtype=pdt).to(gpu)
    norm = Norm(gain.clone(), 1e-5)
    norm.weight.requires_grad_(with_gain)
    G = torch.randn(1, N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    gl = (torch.randn(1, N, generator=g) * 0.3).to(gpu) if with_lse else None

    def run():
        res = ops.route(buf, S, query, norm.weight, 1e-5, torch.bfloat16, True, False)
        loss = (res[0][0].float() * G).sum()
        if gl is not None:
            loss = loss + (res[2][0] * gl).sum()
        loss.backward()
        torch.cuda.synchronize()

    _with_policy(_capi.POLICY_STREAM, run)
    pd = "bf16" if pdt == torch.bfloat16 else "f32"
    qw = O.fold_query(np64(query), np64(norm.weight), pd)
    x = np64(buf).reshape(S, N, D)
    b = O.route_backward(x, qw, 1e-5, np64(G).reshape(N, D), None if gl is None else np64(gl).reshape(N))
    check_grad(buf.grad.reshape(S, N, D), b["dx"], torch.bfloat16, f"seed {seed} dsources")
    if pdt == torch.float32:
        f32 = _route_f32_grads(x, np64(query), np64(norm.weight), 1e-5, np64(G).reshape(N, D))
        check_grad_f32(query.grad, b["dqw"] * np64(norm.weight), f32[1], f"seed {seed} dquery")
    else:
        check_grad(query.grad, b["dqw"] * np64(norm.weight), pdt, f"seed {seed} dquery")


@pytest.mark.parametrize("seed", range(SEEDS or 8))
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
        # merged = inter + pi (p - inter), pi = sigmoid(logit - lse): d merged / d logit
        # = pi (1 - pi) (p - inter)
        pi = 1.0 / (1.0 + np.exp(-(ref["logit"] - np64(lse))))
        sens = (pi * (1.0 - pi))[:, None] * np.abs(np64(partial) - np64(inter))
        lmax = (np.abs(np64(partial)) @ np.abs(np64(q))) * ref["inv_rms"]
        check_f32_logits(merged, ref["out"], sens, lmax, f"seed {seed} merged")
    np.testing.assert_allclose(np64(logit), ref["logit"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(np64(inv), ref["inv_rms"], rtol=1e-5)
    b = O.merge_backward(np64(partial), np64(q), np64(inter), np64(lse), 1e-5, np64(G))
    check_grad(partial.grad, b["dpartial"], pdt, f"seed {seed} dpartial")
    check_grad(inter.grad, b["dinter"], idt, f"seed {seed} dinter")
    check_grad(lse.grad, b["dlse"], torch.float32, f"seed {seed} dlse")
    check_grad(q.grad, b["dq"], qdt, f"seed {seed} dquery")


@pytest.mark.parametrize("seed", range(SEEDS or 8))
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


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_block_arena_forward(gpu, seed):
    # the stack-free caller (fused block steps over one arena): random layer
    # count and boundary set (with or without layer 0), arena dtype, width,
    # rows, gains and kernel policy; every routing point, the committed blocks
    # and the final partial against the oracle's caller loop
    from kotodama_amd.engine import AttnResRouter
    from kotodama_amd.schedule import AttnResSchedule

    rng = np.random.default_rng(7000 + seed)
    dtype = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    L = int(rng.integers(1, 9))
    bounds = sorted(int(b) for b in rng.choice(L, size=int(rng.integers(0, L + 1)), replace=False))
    vec = 8 if dtype == torch.bfloat16 else 4
    D = vec * int(rng.integers(8, (8192 if dtype == torch.bfloat16 else 4096) // vec + 1))
    if rng.integers(2):  # half the cases on widths the row-per-wave kernels take
        D = (512 if dtype == torch.bfloat16 else 256) * int(rng.integers(1, 9))
    sched = AttnResSchedule.build(L, boundaries=bounds)
    N = _rows(rng, D * sum(sched.active_counts) // 4)
    with_gain = bool(rng.integers(2))
    pol = _policy(rng)
    print(f"random arena seed={seed}: {dtype} L={L} boundaries={bounds} D={D} N={N} gain={with_gain} policy={pol}",
          flush=True)
    g = torch.Generator(device="cpu").manual_seed(8000 + seed)
    P = sched.num_points
    embed = torch.randn(N, D, generator=g).to(dtype).to(gpu)
    deltas = (torch.randn(2 * L, N, D, generator=g) * 0.5).to(dtype).to(gpu)
    q = (torch.randn(P, D, generator=g) * [0.05, 0.5][int(rng.integers(2))]).to(dtype).to(gpu)
    gn = [(1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu) if with_gain else None for _ in range(P)]
    router = AttnResRouter(sched, list(q), gn, 1e-5)
    outs = []

    def sublayer(j, h):
        outs.append(h.clone())
        return deltas[j]

    def run():
        arena = router.new_arena((N,), D, dtype, gpu)
        outs.append(router.forward(embed, sublayer, arena=arena))
        torch.cuda.synchronize()
        return arena

    arena = _with_policy(pol, run)
    pd = "bf16" if dtype == torch.bfloat16 else "f32"
    qws = [O.fold_query(np64(q[j]), np64(gn[j]) if with_gain else None, pd) for j in range(P)]
    ref = O.block_forward(np64(embed), [np64(deltas[j]) for j in range(2 * L)], qws, 1e-5, L, set(bounds), dtype=pd)
    assert len(outs) == P and arena.n_committed == len(bounds)
    if dtype == torch.bfloat16:
        for j in range(P):
            check_bf16(outs[j], ref["outs"][j], f"seed {seed} point {j}")
    else:
        # the sources of every point (the partial sums are fp32 additions, as
        # in the arena) for the fp32 bar's sensitivity term
        partial, committed = np64(embed), []
        for j in range(P):
            i, pre_mlp = divmod(j, 2)
            if j < P - 1 and pre_mlp and i in set(bounds):
                committed, partial = committed + [partial], np.zeros_like(partial)
            if j < P - 1 and pre_mlp:
                partial = (partial.astype(np.float32) + np64(deltas[2 * i]).astype(np.float32)).astype(np.float64)
            srcs = np.stack(committed + [partial])
            sens, lmax = route_sensitivity(srcs, qws[j], ref["outs"][j], O.route(srcs, qws[j], 1e-5))
            check_f32_logits(outs[j], ref["outs"][j], sens, lmax, f"seed {seed} point {j}")
            if j < P - 1 and pre_mlp:
                partial = (partial.astype(np.float32) + np64(deltas[2 * i + 1]).astype(np.float32)).astype(np.float64)
    for b in range(len(bounds)):
        assert np.array_equal(np64(arena.committed[b]), ref["committed"][b]), f"seed {seed} committed {b}"
    assert np.array_equal(np64(arena.partial), ref["partial"]), f"seed {seed} partial"


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_list_routing_weights_and_backward(gpu, seed):
    # list routing over separate allocations in a random order (the pointer-
    # table kernel instance when they are not equally spaced), with the
    # routing weights and lse requested, and its backward
    rng = np.random.default_rng(9000 + seed)
    dtype = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    vec = 8 if dtype == torch.bfloat16 else 4
    S = int(rng.integers(1, 13))
    D = vec * int(rng.integers(8, (8192 if dtype == torch.bfloat16 else 4096) // vec + 1))
    if rng.integers(2):
        D = (512 if dtype == torch.bfloat16 else 256) * int(rng.integers(1, 9))
    N = _rows(rng, 2 * S * D)
    want_weights = bool(rng.integers(2))
    pol = _policy(rng)
    print(f"random list seed={seed}: {dtype} S={S} D={D} N={N} weights={want_weights} policy={pol}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(10000 + seed)
    srcs = [(torch.randn(N, D, generator=g) * float(np.exp(rng.uniform(np.log(0.25), np.log(4.0)))))
            .to(dtype).to(gpu).requires_grad_(True) for _ in range(S)]
    lst = [srcs[i] for i in rng.permutation(S)]
    query = (torch.randn(D, generator=g) * 0.2).to(dtype).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu).requires_grad_(True)
    G = torch.randn(N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    GL = torch.randn(N, generator=g).to(gpu)

    def run():
        out, weights, lse, _, _ = ops.route_list(lst, query, gain, 1e-5, dtype, want_weights, False)
        loss = (out.float() * G).sum()
        if want_weights:
            loss = loss + (lse.reshape(-1) * GL).sum()
        loss.backward()
        torch.cuda.synchronize()
        return out, weights, lse

    out, weights, lse = _with_policy(pol, run)
    pd = "bf16" if dtype == torch.bfloat16 else "f32"
    qw = O.fold_query(np64(query), np64(gain), pd)
    x = np.stack([np64(t) for t in lst])
    r = O.route(x, qw, 1e-5)
    if dtype == torch.bfloat16:
        check_bf16(out.reshape(N, D), r["out"][0], f"seed {seed} out")
    else:
        sens, lmax = route_sensitivity(x, qw, r["out"][0], r)
        check_f32_logits(out.reshape(N, D), r["out"][0], sens, lmax, f"seed {seed} out")
    if want_weights:
        np.testing.assert_allclose(np64(weights).reshape(S, N), r["weights"][0], atol=1e-5)
        np.testing.assert_allclose(np64(lse).reshape(N), r["lse"][0], atol=2e-5, rtol=1e-6)
    b = O.route_backward(x, qw, 1e-5, np64(G), np64(GL) if want_weights else None)
    for k, t in enumerate(lst):
        check_grad(t.grad, b["dx"][k], dtype, f"seed {seed} dsource {k}")
    check_grad(query.grad, b["dqw"] * np64(gain), dtype, f"seed {seed} dquery")
    check_grad(gain.grad, b["dqw"] * np64(query), dtype, f"seed {seed} dgain")


CANARY = 7.0  # exact in bf16 and fp32; no routed value here equals it


def _code(dtype):
    return _capi.DTYPE_BF16 if dtype == torch.bfloat16 else _capi.DTYPE_F32


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_row_strides_through_the_c_abi(gpu, seed):
    # attnres_route_fwd / attnres_route_bwd called directly on rows of wider,
    # canary-filled buffers with random strides (16-byte aligned): sources,
    # outputs, query planes, output gradient and gradients; forward with 1-9
    # queries, backward with one; nothing outside the rows may be written
    rng = np.random.default_rng(11000 + seed)
    sdt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    qdt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    odt = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    vec = 8 if sdt == torch.bfloat16 else 4
    ovec = 8 if odt == torch.bfloat16 else 4
    S = int(rng.integers(1, 13))
    Q = 1 if rng.integers(2) else int(rng.integers(2, 10))
    D = vec * int(rng.integers(8, (8192 if sdt == torch.bfloat16 else 4096) // vec + 1))
    N = _rows(rng, (S + Q) * D)
    src_ld = D + vec * int(rng.integers(0, 9))
    out_ld = D + ovec * int(rng.integers(0, 9))
    qstride = N * out_ld + ovec * int(rng.integers(0, 9))
    pol = _policy(rng)
    print(f"random strides seed={seed}: src {sdt} q {qdt} out {odt} S={S} Q={Q} D={D} N={N} src_ld={src_ld} "
          f"out_ld={out_ld} policy={pol}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(12000 + seed)
    big = torch.full((S, N, src_ld), CANARY, dtype=sdt)
    for s in range(S):
        big[s, :, :D] = (torch.randn(N, D, generator=g) * float(np.exp(rng.uniform(np.log(0.25), np.log(4.0))))).to(sdt)
    big = big.to(gpu)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(qdt).to(gpu)
    obuf = torch.full(((Q - 1) * qstride + N * out_ld,), CANARY, dtype=odt, device=gpu)
    weights = torch.full((Q, S, N), CANARY, device=gpu)
    lse = torch.full((Q, N), CANARY, device=gpu)
    before = big.clone()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    prev = _capi.set_kernel_policy(pol)
    try:
        _capi.route_fwd(_capi.pointer_array([big[s].data_ptr() for s in range(S)]), S, N, D, src_ld, _code(sdt),
                        qs.data_ptr(), None, Q, _code(qdt), 1e-5, obuf.data_ptr(), _code(odt), out_ld, qstride,
                        weights.data_ptr(), lse.data_ptr(), None, None, stream)
    finally:
        _capi.set_kernel_policy(prev)
    torch.cuda.synchronize()
    x = np64(big[:, :, :D])
    ref = O.route(x, np64(qs), 1e-5)
    for q in range(Q):
        view = obuf[q * qstride: q * qstride + N * out_ld].view(N, out_ld)
        if odt == torch.bfloat16:
            check_bf16(view[:, :D], ref["out"][q], f"seed {seed} out[{q}]")
        else:
            check_f32(view[:, :D], ref["out"][q], f"seed {seed} out[{q}]")
        assert torch.all(view[:, D:] == CANARY), f"seed {seed}: output row padding written"
        if q + 1 < Q:
            assert torch.all(obuf[q * qstride + N * out_ld: (q + 1) * qstride] == CANARY), f"seed {seed}: gap written"
        assert np.abs(np64(weights[q]) - ref["weights"][q]).max() <= 1e-5, f"seed {seed} weights[{q}]"
        np.testing.assert_allclose(np64(lse[q]), ref["lse"][q], rtol=1e-5, atol=1e-5)
    assert torch.equal(big, before), f"seed {seed}: a source was modified"
    if Q > 1:
        return
    gvec = 8 if sdt == torch.bfloat16 else 4
    gout_ld = D + gvec * int(rng.integers(0, 9))
    grad_ld = D + vec * int(rng.integers(0, 9))
    gbuf = torch.full((N, gout_ld), CANARY, dtype=sdt)
    gbuf[:, :D] = torch.randn(N, D, generator=g).to(sdt)
    gbuf = gbuf.to(gpu)
    glse = (torch.randn(N, generator=g) * 0.1).to(gpu) if rng.integers(2) else None
    dbig = torch.full((S, N, grad_ld), CANARY, dtype=sdt, device=gpu)
    ws = torch.empty(_capi.route_bwd_workspace_size(N, D) // 4, device=gpu)
    dq = torch.full((D,), CANARY, dtype=qdt, device=gpu)
    _capi.route_bwd(_capi.pointer_array([big[s].data_ptr() for s in range(S)]), S, N, D, src_ld, _code(sdt),
                    qs.data_ptr(), None, _code(qdt), 1e-5, gbuf.data_ptr(), _code(sdt), gout_ld,
                    None if glse is None else glse.data_ptr(),
                    _capi.pointer_array([dbig[s].data_ptr() for s in range(S)]), grad_ld, ws.data_ptr(),
                    ws.numel() * 4, dq.data_ptr(), None, stream)
    torch.cuda.synchronize()
    b = O.route_backward(x, np64(qs[0]), 1e-5, np64(gbuf[:, :D]), None if glse is None else np64(glse))
    check_grad(dbig[:, :, :D], b["dx"], sdt, f"seed {seed} dsources")
    assert torch.all(dbig[:, :, D:] == CANARY), f"seed {seed}: gradient row padding written"
    check_grad(dq, b["dqw"], qdt, f"seed {seed} dquery")


def _check_grad_sum(got, ref, first, dtype, label):
    """A gradient summed over two routing calls inside the backward kernels.  The backward
    reaches the second call first, which writes its gradient ``first`` rounded to bf16; the
    first call adds its own in fp32 and rounds again.  So on top of check_grad's bar (one ulp of
    |ref| plus 1e-3 max|ref|, for the fp32 evaluation) an element may carry half an ulp of
    |first|, which exceeds an ulp of |ref| where the two calls' gradients cancel; and at least
    half of the elements equal the correctly rounded sum.  fp32 as check_grad."""
    if dtype == torch.float32:
        check_grad(got, ref, dtype, label)
        return
    g = np64(got)
    err = np.abs(g - ref)

    def ulp(x):
        return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 2.0**-126))) - 7)

    tol = ulp(ref) + 0.5 * ulp(first) + 1e-3 * np.abs(ref).max()
    assert (err <= tol).all(), f"{label}: worst err {err.max():.3e}"
    counted = np.abs(ref) >= 1e-30
    if counted.any():
        assert np.mean(g[counted] == O.bf16_round(ref[counted])) >= 0.5, f"{label}: too few correctly rounded"


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_training_points(gpu, seed):
    # two routing points of the training loop (ops.route_point: the fused partial
    # update and the in-kernel gradient sums) over the same committed blocks, the
    # second routing the first's partial as it is, with random block count,
    # width, rows, dtype, gains, peakedness, with or without a pending sublayer
    # output and kernel policy:
    #   X = partial (+ delta);  h1 = route(C + [X], q1);  h2 = route(C + [X], q2)
    #   loss = <h1, G1> + <h2, G2> + <X, Gp>
    # routed rows against the oracle; dC_k = dx1_k + dx2_k (summed in the GradSlot),
    # dX = dx1_X + dx2_X + Gp (the second call's gradient of the partial output
    # is the first's addend), returned for both partial and delta; query and gain
    # gradients of each call
    _training_points_case(gpu, seed, deferred=False)


@pytest.mark.parametrize("seed", range(SEEDS or 8))
def test_random_deferred_training_points(gpu, seed):
    # the same two points where the committed blocks' gradients are deferred
    # (attnres_route_bwd_defer per point; at each block's commit node one
    # attnres_route_bwd_gather, or for odd seeds one attnres_route_bwd_gather_seg
    # over all blocks at the last block's commit): bf16 at hidden 3072 (1..7
    # blocks) or 4096 (1..8)
    _training_points_case(gpu, seed, deferred=True)


def _training_points_case(gpu, seed, deferred):
    rng = np.random.default_rng((21000 if deferred else 11000) + seed)
    dtype = torch.bfloat16 if deferred else [torch.bfloat16, torch.float32][int(rng.integers(2))]
    if deferred:
        D = [3072, 4096, 1024, 512][int(rng.integers(4))]
        K = int(rng.integers(1, 9 if D == 4096 else 8))
    else:
        K = int(rng.integers(0, 9))
        vec = 8 if dtype == torch.bfloat16 else 4
        D = vec * int(rng.integers(8, (4096 if dtype == torch.bfloat16 else 2048) // vec + 1))
        if rng.integers(2):  # half the cases on widths the row-per-wave kernels take
            D = (512 if dtype == torch.bfloat16 else 256) * int(rng.integers(1, 9))
    N = _rows(rng, (K + 3) * D)
    with_delta = bool(rng.integers(2))
    with_gain = bool(rng.integers(2))
    qscale = 0.05 if dtype == torch.float32 else [0.05, 0.5][int(rng.integers(2))]
    pol = _policy(rng)
    # deferred, odd seeds: the slots share a GradSegments, so the last block's commit sums both points
    # into every block in one attnres_route_bwd_gather_seg (the others finish from its running sums)
    seg_mode = deferred and seed % 2 == 1
    print(f"random training points seed={seed}: {dtype} K={K} D={D} N={N} delta={with_delta} gain={with_gain} "
          f"qscale={qscale} policy={pol} segments={seg_mode}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(12000 + seed)

    def t(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dtype).to(gpu)

    blocks = [t(N, D, scale=float(np.exp(rng.uniform(np.log(0.25), np.log(4.0))))).requires_grad_(True)
              for _ in range(K)]
    partial = t(N, D).requires_grad_(True)
    delta = t(N, D, scale=0.5).requires_grad_(True) if with_delta else None
    q = [t(D, scale=qscale).requires_grad_(True) for _ in range(2)]
    gn = [(1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu).requires_grad_(True) if with_gain else None
          for _ in range(2)]
    G1, G2, Gp = (torch.randn(N, D, generator=g).to(dtype).to(gpu) for _ in range(3))

    def run():
        segs = ops.GradSegments() if seg_mode else None
        slots = [ops.GradSlot(segs) for _ in range(K)]
        committed = [ops.commit_block(b, s) for b, s in zip(blocks, slots)]
        h1, X = ops.route_point(committed, slots, partial, delta, q[0], gn[0], 1e-5, dtype)
        h2, X2 = ops.route_point(committed, slots, X, None, q[1], gn[1], 1e-5, dtype)
        loss = (h1.float() * G1.float()).sum() + (h2.float() * G2.float()).sum() + (X2.float() * Gp.float()).sum()
        loss.backward()
        torch.cuda.synchronize()
        return h1, h2, X

    deferred_calls, records = [], []
    real = ops._route_rows_backward_defer

    def counting(*a, **k):
        r = real(*a, **k)
        deferred_calls.append(r is not None)
        if r is not None:
            records.append((np64(r[1]), np64(r[3]), np64(r[2])))  # (w, c1, c2) records, dL/dout rows, qfold
        return r

    ops._route_rows_backward_defer = counting
    try:
        h1, h2, X = _with_policy(pol, run)
    finally:
        ops._route_rows_backward_defer = real
    if deferred:
        assert deferred_calls == [True, True], f"seed {seed}: the points did not defer ({deferred_calls})"
    pd = "bf16" if dtype == torch.bfloat16 else "f32"
    Xref = np64(partial) + np64(delta) if with_delta else np64(partial)
    Xref = O.bf16_round(Xref).astype(np.float64) if dtype == torch.bfloat16 else Xref.astype(np.float32).astype(np.float64)
    assert np.array_equal(np64(X), Xref), f"seed {seed}: partial + delta not rounded once"
    srcs = np.stack([np64(b) for b in blocks] + [Xref])
    res, f32 = [], []
    for j, (h, G) in enumerate(((h1, G1), (h2, G2))):
        qw = O.fold_query(np64(q[j]), np64(gn[j]) if with_gain else None, pd)
        ref = O.route(srcs, qw, 1e-5)["out"][0]
        if dtype == torch.bfloat16:
            check_bf16(h, ref, f"seed {seed} h{j + 1}")
        else:
            sens, lmax = route_sensitivity(srcs, qw, ref, O.route(srcs, qw, 1e-5))
            check_f32_logits(h, ref, sens, lmax, f"seed {seed} h{j + 1}")
        res.append(O.route_backward(srcs, qw, 1e-5, np64(G), None))
        gq = res[-1]["dqw"] * (np64(gn[j]) if with_gain else 1.0)
        if dtype == torch.float32:
            # fp32: against the reference op sequence differentiated in fp32, as the route family does
            gains = np64(gn[j]) if with_gain else np.ones(D)
            f32.append(_route_f32_grads(srcs, np64(q[j]), gains, 1e-5, np64(G)))
            check_grad_f32(q[j].grad, gq, f32[-1][1], f"seed {seed} dquery{j + 1}")
            if with_gain:
                check_grad_f32(gn[j].grad, res[-1]["dqw"] * np64(q[j]), f32[-1][2], f"seed {seed} dgain{j + 1}")
        else:
            check_grad(q[j].grad, gq, dtype, f"seed {seed} dquery{j + 1}")
            if with_gain:
                check_grad(gn[j].grad, res[-1]["dqw"] * np64(q[j]), dtype, f"seed {seed} dgain{j + 1}")
    dX = res[0]["dx"][K] + res[1]["dx"][K] + np64(Gp)
    if dtype == torch.float32:
        for k in range(K):
            check_grad_f32(blocks[k].grad, res[0]["dx"][k] + res[1]["dx"][k], f32[0][0][k] + f32[1][0][k],
                           f"seed {seed} dblock{k}")
        check_grad_f32(partial.grad, dX, f32[0][0][K] + f32[1][0][K] + np64(Gp), f"seed {seed} dpartial")
    else:
        for k in range(K):
            if seg_mode:
                # block K-1 is finished in the kernel (one rounding); the others from their running sums,
                # rounded to bf16 (both points' w G + c1 qfold) before their x terms are added
                first = np.zeros((N, D)) if k == K - 1 else \
                    sum(c[:, k, 0:1] * Gr + c[:, k, 1:2] * qf[None, :] for c, Gr, qf in records)
            else:
                first = res[1]["dx"][k]
            _check_grad_sum(blocks[k].grad, res[0]["dx"][k] + res[1]["dx"][k], first, dtype,
                            f"seed {seed} dblock{k}")
        _check_grad_sum(partial.grad, dX, res[1]["dx"][K] + np64(Gp), dtype, f"seed {seed} dpartial")
    if with_delta:
        assert torch.equal(delta.grad, partial.grad), f"seed {seed}: d(partial + delta) differs between its inputs"


@pytest.mark.parametrize("seed", range(SEEDS or 12))
def test_random_gather_seg(gpu, seed):
    # attnres_route_bwd_gather_seg over random segments: width 512, 1024, 3072 or 4096, 1..8
    # blocks, 1..48 terms (one launch), ragged row counts, padded row strides,
    # records wider than the blocks summed, running sums and x-coefficient sums
    # present or absent per block and updated in place or into separate
    # buffers, the addend absent, separate or in place.  The sums are those of
    # the kernel's contract (the defer tests pin the records' meaning): float64
    # sums of the records' terms, each within one bf16 ulp plus 2^-15 of the
    # sum of the products' magnitudes |w G| + |c1 q| (fp32 accumulation, the
    # coefficients split into bf16 hi + lo parts: 2^-18 of each product); the
    # x-coefficient sums within 1e-5 relative; no byte of the padding written
    rng = np.random.default_rng(31000 + seed)
    d = [3072, 4096, 1024, 512][int(rng.integers(4))]
    nb = int(rng.integers(1, 9))
    P = int(rng.integers(1, 49)) if rng.integers(4) == 0 else int(rng.integers(1, 17))
    n = int(np.exp(rng.uniform(0, np.log(1200))))
    pad = [8 * int(rng.integers(0, 5)) for _ in range(3)]
    gout_ld, x_ld, out_ld = d + pad[0], d + pad[1], d + pad[2]
    extra = int(rng.integers(0, 3))  # records per token beyond the nb summed
    addend_mode = ["none", "separate", "in_place"][int(rng.integers(3))]
    print(f"random gather_seg seed={seed}: d={d} nb={nb} P={P} n={n} lds={gout_ld},{x_ld},{out_ld} "
          f"extra={extra} addend={addend_mode}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(32000 + seed)
    bf = torch.bfloat16
    CAN = 7.0

    def rows(ld, scale=1.0):
        t = torch.full((n, ld), CAN, device=gpu, dtype=bf)
        t[:, :d] = (torch.randn((n, d), generator=g, device=gpu) * scale).to(bf)
        return t

    gouts = [rows(gout_ld) for _ in range(P)]
    qfolds = [(torch.randn(d, generator=g, device=gpu) * 0.1).to(bf) for _ in range(P)]
    coefs = []
    for _ in range(P):
        c = torch.randn((n, nb + extra, 4), generator=g, device=gpu)
        c[:, :, 2] *= 0.1
        coefs.append(c)
    x = rows(x_ld, 2.0)
    part_out = [torch.full((n, out_ld), CAN, device=gpu, dtype=bf) for _ in range(nb)]
    csum_out = [torch.full((n,), float("nan"), device=gpu) for _ in range(nb)]
    part_in, csum_in, prev, prev_cs = [], [], [], []
    for k in range(nb):
        has = bool(rng.integers(2)) and k < nb - 1 or (k == nb - 1 and rng.integers(4) == 0)
        in_place = bool(rng.integers(2))
        if has:
            src = part_out[k] if in_place else torch.full((n, out_ld), CAN, device=gpu, dtype=bf)
            src[:, :d] = (torch.randn((n, d), generator=g, device=gpu) * 0.5).to(bf)
            cs = csum_out[k] if in_place else torch.empty(n, device=gpu)
            cs.copy_(torch.randn(n, generator=g, device=gpu) * 0.1)
            prev.append(np64(src[:, :d]))
            prev_cs.append(np64(cs))
            part_in.append(src)
            csum_in.append(cs)
        else:
            prev.append(np.zeros((n, d)))
            prev_cs.append(np.zeros(n))
            part_in.append(None)
            csum_in.append(None)
    if addend_mode == "none":
        addend, add64 = None, np.zeros((n, d))
    else:
        addend = part_out[nb - 1] if addend_mode == "in_place" else torch.full((n, out_ld), CAN, device=gpu, dtype=bf)
        if addend_mode == "in_place" and part_in[nb - 1] is not None:
            addend = torch.full((n, out_ld), CAN, device=gpu, dtype=bf)  # the last block's part_in took that buffer
        addend[:, :d] = (torch.randn((n, d), generator=g, device=gpu) * 0.1).to(bf)
        add64 = np64(addend[:, :d])
    torch.cuda.synchronize()
    _capi.route_bwd_gather_seg(
        nb, n, d, _capi.DTYPE_BF16, P, _capi.pointer_array([t.data_ptr() for t in gouts]), gout_ld,
        _capi.pointer_array([c.data_ptr() for c in coefs]), _capi.int64_array([4 * (nb + extra)] * P),
        _capi.pointer_array([q.data_ptr() for q in qfolds]),
        _capi.pointer_array([t.data_ptr() if t is not None else None for t in part_in]),
        _capi.pointer_array([t.data_ptr() if t is not None else None for t in csum_in]),
        _capi.pointer_array([t.data_ptr() for t in part_out]),
        _capi.pointer_array([t.data_ptr() for t in csum_out[:-1]] + [None]),
        x.data_ptr(), x_ld, addend.data_ptr() if addend is not None else None, out_ld,
        torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    C = [np64(c) for c in coefs]
    Gs = [np64(t[:, :d]) for t in gouts]
    Q = [np64(q) for q in qfolds]

    def ulp(v):
        return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0**-126))) - 7)

    for k in range(nb):
        terms = [c[:, k, 0:1] * Gk + c[:, k, 1:2] * q[None, :] for c, Gk, q in zip(C, Gs, Q)]
        want = prev[k] + sum(terms)
        # the products' magnitudes: w G and c1 q enter separately, each coefficient as bf16 hi + lo
        mag = np.abs(prev[k]) + sum(np.abs(c[:, k, 0:1] * Gk) + np.abs(c[:, k, 1:2] * q[None, :])
                                    for c, Gk, q in zip(C, Gs, Q))
        cs = prev_cs[k] + sum(c[:, k, 2] for c in C)
        if k == nb - 1:
            xt = cs[:, None] * np64(x[:, :d])
            want = want + xt + add64
            mag = mag + np.abs(xt) + np.abs(add64)
        got = np64(part_out[k][:, :d])
        err = np.abs(got - want)
        bar = ulp(want) + 2.0**-15 * mag + 1e-30
        if not (err <= bar).all():
            i = np.unravel_index(np.argmax(err / bar), err.shape)
            raise AssertionError(f"seed {seed} block {k}: worst err/bar {(err / bar)[i]:.2f} at {i}: got {got[i]:.6e} "
                                 f"want {want[i]:.6e} |terms| {mag[i]:.3e} prev {prev[k][i]:.4e}")
        if k < nb - 1:
            e = np.abs(np64(csum_out[k]) - cs)
            assert (e <= 1e-5 * np.abs(cs) + 1e-6 * np.abs(cs).max() + 1e-30).all(), f"seed {seed} block {k} csum"
    for t in part_out + gouts + [x] + ([addend] if addend is not None else []):
        assert torch.all(t[:, d:] == CAN), f"seed {seed}: padding written"
