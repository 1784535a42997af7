"""Deferred block gradients of the training loop (GPU).

``attnres_route_bwd_defer`` is the row-per-wave routing backward that writes
only the last source's (the partial block's) gradient and stores, per token
and committed source s, the record (w_s, c1_s, c2_s, 0) with which
dL/dsource_s = w_s G + c1_s qfold + c2_s x_s, plus the folded query.
``attnres_route_bwd_gather`` sums one block's gradient over the calls that
read it from those records.  Checked through the C ABI:
* the partial's gradient and the query and gain gradients at the backward
  bar against the float64 oracle, and within a bf16 ulp of the ``_add``
  row-per-wave kernel on the same inputs;
* the folded query equal to the oracle's fold; each committed source's
  gradient rebuilt in float64 from its records against the oracle's;
* the gather of several calls' terms (different source counts and source
  positions, more terms than one launch takes, with and without an addend,
  in place) against the sum of the oracle's gradients, at the backward bar;
* the training loop that uses them (forward_attn_res under autograd at hidden
  3072 / 4096, bf16) against the loop in float64.
"""

import copy

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops
from oracle import attnres_oracle as O

from ._tiny_model import TinyModel, training_forward
from .test_gpu_accumulate import _call, _case
from .test_gpu_backward import check_grad, np64

pytestmark = pytest.mark.gpu

BF = _capi.DTYPE_BF16


def _defer(gpu, srcs, q, gain, gout, addend=None):
    """One attnres_route_bwd_defer call over the list of (n, d) sources."""
    S = len(srcs)
    n, d = srcs[0].shape
    gp = torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16)
    coef = torch.full((n, S - 1, 4), float("nan"), device=gpu)
    qfold = torch.empty(d, device=gpu, dtype=torch.bfloat16)
    dq = torch.empty(d, device=gpu, dtype=torch.bfloat16)
    dg = torch.empty(d, device=gpu, dtype=torch.bfloat16)
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=gpu)
    rc = _capi.route_bwd_defer(
        _capi.pointer_array([t.data_ptr() for t in srcs]), S, n, d, d, BF, q.data_ptr(), gain.data_ptr(), BF, 1e-5,
        gout.data_ptr(), BF, d, None, gp.data_ptr(), addend.data_ptr() if addend is not None else None, d,
        coef.data_ptr(), qfold.data_ptr(), ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), dg.data_ptr(),
        torch.cuda.current_stream(gpu).cuda_stream)
    _capi.check("attnres_route_bwd_defer", rc)
    torch.cuda.synchronize()
    return gp, coef, qfold, dq, dg


def _gather(gpu, x, terms, addend, out):
    """terms: (grad_out, coef, source index); out = addend + their sum."""
    n, d = x.shape
    _capi.route_bwd_gather(
        x.data_ptr(), n, d, d, BF, len(terms), _capi.pointer_array([g.data_ptr() for g, _, _, _ in terms]), d,
        _capi.pointer_array([c.data_ptr() + 16 * k for _, c, k, _ in terms]),
        _capi.int64_array([4 * c.shape[1] for _, c, _, _ in terms]),
        _capi.pointer_array([qf.data_ptr() for _, _, _, qf in terms]),
        addend.data_ptr() if addend is not None else None, out.data_ptr(), d,
        torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()


# (S, rows, hidden)
CASES = [(2, 2048, 3072), (5, 3000, 3072), (8, 4096, 3072), (3, 1500, 4096), (7, 777, 4096), (9, 1024, 4096),
         (2, 1500, 1024), (8, 2048, 1024), (5, 999, 512), (8, 3000, 512)]


@pytest.mark.parametrize("S,n,d", CASES, ids=[f"s{c[0]}-n{c[1]}-d{c[2]}" for c in CASES])
def test_defer_matches_add_kernel_and_oracle(gpu, S, n, d):
    print(f"route_bwd_defer S={S} n={n} d={d}", flush=True)
    src, q, gain, gout, addend = _case(gpu, S, n, d, torch.bfloat16, 300 + S)
    gp, coef, qfold, dq, dg = _defer(gpu, [src[s] for s in range(S)], q, gain, gout, addend[S - 1])
    prev = _capi.set_kernel_policy(_capi.POLICY_STREAM)
    try:
        grads = torch.full_like(src, 3.0)
        dq1, dg1 = _call(gpu, src, q, gain, gout, grads, [None] * (S - 1) + [addend[S - 1]])
    finally:
        _capi.set_kernel_policy(prev)
    qw = O.fold_query(np64(q), np64(gain), "bf16")
    assert np.array_equal(np64(qfold), qw), "folded query"
    ref = O.route_backward(np64(src), qw, 1e-5, np64(gout), None)
    check_grad(gp, ref["dx"][S - 1] + np64(addend[S - 1]), torch.bfloat16, "partial + addend")
    check_grad(dq, ref["dqw"] * np64(gain), torch.bfloat16, "dquery")
    check_grad(dg, ref["dqw"] * np64(q), torch.bfloat16, "dgain")
    # the _add kernel forms x.qw with fp32 products, this one on v_dot2: the
    # two agree to a bf16 ulp on the partial's gradient and the parameter ones
    for a, b, name in ((gp, grads[S - 1], "partial"), (dq, dq1, "dquery"), (dg, dg1, "dgain")):
        diff = (a.float() - b.float()).abs()
        assert (diff <= b.float().abs() * 2.0**-7 + 1e-3 * b.float().abs().max()).all(), f"{name} vs the _add kernel"
    c = coef.double().cpu().numpy()
    assert (c[..., 3] == 0).all(), "record padding"
    G = np64(gout)
    for s in range(S - 1):
        rebuilt = c[:, s, 0:1] * G + c[:, s, 1:2] * qw[None, :] + c[:, s, 2:3] * np64(src[s])
        want = ref["dx"][s]
        err = np.abs(rebuilt - want).max()
        # fp32 records (sums of D products): within 1e-4 of the largest gradient
        assert err <= 1e-4 * np.abs(want).max(), f"source {s}: records rebuild err {err:.3e}"


def _terms_for(gpu, x, plan, seed):
    """One deferred call per (S, index) of ``plan`` with x as source ``index``;
    returns the terms and the oracle's gradient of x from each."""
    n, d = x.shape
    g = torch.Generator(device=gpu).manual_seed(seed)
    terms, wants = [], []
    for S, k in plan:
        assert k < S - 1, "x must be a committed source (the partial, source S-1, has no record)"
        srcs = [(torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.2 * s)).to(torch.bfloat16)
                for s in range(S)]
        srcs[k] = x
        q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
        gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
        gout = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
        _, coef, qfold, _, _ = _defer(gpu, srcs, q, gain, gout)
        terms.append((gout, coef, k, qfold))
        ref = O.route_backward(np.stack([np64(t) for t in srcs]), O.fold_query(np64(q), np64(gain), "bf16"), 1e-5,
                               np64(gout), None)
        wants.append(ref["dx"][k])
    return terms, wants


GATHER_CASES = [
    (3072, 1500, [(2, 0), (5, 0), (5, 3), (8, 2), (8, 6)]),
    (4096, 1024, [(9, 0), (3, 1), (9, 7), (2, 0)]),
    (3072, 97, [(3, 1)]),
    (1024, 1200, [(8, 0), (4, 2), (6, 4)]),
    (512, 777, [(2, 0), (8, 3)]),
]


@pytest.mark.parametrize("d,n,plan", GATHER_CASES, ids=["d3072-5terms", "d4096-4terms", "d3072-1term-ragged",
                                                        "d1024-3terms", "d512-2terms"])
def test_gather_sums_the_deferred_terms(gpu, d, n, plan):
    print(f"route_bwd_gather d={d} n={n} terms={len(plan)}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(400 + len(plan))
    x = (torch.randn((n, d), generator=g, device=gpu) * 1.5).to(torch.bfloat16)
    add = (torch.randn((n, d), generator=g, device=gpu) * 0.01).to(torch.bfloat16)
    terms, wants = _terms_for(gpu, x, plan, 500 + len(plan))
    want = sum(wants)
    sep = torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16)
    _gather(gpu, x, terms, add, sep)
    check_grad(sep, want + np64(add), torch.bfloat16, "gather + addend")
    inpl = add.clone()
    _gather(gpu, x, terms, inpl, inpl)
    assert torch.equal(inpl, sep), "in place differs from a separate addend"
    none = torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16)
    _gather(gpu, x, terms, None, none)
    check_grad(none, want, torch.bfloat16, "gather without addend")
    # no terms: the addend itself
    zero = torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16)
    _gather(gpu, x, [], add, zero)
    assert torch.equal(zero, add)


def test_gather_more_terms_than_one_launch(gpu):
    # 56 terms (block 0 of the 3B schedule is read by 56 points): two launches,
    # the second adding to the first's output, so the sum of the first 48
    # terms is rounded to bf16 once more: the bar adds half an ulp of it
    from .test_gpu_backward import bf16_ulp

    n, d = 256, 3072
    g = torch.Generator(device=gpu).manual_seed(77)
    x = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
    plan = [(2 + j % 7, j % (1 + j % 7)) for j in range(56)]
    terms, wants = _terms_for(gpu, x, plan, 78)
    out = torch.empty((n, d), device=gpu, dtype=torch.bfloat16)
    _gather(gpu, x, terms, None, out)
    want = sum(wants)
    first = sum(wants[:48])
    err = np.abs(np64(out) - want)
    bar = bf16_ulp(want) + 0.5 * bf16_ulp(first) + 1e-3 * np.abs(want).max()
    assert (err <= bar).all(), f"56 terms: worst err {err.max():.3e} (max|ref| {np.abs(want).max():.3e})"


@pytest.mark.parametrize("d,bounds,max_s", [(3072, (0, 4, 8, 12), 5), (3072, (0, 2, 4, 6, 8, 10, 12, 14), 9),
                                            (4096, (0, 2, 4, 6, 8, 10, 12, 14), 9), (1024, (0, 3, 7, 12), 5),
                                            (512, (0, 2, 4, 6, 8, 10, 12, 14), 9)],
                         ids=["d3072-S5", "d3072-S9-mixed", "d4096-S9", "d1024-dd-S5", "d512-S9-mixed"])
def test_bf16_training_loop_with_deferred_gradients(gpu, d, bounds, max_s, monkeypatch):
    # forward_attn_res under autograd with the committed blocks' gradients
    # deferred to their commit nodes (S <= 8 at hidden 3072 and S <= 9 at 4096;
    # the S = 9 points at hidden 3072 take the _add kernels, so a block's slot
    # then holds both kinds), against the reference loop in float64: loss,
    # output and every parameter gradient.  Bar per tensor as in
    # test_bf16_training_loop_sixteen_layers: within 2x the error of the
    # reference's own op sequence evaluated in bf16, plus 2^-9 of the largest
    # reference magnitude; the loss within the noise its output's error gives.
    from oracle.torch_cpu_path import route_static_cpu

    L = 16
    model = TinyModel(d=d, num_layers=L, boundaries=bounds, seed=71, elementwise=True)
    model = model.to(torch.bfloat16).float()
    assert model._attn_res_max_sources == max_s
    gen = torch.Generator().manual_seed(72)
    embed = (torch.randn((2, 32, d), generator=gen) * 2).to(torch.bfloat16).float()
    G = torch.randn((2, 32, d), generator=gen).to(torch.bfloat16).float()

    def einsum(buf, q, norm, mask, n):
        return route_static_cpu(buf, q * norm.weight, norm.eps, mask)

    def run(m, e, fwd):
        e = e.clone().requires_grad_(True)
        out = fwd(m, e)
        loss = (out.float() * G.to(e.device)).sum()
        loss.backward()
        grads = {n: p.grad.double().cpu() for n, p in m.named_parameters()}
        grads["embed"] = e.grad.double().cpu()
        return loss.item(), out.detach().double().cpu(), grads

    deferred = []
    real = ops._route_rows_backward_defer

    def counting(*a, **k):
        r = real(*a, **k)
        deferred.append(r is not None)
        return r

    monkeypatch.setattr(ops, "_route_rows_backward_defer", counting)
    ref = run(copy.deepcopy(model).double(), embed.double(), lambda m, e: training_forward(m, e, einsum))
    tb = run(copy.deepcopy(model).to(gpu).to(torch.bfloat16), embed.to(gpu).to(torch.bfloat16),
             lambda m, e: training_forward(m, e, einsum))
    ours = run(copy.deepcopy(model).to(gpu).to(torch.bfloat16), embed.to(gpu).to(torch.bfloat16),
               kotodama_amd.forward_attn_res)
    torch.cuda.synchronize()
    # every point with a committed block tried; those within the kernels' S range deferred
    assert deferred and any(deferred)
    if max_s == 9 and d != 4096:
        assert not all(deferred), "the S = 9 points were expected on the _add kernels"
    else:
        assert all(deferred)

    def worst(a, b):
        return (a - b).abs().max().item()

    # the loss is sum(out * G): its error is the output's error weighted by G,
    # whose size (about 1 at this shape, for torch's op sequence as for these
    # kernels) is set by the bf16 outputs' rounding; the bar allows 6 times
    # the size that the output's own errors give, or twice torch's error
    noise = float(torch.sqrt(((ours[1] - ref[1]) * G.double()).pow(2).sum()))
    loss_bar = 2 * abs(tb[0] - ref[0]) + 6 * noise
    print(f"loss err {abs(ours[0] - ref[0]):.3e} (torch bf16 {abs(tb[0] - ref[0]):.3e}, output noise {noise:.3e})",
          flush=True)
    assert abs(ours[0] - ref[0]) <= loss_bar
    floor = 2.0**-9 * ref[1].abs().max().item()
    assert worst(ours[1], ref[1]) <= 2 * worst(tb[1], ref[1]) + floor, "output"
    ratios = []
    for name, want in ref[2].items():
        e_ours, e_tb = worst(ours[2][name], want), worst(tb[2][name], want)
        bar = 2 * e_tb + 2.0**-9 * want.abs().max().item()
        ratios.append(e_ours / max(e_tb, 1e-30))
        assert e_ours <= bar, f"{name}: err {e_ours:.3e}, torch bf16 op sequence {e_tb:.3e}"
    print(f"deferred training loop d={d} S<={max_s}: {len(ratios)} gradients, error / torch-bf16 error: median "
          f"{float(np.median(ratios)):.2f}, max {max(ratios):.2f}", flush=True)


def _gather_seg(gpu, nb, terms, part_in, csum_in, part_out, csum_out, x, addend, out):
    """attnres_route_bwd_gather_seg over blocks 0 .. nb-1; terms: (grad_out, coef, qfold)."""
    n, d = x.shape
    _capi.route_bwd_gather_seg(
        nb, n, d, BF, len(terms), _capi.pointer_array([g.data_ptr() for g, _, _ in terms]), d,
        _capi.pointer_array([c.data_ptr() for _, c, _ in terms]), _capi.int64_array([4 * c.shape[1] for _, c, _ in terms]),
        _capi.pointer_array([q.data_ptr() for _, _, q in terms]),
        _capi.pointer_array([p.data_ptr() if p is not None else None for p in part_in]),
        _capi.pointer_array([c.data_ptr() if c is not None else None for c in csum_in]),
        _capi.pointer_array([p.data_ptr() for p in part_out] + [out.data_ptr()]),
        _capi.pointer_array([c.data_ptr() for c in csum_out] + [None]),
        x.data_ptr(), d, addend.data_ptr() if addend is not None else None, d,
        torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()


# (blocks, points in the segment, rows, hidden)
SEG_CASES = [(1, 3, 700, 3072), (3, 8, 1000, 3072), (7, 8, 513, 3072), (4, 5, 800, 4096), (8, 8, 300, 4096),
             (2, 8, 900, 1024), (7, 8, 700, 1024), (5, 6, 1200, 512), (7, 3, 333, 512)]


@pytest.mark.parametrize("nb,P,n,d", SEG_CASES, ids=[f"b{c[0]}-p{c[1]}-n{c[2]}-d{c[3]}" for c in SEG_CASES])
def test_gather_seg_sums_a_segment(gpu, nb, P, n, d):
    # P points, each routing blocks 0 .. nb-1 and a partial of its own
    # (attnres_route_bwd_defer), then one attnres_route_bwd_gather_seg: blocks
    # j < nb-1 continue from running sums (some with none), the last one is
    # finished with its x term and an addend.  Each block's running sum and
    # x-coefficient sum against the same sums formed in float64 from the
    # records; the last block's gradient against the oracle
    print(f"route_bwd_gather_seg blocks={nb} points={P} n={n} d={d}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(700 + nb * 10 + P)
    blocks = [(torch.randn((n, d), generator=g, device=gpu) * (0.5 + 0.2 * j)).to(torch.bfloat16) for j in range(nb)]
    terms, recs, grads = [], [], []
    for p in range(P):
        own = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
        q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
        gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
        gout = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
        _, coef, qfold, _, _ = _defer(gpu, blocks + [own], q, gain, gout)
        terms.append((gout, coef, qfold))
        ref = O.route_backward(np.stack([np64(t) for t in blocks + [own]]), O.fold_query(np64(q), np64(gain), "bf16"),
                               1e-5, np64(gout), None)
        grads.append(ref["dx"][:nb])
        recs.append((coef.double().cpu().numpy(), np64(gout), np64(qfold)))
    part_in = [None if j % 2 else (torch.randn((n, d), generator=g, device=gpu) * 0.1).to(torch.bfloat16)
               for j in range(nb)]
    csum_in = [None if j % 2 else torch.randn(n, generator=g, device=gpu) * 0.01 for j in range(nb)]
    part_out = [torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16) for _ in range(nb - 1)]
    csum_out = [torch.full((n,), float("nan"), device=gpu) for _ in range(nb - 1)]
    addend = (torch.randn((n, d), generator=g, device=gpu) * 0.01).to(torch.bfloat16)
    out = torch.full((n, d), 3.0, device=gpu, dtype=torch.bfloat16)
    _gather_seg(gpu, nb, terms, part_in, csum_in, part_out, csum_out, blocks[-1], addend, out)
    for j in range(nb - 1):
        want = np.zeros((n, d)) if part_in[j] is None else np64(part_in[j])
        wc = np.zeros(n) if csum_in[j] is None else np64(csum_in[j])
        for c, G, qf in recs:
            want = want + c[:, j, 0:1] * G + c[:, j, 1:2] * qf[None, :]
            wc = wc + c[:, j, 2]
        check_grad(part_out[j], want, torch.bfloat16, f"block {j} running sum")
        err = np.abs(np64(csum_out[j]) - wc)
        assert (err <= 1e-5 * np.abs(wc) + 1e-6 * np.abs(wc).max() + 1e-30).all(), f"block {j} x-coefficient sum"
    last = nb - 1
    want = sum(gr[last] for gr in grads) + np64(addend)
    if part_in[last] is not None:
        want = want + np64(part_in[last]) + np64(csum_in[last])[:, None] * np64(blocks[last])
    check_grad(out, want, torch.bfloat16, "last block's gradient")


def test_gather_seg_more_terms_than_one_launch(gpu):
    # 52 points over 2 blocks: two launches, the second continuing from the
    # first's running sums (the last block's x-coefficient sum in the scratch
    # csum_out[last]); the last block's gradient against the oracle's sum, the
    # bar widened by half an ulp of the running sum the first launch rounds
    from .test_gpu_backward import bf16_ulp

    n, d, nb, P = 256, 3072, 2, 52
    g = torch.Generator(device=gpu).manual_seed(91)
    blocks = [torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16) for _ in range(nb)]
    terms, dx, first = [], [], np.zeros((n, d))
    for p in range(P):
        own = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
        q = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
        gout = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
        gain = torch.ones(d, device=gpu, dtype=torch.bfloat16)
        _, coef, qfold, _, _ = _defer(gpu, blocks + [own], q, gain, gout)
        terms.append((gout, coef, qfold))
        if p < _capi.SEG_MAX_TERMS:  # the running sum the first launch rounds (without its x term)
            c = coef.double().cpu().numpy()
            first += c[:, 1, 0:1] * np64(gout) + c[:, 1, 1:2] * np64(qfold)[None, :]
        dx.append(O.route_backward(np.stack([np64(t) for t in blocks + [own]]),
                                   O.fold_query(np64(q), np64(gain), "bf16"), 1e-5, np64(gout), None)["dx"])
    part_out = [torch.empty((n, d), device=gpu, dtype=torch.bfloat16)]
    csum_out = [torch.empty(n, device=gpu), torch.empty(n, device=gpu)]
    out = torch.empty((n, d), device=gpu, dtype=torch.bfloat16)
    _capi.route_bwd_gather_seg(
        nb, n, d, BF, P, _capi.pointer_array([t[0].data_ptr() for t in terms]), d,
        _capi.pointer_array([t[1].data_ptr() for t in terms]), _capi.int64_array([4 * t[1].shape[1] for t in terms]),
        _capi.pointer_array([t[2].data_ptr() for t in terms]), _capi.pointer_array([None, None]),
        _capi.pointer_array([None, None]), _capi.pointer_array([part_out[0].data_ptr(), out.data_ptr()]),
        _capi.pointer_array([c.data_ptr() for c in csum_out]), blocks[1].data_ptr(), d, None, d,
        torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    want = sum(x[1] for x in dx)
    err = np.abs(np64(out) - want)
    bar = bf16_ulp(want) + 0.5 * bf16_ulp(first) + 1e-3 * np.abs(want).max()
    assert (err <= bar).all(), f"{P} terms: worst err {err.max():.3e}"
