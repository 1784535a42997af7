"""Parity of the gfx950 kernels against the float64 oracle (GPU).

Tolerances (stated per the routing contract):
* fp32 outputs:   |out - ref| <= 1e-5 * |ref| + 1e-6 * max|ref|   (allclose form)
* routing weights: |w - w_ref| <= 1e-5 absolute (fp32 arithmetic on the same inputs)
* bf16 outputs:   |out - ref| <= max(2e-2, 1 bf16 ulp of |ref|), ref = float64
  oracle on the identical bf16 input values.  For |ref| >= 8 one bf16 ulp is
  already 0.0625 > 2e-2, so a correctly rounded result cannot meet 2e-2 there;
  the ulp term keeps the bar at "one rounding step", and the fraction of
  elements equal to the correctly rounded oracle is asserted as well.
The oracle runs on every row for small shapes and on sampled rows (plus
token 0 and the last token) at the full BASELINE sizes, where size-independent
properties (weights sum to 1, output inside the sources' per-element hull)
are checked on every row.
"""

import math

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops, workloads
from kotodama_amd.engine import AttnResRouter, BlockArena
from kotodama_amd.flash_attn_res import (
    phase_1_batched_attention_forward_with_aux,
    phase_1_batched_attention_triton_op,
    phase_2_online_softmax_merge_forward_with_aux,
)
from kotodama_amd.schedule import AttnResSchedule
from oracle import attnres_oracle as O

pytestmark = pytest.mark.gpu


class Norm(torch.nn.Module):
    def __init__(self, weight, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(weight, requires_grad=False)
        self.eps = eps


@pytest.fixture(params=["workgroup", "stream"])
def policy(request, gpu):
    """Run the test with each kernel family (stream falls back where the shape does not allow it)."""
    code = {"workgroup": _capi.POLICY_WORKGROUP, "stream": _capi.POLICY_STREAM}[request.param]
    prev = _capi.set_kernel_policy(code)
    yield request.param
    _capi.set_kernel_policy(prev)


def np64(t):
    return t.detach().float().cpu().double().numpy()


def bf16_ulp(x):
    a = np.abs(x)
    e = np.floor(np.log2(np.maximum(a, 2.0**-126)))
    return 2.0 ** (e - 7)


def check_bf16(out, ref, label, exact_frac=0.98):
    """bf16 bar: |err| <= max(2e-2, 1 ulp of |ref|) and >= exact_frac equal to the correctly rounded
    oracle; where |ref| >= 4 (one ulp >= 2^-5 > 2e-2, so the ulp term sets that bar) the result must
    also be the correct rounding of an fp32 evaluation: |err| <= 0.5 ulp + 2^-16 * max|ref|.  The
    second term bounds an fp32 evaluation's own error (S products and sums at 2^-24 relative plus
    the softmax's exp rounding, far below 2^-16 of the largest magnitude), which can put the fp32
    value on the other side of a rounding midpoint than the float64 one.  Prints the share of
    elements equal to the correctly rounded oracle, the worst error in ulps, and the worst error in
    ulps where |ref| >= 4."""
    out = np64(out)
    err = np.abs(out - ref)
    ulp = bf16_ulp(ref)
    tol = np.maximum(2e-2, ulp)
    bad = err > tol
    assert not bad.any(), f"{label}: {bad.sum()} elements over tolerance, worst err {err.max():.3e}"
    same = np.mean(out == O.bf16_round(ref))
    big = np.abs(ref) >= 4.0
    worst_big = float((err[big] / ulp[big]).max()) if big.any() else 0.0
    print(f"[bf16] {label}: {same:.5f} equal to the rounded oracle; worst {float((err / ulp).max()):.2f} ulp; "
          f"where |ref| >= 4 ({int(big.sum())} elements) worst {worst_big:.2f} ulp", flush=True)
    if big.any():
        half = 0.5 * ulp[big] + 2.0**-16 * float(np.abs(ref).max())
        over = err[big] > half
        assert not over.any(), (f"{label}: {int(over.sum())} elements with |ref| >= 4 are not correctly rounded "
                                f"(worst {worst_big:.3f} ulp)")
    assert same >= exact_frac, f"{label}: only {same:.4f} of elements equal the correctly rounded oracle"


def check_f32(out, ref, label):
    out = np64(out)
    err = np.abs(out - ref)
    tol = 1e-5 * np.abs(ref) + 1e-6 * np.abs(ref).max()
    assert (err <= tol).all(), f"{label}: worst rel err {(err / (np.abs(ref) + 1e-30)).max():.3e}"


def check_weights(w, ref, label, atol=1e-5):
    err = np.abs(np64(w) - ref).max()
    assert err <= atol, f"{label}: weights err {err:.3e}"


def sample_rows(n, k, seed=0):
    rng = np.random.default_rng(seed)
    idx = set(rng.choice(n, size=min(k, n), replace=False).tolist())
    idx.update([0, n - 1])
    return torch.tensor(sorted(idx), dtype=torch.long)


def oracle_rows(pool, s, rows, qw, eps):
    """Oracle on selected token rows of the first s slots of a (max_S, B, T, D) pool."""
    d = pool.shape[-1]
    src = pool[:s].reshape(s, -1, d)[:, rows.to(pool.device)]
    return O.route(np64(src), qw, eps)


def fold(q, g, dtype):
    return O.fold_query(np64(q), np64(g), "bf16" if dtype == torch.bfloat16 else "f32")


# ------------------------------------------------------------ config 1 --


def test_cfg1_fp32_weights_and_outputs(gpu):
    w = workloads.get("cfg1")
    g = torch.Generator(device=gpu).manual_seed(1)
    buf = torch.randn((3, 1, 512, 3072), generator=g, device=gpu, dtype=torch.float32)
    query = torch.randn((3072,), generator=g, device=gpu) * 0.02
    gain = torch.ones(3072, device=gpu)
    out, wts, lse = kotodama_amd.route_weights(buf, 3, query, Norm(gain, w.eps))
    torch.cuda.synchronize()
    ref = O.route(np64(buf).reshape(3, 512, 3072), fold(query, gain, torch.float32), w.eps)
    assert out.dtype == torch.float32 and out.shape == (1, 512, 3072)
    assert wts.shape == (3, 1, 512)
    check_weights(wts.reshape(3, 512), ref["weights"][0], "cfg1")
    check_f32(out.reshape(512, 3072), ref["out"][0], "cfg1")
    np.testing.assert_allclose(np64(lse).reshape(-1), ref["lse"][0], atol=1e-5)
    # the drop-in returns the same tensor values
    h = kotodama_amd.route_static(buf, query, Norm(gain, w.eps), torch.ones(3, dtype=torch.bool, device=gpu), 3)
    assert torch.equal(h, out)


# ------------------------------------------------- route_static, all S --


@pytest.mark.parametrize("d", [3072, 4096, 512])
def test_route_static_every_source_count_bf16(gpu, policy, d):
    max_s = 9 if d == 4096 else 8
    g = torch.Generator(device=gpu).manual_seed(d)
    scales = torch.exp(torch.empty(max_s, device=gpu).uniform_(math.log(0.1), math.log(10), generator=g))
    buf = (torch.randn((max_s, 2, 96, d), generator=g, device=gpu) * scales.view(-1, 1, 1, 1)).to(torch.bfloat16)
    query = (torch.randn(d, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    gain = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
    norm = Norm(gain, 1e-5)
    qw = fold(query, gain, torch.bfloat16)
    for s in range(1, max_s + 1):
        mask = torch.zeros(max_s, dtype=torch.bool, device=gpu)
        mask[:s] = True
        with torch.no_grad():
            h = kotodama_amd.route_static(buf, query, norm, mask, s)
            h_mask = kotodama_amd.route_static(buf, query, norm, mask)  # num_active=0: mask read on the host
        ref = O.route(np64(buf[:s]).reshape(s, -1, d), qw, 1e-5)["out"][0].reshape(2, 96, d)
        assert h.dtype == torch.bfloat16 and h.shape == (2, 96, d)
        check_bf16(h, ref, f"d={d} S={s}")
        assert torch.equal(h, h_mask)


def test_route_static_non_prefix_mask_and_list_shim(gpu, policy):
    d = 3072
    g = torch.Generator(device=gpu).manual_seed(7)
    buf = torch.randn((6, 1, 64, d), generator=g, device=gpu).to(torch.bfloat16)
    query = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    norm = Norm(torch.ones(d, device=gpu, dtype=torch.bfloat16), 1e-5)
    mask = torch.tensor([True, False, True, True, False, True], device=gpu)
    h = kotodama_amd.route_static(buf, query, norm, mask)
    sel = [0, 2, 3, 5]
    ref = O.route(np64(buf[sel]).reshape(4, -1, d), fold(query, norm.weight, torch.bfloat16), 1e-5)["out"][0]
    check_bf16(h.reshape(-1, d), ref, "non-prefix mask")
    h2 = kotodama_amd.block_attn_res_from_list([buf[i] for i in sel], query, norm)
    assert torch.equal(h, h2)


def test_list_of_separate_allocations(gpu, policy):
    # nine sources in separate allocations, passed in an order that is not
    # equally spaced: the streaming family addresses them through its pointer table
    d, n = 4096, 96
    g = torch.Generator(device=gpu).manual_seed(17)
    srcs = [(torch.randn((2, n // 2, d), generator=g, device=gpu) * (0.5 + 0.3 * i)).to(torch.bfloat16)
            for i in range(9)]
    order = [3, 0, 8, 1, 7, 2, 6, 4, 5]
    lst = [srcs[i] for i in order]
    query = (torch.randn(d, generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    norm = Norm((1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16), 1e-5)
    with torch.no_grad():
        h = kotodama_amd.block_attn_res_from_list(lst, query, norm)
    ref = O.route(np.stack([np64(t).reshape(-1, d) for t in lst]), fold(query, norm.weight, torch.bfloat16),
                  1e-5)["out"][0]
    check_bf16(h.reshape(-1, d), ref, "separate allocations")


def test_batched_queries_wide_rows_fp32_queries(gpu):
    # 8 fp32 queries at D=8192 (two chunks per thread): every query's output,
    # lse, weights, logits and the shared inverse RMS must match
    d, n, S, Q = 8192, 40, 5, 8
    g = torch.Generator(device=gpu).manual_seed(19)
    buf = torch.randn((S, 1, n, d), generator=g, device=gpu).to(torch.bfloat16)
    qs = torch.randn((Q, d), generator=g, device=gpu) * 0.03
    out, w, lse, inv, lg = ops.route(buf, S, qs, None, 1e-5, torch.bfloat16, True, True)
    ref = O.route(np64(buf).reshape(S, n, d), np64(qs), 1e-5)
    for q in range(Q):
        check_bf16(out[q].reshape(n, d), ref["out"][q], f"query {q}")
        check_weights(w[q].reshape(S, n), ref["weights"][q], f"weights {q}")
        np.testing.assert_allclose(np64(lse[q]).reshape(n), ref["lse"][q], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(np64(lg[q]).reshape(n, S), ref["logits"][q], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(np64(inv).reshape(n, S), ref["inv_rms"], rtol=1e-5)


def route_kernel(s, n, d, q):
    import ctypes

    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_kernel_name", _capi.lib().attnres_route_kernel_name(s, n, d, 1, 1, 1, q, 0, 1, buf, 128))
    return buf.value.decode()


def test_kernel_name_query_follows_the_launch_choice(gpu):
    # the name query and the launch share one choice: streaming variants by mode and
    # source spacing, and the workgroup kernel for a one-source accumulate
    import ctypes

    def name(s, n, d, fused, spaced):
        buf = ctypes.create_string_buffer(128)
        _capi.check("attnres_route_kernel_name",
                    _capi.lib().attnres_route_kernel_name(s, n, d, 1, 1, 1, 1, fused, spaced, buf, 128))
        return buf.value.decode()

    assert name(4, 32768, 3072, 0, 1) == "attnres_stream_bf_d2_obf_c6_plain"
    assert name(4, 32768, 3072, 0, 0) == "attnres_stream_bf_d2_obf_c6_table"
    assert name(4, 32768, 3072, 1, 1) == "attnres_stream_bf_d2_obf_c6_fused"
    assert name(2, 32768, 3072, 2, 1) == "attnres_stream_bf_d2_obf_c6_fused"
    one = name(1, 32768, 3072, 1, 1)  # S = 1 accumulate: the workgroup kernel
    assert one.startswith("attnres_route_bf_d2_s1_v") and one.endswith("_q1"), one
    assert name(1, 32768, 3072, 0, 1) == "attnres_stream_bf_d2_obf_c6_plain"
    assert name(9, 256, 4096, 1, 1) == "attnres_route_bf_d2_s9_v1_q1"  # decode rows
    buf = ctypes.create_string_buffer(128)
    assert _capi.lib().attnres_route_kernel_name(2, 64, 512, 1, 1, 1, 1, 3, 1, buf, 128) == _capi.ERR_ARG


@pytest.mark.parametrize("d,n,queries", [(1024, 24, (2, 9)), (8192, 12, (3, 8)), (3072, 600, (5,)), (520, 7, (4,)),
                                         (8184, 5, (3,))])
def test_batched_query_kernel_every_source_count(gpu, d, n, queries):
    # bf16 folded queries (the serving engine's phase 1): the batched-query
    # kernel, groups of 8/4/2 queries with a ragged last group, one chunk per
    # thread (d=1024; d=520 leaves 63 idle lanes past the row end), two
    # (d=8192; d=3072 with enough rows; d=8184: the last thread's second
    # chunk is past the row end); every output against the oracle
    g = torch.Generator(device=gpu).manual_seed(d + n)
    for S in range(1, 17):
        if d == 3072 and S not in (1, 6, 7, 13):
            continue
        scales = torch.exp(torch.empty(S, device=gpu).uniform_(math.log(0.2), math.log(5), generator=g))
        buf = (torch.randn((S, n, d), generator=g, device=gpu) * scales.view(-1, 1, 1)).to(torch.bfloat16)
        for Q in queries:
            pq = (torch.randn((Q, d), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
            name = route_kernel(S, n, d, Q)
            assert name.endswith("_qg"), name
            out, w, lse, inv, lg = ops.route(buf, S, pq, None, 1e-5, torch.bfloat16, True, True)
            ref = O.route(np64(buf), np64(pq), 1e-5)
            for q in range(Q):
                label = f"S={S} Q={Q} q={q} {name}"
                check_bf16(out[q], ref["out"][q], label)
                check_weights(w[q], ref["weights"][q], label)
                np.testing.assert_allclose(np64(lse[q]), ref["lse"][q], rtol=1e-5, atol=1e-5)
                np.testing.assert_allclose(np64(lg[q]).reshape(n, S), ref["logits"][q], rtol=1e-4, atol=1e-4)
            np.testing.assert_allclose(np64(inv).reshape(n, S), ref["inv_rms"], rtol=1e-5)


@pytest.mark.parametrize("S,Q", [(3, 8), (7, 5)])
def test_batched_query_kernel_many_rows_per_workgroup(gpu, S, Q):
    # 12288 rows of 512 elements: more rows than the resident grid holds
    # workgroups, so every workgroup walks several rows (next-row loads,
    # double-buffered reduction rows); rows sampled from start, middle and end
    d, n = 512, 12288
    g = torch.Generator(device=gpu).manual_seed(101 + S)
    scales = torch.exp(torch.empty(S, device=gpu).uniform_(math.log(0.3), math.log(4), generator=g))
    buf = (torch.randn((S, n, d), generator=g, device=gpu) * scales.view(-1, 1, 1)).to(torch.bfloat16)
    pq = (torch.randn((Q, d), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    name = route_kernel(S, n, d, Q)
    assert name.endswith("_qg"), name
    print(f"batched-query kernel over {n} rows S={S} Q={Q} {name}", flush=True)
    out, w, lse, _, _ = ops.route(buf, S, pq, None, 1e-5, torch.bfloat16, True, False)
    rows = np.concatenate([np.arange(0, 256), np.arange(n // 2 - 128, n // 2 + 128), np.arange(n - 256, n)])
    ref = O.route(np64(buf)[:, rows], np64(pq), 1e-5)
    for q in range(Q):
        label = f"S={S} Q={Q} q={q} rows sampled"
        check_bf16(out[q][rows], ref["out"][q], label)
        check_weights(w[q][:, rows], ref["weights"][q], label)
        np.testing.assert_allclose(np64(lse[q])[rows], ref["lse"][q], rtol=1e-5, atol=1e-5)


def test_batched_query_kernel_falls_back_past_lds(gpu):
    # 11 queries of 8192 elements (176 KiB of staged queries) exceed one
    # workgroup's LDS: the per-query kernel runs, with the same results
    d, n, S, Q = 8192, 10, 4, 11
    assert route_kernel(S, n, d, Q).endswith("_qn")
    g = torch.Generator(device=gpu).manual_seed(23)
    buf = torch.randn((S, n, d), generator=g, device=gpu).to(torch.bfloat16)
    pq = (torch.randn((Q, d), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    out, w, lse, _, _ = ops.route(buf, S, pq, None, 1e-5, torch.bfloat16, True, False)
    ref = O.route(np64(buf), np64(pq), 1e-5)
    for q in range(Q):
        check_bf16(out[q], ref["out"][q], f"fallback q={q}")
        check_weights(w[q], ref["weights"][q], f"fallback q={q}")
    o8, w8, _, _, _ = ops.route(buf, S, pq[:8], None, 1e-5, torch.bfloat16, True, False)
    assert route_kernel(S, n, d, 8).endswith("_qg")
    for q in range(8):
        check_bf16(o8[q], ref["out"][q], f"batched q={q}")
        check_weights(w8[q], ref["weights"][q], f"batched q={q}")


# ------------------------------------------------------- edge cases --


def test_zero_sources_is_nan_and_one_source_is_exact_copy(gpu, policy):
    d = 1024
    buf = torch.randn((4, 3, 5, d), device=gpu).to(torch.bfloat16)
    q = torch.randn(d, device=gpu).to(torch.bfloat16)
    out0, _, lse0, _, _ = ops.route(buf, 0, q, None, 1e-5, torch.bfloat16, True, False)
    assert torch.isnan(out0).all() and torch.isnan(lse0).all()
    out1, w1, _, _, _ = ops.route(buf, 1, q, None, 1e-5, torch.bfloat16, True, False)
    assert torch.equal(out1[0], buf[0]) and torch.all(w1 == 1)
    f = buf.float()
    out1f, _, _, _, _ = ops.route(f, 1, q.float(), None, 1e-5, torch.float32, False, False)
    assert torch.equal(out1f[0], f[0])


@pytest.mark.parametrize("n,d,s", [(1, 4096, 9), (7, 3072, 5), (1000, 520, 3), (33, 8, 2), (5, 64, 16), (300, 8192, 4)])
def test_ragged_and_extreme_shapes(gpu, policy, n, d, s):
    g = torch.Generator(device=gpu).manual_seed(n * 31 + d + s)
    buf = torch.randn((s, n, d), generator=g, device=gpu).to(torch.bfloat16)
    q = (torch.randn(d, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    out, w, lse, inv, lg = ops.route(buf, s, q, None, 1e-5, torch.bfloat16, True, True)
    ref = O.route(np64(buf), np64(q), 1e-5)
    check_bf16(out[0], ref["out"][0], f"n={n} d={d} s={s}")
    check_weights(w[0], ref["weights"][0], "ragged")
    np.testing.assert_allclose(np64(inv), ref["inv_rms"], rtol=2e-6)
    np.testing.assert_allclose(np64(lg[0]), ref["logits"][0], rtol=1e-4, atol=1e-4)


def test_fp32_sources_and_mixed_parameter_dtypes(gpu, policy):
    d, n = 2048, 64
    g = torch.Generator(device=gpu).manual_seed(11)
    buf = torch.randn((4, n, d), generator=g, device=gpu)
    q32 = torch.randn(d, generator=g, device=gpu) * 0.05
    g32 = 1 + 0.1 * torch.randn(d, generator=g, device=gpu)
    # fp32 sources, fp32 params -> fp32 out
    h = kotodama_amd.route_static(buf, q32, Norm(g32, 1e-5), torch.ones(4, dtype=torch.bool, device=gpu), 4)
    ref = O.route(np64(buf), fold(q32, g32, torch.float32), 1e-5)["out"][0]
    check_f32(h, ref, "f32/f32")
    # bf16 sources with fp32 params (autocast training): the einsum branch promotes to fp32
    hb = kotodama_amd.route_static(buf.to(torch.bfloat16), q32, Norm(g32, 1e-5),
                                   torch.ones(4, dtype=torch.bool, device=gpu), 4)
    assert hb.dtype == torch.float32
    refb = O.route(np64(buf.to(torch.bfloat16)), fold(q32, g32, torch.float32), 1e-5)["out"][0]
    check_f32(hb, refb, "bf16 src / f32 params")
    # fp32 sources with bf16 params: fold in bf16, math in fp32, fp32 out
    qb, gb = q32.to(torch.bfloat16), g32.to(torch.bfloat16)
    hf = kotodama_amd.route_static(buf, qb, Norm(gb, 1e-5), torch.ones(4, dtype=torch.bool, device=gpu), 4)
    assert hf.dtype == torch.float32
    check_f32(hf, O.route(np64(buf), fold(qb, gb, torch.bfloat16), 1e-5)["out"][0], "f32 src / bf16 params")


def test_host_checked_errors_raise(gpu):
    buf = torch.randn((17, 2, 64), device=gpu).to(torch.bfloat16)
    q = torch.randn(64, device=gpu).to(torch.bfloat16)
    with pytest.raises(_capi.AttnResError, match="UNSUPPORTED"):
        ops.route(buf, 17, q, None, 1e-5, torch.bfloat16, False, False)
    odd = torch.randn((2, 2, 12), device=gpu).to(torch.bfloat16)
    with pytest.raises(_capi.AttnResError, match="UNSUPPORTED"):
        ops.route(odd, 2, torch.randn(12, device=gpu).to(torch.bfloat16), None, 1e-5, torch.bfloat16, False, False)
    with pytest.raises(TypeError):
        ops.route(buf.half(), 2, q.half(), None, 1e-5, torch.float16, False, False)


def test_forward_only_paths_on_gpu(gpu):
    # route_static is differentiable; the weights helper and the arena engine are not
    buf = torch.randn((2, 1, 4, 64), device=gpu)
    q = torch.zeros(64, device=gpu, requires_grad=True)
    norm = Norm(torch.ones(64, device=gpu), 1e-5)
    out = kotodama_amd.route_static(buf, q, norm, torch.ones(2, dtype=torch.bool, device=gpu), 2)
    assert out.requires_grad
    with pytest.raises(NotImplementedError, match="forward-only"):
        kotodama_amd.route_weights(buf, 2, q, norm)
    arena = torch.zeros((3, 1, 4, 64), device=gpu)
    with pytest.raises(NotImplementedError, match="forward-only"):
        ops.check_forward_only(arena, q)


# ------------------------------------------------ full-size configs --


def _full_config_check(gpu, name, seed, calls, rows=384):
    w = workloads.get(name)
    pool = workloads.make_pool(w, gpu, seed)
    q, gn = workloads.make_params(w, gpu, seed, len(calls))
    n = w.tokens
    idx = sample_rows(n, rows, seed)
    for j, s in enumerate(calls):
        norm = Norm(gn[j], w.eps)
        out, wts, lse = kotodama_amd.route_weights(pool, s, q[j], norm)
        # size-independent properties on every row
        wsum = wts.sum(0)
        assert torch.allclose(wsum, torch.ones_like(wsum), atol=1e-5), f"{name} S={s}: weights do not sum to 1"
        lo = pool[:s].float().amin(0)
        hi = pool[:s].float().amax(0)
        o = out.float()
        slack = 1e-2 * torch.maximum(lo.abs(), hi.abs()) + 1e-3
        assert bool(((o >= lo - slack) & (o <= hi + slack)).all()), f"{name} S={s}: output outside the source hull"
        del lo, hi, o
        ref = oracle_rows(pool, s, idx, fold(q[j], gn[j], w.dtype), w.eps)
        check_bf16(out.reshape(n, -1)[idx.to(gpu)], ref["out"][0], f"{name} S={s}")
        check_weights(wts.reshape(s, n)[:, idx.to(gpu)], ref["weights"][0], f"{name} S={s}")
    del pool
    torch.cuda.empty_cache()


# (workload, source counts): the streaming kernel's launch shapes at full size -
# four waves per workgroup with batches of 6 output rows staged in LDS plus 4
# held in registers (3B, S >= 3), no staging (S = 2), three waves with 6 + 2
# rows of 8 KiB (8B, S = 9); the last batch of most waves is partial and ends
# in the LDS or in the register rows
STREAM_FULL = [("cfg2", (2, 3, 4, 5, 6, 8)), ("cfg3", (9,))]


@pytest.mark.parametrize("name,calls", STREAM_FULL, ids=[c[0] for c in STREAM_FULL])
def test_streaming_kernel_matches_workgroup_kernel_every_row(gpu, name, calls):
    # every element of every row: the row-per-wave streaming kernel (online
    # softmax, staged and batched output stores) against the row-per-workgroup
    # kernel (two-pass softmax, direct stores), two independent fp32
    # computations of the same rows.  Each is its bf16 rounding (half an ulp)
    # of a fp32 sum whose own error is below S * 2^-24 * max_s |x_s|, so they
    # agree to one ulp plus 2^-16 * max_s |x_s| (the second term matters only
    # where the sum cancels far below its sources), and >= 99% of elements are
    # equal; the oracle checks both on sampled rows elsewhere
    w = workloads.get(name)
    pool = workloads.make_pool(w, gpu, 7)
    q, gn = workloads.make_params(w, gpu, 7, len(calls))
    for j, s in enumerate(calls):
        print(f"stream vs workgroup {name} S={s} rows={w.tokens}", flush=True)
        outs = []
        for pol in (_capi.POLICY_STREAM, _capi.POLICY_WORKGROUP):
            prev = _capi.set_kernel_policy(pol)
            try:
                with torch.no_grad():
                    outs.append(ops.route_call(pool, s, q[j], gn[j], w.eps, w.dtype)[0][0].float())
            finally:
                _capi.set_kernel_policy(prev)
        torch.cuda.synchronize()
        a, b = outs
        xmax = pool[:s].abs().amax(0).float().reshape(b.shape)
        tol = torch.exp2(torch.floor(torch.log2(torch.clamp(b.abs(), min=2.0**-126))) - 7) + 2.0**-16 * xmax
        excess = ((a - b).abs() / tol).max().item()
        same = (a == b).float().mean().item()
        print(f"  max |diff| / tol {excess:.3f}, {same:.5f} of elements equal", flush=True)
        assert excess <= 1.0, f"{name} S={s}: streaming and workgroup kernels differ by {excess:.2f}x the bar"
        assert same >= 0.99, f"{name} S={s}: only {same:.4f} of elements equal"
        del outs, a, b, tol, xmax
    del pool
    torch.cuda.empty_cache()


def _stream_vs_workgroup(pool, s, q, gn, eps, label):
    """Every element: streaming kernel against the workgroup kernel, at the bar of the full-size test above."""
    outs = []
    for pol in (_capi.POLICY_STREAM, _capi.POLICY_WORKGROUP):
        prev = _capi.set_kernel_policy(pol)
        try:
            with torch.no_grad():
                outs.append(ops.route_call(pool, s, q, gn, eps, torch.bfloat16)[0][0].float())
        finally:
            _capi.set_kernel_policy(prev)
    torch.cuda.synchronize()
    a, b = outs
    xmax = pool[:s].abs().amax(0).float().reshape(b.shape)
    tol = torch.exp2(torch.floor(torch.log2(torch.clamp(b.abs(), min=2.0**-126))) - 7) + 2.0**-16 * xmax
    excess = ((a - b).abs() / tol).max().item()
    same = (a == b).float().mean().item()
    print(f"  {label}: max |diff| / tol {excess:.3f}, {same:.5f} of elements equal", flush=True)
    assert excess <= 1.0, f"{label}: streaming and workgroup kernels differ by {excess:.2f}x the bar"
    assert same >= 0.99, f"{label}: only {same:.4f} of elements equal"


# (hidden, S, waves per workgroup, batch rows: LDS + registers) - row counts
# chosen from the device's CU count so that every wave's last batch is either
# exactly full or ends in the register-held rows (the full-size shapes end
# theirs in the LDS rows)
BATCH_TAILS = [(3072, 3, 4, 6 + 4), (3072, 6, 4, 6 + 4), (4096, 5, 3, 6 + 2)]


@pytest.mark.parametrize("d,s,waves,batch", BATCH_TAILS, ids=[f"d{c[0]}_s{c[1]}" for c in BATCH_TAILS])
def test_streaming_batches_ending_in_register_rows(gpu, d, s, waves, batch):
    ncu = torch.cuda.get_device_properties(gpu).multi_processor_count
    nw = ncu * waves
    g = torch.Generator(device=gpu).manual_seed(d + s)
    q = (torch.randn(d, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    gn = (1 + 0.1 * torch.randn(d, generator=g, device=gpu)).to(torch.bfloat16)
    # half the waves get batch - 1 rows, half a full batch; then batch - 3 / batch - 2
    for n in (nw * (batch - 1) + nw // 2, nw * (batch - 3) + nw // 2):
        scales = torch.exp(torch.empty(s, device=gpu).uniform_(math.log(0.5), math.log(4.0), generator=g))
        pool = (torch.randn((s, 1, n, d), generator=g, device=gpu) * scales.view(-1, 1, 1, 1)).to(torch.bfloat16)
        print(f"stream batch tails d={d} S={s} rows={n} (rows per wave {n // nw}-{n // nw + 1})", flush=True)
        _stream_vs_workgroup(pool, s, q, gn, 1e-5, f"d={d} S={s} rows={n}")
        del pool
    torch.cuda.empty_cache()


def test_cfg3_8b_deepest_routing_full_size(gpu):
    _full_config_check(gpu, "cfg3", 3, (9, 9))


def test_cfg2_3b_every_source_count_full_size(gpu):
    _full_config_check(gpu, "cfg2", 2, tuple(range(1, 9)), rows=256)


def test_cfg5_dd_blocks_bos_sink_full_size(gpu):
    w = workloads.get("cfg5")
    assert w.schedule.max_sources == 7 and max(w.calls) == 7 and sum(w.calls) == 267
    pool = workloads.make_pool(w, gpu, 5)
    q, gn = workloads.make_params(w, gpu, 5, 2)
    for j, s in enumerate((4, 7)):
        out, wts, _ = kotodama_amd.route_weights(pool, s, q[j], Norm(gn[j], w.eps))
        # every BOS row (token 0 of each sequence, 20x magnitude) checked exactly
        bos = torch.arange(w.batch, device=gpu) * w.seq
        ref = O.route(np64(pool[:s].reshape(s, -1, w.hidden)[:, bos]), fold(q[j], gn[j], w.dtype), w.eps)
        check_bf16(out.reshape(-1, w.hidden)[bos], ref["out"][0], f"cfg5 BOS S={s}")
        check_weights(wts.reshape(s, -1)[:, bos], ref["weights"][0], f"cfg5 BOS S={s}")
    del pool
    _full_config_check(gpu, "cfg5", 5, (7,), rows=256)


# ------------------------------------------------ decode / arena path --


def test_cfg4_decode_step_block_arena(gpu, policy):
    w = workloads.get("cfg4")
    sched = w.schedule
    L = sched.num_layers
    g = torch.Generator(device=gpu).manual_seed(4)
    embed = torch.randn((w.batch, 1, w.hidden), generator=g, device=gpu).to(torch.bfloat16)
    deltas = workloads.make_deltas(w, gpu, 4, 2 * L)
    q, gn = workloads.make_params(w, gpu, 4, sched.num_points)
    router = AttnResRouter(sched, list(q), list(gn), w.eps)
    outs = []

    def sublayer(j, h):
        outs.append(h.clone())
        return deltas[j]

    final = router.forward(embed, sublayer)
    outs.append(final)
    torch.cuda.synchronize()
    qws = [fold(q[j], gn[j], w.dtype) for j in range(sched.num_points)]
    ref = O.block_forward(
        np64(embed).reshape(w.batch, w.hidden),
        [np64(deltas[j]).reshape(w.batch, w.hidden) for j in range(2 * L)],
        qws, w.eps, L, sched.boundary_set, dtype="bf16",
    )
    assert len(outs) == sched.num_points == 65
    for j in range(sched.num_points):
        check_bf16(outs[j].reshape(w.batch, w.hidden), ref["outs"][j], f"decode point {j}")


def test_block_arena_state_and_fp32(gpu, policy):
    # fp32 arena, small: the partial written back and the commit bookkeeping
    d, n = 256, 10
    sched = AttnResSchedule.build(3, boundaries=[0, 2])
    g = torch.Generator(device=gpu).manual_seed(12)
    embed = torch.randn((n, d), generator=g, device=gpu)
    deltas = torch.randn((6, n, d), generator=g, device=gpu)
    q = torch.randn((7, d), generator=g, device=gpu) * 0.2
    arena = BlockArena(sched.max_sources, (n,), d, torch.float32, gpu)
    router = AttnResRouter(sched, list(q), [None] * 7, 1e-5)
    outs = []

    def sublayer(j, h):
        outs.append(h.clone())
        return deltas[j]

    outs.append(router.forward(embed, sublayer, arena=arena))
    ref = O.block_forward(np64(embed), [np64(deltas[j]) for j in range(6)], [np64(q[j]) for j in range(7)], 1e-5, 3,
                          {0, 2}, dtype="f32")
    assert arena.n_committed == 2
    check_f32(arena.committed[0], ref["committed"][0], "committed 0")
    check_f32(arena.committed[1], ref["committed"][1], "committed 1")
    check_f32(arena.partial, ref["partial"], "partial")
    for j in range(7):
        check_f32(outs[j], ref["outs"][j], f"arena point {j}")


@pytest.mark.parametrize("d", [512, 3072, 4096])
def test_block_arena_accumulate_without_first_boundary(gpu, policy, d):
    # boundaries not including layer 0: the first pre-MLP point accumulates into
    # the partial with S = 1 (routed to the workgroup kernel even under the
    # streaming policy), later points accumulate with S >= 2 (streaming kernel,
    # one delta buffer shared by the two pipeline slots), bf16, rows of whole KiB
    n = 40
    sched = AttnResSchedule.build(5, boundaries=[1, 3])
    g = torch.Generator(device=gpu).manual_seed(13)
    embed = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
    deltas = torch.randn((10, n, d), generator=g, device=gpu).to(torch.bfloat16)
    q = (torch.randn((11, d), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    gn = (1 + 0.1 * torch.randn((11, d), generator=g, device=gpu)).to(torch.bfloat16)
    router = AttnResRouter(sched, list(q), list(gn), 1e-5)
    outs = []

    def sublayer(j, h):
        outs.append(h.clone())
        return deltas[j]

    outs.append(router.forward(embed, sublayer))
    assert sched.active_counts[1] == 1 and not sched.commit_before[1]
    qws = [fold(q[j], gn[j], torch.bfloat16) for j in range(11)]
    ref = O.block_forward(np64(embed), [np64(deltas[j]) for j in range(10)], qws, 1e-5, 5, {1, 3}, dtype="bf16")
    for j in range(11):
        check_bf16(outs[j], ref["outs"][j], f"arena point {j}")


# ------------------------------------------------- phase 1 / phase 2 --


def test_phase1_batched_queries_and_phase2_merge(gpu):
    d = 4096
    g = torch.Generator(device=gpu).manual_seed(21)
    blocks = torch.randn((5, 2, 200, d), generator=g, device=gpu).to(torch.bfloat16)
    pq = (torch.randn((4, d), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    out, lse, inv, lg = phase_1_batched_attention_forward_with_aux(blocks, pq, 1e-5, 5)
    assert out.shape == (4, 2, 200, d) and out.dtype == torch.bfloat16 and lse.shape == (4, 2, 200)
    assert inv.shape == (2, 200, 5) and lg.shape == (4, 2, 200, 5)
    ref = O.route(np64(blocks).reshape(5, -1, d), np64(pq), 1e-5)
    for i in range(4):
        check_bf16(out[i].reshape(-1, d), ref["out"][i], f"phase1 q{i}")
        np.testing.assert_allclose(np64(lse[i]).reshape(-1), ref["lse"][i], atol=2e-5)
    out2, lse2 = phase_1_batched_attention_triton_op(blocks, pq, 1e-5, num_active=3)
    ref3 = O.route(np64(blocks[:3]).reshape(3, -1, d), np64(pq), 1e-5)
    check_bf16(out2[1].reshape(-1, d), ref3["out"][1], "phase1 num_active=3")
    # phase 2: merge the partial into the committed-blocks result
    partial = torch.randn((2, 200, d), generator=g, device=gpu).to(torch.bfloat16)
    merged, logit, inv_p = phase_2_online_softmax_merge_forward_with_aux(partial, pq[2], out2[2], lse2[2], 1e-5)
    assert merged.dtype == torch.bfloat16
    mref = O.merge(np64(partial).reshape(-1, d), np64(pq[2]), np64(out2[2]).reshape(-1, d),
                   np64(lse2[2]).reshape(-1), 1e-5)
    check_bf16(merged.reshape(-1, d), mref["out"], "phase2")
    np.testing.assert_allclose(np64(logit).reshape(-1), mref["logit"], rtol=1e-4, atol=1e-4)
    # identity: merging the partial equals routing over the 4 sources directly
    full = O.route(np.concatenate([np64(blocks[:3]).reshape(3, -1, d), np64(partial).reshape(1, -1, d)]),
                   np64(pq[2]), 1e-5)["out"][0]
    err = np.abs(np64(merged).reshape(-1, d) - full)
    assert (err <= np.maximum(4e-2, 3 * bf16_ulp(full))).all()


MERGE_CASES = [
    # (hidden, rows, query dtype): row-per-wave kernel instances c1, c6, c8 and c4;
    # fewer rows than one grid of waves, a single row, the fp32-query path
    (512, 37, torch.bfloat16),
    (3072, 2050, torch.bfloat16),
    (4096, 300, torch.float32),
    (2048, 1, torch.bfloat16),
    (1536, 4099, torch.bfloat16),  # c3, a prime row count: ragged last rows per wave
    (2560, 997, torch.float32),    # c5, fp32 query
    (3584, 1031, torch.bfloat16),  # c7
    (1024, 5, torch.bfloat16),     # c2, fewer rows than one workgroup's waves
]


@pytest.mark.parametrize("d,rows,qdt", MERGE_CASES, ids=[f"D{c[0]}-N{c[1]}-{str(c[2])[6:]}" for c in MERGE_CASES])
def test_merge_both_kernels_match_oracle(gpu, policy, d, rows, qdt):
    # the phase-2 merge on the row-per-workgroup kernel and on the row-per-wave
    # kernel (bf16 rows of whole KiB, policy "stream"), output and aux against
    # the float64 oracle (kernels/phase_2.py:40-57)
    g = torch.Generator(device=gpu).manual_seed(31 + d + rows)
    partial = torch.randn((rows, d), generator=g, device=gpu).to(torch.bfloat16)
    inter = (0.5 * torch.randn((rows, d), generator=g, device=gpu)).to(torch.bfloat16)
    lse = torch.randn((rows,), generator=g, device=gpu)
    q = (torch.randn((d,), generator=g, device=gpu) * 0.05).to(qdt)
    merged, logit, inv = ops.merge(partial, q, inter, lse, 1e-5)
    ref = O.merge(np64(partial), np64(q), np64(inter), np64(lse), 1e-5)
    check_bf16(merged, ref["out"], f"merge {policy} D={d} N={rows}")
    np.testing.assert_allclose(np64(logit), ref["logit"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(np64(inv), ref["inv_rms"], rtol=1e-5)


def merge_kernel(n, d, qdt=torch.bfloat16):
    import ctypes

    buf = ctypes.create_string_buffer(128)
    code = _capi.DTYPE_BF16
    _capi.check("attnres_merge_kernel_name",
                _capi.lib().attnres_merge_kernel_name(n, d, code, ops.dtype_code(qdt), code, buf, 128))
    return buf.value.decode()


def test_merge_kernel_name_follows_the_launch_choice(gpu):
    # the name query and the launch share one choice: the row-per-wave kernel
    # for bf16 rows of whole KiB over >= 2048 rows (or always under the stream
    # policy), the row-per-workgroup kernel otherwise (or always under the
    # workgroup policy)
    assert merge_kernel(32768, 3072) == "attnres_merge_stream_d2_c6"
    assert merge_kernel(32768, 4096, torch.float32) == "attnres_merge_stream_fm_c8"
    assert merge_kernel(1000, 3072).startswith("attnres_merge_bf_bf_v")
    assert merge_kernel(32768, 3080).startswith("attnres_merge_bf_bf_v")  # rows not whole KiB
    for pol, want in ((_capi.POLICY_STREAM, "attnres_merge_stream_d2_c6"), (_capi.POLICY_WORKGROUP, "attnres_merge_bf_bf_v")):
        prev = _capi.set_kernel_policy(pol)
        try:
            assert merge_kernel(1000 if pol == _capi.POLICY_STREAM else 32768, 3072).startswith(want)
        finally:
            _capi.set_kernel_policy(prev)


def test_streaming_merge_matches_workgroup_merge_every_row(gpu):
    # every element of every row at the 3B shape (32768 rows of 3072): the
    # row-per-wave merge against the row-per-workgroup merge; they differ only
    # in the order of the two row sums, so pi agrees to a few fp32 ulps and
    # the outputs to one bf16 ulp plus 2^-16 of the larger input
    n, d = 32768, 3072
    g = torch.Generator(device=gpu).manual_seed(41)
    partial = torch.randn((n, d), generator=g, device=gpu).to(torch.bfloat16)
    inter = (0.5 * torch.randn((n, d), generator=g, device=gpu)).to(torch.bfloat16)
    lse = torch.randn((n,), generator=g, device=gpu)
    q = (torch.randn((d,), generator=g, device=gpu) * 0.05).to(torch.bfloat16)
    outs = []
    for pol in (_capi.POLICY_STREAM, _capi.POLICY_WORKGROUP):
        prev = _capi.set_kernel_policy(pol)
        try:
            with torch.no_grad():
                outs.append(ops.merge_call(partial, q, inter, lse, 1e-5).float())
        finally:
            _capi.set_kernel_policy(prev)
    torch.cuda.synchronize()
    a, b = outs
    xmax = torch.maximum(partial.abs(), inter.abs()).float()
    tol = torch.exp2(torch.floor(torch.log2(torch.clamp(b.abs(), min=2.0**-126))) - 7) + 2.0**-16 * xmax
    excess = ((a - b).abs() / tol).max().item()
    same = (a == b).float().mean().item()
    print(f"merge stream vs workgroup: max |diff| / tol {excess:.3f}, {same:.5f} of elements equal", flush=True)
    assert excess <= 1.0
    assert same >= 0.99


# ------------------------------------------------------ HIP graphs --


def test_decode_step_graph_replays_match_eager(gpu, policy):
    w = workloads.get("cfg4")
    sched = w.schedule
    L = sched.num_layers
    embed = torch.randn((w.batch, 1, w.hidden), device=gpu).to(torch.bfloat16)
    deltas = workloads.make_deltas(w, gpu, 9, 2 * L)
    q, gn = workloads.make_params(w, gpu, 9, sched.num_points)
    router = AttnResRouter(sched, list(q), list(gn), w.eps)
    arena = router.new_arena((w.batch, 1), w.hidden, w.dtype, gpu)
    eager = router.forward(embed, lambda j, h: deltas[j], arena=arena).clone()
    static_embed = embed.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        router.forward(static_embed, lambda j, h: deltas[j], arena=arena)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = router.forward(static_embed, lambda j, h: deltas[j], arena=arena)
    for rep in range(4):
        arena.buf.normal_()  # eager work between replays; the graph must not depend on arena contents
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {rep} differs from eager"


# ------------------------------------------------ loaded checkpoint weights --


@pytest.mark.parametrize("tokens", [(64, 1), (2, 256)], ids=["decode", "prefill"])
def test_routing_with_loaded_checkpoint_weights(gpu, tmp_path, tokens):
    # trained routing weights are peaky (large query norms): save a checkpoint in the
    # reference's layout, load it through the safe loader, route with it on the GPU
    from kotodama_amd.checkpoint import load_routing_weights

    L, D, eps = 8, 2048, 1e-5
    g = torch.Generator().manual_seed(12)
    sd = {}
    for i in range(L):
        for kind in ("attn", "mlp"):
            sd[f"_orig_mod.layers.{i}.{kind}_res_query"] = (torch.randn(D, generator=g) * 0.3).to(torch.bfloat16)
            sd[f"_orig_mod.layers.{i}.{kind}_res_norm.weight"] = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    sd["_orig_mod.final_res_query"] = (torch.randn(D, generator=g) * 0.3).to(torch.bfloat16)
    sd["_orig_mod.final_res_norm.weight"] = torch.ones(D).to(torch.bfloat16)
    path = tmp_path / "step_00001000.pt"
    torch.save({"step": 1000, "model": sd}, path)
    w = load_routing_weights(path, device=gpu)
    sched = w.schedule(n_blocks=3)
    router = w.router(sched, eps)
    B, T = tokens
    embed = torch.randn((B, T, D), generator=g).to(torch.bfloat16).to(gpu)
    deltas = [torch.randn((B, T, D), generator=g).to(torch.bfloat16).to(gpu) for _ in range(2 * L)]
    outs = []

    def sublayer(j, h):
        outs.append(h.clone())
        return deltas[j]

    with torch.no_grad():
        outs.append(router.forward(embed, sublayer))
    qws = [O.fold_query(np64(w.queries[j]), np64(w.gains[j]), "bf16") for j in range(sched.num_points)]
    ref = O.block_forward(np64(embed).reshape(-1, D), [np64(x).reshape(-1, D) for x in deltas], qws, eps, L,
                          sched.boundary_set, dtype="bf16", want_weights=True)
    # the weights really are peaky: most rows put > 90% on one source somewhere in the forward
    peak = max(float(np.mean(np.max(wj, axis=0) > 0.9)) for wj in ref["weights"][1:])
    assert peak > 0.5
    for j in range(sched.num_points):
        check_bf16(outs[j].reshape(-1, D), ref["outs"][j], f"point {j}")
