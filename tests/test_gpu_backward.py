"""Backward of the routing ops on the GPU against the float64 oracle.

The gradients come from ``torch.autograd`` through the drop-ins
(``route_static``, ``block_attn_res_from_list``, the phase-1 mirror), which
call ``attnres_route_bwd`` through the C ABI.  The oracle is
``route_backward`` (pinned on the CPU by finite differences and by float64
autograd through the einsum branch's op sequence), evaluated on the identical
input values.

Tolerances:
* fp32 gradients: |g - ref| <= 1e-4 |ref| + 1e-5 max|ref|  (fp32 dot products of
  length D and a sum over tokens for the query/gain gradients);
* bf16 gradients: |g - ref| <= 1 bf16 ulp of |ref| + 1e-3 max|ref|, and at least
  95% of the elements equal to the correctly rounded oracle (one rounding of
  an fp32-accumulated value).
At the full BASELINE shape the oracle runs on sampled rows; on every row the
identity x_s . dx_s = w_s (G . x_s) + dl_s l_s eps r_s^2 (logits are
scale-invariant up to eps; dl_s = w_s (g_lse + G.x_s - G.out)) is checked
against an fp32 torch restatement, which also gives the query and gain
gradients summed over all rows.
"""

import numpy as np
import pytest
import torch

import kotodama_amd
from kotodama_amd import _capi, ops, workloads
from kotodama_amd.flash_attn_res import phase_1_batched_attention_triton_op
from oracle import attnres_oracle as O

pytestmark = pytest.mark.gpu


class Norm(torch.nn.Module):
    def __init__(self, weight, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(weight)
        self.eps = eps


def np64(t):
    return t.detach().float().cpu().double().numpy()


def bf16_ulp(x):
    a = np.abs(x)
    e = np.floor(np.log2(np.maximum(a, 2.0**-126)))
    return 2.0 ** (e - 7)


# Gradients this close to fp32's underflow threshold (2^-126 ~ 1.2e-38) are
# products of softmax weights that underflowed: the kernels flush fp32
# subnormals to zero, as the reference's Triton kernels do (their exp is the
# flush-to-zero exp2), so such an element can come out 0 where the float64
# oracle keeps a subnormal or barely normal value.  The exact-rounding count
# leaves them out; the error bar still covers them.
UNDERFLOW_RANGE = 1e-30


def check_grad(g, ref, dtype, label, exact_frac=0.95):
    got = np64(g)
    err = np.abs(got - ref)
    scale = np.abs(ref).max() if ref.size else 0.0
    if dtype == torch.float32:
        tol = 1e-4 * np.abs(ref) + 1e-5 * scale
        assert (err <= tol).all(), f"{label}: worst err {err.max():.3e} (max|ref| {scale:.3e})"
    else:
        tol = bf16_ulp(ref) + 1e-3 * scale
        assert (err <= tol).all(), f"{label}: worst err {err.max():.3e} (max|ref| {scale:.3e})"
        counted = np.abs(ref) >= UNDERFLOW_RANGE
        if counted.any():
            same = np.mean(got[counted] == O.bf16_round(ref[counted]))
            assert same >= exact_frac, f"{label}: only {same:.4f} equal the correctly rounded oracle"


def make_case(gpu, S, extra, B, T, D, dtype, seed, param_dtype=None):
    g = torch.Generator(device="cpu").manual_seed(seed)
    scales = torch.exp(torch.empty(S + extra).uniform_(np.log(0.5), np.log(4.0), generator=g))
    buf = torch.randn(S + extra, B, T, D, generator=g) * scales[:, None, None, None]
    buf[S:] = 0
    pd = param_dtype or dtype
    query = (torch.randn(D, generator=g) * 0.05).to(pd)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(pd)
    # bf16-exact, so the gradient that reaches a bf16 output is G itself
    G = torch.randn(B, T, D, generator=g).to(torch.bfloat16).float()
    return buf.to(dtype).to(gpu), query.to(gpu), gain.to(gpu), G.to(gpu)


def oracle_grads(buf, S, query, gain, G, eps, param, grad_lse=None):
    D = buf.shape[-1]
    x = np64(buf[:S]).reshape(S, -1, D)
    pd = "bf16" if param == torch.bfloat16 else "f32"
    qw = O.fold_query(np64(query), np64(gain), pd)
    b = O.route_backward(x, qw, eps, np64(G).reshape(-1, D), None if grad_lse is None else np64(grad_lse).reshape(-1))
    return b["dx"], b["dqw"] * np64(gain), b["dqw"] * np64(query)


CASES = [
    # (dtype, S, D, B, T)
    (torch.float32, 1, 256, 2, 48),
    (torch.float32, 3, 2048, 1, 64),
    (torch.float32, 9, 1024, 2, 40),
    (torch.float32, 16, 512, 1, 33),
    (torch.bfloat16, 1, 512, 2, 48),
    (torch.bfloat16, 4, 3072, 1, 64),
    (torch.bfloat16, 8, 4096, 2, 32),
    (torch.bfloat16, 9, 8192, 1, 24),
    # 1023 chunks: two chunks per thread on 512 threads, the last thread's second chunk
    # past the row end (odd chunk count, ragged tail)
    (torch.bfloat16, 3, 8184, 1, 40),
    (torch.bfloat16, 8, 8184, 2, 12),
    (torch.bfloat16, 13, 1024, 2, 20),
    (torch.bfloat16, 16, 4096, 1, 17),
]


@pytest.mark.parametrize("dtype,S,D,B,T", CASES, ids=[f"{str(c[0])[6:]}-S{c[1]}-D{c[2]}" for c in CASES])
def test_route_static_backward_matches_oracle(gpu, dtype, S, D, B, T):
    print(f"route_static backward {dtype} S={S} D={D} B={B} T={T}", flush=True)
    eps = 1e-5
    buf, query, gain, G = make_case(gpu, S, 2, B, T, D, dtype, seed=100 + S + D)
    buf.requires_grad_(True)
    query.requires_grad_(True)
    norm = Norm(gain.clone(), eps)
    mask = torch.zeros(S + 2, dtype=torch.bool, device=gpu)
    mask[:S] = True
    out = kotodama_amd.route_static(buf, query, norm, mask, S)
    (out.float() * G).sum().backward()
    dx, dq, dg = oracle_grads(buf, S, query, norm.weight, G, eps, dtype)
    check_grad(buf.grad[:S].reshape(S, -1, D), dx, dtype, "dsources")
    assert torch.all(buf.grad[S:] == 0), "inactive slots must get zero gradient"
    check_grad(query.grad, dq, dtype, "dquery")
    check_grad(norm.weight.grad, dg, dtype, "dgain")


# Rows narrower than one block of the routing backward (11 bf16 chunks or 15
# fp32 chunks in a 64-thread block) with S >= 5, where each thread's query
# chunks sit in LDS: the threads past the row end must not read the slots no
# thread wrote (stale Inf or NaN times a zero source chunk is NaN, which the
# row reduction spreads to the whole row).
NARROW = [(torch.bfloat16, 5, 88, 1, 2402), (torch.float32, 6, 60, 1, 1117)]


@pytest.mark.parametrize("dtype,S,D,B,T", NARROW, ids=[f"{str(c[0])[6:]}-S{c[1]}-D{c[2]}" for c in NARROW])
def test_narrow_rows_backward_ignores_stale_lds(gpu, dtype, S, D, B, T):
    # a streaming forward over NaN rows first: the finished rows it stages in
    # LDS on every CU leave NaN there for the next kernel
    pool = torch.full((3, 1, 32768, 3072), float("nan"), dtype=torch.bfloat16, device=gpu)
    with torch.no_grad():
        ops.route_call(pool, 3, torch.zeros(3072, dtype=torch.bfloat16, device=gpu), None, 1e-5, torch.bfloat16)
    del pool
    print(f"narrow-row backward {dtype} S={S} D={D} rows={B * T}", flush=True)
    eps = 1e-5
    buf, query, gain, G = make_case(gpu, S, 0, B, T, D, dtype, seed=300 + S + D)
    buf.requires_grad_(True)
    query.requires_grad_(True)
    norm = Norm(gain.clone(), eps)
    out = kotodama_amd.route_static(buf, query, norm, torch.ones(S, dtype=torch.bool, device=gpu), S)
    (out.float() * G).sum().backward()
    torch.cuda.synchronize()
    assert torch.isfinite(buf.grad).all() and torch.isfinite(query.grad).all()
    dx, dq, dg = oracle_grads(buf, S, query, norm.weight, G, eps, dtype)
    check_grad(buf.grad.reshape(S, -1, D), dx, dtype, "dsources")
    check_grad(query.grad, dq, dtype, "dquery")
    check_grad(norm.weight.grad, dg, dtype, "dgain")


def test_lse_gradient_kept_next_to_large_dot_products(gpu):
    # dL/dlogit_s = w_s (g_lse + G.x_s - G.out): g_lse (~0.1) must be added after
    # G.x_s - G.out cancels; added to G.x_s (~100) first it is rounded to that
    # number's ulp, a relative error of ~4e-5 in g_lse.  fp32 throughout; with one
    # source the query gradient is exactly sum_n g_lse_n r_n x_n, which fp32
    # sums to ~1e-6 of its largest value.
    S, D, N = 1, 2928, 341
    g = torch.Generator(device="cpu").manual_seed(41)
    x = (torch.randn(S, N, D, generator=g) * 2.0).to(gpu)
    q = (torch.randn(D, generator=g) * 0.05).to(gpu)
    G = torch.randn(N, D, generator=g).to(gpu)
    glse = (torch.randn(N, generator=g) * 0.1).to(gpu)
    dx = torch.empty(S, N, D, device=gpu)
    ws = torch.empty(_capi.route_bwd_workspace_size(N, D) // 4, device=gpu)
    dq = torch.empty(D, device=gpu)
    _capi.route_bwd(_capi.pointer_array([x[s].data_ptr() for s in range(S)]), S, N, D, D, _capi.DTYPE_F32,
                    q.data_ptr(), None, _capi.DTYPE_F32, 1e-5, G.data_ptr(), _capi.DTYPE_F32, D, glse.data_ptr(),
                    _capi.pointer_array([dx[s].data_ptr() for s in range(S)]), D, ws.data_ptr(), ws.numel() * 4,
                    dq.data_ptr(), None, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize()
    b = O.route_backward(np64(x), np64(q), 1e-5, np64(G), np64(glse))
    err = np.abs(np64(dq) - b["dqw"]).max()
    assert err <= 2e-6 * np.abs(b["dqw"]).max(), f"query gradient worst err {err:.3e}"
    assert np.abs(np64(dx) - b["dx"]).max() <= 1e-6 * np.abs(b["dx"]).max()


def test_padded_stack_backward_like_the_training_loop(gpu):
    # llama.py:690-699: committed blocks + partial + zero padding stacked, then
    # routed; the padding does not require grad, so its gradient rows are not
    # written, and the real sources still get the oracle's gradients
    eps = 1e-5
    S, B, T, D = 3, 2, 24, 3072
    buf, query, gain, G = make_case(gpu, S, 0, B, T, D, torch.bfloat16, seed=91)
    srcs = [buf[i].clone().requires_grad_(True) for i in range(S)]
    zero = torch.zeros_like(srcs[0])
    stacked = torch.stack(srcs + [zero] * 5)
    norm = Norm(gain.clone(), eps)
    mask = torch.zeros(8, dtype=torch.bool, device=gpu)
    mask[:S] = True
    out = kotodama_amd.route_static(stacked, query, norm, mask, S)
    (out.float() * G).sum().backward()
    dx, _, dg = oracle_grads(buf, S, query, norm.weight, G, eps, torch.bfloat16)
    for s in range(S):
        check_grad(srcs[s].grad.reshape(-1, D), dx[s], torch.bfloat16, f"dsource[{s}]")
    check_grad(norm.weight.grad, dg, torch.bfloat16, "dgain")
    # an observed buffer gradient keeps exact zeros in the padding slots
    stacked2 = torch.stack([s.detach().clone().requires_grad_(True) for s in srcs] + [zero] * 5)
    stacked2.retain_grad()
    kotodama_amd.route_static(stacked2, query, norm, mask, S).float().mul(G).sum().backward()
    assert torch.all(stacked2.grad[S:] == 0)


def test_list_backward_and_separate_tensors(gpu):
    # block_attn_res_from_list: each source its own allocation (no stacked buffer)
    eps = 1e-5
    S, B, T, D = 5, 2, 30, 2048
    buf, query, gain, G = make_case(gpu, S, 0, B, T, D, torch.bfloat16, seed=7)
    srcs = [buf[i].clone().requires_grad_(True) for i in range(S)]
    norm = Norm(gain.clone(), eps)
    out = kotodama_amd.block_attn_res_from_list(srcs, query, norm)
    (out.float() * G).sum().backward()
    dx, _, dg = oracle_grads(buf, S, query, norm.weight, G, eps, torch.bfloat16)
    for s in range(S):
        check_grad(srcs[s].grad.reshape(-1, D), dx[s], torch.bfloat16, f"dsource[{s}]")
    check_grad(norm.weight.grad, dg, torch.bfloat16, "dgain")
    assert query.grad is None  # query did not require grad


def test_non_prefix_mask_backward(gpu):
    # any active set: the drop-in routes slots {0, 2, 3} of a 5-slot buffer
    eps = 1e-5
    B, T, D = 1, 40, 1024
    buf, query, gain, G = make_case(gpu, 5, 0, B, T, D, torch.float32, seed=9)
    idx = [0, 2, 3]
    buf.requires_grad_(True)
    norm = Norm(gain.clone(), eps)
    mask = torch.zeros(5, dtype=torch.bool, device=gpu)
    mask[idx] = True
    out = kotodama_amd.route_static(buf, query, norm, mask, 0)
    (out * G).sum().backward()
    sub = buf.detach()[idx]
    dx, _, dg = oracle_grads(sub, 3, query, norm.weight, G, eps, torch.float32)
    check_grad(buf.grad[idx].reshape(3, -1, D), dx, torch.float32, "dsources")
    assert torch.all(buf.grad[[1, 4]] == 0)
    check_grad(norm.weight.grad, dg, torch.float32, "dgain")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_phase_1_backward_with_lse_term(gpu, dtype):
    # the phase-1 op with Q = 1: the loss uses both the output and the lse
    eps = 1e-6
    S, B, T, D = 6, 2, 24, 1024
    buf, query, gain, G = make_case(gpu, S, 1, B, T, D, dtype, seed=31)
    qw = (query * gain).detach().requires_grad_(True)
    buf.requires_grad_(True)
    gl = torch.randn(1, B, T, device=gpu)
    out, lse = phase_1_batched_attention_triton_op(buf, qw.unsqueeze(0), eps, num_active=S)
    (out.float() * G).sum().add_((lse * gl).sum()).backward()
    x = np64(buf[:S]).reshape(S, -1, D)
    b = O.route_backward(x, np64(qw), eps, np64(G).reshape(-1, D), np64(gl).reshape(-1))
    check_grad(buf.grad[:S].reshape(S, -1, D), b["dx"], dtype, "dsources")
    assert torch.all(buf.grad[S:] == 0)
    check_grad(qw.grad, b["dqw"], dtype, "dqw")


def test_multi_query_phase_1_backward(gpu):
    # Q = 3 pseudo-queries over one stack (the serving path's batched call)
    eps = 1e-5
    S, B, T, D, Q = 5, 2, 20, 2048, 3
    buf, _, _, _ = make_case(gpu, S, 1, B, T, D, torch.bfloat16, seed=51)
    g = torch.Generator(device="cpu").manual_seed(52)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(torch.bfloat16).to(gpu).requires_grad_(True)
    G = torch.randn(Q, B, T, D, generator=g).to(torch.bfloat16).float().to(gpu)
    gl = torch.randn(Q, B, T, generator=g).to(gpu)
    buf.requires_grad_(True)
    out, lse = phase_1_batched_attention_triton_op(buf, qs, eps, num_active=S)
    (out.float() * G).sum().add_((lse * gl).sum()).backward()
    x = np64(buf[:S]).reshape(S, -1, D)
    dx = np.zeros_like(x)
    for j in range(Q):
        b = O.route_backward(x, np64(qs[j]), eps, np64(G[j]).reshape(-1, D), np64(gl[j]).reshape(-1))
        dx += b["dx"]
        check_grad(qs.grad[j], b["dqw"], torch.bfloat16, f"dq[{j}]")
    check_grad(buf.grad[:S].reshape(S, -1, D), dx, torch.bfloat16, "dsources (sum over queries)")
    assert torch.all(buf.grad[S:] == 0)


MQ_CASES = [
    # (dtype, S, D, B, T, Q, with gain, batched kernel: "mqg" matrix cores, "mq" VALU, None per query)
    (torch.bfloat16, 1, 1024, 2, 20, 2, False, "mqg"),
    (torch.bfloat16, 7, 3072, 1, 40, 8, True, "mqg"),
    (torch.bfloat16, 8, 1024, 2, 16, 5, False, "mqg"),  # a ragged second group of queries
    (torch.bfloat16, 4, 4096, 1, 12, 4, True, "mqg"),  # 256-thread rows
    (torch.bfloat16, 5, 520, 1, 9, 3, False, "mqg"),  # one thread holds the row's last chunk
    (torch.bfloat16, 3, 2056, 1, 10, 6, True, "mqg"),  # 257 chunks: threads past the end
    (torch.bfloat16, 8, 4096, 1, 12, 8, True, "mqg"),  # two chunks per thread, eight queries
    (torch.bfloat16, 6, 3584, 1, 10, 7, False, "mqg"),  # 448 chunks: second chunks past the end
    (torch.bfloat16, 7, 3072, 1, 40, 9, True, "mq"),  # nine queries
    (torch.bfloat16, 9, 2048, 2, 12, 4, False, "mq"),
    (torch.bfloat16, 3, 8192, 1, 16, 3, True, "mq"),
    (torch.bfloat16, 12, 1024, 1, 24, 3, False, None),
    (torch.float32, 16, 1024, 1, 20, 2, True, "mq"),
    (torch.float32, 5, 4096, 1, 16, 9, False, "mq"),
]


def bwd_queries_kernel(S, D, dtype, Q):
    import ctypes

    code = ops.dtype_code(dtype)
    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_bwd_queries_kernel_name",
                _capi.lib().attnres_route_bwd_queries_kernel_name(S, D, code, code, code, Q, buf, 128))
    return buf.value.decode()


@pytest.mark.parametrize("dtype,S,D,B,T,Q,with_gain,kernel", MQ_CASES,
                         ids=[f"{str(c[0])[6:]}-S{c[1]}-D{c[2]}-Q{c[5]}" for c in MQ_CASES])
def test_batched_query_backward_matches_oracle(gpu, monkeypatch, dtype, S, D, B, T, Q, with_gain, kernel):
    # Q queries over one stack with an lse term: the source gradients summed
    # over the queries, every query's gradient and the gain gradient summed
    # over the queries; one pass of attnres_route_bwd_queries where a batched
    # kernel exists (on the matrix cores for bf16 with S <= 8, Q <= 8 and
    # D <= 4096; nine queries: two passes of the query-gradient kernel), one
    # attnres_route_bwd per query otherwise
    name = bwd_queries_kernel(S, D, dtype, Q)
    print(f"batched-query backward {dtype} S={S} D={D} Q={Q} gain={with_gain} kernel={name or 'per query'}",
          flush=True)
    if kernel is None:
        assert name == ""
    else:
        assert name.startswith(f"attnres_route_bwd_{kernel}_"), name
    batched = kernel is not None
    eps = 1e-5
    buf, _, _, _ = make_case(gpu, S, 0, B, T, D, dtype, seed=60 + S + Q)
    g = torch.Generator(device="cpu").manual_seed(61 + D)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(dtype).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype).to(gpu).requires_grad_(True) if with_gain else None
    G = torch.randn(Q, B, T, D, generator=g).to(torch.bfloat16).float().to(gpu)
    GL = torch.randn(Q, B, T, generator=g).to(gpu)
    buf.requires_grad_(True)
    per_query = []
    real = ops._launch_route_bwd
    monkeypatch.setattr(ops, "_launch_route_bwd", lambda *a: per_query.append(1) or real(*a))
    out, _, lse, _, _ = ops.route(buf, S, qs, gain, eps, dtype, True, False)
    (out.float() * G).sum().add_((lse * GL).sum()).backward()
    assert (len(per_query) == 0) == batched, f"per-query launches: {len(per_query)}"
    pd = "bf16" if dtype == torch.bfloat16 else "f32"
    x = np64(buf).reshape(S, -1, D)
    dx = np.zeros_like(x)
    dgain = np.zeros(D)
    for j in range(Q):
        qw = O.fold_query(np64(qs[j]), np64(gain) if with_gain else None, pd)
        b = O.route_backward(x, qw, eps, np64(G[j]).reshape(-1, D), np64(GL[j]).reshape(-1))
        dx += b["dx"]
        check_grad(qs.grad[j], b["dqw"] * (np64(gain) if with_gain else 1.0), dtype, f"dquery[{j}]")
        dgain += b["dqw"] * np64(qs[j])
    check_grad(buf.grad.reshape(S, -1, D), dx, dtype, "dsources (sum over queries)")
    if with_gain:
        check_grad(gain.grad, dgain, dtype, "dgain (sum over queries)")


def _bwd_kernel_name(s, n, d, policy=None):
    import ctypes

    buf = ctypes.create_string_buffer(128)
    code = _capi.DTYPE_BF16
    prev = _capi.set_kernel_policy(policy) if policy is not None else None
    try:
        _capi.check("attnres_route_bwd_kernel_name",
                    _capi.lib().attnres_route_bwd_kernel_name(s, n, d, code, code, buf, 128))
    finally:
        if prev is not None:
            _capi.set_kernel_policy(prev)
    return buf.value.decode()


def test_backward_chunks_per_thread_policy(gpu):
    # row-per-workgroup kernel: two chunks per thread for 5 <= S <= 8 over many
    # rows of at most 384 chunks (3B prefill shape), one elsewhere (fewer rows,
    # wider rows, S <= 4 or S >= 9, whose two-chunk instances spill from S = 12)
    def name(s, n, d):
        return _bwd_kernel_name(s, n, d, _capi.POLICY_WORKGROUP)

    assert name(7, 32768, 3072).endswith("_s7_v2")
    assert name(4, 32768, 3072).endswith("_s4_v1")
    assert name(9, 32768, 3072).endswith("_s9_v1")
    assert name(7, 8192, 3072).endswith("_s7_v1")
    assert name(7, 32768, 4096).endswith("_s7_v1")
    assert name(3, 64, 8192).endswith("_s3_v2")  # rows above 512 chunks: always two


def test_backward_row_per_wave_policy(gpu):
    # under AUTO the row-per-wave kernel takes bf16 calls of >= 64 rows per CU of
    # 6 KiB with S <= 8; its 8 KiB instances (S <= 9) run under the STREAM policy
    auto, stream = _capi.POLICY_AUTO, _capi.POLICY_STREAM
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    assert _bwd_kernel_name(7, 32768, 3072, auto) == "attnres_route_bwd_stream_c6_s7"
    assert _bwd_kernel_name(8, 32768, 3072, auto) == "attnres_route_bwd_stream_c6_s8"
    assert _bwd_kernel_name(1, 64 * cus, 3072, auto) == "attnres_route_bwd_stream_c6_s1"
    assert _bwd_kernel_name(5, 64 * cus - 1, 3072, auto).endswith("_s5_v1")
    assert _bwd_kernel_name(6, 16384, 4096, auto).endswith("_s6_v1")
    assert _bwd_kernel_name(6, 16384, 4096, stream) == "attnres_route_bwd_stream_c8_s6"
    assert _bwd_kernel_name(9, 16384, 4096, stream) == "attnres_route_bwd_stream_c8_s9"
    assert _bwd_kernel_name(10, 16384, 4096, stream).endswith("_s10_v1")
    assert _bwd_kernel_name(9, 32768, 3072, auto).endswith("_s9_v1")
    assert _bwd_kernel_name(7, 1000, 3072, auto).endswith("_s7_v1")  # below the row threshold
    assert _bwd_kernel_name(4, 32768, 2048, auto).endswith("_s4_v1")  # 4 KiB rows
    assert _bwd_kernel_name(7, 100, 3072, _capi.POLICY_STREAM) == "attnres_route_bwd_stream_c6_s7"


# The row-per-wave backward against the oracle: every instance (rows of 6 KiB
# at S = 1..8, 8 KiB at S = 1..9, the last three with rows kept in LDS), row
# counts that leave waves of the last workgroups without a row or with one row
# fewer, fewer rows than one workgroup's waves, and fp32 parameters.
STREAM_BWD = [(3072, s, 1, 3001, None) for s in range(1, 9)] + [(4096, s, 1, 2003, None) for s in range(1, 7)] + \
    [(4096, s, 1, 1500, None) for s in range(7, 10)] + \
    [(3072, 8, 1, 3, None), (3072, 4, 2, 1500, torch.float32), (4096, 6, 1, 5, torch.float32),
     (4096, 9, 1, 7, torch.float32)]


@pytest.mark.parametrize("D,S,B,T,pd", STREAM_BWD,
                         ids=[f"D{c[0]}-S{c[1]}-N{c[2] * c[3]}{'-pf32' if c[4] else ''}" for c in STREAM_BWD])
def test_row_per_wave_backward_matches_oracle(gpu, D, S, B, T, pd):
    print(f"row-per-wave backward D={D} S={S} B={B} T={T} param={pd}", flush=True)
    assert _bwd_kernel_name(S, B * T, D, _capi.POLICY_STREAM) == f"attnres_route_bwd_stream_c{D // 512}_s{S}"
    buf, query, gain, G = make_case(gpu, S, 1, B, T, D, torch.bfloat16, seed=300 + S + D + T, param_dtype=pd)
    buf.requires_grad_(True)
    query.requires_grad_(True)
    norm = Norm(gain.clone(), 1e-5)
    mask = torch.zeros(S + 1, dtype=torch.bool, device=gpu)
    mask[:S] = True
    prev = _capi.set_kernel_policy(_capi.POLICY_STREAM)
    try:
        out = kotodama_amd.route_static(buf, query, norm, mask, S)
        (out.float() * G).sum().backward()
        torch.cuda.synchronize()
    finally:
        _capi.set_kernel_policy(prev)
    dx, dq, dg = oracle_grads(buf, S, query, norm.weight, G, 1e-5, pd or torch.bfloat16)
    check_grad(buf.grad[:S].reshape(S, -1, D), dx, torch.bfloat16, "dsources")
    assert torch.all(buf.grad[S:] == 0), "inactive slot must get zero gradient"
    check_grad(query.grad, dq, query.dtype, "dquery")
    check_grad(norm.weight.grad, dg, query.dtype, "dgain")


@pytest.mark.parametrize("S", [1, 5, 8])
def test_row_per_wave_backward_with_lse_gradient(gpu, S):
    print(f"row-per-wave backward with dL/dlse S={S}", flush=True)
    buf, query, gain, G = make_case(gpu, S, 0, 2, 1100, 3072, torch.bfloat16, seed=77 + S)
    buf.requires_grad_(True)
    query.requires_grad_(True)
    norm = Norm(gain.clone(), 1e-5)
    gl = torch.randn(2, 1100, device=gpu)
    prev = _capi.set_kernel_policy(_capi.POLICY_STREAM)
    try:
        res = ops.route(buf, S, query, norm.weight, 1e-5, torch.bfloat16, True, False)
        (res[0][0].float() * G).sum().add_((res[2][0] * gl).sum()).backward()
        torch.cuda.synchronize()
    finally:
        _capi.set_kernel_policy(prev)
    dx, dq, dg = oracle_grads(buf, S, query, norm.weight, G, 1e-5, torch.bfloat16, grad_lse=gl)
    check_grad(buf.grad.reshape(S, -1, 3072), dx, torch.bfloat16, "dsources")
    check_grad(query.grad, dq, torch.bfloat16, "dquery")
    check_grad(norm.weight.grad, dg, torch.bfloat16, "dgain")


def test_batched_query_backward_without_lse_gradient(gpu):
    # the loss uses the routed rows only: no dL/dlse reaches the batched
    # backward (grad_lse NULL through the C ABI), on the matrix-core kernel
    eps, S, Q, D, N = 1e-5, 4, 5, 1024, 48
    assert bwd_queries_kernel(S, D, torch.bfloat16, Q).startswith("attnres_route_bwd_mqg_")
    buf, _, _, _ = make_case(gpu, S, 0, 1, N, D, torch.bfloat16, seed=300)
    g = torch.Generator(device="cpu").manual_seed(301)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(torch.bfloat16).to(gpu).requires_grad_(True)
    G = torch.randn(Q, 1, N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    buf.requires_grad_(True)
    out, _, _, _, _ = ops.route(buf, S, qs, None, eps, torch.bfloat16, False, False)
    (out.float() * G).sum().backward()
    x = np64(buf).reshape(S, -1, D)
    dx = np.zeros_like(x)
    for j in range(Q):
        b = O.route_backward(x, np64(qs[j]), eps, np64(G[j]).reshape(-1, D), np.zeros(N))
        dx += b["dx"]
        check_grad(qs.grad[j], b["dqw"], torch.bfloat16, f"dquery[{j}]")
    check_grad(buf.grad.reshape(S, -1, D), dx, torch.bfloat16, "dsources (sum over queries)")


@pytest.mark.parametrize("S,Q", [(3, 8), (7, 6)])
def test_batched_query_backward_many_rows_per_workgroup(gpu, S, Q):
    # 12288 rows of 512 elements on the matrix-core kernels: more rows than
    # the resident grid, so every workgroup walks several rows (next-row
    # loads, coefficients and reductions per row, query-gradient accumulators
    # across rows)
    eps, D, N = 1e-5, 512, 12288
    name = bwd_queries_kernel(S, D, torch.bfloat16, Q)
    assert name.startswith("attnres_route_bwd_mqg_"), name
    print(f"batched-query backward over {N} rows S={S} Q={Q} {name}", flush=True)
    buf, _, _, _ = make_case(gpu, S, 0, 1, N, D, torch.bfloat16, seed=200 + S)
    g = torch.Generator(device="cpu").manual_seed(201 + S)
    qs = (torch.randn(Q, D, generator=g) * 0.05).to(torch.bfloat16).to(gpu).requires_grad_(True)
    gain = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(gpu).requires_grad_(True)
    G = torch.randn(Q, 1, N, D, generator=g).to(torch.bfloat16).float().to(gpu)
    GL = torch.randn(Q, 1, N, generator=g).to(gpu)
    buf.requires_grad_(True)
    out, _, lse, _, _ = ops.route(buf, S, qs, gain, eps, torch.bfloat16, True, False)
    (out.float() * G).sum().add_((lse * GL).sum()).backward()
    x = np64(buf).reshape(S, -1, D)
    dx = np.zeros_like(x)
    dgain = np.zeros(D)
    for j in range(Q):
        qw = O.fold_query(np64(qs[j]), np64(gain), "bf16")
        b = O.route_backward(x, qw, eps, np64(G[j]).reshape(-1, D), np64(GL[j]).reshape(-1))
        dx += b["dx"]
        check_grad(qs.grad[j], b["dqw"] * np64(gain), torch.bfloat16, f"dquery[{j}]")
        dgain += b["dqw"] * np64(qs[j])
    check_grad(buf.grad.reshape(S, -1, D), dx, torch.bfloat16, "dsources (sum over queries)")
    check_grad(gain.grad, dgain, torch.bfloat16, "dgain (sum over queries)")


def test_batched_query_backward_unsupported_shape_raises(gpu):
    # bf16 rows above 4096 elements (two chunks per thread) with 5 sources and
    # several queries: no batched kernel, and the per-query composition's fp32
    # copies would exceed the fp32 row limit: a clear error
    S, D, Q = 5, 8192, 2
    buf = torch.randn(S, 1, 4, D, device=gpu).to(torch.bfloat16).requires_grad_(True)
    qs = (torch.randn(Q, D, device=gpu) * 0.05).to(torch.bfloat16)
    out, _, _, _, _ = ops.route(buf, S, qs, None, 1e-5, torch.bfloat16, False, False)
    with pytest.raises(RuntimeError, match="not supported"):
        out.float().sum().backward()


MERGE_CASES = [
    (torch.bfloat16, torch.bfloat16, 3072),
    (torch.bfloat16, torch.bfloat16, 8192),
    (torch.float32, torch.bfloat16, 1024),
    (torch.bfloat16, torch.float32, 512),
    (torch.float32, torch.float32, 2048),
]


@pytest.mark.parametrize("pdt,idt,D", MERGE_CASES, ids=[f"{str(a)[6:]}-{str(b)[6:]}-D{c}" for a, b, c in MERGE_CASES])
def test_merge_backward_matches_oracle(gpu, pdt, idt, D):
    eps = 1e-5
    B, T = 2, 40
    g = torch.Generator(device="cpu").manual_seed(70 + D)
    p = (torch.randn(B, T, D, generator=g) * 2).to(pdt).to(gpu).requires_grad_(True)
    q = (torch.randn(D, generator=g) * 0.05).to(pdt).to(gpu).requires_grad_(True)
    inter = torch.randn(B, T, D, generator=g).to(idt).to(gpu).requires_grad_(True)
    lse = (torch.randn(B, T, generator=g) * 2).to(gpu).requires_grad_(True)
    G = torch.randn(B, T, D, generator=g).to(idt).float().to(gpu)
    out, _, _ = ops.merge(p, q, inter, lse, eps)
    assert out.dtype == idt
    (out.float() * G).sum().backward()
    ref = O.merge_backward(np64(p), np64(q), np64(inter), np64(lse), eps, np64(G))
    check_grad(p.grad, ref["dpartial"], pdt, "dpartial")
    check_grad(inter.grad, ref["dinter"], idt, "dinter")
    check_grad(lse.grad, ref["dlse"], torch.float32, "dlse")
    check_grad(q.grad, ref["dq"], pdt, "dquery")


def test_two_phase_chain_matches_one_pass_backward(gpu):
    # phase 1 over the committed blocks + phase-2 merge of the partial has the
    # same gradients as routing over all sources at once (fp32, tight bar)
    eps = 1e-5
    S, B, T, D = 4, 2, 24, 1024
    buf, query, gain, G = make_case(gpu, S + 1, 0, B, T, D, torch.float32, seed=81)
    qw = (query * gain).detach()
    a = buf.detach().clone().requires_grad_(True)
    qa = qw.clone().requires_grad_(True)
    inter, lse = phase_1_batched_attention_triton_op(a[:S], qa.unsqueeze(0), eps)
    merged = ops.merge(a[S], qa, inter[0].float(), lse[0], eps)[0]
    (merged * G).sum().backward()
    b = buf.detach().clone().requires_grad_(True)
    qb = qw.clone().requires_grad_(True)
    full = ops.route(b, S + 1, qb, None, eps, torch.float32, False, False)[0][0]
    (full * G).sum().backward()
    # phase 1 rounds its output to bf16 (ops/phase_1.py:26-30), so the chain
    # differs from the one-pass routing by that rounding only
    ref_dx = np64(b.grad)
    scale = np.abs(ref_dx).max()
    assert np.abs(np64(a.grad) - ref_dx).max() <= 1e-2 * scale
    assert np.abs(np64(qa.grad) - np64(qb.grad)).max() <= 1e-2 * np.abs(np64(qb.grad)).max()


def test_mixed_param_dtypes_backward(gpu):
    # fp32 query with a bf16 gain: the fold is taken in the promoted dtype
    eps = 1e-5
    S, B, T, D = 4, 1, 32, 512
    buf, query, gain, G = make_case(gpu, S, 0, B, T, D, torch.bfloat16, seed=41, param_dtype=torch.float32)
    query = query.float().requires_grad_(True)
    norm = Norm(gain.to(torch.bfloat16), eps)
    buf.requires_grad_(True)
    out = kotodama_amd.route_static(buf, query, norm, torch.ones(S, dtype=torch.bool, device=gpu), S)
    assert out.dtype == torch.float32
    (out * G).sum().backward()
    x = np64(buf).reshape(S, -1, D)
    qw = np64(query) * np64(norm.weight)  # fp32 product of exact values
    qw = np.asarray(qw, dtype=np.float32).astype(np.float64)
    b = O.route_backward(x, qw, eps, np64(G).reshape(-1, D))
    check_grad(buf.grad.reshape(S, -1, D), b["dx"], torch.bfloat16, "dsources")
    check_grad(query.grad, b["dqw"] * np64(norm.weight), torch.float32, "dquery")


@pytest.mark.parametrize("D", [4096, 3072], ids=["workgroup", "row_per_wave"])
def test_query_gradient_is_deterministic(gpu, D):
    S, B, T = 8, 4, 512
    policy = _capi.POLICY_STREAM if D == 3072 else _capi.POLICY_WORKGROUP
    want = "attnres_route_bwd_stream_c6_s8" if D == 3072 else "attnres_route_bwd_bf_gbf_s8_v1"
    assert _bwd_kernel_name(S, B * T, D, policy) == want
    buf, query, gain, G = make_case(gpu, S, 0, B, T, D, torch.bfloat16, seed=5)
    res = []
    prev = _capi.set_kernel_policy(policy)
    try:
        for _ in range(2):
            q = query.clone().requires_grad_(True)
            out = kotodama_amd.route_static(buf, q, Norm(gain.clone(), 1e-5),
                                            torch.ones(S, dtype=torch.bool, device=gpu), S)
            (out.float() * G).sum().backward()
            res.append(q.grad.clone())
    finally:
        _capi.set_kernel_policy(prev)
    assert torch.equal(res[0], res[1])


def test_capi_backward_argument_errors(gpu):
    lib = _capi.lib()
    x = torch.zeros(4, 256, device=gpu)
    q = torch.zeros(256, device=gpu)
    arr = _capi.pointer_array([x.data_ptr()])
    garr = _capi.pointer_array([x.data_ptr()])
    ws = torch.empty(16, device=gpu)
    # workspace too small
    rc = lib.attnres_route_bwd(arr, 1, 4, 256, 256, _capi.DTYPE_F32, q.data_ptr(), None, _capi.DTYPE_F32, 1e-5,
                               x.data_ptr(), _capi.DTYPE_F32, 256, None, garr, 256, ws.data_ptr(), 64, None, None,
                               None)
    assert rc == _capi.ERR_ARG and b"workspace" in lib.attnres_last_error()
    # S = 0 has nothing to differentiate
    rc = lib.attnres_route_bwd(arr, 0, 4, 256, 256, _capi.DTYPE_F32, q.data_ptr(), None, _capi.DTYPE_F32, 1e-5,
                               x.data_ptr(), _capi.DTYPE_F32, 256, None, garr, 256, ws.data_ptr(), 64, None, None,
                               None)
    assert rc == _capi.ERR_UNSUPPORTED
    # grad_gain without gain
    rc = lib.attnres_route_bwd(arr, 1, 4, 256, 256, _capi.DTYPE_F32, q.data_ptr(), None, _capi.DTYPE_F32, 1e-5,
                               x.data_ptr(), _capi.DTYPE_F32, 256, None, garr, 256, ws.data_ptr(), 64, None,
                               q.data_ptr(), None)
    assert rc == _capi.ERR_ARG


@pytest.mark.parametrize("S", [5, 8])
@pytest.mark.parametrize("kernel", ["row_per_wave", "workgroup"])
def test_full_size_backward_properties(gpu, S, kernel):
    # the 3B prefill shape (B=8, T=4096, D=3072), bf16, at two source counts, through
    # the row-per-wave kernel (AUTO) and the two-chunks-per-thread workgroup kernel
    # (checked through the kernel-name query)
    w = workloads.get("cfg2")
    policy = _capi.POLICY_AUTO if kernel == "row_per_wave" else _capi.POLICY_WORKGROUP
    want = f"attnres_route_bwd_stream_c6_s{S}" if kernel == "row_per_wave" else f"attnres_route_bwd_bf_gbf_s{S}_v2"
    assert _bwd_kernel_name(S, w.tokens, w.hidden, policy) == want
    prev = _capi.set_kernel_policy(policy)
    try:
        _full_size_backward(gpu, w, S)
    finally:
        _capi.set_kernel_policy(prev)


def test_full_size_8b_backward(gpu):
    # config 3's training backward at full size (B=4, T=4096, D=4096, S=9, bf16,
    # peaky queries and source scales from log-uniform[0.1, 10]) through the kernel
    # AUTO launches for it: the one-chunk row-per-workgroup S = 9 instance, the only
    # hot instance compiled under a register cap that spills a few dwords
    w = workloads.get("cfg3")
    assert _bwd_kernel_name(9, w.tokens, w.hidden, _capi.POLICY_AUTO) == "attnres_route_bwd_bf_gbf_s9_v1"
    prev = _capi.set_kernel_policy(_capi.POLICY_AUTO)
    try:
        _full_size_backward(gpu, w, 9)
    finally:
        _capi.set_kernel_policy(prev)


def _full_size_backward(gpu, w, S):
    pool = workloads.make_pool(w, gpu, 3)
    q, gn = workloads.make_params(w, gpu, 3, 1)
    eps = w.eps
    buf = pool[:S].detach().clone().requires_grad_(True)
    del pool
    query = q[0].clone().requires_grad_(True)
    norm = Norm(gn[0].clone(), eps)
    n, D = buf[0].numel() // buf.shape[-1], buf.shape[-1]
    gen = torch.Generator(device=gpu).manual_seed(11)
    G = torch.randn(buf.shape[1:], device=gpu, generator=gen).to(torch.bfloat16).float()
    gl = torch.randn(buf.shape[1:-1], device=gpu, generator=gen)
    print(f"full-size backward S={S} N={n} D={D}", flush=True)
    res = ops.route(buf, S, query, norm.weight, eps, torch.bfloat16, True, False)
    (res[0][0].float() * G).sum().add_((res[2][0] * gl).sum()).backward()
    torch.cuda.synchronize()

    # fp32 torch restatement of the backward on every row
    with torch.no_grad():
        x = buf.detach().reshape(S, n, D).float()
        Gf = G.reshape(n, D)
        qw = (query.detach() * norm.weight.detach()).float()  # bf16 product, as the model folds it
        r = torch.rsqrt(x.pow(2).mean(-1) + eps)
        l = torch.einsum("snd,d->sn", x, qw) * r
        w_ = torch.softmax(l, dim=0)
        a = torch.einsum("snd,nd->sn", x, Gf)
        o = (w_ * a).sum(0)
        dl = w_ * (gl.reshape(1, n) + a - o)
        dqw = torch.einsum("sn,snd->d", dl * r, x)
        # every row: x_s . dx_s = w_s a_s + dl_s l_s eps r_s^2 (logits are scale-invariant up to eps)
        dx = buf.grad.reshape(S, n, D).float()
        lhs = (x * dx).sum(-1)
        rhs = w_ * a + dl * l * eps * r * r
        scale = (x.abs() * dx.abs()).sum(-1) + 1e-30
        rel = ((lhs - rhs).abs() / scale).max().item()
        del dx
    assert rel < 1e-2, f"scale identity violated: rel {rel:.3e}"
    # the query and gain gradients (sums over all rows)
    for got, ref, label in ((query.grad, dqw * norm.weight.detach().float(), "dquery"),
                            (norm.weight.grad, dqw * query.detach().float(), "dgain")):
        g64, r64 = np64(got), ref.double().cpu().numpy()
        tol = bf16_ulp(r64) + 1e-3 * np.abs(r64).max()
        assert (np.abs(g64 - r64) <= tol).all(), f"{label}: worst err {np.abs(g64 - r64).max():.3e}"
    # sampled rows against the float64 oracle, elementwise: the first, middle and last
    # rows (the grid-stride loop's first and last iterations) plus 96 at random
    fixed = {0, 1, n // 2 - 1, n // 2, n - 2, n - 1}
    rows = torch.tensor(sorted(fixed | set(np.random.default_rng(S).choice(n, 96, replace=False).tolist())),
                        device=gpu)
    xs = np64(x[:, rows])
    ref = O.route_backward(xs, O.fold_query(np64(query), np64(norm.weight), "bf16"), eps, np64(Gf[rows]),
                           np64(gl.reshape(n)[rows]))
    check_grad(buf.grad.reshape(S, n, D)[:, rows], ref["dx"], torch.bfloat16, "dsources (sampled rows)")
