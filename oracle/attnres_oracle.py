"""CPU oracle for Block AttnRes routing — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or the
timed CPU baseline), never as a code path of the product.  The product
(``kotodama_amd``) never imports it and has no CPU fallback.

Everything here is float64 numpy restated from the reference's own Python
(``/root/reference``, read, not run):

* :func:`fold_query`     ``qw = query * norm.weight``            llama.py:630
* :func:`route`          RMS-normalised depth softmax + mix      llama.py:640-644,
                         lse / aux outputs                       kernels/phase_1.py:43-101
* :func:`route_masked`   the einsum branch over a padded buffer
                         with a boolean slot mask                llama.py:640-644
* :func:`route_backward` gradients of out (and lse) w.r.t. the
                         sources and the folded query           kernels/phase_1.py:104-280
* :func:`merge`          phase-2 online-softmax merge           kernels/phase_2.py:40-57
* :func:`merge_backward` gradients of the merge                 kernels/phase_2.py:60-230
* :func:`schedule`       boundary set, masks, active counts      llama.py:545-571
* :func:`block_forward`  caller order: route -> commit -> add    llama.py:697-715 (742-762)
* :func:`two_phase_forward` serving schedule: phase 1 per block,
                         phase-2 merge per later sublayer        serve.py:113-164
* :func:`bf16_round`     round-to-nearest-even to bfloat16       (torch's bf16 cast)

Parity pinning (every function has checks that do not retype its formula;
see tests/test_oracle.py): closed forms (S=1 copy; zero query -> mean;
x_s = c_s*u with u in {+-1}^D, qw = beta*u gives logit_s = c_s*beta*D /
sqrt(c_s^2+eps)), invariants (scale invariance of logits, permutation
equivariance, weights sum to 1, masked slots exactly 0, gain folding,
phase-2 merge == routing over one more source), a pure-Python brute force on
tiny shapes, the schedule tables derived by hand from llama.py:545-571, the
two-phase schedule equal to the one-pass caller loop in float64 (the merge
identity at every merged sublayer; the leading-layer skip as a shifted
one-pass loop), and for the backward central finite differences plus float64
torch autograd through the einsum branch's op sequence.
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence

import numpy as np


# ------------------------------------------------------------------ dtypes --


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even); returns float32 values.

    bf16 keeps the top 16 bits of an IEEE float32.  Rounding adds half of the
    dropped 16-bit field (0x7FFF) plus the lowest kept bit (ties to even)
    before truncating.  NaN stays NaN; infinities stay infinite.
    """
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(f)
    if nan.any():
        out[nan] = np.nan
    return out


def round_to(x, dtype: str) -> np.ndarray:
    """Round float values to ``dtype`` ('bf16', 'f32' or 'f64') as float64."""
    if dtype == "bf16":
        return bf16_round(x).astype(np.float64)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32).astype(np.float64)
    if dtype == "f64":
        return np.asarray(x, dtype=np.float64)
    raise ValueError(dtype)


# ------------------------------------------------------------------ fold --


def fold_query(query, gain=None, param_dtype: str = "f32") -> np.ndarray:
    """Effective pseudo-query ``qw = query * norm.weight`` (llama.py:630).

    The reference multiplies in the parameter dtype, so the product is
    rounded to it (a bf16 model folds in bf16; serve.py:85-92 folds the same
    way before stacking the queries).
    """
    q = np.asarray(query, dtype=np.float64)
    if gain is None:
        return round_to(q, param_dtype)
    g = np.asarray(gain, dtype=np.float64)
    # fp32 product, then rounding to the parameter dtype: what torch does for
    # a bf16 or fp32 elementwise multiply.
    prod = (q.astype(np.float32) * g.astype(np.float32)).astype(np.float64)
    return round_to(prod, param_dtype)


# ----------------------------------------------------------------- route --


def route(sources, qw, eps: float) -> dict:
    """Routing over S active sources (llama.py:640-644; kernels/phase_1.py:43-101).

    sources : (S, N, D) array (any float dtype; computed in float64)
    qw      : (D,) or (Q, D) folded pseudo-queries
    Returns out (Q, N, D), weights (Q, S, N), lse (Q, N), inv_rms (N, S),
    logits (Q, N, S).  With S == 0 every output is NaN (softmax over an empty
    set), as in the reference with an all-false mask.
    """
    x = np.asarray(sources, dtype=np.float64)
    q = np.asarray(qw, dtype=np.float64)
    if q.ndim == 1:
        q = q[None, :]
    S, N, D = x.shape
    Q = q.shape[0]
    if S == 0:
        nan = np.full
        return {
            "out": nan((Q, N, D), np.nan),
            "weights": np.zeros((Q, 0, N)),
            "lse": nan((Q, N), np.nan),
            "inv_rms": np.zeros((N, 0)),
            "logits": np.zeros((Q, N, 0)),
        }
    inv_rms = 1.0 / np.sqrt(np.mean(x * x, axis=-1) + eps)  # (S, N)
    dots = np.einsum("snd,qd->qsn", x, q)  # (Q, S, N)
    logits = dots * inv_rms[None]  # (Q, S, N)
    m = logits.max(axis=1, keepdims=True)
    e = np.exp(logits - m)
    z = e.sum(axis=1, keepdims=True)
    w = e / z  # (Q, S, N)
    out = np.einsum("qsn,snd->qnd", w, x)
    lse = (m + np.log(z))[:, 0, :]
    return {
        "out": out,
        "weights": w,
        "lse": lse,
        "inv_rms": inv_rms.T.copy(),
        "logits": np.transpose(logits, (0, 2, 1)).copy(),
    }


def route_masked(buf, qw, eps: float, active_mask) -> dict:
    """The einsum branch verbatim in structure: all max_S slots of a padded
    buffer, inactive ones masked to -inf before the softmax (llama.py:640-644).

    buf (max_S, N, D); active_mask (max_S,) bool.  Returns out (N, D) and
    weights (max_S, N) for one query.
    """
    x = np.asarray(buf, dtype=np.float64)
    q = np.asarray(qw, dtype=np.float64)
    mask = np.asarray(active_mask, dtype=bool)
    rs = 1.0 / np.sqrt(np.mean(x * x, axis=-1) + eps)  # (max_S, N)
    logits = np.einsum("snd,d->sn", x, q) * rs
    logits = np.where(mask[:, None], logits, -np.inf)
    with np.errstate(invalid="ignore"):
        m = logits.max(axis=0, keepdims=True)
        e = np.exp(logits - m)
        w = e / e.sum(axis=0, keepdims=True)
        out = np.einsum("sn,snd->nd", w, x)
    return {"out": out, "weights": w}


def merge(partial, q, inter, inter_lse, eps: float) -> dict:
    """Phase-2 merge (kernels/phase_2.py:40-57).

    inv_rms = rsqrt(mean(p^2)+eps); logit = (p.q)*inv_rms;
    pi = sigmoid(logit - inter_lse); out = inter + pi*(p - inter).
    """
    p = np.asarray(partial, dtype=np.float64)
    qv = np.asarray(q, dtype=np.float64)
    it = np.asarray(inter, dtype=np.float64)
    lse = np.asarray(inter_lse, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(p * p, axis=-1) + eps)
    logit = (p @ qv) * inv
    pi = 1.0 / (1.0 + np.exp(-(logit - lse)))
    out = it + pi[..., None] * (p - it)
    return {"out": out, "logit": logit, "inv_rms": inv}


def merge_backward(partial, q, inter, inter_lse, eps: float, grad_out) -> dict:
    """Gradients of the phase-2 merge (kernels/phase_2.py:60-230).

    With pi = sigmoid(logit - lse), a = G.(p - inter) and gl = pi (1 - pi) a
    (= dL/dlogit):  dinter = (1 - pi) G;  dlse = -gl;
    dp = pi G + gl (r q - logit r^2 p / D);  dq = sum over rows of gl r p.
    Returns dpartial, dinter (N, D), dlse (N,), dq (D,).
    """
    p = np.asarray(partial, dtype=np.float64)
    qv = np.asarray(q, dtype=np.float64)
    it = np.asarray(inter, dtype=np.float64)
    lse = np.asarray(inter_lse, dtype=np.float64)
    g = np.asarray(grad_out, dtype=np.float64)
    D = p.shape[-1]
    r = 1.0 / np.sqrt(np.mean(p * p, axis=-1) + eps)
    logit = (p @ qv) * r
    # pi and 1 - pi each from its own exponential (1 - pi = sigmoid(lse - logit)):
    # 1.0 - pi cancels to nothing as pi -> 1, where dinter and pi (1 - pi) are small
    with np.errstate(over="ignore"):
        pi = 1.0 / (1.0 + np.exp(-(logit - lse)))
        qi = 1.0 / (1.0 + np.exp(logit - lse))
    a = np.sum(g * (p - it), axis=-1)
    gl = pi * qi * a
    dp = pi[..., None] * g + gl[..., None] * (r[..., None] * qv - (logit * r * r / D)[..., None] * p)
    return {
        "dpartial": dp,
        "dinter": qi[..., None] * g,
        "dlse": -gl,
        "dq": np.einsum("n,nd->d", (gl * r).reshape(-1), p.reshape(-1, D)),
    }


# -------------------------------------------------------------- schedule --


def schedule(num_layers: int, n_blocks: Optional[int] = None, boundaries: Optional[Iterable[int]] = None) -> dict:
    """Block boundaries and per-routing-point source counts (llama.py:545-571).

    * explicit ``boundaries`` win; otherwise the boundary set is
      ``range(0, L, ceil(L / n_blocks))``;
    * ``max_sources`` = number of boundaries + 1 (the partial slot);
    * routing point 2i (pre-attention) sees n_committed + 1 sources, then
      layer i commits if it is a boundary, then point 2i+1 (pre-MLP) sees the
      new n_committed + 1; the final point 2L sees all.
    Returns boundary_set, max_sources, masks ((2L+1, max_S) bool),
    active_counts (list of 2L+1 ints) and commit_before (2L+1 bools: the
    routing point directly follows a commit).
    """
    if boundaries is not None:
        bset = frozenset(int(b) for b in boundaries)
    else:
        if not n_blocks:
            raise ValueError("need n_blocks or boundaries")
        block = math.ceil(num_layers / n_blocks)
        bset = frozenset(range(0, num_layers, block))
    max_s = len(bset) + 1
    npts = 2 * num_layers + 1
    masks = np.zeros((npts, max_s), dtype=bool)
    counts = [0] * npts
    commit_before = [False] * npts
    nc = 0
    for i in range(num_layers):
        counts[2 * i] = nc + 1
        if i in bset:
            nc += 1
            commit_before[2 * i + 1] = True
        counts[2 * i + 1] = nc + 1
    counts[npts - 1] = nc + 1
    for j, c in enumerate(counts):
        masks[j, :c] = True
    return {
        "boundary_set": bset,
        "max_sources": max_s,
        "masks": masks,
        "active_counts": counts,
        "commit_before": commit_before,
    }


# --------------------------------------------------------- caller order --


def block_forward(
    embed,
    deltas: Sequence,
    qws: Sequence,
    eps: float,
    num_layers: int,
    boundary_set,
    dtype: str = "f64",
    want_weights: bool = False,
) -> dict:
    """Routing outputs of one forward in the reference's caller order.

    Restates the loop of llama.py:697-715 (and 742-762) with the sublayer
    outputs given: ``deltas[2i]`` is layer i's attention output and
    ``deltas[2i+1]`` its MLP output (the reference computes them from the
    routed h; here they are inputs).  Per layer: route (pre-attn) -> commit
    if i is a boundary (partial joins the committed list, a zero partial
    starts) -> partial += attn -> route (pre-MLP) -> partial += mlp; final
    route.  ``partial`` additions round to ``dtype`` as the model's tensors
    do.  qws[j] is the folded query of routing point j (2L+1 of them).
    Returns outs (list of 2L+1 (N, D) arrays), weights (if asked), the
    committed list and the final partial.
    """
    partial = round_to(embed, dtype)
    committed: list[np.ndarray] = []
    outs, wts = [], []

    def do_route(j: int) -> None:
        r = route(np.stack(committed + [partial]), qws[j], eps)
        outs.append(r["out"][0])
        wts.append(r["weights"][0])

    for i in range(num_layers):
        do_route(2 * i)
        if i in boundary_set:
            committed.append(partial.copy())
            partial = np.zeros_like(partial)
        partial = round_to(partial + np.asarray(deltas[2 * i], dtype=np.float64), dtype)
        do_route(2 * i + 1)
        partial = round_to(partial + np.asarray(deltas[2 * i + 1], dtype=np.float64), dtype)
    do_route(2 * num_layers)
    res = {"outs": outs, "committed": committed, "partial": partial}
    if want_weights:
        res["weights"] = wts
    return res


def two_phase_forward(
    embed,
    deltas: Sequence,
    qws: Sequence,
    eps: float,
    num_layers: int,
    boundary_set,
    dtype: str = "f64",
) -> dict:
    """The serving engine's two-phase forward (serve.py:113-164) with the sublayer outputs given.

    Sublayer j returns ``deltas[j]`` (its routed input h_j is recorded, not
    consumed), as in :func:`block_forward`.  Block ranges of sublayers start at
    ``2*b`` for the sorted boundaries b and end at the next start or at 2L
    (serve.py:117-126; sublayers before the first boundary never run).  Per
    range: one phase-1 routing of the range's folded queries over the committed
    blocks (serve.py:128-136); the range's first sublayer takes the phase-1
    output directly, every later one the phase-2 merge of the running block
    into it (serve.py:138-156); the block's sum joins the blocks
    (serve.py:158).  Final: phase 1 over every block with the last query
    (serve.py:160-166).

    With ``dtype == 'bf16'`` the values are rounded where the reference's
    kernels and tensors round them: the phase-1 output to bf16
    (kernels/phase_1.py:94, always bf16), its lse to fp32, the merge output
    to the inter dtype bf16 (kernels/phase_2.py:54-57), and the running block
    ``curr + delta`` to the model dtype.  With 'f64' nothing is rounded.
    ``qws`` holds the 2L+1 folded queries ``[attn_0, mlp_0, ..., final]``.
    Returns ``h`` ({sublayer j: its routed input (N, D)}), ``pi`` ({j: the
    merge's weight of the running block, merged sublayers only}), ``inter``
    ({j: the phase-1 output row it merged into}), ``final`` and ``blocks``.
    """
    rnd = (lambda a: round_to(a, dtype)) if dtype != "f64" else (lambda a: np.asarray(a, dtype=np.float64))
    rnd_lse = (lambda a: round_to(a, "f32")) if dtype != "f64" else (lambda a: np.asarray(a, dtype=np.float64))
    blocks = [rnd(embed)]
    n_sub = 2 * num_layers
    starts = [2 * b for b in sorted(boundary_set)]
    ranges = [(st, starts[i + 1] if i + 1 < len(starts) else n_sub) for i, st in enumerate(starts)]
    h, pis, inters = {}, {}, {}
    for st, end in ranges:
        p1 = route(np.stack(blocks), np.stack([qws[j] for j in range(st, end)]), eps)
        p1_out, p1_lse = rnd(p1["out"]), rnd_lse(p1["lse"])
        curr = None
        for qo in range(end - st):
            j = st + qo
            if qo == 0:
                h[j] = p1_out[0]
                curr = rnd(deltas[j])
            else:
                mg = merge(curr, qws[j], p1_out[qo], p1_lse[qo], eps)
                h[j] = rnd(mg["out"])
                pis[j] = 1.0 / (1.0 + np.exp(-(mg["logit"] - p1_lse[qo])))
                inters[j] = p1_out[qo]
                curr = rnd(curr + np.asarray(deltas[j], dtype=np.float64))
        blocks.append(curr)
    final = rnd(route(np.stack(blocks), qws[n_sub], eps)["out"][0])
    return {"h": h, "pi": pis, "inter": inters, "final": final, "blocks": blocks}


# ------------------------------------------------------- brute force --


def route_bruteforce(sources, qw, eps: float) -> dict:
    """Scalar-loop routing for tiny shapes (math.fsum), independent of numpy
    broadcasting: used to pin :func:`route` against index/transposition slips."""
    S = len(sources)
    N = len(sources[0])
    D = len(sources[0][0])
    out = [[0.0] * D for _ in range(N)]
    weights = [[0.0] * N for _ in range(S)]
    for t in range(N):
        logit = []
        for s in range(S):
            row = [float(v) for v in sources[s][t]]
            ms = math.fsum(v * v for v in row) / D
            dot = math.fsum(row[k] * float(qw[k]) for k in range(D))
            logit.append(dot / math.sqrt(ms + eps))
        m = max(logit)
        e = [math.exp(lv - m) for lv in logit]
        z = math.fsum(e)
        for s in range(S):
            weights[s][t] = e[s] / z
        for k in range(D):
            out[t][k] = math.fsum(weights[s][t] * float(sources[s][t][k]) for s in range(S))
    return {"out": out, "weights": weights}


# -------------------------------------------------------------- backward --


def route_backward(sources, qw, eps: float, grad_out, grad_lse=None) -> dict:
    """Gradients of the routing output w.r.t. the sources and the folded query.

    For one query: with r_s = rsqrt(mean(x_s^2)+eps), l_s = (x_s.qw) r_s,
    w = softmax(l), out = sum_s w_s x_s, lse = logsumexp(l), G = dL/dout and
    g_lse = dL/dlse (zero when absent),
      a_s  = G . x_s,  o = G . out,  dl_s = w_s (g_lse + a_s - o)
      dx_s = w_s G + dl_s r_s qw - dl_s l_s r_s^2 / D * x_s
      dqw  = sum over tokens and s of dl_s r_s x_s
    (the chain rule through llama.py:640-644; the Triton backward computes the
    same terms, kernels/phase_1.py:104-280).  Returns dx (S, N, D), dqw (D,).
    """
    x = np.asarray(sources, dtype=np.float64)
    q = np.asarray(qw, dtype=np.float64).reshape(-1)
    g = np.asarray(grad_out, dtype=np.float64)
    S, N, D = x.shape
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1) + eps)  # (S, N)
    l = np.einsum("snd,d->sn", x, q) * r
    m = l.max(axis=0, keepdims=True)
    e = np.exp(l - m)
    w = e / e.sum(axis=0, keepdims=True)  # (S, N)
    out = np.einsum("sn,snd->nd", w, x)
    a = np.einsum("nd,snd->sn", g, x)
    o = np.einsum("nd,nd->n", g, out)
    gl = np.zeros(N) if grad_lse is None else np.asarray(grad_lse, dtype=np.float64).reshape(N)
    dl = w * (gl[None, :] + a - o[None, :])
    dx = (
        w[:, :, None] * g[None]
        + (dl * r)[:, :, None] * q[None, None, :]
        - (dl * l * r * r / D)[:, :, None] * x
    )
    dqw = np.einsum("sn,snd->d", dl * r, x)
    return {"dx": dx, "dqw": dqw}
