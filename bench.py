"""Benchmark of MI355X AttnRes routing: achieved HBM GB/s on the 3B prefill sweep.

A step is one forward's routing work at the 3B prefill shape (workload cfg2):
57 routing calls (S = 1..8 per the block schedule) over bf16 sources with
B=8, T=4096, D=3072, sources resident in HBM.  ``value`` = algorithmic bytes
of the step ((S+1) * B*T*D * 2 bytes per call, 68.05 GB) / step time.

Also on the JSON line:
* ``roofline`` — the dominant kernel (the S=8 routing kernel): its algorithmic
  bytes per launch / its average launch time from HIP events around every
  S=8 launch inside the timed region, against MI355X's 8 TB/s HBM peak;
  ``traffic`` is the measured HBM bytes per launch from rocprofv3 FETCH_SIZE
  + WRITE_SIZE counters when a committed summary holds them.
* ``cfg3`` — the 8B prefill shape (S=9, D=4096, B=4, T=4096, 8 calls),
  measured in the same run with the same steps: step time, GB/s and its own
  ``roofline`` block for the S=9 kernel.
* ``cfg5`` — the 3B data-driven blocks (57 calls, S=1..7, B=2), the same way.
* ``cfg2_bwd`` — the backward of cfg2's 57 routing calls (the training path):
  (2S+1) rows per call, with a ``roofline`` block for the S=8 backward.
* ``cfg4`` (the 8B decode step), ``cfg2arena`` (the stack-free prefill) and
  ``cfg2train`` / ``cfg3train`` / ``cfg1btrain`` (the 3B, 8B and 1B training
  steps) — as their own ``--workload`` runs report them, each also recorded in
  a HIP graph and replayed (``hip_graph``: the step without its host launches).
* ``lmstep_proxy`` / ``lmstep_3b`` — a whole training step of the reference's
  model (kotodama_amd.lmstep) at the proxy and 3B shapes with the standard
  residual stream, AttnRes through this package's kernels and AttnRes through
  the reference's routing ops compiled by inductor, as ``--workload lmstep``
  reports them.
* ``cpu_baseline`` — the reference's CPU routing path (oracle/torch_cpu_path:
  the einsum-branch op sequence over the padded buffer, fp32) timed on this
  host on a bounded sample (the whole call schedule over 4096 token rows, at
  least 5 passes, the median), extrapolated to the full step; with the threads
  used, the host's logical CPUs, the CPUs this process may use and the CPU model.

``--workload cfg3|cfg4|cfg5`` measures the other shapes (cfg4 = 8B decode step,
65 fused block steps captured in one HIP graph); ``cfg2serve`` the serving
engine's two-phase routing at the 3B shape (batched phase 1 per block + phase-2
merges: (S + Q) rows per phase-1 call, 3 rows per merge).  ``--pass bwd`` times the
backward of the same routing calls instead (attnres_route_bwd on preallocated
gradient buffers: (2S+1) * B*T*D * 2 algorithmic bytes per call — sources and
dL/dout read, source gradients written; for cfg2serve the batched-query
backward of each phase-1 call, (3S+Q) rows, and the merge backward, 5 rows).
``cfg2arena`` runs the stack-free caller's prefill at the 3B shape (fused block
steps over one arena: (S+3) rows per point, S+2 right after a commit).
``cfg2train`` times the reference's training step on the routing path at the
3B shape (forward under autograd + backward; ``--variant list|stack``,
``--compile`` for torch.compile with inductor), ``cfg3train`` the same at the
8B model's schedule (32 layers, 65 points, S up to 9; D=4096, B=4, T=4096) and
``cfg1btrain`` at the 1B intermediate model's (D=1024, B=4, T=2048).
``--workload lmstep --lm proxy|1b|3b|8b`` times a whole training step of the
reference's Llama-family model (attention, SwiGLU, loss, AdamW; sublayers
compiled by inductor) with each residual stream of ``--residuals``.
``--workload narrow`` times routing steps and calls at hidden 512 / 1024.
``--workload segsum`` times the training step's deferred-gradient segment sums
(attnres_route_bwd_gather_seg) per block count at the 3B and 8B shapes.
``--workload mall`` checks what the 256 MB last-level cache serves of a call's
bytes (the dominant calls back to back vs after other memory traffic).
``--gpus`` above 1 exits: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "AttnRes routing achieved HBM GB/s (% of peak) and tokens/s, 3B/8B shapes"
WORKLOAD_TEXT = {
    "cfg2": "3B prefill sweep: D=3072, B=8, T=4096, 28 layers / 8 blocks, 57 routing calls S=1..8 (sum S=281), bf16 in, fp32 accumulate",
    "cfg3": "8B deepest routing: D=4096, B=4, T=4096, S=9, 8 calls, bf16",
    "cfg4": "8B decode step: T=1, B=256, D=4096, 65 fused block steps (S=1..9) in one HIP graph, bf16",
    "cfg5": "3B data-driven blocks {0,3,7,12,18,23}: D=3072, B=2, T=4096, 57 calls S=1..7 (sum S=267), BOS x20, bf16",
    "copy": "calibration: torch device copy of 1 GiB (bf16), the plain copy kernel that scales rocprof byte counters",
    "cfg2arena": "3B stack-free prefill (llama.py:680-716): 57 fused block steps over one arena (partial update, "
    "commit, route), D=3072, B=8, T=4096, bf16",
    "mall": "cache check: the dominant cfg2 (S=8) and cfg3 (S=9) calls back to back vs after a 512 MiB write, "
    "a 512 MiB read, or a call on a second pool",
    "cfg2serve": "3B serving two-phase routing (serve.py:113-164): 7 blocks of 8 sublayers, one batched phase-1 call "
    "(Q=8, S=1..7) + 7 phase-2 merges per block, final phase 1 (S=8); D=3072, B=8, T=4096, bf16",
    "cfg2train": "3B training step (train.py:610-614 on llama.py:666-716): forward of the 57-point routing loop "
    "under autograd + backward, D=3072, B=8, T=4096, bf16 model; sublayers x*0.5 (no GEMMs)",
    "cfg1btrain": "1B intermediate training step (configs/1b-intermediate.yaml on llama.py:666-716): forward of the "
    "57-point routing loop (28 layers, DD-v1 boundaries 0,3,7,12,21,25, S up to 7) under autograd + backward, D=1024, "
    "B=4, T=2048, bf16 model; sublayers x*0.5 (at this size bound by the host's launches: 4.2 ms of kernels per step)",
    "cfg3train": "8B training step (train.py:610-614 on llama.py:666-716): forward of the 65-point routing loop "
    "(32 layers / 8 blocks, S up to 9) under autograd + backward, D=4096, B=4, T=4096, bf16 model; sublayers x*0.5",
    "lmstep": "whole training step of the reference's Llama-family model (configs/model.yaml; forward, CE + z-loss, "
    "backward, AdamW; bf16) with the standard residual stream, AttnRes through this package's kernels, and AttnRes "
    "through the reference's routing ops compiled by inductor",
    "narrow": "routing steps and calls at hidden 512 / 1024 (the proxy and 1B models), S = 2 and 8, 8192-131072 "
    "rows, bf16",
    "segsum": "the training step's deferred-gradient segment sums alone: 8 points' terms into 1..8 blocks, "
    "D=3072 x 32768 rows and D=4096 x 16384 rows, bf16",
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg2", choices=sorted(WORKLOAD_TEXT))
    ap.add_argument("--pass", dest="pass_", default="fwd", choices=("fwd", "bwd"),
                    help="time the routing forward (default) or its backward")
    ap.add_argument("--variant", default="list", choices=("list", "stack"),
                    help="cfg2train / cfg3train: forward_attn_res under autograd (list) or the reference loop with "
                         "route_static and its per-call stacks (stack)")
    ap.add_argument("--compile", action="store_true",
                    help="cfg2train / cfg3train: run the forward under torch.compile(fullgraph=True, backend='inductor')")
    ap.add_argument("--compile-breaks", action="store_true",
                    help="cfg2train / cfg3train: torch.compile(backend='inductor') without fullgraph, the routing "
                         "points run eagerly as graph breaks (kotodama_amd.engine.defer_under_compile)")
    ap.add_argument("--lm", default="proxy", choices=("proxy", "1b", "3b", "8b"),
                    help="lmstep: the model (configs/model.yaml) and its benchmark batch")
    ap.add_argument("--residuals", default="standard,attnres,torch",
                    help="lmstep: comma-separated residual streams to time (standard, attnres, torch)")
    ap.add_argument("--eager-sublayers", action="store_true", help="lmstep: run the dense sublayers uncompiled")
    ap.add_argument("--graph", action="store_true",
                    help="cfg2train / cfg3train / cfg1btrain (list, eager): also time the step recorded in a HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", action="store_true",
                    help="cfg2: measure the sweep alone, without the other workloads' records (for profiling)")
    ap.add_argument("--cpu-tokens", type=int, default=4096, help="tokens per CPU-baseline sample call")
    return ap.parse_args()


def load_traffic(kernel_tag: str):
    """Measured HBM bytes per launch of the dominant kernel, if profiled (profiles/traffic.json)."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None, None
    try:
        data = json.loads(p.read_text())
        rec = data.get(kernel_tag)
        if rec is None:
            return None, None
        return float(rec["bytes_per_launch"]), rec.get("source")
    except (ValueError, KeyError, TypeError):
        return None, None


def kernel_name(s: int, tokens: int, hidden: int, dtype, queries: int = 1, mode: int = 0) -> str:
    """The kernel symbol the library launches for one routing call of this shape
    (mode: 0 a routing call, 1 a block step accumulating into the partial, 2 a
    block step with a commit)."""
    import ctypes

    from kotodama_amd import _capi, ops

    buf = ctypes.create_string_buffer(128)
    code = ops.dtype_code(dtype)
    _capi.check("attnres_route_kernel_name",
                _capi.lib().attnres_route_kernel_name(s, tokens, hidden, code, code, code, queries, mode, 1, buf,
                                                      len(buf)))
    return buf.value.decode()


def host_cpu_info() -> dict:
    """The host the CPU baseline ran on: logical CPUs, those this process may use, and the model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"host_logical_cpus": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def cpu_baseline(w, tokens: int) -> dict:
    """The reference's CPU path on a bounded sample, extrapolated to one step."""
    import torch

    from oracle import torch_cpu_path as TP

    threads = torch.get_num_threads()
    host = host_cpu_info()
    max_s = max(w.calls)
    g = torch.Generator().manual_seed(0)
    buf = torch.randn((max_s, 1, tokens, w.hidden), generator=g).to(torch.bfloat16).float()
    qw = (torch.randn(w.hidden, generator=g) * w.w_std).to(w.dtype).float()
    masks = {}
    for s in sorted(set(w.calls)):
        masks[s] = torch.zeros(max_s, dtype=torch.bool)
        masks[s][:s] = True
        TP.route_static_cpu(buf, qw, w.eps, masks[s])  # warm-up
    passes: list = []
    # the whole call schedule, in order, per pass; at least 5 passes and ~10 s of CPU work
    while len(passes) < 5 or (sum(passes) < 10.0 and len(passes) < 15):
        t0 = time.perf_counter()
        for s in w.calls:
            TP.route_static_cpu(buf, qw, w.eps, masks[s])
        passes.append(time.perf_counter() - t0)
    scale = w.tokens / tokens
    step_s = statistics.median(passes) * scale
    gbs = w.step_bytes() / step_s / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        **host,
        "kind": "port",
        "sample": (
            f"reference CPU op sequence (llama.py:640-644, fp32, padded max_S={max_s} buffer) over the whole "
            f"{len(w.calls)}-call schedule on {tokens} of the workload's {w.tokens} token rows (median of "
            f"{len(passes)} passes, {sum(passes):.1f} s of CPU work), extrapolated x{scale:.0f}; step {step_s:.2f} s, "
            f"{w.tokens / step_s:.0f} tok/s"
        ),
        "tokens_per_s": round(w.tokens / step_s, 1),
    }


def bench_sweep(w, steps: int, warmup: int, dev):
    """Prefill sweep / single-point configs: one routing call per schedule entry."""
    import torch

    from kotodama_amd import ops, workloads

    pool = workloads.make_pool(w, dev, seed=2)
    q, gn = workloads.make_params(w, dev, seed=2, count=len(w.calls))
    dominant = max(w.calls)
    calls = list(enumerate(w.calls))

    def step(events=None):
        for j, s in calls:
            if events is not None and s == dominant:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                ops.route_call(pool, s, q[j], gn[j], w.eps, w.dtype)
                e1.record()
                events.append((e0, e1))
            else:
                ops.route_call(pool, s, q[j], gn[j], w.eps, w.dtype)

    with torch.inference_mode():
        for _ in range(warmup):  # the same calls as the timed steps, event records included
            step([])
        torch.cuda.synchronize()
        events: list = []
        t0 = time.perf_counter()
        for _ in range(steps):
            step(events)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    dom_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1 in events)
    return elapsed, dominant, dom_ms, w.call_bytes(dominant)


def bench_serve(steps: int, warmup: int, dev):
    """cfg2serve: the routing calls of serve.py:113-164 at the 3B prefill shape.

    Per block of sublayers: one batched phase-1 call over the committed blocks
    for all its pseudo-queries, then a phase-2 merge for every sublayer after
    the first; a final phase-1 call over all blocks.  The running partials fed
    to the merges are synthetic rows generated up front (the sublayers
    themselves are not part of the routing path), so the timed region holds
    only the routing kernels.  Returns (elapsed, step_bytes, merge_ms,
    merge_bytes, p1_ms, p1_bytes) with the per-launch averages of the merges
    and of the deepest phase-1 call.
    """
    import torch

    from kotodama_amd import ops, workloads

    w = workloads.get("cfg2")
    sched = w.schedule
    n, d = w.tokens, w.hidden
    row = n * d * w.elem_bytes
    pool = workloads.make_pool(w, dev, seed=2)  # blocks: embed + committed summaries
    blocks_all = [pool[i] for i in range(pool.shape[0])]
    q, gn = workloads.make_params(w, dev, seed=2, count=sched.num_points)
    pq = (q * gn).contiguous()  # folded in the parameter dtype, stacked [attn_0, mlp_0, ..., final]
    bounds = [2 * b for b in sorted(sched.boundary_set)]
    n_sub = 2 * sched.num_layers
    ranges = [(st, bounds[i + 1] if i + 1 < len(bounds) else n_sub) for i, st in enumerate(bounds)]
    partials = workloads.make_deltas(w, dev, 7, max(e - st for st, e in ranges))
    step_bytes = 0
    for k, (st, e) in enumerate(ranges):
        step_bytes += (k + 1 + (e - st)) * row + (e - st - 1) * 3 * row
    step_bytes += (len(ranges) + 2) * row  # final phase 1 over every block + the partial's block
    deepest = len(ranges)  # S of the last block's phase-1 call

    def step(ev_merge=None, ev_p1=None):
        for k, (st, e) in enumerate(ranges):
            blocks = blocks_all[: k + 1]
            if ev_p1 is not None and k + 1 == deepest:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
            out, _, lse, _, _ = ops.route_list_call(blocks, pq[st:e], None, w.eps, torch.bfloat16, want_lse=True)
            if ev_p1 is not None and k + 1 == deepest:
                e1.record()
                ev_p1.append((e0, e1))
            for qo in range(1, e - st):
                if ev_merge is not None:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                ops.merge_call(partials[qo - 1], pq[st + qo], out[qo], lse[qo], w.eps)
                if ev_merge is not None:
                    e1.record()
                    ev_merge.append((e0, e1))
        ops.route_list_call(blocks_all[: len(ranges) + 1], pq[-1:], None, w.eps, torch.bfloat16, want_lse=True)

    with torch.inference_mode():
        for _ in range(warmup):  # the same calls as the timed steps, event records included
            step([], [])
        torch.cuda.synchronize()
        evm: list = []
        evp: list = []
        t0 = time.perf_counter()
        for _ in range(steps):
            step(evm, evp)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    merge_ms = statistics.mean(a.elapsed_time(b) for a, b in evm)
    p1_ms = statistics.mean(a.elapsed_time(b) for a, b in evp)
    p1_q = ranges[-1][1] - ranges[-1][0]
    return elapsed, step_bytes, merge_ms, 3 * row, p1_ms, (deepest + p1_q) * row


def bwd_kernel_name(s: int, tokens: int, hidden: int, dtype) -> str:
    """Symbol of the single-query backward kernel for this shape (dL/dout in the source dtype)."""
    import ctypes

    from kotodama_amd import _capi, ops

    code = ops.dtype_code(dtype)
    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_bwd_kernel_name",
                _capi.lib().attnres_route_bwd_kernel_name(s, tokens, hidden, code, code, buf, 128))
    return buf.value.decode()


def merge_kernel_name(tokens: int, hidden: int) -> str:
    """Symbol of the kernel a bf16 merge call launches (C-ABI name query)."""
    import ctypes

    from kotodama_amd import _capi

    buf = ctypes.create_string_buffer(128)
    code = _capi.DTYPE_BF16
    _capi.check("attnres_merge_kernel_name",
                _capi.lib().attnres_merge_kernel_name(tokens, hidden, code, code, code, buf, 128))
    return buf.value.decode()


def bwdq_kernel_name(s: int, hidden: int, queries: int) -> str:
    """Symbol of the first kernel of the bf16 batched-query backward for this shape."""
    import ctypes

    from kotodama_amd import _capi

    buf = ctypes.create_string_buffer(128)
    _capi.check("attnres_route_bwd_queries_kernel_name", _capi.lib().attnres_route_bwd_queries_kernel_name(
        s, hidden, _capi.DTYPE_BF16, _capi.DTYPE_BF16, _capi.DTYPE_BF16, queries, buf, 128))
    return buf.value.decode()


def bwd_call_bytes(w, s: int) -> int:
    """Algorithmic bytes of one backward call: S source rows + dL/dout read, S gradient rows written."""
    return (2 * s + 1) * w.tokens * w.hidden * w.elem_bytes


def bench_backward(w, steps: int, warmup: int, dev):
    """The backward of every routing call of the schedule, through the C ABI on preallocated buffers."""
    import torch

    from kotodama_amd import _capi, ops, workloads

    pool = workloads.make_pool(w, dev, seed=2)
    q, gn = workloads.make_params(w, dev, seed=2, count=len(w.calls))
    gen = torch.Generator(device=dev).manual_seed(5)
    gout = torch.randn(pool.shape[1:], device=dev, generator=gen).to(w.dtype)
    grad = torch.empty_like(pool)
    n, d = w.tokens, w.hidden
    ws = torch.empty(_capi.route_bwd_workspace_size(n, d) // 4, device=dev, dtype=torch.float32)
    dq = torch.empty(d, device=dev, dtype=q.dtype)
    dg = torch.empty(d, device=dev, dtype=gn.dtype)
    slot = n * d * pool.element_size()
    src_ptrs = [pool.data_ptr() + i * slot for i in range(pool.shape[0])]
    grad_ptrs = [grad.data_ptr() + i * slot for i in range(pool.shape[0])]
    code = ops.dtype_code(w.dtype)
    pcode = ops.dtype_code(q.dtype)
    dominant = max(w.calls)
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = []
    for j, s in enumerate(w.calls):
        args.append((s, (
            _capi.pointer_array(src_ptrs[:s]), s, n, d, d, code, q[j].data_ptr(), gn[j].data_ptr(), pcode, w.eps,
            gout.data_ptr(), code, d, None, _capi.pointer_array(grad_ptrs[:s]), d, ws.data_ptr(), ws.numel() * 4,
            dq.data_ptr(), dg.data_ptr(), stream)))

    def step(events=None):
        for s, a in args:
            if events is not None and s == dominant:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                _capi.route_bwd(*a)
                e1.record()
                events.append((e0, e1))
            else:
                _capi.route_bwd(*a)

    for _ in range(warmup):  # the same calls as the timed steps, event records included
        step([])
    torch.cuda.synchronize()
    events: list = []
    t0 = time.perf_counter()
    for _ in range(steps):
        step(events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dom_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1 in events)
    step_bytes = sum(bwd_call_bytes(w, s) for s in w.calls)
    return elapsed, dominant, dom_ms, bwd_call_bytes(w, dominant), step_bytes


def bench_serve_backward(steps: int, warmup: int, dev):
    """Backward of cfg2serve's routing calls, through the C ABI on preallocated buffers.

    Per block of sublayers: the batched-query backward of its phase-1 call
    (attnres_route_bwd_queries, Q=8 over S=1..7 blocks) and the backward of
    its 7 merges (attnres_merge_bwd); the final phase-1 call's backward
    (attnres_route_bwd, S=8).  Algorithmic bytes: batched backward (3S + Q)
    rows (S read for the source gradients and again for the query gradients,
    Q output gradients read, S gradients written), merge backward 5 rows
    (partial, inter, dL/dout read; dL/dpartial, dL/dinter written), final
    2S + 1 rows.  Returns (elapsed, step_bytes, deepest_ms, deepest_bytes).
    """
    import torch

    from kotodama_amd import _capi, ops, workloads

    w = workloads.get("cfg2")
    sched = w.schedule
    n, d = w.tokens, w.hidden
    row = n * d * w.elem_bytes
    pool = workloads.make_pool(w, dev, seed=2)
    q, gn = workloads.make_params(w, dev, seed=2, count=sched.num_points)
    pq = (q * gn).contiguous()
    bounds = [2 * b for b in sorted(sched.boundary_set)]
    n_sub = 2 * sched.num_layers
    ranges = [(st, bounds[i + 1] if i + 1 < len(bounds) else n_sub) for i, st in enumerate(bounds)]
    qmax = max(e - st for st, e in ranges)
    gen = torch.Generator(device=dev).manual_seed(6)
    gout = torch.randn((qmax, n, d), device=dev, generator=gen).to(w.dtype)
    glse = torch.randn((qmax, n), device=dev, generator=gen)
    partials = workloads.make_deltas(w, dev, 7, 1)
    grad = torch.empty_like(pool)
    slot = n * d * pool.element_size()
    src_ptrs = [pool.data_ptr() + i * slot for i in range(pool.shape[0])]
    grad_ptrs = [grad.data_ptr() + i * slot for i in range(pool.shape[0])]
    nbw = max(_capi.route_bwd_queries_workspace_size(n, d, k + 1, e - st) for k, (st, e) in enumerate(ranges))
    nbw = max(nbw, _capi.route_bwd_workspace_size(n, d))
    ws = torch.empty(nbw // 4 + 1, device=dev, dtype=torch.float32)
    dq = torch.empty((qmax, d), device=dev, dtype=pq.dtype)
    gp, gi = torch.empty((n, d), device=dev, dtype=w.dtype), torch.empty((n, d), device=dev, dtype=w.dtype)
    gl = torch.empty(n, device=dev, dtype=torch.float32)
    code = ops.dtype_code(w.dtype)
    pcode = ops.dtype_code(pq.dtype)
    stream = torch.cuda.current_stream(dev).cuda_stream
    deepest = len(ranges)
    calls, step_bytes = [], 0
    for k, (st, e) in enumerate(ranges):
        s, nq = k + 1, e - st
        calls.append(("q", s == deepest, (
            _capi.pointer_array(src_ptrs[:s]), s, n, d, d, code, pq[st].data_ptr(), None, nq, pcode, w.eps,
            gout.data_ptr(), code, d, n * d, glse.data_ptr(), _capi.pointer_array(grad_ptrs[:s]), d, ws.data_ptr(),
            ws.numel() * 4, dq.data_ptr(), None, stream)))
        step_bytes += (3 * s + nq) * row
        for qo in range(1, nq):
            calls.append(("m", False, (
                partials[0].data_ptr(), n, d, code, pq[st + qo].data_ptr(), pcode, gout[qo].data_ptr(), code,
                glse[qo].data_ptr(), w.eps, gout[0].data_ptr(), gp.data_ptr(), gi.data_ptr(), gl.data_ptr(),
                ws.data_ptr(), ws.numel() * 4, dq.data_ptr(), stream)))
            step_bytes += 5 * row
    s = len(ranges) + 1
    calls.append(("r", False, (
        _capi.pointer_array(src_ptrs[:s]), s, n, d, d, code, pq[-1].data_ptr(), None, pcode, w.eps,
        gout[0].data_ptr(), code, d, glse[0].data_ptr(), _capi.pointer_array(grad_ptrs[:s]), d, ws.data_ptr(),
        ws.numel() * 4, dq.data_ptr(), None, stream)))
    step_bytes += (2 * s + 1) * row

    def step(events=None):
        for kind, timed, a in calls:
            if events is not None and timed:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
            if kind == "q":
                if _capi.route_bwd_queries(*a) != _capi.OK:
                    raise RuntimeError("batched-query backward unsupported for the serving shape")
            elif kind == "m":
                _capi.merge_bwd(*a)
            else:
                _capi.route_bwd(*a)
            if events is not None and timed:
                e1.record()
                events.append((e0, e1))

    with torch.inference_mode():
        for _ in range(warmup):  # the same calls as the timed steps, event records included
            step([])
        torch.cuda.synchronize()
        events: list = []
        t0 = time.perf_counter()
        for _ in range(steps):
            step(events)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    deepest_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1 in events)
    return elapsed, step_bytes, deepest_ms, (3 * deepest + (ranges[-1][1] - ranges[-1][0])) * row


def arena_step_rows(sched) -> int:
    """Algorithmic rows moved by one pass of fused block steps over an arena:
    the first point reads the partial and writes its output (2 rows); a point
    that updates the partial reads S sources and the delta and writes the
    partial and its output (S + 3); a point right after a block commit starts
    the new partial from the delta, so it reads S - 1 committed blocks and the
    delta (S + 2)."""
    return 2 + sum(s + (2 if commit else 3) for s, commit in zip(sched.active_counts[1:], sched.commit_before[1:]))


def bench_decode(w, steps: int, warmup: int, dev):
    """cfg4: one decode step = 65 fused block steps, captured in a HIP graph."""
    import torch

    from kotodama_amd import workloads
    from kotodama_amd.engine import AttnResRouter

    sched = w.schedule
    L = sched.num_layers
    embed = torch.randn((w.batch, 1, w.hidden), device=dev).to(w.dtype)
    deltas = workloads.make_deltas(w, dev, 4, 2 * L)
    q, gn = workloads.make_params(w, dev, 4, sched.num_points)
    router = AttnResRouter(sched, list(q), list(gn), w.eps)
    arena = router.new_arena((w.batch, 1), w.hidden, w.dtype, dev)
    with torch.inference_mode():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            router.forward(embed, lambda j, h: deltas[j], arena=arena)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            router.forward(embed, lambda j, h: deltas[j], arena=arena)
        for _ in range(warmup):  # as the timed steps, event records included
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
        torch.cuda.synchronize()
        events = []
        t0 = time.perf_counter()
        for _ in range(steps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            events.append((e0, e1))
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    step_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1 in events)
    return elapsed, arena_step_rows(sched) * w.batch * w.hidden * w.elem_bytes, step_ms


def bench_arena(w, steps: int, warmup: int, dev):
    """cfg2arena: the stack-free caller's prefill at the 3B shape (llama.py:680-716
    without the per-call stacked copy): the 57 routing points as fused block
    steps over one arena, each updating the partial from a sublayer output
    (four distinct outputs, reused).  Events around the S = 8 points give the
    dominant kernel's time."""
    import torch

    from kotodama_amd import workloads
    from kotodama_amd.engine import AttnResRouter

    sched = w.schedule
    embed = torch.randn((w.batch, w.seq, w.hidden), device=dev).to(w.dtype)
    deltas = workloads.make_deltas(w, dev, 5, 4)
    q, gn = workloads.make_params(w, dev, 5, sched.num_points)
    router = AttnResRouter(sched, list(q), list(gn), w.eps)
    arena = router.new_arena((w.batch, w.seq), w.hidden, w.dtype, dev)
    top = max(sched.active_counts)

    def step(events=None):
        arena.start(embed)
        delta = None
        for j in range(sched.num_points):
            timed = events is not None and sched.active_counts[j] == top and not sched.commit_before[j]
            if timed:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
            arena.step(q[j], gn[j], w.eps, delta=delta, commit=sched.commit_before[j])
            if timed:
                e1.record()
                events.append((e0, e1))
            delta = deltas[j % 4]

    with torch.inference_mode():
        for _ in range(warmup):
            step([])
        torch.cuda.synchronize()
        events: list = []
        t0 = time.perf_counter()
        for _ in range(steps):
            step(events)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    dom_ms = statistics.mean(e0.elapsed_time(e1) for e0, e1 in events)
    row = w.tokens * w.hidden * w.elem_bytes
    return elapsed, arena_step_rows(sched) * row, top, dom_ms, (top + 3) * row


def bench_copy(steps: int, warmup: int, dev):
    """A plain 1 GiB device copy: its FETCH_SIZE / WRITE_SIZE counters calibrate the routing kernels' ones."""
    import torch

    n = (1 << 30) // 2
    src = torch.randn(n, device=dev).to(torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, 2 * n * 2


def bench_mall(steps: int, warmup: int, dev) -> dict:
    """Does the 256 MB last-level cache (MALL) serve part of a call's bytes?

    The dominant call of cfg2 (S=8) and of cfg3 (S=9) timed with HIP events,
    in alternating rounds, four ways: back to back on one pool (consecutive
    calls of one block read the same sources); with a 512 MiB write between
    launches; with a 512 MiB read between launches (evicts without leaving
    dirty lines); and alternating between two pools of the same shape, so
    every call follows one that touched other memory, as in the model where
    attention and MLP sublayers run between routing calls.
    """
    import torch

    from kotodama_amd import ops, workloads

    flush = torch.ones(256 << 20, dtype=torch.bfloat16, device=dev)  # 512 MiB
    modes = ("back_to_back", "write_flushed", "read_flushed", "alternating_pools")
    out = {}
    for name in ("cfg2", "cfg3"):
        w = workloads.get(name)
        pools = [workloads.make_pool(w, dev, seed=2), workloads.make_pool(w, dev, seed=3)]
        q, gn = workloads.make_params(w, dev, seed=2, count=len(w.calls))
        s = max(w.calls)
        j = w.calls.index(s)
        times = {m: [] for m in modes}
        with torch.inference_mode():
            for rnd in range(4):
                for mode in modes:
                    ev = []
                    for i in range(warmup + steps):
                        if mode == "write_flushed":
                            flush.fill_(float(1 + (rnd + i) % 7))
                        elif mode == "read_flushed":
                            flush.amax()
                        pool = pools[i % 2] if mode == "alternating_pools" else pools[0]
                        e0 = torch.cuda.Event(enable_timing=True)
                        e1 = torch.cuda.Event(enable_timing=True)
                        e0.record()
                        ops.route_call(pool, s, q[j], gn[j], w.eps, w.dtype)
                        e1.record()
                        if i >= warmup:
                            ev.append((e0, e1))
                    torch.cuda.synchronize()
                    times[mode] += [a.elapsed_time(b) for a, b in ev]
        nbytes = w.call_bytes(s)
        rec = {"kernel": kernel_name(s, w.tokens, w.hidden, w.dtype), "algorithmic_bytes": nbytes,
               "launches_each": steps * 4}
        base = statistics.median(times["back_to_back"])
        for mode, ts in times.items():
            med = statistics.median(ts)
            rec[mode] = {"median_us": round(med * 1e3, 2), "mean_us": round(statistics.mean(ts) * 1e3, 2),
                         "GB/s": round(nbytes / (med * 1e-3) / 1e9, 1), "vs_back_to_back": round(med / base, 4)}
        out[f"{name}_s{s}"] = rec
        del pools, q, gn
        torch.cuda.empty_cache()
    return out


def train_path_bytes(w) -> tuple[int, int]:
    """Algorithmic bytes per step of the kernels the eager training loop runs at
    ``w``'s schedule (bf16, hidden 3072 / 4096: the deferred backward and the
    segment sums), in rows of tokens * hidden * 2 bytes, 16-byte coefficient
    records per token and block, and 4-byte per-token sums.  Forward: a point
    that updates the partial reads S - 1 blocks, the partial and the sublayer
    output and writes the new partial and the routed row; the first point and
    a point after a commit read S and write one.  Backward: a point with
    committed blocks reads its S sources, dL/dout and the next point's partial
    gradient (none at the last point), writes the partial's gradient and its
    records; the first point (S = 1) the same with its one gradient row; at
    the commit of block k the segment sum reads the dL/dout rows of the points
    since the previous commit and their records of blocks 0 .. k, the running
    sums those blocks carry from later segments and block k's row, and writes
    the blocks' running sums (block k's gradient)."""
    sched = w.schedule
    S, C = list(sched.active_counts), list(sched.commit_before)
    P = len(S)
    row = w.tokens * w.hidden * w.elem_bytes
    rec = w.tokens * 16
    tsum = w.tokens * 4
    fwd = bwd = 0
    for j in range(P):
        fwd += (S[j] + 1) * row if (j == 0 or C[j]) else (S[j] + 3) * row
        add = 1 if j < P - 1 else 0
        bwd += (S[j] + 2 + add) * row + ((S[j] - 1) * rec if S[j] >= 2 else 0)
    commits = [j for j in range(P) if C[j]]
    for i in range(len(commits) - 1, -1, -1):
        j0 = commits[i]
        j1 = commits[i + 1] if i + 1 < len(commits) else P
        nb, terms = i + 1, j1 - j0
        carried = nb if i + 1 < len(commits) else 0  # running sums from later segments
        bwd += (terms + carried + 1 + nb) * row + terms * nb * rec + (carried + nb - 1) * tsum
    return fwd, bwd


def bench_segsum(steps: int, warmup: int, dev) -> dict:
    """attnres_route_bwd_gather_seg, the training loop's deferred-gradient sums, per block count:
    8 points' terms summed into blocks 0..NB-1 (blocks 0..NB-2 continuing running sums, the last one
    finished with x and an addend), at the 3B (D=3072, 32768 rows) and 8B (D=4096, 16384 rows)
    shapes; HIP events around each launch, median over the steps."""
    import torch

    from kotodama_amd import _capi

    P = 8
    out = {}
    for d, n in ((3072, 32768), (4096, 16384)):
        g = torch.Generator(device=dev).manual_seed(d)
        gouts = [torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(P)]
        qfolds = [(torch.randn(d, generator=g, device=dev) * 0.05).to(torch.bfloat16) for _ in range(P)]
        coefs = [torch.randn((n, 8, 4), generator=g, device=dev) * 0.1 for _ in range(P)]
        x = torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16)
        addend = torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16)
        part_in = [torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(7)]
        csum_in = [torch.randn(n, generator=g, device=dev) for _ in range(7)]
        part_out = [torch.empty((n, d), device=dev, dtype=torch.bfloat16) for _ in range(8)]
        csum_out = [torch.empty(n, device=dev) for _ in range(8)]
        row = n * d * 2
        rows = {}
        for nb in range(1, 9):
            args = (nb, n, d, _capi.DTYPE_BF16, P, _capi.pointer_array([t.data_ptr() for t in gouts]), d,
                    _capi.pointer_array([c.data_ptr() for c in coefs]), _capi.int64_array([32] * P),
                    _capi.pointer_array([q.data_ptr() for q in qfolds]),
                    _capi.pointer_array([part_in[k].data_ptr() if k < nb - 1 else None for k in range(nb)]),
                    _capi.pointer_array([csum_in[k].data_ptr() if k < nb - 1 else None for k in range(nb)]),
                    _capi.pointer_array([part_out[k].data_ptr() for k in range(nb)]),
                    _capi.pointer_array([csum_out[k].data_ptr() if k < nb - 1 else None for k in range(nb)]),
                    x.data_ptr(), d, addend.data_ptr(), d, torch.cuda.current_stream(dev).cuda_stream)
            for _ in range(warmup):
                _capi.route_bwd_gather_seg(*args)
            torch.cuda.synchronize()
            ts = []
            for _ in range(steps):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                _capi.route_bwd_gather_seg(*args)
                b.record()
                b.synchronize()
                ts.append(a.elapsed_time(b))
            ms = statistics.median(ts)
            # read: the P dL/dout rows, NB-1 running sums, x, the addend, the P x NB records and NB-1
            # x-coefficient sums; written: NB rows and NB-1 coefficient sums
            nbytes = (P + (nb - 1) + 2 + nb) * row + P * n * nb * 16 + 2 * (nb - 1) * n * 4
            gbs = nbytes / (ms * 1e-3) / 1e9
            rows[f"b{nb}"] = {"us": round(ms * 1e3, 1), "algorithmic_bytes": nbytes, "GB/s": round(gbs, 1),
                              "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        out[f"d{d}"] = rows
        del gouts, qfolds, coefs, x, addend, part_in, csum_in, part_out, csum_out
        torch.cuda.empty_cache()
    return out


def bench_train(steps: int, warmup: int, dev, variant: str, compiled: bool, name: str = "cfg2train",
                breaks: bool = False, graph: bool = False) -> dict:
    """cfg2train / cfg3train: the reference's training step on the routing path at the 3B / 8B shape.

    A model with the reference's AttnRes attributes (workloads.TrainingModel:
    bf16 queries and gains, trainable; sublayers ``x * 0.5``) runs the forward
    under autograd on a bf16 embedding that requires grad, then
    ``out.backward(G)`` (train.py:610-614: ``model(...)`` then
    ``loss.backward()``).  ``variant`` "list": ``forward_attn_res`` (the
    stack-free caller, list-based routing calls); "stack": the reference's loop
    with only ``_route_static`` swapped (per-call pad + stack, clones at
    commits).  HIP events split each step into forward and backward.
    """
    import torch

    from kotodama_amd import engine, routing, workloads

    w = workloads.get(name if name in ("cfg3train", "cfg1btrain") else "cfg2")
    model = workloads.TrainingModel(w, dev, seed=8)
    gen = torch.Generator(device=dev).manual_seed(9)
    embed = torch.randn((w.batch, w.seq, w.hidden), generator=gen, device=dev).to(w.dtype).requires_grad_(True)
    G = torch.randn((w.batch, w.seq, w.hidden), generator=gen, device=dev).to(w.dtype)
    if variant == "stack":
        def fwd(m, x):
            return workloads.stacked_training_forward(m, x, routing.route_static)
    else:
        def fwd(m, x):
            return engine.forward_attn_res(m, x)
    engine.defer_under_compile(breaks)
    if compiled or breaks:
        torch._dynamo.reset()
        fwd = torch.compile(fwd, fullgraph=not breaks, backend="inductor")

    def step(events):
        model.zero_grad(set_to_none=True)
        embed.grad = None
        e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        e0.record()
        out = fwd(model, embed)
        e1.record()
        out.backward(G)
        e2.record()
        events.append((e0, e1, e2))

    t_first = time.perf_counter()
    for i in range(warmup):
        print(f"{name} {variant}{' compiled' if compiled else ''}{' compiled (graph breaks)' if breaks else ''}: "
              f"warm-up step {i}", flush=True)
        step([])
        torch.cuda.synchronize()
    first_s = time.perf_counter() - t_first
    torch.cuda.reset_peak_memory_stats(dev)
    events: list = []
    t0 = time.perf_counter()
    for _ in range(steps):
        step(events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    fwd_ms = statistics.mean(a.elapsed_time(b) for a, b, _ in events)
    bwd_ms = statistics.mean(b.elapsed_time(c) for _, b, c in events)
    row = w.tokens * w.hidden * w.elem_bytes
    fwd_rows = sum(s + 1 for s in w.calls)
    bwd_rows = sum(2 * s + 1 for s in w.calls)
    ms = elapsed * 1e3 / steps
    extra = {}
    if variant == "list" and not compiled and not breaks:
        # what the eager list path's kernels move (fused forward points, deferred backward + per-block sums)
        fb, bb = train_path_bytes(w)
        extra = {"path_kernel_bytes": {"fwd": fb, "bwd": bb},
                 "path_kernel_GB/s": {"fwd": round(fb / (fwd_ms * 1e-3) / 1e9, 1),
                                      "bwd": round(bb / (bwd_ms * 1e-3) / 1e9, 1)}}
    if graph and variant == "list" and not compiled and not breaks:
        # the same step recorded in a HIP graph (no host synchronisation or memset in it) and replayed
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model.zero_grad(set_to_none=True)
            embed.grad = None
            fwd(model, embed).backward(G)
        torch.cuda.current_stream().wait_stream(side)
        model.zero_grad(set_to_none=True)
        embed.grad = None
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fwd(model, embed).backward(G)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        gms = (time.perf_counter() - t0) * 1e3 / steps
        extra["hip_graph"] = {"ms_per_step": round(gms, 4), "tokens_per_s": round(w.tokens / (gms * 1e-3), 1)}
        del g
    return {"ms_per_step": round(ms, 4), "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
            "routing_kernel_bytes": {"fwd": fwd_rows * row, "bwd": bwd_rows * row},
            "routing_kernel_bytes_per_ms": round((fwd_rows + bwd_rows) * row / ms / 1e6, 1), **extra,
            "tokens_per_s": round(w.tokens / (ms * 1e-3), 1),
            "peak_allocated_GiB": round(torch.cuda.max_memory_allocated(dev) / 2**30, 2),
            "warmup_s": round(first_s, 2)}


def bench_narrow(steps: int, warmup: int, dev) -> dict:
    """narrow: single training-path routing steps (attnres_route_step, the fused
    forward of a routing point: S - 1 committed blocks, the partial and the
    sublayer output read, the routed row and the updated partial written; (S+3)
    rows) and routing calls over S sources ((S+1) rows) at the narrow widths of
    the proxy and 1B models (hidden 512 / 1024, bf16), S = 2 and 8, 8192-131072
    rows: HIP events over ``steps`` back-to-back calls per case."""
    import torch

    from kotodama_amd import ops

    out = {}
    g = torch.Generator(device=dev).manual_seed(21)
    with torch.no_grad():
        for d in (512, 1024):
            for n in (8192, 32768, 131072):
                for S in (2, 8):
                    com = [torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16) for _ in range(S - 1)]
                    part = torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16)
                    delta = torch.randn((n, d), generator=g, device=dev).to(torch.bfloat16)
                    q = (torch.randn(d, generator=g, device=dev) * 0.05).to(torch.bfloat16)
                    gain = torch.ones(d, device=dev, dtype=torch.bfloat16)
                    calls = {"step": lambda: ops._route_rows_step(com, part, delta, q, gain, 1e-5, torch.bfloat16),
                             "route": lambda: ops._route_rows_forward(com + [part], q, gain, 1e-5, torch.bfloat16)}
                    for kind, fn in calls.items():
                        for _ in range(warmup):
                            fn()
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record()
                        for _ in range(steps):
                            fn()
                        e1.record()
                        torch.cuda.synchronize()
                        us = e0.elapsed_time(e1) * 1e3 / steps
                        rows = S + 3 if kind == "step" else S + 1
                        out[f"{kind}_d{d}_n{n}_s{S}"] = {"us": round(us, 2),
                                                         "GB/s": round(rows * n * d * 2 / (us * 1e-6) / 1e9, 1)}
                    del com, part, delta
    return out


def reference_routing_loop():
    """A comparator for the whole-step timing, not part of the package: the
    reference's training caller (llama.py:666-716) with its own routing ops
    (``_route_static``'s PyTorch path, llama.py:630-644), compiled by inductor
    for the fixed max_S shape as the reference intends (llama.py:615-616).  The
    padded source list is stacked inside the compiled function, so inductor may
    fuse the stack into the routing reductions as a whole-model compile would;
    the commits' clones (llama.py:701-702) are left out for the same reason
    (a compiled graph drops them); the partial's adds stay eager adds."""
    import torch

    def route(srcs, query, gain, eps: float, mask):
        buf = torch.stack(srcs, 0)
        rsqrt = torch.rsqrt(buf.pow(2).mean(-1) + eps)
        logits = (buf * (query * gain)).sum(-1) * rsqrt
        logits = logits.masked_fill(~mask.view(-1, 1, 1), float("-inf"))
        return (torch.softmax(logits, dim=0).unsqueeze(-1) * buf).sum(0)

    croute = torch.compile(route, dynamic=False)

    def loop(model, embed):
        masks, max_s, bset = model._attn_res_masks, model._attn_res_max_sources, model._attn_res_boundary_set
        committed: list = []
        zero = torch.zeros_like(embed)

        def point(j, partial, query, norm):
            srcs = committed + [partial] + [zero] * (max_s - len(committed) - 1)
            return croute(srcs, query, norm.weight, norm.eps, masks[j])

        partial = embed
        for i, layer in enumerate(model.layers):
            h = point(2 * i, partial, layer.attn_res_query, layer.attn_res_norm)
            if i in bset:
                committed.append(partial)
                partial = zero
            partial = partial + layer.attn(layer.attn_norm(h), model.rope_cos, model.rope_sin, None)
            h = point(2 * i + 1, partial, layer.mlp_res_query, layer.mlp_res_norm)
            partial = partial + layer.ffn(layer.ffn_norm(h))
        return point(2 * len(model.layers), partial, model.final_res_query, model.final_res_norm)

    return loop


def bench_lmstep(steps: int, warmup: int, dev, lm: str, residuals, compiled: bool = True) -> dict:
    """lmstep: one training step of the reference's Llama-family model
    (kotodama_amd.lmstep: forward, cross-entropy + z-loss, backward, AdamW step;
    train.py:610-640) with each residual stream in ``residuals``: "standard"
    (x + f(norm(x))), "attnres" (this package's routing kernels) and "torch"
    (the reference's routing ops compiled by inductor, :func:`reference_routing_loop`).
    The dense sublayers are the same torch functions in every variant, compiled
    by inductor unless ``compiled`` is false.  HIP events split each step into
    forward (with the loss), backward and optimizer step."""
    import torch

    from kotodama_amd import lmstep

    c = lmstep.PRESETS[lm]
    torch.backends.cuda.enable_math_sdp(False)  # SDPA runs a fused kernel or raises
    torch._dynamo.reset()
    lmstep.compile_sublayers(compiled)
    ids, labels = lmstep.make_batch(c, dev)
    loops = {"standard": "standard", "attnres": "attnres", "torch": reference_routing_loop()}
    out = {"model": c.name, "hidden": c.hidden_size, "layers": c.num_layers, "batch": c.batch, "seq": c.seq,
           "vocab": c.vocab_size, "routing_points": 2 * c.num_layers + 1, "sublayers_compiled": compiled}
    for name in residuals:
        residual = loops[name]
        model = lmstep.LanguageModel(c, dev, seed=3)  # every variant starts from the same weights
        opt = lmstep.optimizer(model)
        out.setdefault("params_M", round(sum(p.numel() for p in model.parameters()) / 1e6, 1))
        out.setdefault("blocks", len(model._attn_res_boundary_set))

        def step(events):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            opt.zero_grad(set_to_none=True)
            e[0].record()
            loss = model(ids, labels, residual)
            e[1].record()
            loss.backward()
            e[2].record()
            opt.step()
            e[3].record()
            events.append(e)
            return loss

        t_first = time.perf_counter()
        for i in range(warmup):
            print(f"lmstep {lm} {name}: warm-up step {i}", flush=True)
            step([])
            torch.cuda.synchronize()
        first_s = time.perf_counter() - t_first
        torch.cuda.reset_peak_memory_stats(dev)
        events: list = []
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step(events)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        split = [statistics.mean(e[k].elapsed_time(e[k + 1]) for e in events) for k in range(3)]
        out[name] = {"ms_per_step": round(ms, 3), "tokens_per_s": round(c.tokens / (ms * 1e-3), 1),
                     "fwd_ms": round(split[0], 3), "bwd_ms": round(split[1], 3), "opt_ms": round(split[2], 3),
                     "loss": round(float(loss), 4),
                     "peak_allocated_GiB": round(torch.cuda.max_memory_allocated(dev) / 2**30, 2),
                     "warmup_s": round(first_s, 1)}
        print(f"lmstep {lm} {name}: {json.dumps(out[name])}", flush=True)
        del model, opt
        torch.cuda.empty_cache()
    base = out.get("standard", {}).get("ms_per_step")
    if base:
        for name in residuals:
            if name != "standard":
                out[name]["overhead_vs_standard"] = round(out[name]["ms_per_step"] / base - 1.0, 4)
    return out


def secondary_sweep(name: str, steps: int, warmup: int, dev) -> dict:
    """Another sweep workload (cfg3: the 8B prefill shape, S=9, 8 calls; cfg5: the 3B data-driven
    blocks, 57 calls) measured in the same run as cfg2, with its own roofline block."""
    from kotodama_amd import workloads

    w = workloads.get(name)
    elapsed, dominant, dom_ms, dom_bytes = bench_sweep(w, steps, warmup, dev)
    ms = elapsed * 1e3 / steps
    gbs = w.step_bytes() / (ms * 1e-3) / 1e9
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic, traffic_src = load_traffic(f"{name}_s{dominant}")
    roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": kernel_name(dominant, w.tokens, w.hidden, w.dtype), "algorithmic_bytes": dom_bytes,
            "avg_ms": round(dom_ms, 4)}
    if traffic_src:
        roof["traffic_source"] = traffic_src
    return {"workload": WORKLOAD_TEXT[name], "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
            "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w.tokens / (ms * 1e-3), 1), "algorithmic_bytes_per_step": w.step_bytes(),
            "roofline": roof}


def secondary_backward(name: str, steps: int, warmup: int, dev) -> dict:
    """The backward of a sweep workload's routing calls (the training path), measured in the same run."""
    from kotodama_amd import workloads

    w = workloads.get(name)
    elapsed, dominant, dom_ms, dom_bytes, step_bytes = bench_backward(w, steps, warmup, dev)
    ms = elapsed * 1e3 / steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic, traffic_src = load_traffic(f"bwd_{name}_s{dominant}")
    roof = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": bwd_kernel_name(dominant, w.tokens, w.hidden, w.dtype) + " (+ attnres_reduce_dqw_cols)",
            "algorithmic_bytes": dom_bytes, "avg_ms": round(dom_ms, 4)}
    if traffic_src:
        roof["traffic_source"] = traffic_src
    return {"workload": "backward of: " + WORKLOAD_TEXT[name], "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms, 4), "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w.tokens / (ms * 1e-3), 1), "algorithmic_bytes_per_step": step_bytes,
            "roofline": roof}


def secondary_decode(steps: int, warmup: int, dev) -> dict:
    """cfg4 (the 8B decode step: 65 fused block steps in one HIP graph), measured in the same run."""
    from kotodama_amd import workloads

    w = workloads.get("cfg4")
    elapsed, step_bytes, graph_ms = bench_decode(w, steps, warmup, dev)
    ms = elapsed * 1e3 / steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    ach = step_bytes / (graph_ms * 1e-3) / 1e9
    return {"workload": WORKLOAD_TEXT["cfg4"], "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
            "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w.batch / (ms * 1e-3), 1), "algorithmic_bytes_per_step": step_bytes,
            "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "one decode step (65 fused attnres_route_bf_d2_s*_v1_q1 launches, HIP graph)",
                         "avg_ms": round(graph_ms, 4)}}


def secondary_arena(steps: int, warmup: int, dev) -> dict:
    """cfg2arena (the stack-free prefill: 57 fused block steps over one arena), measured in the same run."""
    from kotodama_amd import workloads

    w = workloads.get("cfg2")
    elapsed, step_bytes, top, dom_ms, dom_bytes = bench_arena(w, steps, warmup, dev)
    ms = elapsed * 1e3 / steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    ach = dom_bytes / (dom_ms * 1e-3) / 1e9
    return {"workload": WORKLOAD_TEXT["cfg2arena"], "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
            "value": round(gbs, 2), "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w.tokens / (ms * 1e-3), 1), "algorithmic_bytes_per_step": step_bytes,
            "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": kernel_name(top, w.tokens, w.hidden, w.dtype, mode=1) + f" (S={top} points)",
                         "algorithmic_bytes": dom_bytes, "avg_ms": round(dom_ms, 4)}}


def secondary_train(steps: int, warmup: int, dev, name: str = "cfg2train", graph: bool = False) -> dict:
    """cfg2train / cfg3train / cfg1btrain (the 3B / 8B / 1B training step on the routing path, stack-free
    drop-in, eager; with ``graph`` also recorded in a HIP graph), measured in the same run."""
    rec = bench_train(steps, warmup, dev, "list", False, name, graph=graph)
    rb = rec["routing_kernel_bytes"]
    gbs = (rb["fwd"] + rb["bwd"]) / (rec["ms_per_step"] * 1e-3) / 1e9
    return {"workload": WORKLOAD_TEXT[name], "variant": "list (forward_attn_res under autograd)",
            "steps": steps, "warmup": warmup, "value": rec["tokens_per_s"], "unit": "tokens/s",
            "routing_GB/s_over_step": round(gbs, 2), **rec}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X (routing is "
            "per-token and shards over B*T with no communication; see the design notes). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    import torch

    from kotodama_amd import workloads

    dev = torch.device("cuda", 0)
    if args.workload == "copy":
        elapsed, nbytes = bench_copy(args.steps, args.warmup, dev)
        ms = elapsed * 1e3 / args.steps
        print(json.dumps({"workload": WORKLOAD_TEXT["copy"], "bytes_read": nbytes // 2, "bytes_written": nbytes // 2,
                          "ms_per_copy": round(ms, 4), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    if args.workload == "cfg2arena":
        w2 = workloads.get("cfg2")
        elapsed, step_bytes, top, dom_ms, dom_bytes = bench_arena(w2, args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        ach = dom_bytes / (dom_ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "AttnRes stack-free prefill (fused block steps over an arena) achieved HBM GB/s",
            "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bf16", "data": "synthetic (seeded embedding, sublayer outputs and routing weights, in HBM)",
            "config": {"workload": WORKLOAD_TEXT["cfg2arena"], "algorithmic_bytes_per_step": step_bytes},
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(w2.tokens / (ms_per_step * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": kernel_name(top, w2.tokens, w2.hidden, w2.dtype, mode=1) + f" (S={top} points)",
                         "algorithmic_bytes": dom_bytes, "avg_ms": round(dom_ms, 4)},
        }), flush=True)
        return 0
    if args.workload in ("cfg2train", "cfg3train", "cfg1btrain"):
        rec = bench_train(args.steps, args.warmup, dev, args.variant, args.compile, args.workload, args.compile_breaks,
                          args.graph)
        ms = rec["ms_per_step"]
        rb = rec["routing_kernel_bytes"]
        gbs = (rb["fwd"] + rb["bwd"]) / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "AttnRes training step (routing caller loop forward + backward): tokens/s and the routing "
                      "kernels' algorithmic bytes per step time",
            "value": rec["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded embedding, output gradient and routing parameters, resident in HBM)",
            "config": {"workload": WORKLOAD_TEXT[args.workload], "variant": args.variant,
                       "compiled": "fullgraph" if args.compile else ("graph breaks at the routing points"
                                                                      if args.compile_breaks else False)},
            "routing_GB/s_over_step": round(gbs, 2), "hbm_frac_routing_bytes": round(gbs / HBM_PEAK_GBS, 4),
            **rec,
        }), flush=True)
        return 0
    if args.workload == "lmstep":
        rec = bench_lmstep(args.steps, args.warmup, dev, args.lm, args.residuals.split(","), not args.eager_sublayers)
        head = rec.get("attnres") or next(rec[k] for k in args.residuals.split(","))
        print(json.dumps({
            "metric": "whole training step tokens/s with AttnRes routing (and the standard residual stream beside it)",
            "value": head["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random token ids, random-init weights)",
            "config": {"workload": WORKLOAD_TEXT["lmstep"], "lm": args.lm}, **rec,
        }), flush=True)
        return 0
    if args.workload == "narrow":
        print(json.dumps({"workload": WORKLOAD_TEXT["narrow"], "steps": args.steps, "warmup": args.warmup,
                          **bench_narrow(args.steps, args.warmup, dev)}), flush=True)
        return 0
    if args.workload == "segsum":
        print(json.dumps({"workload": WORKLOAD_TEXT["segsum"], "steps": args.steps, "warmup": args.warmup,
                          **bench_segsum(args.steps, args.warmup, dev)}), flush=True)
        return 0
    if args.workload == "mall":
        print(json.dumps({"workload": WORKLOAD_TEXT["mall"], "steps": args.steps, "warmup": args.warmup,
                          **bench_mall(args.steps, args.warmup, dev)}), flush=True)
        return 0
    if args.workload == "cfg2serve" and args.pass_ == "bwd":
        elapsed, step_bytes, deep_ms, deep_bytes = bench_serve_backward(args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        w2 = workloads.get("cfg2")
        ach = deep_bytes / (deep_ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "AttnRes serving two-phase routing backward achieved HBM GB/s",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded blocks, partials and output gradients, resident in HBM)",
            "config": {"workload": "backward of: " + WORKLOAD_TEXT["cfg2serve"], "algorithmic_bytes_per_step": step_bytes},
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w2.tokens / (ms_per_step * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": bwdq_kernel_name(7, w2.hidden, 8) + " (+ query-gradient pass, reduction; S=7, Q=8)",
                         "algorithmic_bytes": deep_bytes, "avg_ms": round(deep_ms, 4)},
        }), flush=True)
        return 0
    if args.workload == "cfg2serve":
        elapsed, step_bytes, merge_ms, merge_bytes, p1_ms, p1_bytes = bench_serve(args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        w2 = workloads.get("cfg2")
        ach = merge_bytes / (merge_ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": "AttnRes serving two-phase routing achieved HBM GB/s",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded blocks and partials, resident in HBM)",
            "config": {"workload": WORKLOAD_TEXT["cfg2serve"], "algorithmic_bytes_per_step": step_bytes},
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w2.tokens / (ms_per_step * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": merge_kernel_name(w2.tokens, w2.hidden) + " (phase-2 merge, 3 rows per token)",
                         "algorithmic_bytes": merge_bytes, "avg_ms": round(merge_ms, 4)},
            "phase1_deepest": {"kernel": kernel_name(7, w2.tokens, w2.hidden, w2.dtype, 8) + " (Q=8)",
                               "algorithmic_bytes": p1_bytes,
                               "avg_ms": round(p1_ms, 4),
                               "GB/s": round(p1_bytes / (p1_ms * 1e-3) / 1e9, 2)},
        }), flush=True)
        return 0
    w = workloads.get(args.workload)
    roofline = None
    if args.pass_ == "bwd":
        if args.workload == "cfg4":
            print("bench.py: --pass bwd covers the prefill workloads (cfg2, cfg3, cfg5)", file=sys.stderr)
            return 2
        elapsed, dominant, dom_ms, dom_bytes, step_bytes = bench_backward(w, args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
        name = bwd_kernel_name(dominant, w.tokens, w.hidden, w.dtype) + " (+ attnres_reduce_dqw_cols)"
        traffic, traffic_src = load_traffic(f"bwd_{args.workload}_s{dominant}")
        print(json.dumps({
            "metric": "AttnRes routing backward achieved HBM GB/s",
            "value": round(gbs, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16" if w.dtype == torch.bfloat16 else "fp32",
            "data": "synthetic (seeded sources and dL/dout, resident in HBM)",
            "config": {"workload": "backward of: " + WORKLOAD_TEXT[args.workload], "routing_calls": len(w.calls),
                       "algorithmic_bytes_per_step": step_bytes},
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(w.tokens / (ms_per_step * 1e-3), 1),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": name,
                         "algorithmic_bytes": dom_bytes, "avg_ms": round(dom_ms, 4),
                         **({"traffic_source": traffic_src} if traffic_src else {})},
        }), flush=True)
        return 0
    if args.workload == "cfg4":
        elapsed, step_bytes, graph_ms = bench_decode(w, args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        tokens = w.batch
        roofline = {
            "bound": "hbm",
            "achieved": round(step_bytes / (graph_ms * 1e-3) / 1e9, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(step_bytes / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "one decode step (65 attnres_route_bf_d2_s*_v1_q1 launches, HIP graph)",
            "avg_ms": round(graph_ms, 4),
        }
    else:
        elapsed, dominant, dom_ms, dom_bytes = bench_sweep(w, args.steps, args.warmup, dev)
        ms_per_step = elapsed * 1e3 / args.steps
        step_bytes = w.step_bytes()
        gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
        tokens = w.tokens
        tag = f"{args.workload}_s{dominant}"
        traffic, traffic_src = load_traffic(tag)
        achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
        roofline = {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": kernel_name(dominant, w.tokens, w.hidden, w.dtype),
            "algorithmic_bytes": dom_bytes,
            "avg_ms": round(dom_ms, 4),
        }
        if traffic_src:
            roofline["traffic_source"] = traffic_src
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) sources x per-source log-uniform scales, resident in HBM)",
        "config": {
            "workload": WORKLOAD_TEXT[args.workload],
            "hidden": w.hidden,
            "batch": w.batch,
            "seq": w.seq,
            "routing_calls": len(w.calls),
            "sum_S": sum(w.calls),
            "algorithmic_bytes_per_step": step_bytes,
        },
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(tokens / (ms_per_step * 1e-3), 1),
        "roofline": roofline,
    }
    if args.workload == "cfg2" and not args.only:
        line["cfg3"] = secondary_sweep("cfg3", args.steps, args.warmup, dev)
        line["cfg5"] = secondary_sweep("cfg5", args.steps, args.warmup, dev)
        line["cfg2_bwd"] = secondary_backward("cfg2", args.steps, args.warmup, dev)
        line["cfg4"] = secondary_decode(args.steps, args.warmup, dev)
        line["cfg2arena"] = secondary_arena(args.steps, args.warmup, dev)
        line["cfg2train"] = secondary_train(min(args.steps, 5), min(args.warmup, 2), dev, graph=True)
        line["cfg3train"] = secondary_train(min(args.steps, 5), min(args.warmup, 2), dev, "cfg3train", graph=True)
        line["cfg1btrain"] = secondary_train(min(args.steps, 10), min(args.warmup, 3), dev, "cfg1btrain", graph=True)
        # whole training steps of the reference's model: AttnRes against the standard residual stream
        line["lmstep_proxy"] = {"workload": WORKLOAD_TEXT["lmstep"] + ": proxy model (D=512, 28 layers, B=4, T=2048)",
                                **bench_lmstep(min(args.steps, 10), min(args.warmup, 3), dev, "proxy",
                                               ("standard", "attnres", "torch")),
                                # the reference's published figures for this comparison (another GPU, another
                                # variant): docs/attnres-performance-brief.md:53-59
                                "reference_published": {"standard_tokens_per_s": 256000, "attnres_tokens_per_s": 117000,
                                                        "overhead": 0.54, "hardware": "1x B200",
                                                        "variant": "once-per-layer routing (29 calls), whole model "
                                                                   "under torch.compile"}}
        line["lmstep_3b"] = {"workload": WORKLOAD_TEXT["lmstep"] + ": 3B model (D=3072, 28 layers, B=4, T=4096)",
                             **bench_lmstep(min(args.steps, 5), min(args.warmup, 2), dev, "3b",
                                            ("standard", "attnres", "torch"))}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, min(args.cpu_tokens, w.tokens)) if args.workload != "cfg4" else \
            cpu_baseline(w, w.tokens)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
