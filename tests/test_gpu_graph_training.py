"""The training step of the routing path recorded in a HIP graph.

forward_attn_res under autograd plus its backward (the fused routing steps, the
deferred block gradients with their segment sums or, in fp32, the in-place
block sums, the query-gradient reductions; torch's elementwise stand-in
sublayers) issues no host synchronisation and no memset, so torch.cuda.graph
can record the whole step.
Each replay, with the program's own eager work and synchronisations between the
replays, must give the eager step's gradients bit for bit (every kernel of the
step is deterministic).
"""

import dataclasses

import pytest
import torch

from kotodama_amd import engine, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _grads(model, embed):
    out = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
    out["embed"] = embed.grad.detach().clone()
    return out


@pytest.mark.parametrize("name,hidden,seq,dtype", [
    ("cfg1btrain", 1024, 256, torch.bfloat16), ("cfg2train", 3072, 128, torch.bfloat16),
    ("cfg1btrain", 512, 384, torch.bfloat16),
    ("cfg1btrain", 512, 192, torch.float32),  # fp32: the in-place sums (attnres_route_bwd_add) instead of deferral
], ids=["d1024-dd", "d3072-uniform", "d512-dd", "d512-fp32"])
def test_captured_training_step_replays_bit_exact(name, hidden, seq, dtype):
    base = workloads.get("cfg2" if name == "cfg2train" else name)
    w = dataclasses.replace(base, hidden=hidden, batch=2, seq=seq, dtype=dtype)
    model = workloads.TrainingModel(w, DEV, seed=12)
    g = torch.Generator(device=DEV).manual_seed(13)
    embed = torch.randn((w.batch, w.seq, w.hidden), generator=g, device=DEV).to(w.dtype).requires_grad_(True)
    G = torch.randn((w.batch, w.seq, w.hidden), generator=g, device=DEV).to(w.dtype)
    print(f"graph training {name} D={hidden} T={seq} {dtype}", flush=True)

    def step():
        engine.forward_attn_res(model, embed).backward(G)

    model.zero_grad(set_to_none=True)
    embed.grad = None
    step()
    eager = _grads(model, embed)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            embed.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    embed.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()

    x = torch.randn((256, 256), generator=g, device=DEV)
    for r in range(3):
        x = torch.tanh(x @ x.T)  # the program's own eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = _grads(model, embed)
        assert got.keys() == eager.keys()
        for k, v in eager.items():
            assert torch.equal(got[k], v), (r, k)
