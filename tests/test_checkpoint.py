"""Real-weight loading (CPU): formats, key handling, order, and safe loading only."""

import numpy as np
import pytest
import torch

from kotodama_amd import checkpoint as C
from oracle import attnres_oracle as O

_EXECUTED = []


def _mark():
    _EXECUTED.append(True)
    return {}


class _Evil:
    """An object whose unpickling would run code: a weights-only load must refuse it."""

    def __reduce__(self):
        return (_mark, ())


def model_state(L=4, D=64, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    sd = {"embed_tokens.weight": torch.randn(100, D, generator=g).to(dtype)}
    for i in range(L):
        sd[f"layers.{i}.attn.wq.weight"] = torch.randn(D, D, generator=g).to(dtype)
        for kind in ("attn", "mlp"):
            sd[f"layers.{i}.{kind}_res_query"] = (torch.randn(D, generator=g) * 2).to(dtype)
            sd[f"layers.{i}.{kind}_res_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    sd["final_res_query"] = torch.randn(D, generator=g).to(dtype)
    sd["final_res_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    sd["norm.weight"] = torch.ones(D, dtype=dtype)
    return sd


def test_training_checkpoint_layout_and_order(tmp_path):
    sd = model_state()
    path = tmp_path / "step_00000123.pt"
    opt = {"state": {0: {"momentum_buffer": torch.zeros(3)}}, "param_groups": [{"lr": 0.02, "params": [0]}]}
    torch.save({"step": 123, "tokens_consumed": 4567, "model": sd, "muon_optimizer": opt}, path)
    w = C.load_routing_weights(path)
    assert w.num_layers == 4 and w.hidden == 64 and w.step == 123 and w.tokens_consumed == 4567
    assert w.queries.shape == (9, 64) and w.queries.dtype == torch.bfloat16
    for i in range(4):
        assert torch.equal(w.queries[2 * i], sd[f"layers.{i}.attn_res_query"])
        assert torch.equal(w.queries[2 * i + 1], sd[f"layers.{i}.mlp_res_query"])
        assert torch.equal(w.gains[2 * i + 1], sd[f"layers.{i}.mlp_res_norm.weight"])
    assert torch.equal(w.queries[8], sd["final_res_query"]) and torch.equal(w.gains[8], sd["final_res_norm.weight"])
    # the fold in the parameter dtype is the reference's query * norm.weight
    f = w.folded()
    np.testing.assert_array_equal(
        f[3].float().numpy(), O.fold_query(w.queries[3].float().numpy(), w.gains[3].float().numpy(), "bf16"))


def test_prefixes_bare_dict_and_safetensors(tmp_path):
    sd = model_state(L=2, D=32, seed=1, dtype=torch.float32)
    compiled = {f"_orig_mod.{k}": v for k, v in sd.items()}
    ddp = {f"module.{k}": v for k, v in sd.items()}
    torch.save({"model": compiled}, tmp_path / "a.pt")
    torch.save(ddp, tmp_path / "b.pt")
    from safetensors.torch import save_file

    save_file(sd, str(tmp_path / "c.safetensors"))
    ws = [C.load_routing_weights(tmp_path / n) for n in ("a.pt", "b.pt", "c.safetensors")]
    for w in ws:
        assert torch.equal(w.queries, ws[0].queries) and torch.equal(w.gains, ws[0].gains)
    assert ws[0].step is None
    assert torch.equal(ws[2].queries[0], sd["layers.0.attn_res_query"])


def test_unsafe_pickle_is_refused_without_running_it(tmp_path):
    path = tmp_path / "evil.pt"
    torch.save({"model": model_state(L=1, D=8), "data": _Evil()}, path)
    _EXECUTED.clear()
    with pytest.raises(C.CheckpointError, match="weights_only=True"):
        C.load_routing_weights(path)
    assert not _EXECUTED


def test_missing_and_foreign_checkpoints(tmp_path):
    sd = model_state(L=3, D=16)
    del sd["layers.1.mlp_res_norm.weight"]
    torch.save({"model": sd}, tmp_path / "m.pt")
    with pytest.raises(C.CheckpointError, match="missing"):
        C.load_routing_weights(tmp_path / "m.pt")
    torch.save({"model": {"embed_tokens.weight": torch.zeros(4, 4)}}, tmp_path / "plain.pt")
    with pytest.raises(C.CheckpointError, match="not an AttnRes model"):
        C.load_routing_weights(tmp_path / "plain.pt")
    with pytest.raises(FileNotFoundError):
        C.load_routing_weights(tmp_path / "nope.pt")
    (tmp_path / "x.pt.zst").write_bytes(b"\x28\xb5\x2f\xfd")
    with pytest.raises(C.CheckpointError, match="zstd"):
        C.load_routing_weights(tmp_path / "x.pt.zst")


def test_registry_and_schedule(tmp_path):
    (tmp_path / "reg.yaml").write_text(
        "attnres_sweep:\n"
        "  checkpoints:\n"
        "    P3-AttnRes:\n"
        "      path: checkpoints/a/step_1.pt\n"
        "      attn_res: true\n"
        "      attn_res_n_blocks: 7\n"
        "      tags: [muon, attnres]\n"
        "    DD:\n"
        "      path: checkpoints/b/step_1.pt\n"
        "      attn_res_boundaries: [0, 3, 7, 12, 18, 23]\n"
        "plain:\n"
        "  checkpoints:\n"
        "    Base:\n"
        "      path: checkpoints/c.pt\n"
    )
    reg = C.load_checkpoint_registry(tmp_path / "reg.yaml")
    assert set(reg) == {"P3-AttnRes", "DD", "Base"}
    assert reg["P3-AttnRes"].attn_res_config == {"attn_res": True, "attn_res_n_blocks": 7}
    assert reg["P3-AttnRes"].group == "attnres_sweep" and reg["P3-AttnRes"].tags == ["muon", "attnres"]
    assert reg["Base"].attn_res_config is None
    w = C.RoutingWeights(torch.zeros(57, 8), torch.ones(57, 8))
    s7 = w.schedule(attn_res_config=reg["P3-AttnRes"].attn_res_config)
    assert s7.boundary_set == frozenset(range(0, 28, 4)) and s7.max_sources == 8
    sdd = w.schedule(attn_res_config=reg["DD"].attn_res_config)
    assert sdd.boundary_set == frozenset([0, 3, 7, 12, 18, 23])
    with pytest.raises(ValueError):
        w.schedule()
