"""Routing weights from trained checkpoints (real-weight loading).

The reference loads whole models from ``.pt`` checkpoints
(``serve.py:186-232``; ``src/eval/model_loader.py:109-199``): the file is
``{"model": state_dict, "step": ..., ...}`` or a bare state dict, and keys
may carry ``torch.compile``'s ``_orig_mod.`` or DDP's ``module.`` prefix
(stripped at ``model_loader.py:154-159``).  The routing path needs only
the AttnRes parameters (``llama.py:460-464, 541-543``):

    layers.{i}.attn_res_query, layers.{i}.attn_res_norm.weight,
    layers.{i}.mlp_res_query,  layers.{i}.mlp_res_norm.weight,
    final_res_query, final_res_norm.weight

This module reads them, in the routing-point order ``[attn_0, mlp_0, ...,
attn_{L-1}, mlp_{L-1}, final]`` (the order of the 2L+1 routing points and of
``serve.py:85-96``'s stacked queries).

Loading executes nothing from the file: ``.pt`` files go through
``torch.load(..., weights_only=True, mmap=True)`` (the reference passes
``weights_only=False``; a training checkpoint whose optimizer or data-loader
state holds objects outside the weights-only allow-list is refused with an
error that says how to export the model weights), ``.safetensors`` files
through safetensors.  With ``mmap`` only the routing tensors are read from
disk, not the whole multi-GB model.  Zstandard-compressed async checkpoints
(``checkpoint.py:413``) must be decompressed first (``zstd -d``).
"""

from __future__ import annotations

import pickle
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Mapping, Optional, Sequence

import torch
from torch import Tensor

from .schedule import AttnResSchedule

_LAYER_KEY = re.compile(r"^layers\.(\d+)\.attn_res_query$")
_AR_KEYS = ("attn_res", "attn_res_n_blocks", "attn_res_boundaries")


class CheckpointError(RuntimeError):
    """A checkpoint could not be read safely or lacks the routing weights."""


def clean_state_dict(state: Mapping[str, Any]) -> dict[str, Any]:
    """Unwrap ``{"model": ...}`` and strip ``_orig_mod.`` / ``module.`` prefixes (model_loader.py:151-159)."""
    model_state = state.get("model", state) if isinstance(state, Mapping) else state
    if not isinstance(model_state, Mapping):
        raise CheckpointError(f"checkpoint holds a {type(model_state).__name__}, not a state dict")
    return {str(k).replace("_orig_mod.", "").replace("module.", ""): v for k, v in model_state.items()}


def load_state_dict(path: Path | str) -> dict[str, Any]:
    """The model state dict of a ``.pt`` / ``.safetensors`` checkpoint, loaded safely (on the CPU)."""
    path = Path(path)
    if not path.exists():
        raise FileNotFoundError(f"Checkpoint not found: {path}")
    if path.suffix == ".zst":
        raise CheckpointError(f"{path} is zstd-compressed; decompress it first (zstd -d {path})")
    if path.suffix == ".safetensors":
        from safetensors.torch import load_file

        return clean_state_dict(load_file(str(path), device="cpu"))
    try:
        state = torch.load(path, map_location="cpu", weights_only=True, mmap=True)
    except (pickle.UnpicklingError, RuntimeError, AttributeError, TypeError) as e:
        raise CheckpointError(
            f"{path} cannot be loaded with torch.load(weights_only=True): {e}\n"
            "It holds objects beyond plain tensors and containers (typically optimizer or data-loader "
            "state). Export the model weights once, e.g. torch.save({'model': model.state_dict()}, out) "
            "or safetensors.torch.save_file(model.state_dict(), out), and load that file."
        ) from None
    out = clean_state_dict(state)
    if isinstance(state, Mapping):
        for k in ("step", "tokens_consumed"):
            if k in state and not isinstance(state[k], Mapping):
                out.setdefault(f"__{k}__", state[k])
    return out


@dataclass
class RoutingWeights:
    """The 2L+1 pseudo-queries and key-norm gains of an AttnRes model, in routing-point order."""

    queries: Tensor  # (2L+1, D)
    gains: Tensor  # (2L+1, D)
    step: Optional[int] = None
    tokens_consumed: Optional[int] = None

    @property
    def num_layers(self) -> int:
        return (self.queries.shape[0] - 1) // 2

    @property
    def hidden(self) -> int:
        return self.queries.shape[1]

    def to(self, device=None, dtype: Optional[torch.dtype] = None) -> "RoutingWeights":
        return RoutingWeights(
            self.queries.to(device=device, dtype=dtype), self.gains.to(device=device, dtype=dtype), self.step,
            self.tokens_consumed,
        )

    def folded(self) -> Tensor:
        """``query * norm.weight`` per point in the parameter dtype (llama.py:630, serve.py:85-92)."""
        return self.queries * self.gains

    def schedule(
        self,
        n_blocks: Optional[int] = None,
        boundaries: Optional[Sequence[int]] = None,
        attn_res_config: Optional[Mapping[str, Any]] = None,
    ) -> AttnResSchedule:
        """The block schedule; boundaries are not stored in checkpoints, so they come from the
        caller or a registry entry's ``attn_res_n_blocks`` / ``attn_res_boundaries``."""
        if attn_res_config is not None:
            n_blocks = attn_res_config.get("attn_res_n_blocks", n_blocks)
            boundaries = attn_res_config.get("attn_res_boundaries", boundaries)
        if boundaries is None and n_blocks is None:
            raise ValueError("the block schedule needs n_blocks or explicit boundaries (not stored in checkpoints)")
        return AttnResSchedule.build(self.num_layers, n_blocks=n_blocks, boundaries=boundaries)

    def router(self, schedule: AttnResSchedule, eps: float):
        """An :class:`~kotodama_amd.engine.AttnResRouter` over these weights (on their device)."""
        from .engine import AttnResRouter

        if schedule.num_layers != self.num_layers:
            raise ValueError(f"schedule has {schedule.num_layers} layers, the weights {self.num_layers}")
        return AttnResRouter(schedule, list(self.queries), list(self.gains), eps)


def routing_weights_from_state_dict(state: Mapping[str, Any]) -> RoutingWeights:
    """Collect the AttnRes parameters of a (cleaned) model state dict."""
    layers = sorted(int(m.group(1)) for k in state for m in [_LAYER_KEY.match(k)] if m)
    if not layers:
        raise CheckpointError("no 'layers.{i}.attn_res_query' keys: the checkpoint is not an AttnRes model")
    num_layers = layers[-1] + 1
    if layers != list(range(num_layers)):
        raise CheckpointError(f"attn_res_query missing for layers {sorted(set(range(num_layers)) - set(layers))}")
    names = []
    for i in range(num_layers):
        names.append((f"layers.{i}.attn_res_query", f"layers.{i}.attn_res_norm.weight"))
        names.append((f"layers.{i}.mlp_res_query", f"layers.{i}.mlp_res_norm.weight"))
    names.append(("final_res_query", "final_res_norm.weight"))
    missing = [k for pair in names for k in pair if k not in state]
    if missing:
        raise CheckpointError(f"routing weights missing from the checkpoint: {missing[:6]}")
    qs = [torch.as_tensor(state[q]) for q, _ in names]
    gs = [torch.as_tensor(state[g]) for _, g in names]
    d = qs[0].shape
    bad = [q for (q, _), t, u in zip(names, qs, gs) if t.shape != d or u.shape != d or t.dim() != 1]
    if bad:
        raise CheckpointError(f"routing weights with inconsistent shapes: {bad[:4]}")
    step = state.get("__step__")
    tokens = state.get("__tokens_consumed__")
    return RoutingWeights(torch.stack(qs), torch.stack(gs), step if isinstance(step, int) else None,
                          tokens if isinstance(tokens, int) else None)


def load_routing_weights(
    path: Path | str, device=None, dtype: Optional[torch.dtype] = None
) -> RoutingWeights:
    """Routing weights of a checkpoint file, optionally moved/cast (serve.py casts the model to bf16)."""
    w = routing_weights_from_state_dict(load_state_dict(path))
    return w.to(device=device, dtype=dtype) if (device is not None or dtype is not None) else w


@dataclass
class CheckpointInfo:
    """Registry entry for a named checkpoint (model_loader.py:24-31)."""

    name: str
    path: Path
    attn_res_config: Optional[dict[str, Any]] = None
    group: Optional[str] = None
    tags: list[str] = field(default_factory=list)


def load_checkpoint_registry(config_path: Path | str) -> dict[str, CheckpointInfo]:
    """Name -> :class:`CheckpointInfo` from a registry YAML (model_loader.py:67-107; configs/checkpoints.yaml)."""
    import yaml

    config_path = Path(config_path)
    if not config_path.exists():
        raise FileNotFoundError(f"Checkpoint registry not found: {config_path}")
    with open(config_path) as f:
        raw = yaml.safe_load(f) or {}
    registry: dict[str, CheckpointInfo] = {}
    for group_name, group_data in raw.items():
        for ckpt_name, data in (group_data or {}).get("checkpoints", {}).items():
            ar = {k: v for k, v in data.items() if k in _AR_KEYS} or None
            registry[ckpt_name] = CheckpointInfo(
                name=ckpt_name, path=Path(data["path"]), attn_res_config=ar, group=group_name,
                tags=list(data.get("tags", [])),
            )
    return registry


__all__ = [
    "CheckpointError",
    "CheckpointInfo",
    "RoutingWeights",
    "clean_state_dict",
    "load_checkpoint_registry",
    "load_routing_weights",
    "load_state_dict",
    "routing_weights_from_state_dict",
]
