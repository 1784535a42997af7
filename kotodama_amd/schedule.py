"""Block schedule of the AttnRes routing points (llama.py:545-571).

A model with L layers routes 2L+1 times per forward: before attention and
before the MLP of every layer, plus one final aggregation.  Layer i commits
the running partial block *between* its two routing points when i is a block
boundary (llama.py:697-712), so:

* routing point 2i   sees n_committed + 1 sources (committed blocks + partial);
* if i is a boundary, n_committed += 1 (the partial becomes a committed block
  and a fresh partial starts from that layer's attention output);
* routing point 2i+1 sees the new n_committed + 1;
* the final point 2L sees every committed block plus the partial.

Boundaries are an explicit list (``attn_res_boundaries``) or
``range(0, L, ceil(L / n_blocks))``; ``max_sources`` is the number of
boundaries plus one.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Iterable, Optional

import torch


@dataclass(frozen=True)
class AttnResSchedule:
    num_layers: int
    boundary_set: frozenset
    max_sources: int
    active_counts: tuple  # sources seen by each of the 2L+1 routing points
    commit_before: tuple  # routing point j directly follows a block commit
    _masks: Optional[torch.Tensor] = field(default=None, compare=False, repr=False)

    @classmethod
    def build(
        cls, num_layers: int, n_blocks: Optional[int] = None, boundaries: Optional[Iterable[int]] = None
    ) -> "AttnResSchedule":
        if num_layers < 1:
            raise ValueError("num_layers must be >= 1")
        if boundaries is not None:
            bset = frozenset(int(b) for b in boundaries)
        else:
            if not n_blocks or n_blocks < 1:
                raise ValueError("need n_blocks >= 1 or explicit boundaries")
            step = math.ceil(num_layers / n_blocks)
            bset = frozenset(range(0, num_layers, step))
        npts = 2 * num_layers + 1
        counts = [0] * npts
        commits = [False] * npts
        n_committed = 0
        for i in range(num_layers):
            counts[2 * i] = n_committed + 1
            if i in bset:
                n_committed += 1
                commits[2 * i + 1] = True
            counts[2 * i + 1] = n_committed + 1
        counts[-1] = n_committed + 1
        return cls(num_layers, bset, len(bset) + 1, tuple(counts), tuple(commits))

    @classmethod
    def from_config(cls, config) -> "AttnResSchedule":
        """From an object with the LuxiaModelConfig fields (llama.py:113-116)."""
        return cls.build(
            config.num_layers,
            n_blocks=getattr(config, "attn_res_n_blocks", None),
            boundaries=getattr(config, "attn_res_boundaries", None),
        )

    @property
    def num_points(self) -> int:
        return 2 * self.num_layers + 1

    def masks(self, device=None) -> torch.Tensor:
        """(2L+1, max_S) bool prefix masks, as the reference's ``_attn_res_masks``."""
        m = torch.zeros(self.num_points, self.max_sources, dtype=torch.bool)
        for j, c in enumerate(self.active_counts):
            m[j, :c] = True
        return m if device is None else m.to(device)

    def total_sources(self) -> int:
        return sum(self.active_counts)
