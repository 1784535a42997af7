"""Schedule of routing points (llama.py:545-571) against tables derived by hand.

Run-length form of the source counts S_j: a block of b layers that starts at
boundary layer i contributes the pre-MLP point of layer i, the 2(b-1) points
of its inner layers and the pre-attention point of the next boundary layer,
all seeing the same S.
"""

import pytest

from kotodama_amd.schedule import AttnResSchedule
from oracle import attnres_oracle as O


def runs(*pairs):
    out = []
    for value, count in pairs:
        out += [value] * count
    return out


CASES = [
    # 3B canary, attn_res_n_blocks=8 -> ceil(28/8)=4 -> {0,4,...,24}
    (dict(num_layers=28, n_blocks=8), {0, 4, 8, 12, 16, 20, 24}, 8, runs((1, 1), *[(k, 8) for k in range(2, 9)]), 281),
    # n_blocks=7 gives the same boundaries for 28 layers
    (dict(num_layers=28, n_blocks=7), {0, 4, 8, 12, 16, 20, 24}, 8, runs((1, 1), *[(k, 8) for k in range(2, 9)]), 281),
    # 8B, 32 layers, n_blocks=8 -> {0,4,...,28}
    (dict(num_layers=32, n_blocks=8), set(range(0, 32, 4)), 9, runs((1, 1), *[(k, 8) for k in range(2, 10)]), 353),
    # DD-v1 proxy boundaries (serve.py:52): blocks of 3,4,5,9,4,3 layers
    (dict(num_layers=28, boundaries=[0, 3, 7, 12, 21, 25]), {0, 3, 7, 12, 21, 25}, 7,
     runs((1, 1), (2, 6), (3, 8), (4, 10), (5, 18), (6, 8), (7, 6)), 257),
    # data-driven blocks {0,3,7,12,18,23}: blocks of 3,4,5,6,5,5 layers
    (dict(num_layers=28, boundaries=[0, 3, 7, 12, 18, 23]), {0, 3, 7, 12, 18, 23}, 7,
     runs((1, 1), (2, 6), (3, 8), (4, 10), (5, 12), (6, 10), (7, 10)), 267),
    # block *ends* read as boundaries: layer 28 never occurs, so S stops at 6
    (dict(num_layers=28, boundaries=[3, 7, 12, 18, 23, 28]), {3, 7, 12, 18, 23, 28}, 7,
     runs((1, 7), (2, 8), (3, 10), (4, 12), (5, 10), (6, 10)), 211),
]


@pytest.mark.parametrize("kw,bset,max_s,counts,total", CASES)
def test_schedule_tables(kw, bset, max_s, counts, total):
    for impl in ("product", "oracle"):
        if impl == "product":
            s = AttnResSchedule.build(**kw)
            b, m, c = s.boundary_set, s.max_sources, list(s.active_counts)
        else:
            r = O.schedule(**kw)
            b, m, c = r["boundary_set"], r["max_sources"], r["active_counts"]
        assert set(b) == bset, impl
        assert m == max_s, impl
        assert len(c) == 2 * kw["num_layers"] + 1, impl
        assert c == counts, impl
        assert sum(c) == total, impl


def test_masks_and_commit_points():
    s = AttnResSchedule.build(28, n_blocks=8)
    m = s.masks()
    assert m.shape == (57, 8)
    for j, c in enumerate(s.active_counts):
        assert m[j, :c].all() and not m[j, c:].any()
    # a commit happens right before the pre-MLP point of every boundary layer
    assert [j for j, c in enumerate(s.commit_before) if c] == [2 * i + 1 for i in sorted(s.boundary_set)]
    r = O.schedule(28, n_blocks=8)
    assert (r["masks"] == m.numpy()).all()
    assert list(r["commit_before"]) == list(s.commit_before)


def test_schedule_rejects_bad_config():
    with pytest.raises(ValueError):
        AttnResSchedule.build(0, n_blocks=1)
    with pytest.raises(ValueError):
        AttnResSchedule.build(28)
