"""Packed-batch boundaries without a GPU: cu_seqlens from the position_ids
layout of mini_trainer's collator (sampler.py:182-188: positions restart at
0 for every sample) and from sample lengths, against a brute-force scan and
the synthetic-batch generator."""
from __future__ import annotations

import numpy as np
import torch

from mini_trainer_amd import cu_seqlens_from_lengths, cu_seqlens_from_position_ids, synth


def positions_of(lengths):
    return torch.cat([torch.arange(int(L)) for L in lengths])[None, :]


def brute(pos):
    p = pos.reshape(-1).tolist()
    cu = [0]
    for t in range(1, len(p)):
        if p[t] == 0:
            cu.append(t)
    cu.append(len(p))
    return cu


def test_cu_seqlens_round_trip():
    rng = np.random.default_rng(5)
    for _ in range(20):
        L = rng.integers(1, 50, rng.integers(1, 12))
        pos = positions_of(L)
        cu = cu_seqlens_from_position_ids(pos)
        assert cu.dtype == torch.int32
        assert cu.tolist() == brute(pos)
        assert torch.equal(cu, cu_seqlens_from_lengths(L))


def test_cu_seqlens_matches_the_synthetic_batches():
    for key in (2, 3, 5):
        b = synth.make_batch(synth.CONFIGS[key], 0, with_tensors=False)
        pos = positions_of(b["lengths"])
        assert torch.equal(cu_seqlens_from_position_ids(pos), b["cu_seqlens"].to(torch.int32))


def test_cu_seqlens_edge_cases():
    assert cu_seqlens_from_position_ids(torch.zeros(0, dtype=torch.long)).tolist() == [0]
    # a row that does not start at position 0 (a continued sample) still starts a segment
    assert cu_seqlens_from_position_ids(torch.tensor([[3, 4, 0, 1]])).tolist() == [0, 2, 4]
    assert cu_seqlens_from_position_ids(torch.tensor([0, 0, 0])).tolist() == [0, 1, 2, 3]
