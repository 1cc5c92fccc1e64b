"""Seeded synthetic inputs (CPU): determinism and the distribution rules."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from mini_trainer_amd import synth


@pytest.mark.parametrize("key", [1, 2, 3, 4, 5])
def test_layout_and_masks(key):
    cfg = synth.CONFIGS[key]
    for mb in range(cfg.minibatches):
        b = synth.make_batch(cfg, mb, with_tensors=False)
        t, L, cu = b["target"].numpy(), b["lengths"], b["cu_seqlens"].numpy()
        assert t.size == cfg.T == L.sum() and len(L) == cfg.S and L.min() >= 2
        assert cu.dtype == np.int32 and cu[0] == 0 and cu[-1] == cfg.T
        assert np.array_equal(np.diff(cu), L)
        valid = t != -100
        assert abs((~valid).mean() - cfg.mask_frac) < 0.02
        assert t[valid].min() >= 0 and t[valid].max() < cfg.V
        # masked positions form a prefix of every sample
        for s in range(cfg.S):
            seg = valid[cu[s]:cu[s + 1]]
            k = int((~seg).sum())
            assert not seg[:k].any() and seg[k:].all()
        if cfg.n_fully_masked:
            full = [not valid[cu[s]:cu[s + 1]].any() for s in range(cfg.S)]
            assert sum(full) >= cfg.n_fully_masked


def test_determinism_and_dtypes():
    cfg = synth.CONFIGS[1]
    a = synth.make_batch(cfg, T=256)
    b = synth.make_batch(cfg, T=256)
    assert torch.equal(a["X"], b["X"]) and torch.equal(a["target"], b["target"])
    assert a["X"].dtype == torch.float32 and a["W"].shape == (cfg.V, cfg.H)
    assert abs(float(a["W"].std()) - cfg.w_std) < 1e-3


def test_zipf_labels_are_heavy_headed():
    rng = np.random.default_rng(0)
    lab = synth.draw_labels(rng, 20000, 128256, "zipf")
    assert lab.min() >= 0 and lab.max() < 128256
    assert (lab == 0).mean() > 0.05  # token 0 dominates under Zipf(1.1)
