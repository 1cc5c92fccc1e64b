"""Seeded synthetic packed batches of the five benchmark shapes.

Convention (shared by tests and bench):
  * numpy.random.default_rng(seed) draws sample lengths, masks and labels;
    torch.Generator().manual_seed(seed) on the CPU draws X ~ N(0, 1), and a
    second generator seeded 1000 + k draws W ~ N(0, w_std), both in fp32 and
    then cast to the config dtype (round to nearest even).
  * Config k uses seed k; minibatch j of config 5 uses seed 50 + j for its
    lengths, labels and X (W is the same for every minibatch).
  * Lengths: S lognormal(mu, sigma) draws scaled to T with
    L_i = max(2, floor(L_i * T / sum L)); the remainder goes to the longest.
  * Masks: each sample has a masked prefix ("prompt") of round(m * L_i)
    tokens; config 5 additionally masks n_fully_masked whole samples and
    rescales the other prefixes so the global fraction stays ~m.
  * Labels (already shifted targets): uniform in [0, V) or Zipf(1.1) - 1,
    redrawn while >= V.  Masked positions hold -100.
The packed layout (samples concatenated, boundaries in cu_seqlens) is the
one mini_trainer's collator builds (sampler.py:144-208).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np
import torch

IGNORE_INDEX = -100


@dataclass(frozen=True)
class Config:
    key: int
    name: str
    T: int
    H: int
    V: int
    dtype: torch.dtype
    S: int
    mu: float
    sigma: float
    mask_frac: float
    labels: str  # "uniform" | "zipf"
    w_std: float = 0.02
    n_fully_masked: int = 0
    minibatches: int = 1


CONFIGS: Dict[int, Config] = {
    1: Config(1, "qwen2.5-0.5b-head-fp32", 2048, 896, 151936, torch.float32, 8, 5.3, 0.6, 0.40,
              "uniform"),
    2: Config(2, "qwen2.5-1.5b-head-bf16", 32768, 1536, 151936, torch.bfloat16, 64, 6.0, 0.8,
              0.50, "uniform"),
    3: Config(3, "llama3-8b-head-bf16", 65536, 4096, 128256, torch.bfloat16, 128, 6.2, 0.9, 0.30,
              "zipf"),
    4: Config(4, "qwen2.5-7b-head-bf16-128k", 128000, 3584, 152064, torch.bfloat16, 200, 6.1, 1.0,
              0.45, "uniform"),
    5: Config(5, "llama3-70b-head-bf16-4mb", 16384, 8192, 128256, torch.bfloat16, 32, 6.0, 1.2,
              0.60, "zipf", w_std=0.015, n_fully_masked=5, minibatches=4),
}


def sample_lengths(rng: np.random.Generator, S: int, mu: float, sigma: float, T: int) -> np.ndarray:
    raw = rng.lognormal(mu, sigma, S)
    L = np.maximum(2, np.floor(raw * T / raw.sum())).astype(np.int64)
    L[int(np.argmax(L))] += T - int(L.sum())
    if L.min() < 1:
        raise ValueError("sample lengths do not fit T")
    return L


def draw_labels(rng: np.random.Generator, n: int, V: int, kind: str) -> np.ndarray:
    if kind == "uniform":
        return rng.integers(0, V, size=n, dtype=np.int64)
    if kind == "zipf":
        out = rng.zipf(1.1, size=n).astype(np.int64) - 1
        bad = out >= V
        while bad.any():
            out[bad] = rng.zipf(1.1, size=int(bad.sum())).astype(np.int64) - 1
            bad = out >= V
        return out
    raise ValueError(kind)


def make_targets(rng: np.random.Generator, lengths: np.ndarray, V: int, mask_frac: float,
                 kind: str, n_fully_masked: int = 0) -> np.ndarray:
    T = int(lengths.sum())
    labels = draw_labels(rng, T, V, kind)
    S = len(lengths)
    full = np.zeros(S, dtype=bool)
    if n_fully_masked:
        full[rng.choice(S, size=n_fully_masked, replace=False)] = True
    frac = mask_frac
    if n_fully_masked:
        rest = T - int(lengths[full].sum())
        frac = (mask_frac * T - int(lengths[full].sum())) / max(rest, 1)
        frac = float(min(max(frac, 0.0), 1.0))
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    for s in range(S):
        a, L = int(starts[s]), int(lengths[s])
        m = L if full[s] else int(round(frac * L))
        labels[a:a + m] = IGNORE_INDEX
    return labels


def cu_seqlens_of(lengths: np.ndarray) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def make_batch(cfg: Config, minibatch: int = 0, with_tensors: bool = True,
               T: Optional[int] = None) -> Dict[str, object]:
    """Seeded inputs of one (mini)batch on the CPU.

    Returns dict(X, W, target, cu_seqlens, lengths).  T overrides the token
    count (same distributions) for bounded samples.
    """
    seed = cfg.key if cfg.minibatches == 1 else 50 + minibatch
    Tn = cfg.T if T is None else int(T)
    rng = np.random.default_rng(seed)
    S = max(1, min(cfg.S, Tn // 2)) if T is not None else cfg.S
    lengths = sample_lengths(rng, S, cfg.mu, cfg.sigma, Tn)
    nfm = min(cfg.n_fully_masked, S - 1) if cfg.n_fully_masked else 0
    target = make_targets(rng, lengths, cfg.V, cfg.mask_frac, cfg.labels, nfm)
    out: Dict[str, object] = {
        "target": torch.from_numpy(target),
        "cu_seqlens": torch.from_numpy(cu_seqlens_of(lengths)),
        "lengths": lengths,
    }
    if with_tensors:
        g = torch.Generator().manual_seed(seed)
        out["X"] = torch.randn(Tn, cfg.H, generator=g, dtype=torch.float32).to(cfg.dtype)
        out["W"] = make_weight(cfg)
    return out


def make_weight(cfg: Config) -> torch.Tensor:
    g = torch.Generator().manual_seed(1000 + cfg.key)
    return (torch.randn(cfg.V, cfg.H, generator=g, dtype=torch.float32) * cfg.w_std).to(cfg.dtype)
