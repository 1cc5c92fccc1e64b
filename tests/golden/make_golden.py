"""Writes the golden vectors of the fused linear + CE path (tests/golden/*.npz).

The reference ships no test or fixture for this path (its tests/ only cover
the batch packer), so the vectors are produced by the reference's own torch
arithmetic, restated in oracle/torch_path.py: F.linear in the input dtype ->
.float() -> [softcap] -> F.cross_entropy(reduction='none', ignore_index)
(none_reduction_losses.py:35) and its autograd backward with a per-token
upstream gradient; dW accumulated in fp32.  The reference's Python is not
imported.  bf16 tensors are stored as their uint16 bit patterns.

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle.torch_path import torch_path  # noqa: E402

CASES = {
    # name: (T, H, V, dtype, mask_frac, w_std, softcap, seed)
    "fp32_small": (48, 64, 515, torch.float32, 0.3, 0.2, None, 101),
    "bf16_small": (96, 64, 600, torch.bfloat16, 0.4, 0.05, None, 102),
    "bf16_softcap": (64, 64, 300, torch.bfloat16, 0.25, 0.5, 5.0, 103),
}


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def unbits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def make(name):
    T, H, V, dt, mf, ws, cap, seed = CASES[name]
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(T, H, generator=g).to(dt)
    W = (torch.randn(V, H, generator=g) * ws).to(dt)
    y = torch.randint(0, V, (T,), generator=g)
    y[torch.rand(T, generator=g) < mf] = -100
    y[:5] = -100  # a fully masked leading sample
    grad = torch.rand(T, generator=g) * 1.5 + 0.1
    loss, dX, dW = torch_path(X, W, y, grad=grad, softcap=cap)
    return dict(X=bits(X), W=bits(W), target=y.numpy(), grad=grad.numpy(), loss=loss.numpy(),
                dX=bits(dX), dW=dW.numpy(), softcap=np.float64(cap or 0.0),
                dtype=np.array(str(dt)))


if __name__ == "__main__":
    for n in CASES:
        np.savez_compressed(HERE / f"{n}.npz", **make(n))
        print("wrote", HERE / f"{n}.npz")
