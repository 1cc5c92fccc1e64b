"""bench.py's torch-on-the-GPU comparator at a small size: it runs the
reference graph and reports a time, and it declines sizes that do not fit."""
from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

pytestmark = pytest.mark.gpu


def test_torch_gpu_path_small(gpu):
    import bench

    g = torch.Generator(device=gpu).manual_seed(5)
    X = torch.randn(512, 256, device=gpu, generator=g).to(torch.bfloat16)
    W = (torch.randn(1000, 256, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, 1000, (512,), device=gpu, generator=g)
    y[::4] = -100
    out = bench.torch_gpu_path([(X, y)], W, 1.0 / 384, steps=1)
    assert out["ms_per_step"] > 0 and out["tokens_per_s"] > 0
    # a [T, V] too large for the device is reported as skipped, not attempted
    big_V = torch.cuda.get_device_properties(gpu).total_memory // (16 * 512) + 1
    Wb = torch.empty(big_V, 1, device=gpu, dtype=torch.bfloat16)
    out = bench.torch_gpu_path([(X[:, :1], y)], Wb, 1.0, steps=1)
    assert "skipped" in out
