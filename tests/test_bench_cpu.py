"""bench.py's contract pieces that run without a GPU: the multi-GPU request is
refused with a message before any device is touched, and the CPU baseline
leg (the reference torch path over a bounded prefix) returns the fields the
bench line carries."""
from __future__ import annotations

import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_cpu_baseline_fields():
    import bench
    from mini_trainer_amd import synth

    torch.set_num_threads(min(4, os.cpu_count() or 1))
    out = bench.cpu_baseline(synth.CONFIGS[1], budget_s=0.5)
    assert set(out) == {"value", "unit", "cores", "kind", "sample"}
    assert out["unit"] == "tokens/s" and out["kind"] == "port"
    assert out["value"] > 0 and out["cores"] >= 1
    assert "none_reduction_losses.py:35" in out["sample"]
