"""The C restatement under AddressSanitizer and UndefinedBehaviorSanitizer
(host code; oracle/build.py's sanitize build): a child process with the
sanitizer runtimes preloaded runs the restatement's entry points over ragged
shapes -- empty, one row, all rows ignored, V not a multiple of anything,
softcap, shifted labels, segment sums with empty samples, materialised CE --
and checks them against the float64 closed forms.  Any out-of-bounds access
or undefined behaviour aborts the child."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

CHILD = r"""
import numpy as np
from oracle import brute, ref

rng = np.random.default_rng(0)
for T, H, V, mask, cap in ((0, 8, 5, 0.0, 0.0), (1, 3, 7, 0.0, 0.0), (9, 5, 13, 1.0, 0.0),
                           (37, 11, 101, 0.3, 0.0), (25, 6, 50, 0.2, 2.5)):
    X = rng.standard_normal((T, H)).astype(np.float32)
    W = (rng.standard_normal((V, H)) * 0.3).astype(np.float32)
    y = rng.integers(0, V, T)
    y[rng.random(T) < mask] = -100
    g = (rng.random(T) + 0.5).astype(np.float32)
    loss, dX, dW = ref.backward(X, W, y, g, round_bf16=False, softcap=cap)
    bl, bdX, bdW, _ = brute.flce_f64(X, W, y, g, softcap=cap or None)
    assert np.allclose(loss, bl, rtol=1e-5, atol=1e-6), (T, H, V)
    assert np.allclose(dX, bdX, rtol=1e-4, atol=1e-6) and np.allclose(dW, bdW, rtol=1e-4, atol=1e-6)
    ri, rl, counts = ref.prepare(y, V, shift=True)
    assert counts[0] == int((np.concatenate([y[1:], [-100]]) != -100).sum())
    cu = np.array(sorted({0, T} | set(rng.integers(0, T + 1, 4).tolist())), np.int32)
    sl, sc, st = ref.segment_sum(loss, y, cu)
    assert st == 0 and np.isclose(sl.sum(), loss.sum(), rtol=1e-5, atol=1e-6)
    if T and not cap:
        L = (X @ W.T).astype(np.float32)
        cl, lse, st = ref.ce_forward(L, y)
        assert st == 0 and np.allclose(cl, bl, rtol=1e-4, atol=1e-5)
print("asan child ok")
"""


def test_oracle_under_sanitizers():
    from oracle.build import build

    runtimes = []
    for name in ("libasan.so", "libubsan.so"):
        p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
        path = p.stdout.strip()
        if p.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
            pytest.skip(f"{name} not available to gcc")
        runtimes.append(path)
    san = build(sanitize=True)
    env = dict(os.environ, MT_ORACLE_LIB=str(san), LD_PRELOAD=" ".join(runtimes),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", PYTHONPATH=str(ROOT))
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "asan child ok" in r.stdout
