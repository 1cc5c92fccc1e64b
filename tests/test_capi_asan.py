"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(the CPU build of mini_trainer_amd/build.py's build_sanitized: the sanitizers
on the host pass only).  A child process with the clang ASan runtime
preloaded loads that build in place of libmt_flce.so and runs the C-ABI
host-logic tests (argument checks, planners, layouts), a planner sweep over
random and extreme sizes (64-bit size arithmetic, 32-bit limits) and the
launch-failure path.  Any out-of-bounds access, overflow or other undefined
behaviour aborts the child."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

SWEEP = r"""
import ctypes
import numpy as np
from mini_trainer_amd import _lib

lib = _lib.load()
assert "libmt_flce_san" in str(_lib.LIB_PATH)
rng = np.random.default_rng(11)
I64, SZ, INT = ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
big = [1, 2, 255, 256, 257, 65535, 65536, 131071, 1 << 20, (1 << 31) - 1]
shapes = [(int(rng.choice(big)), int(rng.choice(big)), int(rng.choice([8, 64, 1000, 1536, 4096,
                                                                       8192, 16384, 1 << 20])),
           int(rng.choice(big))) for _ in range(300)]
shapes += [(int(rng.integers(1, 1 << 20)), 0, int(rng.integers(1, 200)) * 8,
            int(rng.integers(1, 1 << 18))) for _ in range(100)]
for T, n, H, V in shapes:
    n = min(n, T)
    for budget in (0, 1, 1 << 30, (1 << 64) - 1):
        C, Cv, ws = I64(), I64(), SZ()
        for fn in (lib.mt_flce_backward_plan, lib.mt_flce_backward_narrow_plan):
            st = fn(T, n, H, V, 1, budget, ctypes.byref(C), ctypes.byref(Cv), ctypes.byref(ws))
            assert st in (0, 1, 3), st
            if st == 0 and n > 0:
                assert C.value % 256 == 0 and Cv.value % 256 == 0
        pays = INT()
        for acc in (0, 1):
            st = lib.mt_flce_fused_plan(T, n, H, V, 1, budget, acc, ctypes.byref(C),
                                        ctypes.byref(ws), ctypes.byref(pays))
            assert st in (0, 1, 3), st
    lo, rows, hi = SZ(), I64(), SZ()
    st = lib.mt_flce_dw_tiles_layout(V, H, ctypes.byref(lo), ctypes.byref(rows), ctypes.byref(hi))
    assert st == 0 and lo.value == V * H * 2 and 0 <= rows.value <= -(-V // 256)
    lib.mt_flce_narrow_scratch_bytes(V, H, n)
    lib.mt_flce_forward_workspace_bytes(T, n, H, V, 1)
    lib.mt_flce_forward_workspace_bytes(T, n, H, V, 0)
for bad in ((-1, 1, 8, 8), (8, 9, 8, 8), (8, 4, 0, 8), (8, 4, 8, 0), (8, 4, 8, 1 << 40)):
    C, Cv, ws, pays = I64(), I64(), SZ(), INT()
    assert lib.mt_flce_backward_plan(*bad, 1, 0, ctypes.byref(C), ctypes.byref(Cv),
                                     ctypes.byref(ws)) != 0
    assert lib.mt_flce_fused_plan(*bad, 1, 0, 0, ctypes.byref(C), ctypes.byref(ws),
                                  ctypes.byref(pays)) != 0
print("sweep ok")
"""


def test_library_host_code_under_sanitizers():
    from mini_trainer_amd.build import asan_runtime, build_sanitized, san_is_stale

    rt = asan_runtime()
    if not rt.is_absolute() or not rt.exists():
        pytest.skip("clang ASan runtime not found next to hipcc")
    lib = build_sanitized() if san_is_stale() else \
        ROOT / "mini_trainer_amd" / "_build" / "libmt_flce_san.so"
    env = dict(os.environ, MT_FLCE_LIB=str(lib), LD_PRELOAD=str(rt), PYTHONPATH=str(ROOT),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sys.executable, "-c", SWEEP], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0 and "sweep ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        "tests/test_capi_cpu.py"], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert " passed" in r.stdout and "failed" not in r.stdout
