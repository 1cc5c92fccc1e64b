"""Build recipe for libmt_flce.so (gfx950 only).

The library is one translation unit (csrc/flce_capi.hip, which includes the
kernel headers) compiled with hipcc for gfx950 into the package directory, so
it travels with the source tree.  `python -m mini_trainer_amd.build` rebuilds it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libmt_flce.so"
SOURCES = [CSRC / "flce_capi.hip"]
DEPENDS = sorted(CSRC.glob("*.h")) + SOURCES + [PKG_DIR.parent / "include" / "mt_flce.h"]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay disabled in all device code of this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmt_flce.so)")


SAN_LIB_PATH = PKG_DIR / "_build" / "libmt_flce_san.so"
# The CPU tests' build: AddressSanitizer and UndefinedBehaviorSanitizer on
# the host pass only (the device code is compiled plainly, at -O1, and never
# runs: the CPU tests exercise the argument checks, planners and error
# paths, on a machine without a GPU).
SAN_FLAGS = [
    f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", "-fPIC", "-shared",
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_device", "-g0",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def san_is_stale() -> bool:
    if not SAN_LIB_PATH.exists():
        return True
    t = SAN_LIB_PATH.stat().st_mtime
    return any(p.stat().st_mtime > t for p in DEPENDS if p.exists())


def build_sanitized(verbose: bool = False) -> Path:
    """Compile the sanitized test build (_build/libmt_flce_san.so).  Always
    recompiles (about a minute).  Load it with the clang ASan runtime
    preloaded."""
    SAN_LIB_PATH.parent.mkdir(exist_ok=True)
    tmp = SAN_LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *SAN_FLAGS, "-o", str(tmp), *map(str, SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc (sanitized build) failed ({proc.returncode}):\n{proc.stderr}")
    os.replace(tmp, SAN_LIB_PATH)
    return SAN_LIB_PATH


def asan_runtime() -> Path:
    """The clang ASan runtime matching hipcc (to LD_PRELOAD into Python)."""
    clang = Path(hipcc()).resolve().parent.parent / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path("/opt/rocm/llvm/bin/clang")
    out = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    return Path(out)


def build_library(verbose: bool = False) -> Path:
    """Compile libmt_flce.so for gfx950.  Always recompiles."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *map(str, SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def is_stale() -> bool:
    if not LIB_PATH.exists():
        return True
    t = LIB_PATH.stat().st_mtime
    return any(p.stat().st_mtime > t for p in DEPENDS if p.exists())


if __name__ == "__main__":
    print(build_library(verbose=True))
