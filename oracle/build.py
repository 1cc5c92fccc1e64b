"""Build recipe of the C restatement (test infrastructure only).

gcc -O2 -shared -fPIC oracle/flce_ref.c -> oracle/_build/libflce_ref.so.
The reference itself is pure Python (no C/C++ sources), so there is no
compiled reference build under oracle/_ref.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "flce_ref.c"
OUT_DIR = ORACLE_DIR / "_build"
LIB = OUT_DIR / "libflce_ref.so"


def build(sanitize: bool = False) -> Path:
    """Always recompiles.  sanitize=True adds ASan/UBSan (host code only)."""
    OUT_DIR.mkdir(exist_ok=True)
    out = LIB if not sanitize else OUT_DIR / "libflce_ref_san.so"
    cmd = ["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-Wall", "-Wextra", "-o", str(out) + ".tmp",
           str(SRC), "-lm"]
    if sanitize:
        cmd[1:1] = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"]
    subprocess.run(cmd, check=True)
    os.replace(str(out) + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build())
