"""Build the float64 C oracle (oracle/scan64c.c) — TEST INFRASTRUCTURE ONLY.

Usage: python oracle/build_oracle.py
Output: oracle/_build/libscan64c.so (git-ignored; it travels to the GPU box with the tree).
gcc, OpenMP, -O2 without fast-math, so float64 arithmetic keeps IEEE semantics.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "libscan64c.so"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fopenmp", "-fPIC", "-shared", "-Wall",
           str(HERE / "scan64c.c"), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
