"""Build libmamba_selective_scan_hip.so for gfx950 with hipcc (no GPU needed).

Usage: python jax-mambas_amd/build.py [--verbose]
Output: jax-mambas_amd/build/libmamba_selective_scan_hip.so
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "build"
LIB_NAME = "libmamba_selective_scan_hip.so"
SOURCES = ["mss_fwd.hip", "mss_fwd_bf16.hip", "mss_bwd.hip", "mss_conv.hip", "mss_norm.hip", "mss_xent.hip", "mss_step.hip", "mss_complex.hip", "mss_gemv.hip", "mss_proj.hip",
           "mss_wgrad.hip", "mss_shadow.hip", "mss_adamw.hip", "mss_embed.hip", "mss_capi.cpp"]
ARCH = os.environ.get("MSS_OFFLOAD_ARCH", "gfx950")
# Per-source machine-scheduler choice (MI355X, 11 interleaved trials, bit-identical outputs):
# the backward scan and the bf16-I/O forward compiled with the ILP-maximising strategy run
# 2-3.5 % faster (c2 backward 221.7 -> 216.3 us, c3 924.5 -> 903.5, c4 3172 -> 3062, a c5
# layer 364.0 -> 356.7; c3 forward 424.7 -> 416.4, a c5 layer's 165.7 -> 162.9); the float32
# forward runs slower with it (c2 102 -> 108 us, c4 1345 -> 1411), so it and the other
# sources keep the default.
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {"mss_bwd.hip": _MAX_ILP, "mss_fwd_bf16.hip": _MAX_ILP}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed FP32 VALU forms are kept out of every kernel of this library.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
    ]


def build(verbose: bool = False, out_dir: Path | None = None, defines: dict | None = None) -> Path:
    """Compile the library; `defines` (name -> value) are passed as -D options."""
    out_dir = Path(out_dir) if out_dir is not None else BUILD
    out_dir.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{k}={v}" for k, v in (defines or {}).items()]
    objs = []
    for src in SOURCES:
        obj = out_dir / (src + ".o")
        cmd = [hipcc(), *flags(), *SOURCE_FLAGS.get(src, []), *extra, "-c", str(CSRC / src), "-o", str(obj)]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    out = out_dir / LIB_NAME
    tmp = out_dir / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="--verbose" in sys.argv)
    print(path)
