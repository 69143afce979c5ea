"""The benchmark configurations and their seeded synthetic inputs (numpy, host side).

Input recipe (seed 0, ``np.random.default_rng``), channel-major layout:
  u, z, delta_raw ~ N(0, 1) with shape (B, D, L); B, C ~ N(0, 1) with shape (B, N, L);
  dt ~ U[1e-3, 1e-1] per channel, delta_bias = dt + log(-expm1(-dt)) (inverse softplus,
  as the reference's dt-bias initialiser, mamba/mamba1.py:79-90); delta_softplus on;
  A[d, n] = -(n + 1) (S4D-real, mamba/mamba1.py:40-45); D = 1; initial state 0.
bf16 configs sample in float32 and round u/delta/B/C/z/dout to bfloat16; A, D, bias
stay float32. Variable-length configs draw lengths uniformly in [lo, hi] and fill the
padded positions with N(0, 1) values so a leak would be visible.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class ScanConfig:
    name: str
    batch: int
    dim: int
    length: int
    dstate: int = 16
    dtype: str = "f32"  # activation dtype: "f32" or "bf16"
    varlen: tuple | None = None  # (lo, hi) inclusive
    description: str = ""


C2 = ScanConfig("c2", 4, 1536, 2048, 16, "f32", None,
                "selective_scan fp32 B=4 D=1536 L=2048 N=16 (softplus+bias, D, z, last state)")
C3 = ScanConfig("c3", 8, 2048, 4096, 16, "bf16", None,
                "selective_scan bf16 I/O, fp32 accumulation, B=8 D=2048 L=4096 N=16")
C4 = ScanConfig("c4", 16, 2560, 8192, 16, "f32", (512, 8192),
                "variable-length fp32 B=16 D=2560 L=8192 N=16, lengths U[512, 8192]")
CONFIGS = {c.name: c for c in (C2, C3, C4)}


def make_scan_inputs(cfg: ScanConfig, seed: int = 0, with_z: bool = True, with_dout: bool = False):
    rng = np.random.default_rng(seed)
    b, d, l, n = cfg.batch, cfg.dim, cfg.length, cfg.dstate
    f = np.float32
    x = {}
    x["u"] = rng.standard_normal((b, d, l), dtype=f)
    x["delta"] = rng.standard_normal((b, d, l), dtype=f)
    x["B"] = rng.standard_normal((b, n, l), dtype=f)
    x["C"] = rng.standard_normal((b, n, l), dtype=f)
    if with_z:
        x["z"] = rng.standard_normal((b, d, l), dtype=f)
    dt = rng.uniform(1e-3, 1e-1, size=d)
    x["delta_bias"] = (dt + np.log(-np.expm1(-dt))).astype(f)
    x["A"] = np.broadcast_to(-(np.arange(n, dtype=f) + 1), (d, n)).copy()
    x["D"] = np.ones(d, dtype=f)
    if cfg.varlen is not None:
        lo, hi = cfg.varlen
        x["seq_lens"] = rng.integers(lo, hi + 1, size=b).astype(np.int32)
    if with_dout:
        x["dout"] = rng.standard_normal((b, d, l), dtype=f)
    if cfg.dtype == "bf16":
        for k in ("u", "delta", "B", "C", "z", "dout"):
            if k in x:
                x[k] = round_to_bf16(x[k])
    return x


def round_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def algorithmic_bytes(cfg: ScanConfig, seq_lens=None, with_z: bool = True):
    """Roofline denominators (each tensor counted once) for forward and backward.

    fwd = s*(3E) [u, delta, z] + s*2BNL [B, C] + 4(DN + 2D) [A, D, bias] + s*E [out]
          + 4*BDN [last state]
    bwd = s*(4E) [u, delta, z, dout] + s*2BNL + 4(DN + 2D) + 4*BDN [dlast]
          + s*(3E) [du, ddelta, dz] + 4*2BNL [dB, dC] + 4(DN + 2D) [dA, dD, dbias]
    For variable lengths E counts valid steps for reads and the full padded size for
    the zero-filled writes.
    """
    s = 2 if cfg.dtype == "bf16" else 4
    b, d, l, n = cfg.batch, cfg.dim, cfg.length, cfg.dstate
    e_full = b * d * l
    e_read = d * int(np.sum(seq_lens)) if seq_lens is not None else e_full
    nz = 1 if with_z else 0
    bnl = b * n * l
    small = 4 * (d * n + 2 * d)
    fwd = s * (2 + nz) * e_read + s * 2 * bnl + small + s * e_full + 4 * b * d * n
    bwd = (s * (3 + nz) * e_read + s * 2 * bnl + small + 4 * b * d * n
           + s * (2 + nz) * e_full + 4 * 2 * bnl + small)
    return fwd, bwd
