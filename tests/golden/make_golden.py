"""Writes the golden fixtures of the scan's reference API (tests/golden/*.npz).

Inputs follow the reference tests' recipe (tests/test_selective_scan_cuda.py:11-19: A =
-exp(N(0,1)) of shape (D, N), deltas = softplus(N(0,1)), Bs, Cs, u, x0 ~ N(0,1)) drawn with
numpy's seeded generator at the reference's lengths — forward L in {1, 17, 128, 513}
(B=2, D=8, N=16), VJP L in {1, 31, 513, 2051} (B=1, D=4, N=8) for Euler and ZOH — and the
expected outputs come from the float64 oracle (oracle/scan64.py). The reference cannot be
run here (no jax, no CUDA), so the fixtures pin the build's HIP path to its oracle at the
reference's own test points, and pin the oracle against later edits.

Usage: python tests/golden/make_golden.py   (rewrites the .npz files next to this script)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import scan64  # noqa: E402

FWD_LENGTHS = (1, 17, 128, 513)
VJP_LENGTHS = (1, 31, 513, 2051)


def recipe(seed, batch, length, dim, n):
    rng = np.random.default_rng(seed)
    A = -np.exp(rng.standard_normal((dim, n)))
    deltas = np.log1p(np.exp(rng.standard_normal((batch, length, dim))))
    Bs = rng.standard_normal((batch, length, n))
    Cs = rng.standard_normal((batch, length, n))
    u = rng.standard_normal((batch, length, dim))
    x0 = rng.standard_normal((batch, dim, n))
    return [a.astype(np.float32) for a in (A, deltas, Bs, Cs, u, x0)]


def fwd_case(length, euler):
    A, dl, Bs, Cs, u, x0 = recipe(1000 + length, 2, length, 8, 16)
    y, fin, cs = scan64.reference_api_forward(A, dl, Bs, Cs, u, x0, use_euler_barB_approx=euler)
    return dict(A=A, deltas=dl, Bs=Bs, Cs=Cs, u=u, x0=x0, y=y, final_x=fin, chunk_states=cs)


def vjp_case(length, euler):
    A, dl, Bs, Cs, u, x0 = recipe(2000 + length, 1, length, 4, 8)
    rng = np.random.default_rng(3000 + length)
    dy = rng.standard_normal((1, length, 4)).astype(np.float32)
    dfin = rng.standard_normal((1, 4, 8)).astype(np.float32)
    y, fin, _ = scan64.reference_api_forward(A, dl, Bs, Cs, u, x0, use_euler_barB_approx=euler)
    g = scan64.reference_api_backward(A, dl, Bs, Cs, u, x0, dy, dfin, use_euler_barB_approx=euler)
    names = ("dA", "ddeltas", "dBs", "dCs", "du", "dx0")
    return dict(A=A, deltas=dl, Bs=Bs, Cs=Cs, u=u, x0=x0, dy=dy, dfinal_x=dfin, y=y, final_x=fin,
                **{k: v for k, v in zip(names, g)})


def cases():
    for euler in (True, False):
        tag = "euler" if euler else "zoh"
        for length in FWD_LENGTHS:
            yield f"fwd_{tag}_L{length}", fwd_case(length, euler)
        for length in VJP_LENGTHS:
            yield f"vjp_{tag}_L{length}", vjp_case(length, euler)


if __name__ == "__main__":
    for name, arrays in cases():
        np.savez_compressed(HERE / f"{name}.npz", **{k: np.asarray(v) for k, v in arrays.items()})
        print(name)
