"""Skinny projection GEMMs of the training step on MI355X (HIP kernels behind the C ABI).

The selective scan's input projections (the reference's s_B / s_C / Linear_R stacked as one
x-projection, d_inner -> R + 2N, and Linear_Delta, R -> d_inner; mamba/mamba1.py:52-67,
107-124) each stream one (features, tokens) activation matrix past a weight with at most
128 rows or columns. These run them on the matrix cores with the big operand read once:

``proj(W, X, out=None, accumulate=False) -> C`` — C = W @ X (+ C), bf16 (M, K) @ (K, T),
float32 sums rounded to bf16 once (mss_proj). W may be the transposed view of a stored
(K, M) weight (``Wt.t()``): the kernels read it in place.

``proj_fits`` says whether a call has a shape and layout these kernels take (rows
contiguous, 16-byte aligned, row strides multiples of 8; the shape limits of
include/mamba_selective_scan.h); callers use a library GEMM for the others, and for the
weight gradients.
"""
from __future__ import annotations

import torch

from . import _lib
from .selective_scan_hip import _require_gpu, _stream

__all__ = ["proj", "proj_fits"]


def _rows_ok(t):
    return (t.dtype == torch.bfloat16 and t.dim() == 2 and t.is_cuda and t.stride(1) == 1
            and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0)


def _weight_rows(W):
    """(rows-contiguous matrix holding W, transposed?) for W or a transposed view W = Wt.t()."""
    if W.dim() == 2 and W.stride(1) != 1 and W.stride(0) == 1:
        return W.t(), True
    return W, False


def proj_fits(W, X, out=None):
    Wr, _ = _weight_rows(W)
    if not (_rows_ok(Wr) and _rows_ok(X)) or (out is not None and not _rows_ok(out)):
        return False
    M, K = W.shape
    if X.shape[0] != K:
        return False
    T = X.shape[1]
    shape_ok = (K <= 128 and K % 16 == 0) or (K % 64 == 0 and M <= 128)
    return M % 16 == 0 and T % 64 == 0 and shape_ok


def proj(W, X, out=None, accumulate=False):
    """C = W @ X (+ C when accumulate): W (M, K) (or a transposed view of a (K, M) matrix), X
    (K, T), C (M, T), all bf16 with contiguous rows. Raises _lib.MSSError for shapes mss_proj
    does not take (check proj_fits first)."""
    _require_gpu(W, X)
    M, K = W.shape
    T = X.shape[1]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an output to add to")
        out = torch.empty(M, T, dtype=torch.bfloat16, device=X.device)
    lib = _lib.register_hip_kernel()
    Wr, trans = _weight_rows(W)
    a = _lib.ProjArgs(M=M, K=K, T=T, accumulate=int(bool(accumulate)), w_trans=int(trans), ldw=Wr.stride(0),
                      ldx=X.stride(0), ldc=out.stride(0), W=Wr.data_ptr(), X=X.data_ptr(), C=out.data_ptr())
    _lib.check(lib.mss_proj(a, _stream(X)), "mss_proj")
    return out
