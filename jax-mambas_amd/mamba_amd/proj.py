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
include/mamba_selective_scan.h); callers use a library GEMM for the others.

``wgrad(dY, X, out=None, accumulate=False) -> C`` — the weight gradient of a dense
projection over channel-major activations, C = dY @ X^T (+ C) in float32 for dY (M, T) and
X (N, T), bf16 with contiguous rows (mss_wgrad: the tokens split over workgroups, partial
tiles added in a fixed order). ``wgrad_fits`` says whether a call should take it (N a
multiple of 4, T of 64, both M and N at least 192); callers use a library GEMM for the others.
"""
from __future__ import annotations

import torch

from . import _lib
from .selective_scan_hip import _require_gpu, _stream

__all__ = ["proj", "proj_fits", "wgrad", "wgrad_fits"]


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


def wgrad_fits(dY, X, out=None):
    if not (_rows_ok(dY) and _rows_ok(X)) or dY.shape[1] != X.shape[1]:
        return False
    if out is not None and not (out.dtype == torch.float32 and out.dim() == 2 and out.stride(1) == 1
                                and out.stride(0) % 4 == 0 and out.data_ptr() % 16 == 0):
        return False
    M, (N, T) = dY.shape[0], X.shape
    # The kernel takes any M and N % 4 == 0 (96 x 96 tiles when a side is below 192); for the
    # config-5 S6 projections' gradients (80 x 1536 and 1536 x 48 over 16384 tokens) the
    # library GEMM stays faster (kernel + sums 27.5-28.5 us against 21.5, MI355X), so
    # shapes with a side below 192 are left to it.
    return N % 4 == 0 and T % 64 == 0 and T > 0 and M >= 192 and N >= 192


def wgrad(dY, X, out=None, accumulate=False):
    """C = dY @ X^T (+ C when accumulate), float32 (M, N), for bf16 dY (M, T) and X (N, T) with
    contiguous rows. Raises _lib.MSSError for shapes mss_wgrad does not take (check
    wgrad_fits first)."""
    _require_gpu(dY, X)
    M, T = dY.shape
    N = X.shape[0]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an output to add to")
        out = torch.empty(M, N, dtype=torch.float32, device=X.device)
    lib = _lib.register_hip_kernel()
    ws_bytes = int(lib.mss_wgrad_workspace_bytes(M, N, T))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=X.device) if ws_bytes > 0 else None
    a = _lib.WgradArgs(M=M, N=N, K=T, accumulate=int(bool(accumulate)), lda=dY.stride(0), ldb=X.stride(0),
                       ldc=out.stride(0), A=dY.data_ptr(), B=X.data_ptr(), C=out.data_ptr(),
                       workspace=ws.data_ptr() if ws is not None else None, workspace_bytes=ws_bytes)
    _lib.check(lib.mss_wgrad(a, _stream(X)), "mss_wgrad")
    return out
