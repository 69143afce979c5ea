"""Single-token recurrent step (decode) on MI355X: HIP kernels behind the C ABI.

``selective_state_update(state, u, delta, A, B, C, D=None, z=None, delta_bias=None,
delta_softplus=True, discretization="euler") -> out`` — one step of the selective scan for
every (b, d) channel, updating ``state`` (B, D, N) float32 in place (the layout of the
scan's last state, so a prefill hands over directly): S6.step, mamba/mamba1.py:200-214,
with the scan's fused extras (softplus(delta + bias), D skip, silu(z) gate).
u/delta/z: (B, D); B/C: (B, N); any strides (e.g. views of (D, B) activation matrices).
A complex64 A selects the complex-state step (state complex64, the complex scan's last
state; output sum_n C Re(state) + D u).

``causal_conv1d_update(conv_state, x, weight, bias=None, activation="silu") -> y`` — the
conv window step of Mamba.step (:339-363): y = act(bias + sum_k weight[:, k] * window[k])
for window = [conv_state, x]; ``conv_state`` (B, D, K-1) shifts in place.

``gemv(w, x) -> y`` — ``w @ x`` for decode shapes (the block's projections over a few
tokens): w (M, K) bf16 with 16-byte aligned rows, x (K, N) bf16 contiguous and 16-byte
aligned with N in {1, 2, 4, 8}, K % 8 == 0, 2*K*N <= 64 KiB; y (M, N) bf16, float32
accumulation. Other shapes and dtypes go through ``torch.mm``.

Inference only (no autograd); there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib
from .selective_scan_hip import _io_tag, _ptr, _require_gpu, _stream

__all__ = ["selective_state_update", "causal_conv1d_update", "gemv"]


def _strides2(t):
    """(batch stride, row stride) of a (B, X) tensor; the kernels take any non-negative pair."""
    sb, sx = t.stride()
    if sb < 0 or sx < 0:
        raise ValueError("negative strides are not supported")
    return sb, sx


def selective_state_update(state, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=True,
                           discretization="euler"):
    cplx = A.is_complex()
    sdt, adt = (torch.complex64, torch.complex64) if cplx else (torch.float32, torch.float32)
    if state.dtype != sdt or state.ndim != 3 or not state.is_contiguous():
        raise ValueError(f"state must be a contiguous {sdt} (B, D, N) tensor")
    batch, dim, n = state.shape
    if not 1 <= n <= _lib.MSS_MAX_DSTATE:
        raise ValueError(f"N must be between 1 and {_lib.MSS_MAX_DSTATE}")
    if discretization not in ("euler", "zoh"):
        raise ValueError("discretization must be 'euler' or 'zoh'")
    for name, t in (("u", u), ("delta", delta), ("z", z)):
        if t is not None and (tuple(t.shape) != (batch, dim) or t.dtype != u.dtype or t.stride() != u.stride()):
            raise ValueError(f"{name} must be ({batch}, {dim}) with u's dtype and strides")
    for name, t in (("B", B), ("C", C)):
        if tuple(t.shape) != (batch, n) or t.dtype != B.dtype or t.stride() != B.stride():
            raise ValueError(f"{name} must be ({batch}, {n}) with B's dtype and strides")
    if A.dtype != adt or tuple(A.shape) != (dim, n):
        raise ValueError(f"A must be {adt} ({dim}, {n})")
    _require_gpu(state, u, delta, A, B, C, D, z, delta_bias)
    lib = _lib.register_hip_kernel()
    out = torch.empty_strided(u.shape, u.stride(), dtype=u.dtype, device=u.device)
    io_b, io_d = _strides2(u)
    bc_b, bc_n = _strides2(B)
    Ac = A.contiguous()  # complex A and state: interleaved (real, imaginary) float32 pairs
    a = _lib.StepArgs(batch=batch, dim=dim, dstate=n,
                      discretization=_lib.MSS_ZOH if discretization == "zoh" else _lib.MSS_EULER,
                      delta_softplus=int(bool(delta_softplus)), io_dtype=_io_tag(u.dtype, "u"),
                      bc_dtype=_io_tag(B.dtype, "B"), state=state.data_ptr(), u=u.data_ptr(),
                      delta=delta.data_ptr(), A=Ac.data_ptr(), B=B.data_ptr(), C=C.data_ptr(),
                      D=_ptr(None if D is None else D.contiguous()), z=_ptr(z),
                      delta_bias=_ptr(None if delta_bias is None else delta_bias.contiguous()), out=out.data_ptr(),
                      strides=_lib.Strides(io_batch=io_b, io_dim=io_d, bc_batch=bc_b, bc_state=bc_n))
    if cplx:
        _lib.check(lib.mss_cscan_step(a, _stream(u)), "mss_cscan_step")
    else:
        _lib.check(lib.mss_scan_step(a, _stream(u)), "mss_scan_step")
    return out


def causal_conv1d_update(conv_state, x, weight, bias=None, activation="silu"):
    batch, dim = x.shape
    k = weight.shape[1]
    if tuple(conv_state.shape) != (batch, dim, k - 1) or conv_state.dtype != x.dtype or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be a contiguous ({batch}, {dim}, {k - 1}) tensor of x's dtype")
    if weight.dtype != torch.float32 or not 1 <= k <= 4:
        raise ValueError("weight must be float32 (D, K) with K <= 4")
    _require_gpu(conv_state, x, weight, bias)
    lib = _lib.register_hip_kernel()
    y = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device)
    sb, sd = _strides2(x)
    a = _lib.ConvStepArgs(batch=batch, dim=dim, width=k, io_dtype=_io_tag(x.dtype, "x"),
                          activation=1 if activation == "silu" else 0, conv_state=conv_state.data_ptr(),
                          x=x.data_ptr(), weight=weight.contiguous().data_ptr(),
                          bias=_ptr(None if bias is None else bias.contiguous()), y=y.data_ptr(),
                          strides=_lib.Strides(io_batch=sb, io_dim=sd))
    _lib.check(lib.mss_conv_step(a, _stream(x)), "mss_conv_step")
    return y


def gemv(w, x):
    m, k = w.shape
    if (w.dtype != torch.bfloat16 or x.dtype != torch.bfloat16 or not w.is_cuda or x.device != w.device
            or x.ndim != 2 or x.shape[0] != k or x.shape[1] not in (1, 2, 4, 8) or k % 8 != 0
            or not x.is_contiguous() or x.data_ptr() % 16 != 0 or 2 * k * x.shape[1] > 65536
            or w.stride(1) != 1 or w.stride(0) % 8 != 0 or w.data_ptr() % 16 != 0):
        return torch.mm(w, x)
    lib = _lib.register_hip_kernel()
    n = x.shape[1]
    y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    a = _lib.GemvArgs(M=m, K=k, N=n, ldw=w.stride(0), W=w.data_ptr(), X=x.data_ptr(), Y=y.data_ptr())
    _lib.check(lib.mss_gemv(a, _stream(x)), "mss_gemv")
    return y
