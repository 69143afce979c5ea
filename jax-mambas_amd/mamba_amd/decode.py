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

``norm_gemv_conv_update(h, delta, norm_weight, eps, w, conv_state, weight, bias=None)
-> (hn, u, rest)`` — the block entry of a decode step: hn, x = add_rmsnorm(h, delta,
norm_weight, eps) followed by gemv_conv_update(w, x, ...), as one kernel (every workgroup
normalises the few tokens itself) where it applies, else the two calls; same results.

``gemv_conv_update(w, x, conv_state, weight, bias=None) -> (u, rest)`` and
``gemv_state_update(w, x, state, u, A, B, C, ...) -> out`` — a decode GEMM with the next
step fused behind it (one kernel instead of two): the conv window step on the first D
rows of ``w @ x`` (the in-projection), and the selective-state step with ``w @ x`` as the
raw delta (the dt projection). Same results as ``gemv`` followed by the step call.

Inference only (no autograd); there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib
from .lm_ops import add_rmsnorm
from .selective_scan_hip import _io_tag, _ptr, _require_gpu, _stream

__all__ = ["selective_state_update", "causal_conv1d_update", "gemv", "gemv_conv_update", "gemv_state_update",
           "norm_gemv_conv_update"]


def _strides2(t):
    """(batch stride, row stride) of a (B, X) tensor; the kernels take any non-negative pair."""
    sb, sx = t.stride()
    if sb < 0 or sx < 0:
        raise ValueError("negative strides are not supported")
    return sb, sx


def _step_args(state, u, delta, A, B, C, D, z, delta_bias, delta_softplus, discretization):
    """Checked StepArgs, the output tensor and the tensors the call must keep alive;
    delta None when the raw delta comes from a fused GEMM."""
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
    out = torch.empty_strided(u.shape, u.stride(), dtype=u.dtype, device=u.device)
    io_b, io_d = _strides2(u)
    bc_b, bc_n = _strides2(B)
    keep = (A.contiguous(),  # complex A and state: interleaved (real, imaginary) float32 pairs
            None if D is None else D.contiguous(), None if delta_bias is None else delta_bias.contiguous())
    a = _lib.StepArgs(batch=batch, dim=dim, dstate=n,
                      discretization=_lib.MSS_ZOH if discretization == "zoh" else _lib.MSS_EULER,
                      delta_softplus=int(bool(delta_softplus)), io_dtype=_io_tag(u.dtype, "u"),
                      bc_dtype=_io_tag(B.dtype, "B"), state=state.data_ptr(), u=u.data_ptr(),
                      delta=_ptr(delta), A=keep[0].data_ptr(), B=B.data_ptr(), C=C.data_ptr(),
                      D=_ptr(keep[1]), z=_ptr(z), delta_bias=_ptr(keep[2]), out=out.data_ptr(),
                      strides=_lib.Strides(io_batch=io_b, io_dim=io_d, bc_batch=bc_b, bc_state=bc_n))
    return a, out, keep


def selective_state_update(state, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=True,
                           discretization="euler"):
    a, out, keep = _step_args(state, u, delta, A, B, C, D, z, delta_bias, delta_softplus, discretization)
    lib = _lib.register_hip_kernel()
    if A.is_complex():
        _lib.check(lib.mss_cscan_step(a, _stream(u)), "mss_cscan_step")
    else:
        _lib.check(lib.mss_scan_step(a, _stream(u)), "mss_scan_step")
    return out


def _conv_step_args(conv_state, x, weight, bias, activation, y):
    """Checked ConvStepArgs writing y (x's shape and strides); x may be a shape-only
    stand-in when the conv input comes from a fused GEMM."""
    batch, dim = x.shape
    k = weight.shape[1]
    if tuple(conv_state.shape) != (batch, dim, k - 1) or conv_state.dtype != x.dtype or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be a contiguous ({batch}, {dim}, {k - 1}) tensor of x's dtype")
    if weight.dtype != torch.float32 or not 1 <= k <= 4:
        raise ValueError("weight must be float32 (D, K) with K <= 4")
    _require_gpu(conv_state, x, weight, bias)
    sb, sd = _strides2(x)
    keep = (weight.contiguous(), None if bias is None else bias.contiguous())
    a = _lib.ConvStepArgs(batch=batch, dim=dim, width=k, io_dtype=_io_tag(x.dtype, "x"),
                          activation=1 if activation == "silu" else 0, conv_state=conv_state.data_ptr(),
                          x=x.data_ptr(), weight=keep[0].data_ptr(), bias=_ptr(keep[1]), y=y.data_ptr(),
                          strides=_lib.Strides(io_batch=sb, io_dim=sd))
    return a, keep


def causal_conv1d_update(conv_state, x, weight, bias=None, activation="silu"):
    y = torch.empty_strided(x.shape, x.stride(), dtype=x.dtype, device=x.device)
    a, keep = _conv_step_args(conv_state, x, weight, bias, activation, y)
    lib = _lib.register_hip_kernel()
    _lib.check(lib.mss_conv_step(a, _stream(x)), "mss_conv_step")
    return y


def _gemv_w_ok(w, k, n, device):
    """Whether mss_gemv takes w for a (k, n) bf16 X on `device` (a few token columns,
    aligned rows, X fits in LDS)."""
    return not (w.dtype != torch.bfloat16 or not w.is_cuda or w.device != device or w.ndim != 2
                or w.shape[1] != k or n not in (1, 2, 4, 8) or k % 8 != 0 or 2 * k * n > 65536
                or w.stride(1) != 1 or w.stride(0) % 8 != 0 or w.data_ptr() % 16 != 0)


def _gemv_ok(w, x):
    """Whether mss_gemv takes w @ x (bf16, a few token columns, aligned, X fits in LDS)."""
    return (x.dtype == torch.bfloat16 and x.ndim == 2 and x.is_contiguous() and x.data_ptr() % 16 == 0
            and _gemv_w_ok(w, x.shape[0], x.shape[1], x.device))


def _gemv_args(w, x, y):
    m, k = w.shape
    return _lib.GemvArgs(M=m, K=k, N=x.shape[1], ldw=w.stride(0), W=w.data_ptr(), X=x.data_ptr(),
                         Y=_ptr(y))


def gemv(w, x):
    """w @ x for a decode step: the HIP decode GEMM (bf16 in and out, float32 sums) where it
    applies, else torch.mm."""
    if not _gemv_ok(w, x):
        return torch.mm(w, x)
    lib = _lib.register_hip_kernel()
    y = torch.empty(w.shape[0], x.shape[1], dtype=torch.bfloat16, device=x.device)
    _lib.check(lib.mss_gemv(_gemv_args(w, x, y), _stream(x)), "mss_gemv")
    return y


def gemv_conv_update(w, x, conv_state, weight, bias=None, activation="silu"):
    """(u, rest) for v = w @ x (rows, tokens) whose first D rows are the conv input of a
    decode step: u = causal_conv1d_update(conv_state, v[:D].t(), weight, bias).t() (D, B)
    and rest = v[D:]. One fused HIP kernel where the GEMM applies, else the two calls."""
    dim = weight.shape[0]
    if not _gemv_ok(w, x) or conv_state.dtype != torch.bfloat16 or not dim <= w.shape[0]:
        v = gemv(w, x)
        return causal_conv1d_update(conv_state, v[:dim].t(), weight, bias, activation).t(), v[dim:]
    n = x.shape[1]
    u = torch.empty(dim, n, dtype=torch.bfloat16, device=x.device)
    v = torch.empty(w.shape[0], n, dtype=torch.bfloat16, device=x.device)
    a, keep = _conv_step_args(conv_state, u.t(), weight, bias, activation, u.t())
    a.x = None
    lib = _lib.register_hip_kernel()
    _lib.check(lib.mss_gemv_conv_step(_gemv_args(w, x, v), a, _stream(x)), "mss_gemv_conv_step")
    return u, v[dim:]


def _aligned_matrix(t, shape, dtype):
    return t.dtype == dtype and tuple(t.shape) == shape and t.is_contiguous() and t.data_ptr() % 16 == 0


def norm_gemv_conv_update(h, delta, norm_weight, eps, w, conv_state, weight, bias=None, activation="silu"):
    """(hn, u, rest): hn, x = add_rmsnorm(h, delta, norm_weight, eps) (h: the float32
    (features, B) stream, delta: the previous block's bf16 output or None) and
    u, rest = gemv_conv_update(w, x, conv_state, weight, bias, activation), as one HIP
    kernel (mss_norm_gemv_conv_step) where it applies, else the calls; same results."""
    f, n = h.shape
    dim = weight.shape[0]
    fused = (_aligned_matrix(h, (f, n), torch.float32) and f <= _lib.MSS_NORM_GEMV_MAX_FEATURES
             and (delta is None or _aligned_matrix(delta, (f, n), torch.bfloat16))
             and norm_weight.dtype == torch.float32 and tuple(norm_weight.shape) == (f,)
             and conv_state.dtype == torch.bfloat16 and dim <= w.shape[0] and _gemv_w_ok(w, f, n, h.device))
    if not fused:
        hn, x = add_rmsnorm(h, delta, norm_weight, eps, torch.bfloat16)
        u, rest = gemv_conv_update(w, x, conv_state, weight, bias, activation)
        return hn, u, rest
    _require_gpu(h, delta, norm_weight)
    hn = torch.empty_like(h) if delta is not None else h
    u = torch.empty(dim, n, dtype=torch.bfloat16, device=h.device)
    v = torch.empty(w.shape[0], n, dtype=torch.bfloat16, device=h.device)
    a, keep = _conv_step_args(conv_state, u.t(), weight, bias, activation, u.t())
    a.x = None
    nw = norm_weight.contiguous()
    na = _lib.NormArgs(features=f, tokens=n, eps=float(eps), io_dtype=_lib.MSS_BF16, h=h.data_ptr(),
                       delta=_ptr(delta), weight=nw.data_ptr(), hn=hn.data_ptr() if delta is not None else None)
    g = _lib.GemvArgs(M=w.shape[0], K=f, N=n, ldw=w.stride(0), W=w.data_ptr(), X=None, Y=v.data_ptr())
    lib = _lib.register_hip_kernel()
    _lib.check(lib.mss_norm_gemv_conv_step(na, g, a, _stream(h)), "mss_norm_gemv_conv_step")
    return hn, u, v[dim:]


def gemv_state_update(w, x, state, u, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=True,
                      discretization="euler"):
    """selective_state_update(state, u, (w @ x).t(), ...): the raw delta of a decode step
    as a GEMM, fused with the state update in one HIP kernel where the GEMM applies (real
    A, bf16 u and B), else the two calls."""
    if (not _gemv_ok(w, x) or A.is_complex() or u.dtype != torch.bfloat16 or B.dtype != torch.bfloat16
            or w.shape[0] != u.shape[1] or x.shape[1] != u.shape[0]):
        return selective_state_update(state, u, gemv(w, x).t(), A, B, C, D, z, delta_bias, delta_softplus,
                                      discretization)
    a, out, keep = _step_args(state, u, None, A, B, C, D, z, delta_bias, delta_softplus, discretization)
    lib = _lib.register_hip_kernel()
    _lib.check(lib.mss_gemv_scan_step(_gemv_args(w, x, None), a, _stream(x)), "mss_gemv_scan_step")
    return out
