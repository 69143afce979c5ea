"""Causal depthwise conv1d + SiLU on MI355X (HIP kernels behind the C ABI).

``causal_conv1d_fn(x, weight, bias=None, seq_lens=None, activation="silu")`` —
x: (B, D, L) with contiguous steps (batch-outer [B][D][L] rows or channel-outer
[D][B][L] rows, e.g. an (D, B*L) activation matrix viewed as (B, D, L)); weight (D, K)
float32 with K <= 4; bias (D,) float32. Returns y in x's layout and dtype:
``y[t] = act(bias + sum_k weight[:, k] * x[t - (K-1) + k])``, 0 for t >= seq_lens[b].
This is the Mamba-1 block's short convolution (reference ``mamba/mamba1.py:250-255,
313-329``, an XLA convolution there). Differentiable; the backward is a HIP kernel too.
There is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib
from .selective_scan_hip import _conform, _empty_rows, _io_tag, _layout_of, _ptr, _require_gpu, _row_strides, _stream

__all__ = ["causal_conv1d_fn"]

_ACT = {"silu": 1, None: 0, "none": 0}


def _args(x, weight, bias, seq_lens, act, layout):
    b, d, l = x.shape
    sb, sd = _row_strides(x, layout)
    return _lib.ConvArgs(batch=b, dim=d, seqlen=l, width=weight.shape[1], io_dtype=_io_tag(x.dtype, "x"),
                         activation=act, x=_ptr(x), weight=_ptr(weight), bias=_ptr(bias),
                         seq_lens=_ptr(seq_lens), strides=_lib.Strides(io_batch=sb, io_dim=sd))


class _CausalConv1d(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, seq_lens, act, layout):
        lib = _lib.register_hip_kernel()
        y = _empty_rows(x.shape, layout, x.dtype, x.device)
        a = _args(x, weight, bias, seq_lens, act, layout)
        a.y = y.data_ptr()
        _lib.check(lib.mss_conv_fwd(a, _stream(x)), "mss_conv_fwd")
        ctx.save_for_backward(x, weight, bias, seq_lens)
        ctx.act, ctx.layout = act, layout
        return y

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.register_hip_kernel()
        x, weight, bias, seq_lens = ctx.saved_tensors
        dy = _conform(dy.to(x.dtype), ctx.layout)
        dx = _empty_rows(x.shape, ctx.layout, x.dtype, x.device)
        dw = torch.empty_like(weight)
        db = None if bias is None else torch.empty_like(bias)
        a = _args(x, weight, bias, seq_lens, ctx.act, ctx.layout)
        a.dy, a.dx, a.dweight, a.dbias = dy.data_ptr(), dx.data_ptr(), dw.data_ptr(), _ptr(db)
        ws_bytes = int(lib.mss_conv_bwd_workspace_bytes(a))
        ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
        _lib.check(lib.mss_conv_bwd(a, _stream(x)), "mss_conv_bwd")
        return dx, dw, db, None, None, None


def causal_conv1d_fn(x, weight, bias=None, seq_lens=None, activation="silu"):
    if activation not in _ACT:
        raise ValueError("activation must be 'silu' or None")
    if x.ndim != 3 or weight.ndim != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError("x must be (B, D, L) and weight (D, K)")
    if not 1 <= weight.shape[1] <= 4:
        raise ValueError("the kernel width K must be between 1 and 4")
    if x.shape[2] == 0:
        raise ValueError("The sequence length must be positive")
    _io_tag(x.dtype, "x")
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32, got {t.dtype}")
    if bias is not None and tuple(bias.shape) != (x.shape[1],):
        raise ValueError(f"bias must have shape ({x.shape[1]},)")
    if seq_lens is not None and (seq_lens.dtype != torch.int32 or tuple(seq_lens.shape) != (x.shape[0],)):
        raise ValueError(f"seq_lens must be int32 with shape ({x.shape[0]},)")
    _require_gpu(x, weight, bias, seq_lens)
    _lib.register_hip_kernel()
    layout = _layout_of(x) or "brl"
    return _CausalConv1d.apply(_conform(x, layout), weight.contiguous(),
                               None if bias is None else bias.contiguous(),
                               None if seq_lens is None else seq_lens.contiguous(),
                               _ACT[activation], layout)
