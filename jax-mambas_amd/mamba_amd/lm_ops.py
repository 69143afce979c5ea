"""Language-model glue on MI355X (HIP kernels behind the C ABI): residual add + RMSNorm over
a channel-major stream, and cross-entropy over bf16 logits.

``add_rmsnorm(h, delta, weight, eps=1e-5, out_dtype=torch.bfloat16) -> (hn, x)`` —
h: (features, tokens) float32 residual stream; delta: the previous block's output in
out_dtype, or None; returns hn = h + delta (h itself when delta is None) and
x = rmsnorm(hn) * weight in out_dtype (mamba/mamba1.py:300-337, nnx.RMSNorm(epsilon)).

``cross_entropy(logits, targets) -> mean loss`` — logits (rows, vocab) bfloat16, targets
(rows,) int64; fp32 math; the backward writes bf16 logit gradients in one pass.

``embed_cm(table, tokens, holder=None) -> h`` — the input embedding gathered straight into
the channel-major stream (D, T) (nnx.Embed, mamba/mamba1.py:378-380), its gradient summed
per token deterministically, optionally into the tied head's gradient (GradHolder).

All are differentiable; there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib
from .selective_scan_hip import _io_tag, _ptr, _require_gpu, _stream

__all__ = ["add_rmsnorm", "cross_entropy", "embed_cm", "GradHolder"]


def _norm_args(hsrc, weight, eps, io):
    f, t = hsrc.shape
    return _lib.NormArgs(features=f, tokens=t, eps=eps, io_dtype=io, h=hsrc.data_ptr(), weight=weight.data_ptr())


class _AddRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, delta, weight, eps, out_dtype):
        lib = _lib.register_hip_kernel()
        io = _io_tag(out_dtype, "out_dtype")
        a = _norm_args(h, weight, eps, io)
        hn = torch.empty_like(h) if delta is not None else h
        x = torch.empty(h.shape, dtype=out_dtype, device=h.device)
        rstd = torch.empty(h.shape[1], dtype=torch.float32, device=h.device)
        a.delta, a.hn, a.x, a.rstd = _ptr(delta), (hn.data_ptr() if delta is not None else None), x.data_ptr(), rstd.data_ptr()
        _lib.check(lib.mss_norm_fwd(a, _stream(h)), "mss_norm_fwd")
        ctx.save_for_backward(hn, weight, rstd)
        ctx.eps, ctx.io, ctx.has_delta = eps, io, delta is not None
        return (hn, x) if delta is not None else x

    @staticmethod
    def backward(ctx, *grads):
        lib = _lib.register_hip_kernel()
        hn, weight, rstd = ctx.saved_tensors
        if ctx.has_delta:
            dhn_in, dx = grads
        else:
            dhn_in, dx = None, grads[0]
        out_dtype = torch.bfloat16 if ctx.io == _lib.MSS_BF16 else torch.float32
        dx = torch.zeros(hn.shape, dtype=out_dtype, device=hn.device) if dx is None else dx.to(out_dtype).contiguous()
        dhn_in = None if dhn_in is None else dhn_in.float().contiguous()
        a = _norm_args(hn, weight, ctx.eps, ctx.io)
        dhn = torch.empty_like(hn)
        ddelta = torch.empty(hn.shape, dtype=out_dtype, device=hn.device) if ctx.has_delta else None
        dw = torch.empty_like(weight)
        ws_bytes = int(lib.mss_norm_bwd_workspace_bytes(a))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=hn.device)
        a.rstd, a.dx, a.dhn_in, a.dhn, a.ddelta, a.dweight = (rstd.data_ptr(), dx.data_ptr(), _ptr(dhn_in),
                                                             dhn.data_ptr(), _ptr(ddelta), dw.data_ptr())
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
        _lib.check(lib.mss_norm_bwd(a, _stream(hn)), "mss_norm_bwd")
        return dhn, ddelta, dw, None, None


def add_rmsnorm(h, delta, weight, eps=1e-5, out_dtype=torch.bfloat16):
    if h.dtype != torch.float32 or h.ndim != 2:
        raise TypeError("h must be a float32 (features, tokens) matrix")
    if weight.dtype != torch.float32 or tuple(weight.shape) != (h.shape[0],):
        raise ValueError(f"weight must be float32 with shape ({h.shape[0]},)")
    if delta is not None and (delta.dtype != out_dtype or delta.shape != h.shape):
        raise ValueError("delta must have h's shape and the output dtype")
    _require_gpu(h, delta, weight)
    h = h.contiguous()
    delta = None if delta is None else delta.contiguous()
    if delta is None:
        return h, _AddRMSNorm.apply(h, None, weight, float(eps), out_dtype)
    return _AddRMSNorm.apply(h, delta, weight, float(eps), out_dtype)


class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets):
        lib = _lib.register_hip_kernel()
        rows, vocab = logits.shape
        loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
        lse = torch.empty(rows, dtype=torch.float32, device=logits.device)
        a = _lib.XentArgs(rows=rows, vocab=vocab, logits=logits.data_ptr(), targets=targets.data_ptr(),
                          loss=loss.data_ptr(), lse=lse.data_ptr())
        _lib.check(lib.mss_xent_fwd(a, _stream(logits)), "mss_xent_fwd")
        ctx.save_for_backward(logits, targets, lse)
        return loss.mean()

    @staticmethod
    def backward(ctx, grad):
        lib = _lib.register_hip_kernel()
        logits, targets, lse = ctx.saved_tensors
        rows, vocab = logits.shape
        scale = (grad.float() / rows).reshape(1).contiguous()
        dlogits = torch.empty_like(logits)
        a = _lib.XentArgs(rows=rows, vocab=vocab, logits=logits.data_ptr(), targets=targets.data_ptr(),
                          lse=lse.data_ptr(), grad_scale=scale.data_ptr(), dlogits=dlogits.data_ptr())
        _lib.check(lib.mss_xent_bwd(a, _stream(logits)), "mss_xent_bwd")
        return dlogits, None


class _CrossEntropyFused(torch.autograd.Function):
    """The loss and its gradient for the mean in one pass over the logits
    (mss_xent_fwd_grad); the backward only multiplies by the upstream gradient, and skips
    even that when it is 1 (mss_xent_rescale checks on the device). The logits are not kept."""

    @staticmethod
    def forward(ctx, logits, targets):
        lib = _lib.register_hip_kernel()
        rows, vocab = logits.shape
        loss = torch.empty(rows, dtype=torch.float32, device=logits.device)
        lse = torch.empty(rows, dtype=torch.float32, device=logits.device)
        scale = torch.full((1,), 1.0 / rows, dtype=torch.float32, device=logits.device)
        dlogits = torch.empty_like(logits)
        a = _lib.XentArgs(rows=rows, vocab=vocab, logits=logits.data_ptr(), targets=targets.data_ptr(),
                          loss=loss.data_ptr(), lse=lse.data_ptr(), grad_scale=scale.data_ptr(),
                          dlogits=dlogits.data_ptr())
        _lib.check(lib.mss_xent_fwd_grad(a, _stream(logits)), "mss_xent_fwd_grad")
        ctx.save_for_backward(dlogits)
        return loss.mean()

    @staticmethod
    def backward(ctx, grad):
        lib = _lib.register_hip_kernel()
        (dlogits,) = ctx.saved_tensors
        factor = grad.float().reshape(1).contiguous()
        _lib.check(lib.mss_xent_rescale(dlogits.data_ptr(), dlogits.numel(), factor.data_ptr(), _stream(dlogits)),
                   "mss_xent_rescale")
        return dlogits, None


def _fused_fits(logits):
    return (logits.shape[1] % 8 == 0 and logits.shape[1] <= _lib.MSS_XENT_FUSED_MAX_VOCAB
            and logits.data_ptr() % 16 == 0)


def cross_entropy(logits, targets):
    """Mean cross-entropy of bf16 (rows, vocab) logits against int64 targets. When the
    result will be differentiated (grad enabled, logits requiring grad) and the row fits,
    the loss and its gradient come from one pass over the logits."""
    if logits.dtype != torch.bfloat16 or logits.ndim != 2:
        raise TypeError("logits must be a bfloat16 (rows, vocab) matrix")
    if targets.dtype != torch.int64 or tuple(targets.shape) != (logits.shape[0],):
        raise ValueError(f"targets must be int64 with shape ({logits.shape[0]},)")
    _require_gpu(logits, targets)
    logits, targets = logits.contiguous(), targets.contiguous()
    if torch.is_grad_enabled() and logits.requires_grad and _fused_fits(logits):
        return _CrossEntropyFused.apply(logits, targets)
    return _CrossEntropy.apply(logits, targets)


class GradHolder:
    """Passes the tied output head's float32 gradient of the shared table to the embedding's
    backward, which adds its own part in place and hands the sum to autograd as the table's
    one gradient (instead of two dense gradients and an add). The head's backward runs first:
    it belongs to the end of the forward."""

    def __init__(self):
        self.grad = None

    def put(self, g):
        self.grad = g

    def take(self):
        g, self.grad = self.grad, None
        return g


class _EmbedCM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, table, tokens, holder):
        lib = _lib.register_hip_kernel()
        V, D = table.shape
        T = tokens.numel()
        h = torch.empty(D, T, dtype=torch.float32, device=table.device)
        _lib.check(lib.mss_embed_cm(tokens.data_ptr(), T, table.data_ptr(), V, D, h.data_ptr(), T, _stream(table)),
                   "mss_embed_cm")
        ctx.save_for_backward(tokens)
        ctx.holder, ctx.shape = holder, table.shape
        return h

    @staticmethod
    def backward(ctx, dh):
        (tokens,) = ctx.saved_tensors
        de = ctx.holder.take() if ctx.holder is not None else None
        if de is None:
            de = torch.zeros(ctx.shape, dtype=torch.float32, device=dh.device)
        if not ctx.needs_input_grad[0]:
            return None, None, None
        dh = dh.contiguous()
        V, D = ctx.shape
        T = tokens.numel()
        st, order = torch.sort(tokens, stable=True)
        work = torch.empty(T, D, dtype=torch.float32, device=dh.device)
        lib = _lib.register_hip_kernel()
        _lib.check(lib.mss_embed_cm_backward(dh.data_ptr(), dh.stride(0), st.data_ptr(), order.data_ptr(), T, V, D,
                                             de.data_ptr(), work.data_ptr(), work.numel() * 4, _stream(dh)),
                   "mss_embed_cm_backward")
        return de, None, None


def embed_cm(table, tokens, holder=None):
    """h (D, T) float32 = table[tokens].T: the embedding rows of the flattened int64 tokens as
    the columns of a channel-major stream (HIP gather through LDS tiles; a token outside the
    table gives a column of NaN). Differentiable in `table`: the gradient is summed per token
    in a fixed association (deterministic); `holder` (GradHolder) carries a gradient of the
    same table from elsewhere (the tied head) to add to. Float32 tables, width a multiple of 4
    up to 1024 for the gradient."""
    _require_gpu(table, tokens)
    if table.dtype != torch.float32 or table.dim() != 2 or not table.is_contiguous():
        raise ValueError("embed_cm takes a contiguous float32 (vocab, width) table")
    tokens = tokens.reshape(-1)
    if tokens.dtype != torch.int64:
        raise ValueError("embed_cm takes int64 tokens")
    return _EmbedCM.apply(table, tokens.contiguous(), holder)
