"""AdamW for the float32 master weights of the training step, one HIP launch per step
(mss_adamw), which also writes the bf16 shadows of the updated weights (ShadowWeights) so the
next forward does not re-read the masters to refresh them.

The reference's training leaves the optimizer to optax (experiments/mamba_inductionheads.py:
126-139); this is the optimizer of this build's config-5 step. The update is torch.optim.AdamW's
(decoupled weight decay, bias-corrected moments), in float32 per element, with the step count
kept in device memory, so a captured step (HIP graph) replays with the right count. The
hyperparameters are read at each call (a captured step keeps the values it was captured with,
as torch's AdamW with a float learning rate does).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .selective_scan_hip import _require_gpu, _stream

__all__ = ["AdamW"]


class AdamW(torch.optim.Optimizer):
    """AdamW(params, lr, betas, eps, weight_decay, shadows=None): float32, contiguous GPU
    parameters with dense gradients of the same layout. `shadows` (a ShadowWeights, e.g.
    MambaLM.shadow_weights) gets the bf16 copies of the parameters it holds written by the
    same launch; it is marked as matching its masters afterwards when it matched them before
    the step (so a forward in between does not refresh it again)."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, shadows=None):
        if not (lr >= 0.0 and 0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0 and eps > 0.0 and weight_decay >= 0.0):
            raise ValueError(f"invalid AdamW hyperparameters lr={lr} betas={betas} eps={eps} "
                             f"weight_decay={weight_decay}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))
        self.shadows = shadows
        self._tables = {}  # group index -> (pointers and shapes, mss_adamw entry array) of its last call
        self._step_bufs = {}  # group index -> (buffer of step counts, their views)

    def _init_state(self, gi, params):
        """Moments of every parameter without state, and its step count (0): the first time a
        group is seen, the counts are views of one buffer, so a step that updates every
        parameter advances them all with one add."""
        new = [p for p in params if not self.state[p]]
        if not new:
            return
        if gi not in self._step_bufs and len(new) == len(params):
            buf = torch.zeros(len(params), dtype=torch.float32, device=params[0].device)
            counts = list(buf.unbind(0))
            self._step_bufs[gi] = (buf, counts)
        else:
            counts = [torch.zeros((), dtype=torch.float32, device=p.device) for p in new]
        for p, t in zip(new, counts):
            self.state[p]["step"] = t
            self.state[p]["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            self.state[p]["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)

    @staticmethod
    def _check(p):  # (alignment and shadow layouts are checked by mss_adamw itself)
        g = p.grad
        if p.dtype != torch.float32 or not p.is_contiguous():
            raise ValueError("mamba_amd.optim.AdamW takes contiguous float32 parameters")
        if g.is_sparse or g.dtype != torch.float32 or g.shape != p.shape or not g.is_contiguous():
            raise ValueError("mamba_amd.optim.AdamW takes dense contiguous float32 gradients")

    def _entries(self, gi, params, steps):
        """(the mss_adamw entry array of `params` in host memory, rebuilt when a pointer moved;
        whether every shadow of them is written). A transposed shadow whose layout the kernel
        does not take (a column count that is not a multiple of 4, a row stride that is not a
        multiple of 8, misalignment) is left to the next refresh."""
        rows, complete = [], True
        for p, step in zip(params, steps):
            st = self.state[p]
            tgt = self.shadows.targets(p) if self.shadows is not None else None
            shadow, shadow_t, ld_t = tgt if tgt is not None else (None, None, 0)
            if shadow is not None and shadow.device != p.device:
                raise ValueError("mamba_amd.optim.AdamW: the shadows live on another device than the parameters")
            r, c = (p.shape[0], p.numel() // p.shape[0]) if p.dim() >= 2 else (1, p.numel())
            if shadow_t is not None and not (c % 4 == 0 and ld_t % 8 == 0 and shadow_t.data_ptr() % 16 == 0):
                shadow_t, ld_t, complete = None, 0, False
            rows.append((p.data_ptr(), p.grad.data_ptr(), st["exp_avg"].data_ptr(), st["exp_avg_sq"].data_ptr(),
                         step.data_ptr(), shadow.data_ptr() if shadow is not None else None,
                         shadow_t.data_ptr() if shadow_t is not None else None, r, c, ld_t, p.numel()))
        key = tuple(rows)
        cached = self._tables.get(gi)
        if cached is not None and cached[0] == key:
            return cached[1], complete
        arr = (_lib.AdamWEntry * len(rows))(*[
            _lib.AdamWEntry(param=a, grad=g, exp_avg=m, exp_avg_sq=v, step=t, shadow=sh, shadow_t=sht, rows=r, cols=c,
                            ld_t=ld, numel=n) for a, g, m, v, t, sh, sht, r, c, ld, n in rows])
        self._tables[gi] = (key, arr)
        return arr, complete

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        # The shadows stay current only if they were before and this launch writes them.
        shadows_current = (self.shadows is not None and self.shadows.bufs is not None
                           and self.shadows.flat.dtype == torch.bfloat16 and self.shadows.is_current())
        lib = _lib.register_hip_kernel()
        for gi, group in enumerate(self.param_groups):
            every = [p for p in group["params"] if p.numel() > 0]
            params = [p for p in every if p.grad is not None]
            if not params:
                continue
            _require_gpu(*params)
            for p in params:
                self._check(p)
            self._init_state(gi, every)
            # Each parameter counts its own updates (as torch's AdamW): a parameter without a
            # gradient is skipped, its count included.
            steps = [self.state[p]["step"] for p in params]
            buf = self._step_bufs.get(gi)
            if buf is not None and len(steps) == len(buf[1]) and all(a is b for a, b in zip(steps, buf[1])):
                buf[0].add_(1)
            else:
                torch._foreach_add_(steps, 1)
            arr, complete = self._entries(gi, params, steps)
            shadows_current = shadows_current and complete
            b1, b2 = group["betas"]
            args = _lib.AdamWArgs(entries=ctypes.cast(arr, ctypes.c_void_p), n_entries=len(arr), lr=group["lr"],
                                  beta1=b1, beta2=b2, eps=group["eps"], weight_decay=group["weight_decay"])
            _lib.check(lib.mss_adamw(ctypes.byref(args), _stream(params[0])), "mss_adamw")
            # The launch changed the parameters behind autograd's back: count it, so a graph
            # that saved one of them refuses a backward, as after any in-place update.
            torch.autograd.graph.increment_version(params)
        if shadows_current:
            self.shadows.mark_current()
        return loss
