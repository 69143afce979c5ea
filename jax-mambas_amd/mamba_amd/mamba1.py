"""Mamba-1 blocks on MI355X: the callers of the selective scan, channel-major end to end.

Restates the reference's ``S6`` (``mamba/mamba1.py:23-198``) and ``Mamba`` block
(``mamba/mamba1.py:216-337``) for the training path, plus the stacked language model of
the build's config 5 (embedding, N blocks, final RMSNorm, tied head).

Layout: activations are ``(features, B*L)`` matrices ("channel-major"): every projection is
one plain 2-D GEMM ``W @ X`` (hipBLASLt), and a feature row of the matrix viewed as
``(B, features, L)`` is exactly the row layout the HIP scan reads through its row strides,
so nothing is transposed around the scan. The reference works in ``(B, L, D)`` and lets XLA
transpose into its kernel's ``[B][D][L]`` layout (``mamba/selective_scan_cuda.py:135-147``).

The block's causal depthwise conv + silu is a HIP kernel too (``conv1d_hip``).
Fused into the HIP scan (one kernel per direction): ``softplus(dt_proj(x) + bias)``
(``mamba1.py:117-126, 165``), ``y += D * u`` (``:195-196``) and the ``silu(z)`` gate of the
block (``:308, 331-332``); the scan accumulates in fp32 whatever the activation dtype.

Variable length is right padding given as ``seq_lens`` (int32 per row): the scan treats
steps past a row's length as the identity and outputs 0 there (the reference multiplies
delta by a 0/1 mask, ``mamba1.py:167-168``, which leaves ``C h`` of the frozen state at
padded steps; valid steps agree).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .conv1d_hip import causal_conv1d_fn
from .lm_ops import add_rmsnorm
from .selective_scan_hip import selective_scan_fn

__all__ = ["S6", "MambaBlock", "MambaLM", "RMSNormCM"]


def _uniform_(t, bound):
    with torch.no_grad():
        return t.uniform_(-bound, bound)


def _rows(m, batch):
    """(R, B*L) matrix -> (B, R, L) view (no copy)."""
    return m.view(m.shape[0], batch, -1).permute(1, 0, 2)


def _matrix(x):
    """(B, R, L) view in row-outer layout -> (R, B*L) matrix (no copy)."""
    b, r, l = x.shape
    return x.permute(1, 0, 2).reshape(r, b * l)


class RMSNormCM(nn.Module):
    """RMSNorm over the feature axis (dim 0) of a (features, tokens) fp32 stream, fused
    with the residual add of the previous block's output (HIP kernel, lm_ops.add_rmsnorm)."""

    def __init__(self, dim, eps=1e-5, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, device=device))

    def forward(self, h, delta=None, out_dtype=torch.bfloat16):
        """Returns (h + delta, rmsnorm(h + delta) * weight in out_dtype)."""
        return add_rmsnorm(h, delta, self.weight, self.eps, out_dtype)


class S6(nn.Module):
    """Selective SSM (``mamba/mamba1.py:23-198``) over channel-major activations.

    Parameters follow the reference's initialisation: ``A_log = log(n + 1)`` (S4D-real,
    ``A = -exp(A_log)``, fp32), ``D = 1`` (fp32), input-dependent B, C and the low-rank
    delta path drawn U(+-d_inner^-0.5), the delta up-projection U(+-R^-0.5) with the
    inverse-softplus bias of a log-uniform dt in [1e-3, 1e-1] (``:79-90``). The three
    reference projections of the input (``s_B``, ``s_C``, ``Linear_R``) are one GEMM here
    (rows [dt | B | C] of ``x_proj``), as in the official Mamba.
    """

    def __init__(self, d_inner, d_state=16, dt_rank=None, use_euler_barB_approx=True,
                 use_D_param=True, device=None):
        super().__init__()
        self.d_inner, self.d_state = d_inner, d_state
        self.dt_rank = dt_rank if dt_rank is not None else max(1, (d_inner + 15) // 16)
        self.discretization = "euler" if use_euler_barB_approx else "zoh"
        n = torch.arange(1, d_state + 1, dtype=torch.float32, device=device)
        self.A_log = nn.Parameter(torch.log(n).repeat(d_inner, 1))
        self.D = nn.Parameter(torch.ones(d_inner, device=device)) if use_D_param else None
        self.x_proj = nn.Parameter(torch.empty(self.dt_rank + 2 * d_state, d_inner, device=device))
        _uniform_(self.x_proj, d_inner ** -0.5)
        self.dt_proj = nn.Parameter(torch.empty(d_inner, self.dt_rank, device=device))
        _uniform_(self.dt_proj, self.dt_rank ** -0.5)
        log_dt = torch.empty(d_inner, device=device).uniform_(math.log(1e-3), math.log(1e-1))
        dt = torch.clamp(torch.exp(log_dt), min=1e-4)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))

    def forward(self, u, batch, z=None, seq_lens=None):
        """u, z: (d_inner, B*L) matrices; returns (d_inner, B*L): (scan(u) + D u) * silu(z)."""
        r, n = self.dt_rank, self.d_state
        x_dbl = self.x_proj.to(u.dtype) @ u                     # (R + 2N, B*L)
        dt = self.dt_proj.to(u.dtype) @ x_dbl[:r]               # (d_inner, B*L), bias fused below
        A = -torch.exp(self.A_log.float())
        y = selective_scan_fn(
            _rows(u, batch), _rows(dt, batch), A, _rows(x_dbl[r:r + n], batch),
            _rows(x_dbl[r + n:], batch), D=None if self.D is None else self.D.float(),
            z=None if z is None else _rows(z, batch), delta_bias=self.dt_bias.float(),
            delta_softplus=True, seq_lens=seq_lens, discretization=self.discretization)
        return _matrix(y)


class MambaBlock(nn.Module):
    """Mamba-1 block (``mamba/mamba1.py:216-337``): norm -> in-projections -> causal conv
    + silu -> S6 with D skip -> * silu(z) -> out-projection -> + residual."""

    def __init__(self, d_model, expand=2, d_state=16, dt_rank=None, d_conv=4, n_layers=1,
                 norm="rmsnorm", use_euler_barB_approx=True, device=None):
        super().__init__()
        d_inner = d_model * expand
        dt_rank = dt_rank if dt_rank is not None else max(1, (d_model + 15) // 16)  # from d_model
        if norm != "rmsnorm":
            raise ValueError("only rmsnorm is implemented for the channel-major block")
        self.norm = RMSNormCM(d_model, device=device)
        self.in_proj = nn.Parameter(_uniform_(torch.empty(d_inner, d_model, device=device), d_model ** -0.5))
        self.z_proj = nn.Parameter(_uniform_(torch.empty(d_inner, d_model, device=device), d_model ** -0.5))
        self.conv_weight = nn.Parameter(_uniform_(torch.empty(d_inner, d_conv, device=device), d_conv ** -0.5))
        self.conv_bias = nn.Parameter(_uniform_(torch.empty(d_inner, device=device), d_conv ** -0.5))
        self.s6 = S6(d_inner, d_state, dt_rank, use_euler_barB_approx=use_euler_barB_approx, device=device)
        self.out_proj = nn.Parameter(_uniform_(torch.empty(d_model, d_inner, device=device),
                                               d_inner ** -0.5 * n_layers ** -0.5))

    def forward(self, h, delta, batch, seq_lens=None, act_dtype=torch.bfloat16):
        """h: (d_model, B*L) fp32 residual stream before the previous block's output `delta`
        (act_dtype, or None for the first block) is added. Returns (h + delta, this block's
        output): the residual add is fused into the next norm."""
        h, x = self.norm(h, delta, act_dtype)
        xin = self.in_proj.to(act_dtype) @ x
        z = self.z_proj.to(act_dtype) @ x
        # causal depthwise conv + silu (HIP kernel), masked past each row's length
        u = _matrix(causal_conv1d_fn(_rows(xin, batch), self.conv_weight, self.conv_bias, seq_lens))
        y = self.s6(u, batch, z=z, seq_lens=seq_lens)
        return h, self.out_proj.to(act_dtype) @ y


class MambaLM(nn.Module):
    """Stacked Mamba-1 language model: embedding -> blocks -> RMSNorm -> tied head."""

    def __init__(self, vocab, d_model, n_layers, expand=2, d_state=16, dt_rank=None, d_conv=4,
                 use_euler_barB_approx=True, device=None):
        super().__init__()
        self.embedding = nn.Parameter(torch.randn(vocab, d_model, device=device) * 0.02)
        self.blocks = nn.ModuleList(
            MambaBlock(d_model, expand, d_state, dt_rank, d_conv, n_layers,
                       use_euler_barB_approx=use_euler_barB_approx, device=device)
            for _ in range(n_layers))
        self.final_norm = RMSNormCM(d_model, device=device)

    def forward(self, tokens, seq_lens=None, act_dtype=torch.bfloat16):
        """tokens (B, L) int64 -> logits (B*L, vocab) in act_dtype (rows in (b, t) order)."""
        batch = tokens.shape[0]
        h = self.embedding[tokens.reshape(-1)].t().contiguous()   # (d_model, B*L) fp32
        delta = None
        for blk in self.blocks:
            h, delta = blk(h, delta, batch, seq_lens, act_dtype)
        _, hn = self.final_norm(h, delta, act_dtype)
        return hn.t() @ self.embedding.to(act_dtype).t()
