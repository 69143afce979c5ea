"""Torch restatement of the reference's Mamba-1 model — TEST INFRASTRUCTURE ONLY.

The callers of the scan in the reference's own logical layout (B, L, features), any float
dtype (tests use float64 on the CPU), differentiable through torch autograd:

* ``S6.__call__`` — ``mamba/mamba1.py:160-198``: ``A = -exp(A_log)``; B, C and the
  low-rank delta from linear maps of the input; ``delta = softplus(dt_proj(.) + bias)``;
  scan (``oracle/assoc_torch.py``, the reference's ``selective_scan_reference``);
  ``y += D * u``. With an ``A_imag`` parameter, the complex_ssm branch (``:143-176, 198``).
* ``Mamba.__call__`` — ``mamba/mamba1.py:300-337``: norm, two up-projections, causal
  depthwise conv (``nnx.Conv(..., feature_group_count=D, padding="CAUSAL")``,
  ``:250-255``: out[t] = bias + sum_k w[k] x[t - (K-1) + k]) + silu, S6, times
  ``silu(z)``, down-projection, residual.
* Stack — ``experiments/mamba_inductionheads.py:85-120``: embedding, blocks, final
  RMSNorm (``nnx.RMSNorm(epsilon=1e-5)``), head; the head is tied to the embedding here.

Parameters come in a dict named like the product's ``MambaLM.state_dict()`` so a test can
copy one model into the other; the x_proj rows are [dt | B | C] (the reference's
``Linear_R``, ``s_B``, ``s_C``).

``seq_scan=True`` runs the real-A scan through the float64 C oracle's sequential recurrence
(``oracle/scan64c.c``, the same math; its backward is the oracle's adjoint) instead of the
associative scan, whose (B, L, D, N) intermediates do not fit at the config-5 widths.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .assoc_torch import _compose, associative_scan, selective_scan_reference


def rmsnorm(x, weight, eps=1e-5):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight


def causal_depthwise_conv(x, weight, bias):
    """x (B, L, D), weight (D, K), bias (D): out[t] = bias + sum_k w[k] x[t - (K-1) + k]."""
    k = weight.shape[1]
    xp = F.pad(x, (0, 0, k - 1, 0))
    length = x.shape[1]
    out = bias.expand_as(x).clone()
    for j in range(k):
        out = out + weight[:, j] * xp[:, j:j + length, :]
    return out


def complex_s6_scan(A, deltas, Bs, Cs, x, euler=True):
    """The complex_ssm branch of S6.__call__ (``mamba/mamba1.py:143-158, 170-176``):
    complex discretisation, associative scan of (a_bar, b_bar x) from a zero state,
    ``einsum("bln,bldn->bld", C, states)``; returns (complex y (B, L, D), last state)."""
    ctype = A.dtype
    mul = torch.einsum("bld,dn->bldn", deltas.to(ctype), A)
    a_bars = torch.exp(mul)
    if euler:
        b_bars = torch.einsum("bld,bln->bldn", deltas.to(ctype), Bs.to(ctype))
    else:
        b_bars = (torch.expm1(mul) / A[None, None]) * Bs.to(ctype)[:, :, None, :]
    bx = b_bars * x.to(ctype)[..., None]
    _, states = associative_scan(_compose, (a_bars, bx), dim=1)
    return torch.einsum("bln,bldn->bld", Cs.to(ctype), states), states[:, -1]


class _SeqScan(torch.autograd.Function):
    """y = scan(u, softplus(dt_raw + bias), A, B, C) + D u in float64 through the sequential C
    oracle; inputs in the reference's (B, L, features) layout; backward from the oracle's
    adjoint (du, d dt_raw, dA, dB, dC, dD, dbias)."""

    @staticmethod
    def forward(ctx, u, dt_raw, A, Bs, Cs, D, bias, euler):
        from . import scan64c
        sw = lambda t: t.detach().transpose(1, 2).contiguous().numpy()
        args = (sw(u), sw(dt_raw), A.detach().numpy(), sw(Bs), sw(Cs))
        kw = dict(D=D.detach().numpy(), delta_bias=bias.detach().numpy(), delta_softplus=True,
                  discretization="euler" if euler else "zoh")
        fw = scan64c.forward(*args, **kw)
        ctx.args, ctx.kw = args, kw
        return torch.from_numpy(fw["out"]).transpose(1, 2).contiguous()

    @staticmethod
    def backward(ctx, dy):
        from . import scan64c
        g = scan64c.backward(*ctx.args, dy.detach().transpose(1, 2).contiguous().numpy(), **ctx.kw)
        tb = lambda a: torch.from_numpy(a).transpose(1, 2)
        return (tb(g["du"]), tb(g["ddelta"]), torch.from_numpy(g["dA"]), tb(g["dB"]), tb(g["dC"]),
                torch.from_numpy(g["dD"]), torch.from_numpy(g["ddelta_bias"]), None)


def s6(p, prefix, u, dt_rank, d_state, euler=True, seq_scan=False):
    x_dbl = u @ p[prefix + "x_proj"].t()
    r, n = dt_rank, d_state
    if seq_scan and prefix + "A_imag" not in p:
        dt_raw = x_dbl[..., :r] @ p[prefix + "dt_proj"].t()
        return _SeqScan.apply(u, dt_raw, -torch.exp(p[prefix + "A_log"]), x_dbl[..., r:r + n],
                              x_dbl[..., r + n:], p[prefix + "D"], p[prefix + "dt_bias"], euler)
    delta = F.softplus(x_dbl[..., :r] @ p[prefix + "dt_proj"].t() + p[prefix + "dt_bias"])
    if prefix + "A_imag" in p:  # complex SSM: A = -exp(A.real) + i A.imag (:162), y.real (:198)
        A = torch.complex(-torch.exp(p[prefix + "A_log"]), p[prefix + "A_imag"])
        y, _ = complex_s6_scan(A, delta, x_dbl[..., r:r + n], x_dbl[..., r + n:], u, euler)
        return (y + p[prefix + "D"] * u).real
    A = -torch.exp(p[prefix + "A_log"])
    y, _ = selective_scan_reference(A, delta, x_dbl[..., r:r + n], x_dbl[..., r + n:], u,
                                    use_euler_barB_approx=euler)
    return y + p[prefix + "D"] * u


def mamba_block(p, prefix, h, dt_rank, d_state, euler=True, seq_scan=False):
    x = rmsnorm(h, p[prefix + "norm.weight"])
    projed = x @ p[prefix + "in_proj"].t()
    skip = F.silu(x @ p[prefix + "z_proj"].t())
    u = F.silu(causal_depthwise_conv(projed, p[prefix + "conv_weight"], p[prefix + "conv_bias"]))
    y = s6(p, prefix + "s6.", u, dt_rank, d_state, euler, seq_scan)
    return (y * skip) @ p[prefix + "out_proj"].t() + h


def mamba_lm(p, tokens, n_layers, dt_rank, d_state, euler=True, seq_scan=False):
    """tokens (B, L) -> logits (B*L, vocab) in (b, t) row order."""
    h = p["embedding"][tokens]
    for i in range(n_layers):
        h = mamba_block(p, f"blocks.{i}.", h, dt_rank, d_state, euler, seq_scan)
    hn = rmsnorm(h, p["final_norm.weight"])
    logits = hn @ p["embedding"].t()
    return logits.reshape(-1, logits.shape[-1])
