"""Torch-CPU restatement of the reference's pure-JAX scan — TEST INFRASTRUCTURE / CPU BASELINE.

Follows ``mamba/selective_scan_cuda.py:56-90`` (``selective_scan_reference``) step by
step in the reference's logical layout: materialise ``delta*A`` as (B, L, D, N),
``a_bar = exp``, Euler or ZOH ``b_bar`` (``:74-79``), fold the initial state into the
first step (``:80-81``), run an associative scan with the compose operator
``(a_r*a_l, a_r*h_l + h_r)`` (``:83-88``), contract with C (``:89``) and return the last
state (``:90``). The associative scan restates the odd/even recursion that
``jax.lax.associative_scan`` (jax 0.10.2, a dependency absent here) uses, so the work
and memory profile match the reference's CPU path. Backward is torch autograd, the
counterpart of the reference's ``jax.vjp`` of this function (``:250-256``).

This is the reported CPU baseline of ``bench.py`` (kind "port") and an independent
formulation the sequential float64 oracle is cross-checked against in tests.
"""
from __future__ import annotations

import torch


def _interleave(even, odd, dim):
    """Interleave ``even`` (len m or m+1) and ``odd`` (len m) along ``dim``."""
    n_even, n_odd = even.shape[dim], odd.shape[dim]
    if n_even == n_odd:
        stacked = torch.stack([even, odd], dim=dim + 1)
        shape = list(even.shape)
        shape[dim] = n_even + n_odd
        return stacked.reshape(shape)
    head = _interleave(even.narrow(dim, 0, n_odd), odd, dim)
    return torch.cat([head, even.narrow(dim, n_odd, 1)], dim=dim)


def associative_scan(fn, elems, dim=1):
    """Inclusive scan of a tuple of tensors with the associative binary ``fn``."""
    n = elems[0].shape[dim]
    if n < 2:
        return elems
    sl = lambda t, start, step: t.narrow(dim, start, t.shape[dim] - start)[
        (slice(None),) * dim + (slice(None, None, step),)]
    evens = tuple(sl(t, 0, 2) for t in elems)
    odds = tuple(sl(t, 1, 2) for t in elems)
    m = odds[0].shape[dim]
    reduced = fn(tuple(e.narrow(dim, 0, m) for e in evens), odds)
    odd_scan = associative_scan(fn, reduced, dim)
    if n % 2 == 0:
        even_tail = fn(tuple(o.narrow(dim, 0, m - 1) for o in odd_scan),
                       tuple(e.narrow(dim, 1, m - 1) for e in evens))
    else:
        even_tail = fn(odd_scan, tuple(e.narrow(dim, 1, m) for e in evens))
    even_scan = tuple(torch.cat([e.narrow(dim, 0, 1), t], dim=dim) for e, t in zip(evens, even_tail))
    return tuple(_interleave(e, o, dim) for e, o in zip(even_scan, odd_scan))


def _compose(left, right):
    left_a, left_h = left
    right_a, right_h = right
    return right_a * left_a, right_a * left_h + right_h


def selective_scan_reference(A, deltas, Bs, Cs, u, initial_x=None, *, use_euler_barB_approx=True):
    """(A (D,N), deltas/u (B,L,D), Bs/Cs (B,L,N), initial_x (B,D,N)) -> (y (B,L,D), final (B,D,N))."""
    if initial_x is None:
        initial_x = torch.zeros(u.shape[0], u.shape[2], A.shape[1], dtype=u.dtype)
    delta_a = torch.einsum("bld,dn->bldn", deltas, A)
    a_bars = torch.exp(delta_a)
    if use_euler_barB_approx:
        b_bars = torch.einsum("bld,bln->bldn", deltas, Bs)
    else:
        b_bars = torch.expm1(delta_a) * torch.einsum("dn,bln->bldn", torch.reciprocal(A), Bs)
    bu = b_bars * u[..., None]
    bu = torch.cat([bu[:, :1] + a_bars[:, :1] * initial_x[:, None], bu[:, 1:]], dim=1)
    _, states = associative_scan(_compose, (a_bars, bu), dim=1)
    y = torch.einsum("bln,bldn->bld", Cs, states)
    return y, states[:, -1]
