"""Float64 CPU oracle for the complex-SSM selective scan — TEST INFRASTRUCTURE ONLY.

Restates, in numpy complex128 with a sequential loop over L, the reference's complex-SSM
path of S6 (``mamba/mamba1.py:143-176``):

* ``A = -exp(A_log.real) + 1j * A_imag`` (``:162``); this oracle takes A directly as a complex
  (D, N) array, the caller applies the parameterisation;
* ``discretize`` (``:143-152``): ``a_bar = exp(delta * A)``; Euler ``b_bar = delta * B``, ZOH
  ``b_bar = expm1(delta * A) / A * B``;
* ``Bx = b_bar * x`` and ``lax.associative_scan`` with the affine operator (``:154-158, 170-174``)
  from a zero state — the same first-order recurrence ``h_t = a_bar_t h_{t-1} + Bx_t`` written
  as a loop (an optional initial state generalises it; zero reproduces the reference);
* ``ys = einsum("bln,bldn->bld", Cs, xs)``, ``ys += D * x``, ``ys.real`` (``:175-198``): C real,
  so ``y = sum_n C * Re(h) + D * u``;
* the caller's fusions as in ``scan64``: ``delta = softplus(delta_raw + bias)``
  (``:117-126, 165``), the padding mask on delta (``:167-168``), ``out = y * silu(z)``
  (``:308, 332``).

Backward (hand-derived; the reference takes it by JAX autodiff): with the complex state seen
as a real 2-vector, ``h_t = M_t h_{t-1} + bu_t`` with ``M_t`` the rotation-scaling of
``a_bar_t``, the adjoint is ``lambda_t = (C_t g_t, 0) + conj(a_bar_{t+1}) lambda_{t+1}``
(``M^T`` acts as the conjugate). With ``W_t = lambda_t conj(a_bar_t h_{t-1})``:
``dA += delta_t W_t`` and ``ddelta += Re(W_t) Re(A) + Im(W_t) Im(A)``; Euler feeds
``Re(lambda)`` into du, ddelta and dB like the real scan; ZOH adds the terms of
``E = expm1(delta A)/A`` (``dE/ddelta = a_bar``, ``dE/dA = (delta a_bar - E)/A``).
Complex gradients follow torch's convention for a real loss: ``dRe + 1j * dIm``.

Pinning (tests/test_cscan_oracle.py): torch complex128 autograd of an independent loop,
central finite differences, and the real scan (``scan64``) when ``Im(A) = 0`` (gradients and
the |term| sums); the |term| sums also by the triangle inequality and an all-positive case.
"""
from __future__ import annotations

import numpy as np

from .scan64 import SOFTPLUS_THRESHOLD, sigmoid64, softplus64


def _prep(u, delta, A, B, C, D, z, delta_bias, delta_softplus, initial_state, seq_lens):
    f = lambda a: None if a is None else np.asarray(a, np.float64)
    u, delta, B, C = f(u), f(delta), f(B), f(C)
    A = np.asarray(A, np.complex128)
    bsz, dim, L = u.shape
    n = A.shape[1]
    assert A.shape == (dim, n) and B.shape == (bsz, n, L) and C.shape == (bsz, n, L)
    bias = np.zeros(dim) if delta_bias is None else f(delta_bias)
    x = delta + bias[None, :, None]
    dl = softplus64(x) if delta_softplus else x.copy()
    lens = np.full(bsz, L) if seq_lens is None else np.clip(np.asarray(seq_lens, np.int64), 0, L)
    mask = (np.arange(L)[None, :] < lens[:, None]).astype(np.float64)
    dl = dl * mask[:, None, :]
    h0 = np.zeros((bsz, dim, n), np.complex128) if initial_state is None else np.asarray(initial_state, np.complex128).copy()
    return u, dl, x, A, B, C, f(D), f(z), h0, mask


def _disc(dl_t, u_t, A, B_t, zoh):
    w = dl_t[:, :, None] * A[None]  # (B, D, N) complex
    a_bar = np.exp(w)
    E = np.expm1(w) / A[None] if zoh else dl_t[:, :, None] * np.ones_like(w)
    s = B_t[:, None, :] * u_t[:, :, None]  # (B, D, N) real
    return a_bar, E, s, E * s


def forward(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
            initial_state=None, seq_lens=None, discretization="euler"):
    """Returns dict(out, y, last_state). Layouts as ``scan64.forward``; A, initial_state and
    last_state complex."""
    zoh = discretization == "zoh"
    u, dl, x, A, B, C, Dv, zz, h, mask = _prep(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                               initial_state, seq_lens)
    bsz, dim, L = u.shape
    y = np.empty((bsz, dim, L))
    for t in range(L):
        a_bar, _, _, bu = _disc(dl[:, :, t], u[:, :, t], A, B[:, :, t], zoh)
        h = a_bar * h + bu
        y[:, :, t] = np.einsum("bn,bdn->bd", C[:, :, t], h.real)
    if Dv is not None:
        y = y + Dv[None, :, None] * u
    out = y * (zz * sigmoid64(zz)) if zz is not None else y.copy()
    return dict(out=out * mask[:, None, :], y=y, last_state=h)


def backward(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
             initial_state=None, seq_lens=None, discretization="euler", dlast_state=None,
             abs_terms=False):
    """Gradients of sum(out * dout) + Re(sum(conj(dlast_state) * last_state)) w.r.t. every
    input: dict(du, ddelta, dA (complex), dB, dC, dD, dz, ddelta_bias, dinitial_state
    (complex)). States are stored in full (O(B*D*N*L)): small cases only.

    With ``abs_terms`` the dict also holds, for each gradient that sums over channels, batch
    rows or steps, the sum of the absolute values of the terms it adds up (``dA_abs``, with
    the real and imaginary parts summed separately, ``dB_abs``, ``dC_abs``, ``dD_abs``,
    ``ddelta_bias_abs``): the scale that bounds the rounding error of any summation order."""
    zoh = discretization == "zoh"
    fw = forward(u, delta, A, B, C, D, z, delta_bias, delta_softplus, initial_state, seq_lens,
                 discretization)
    u, dl, x, A, B, C, Dv, zz, h, mask = _prep(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                               initial_state, seq_lens)
    bsz, dim, L = u.shape
    n = A.shape[1]
    dout = np.asarray(dout, np.float64) * mask[:, None, :]
    if zz is not None:
        sz = sigmoid64(zz)
        g = dout * zz * sz
        dz = dout * fw["y"] * sz * (1.0 + zz * (1.0 - sz))
    else:
        g, dz = dout, None
    hs, disc = [h], []
    for t in range(L):
        d = _disc(dl[:, :, t], u[:, :, t], A, B[:, :, t], zoh)
        disc.append(d)
        h = d[0] * h + d[3]
        hs.append(h)
    m = np.zeros((bsz, dim, n), np.complex128) if dlast_state is None else np.asarray(dlast_state, np.complex128).copy()
    du = np.zeros((bsz, dim, L))
    ddl = np.zeros((bsz, dim, L))
    dA = np.zeros((dim, n), np.complex128)
    dB = np.zeros((bsz, n, L))
    dC = np.zeros((bsz, n, L))
    ddl_a, dA_a, dB_a, dC_a = np.zeros_like(ddl), np.zeros_like(dA), np.zeros_like(dB), np.zeros_like(dC)
    cabs = lambda c: np.abs(c.real) + 1j * np.abs(c.imag)
    Ar, Ai = A.real[None], A.imag[None]
    for t in range(L - 1, -1, -1):
        a_bar, E, s, _ = disc[t]
        h_prev, h_t = hs[t], hs[t + 1]
        lam = C[:, None, :, t] * g[:, :, t, None] + m  # (B, D, N) complex
        W = lam * np.conj(a_bar * h_prev)
        dl_t = dl[:, :, t][:, :, None]
        u_t = u[:, :, t][:, :, None]
        B_t = B[:, None, :, t]
        ta = dl_t * W
        dA += np.sum(ta, axis=0)
        tq = W.real * Ar + W.imag * Ai
        ddl[:, :, t] += np.sum(tq, axis=2)
        if abs_terms:
            dA_a += np.sum(cabs(ta), axis=0)
            ddl_a[:, :, t] += np.sum(np.abs(W.real * Ar) + np.abs(W.imag * Ai), axis=2)
        if zoh:
            ge = (np.conj(E) * lam).real  # d L / d s, s = B u
            du[:, :, t] += np.sum(B_t * ge, axis=2)
            tB = u_t * ge
            dB[:, :, t] += np.sum(tB, axis=1)
            tr = s * (np.conj(a_bar) * lam).real
            ddl[:, :, t] += np.sum(tr, axis=2)
            tb = np.conj((dl_t * a_bar - E) / A[None]) * lam * s
            dA += np.sum(tb, axis=0)
            if abs_terms:
                dB_a[:, :, t] += np.sum(np.abs(tB), axis=1)
                ddl_a[:, :, t] += np.sum(np.abs(tr), axis=2)
                dA_a += np.sum(cabs(tb), axis=0)
        else:
            lr = lam.real
            du[:, :, t] += dl_t[:, :, 0] * np.sum(lr * B_t, axis=2)
            ddl[:, :, t] += u_t[:, :, 0] * np.sum(lr * B_t, axis=2)
            tB = lr * (dl_t * u_t)
            dB[:, :, t] += np.sum(tB, axis=1)
            if abs_terms:
                ddl_a[:, :, t] += np.abs(u_t[:, :, 0]) * np.sum(np.abs(lr * B_t), axis=2)
                dB_a[:, :, t] += np.sum(np.abs(tB), axis=1)
        tC = g[:, :, t, None] * h_t.real
        dC[:, :, t] += np.sum(tC, axis=1)
        if abs_terms:
            dC_a[:, :, t] += np.sum(np.abs(tC), axis=1)
        m = np.conj(a_bar) * lam
    dD = dD_a = None
    if Dv is not None:
        du += Dv[None, :, None] * g
        dD = np.sum(g * u, axis=(0, 2))
        dD_a = np.sum(np.abs(g * u), axis=(0, 2))
    sp = np.where(x > SOFTPLUS_THRESHOLD, 1.0, sigmoid64(x)) if delta_softplus else 1.0
    dx = ddl * sp * mask[:, None, :]
    dx_a = ddl_a * sp * mask[:, None, :]
    du = du * mask[:, None, :]
    if dz is not None:
        dz = dz * mask[:, None, :]
    ddelta_bias = None if delta_bias is None else np.sum(dx, axis=(0, 2))
    res = dict(du=du, ddelta=dx, dA=dA, dB=dB, dC=dC, dD=dD, dz=dz, ddelta_bias=ddelta_bias,
               dinitial_state=m)
    if abs_terms:
        res.update(dA_abs=dA_a, dB_abs=dB_a, dC_abs=dC_a, dD_abs=dD_a,
                   ddelta_bias_abs=None if delta_bias is None else np.sum(dx_a, axis=(0, 2)))
    return res
