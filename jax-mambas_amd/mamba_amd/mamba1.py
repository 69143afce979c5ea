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

from . import _lib
from .decode import (causal_conv1d_update, gemv, gemv_conv_update, gemv_state_update, norm_gemv_conv_update,
                     selective_state_update)
from .lm_ops import GradHolder, add_rmsnorm, embed_cm
from .proj import proj, proj_fits, wgrad, wgrad_fits
from .selective_scan_hip import _io_tag, _ptr, _stream, selective_scan_fn

__all__ = ["S6", "MambaBlock", "MambaLM", "RMSNormCM", "ShadowWeights", "GraphedTrainStep"]


_MM_FP32_OUT = None  # whether torch.mm(bf16, bf16, out_dtype=float32) runs on this device


def _mm_fp32(a, b):
    """a @ b with float32 output (accumulation is float32 either way)."""
    global _MM_FP32_OUT
    if _MM_FP32_OUT is None:
        try:
            torch.mm(a[:1, :1], b[:1, :1], out_dtype=torch.float32)
            _MM_FP32_OUT = True
        except (RuntimeError, NotImplementedError, TypeError):
            _MM_FP32_OUT = False
    if _MM_FP32_OUT:
        return torch.mm(a, b, out_dtype=torch.float32)
    return torch.mm(a, b).float()


def _wgrad_mm(dy, x):
    """dy @ x^T in float32 for activations dy (M, T), x (N, T): the split-token matrix-core
    kernel where the shape fits, else the library GEMM."""
    if wgrad_fits(dy, x):
        return wgrad(dy, x)
    return _mm_fp32(dy, x.t())


def _proj_mm(w, x, out=None, accumulate=False):
    """w @ x (+ out when accumulate) for the S6 input projections (w may be a transposed view
    of a stored weight): the skinny-GEMM kernels where the shape and layout fit, else the
    library GEMM."""
    if proj_fits(w, x, out):
        return proj(w, x, out=out, accumulate=accumulate)
    if out is None:
        return torch.mm(w, x)
    if accumulate:
        return out.addmm_(w, x)
    return torch.mm(w, x, out=out)


class _WeightMM(torch.autograd.Function):
    """y = W_act @ x with a low-precision shadow W_act of the float32 master weight W:
    dx = W_act^T dy (from the contiguous transposed shadow W_act_t when given); dW = dy x^T,
    produced in float32 for the master weight."""

    @staticmethod
    def forward(ctx, x, w, w_act, w_act_t=None):
        ctx.save_for_backward(x, w_act, w_act_t)
        return w_act @ x

    @staticmethod
    def backward(ctx, dy):
        x, w_act, w_act_t = ctx.saved_tensors
        dx = None
        if ctx.needs_input_grad[0]:
            dx = w_act_t @ dy if w_act_t is not None else w_act.t() @ dy
        dw = _wgrad_mm(dy, x) if ctx.needs_input_grad[1] else None
        return dx, dw, None, None


class _TiedHeadMM(torch.autograd.Function):
    """logits = x^T E_act^T for x (features, tokens) and the tied embedding E (vocab,
    features); dE in float32 for the master embedding, handed to the embedding gather's
    backward through `holder` when given (one gradient edge for the shared table)."""

    @staticmethod
    def forward(ctx, x, e, e_act, holder=None):
        ctx.save_for_backward(x, e_act)
        ctx.holder = holder
        # From a token-major copy of x: hipBLASLt's product with both operands K-contiguous
        # took 1.128 ms against 1.420 from the features-major view at the 130M shape (16384
        # tokens, 768 features, 50280 words; MI355X), and the copy 0.054 ms.
        return x.t().contiguous() @ e_act.t()

    @staticmethod
    def backward(ctx, dy):
        x, e_act = ctx.saved_tensors
        dx = e_act.t() @ dy.t() if ctx.needs_input_grad[0] else None
        de = _mm_fp32(dy.t(), x.t()) if ctx.needs_input_grad[1] else None
        if de is not None and ctx.holder is not None:
            ctx.holder.put(de)  # the embedding's backward adds its part and returns the sum
            de = None
        return dx, de, None, None


class ShadowWeights:
    """Low-precision copies of float32 weights, refreshed together once per step (instead of
    one cast per weight per use, plus one per gradient). The copies are views of one buffer
    in the order given (offsets padded to 64 elements), so consecutive weights with the same
    column count can be used as one stacked matrix. `transposed` lists groups of such
    consecutive weights whose stacked matrix is also kept transposed and contiguous (the
    operand layout the input-gradient GEMMs W^T dY run fastest on). In bf16 on the GPU the
    refresh is one HIP launch over a device table (mss_shadow_refresh) writing both copies."""

    def __init__(self, params, transposed=()):
        self.params = list(params)
        self.groups = [tuple(g) for g in transposed]
        self.bufs = None
        self.flat = None
        self.tflat = None
        self.offsets = {}
        self.by_id = {}
        self.t_by_key = {}
        self._table = None   # (device entry table, n_entries, n_tiles, master pointers)
        self._current = None  # the masters' (pointer, version) when the copies last matched them

    def _layout(self, dtype):
        offs, off = [], 0
        for p in self.params:
            offs.append(off)
            off += (p.numel() + 63) // 64 * 64
        dev = self.params[0].device
        self.flat = torch.empty(off, dtype=dtype, device=dev)
        self.bufs = [self.flat[o:o + p.numel()].view(p.shape) for o, p in zip(offs, self.params)]
        self.by_id = {id(p): b for p, b in zip(self.params, self.bufs)}
        self.offsets = {id(p): o for p, o in zip(self.params, offs)}
        toff, self._tslot = 0, {}   # id(w) -> (offset of its group, column offset, group rows)
        gspec = []
        for g in self.groups:
            cols, rows = g[0].shape[1], sum(w.shape[0] for w in g)
            gspec.append((toff, cols, rows))
            c = 0
            for w in g:
                self._tslot[id(w)] = (toff, c, rows)
                c += w.shape[0]
            toff += (cols * rows + 63) // 64 * 64
        self.tflat = torch.empty(max(toff, 1), dtype=dtype, device=dev)
        self.t_by_key = {tuple(id(w) for w in g): self.tflat[o:o + c * r].view(c, r)
                         for g, (o, c, r) in zip(self.groups, gspec)}
        self._table = None

    def _native_table(self):
        """The device table of mss_shadow_refresh, rebuilt when a master moved."""
        ptrs = tuple(p.data_ptr() for p in self.params)
        if self._table is not None and self._table[3] == ptrs:
            return self._table
        entries, tile0 = [], 0
        esz = self.flat.element_size()
        for p, b in zip(self.params, self.bufs):
            rows, cols = (p.shape[0], p.shape[1]) if p.dim() == 2 else (1, p.numel())
            dst_t, ld_t = None, 0
            if id(p) in self._tslot:
                o, c, r = self._tslot[id(p)]
                dst_t, ld_t = self.tflat.data_ptr() + (o + c) * esz, r
            entries.append(_lib.ShadowEntry(src=p.data_ptr(), dst=b.data_ptr(), dst_t=dst_t, rows=rows, cols=cols,
                                            ld_t=ld_t, tile0=tile0))
            tile0 += ((rows + 63) // 64) * ((cols + 63) // 64)
        raw = (_lib.ShadowEntry * len(entries))(*entries)
        table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.flat.device)
        self._table = (table, len(entries), tile0, ptrs)
        return self._table

    def _token(self):
        return tuple((p.data_ptr(), p._version) for p in self.params)

    def is_current(self):
        """Whether the copies match the masters: nothing replaced or changed a master in place
        (autograd's version counters) since they were last written."""
        return self._current is not None and self._current == self._token()

    def mark_current(self):
        """Records that the copies match the masters as they are now (called by whatever wrote
        both, e.g. mamba_amd.optim.AdamW after its update)."""
        self._current = self._token()

    def targets(self, p):
        """(shadow, transposed shadow or None, ld_t) of master p in the bf16 layout, else None."""
        if self.bufs is None or self.flat.dtype != torch.bfloat16 or id(p) not in self.by_id:
            return None
        dst_t, ld_t = None, 0
        if id(p) in self._tslot:
            o, c, r = self._tslot[id(p)]
            dst_t, ld_t = self.tflat[o + c:], r
        return self.by_id[id(p)], dst_t, ld_t

    def refresh(self, dtype):
        """Writes the copies from the masters, unless they already match them."""
        if self.bufs is None or self.flat.dtype != dtype:
            self._layout(dtype)
            self._current = None
        if self.is_current():
            return
        native = (dtype == torch.bfloat16 and self.flat.is_cuda
                  and all(p.dtype == torch.float32 and p.is_contiguous() for p in self.params))
        with torch.no_grad():
            if native:
                table, n, tiles, _ = self._native_table()
                lib = _lib.register_hip_kernel()
                _lib.check(lib.mss_shadow_refresh(table.data_ptr(), n, tiles, _stream(self.flat)),
                           "mss_shadow_refresh")
            else:
                torch._foreach_copy_(self.bufs, [p.detach() for p in self.params])
                for g in self.groups:
                    self.t_by_key[tuple(id(w) for w in g)].copy_(torch.cat([w.detach() for w in g]).t())
        self.mark_current()

    def stacked_t(self, *ws):
        """The contiguous transpose of the stacked shadows of ws, when kept, else None."""
        return self.t_by_key.get(tuple(id(w) for w in ws)) if self.t_by_key else None

    def stacked(self, *ws):
        """The shadows of ws as one (sum of rows, cols) matrix when they lie back to back,
        else None."""
        if not self.by_id or any(id(w) not in self.by_id for w in ws):
            return None
        o, rows = self.offsets[id(ws[0])], 0
        for w in ws:
            if self.offsets[id(w)] != o + rows * w.shape[1] or w.shape[1] != ws[0].shape[1]:
                return None
            rows += w.shape[0]
        return self.flat[o:o + rows * ws[0].shape[1]].view(rows, ws[0].shape[1])

    def shadow(self, w):
        """The low-precision copy of w, or None."""
        return self.by_id.get(id(w))

    def act(self, w, dtype):
        """The weight in the activation dtype: its shadow, or a cast of the master."""
        b = self.by_id.get(id(w))
        return b if b is not None and b.dtype == dtype else w.to(dtype)

    def mv(self, w, x):
        """w @ x for a decode step (no autograd): the decode-shaped HIP GEMM on the shadow of
        w when x is a few bf16 token columns, else mm."""
        b = self.by_id.get(id(w))
        if b is not None and b.dtype == x.dtype and not torch.is_grad_enabled():
            return gemv(b, x)
        return self.mm(w, x)

    def mm(self, w, x):
        """w @ x: plain autograd in float32, else through the shadow of w (and its transposed
        shadow for the input gradient, when kept)."""
        if x.dtype == torch.float32 or not self.by_id:
            return w.to(x.dtype) @ x
        return _WeightMM.apply(x, w, self.by_id[id(w)], self.stacked_t(w))

    def head(self, x, e, holder=None):
        if x.dtype == torch.float32 or not self.by_id:
            return x.t() @ e.to(x.dtype).t()
        return _TiedHeadMM.apply(x, e, self.by_id[id(e)], holder)


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

    ``complex_ssm=True`` is the reference's complex-state variant (``:38, 47, 162, 170-176,
    198``): ``A = -exp(A_log) + i*A_imag`` with ``A_log + i*A_imag = log(1/2 - i*n)``
    (n = 0..N-1), complex states, real output ``sum_n C Re(h) + D u``; the complex scan
    kernels run it.
    """

    def __init__(self, d_inner, d_state=16, dt_rank=None, use_euler_barB_approx=True,
                 use_D_param=True, complex_ssm=False, device=None):
        super().__init__()
        self.d_inner, self.d_state = d_inner, d_state
        self.dt_rank = dt_rank if dt_rank is not None else max(1, (d_inner + 15) // 16)
        self.discretization = "euler" if use_euler_barB_approx else "zoh"
        self.complex_ssm = complex_ssm
        if complex_ssm:
            n = torch.arange(d_state, dtype=torch.float64, device=device)
            a0 = torch.log(torch.complex(torch.full_like(n, 0.5), -n))
            self.A_log = nn.Parameter(a0.real.float().repeat(d_inner, 1))
            self.A_imag = nn.Parameter(a0.imag.float().repeat(d_inner, 1))
        else:
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

    def a_matrix(self):
        """The state matrix: -exp(A_log) (float32), or complex64 -exp(A_log) + i*A_imag."""
        a = -torch.exp(self.A_log.float())
        return torch.complex(a, self.A_imag.float()) if self.complex_ssm else a

    def forward(self, u, batch, z=None, seq_lens=None, weights=None):
        """u, z: (d_inner, B*L) matrices; returns (d_inner, B*L): (scan(u) + D u) * silu(z).
        `weights` (ShadowWeights) supplies low-precision copies of the projections."""
        r, n = self.dt_rank, self.d_state
        weights = weights or _PLAIN
        x_dbl = weights.mm(self.x_proj, u)                      # (R + 2N, B*L)
        dt = weights.mm(self.dt_proj, x_dbl[:r])                # (d_inner, B*L), bias fused below
        A = self.a_matrix()
        y, last = selective_scan_fn(
            _rows(u, batch), _rows(dt, batch), A, _rows(x_dbl[r:r + n], batch),
            _rows(x_dbl[r + n:], batch), D=None if self.D is None else self.D.float(),
            z=None if z is None else _rows(z, batch), delta_bias=self.dt_bias.float(),
            delta_softplus=True, return_last_state=True, seq_lens=seq_lens,
            discretization=self.discretization)
        self.last_state = last if not torch.is_grad_enabled() else None
        return _matrix(y)

    def step(self, u, z, state, weights=None, A=None):
        """One token: u, z (d_inner, B) matrices; state (B, d_inner, N) updated in place.
        A: the state matrix computed once per generation (recomputed when None)."""
        r, n = self.dt_rank, self.d_state
        weights = weights or _PLAIN
        x_dbl = weights.mv(self.x_proj, u)
        A = self.a_matrix() if A is None else A
        args = (A, x_dbl[r:r + n].t(), x_dbl[r + n:].t())
        kw = dict(D=None if self.D is None else self.D.float(), z=None if z is None else z.t(),
                  delta_bias=self.dt_bias.float(), delta_softplus=True, discretization=self.discretization)
        w_dt = weights.shadow(self.dt_proj)
        if w_dt is not None and w_dt.dtype == u.dtype and not torch.is_grad_enabled():
            y = gemv_state_update(w_dt, x_dbl[:r], state, u.t(), *args, **kw)  # dt GEMM + state step
        else:
            dt = weights.mv(self.dt_proj, x_dbl[:r])
            y = selective_state_update(state, u.t(), dt.t(), *args, **kw)
        return y.t()


_PLAIN = ShadowWeights([])  # no shadows: weights cast per use


def _rows_strides(batch, tokens):
    """mss_strides of (R, B*L) matrices read as (B, R, L) rows: b -> L, r -> B*L."""
    l = tokens // batch
    return _lib.Strides(io_batch=l, io_dim=tokens, bc_batch=l, bc_state=tokens)


class _MambaMixer(torch.autograd.Function):
    """The block between its norm and its out-projection, as one autograd node over the HIP
    kernels (``mamba/mamba1.py:300-332`` with S6 ``:160-198``): [xin; z] = [W_in; W_z] x (one
    GEMM when the two weights lie back to back), u = silu(conv(xin)), x_dbl = W_x u,
    dt = W_dt x_dbl[:R], y = scan(u, dt, A, B = x_dbl[R:R+N], C = x_dbl[R+N:], D, z, dt_bias)
    gated by silu(z). All activations are (features, B*L) matrices; the scan and conv read
    their rows in place through row strides. The backward writes the scan's dB/dC straight
    into the x_dbl gradient, the scan's dz and the conv's dxin into one [dxin; dz] buffer,
    adds W_x^T dx_dbl to du in place, and takes dx and d[W_in; W_z] as one GEMM each:
    no gradient sums or copies between the kernels. Weight gradients are float32."""

    @staticmethod
    def forward(ctx, x, w_in, w_z, conv_w, conv_b, w_x, w_dt, A, D, dt_bias, w_xz_act, w_x_act, w_dt_act,
                batch, seq_lens, zoh, w_xz_t=None):
        lib = _lib.register_hip_kernel()
        di, T = w_in.shape[0], x.shape[1]
        r = w_dt.shape[1]
        n = (w_x.shape[0] - r) // 2
        L = T // batch
        dev, act = x.device, x.dtype
        cplx = A.is_complex()
        io = _io_tag(act, "x")
        st = _rows_strides(batch, T)
        stream = _stream(x)
        xz = torch.mm(w_xz_act, x)                       # (2 di, T): [xin; z]
        xin, z = xz[:di], xz[di:]
        u = torch.empty(di, T, dtype=act, device=dev)
        ca = _lib.ConvArgs(batch=batch, dim=di, seqlen=L, width=conv_w.shape[1], io_dtype=io, activation=1,
                           x=xin.data_ptr(), weight=conv_w.data_ptr(), bias=_ptr(conv_b),
                           seq_lens=_ptr(seq_lens), y=u.data_ptr(), strides=st)
        _lib.check(lib.mss_conv_fwd(ca, stream), "mss_conv_fwd")
        x_dbl = _proj_mm(w_x_act, u)                     # (R + 2N, T)
        dt = _proj_mm(w_dt_act, x_dbl[:r])               # (di, T), bias fused in the scan
        n_seg = (L + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
        sdt = torch.complex64 if cplx else torch.float32
        rv = (lambda t: torch.view_as_real(t).data_ptr()) if cplx else (lambda t: t.data_ptr())
        y = torch.empty(di, T, dtype=act, device=dev)
        y_pre = torch.empty(di, T, dtype=act, device=dev)
        last = torch.empty(batch, di, n, dtype=sdt, device=dev)
        carries = torch.empty(batch, di, n, n_seg, dtype=sdt, device=dev)
        fa = _lib.FwdArgs(batch=batch, dim=di, seqlen=L, dstate=n,
                          discretization=_lib.MSS_ZOH if zoh else _lib.MSS_EULER, delta_softplus=1,
                          io_dtype=io, bc_dtype=io, u=u.data_ptr(), delta=dt.data_ptr(), A=rv(A),
                          B=x_dbl[r].data_ptr(), C=x_dbl[r + n].data_ptr(), D=_ptr(D), z=z.data_ptr(),
                          delta_bias=dt_bias.data_ptr(), seq_lens=_ptr(seq_lens), out=y.data_ptr(),
                          last_state=rv(last), carries=rv(carries), y_pre=y_pre.data_ptr(), strides=st)
        _lib.check((lib.mss_cfwd if cplx else lib.mss_fwd)(fa, stream), "scan forward")
        ctx.save_for_backward(x, xz, u, x_dbl, dt, carries, y_pre, A, D, dt_bias, conv_w, conv_b,
                              w_xz_act, w_x_act, w_dt_act, seq_lens, w_xz_t, y)
        ctx.batch, ctx.zoh, ctx.dims = batch, zoh, (di, r, n, L)
        ctx.mark_non_differentiable(last, xz)
        ctx.set_materialize_grads(False)  # no zero-filled gradients for last / xz
        return y, last, xz

    @staticmethod
    def backward(ctx, dy, _dlast, _dxz):
        lib = _lib.register_hip_kernel()
        (x, xz, u, x_dbl, dt, carries, y_pre, A, D, dt_bias, conv_w, conv_b, w_xz_act, w_x_act, w_dt_act,
         seq_lens, w_xz_t, y) = ctx.saved_tensors
        di, r, n, L = ctx.dims
        batch = ctx.batch
        T = x.shape[1]
        dev, act = x.device, x.dtype
        cplx = A.is_complex()
        io = _io_tag(act, "x")
        st = _rows_strides(batch, T)
        stream = _stream(x)
        rv = (lambda t: torch.view_as_real(t).data_ptr()) if cplx else (lambda t: t.data_ptr())
        dy = torch.zeros(di, T, dtype=act, device=dev) if dy is None else dy.to(act).contiguous()
        dxz = torch.empty(2 * di, T, dtype=act, device=dev)   # [dxin; dz]
        dx_dbl = torch.empty(r + 2 * n, T, dtype=act, device=dev)
        du = torch.empty(di, T, dtype=act, device=dev)
        ddt = torch.empty(di, T, dtype=act, device=dev)
        dA = torch.empty_like(A)
        dD = None if D is None else torch.empty_like(D)
        dbias = torch.empty_like(dt_bias)
        ba = _lib.BwdArgs(batch=batch, dim=di, seqlen=L, dstate=n,
                          discretization=_lib.MSS_ZOH if ctx.zoh else _lib.MSS_EULER, delta_softplus=1,
                          io_dtype=io, bc_dtype=io, u=u.data_ptr(), delta=dt.data_ptr(), A=rv(A),
                          B=x_dbl[r].data_ptr(), C=x_dbl[r + n].data_ptr(), D=_ptr(D), z=xz[di].data_ptr(),
                          delta_bias=dt_bias.data_ptr(), seq_lens=_ptr(seq_lens), carries=rv(carries),
                          y_pre=y_pre.data_ptr(), out=y.data_ptr(), dout=dy.data_ptr(), du=du.data_ptr(),
                          ddelta=ddt.data_ptr(),
                          dA=rv(dA), dB=dx_dbl[r].data_ptr(), dC=dx_dbl[r + n].data_ptr(), dD=_ptr(dD),
                          dz=dxz[di].data_ptr(), ddelta_bias=dbias.data_ptr(), strides=st)
        ws_bytes = int((lib.mss_cbwd_workspace_bytes if cplx else lib.mss_bwd_workspace_bytes)(ba))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ba.workspace, ba.workspace_bytes = ws.data_ptr(), ws_bytes
        _lib.check((lib.mss_cbwd if cplx else lib.mss_bwd)(ba, stream), "scan backward")
        dw_dt = _wgrad_mm(ddt, x_dbl[:r])
        _proj_mm(w_dt_act.t(), ddt, out=dx_dbl[:r])
        dw_x = _wgrad_mm(dx_dbl, u)
        _proj_mm(w_x_act.t(), dx_dbl, out=du, accumulate=True)  # du += W_x^T dx_dbl
        dconv_w = torch.empty_like(conv_w)
        dconv_b = None if conv_b is None else torch.empty_like(conv_b)
        ca = _lib.ConvArgs(batch=batch, dim=di, seqlen=L, width=conv_w.shape[1], io_dtype=io, activation=1,
                           x=xz.data_ptr(), weight=conv_w.data_ptr(), bias=_ptr(conv_b),
                           seq_lens=_ptr(seq_lens), dy=du.data_ptr(), dx=dxz.data_ptr(),
                           dweight=dconv_w.data_ptr(), dbias=_ptr(dconv_b), strides=st)
        cws_bytes = int(lib.mss_conv_bwd_workspace_bytes(ca))
        cws = torch.empty(cws_bytes, dtype=torch.uint8, device=dev)
        ca.workspace, ca.workspace_bytes = cws.data_ptr(), cws_bytes
        _lib.check(lib.mss_conv_bwd(ca, stream), "mss_conv_bwd")
        dw_xz = _wgrad_mm(dxz, x)
        dx = torch.mm(w_xz_t if w_xz_t is not None else w_xz_act.t(), dxz)
        return (dx, dw_xz[:di], dw_xz[di:], dconv_w, dconv_b, dw_x, dw_dt, dA, dD, dbias,
                None, None, None, None, None, None, None)


class MambaBlock(nn.Module):
    """Mamba-1 block (``mamba/mamba1.py:216-337``): norm -> in-projections -> causal conv
    + silu -> S6 with D skip -> * silu(z) -> out-projection -> + residual."""

    def __init__(self, d_model, expand=2, d_state=16, dt_rank=None, d_conv=4, n_layers=1,
                 norm="rmsnorm", use_euler_barB_approx=True, complex_ssm=False, device=None):
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
        self.s6 = S6(d_inner, d_state, dt_rank, use_euler_barB_approx=use_euler_barB_approx,
                     complex_ssm=complex_ssm, device=device)
        self.out_proj = nn.Parameter(_uniform_(torch.empty(d_model, d_inner, device=device),
                                               d_inner ** -0.5 * n_layers ** -0.5))

    def gemm_weights(self):
        return [self.in_proj, self.z_proj, self.out_proj, self.s6.x_proj, self.s6.dt_proj]

    def forward(self, h, delta, batch, seq_lens=None, act_dtype=torch.bfloat16, weights=None, A=None):
        """h: (d_model, B*L) fp32 residual stream before the previous block's output `delta`
        (act_dtype, or None for the first block) is added. Returns (h + delta, this block's
        output): the residual add is fused into the next norm. The mixer between the norm and
        the out-projection is one autograd node (_MambaMixer). A: the S6 state matrix when the
        caller computed it (MambaLM does so for all blocks at once), else computed here."""
        weights = weights or _PLAIN
        h, x = self.norm(h, delta, act_dtype)
        s6 = self.s6
        w_xz = weights.stacked(self.in_proj, self.z_proj)
        w_xz_t = None
        if w_xz is None or w_xz.dtype != act_dtype:
            w_xz = torch.cat([self.in_proj.detach(), self.z_proj.detach()]).to(act_dtype)
        else:
            w_xz_t = weights.stacked_t(self.in_proj, self.z_proj)
        A = s6.a_matrix() if A is None else A
        y, last, xz = _MambaMixer.apply(
            x, self.in_proj, self.z_proj, self.conv_weight, self.conv_bias, s6.x_proj, s6.dt_proj, A,
            None if s6.D is None else s6.D.float(), s6.dt_bias.float(), w_xz,
            weights.act(s6.x_proj, act_dtype), weights.act(s6.dt_proj, act_dtype), batch, seq_lens,
            s6.discretization == "zoh", w_xz_t)
        if not torch.is_grad_enabled():  # inference: keep the decode caches of this prompt
            xin = xz[:self.in_proj.shape[0]]
            k = self.conv_weight.shape[1]
            tail = _rows(xin, batch)[:, :, max(0, xin.shape[1] // batch - (k - 1)):]
            conv = torch.zeros(batch, xin.shape[0], k - 1, dtype=xin.dtype, device=xin.device)
            if k > 1:
                conv[:, :, conv.shape[2] - tail.shape[2]:] = tail
            self.cache = {"conv": conv, "ssm": last, "A": A.detach()}
        return h, weights.mm(self.out_proj, y)

    def step(self, h, delta, cache, act_dtype=torch.bfloat16, weights=None):
        """One token per row: h (d_model, B) stream; cache {"conv": (B, d_inner, K-1),
        "ssm": (B, d_inner, N)} updated in place (Mamba.step, mamba/mamba1.py:339-363)."""
        weights = weights or _PLAIN
        w_xz = weights.stacked(self.in_proj, self.z_proj)
        if w_xz is not None and w_xz.dtype == act_dtype == torch.bfloat16:
            # residual add + norm, then [xin; z] in one GEMM with the conv window step fused
            # on the xin rows: one kernel
            h, u, z = norm_gemv_conv_update(h, delta, self.norm.weight, self.norm.eps, w_xz, cache["conv"],
                                            self.conv_weight, self.conv_bias)
        else:
            h, x = self.norm(h, delta, act_dtype)
            xin = weights.mm(self.in_proj, x)
            z = weights.mm(self.z_proj, x)
            u = causal_conv1d_update(cache["conv"], xin.t(), self.conv_weight, self.conv_bias).t()
        y = self.s6.step(u, z, cache["ssm"], weights, cache.get("A"))
        return h, weights.mv(self.out_proj, y)


class MambaLM(nn.Module):
    """Stacked Mamba-1 language model: embedding -> blocks -> RMSNorm -> tied head."""

    def __init__(self, vocab, d_model, n_layers, expand=2, d_state=16, dt_rank=None, d_conv=4,
                 use_euler_barB_approx=True, complex_ssm=False, device=None):
        super().__init__()
        self.embedding = nn.Parameter(torch.randn(vocab, d_model, device=device) * 0.02)
        self.blocks = nn.ModuleList(
            MambaBlock(d_model, expand, d_state, dt_rank, d_conv, n_layers,
                       use_euler_barB_approx=use_euler_barB_approx, complex_ssm=complex_ssm,
                       device=device)
            for _ in range(n_layers))
        self.final_norm = RMSNormCM(d_model, device=device)
        self._shadows = ShadowWeights([self.embedding] + [w for b in self.blocks for w in b.gemm_weights()],
                                      transposed=[g for b in self.blocks for g in ((b.in_proj, b.z_proj), (b.out_proj,))])

    @property
    def shadow_weights(self):
        """The bf16 copies of the GEMM weights (ShadowWeights), e.g. for mamba_amd.optim.AdamW
        to write with its update."""
        return self._shadows

    def forward(self, tokens, seq_lens=None, act_dtype=torch.bfloat16, shadow_weights=True):
        """tokens (B, L) int64 -> logits (B*L, vocab) in act_dtype (rows in (b, t) order).
        Low-precision GEMM weights are refreshed from the float32 masters once per call unless
        they already match them (shadow_weights=False casts each weight at its use instead)."""
        batch = tokens.shape[0]
        weights = _PLAIN
        if act_dtype != torch.float32 and shadow_weights:
            self._shadows.refresh(act_dtype)
            weights = self._shadows
        holder = None
        d_model = self.embedding.shape[1]
        if tokens.is_cuda and d_model % 4 == 0 and d_model <= 1024:
            holder = GradHolder()
            h = embed_cm(self.embedding, tokens, holder)             # (d_model, B*L) fp32
        else:
            h = self.embedding[tokens.reshape(-1)].t().contiguous()
        delta = None
        for blk, A in zip(self.blocks, self.a_matrices()):
            h, delta = blk(h, delta, batch, seq_lens, act_dtype, weights, A)
        _, hn = self.final_norm(h, delta, act_dtype)
        return weights.head(hn, self.embedding, holder)

    def a_matrices(self):
        """Every block's S6 state matrix. Real A = -exp(A_log) of all blocks in one batched op
        (a few launches per step each way instead of two per block and direction)."""
        s6s = [blk.s6 for blk in self.blocks]
        if any(s.complex_ssm for s in s6s) or len({tuple(s.A_log.shape) for s in s6s}) != 1:
            return [s.a_matrix() for s in s6s]
        return torch.stack([s.A_log for s in s6s]).float().exp().neg().unbind(0)

    @torch.no_grad()
    def prefill(self, tokens, act_dtype=torch.bfloat16):
        """Runs a prompt (B, L) without gradients; returns (logits of its last position
        (B, vocab), per-block decode caches). Right-aligned prompts only (no seq_lens)."""
        logits = self.forward(tokens, act_dtype=act_dtype)
        caches = []
        for blk in self.blocks:
            caches.append(blk.cache)
            blk.cache = None
            blk.s6.last_state = None
        b, l = tokens.shape
        return logits.view(b, l, -1)[:, -1], caches

    @torch.no_grad()
    def step(self, token, caches, act_dtype=torch.bfloat16):
        """One decode step: token (B,) int64 -> logits (B, vocab); caches update in place.
        Uses the low-precision weights of the last prefill (weights do not change while
        generating)."""
        weights = _PLAIN
        if act_dtype != torch.float32:
            if not self._shadows.by_id or self._shadows.bufs[0].dtype != act_dtype:
                self._shadows.refresh(act_dtype)
            weights = self._shadows
        h = self.embedding[token].t().contiguous()  # (d_model, B)
        delta = None
        for blk, cache in zip(self.blocks, caches):
            h, delta = blk.step(h, delta, cache, act_dtype, weights)
        _, hn = self.final_norm(h, delta, act_dtype)
        return weights.mv(self.embedding, hn).t()  # (B, vocab) logits of the tied head


class GraphedTrainStep:
    """One training step (forward, loss, backward, optimizer step) captured once in a HIP
    graph and replayed: removes the host's per-kernel launch work (~1200 launches per step
    for the 130M model). The inputs are static tensors the caller refills between replays;
    `loss` is the static loss of the last replay. The optimizer must be capturable
    (e.g. AdamW(capturable=True)). Capture follows torch.cuda.graph's whole-network recipe:
    warm-up steps on a side stream, then one captured step with gradients allocated inside
    the graph's memory pool. Callers must hold no autograd graph of earlier steps (e.g. a
    loss tensor): it keeps the parameters' gradient-accumulation nodes bound to the stream
    they ran on, which breaks the capture."""

    def __init__(self, model, optimizer, loss_fn, tokens, targets, warmup=3, act_dtype=torch.bfloat16):
        self.tokens, self.targets = tokens, targets
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                optimizer.zero_grad(set_to_none=True)
                loss_fn(model(tokens, act_dtype=act_dtype), targets).backward()
                optimizer.step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        optimizer.zero_grad(set_to_none=True)
        with torch.cuda.graph(self.graph):
            self.loss = loss_fn(model(tokens, act_dtype=act_dtype), targets)
            self.loss.backward()
            optimizer.step()

    def step(self):
        self.graph.replay()
        return self.loss
