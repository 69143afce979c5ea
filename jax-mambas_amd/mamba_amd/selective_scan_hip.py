"""Selective scan on MI355X: the reference's call signatures over the HIP C ABI.

Two entry points, one pair of kernels:

* ``selective_scan(A, deltas, Bs, Cs, u, initial_x=None, *, use_euler_barB_approx=True,
  use_cuda=True, remat=False)`` — the reference's public contract
  (``mamba/selective_scan_cuda.py:262-308``): logical (B, L, D) / (B, L, N) tensors,
  float32 only, returns ``(y, final_x)``; same validation and error types as
  ``_validate_inputs`` (``:93-121``). ``use_cuda`` and ``remat`` are accepted for
  signature compatibility: the HIP kernels always run, and their backward recomputes the
  per-step states (what ``remat`` asks of the reference path).
* ``selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None,
  delta_softplus=False, return_last_state=False, initial_state=None, seq_lens=None,
  discretization="euler")`` — the fused form in channel-major layout (u/delta/z:
  (B, D, L); B/C: (B, N, L)), with float32 or bfloat16 activations and float32 A, D,
  delta_bias and states. Softplus(delta + bias), the D skip, the silu(z) gate, the
  initial/last state and per-row lengths run inside the kernels.

Both are differentiable (torch autograd); gradients come from the HIP backward kernel.
There is no CPU path: inputs must live on a ROCm GPU and the library must be built.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["selective_scan", "selective_scan_fn", "register_hip_kernel", "bwd_workspace_bytes"]

register_hip_kernel = _lib.register_hip_kernel


def _ptr(t):
    return None if t is None else t.data_ptr()


def _io_tag(dtype, what):
    if dtype == torch.float32:
        return _lib.MSS_F32
    if dtype == torch.bfloat16:
        return _lib.MSS_BF16
    raise TypeError(f"{what} must be float32 or bfloat16, got {dtype}")


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the HIP selective scan requires tensors on a ROCm GPU device")


def _strides(u, io_layout, B, bc_layout):
    io_b, io_r = _row_strides(u, io_layout)
    bc_b, bc_r = _row_strides(B, bc_layout)
    return _lib.Strides(io_batch=io_b, io_dim=io_r, bc_batch=bc_b, bc_state=bc_r)


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_f32(name, t, shape):
    if t is None:
        return
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _validate_fused(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, discretization):
    if u.ndim != 3 or A.ndim != 2:
        raise ValueError("u must have shape (B, D, L) and A shape (D, N)")
    batch, dim, length = u.shape
    n = A.shape[1]
    if length == 0:
        raise ValueError("The sequence length must be positive")
    if not 1 <= n <= _lib.MSS_MAX_DSTATE:
        raise ValueError(f"N must be between 1 and {_lib.MSS_MAX_DSTATE}")
    if discretization not in ("euler", "zoh"):
        raise ValueError("discretization must be 'euler' or 'zoh'")
    _io_tag(u.dtype, "u")
    for name, t in (("delta", delta), ("z", z)):
        if t is None:
            continue
        if t.dtype != u.dtype:
            raise TypeError(f"{name} must have the dtype of u ({u.dtype}), got {t.dtype}")
        if tuple(t.shape) != (batch, dim, length):
            raise ValueError(f"{name} must have shape {(batch, dim, length)}, got {tuple(t.shape)}")
    _io_tag(B.dtype, "B")
    if C.dtype != B.dtype:
        raise TypeError(f"C must have the dtype of B ({B.dtype}), got {C.dtype}")
    for name, t in (("B", B), ("C", C)):
        if tuple(t.shape) != (batch, n, length):
            raise ValueError(f"{name} must have shape {(batch, n, length)}, got {tuple(t.shape)}")
    _check_f32("A", A, (dim, n))
    _check_f32("D", D, (dim,))
    _check_f32("delta_bias", delta_bias, (dim,))
    _check_f32("initial_state", initial_state, (batch, dim, n))
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or tuple(seq_lens.shape) != (batch,):
            raise ValueError(f"seq_lens must be int32 with shape ({batch},)")
    _require_gpu(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens)
    return batch, dim, length, n


def bwd_workspace_bytes(batch, dim, length, dstate):
    lib = register_hip_kernel()
    a = _lib.BwdArgs(batch=batch, dim=dim, seqlen=length, dstate=dstate)
    return int(lib.mss_bwd_workspace_bytes(a))


def _contig(t):
    return None if t is None else t.contiguous()


# Row layouts of a (batch, rows, steps) tensor the kernels read without a copy: steps
# contiguous and rows dense either batch-outer ("brl": [B][R][L]) or row-outer ("rbl":
# [R][B][L], the layout of an (R, B*L) activation matrix).
def _dense_strides(shape, layout):
    b, r, l = shape
    return (r * l, l, 1) if layout == "brl" else (l, b * l, 1)


def _strides_match(t, layout):
    b, r, l = t.shape
    want = _dense_strides(t.shape, layout)
    got = t.stride()
    return got[2] == 1 and (b == 1 or got[0] == want[0]) and (r == 1 or got[1] == want[1])


def _layout_of(t):
    for layout in ("brl", "rbl"):
        if _strides_match(t, layout):
            return layout
    return None


def _empty_rows(shape, layout, dtype, device):
    b, r, l = shape
    if layout == "rbl":
        return torch.empty(r, b, l, dtype=dtype, device=device).permute(1, 0, 2)
    return torch.empty(b, r, l, dtype=dtype, device=device)


def _conform(t, layout):
    """t in the given dense row layout (a copy only when its strides differ)."""
    if t is None or _strides_match(t, layout):
        return t
    out = _empty_rows(t.shape, layout, t.dtype, t.device)
    out.copy_(t)
    return out


def _row_strides(t, layout):
    """(batch stride, row stride) the kernels use for tensors in this layout."""
    s = _dense_strides(t.shape, layout)
    return s[0], s[1]


class _SelectiveScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, delta_softplus, zoh,
                io_layout, bc_layout):
        lib = register_hip_kernel()
        batch, dim, length = u.shape
        n = A.shape[1]
        n_seg = (length + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
        out = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        last = torch.empty(batch, dim, n, device=u.device, dtype=torch.float32)
        # Residual: the state entering every 8-step segment, [B][D][N][ceil(L/8)].
        carries = torch.empty(batch, dim, n, n_seg, device=u.device, dtype=torch.float32)
        # Pre-gate output: the backward's dz needs it (kept only when z is given).
        y_pre = _empty_rows(u.shape, io_layout, u.dtype, u.device) if z is not None else None
        args = _lib.FwdArgs(
            batch=batch, dim=dim, seqlen=length, dstate=n,
            discretization=_lib.MSS_ZOH if zoh else _lib.MSS_EULER,
            delta_softplus=int(bool(delta_softplus)),
            io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
            u=_ptr(u), delta=_ptr(delta), A=_ptr(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
            delta_bias=_ptr(delta_bias), initial_state=_ptr(initial_state), seq_lens=_ptr(seq_lens),
            out=_ptr(out), last_state=_ptr(last), carries=_ptr(carries), y_pre=_ptr(y_pre),
            strides=_strides(u, io_layout, B, bc_layout),
        )
        _lib.check(lib.mss_fwd(args, _stream(u)), "mss_fwd")
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre)
        ctx.delta_softplus = bool(delta_softplus)
        ctx.zoh = bool(zoh)
        ctx.layouts = (io_layout, bc_layout)
        return out, last

    @staticmethod
    def backward(ctx, dout, dlast):
        lib = register_hip_kernel()
        u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre = ctx.saved_tensors
        batch, dim, length = u.shape
        n = A.shape[1]
        io_layout, bc_layout = ctx.layouts
        if dout is None:
            dout = torch.zeros_like(u)
        dout = _conform(dout.to(u.dtype), io_layout)
        dlast = None if dlast is None else dlast.float().contiguous()
        du = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        ddelta = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        dA = torch.empty_like(A)
        dB = _empty_rows(B.shape, bc_layout, B.dtype, B.device)
        dC = _empty_rows(C.shape, bc_layout, C.dtype, C.device)
        dD = None if D is None else torch.empty_like(D)
        dz = None if z is None else _empty_rows(u.shape, io_layout, u.dtype, u.device)
        dbias = None if delta_bias is None else torch.empty_like(delta_bias)
        dinit = None if initial_state is None else torch.empty_like(initial_state)
        args = _lib.BwdArgs(
            batch=batch, dim=dim, seqlen=length, dstate=n,
            discretization=_lib.MSS_ZOH if ctx.zoh else _lib.MSS_EULER,
            delta_softplus=int(ctx.delta_softplus),
            io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
            u=_ptr(u), delta=_ptr(delta), A=_ptr(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
            delta_bias=_ptr(delta_bias), initial_state=_ptr(initial_state), seq_lens=_ptr(seq_lens),
            carries=_ptr(carries), y_pre=_ptr(y_pre), dout=_ptr(dout), dlast_state=_ptr(dlast),
            du=_ptr(du), ddelta=_ptr(ddelta), dA=_ptr(dA), dB=_ptr(dB), dC=_ptr(dC), dD=_ptr(dD),
            dz=_ptr(dz), ddelta_bias=_ptr(dbias), dinitial_state=_ptr(dinit),
            strides=_strides(u, io_layout, B, bc_layout),
        )
        ws_bytes = int(lib.mss_bwd_workspace_bytes(args))
        ws = torch.empty(ws_bytes, device=u.device, dtype=torch.uint8)
        args.workspace = ws.data_ptr()
        args.workspace_bytes = ws_bytes
        _lib.check(lib.mss_bwd(args, _stream(u)), "mss_bwd")
        return du, ddelta, dA, dB, dC, dD, dz, dbias, dinit, None, None, None, None, None


class _ComplexSelectiveScan(torch.autograd.Function):
    """Complex A (mss_cfwd / mss_cbwd): A (D, N), initial and last state (B, D, N) complex64,
    passed to the kernels as interleaved float32 pairs (torch.view_as_real, no copy)."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, delta_softplus, zoh,
                io_layout, bc_layout):
        lib = register_hip_kernel()
        batch, dim, length = u.shape
        n = A.shape[1]
        n_seg = (length + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
        out = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        last = torch.empty(batch, dim, n, device=u.device, dtype=torch.complex64)
        carries = torch.empty(batch, dim, n, n_seg, device=u.device, dtype=torch.complex64)
        y_pre = _empty_rows(u.shape, io_layout, u.dtype, u.device) if z is not None else None
        rv = lambda t: None if t is None else torch.view_as_real(t).data_ptr()
        args = _lib.FwdArgs(
            batch=batch, dim=dim, seqlen=length, dstate=n,
            discretization=_lib.MSS_ZOH if zoh else _lib.MSS_EULER,
            delta_softplus=int(bool(delta_softplus)),
            io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
            u=_ptr(u), delta=_ptr(delta), A=rv(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
            delta_bias=_ptr(delta_bias), initial_state=rv(initial_state), seq_lens=_ptr(seq_lens),
            out=_ptr(out), last_state=rv(last), carries=rv(carries), y_pre=_ptr(y_pre),
            strides=_strides(u, io_layout, B, bc_layout),
        )
        _lib.check(lib.mss_cfwd(args, _stream(u)), "mss_cfwd")
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre)
        ctx.delta_softplus = bool(delta_softplus)
        ctx.zoh = bool(zoh)
        ctx.layouts = (io_layout, bc_layout)
        return out, last

    @staticmethod
    def backward(ctx, dout, dlast):
        lib = register_hip_kernel()
        u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre = ctx.saved_tensors
        batch, dim, length = u.shape
        n = A.shape[1]
        io_layout, bc_layout = ctx.layouts
        if dout is None:
            dout = torch.zeros_like(u)
        dout = _conform(dout.to(u.dtype), io_layout)
        # Torch's gradient of a complex tensor for a real loss is dL/dRe + i dL/dIm: the
        # convention of the C ABI's complex cotangents and gradients.
        dlast = None if dlast is None else dlast.to(torch.complex64).contiguous()
        rv = lambda t: None if t is None else torch.view_as_real(t).data_ptr()
        du = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        ddelta = _empty_rows(u.shape, io_layout, u.dtype, u.device)
        dA = torch.empty_like(A)
        dB = _empty_rows(B.shape, bc_layout, B.dtype, B.device)
        dC = _empty_rows(C.shape, bc_layout, C.dtype, C.device)
        dD = None if D is None else torch.empty_like(D)
        dz = None if z is None else _empty_rows(u.shape, io_layout, u.dtype, u.device)
        dbias = None if delta_bias is None else torch.empty_like(delta_bias)
        dinit = None if initial_state is None else torch.empty_like(initial_state)
        args = _lib.BwdArgs(
            batch=batch, dim=dim, seqlen=length, dstate=n,
            discretization=_lib.MSS_ZOH if ctx.zoh else _lib.MSS_EULER,
            delta_softplus=int(ctx.delta_softplus),
            io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
            u=_ptr(u), delta=_ptr(delta), A=rv(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
            delta_bias=_ptr(delta_bias), initial_state=rv(initial_state), seq_lens=_ptr(seq_lens),
            carries=rv(carries), y_pre=_ptr(y_pre), dout=_ptr(dout), dlast_state=rv(dlast),
            du=_ptr(du), ddelta=_ptr(ddelta), dA=rv(dA), dB=_ptr(dB), dC=_ptr(dC), dD=_ptr(dD),
            dz=_ptr(dz), ddelta_bias=_ptr(dbias), dinitial_state=rv(dinit),
            strides=_strides(u, io_layout, B, bc_layout),
        )
        ws_bytes = int(lib.mss_cbwd_workspace_bytes(args))
        ws = torch.empty(ws_bytes, device=u.device, dtype=torch.uint8)
        args.workspace = ws.data_ptr()
        args.workspace_bytes = ws_bytes
        _lib.check(lib.mss_cbwd(args, _stream(u)), "mss_cbwd")
        return du, ddelta, dA, dB, dC, dD, dz, dbias, dinit, None, None, None, None, None


def _validate_complex(A, initial_state):
    if A.dtype != torch.complex64:
        raise TypeError(f"a complex A must be complex64, got {A.dtype}")
    if initial_state is not None and initial_state.dtype != torch.complex64:
        raise TypeError(f"with a complex A, initial_state must be complex64, got {initial_state.dtype}")


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False, initial_state=None, seq_lens=None,
                      discretization="euler"):
    """Fused selective scan in channel-major layout; see the module docstring. A complex64 A
    selects the complex-state scan (the reference's complex_ssm branch,
    mamba/mamba1.py:160-176, 198): complex states, real output y = sum_n C Re(h) + D u,
    complex64 initial/last state."""
    cplx = A.is_complex()
    if cplx:
        _validate_complex(A, initial_state)
        _validate_fused(u, delta, torch.view_as_real(A)[..., 0], B, C, D, z, delta_bias,
                        None if initial_state is None else torch.view_as_real(initial_state)[..., 0],
                        seq_lens, discretization)
    else:
        _validate_fused(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, discretization)
    register_hip_kernel()
    # Rows of u/delta/z (and B/C) may be batch-outer or channel-outer; the others follow
    # u's (B's) layout, copied only when they differ.
    io_layout = _layout_of(u) or "brl"
    bc_layout = _layout_of(B) or "brl"
    fn = _ComplexSelectiveScan if cplx else _SelectiveScan
    out, last = fn.apply(
        _conform(u, io_layout), _conform(delta, io_layout), A.contiguous(),
        _conform(B, bc_layout), _conform(C, bc_layout),
        _contig(D), _conform(z, io_layout), _contig(delta_bias), _contig(initial_state),
        _contig(seq_lens), bool(delta_softplus), discretization == "zoh", io_layout, bc_layout)
    return (out, last) if return_last_state else out


def _validate_inputs(A, deltas, Bs, Cs, u, initial_x):
    """Error contract of the reference's ``_validate_inputs`` (mamba/selective_scan_cuda.py:93-121)."""
    if any(v.dtype != torch.float32 for v in (A, deltas, Bs, Cs, u, initial_x)):
        raise TypeError("The HIP selective scan reference API supports float32 only")
    if A.ndim != 2 or u.ndim != 3:
        raise ValueError("A must have shape (D, N) and u must have shape (B, L, D)")
    batch, length, dim = u.shape
    n = A.shape[1]
    if length == 0:
        raise ValueError("The sequence length must be positive")
    if n not in (1, 2, 4, 8, 16):
        raise ValueError("N must be one of 1, 2, 4, 8, or 16")
    expected = {
        "A": (dim, n),
        "deltas": (batch, length, dim),
        "Bs": (batch, length, n),
        "Cs": (batch, length, n),
        "initial_x": (batch, dim, n),
    }
    actual = {"A": A.shape, "deltas": deltas.shape, "Bs": Bs.shape, "Cs": Cs.shape,
              "initial_x": initial_x.shape}
    for name, shape in expected.items():
        if tuple(actual[name]) != shape:
            raise ValueError(f"{name} must have shape {shape}, got {tuple(actual[name])}")


def selective_scan(A, deltas, Bs, Cs, u, initial_x=None, *, use_euler_barB_approx=True,
                   use_cuda=True, remat=False):
    """Reference-compatible scan: (B, L, D) / (B, L, N) in, ``(y (B, L, D), final_x (B, D, N))`` out."""
    del use_cuda, remat  # the HIP kernels always run; their backward recomputes states
    if initial_x is None:
        initial_x = torch.zeros(u.shape[0], u.shape[2], A.shape[1], dtype=torch.result_type(A, u),
                                device=u.device)
    _validate_inputs(A, deltas, Bs, Cs, u, initial_x)
    _require_gpu(A, deltas, Bs, Cs, u, initial_x)
    register_hip_kernel()
    # Channel-major physical layout at the kernel boundary (the reference gets the same
    # layout from XLA input_layouts=(0,2,1), mamba/selective_scan_cuda.py:135-147).
    t = lambda x: x.transpose(1, 2).contiguous()
    out, last = _SelectiveScan.apply(t(u), t(deltas), A.contiguous(), t(Bs), t(Cs), None, None,
                                     None, initial_x.contiguous(), None, False,
                                     not use_euler_barB_approx, "brl", "brl")
    return out.transpose(1, 2), last
