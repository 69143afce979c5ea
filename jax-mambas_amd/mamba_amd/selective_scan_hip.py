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

Both run through two torch.library custom ops, ``torch.ops.mamba_amd.selective_scan_fwd``
and ``selective_scan_bwd`` (the C ABI's mss_fwd/mss_bwd, or mss_cfwd/mss_cbwd for a complex
A), with fake implementations (shapes, dtypes and row layouts) and registered autograd, so
they are differentiable and traceable by torch.compile; gradients come from the HIP backward
kernel. There is no CPU path: inputs must live on a ROCm GPU and the library must be built.
"""
from __future__ import annotations

from typing import Optional, Tuple

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


def _validate_fused(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, discretization,
                    cplx=False):
    if u.ndim != 3 or A.ndim != 2:
        raise ValueError("u must have shape (B, D, L) and A shape (D, N)")
    batch, dim, length = u.shape
    n = A.shape[1]
    if length == 0:
        raise ValueError("The sequence length must be positive")
    # float32 real-A scans take up to 256 states (the backward runs over groups of 16)
    wide = not cplx and u.dtype == torch.float32 and B.dtype == torch.float32
    n_max = _lib.MSS_MAX_DSTATE_WIDE if wide else _lib.MSS_MAX_DSTATE
    if not 1 <= n <= n_max:
        kind = "float32 real-A" if wide else "bf16 or complex-A"
        raise ValueError(f"N must be between 1 and {n_max} for {kind} scans")
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


# ---- torch.library custom ops over the C ABI (real and complex A). Optional results are
# returned as empty tensors (custom ops return tensors only). The fake implementations give
# the real ones' shapes, dtypes and row layouts, so torch.compile can trace the scan.

_EMPTY = 0  # numel of an absent optional result


def _layouts(u, B):
    return _layout_of(u) or "brl", _layout_of(B) or "brl"


def _state_dtype(A):
    return torch.complex64 if A.is_complex() else torch.float32


def _fwd_outputs(u, A, B, z):
    """(out, last, carries, y_pre) allocated in the layouts the kernels write."""
    batch, dim, length = u.shape
    n = A.shape[1]
    io_layout, _ = _layouts(u, B)
    n_seg = (length + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
    sdt = _state_dtype(A)
    out = _empty_rows(u.shape, io_layout, u.dtype, u.device)
    last = torch.empty(batch, dim, n, device=u.device, dtype=sdt)
    # Residual: the state entering every 8-step segment, [B][D][N][ceil(L/8)].
    carries = torch.empty(batch, dim, n, n_seg, device=u.device, dtype=sdt)
    # Pre-gate output: the backward's dz needs it (kept only when z is given).
    y_pre = (_empty_rows(u.shape, io_layout, u.dtype, u.device) if z is not None
             else torch.empty(_EMPTY, device=u.device, dtype=u.dtype))
    return out, last, carries, y_pre


def _rv(t):
    """Device pointer; complex tensors as interleaved (real, imaginary) float32 pairs."""
    if t is None:
        return None
    return torch.view_as_real(t).data_ptr() if t.is_complex() else t.data_ptr()


@torch.library.custom_op("mamba_amd::selective_scan_fwd", mutates_args=(), device_types="cuda")
def _scan_fwd_op(u: torch.Tensor, delta: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                 D: Optional[torch.Tensor], z: Optional[torch.Tensor], delta_bias: Optional[torch.Tensor],
                 initial_state: Optional[torch.Tensor], seq_lens: Optional[torch.Tensor],
                 delta_softplus: bool, zoh: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """mss_fwd (mss_cfwd for a complex A): returns (out, last_state, carries, y_pre)."""
    lib = register_hip_kernel()
    io_layout, bc_layout = _layouts(u, B)
    delta, z = _conform(delta, io_layout), _conform(z, io_layout)
    C = _conform(C, bc_layout)
    batch, dim, length = u.shape
    out, last, carries, y_pre = _fwd_outputs(u, A, B, z)
    args = _lib.FwdArgs(
        batch=batch, dim=dim, seqlen=length, dstate=A.shape[1],
        discretization=_lib.MSS_ZOH if zoh else _lib.MSS_EULER, delta_softplus=int(bool(delta_softplus)),
        io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
        u=_ptr(u), delta=_ptr(delta), A=_rv(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
        delta_bias=_ptr(delta_bias), initial_state=_rv(initial_state), seq_lens=_ptr(seq_lens),
        out=_ptr(out), last_state=_rv(last), carries=_rv(carries), y_pre=_ptr(y_pre) if z is not None else None,
        strides=_strides(u, io_layout, B, bc_layout),
    )
    fn, name = (lib.mss_cfwd, "mss_cfwd") if A.is_complex() else (lib.mss_fwd, "mss_fwd")
    _lib.check(fn(args, _stream(u)), name)
    return out, last, carries, y_pre


@_scan_fwd_op.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, delta_softplus, zoh):
    return _fwd_outputs(u, A, B, z)


def _bwd_outputs(u, A, B, D, z, delta_bias, initial_state):
    io_layout, bc_layout = _layouts(u, B)
    empty = lambda dt: torch.empty(_EMPTY, device=u.device, dtype=dt)
    du = _empty_rows(u.shape, io_layout, u.dtype, u.device)
    ddelta = _empty_rows(u.shape, io_layout, u.dtype, u.device)
    dA = torch.empty_like(A)
    dB = _empty_rows(B.shape, bc_layout, B.dtype, B.device)
    dC = _empty_rows(B.shape, bc_layout, B.dtype, B.device)
    dD = empty(torch.float32) if D is None else torch.empty_like(D)
    dz = empty(u.dtype) if z is None else _empty_rows(u.shape, io_layout, u.dtype, u.device)
    dbias = empty(torch.float32) if delta_bias is None else torch.empty_like(delta_bias)
    dinit = empty(_state_dtype(A)) if initial_state is None else torch.empty_like(initial_state)
    return du, ddelta, dA, dB, dC, dD, dz, dbias, dinit


@torch.library.custom_op("mamba_amd::selective_scan_bwd", mutates_args=(), device_types="cuda")
def _scan_bwd_op(u: torch.Tensor, delta: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                 D: Optional[torch.Tensor], z: Optional[torch.Tensor], delta_bias: Optional[torch.Tensor],
                 initial_state: Optional[torch.Tensor], seq_lens: Optional[torch.Tensor],
                 carries: torch.Tensor, y_pre: torch.Tensor, out: Optional[torch.Tensor], dout: torch.Tensor,
                 dlast: Optional[torch.Tensor], delta_softplus: bool, zoh: bool
                 ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                            torch.Tensor, torch.Tensor, torch.Tensor]:
    """mss_bwd (mss_cbwd for a complex A): returns (du, ddelta, dA, dB, dC, dD, dz,
    ddelta_bias, dinitial_state), empty where the input is absent."""
    lib = register_hip_kernel()
    io_layout, bc_layout = _layouts(u, B)
    delta, z, dout = _conform(delta, io_layout), _conform(z, io_layout), _conform(dout.to(u.dtype), io_layout)
    C = _conform(C, bc_layout)
    y_pre = _conform(y_pre, io_layout) if z is not None else None
    out = _conform(out, io_layout) if z is not None and out is not None else None
    dlast = None if dlast is None else dlast.to(_state_dtype(A)).contiguous()
    batch, dim, length = u.shape
    du, ddelta, dA, dB, dC, dD, dz, dbias, dinit = _bwd_outputs(u, A, B, D, z, delta_bias, initial_state)
    opt = lambda t, given: _rv(t) if given is not None else None
    args = _lib.BwdArgs(
        batch=batch, dim=dim, seqlen=length, dstate=A.shape[1],
        discretization=_lib.MSS_ZOH if zoh else _lib.MSS_EULER, delta_softplus=int(bool(delta_softplus)),
        io_dtype=_io_tag(u.dtype, "u"), bc_dtype=_io_tag(B.dtype, "B"),
        u=_ptr(u), delta=_ptr(delta), A=_rv(A), B=_ptr(B), C=_ptr(C), D=_ptr(D), z=_ptr(z),
        delta_bias=_ptr(delta_bias), initial_state=_rv(initial_state), seq_lens=_ptr(seq_lens),
        carries=_rv(carries), y_pre=_ptr(y_pre), out=_ptr(out), dout=_ptr(dout), dlast_state=_rv(dlast),
        du=_ptr(du), ddelta=_ptr(ddelta), dA=_rv(dA), dB=_ptr(dB), dC=_ptr(dC), dD=opt(dD, D),
        dz=opt(dz, z), ddelta_bias=opt(dbias, delta_bias), dinitial_state=opt(dinit, initial_state),
        strides=_strides(u, io_layout, B, bc_layout),
    )
    cplx = A.is_complex()
    ws_bytes = int((lib.mss_cbwd_workspace_bytes if cplx else lib.mss_bwd_workspace_bytes)(args))
    ws = torch.empty(ws_bytes, device=u.device, dtype=torch.uint8)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws_bytes
    fn, name = (lib.mss_cbwd, "mss_cbwd") if cplx else (lib.mss_bwd, "mss_bwd")
    _lib.check(fn(args, _stream(u)), name)
    return du, ddelta, dA, dB, dC, dD, dz, dbias, dinit


@_scan_bwd_op.register_fake
def _(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre, out, dout, dlast,
      delta_softplus, zoh):
    return _bwd_outputs(u, A, B, D, z, delta_bias, initial_state)


def _scan_setup_context(ctx, inputs, output):
    u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, delta_softplus, zoh = inputs
    out, _, carries, y_pre = output
    # (the gate's backward reads the output itself: y sigma(z) = out / z)
    out = out if z is not None else None
    ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre, out)
    ctx.delta_softplus, ctx.zoh = delta_softplus, zoh


def _scan_backward(ctx, dout, dlast, _dcarries, _dy_pre):
    u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, carries, y_pre, out = ctx.saved_tensors
    if dout is None:
        dout = torch.zeros_like(u)
    g = torch.ops.mamba_amd.selective_scan_bwd(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens,
                                               carries, y_pre, out, dout, dlast, ctx.delta_softplus, ctx.zoh)
    du, ddelta, dA, dB, dC, dD, dz, dbias, dinit = g
    pick = lambda t, given: t if given is not None else None
    return (du, ddelta, dA, dB, dC, pick(dD, D), pick(dz, z), pick(dbias, delta_bias),
            pick(dinit, initial_state), None, None, None)


torch.library.register_autograd("mamba_amd::selective_scan_fwd", _scan_backward, setup_context=_scan_setup_context)


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
                        seq_lens, discretization, cplx=True)
    else:
        _validate_fused(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens, discretization)
    if not torch.compiler.is_compiling():
        register_hip_kernel()  # fail early when the library is missing (the op loads it too)
    # Rows of u/delta/z (and B/C) may be batch-outer or channel-outer; the others follow
    # u's (B's) layout, copied only when they differ.
    io_layout = _layout_of(u) or "brl"
    bc_layout = _layout_of(B) or "brl"
    out, last, _, _ = torch.ops.mamba_amd.selective_scan_fwd(
        _conform(u, io_layout), _conform(delta, io_layout), A.contiguous(),
        _conform(B, bc_layout), _conform(C, bc_layout),
        _contig(D), _conform(z, io_layout), _contig(delta_bias), _contig(initial_state),
        _contig(seq_lens), bool(delta_softplus), discretization == "zoh")
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
    out, last, _, _ = torch.ops.mamba_amd.selective_scan_fwd(
        t(u), t(deltas), A.contiguous(), t(Bs), t(Cs), None, None, None, initial_x.contiguous(), None,
        False, not use_euler_barB_approx)
    return out.transpose(1, 2), last
