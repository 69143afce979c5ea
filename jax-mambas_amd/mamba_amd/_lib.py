"""ctypes binding of libmamba_selective_scan_hip.so (the C ABI in include/mamba_selective_scan.h).

Loader behaviour mirrors the reference's ``register_cuda_kernel``
(``mamba/selective_scan_cuda.py:18-53``): an explicit path or a fixed candidate list,
``FileNotFoundError`` naming every searched path when nothing is built, idempotent
registration. There is no fallback: without the library nothing in this package runs.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIBRARY_NAME = "libmamba_selective_scan_hip.so"

MSS_ABI_VERSION = 16
MSS_OK = 0
MSS_ERR_INVALID_ARGUMENT = 1
MSS_ERR_UNSUPPORTED = 2
MSS_ERR_HIP = 3
MSS_ERR_WORKSPACE = 4
MSS_ERR_SCRATCH_LIMIT = 5
MSS_NOALLOC_SCRATCH_BYTES = 128 << 20
MSS_F32 = 0
MSS_BF16 = 1
MSS_EULER = 0
MSS_ZOH = 1
MSS_MAX_DSTATE = 16
MSS_MAX_DSTATE_WIDE = 256  # float32 real-A scans (backward over groups of MSS_MAX_DSTATE states)
MSS_SEG_STEPS = 8
MSS_REF_CHUNK = 2048
MSS_NORM_GEMV_MAX_FEATURES = 1024
MSS_XENT_FUSED_MAX_VOCAB = 65536

# Every symbol include/mamba_selective_scan.h declares.
EXPORTED_SYMBOLS = (
    "mss_bwd_workspace_bytes",
    "mss_bwd_plan",
    "mss_fwd",
    "mss_bwd",
    "mss_bwd_noalloc",
    "mss_bwd_scan",
    "mss_bwd_reduce",
    "mss_cbwd_workspace_bytes",
    "mss_cfwd",
    "mss_cbwd",
    "mss_scan_fwd",
    "mss_scan_fwd_repeat",
    "mss_scan_bwd",
    "mss_scan_bwd_workspace_bytes",
    "mss_scan_bwd_ws",
    "mss_conv_bwd_workspace_bytes",
    "mss_conv_fwd",
    "mss_conv_bwd",
    "mss_norm_bwd_workspace_bytes",
    "mss_norm_fwd",
    "mss_norm_bwd",
    "mss_xent_fwd",
    "mss_xent_bwd",
    "mss_xent_fwd_grad",
    "mss_xent_rescale",
    "mss_scan_step",
    "mss_cscan_step",
    "mss_conv_step",
    "mss_gemv",
    "mss_gemv_conv_step",
    "mss_gemv_scan_step",
    "mss_norm_gemv_conv_step",
    "mss_proj",
    "mss_wgrad_workspace_bytes",
    "mss_wgrad",
    "mss_shadow_refresh",
    "mss_adamw",
    "mss_embed_cm",
    "mss_embed_cm_backward",
    "mss_strerror",
    "mss_last_hip_error",
    "mss_abi_version",
)

_p = ctypes.c_void_p
_i32 = ctypes.c_int32


class Strides(ctypes.Structure):
    """mss_strides: row strides in elements (0 = contiguous default)."""
    _fields_ = [("io_batch", ctypes.c_int64), ("io_dim", ctypes.c_int64),
                ("bc_batch", ctypes.c_int64), ("bc_state", ctypes.c_int64)]


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("dim", _i32), ("seqlen", _i32), ("dstate", _i32),
        ("discretization", _i32), ("delta_softplus", _i32), ("io_dtype", _i32), ("bc_dtype", _i32),
        ("u", _p), ("delta", _p), ("A", _p), ("B", _p), ("C", _p),
        ("D", _p), ("z", _p), ("delta_bias", _p), ("initial_state", _p), ("seq_lens", _p),
        ("out", _p), ("last_state", _p), ("carries", _p), ("y_pre", _p),
        ("strides", Strides),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("dim", _i32), ("seqlen", _i32), ("dstate", _i32),
        ("discretization", _i32), ("delta_softplus", _i32), ("io_dtype", _i32), ("bc_dtype", _i32),
        ("u", _p), ("delta", _p), ("A", _p), ("B", _p), ("C", _p),
        ("D", _p), ("z", _p), ("delta_bias", _p), ("initial_state", _p), ("seq_lens", _p),
        ("carries", _p), ("y_pre", _p), ("out", _p), ("dout", _p), ("dlast_state", _p),
        ("du", _p), ("ddelta", _p), ("dA", _p), ("dB", _p), ("dC", _p), ("dD", _p), ("dz", _p),
        ("ddelta_bias", _p), ("dinitial_state", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
        ("strides", Strides),
    ]


class ConvArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("dim", _i32), ("seqlen", _i32), ("width", _i32), ("io_dtype", _i32),
        ("activation", _i32),
        ("x", _p), ("weight", _p), ("bias", _p), ("seq_lens", _p), ("y", _p), ("dy", _p), ("dx", _p),
        ("dweight", _p), ("dbias", _p), ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
        ("strides", Strides),
    ]


class NormArgs(ctypes.Structure):
    _fields_ = [
        ("features", _i32), ("tokens", _i32), ("eps", ctypes.c_float), ("io_dtype", _i32),
        ("h", _p), ("delta", _p), ("weight", _p), ("hn", _p), ("x", _p), ("rstd", _p),
        ("dx", _p), ("dhn_in", _p), ("dhn", _p), ("ddelta", _p), ("dweight", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class XentArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _i32), ("vocab", _i32), ("logits", _p), ("targets", _p), ("loss", _p), ("lse", _p),
        ("grad_scale", _p), ("dlogits", _p),
    ]


class StepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("dim", _i32), ("dstate", _i32), ("discretization", _i32), ("delta_softplus", _i32),
        ("io_dtype", _i32), ("bc_dtype", _i32),
        ("state", _p), ("u", _p), ("delta", _p), ("A", _p), ("B", _p), ("C", _p), ("D", _p), ("z", _p),
        ("delta_bias", _p), ("out", _p), ("strides", Strides),
    ]


class GemvArgs(ctypes.Structure):
    _fields_ = [("M", _i32), ("K", _i32), ("N", _i32), ("ldw", ctypes.c_int64), ("W", _p), ("X", _p), ("Y", _p)]


class ProjArgs(ctypes.Structure):
    _fields_ = [("M", _i32), ("K", _i32), ("T", _i32), ("accumulate", _i32), ("w_trans", _i32), ("ldw", ctypes.c_int64),
                ("ldx", ctypes.c_int64), ("ldc", ctypes.c_int64), ("W", _p), ("X", _p), ("C", _p)]


class WgradArgs(ctypes.Structure):
    _fields_ = [("M", _i32), ("N", _i32), ("K", _i32), ("accumulate", _i32), ("lda", ctypes.c_int64),
                ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64), ("A", _p), ("B", _p), ("C", _p), ("workspace", _p),
                ("workspace_bytes", ctypes.c_int64)]


class ShadowEntry(ctypes.Structure):
    _fields_ = [("src", _p), ("dst", _p), ("dst_t", _p), ("rows", _i32), ("cols", _i32), ("ld_t", ctypes.c_int64),
                ("tile0", ctypes.c_int64)]


class AdamWEntry(ctypes.Structure):
    _fields_ = [("param", _p), ("grad", _p), ("exp_avg", _p), ("exp_avg_sq", _p), ("step", _p), ("shadow", _p),
                ("shadow_t", _p), ("rows", _i32), ("cols", _i32), ("ld_t", ctypes.c_int64), ("numel", ctypes.c_int64)]


class AdamWArgs(ctypes.Structure):
    _fields_ = [("entries", _p), ("n_entries", _i32), ("lr", ctypes.c_float), ("beta1", ctypes.c_float),
                ("beta2", ctypes.c_float), ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float)]


class ConvStepArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("dim", _i32), ("width", _i32), ("io_dtype", _i32), ("activation", _i32),
        ("conv_state", _p), ("x", _p), ("weight", _p), ("bias", _p), ("y", _p), ("strides", Strides),
    ]


_LIBRARY = None
_LIBRARY_PATH = None


def library_candidates():
    env = os.environ.get("MSS_LIBRARY")
    if env:
        yield Path(env)
    pkg_root = Path(__file__).resolve().parents[1]  # jax-mambas_amd/
    yield pkg_root / "build" / LIBRARY_NAME
    yield pkg_root / LIBRARY_NAME


def register_hip_kernel(library_path=None):
    """Load the HIP library once; raise FileNotFoundError if it is not built."""
    global _LIBRARY, _LIBRARY_PATH
    if _LIBRARY is not None:
        return _LIBRARY
    candidates = [Path(library_path)] if library_path is not None else list(library_candidates())
    path = next((c for c in candidates if c.is_file()), None)
    if path is None:
        searched = ", ".join(str(c) for c in candidates)
        raise FileNotFoundError(f"The selective-scan HIP library is not built; searched: {searched}")
    lib = ctypes.CDLL(str(path))
    lib.mss_fwd.argtypes = [ctypes.POINTER(FwdArgs), _p]
    lib.mss_fwd.restype = ctypes.c_int
    lib.mss_bwd.argtypes = [ctypes.POINTER(BwdArgs), _p]
    lib.mss_bwd.restype = ctypes.c_int
    for name in ("mss_bwd_noalloc", "mss_bwd_scan", "mss_bwd_reduce", "mss_cbwd"):
        getattr(lib, name).argtypes = [ctypes.POINTER(BwdArgs), _p]
        getattr(lib, name).restype = ctypes.c_int
    lib.mss_cfwd.argtypes = [ctypes.POINTER(FwdArgs), _p]
    lib.mss_cfwd.restype = ctypes.c_int
    for name in ("mss_bwd_workspace_bytes", "mss_cbwd_workspace_bytes"):
        getattr(lib, name).argtypes = [ctypes.POINTER(BwdArgs)]
        getattr(lib, name).restype = ctypes.c_size_t
    lib.mss_bwd_plan.argtypes = [ctypes.POINTER(BwdArgs), ctypes.POINTER(_i32), ctypes.POINTER(_i32)]
    lib.mss_bwd_plan.restype = ctypes.c_int
    lib.mss_scan_fwd.argtypes = [_p, _i32, _i32, _i32, _i32, _i32] + [_p] * 9
    lib.mss_scan_fwd.restype = ctypes.c_int
    lib.mss_scan_fwd_repeat.argtypes = [_p, _i32, _i32, _i32, _i32, _i32, _i32] + [_p] * 9
    lib.mss_scan_fwd_repeat.restype = ctypes.c_int
    lib.mss_scan_bwd.argtypes = [_p, _i32, _i32, _i32, _i32] + [_p] * 15
    lib.mss_scan_bwd.restype = ctypes.c_int
    lib.mss_scan_bwd_ws.argtypes = [_p, _i32, _i32, _i32, _i32] + [_p] * 16 + [ctypes.c_size_t]
    lib.mss_scan_bwd_ws.restype = ctypes.c_int
    lib.mss_scan_bwd_workspace_bytes.argtypes = [_i32, _i32, _i32, _i32]
    lib.mss_scan_bwd_workspace_bytes.restype = ctypes.c_size_t
    for name in ("mss_conv_fwd", "mss_conv_bwd"):
        getattr(lib, name).argtypes = [ctypes.POINTER(ConvArgs), _p]
        getattr(lib, name).restype = ctypes.c_int
    lib.mss_conv_bwd_workspace_bytes.argtypes = [ctypes.POINTER(ConvArgs)]
    lib.mss_conv_bwd_workspace_bytes.restype = ctypes.c_size_t
    for name in ("mss_norm_fwd", "mss_norm_bwd"):
        getattr(lib, name).argtypes = [ctypes.POINTER(NormArgs), _p]
        getattr(lib, name).restype = ctypes.c_int
    lib.mss_norm_bwd_workspace_bytes.argtypes = [ctypes.POINTER(NormArgs)]
    lib.mss_norm_bwd_workspace_bytes.restype = ctypes.c_size_t
    for name in ("mss_xent_fwd", "mss_xent_bwd", "mss_xent_fwd_grad"):
        getattr(lib, name).argtypes = [ctypes.POINTER(XentArgs), _p]
        getattr(lib, name).restype = ctypes.c_int
    lib.mss_xent_rescale.argtypes = [_p, ctypes.c_int64, _p, _p]
    lib.mss_xent_rescale.restype = ctypes.c_int
    for name in ("mss_scan_step", "mss_cscan_step"):
        getattr(lib, name).argtypes = [ctypes.POINTER(StepArgs), _p]
        getattr(lib, name).restype = ctypes.c_int
    lib.mss_conv_step.argtypes = [ctypes.POINTER(ConvStepArgs), _p]
    lib.mss_conv_step.restype = ctypes.c_int
    lib.mss_gemv.argtypes = [ctypes.POINTER(GemvArgs), _p]
    lib.mss_gemv.restype = ctypes.c_int
    lib.mss_gemv_conv_step.argtypes = [ctypes.POINTER(GemvArgs), ctypes.POINTER(ConvStepArgs), _p]
    lib.mss_gemv_conv_step.restype = ctypes.c_int
    lib.mss_gemv_scan_step.argtypes = [ctypes.POINTER(GemvArgs), ctypes.POINTER(StepArgs), _p]
    lib.mss_gemv_scan_step.restype = ctypes.c_int
    lib.mss_norm_gemv_conv_step.argtypes = [ctypes.POINTER(NormArgs), ctypes.POINTER(GemvArgs),
                                            ctypes.POINTER(ConvStepArgs), _p]
    lib.mss_norm_gemv_conv_step.restype = ctypes.c_int
    lib.mss_proj.argtypes = [ctypes.POINTER(ProjArgs), _p]
    lib.mss_proj.restype = ctypes.c_int
    lib.mss_wgrad_workspace_bytes.argtypes = [_i32, _i32, _i32]
    lib.mss_wgrad_workspace_bytes.restype = ctypes.c_int64
    lib.mss_wgrad.argtypes = [ctypes.POINTER(WgradArgs), _p]
    lib.mss_wgrad.restype = ctypes.c_int
    lib.mss_shadow_refresh.argtypes = [_p, _i32, ctypes.c_int64, _p]
    lib.mss_shadow_refresh.restype = ctypes.c_int
    lib.mss_adamw.argtypes = [ctypes.POINTER(AdamWArgs), _p]
    lib.mss_adamw.restype = ctypes.c_int
    lib.mss_embed_cm.argtypes = [_p, ctypes.c_int64, _p, _i32, _i32, _p, ctypes.c_int64, _p]
    lib.mss_embed_cm.restype = ctypes.c_int
    lib.mss_embed_cm_backward.argtypes = [_p, ctypes.c_int64, _p, _p, ctypes.c_int64, _i32, _i32, _p, _p, ctypes.c_int64,
                                          _p]
    lib.mss_embed_cm_backward.restype = ctypes.c_int
    lib.mss_strerror.argtypes = [ctypes.c_int]
    lib.mss_strerror.restype = ctypes.c_char_p
    lib.mss_last_hip_error.argtypes = []
    lib.mss_last_hip_error.restype = ctypes.c_char_p
    lib.mss_abi_version.argtypes = []
    lib.mss_abi_version.restype = ctypes.c_int
    if lib.mss_abi_version() != MSS_ABI_VERSION:
        raise ImportError(f"{path} has ABI version {lib.mss_abi_version()}, this front-end "
                          f"expects {MSS_ABI_VERSION}; rebuild the library")
    _LIBRARY = lib
    _LIBRARY_PATH = path
    return lib


def library_path():
    return _LIBRARY_PATH


class MSSError(RuntimeError):
    def __init__(self, status, op):
        lib = register_hip_kernel()
        msg = lib.mss_strerror(status).decode()
        if status == MSS_ERR_HIP:
            msg += ": " + lib.mss_last_hip_error().decode()
        super().__init__(f"{op} failed with status {status}: {msg}")
        self.status = status


def bwd_plan(batch, dim, dstate, seqlen=2048, varlen=False, zoh=False, io_bf16=False, bc_bf16=None,
             z=True, strides=None):
    """(waves per workgroup, channels per workgroup) of the backward scan mss_bwd would run
    for a call with these shapes."""
    lib = register_hip_kernel()
    bc_bf16 = io_bf16 if bc_bf16 is None else bc_bf16
    a = BwdArgs(batch=batch, dim=dim, seqlen=seqlen, dstate=dstate, discretization=MSS_ZOH if zoh else MSS_EULER,
                io_dtype=MSS_BF16 if io_bf16 else MSS_F32, bc_dtype=MSS_BF16 if bc_bf16 else MSS_F32,
                u=256, delta=256, A=256, B=256, C=256, carries=256, dout=256, du=256, ddelta=256, dA=256,
                dB=256, dC=256, seq_lens=256 if varlen else None, z=256 if z else None,
                y_pre=256 if z else None, out=256 if z else None, dz=256 if z else None)
    if strides is not None:
        a.strides = strides
    w, c = _i32(), _i32()
    check(lib.mss_bwd_plan(ctypes.byref(a), ctypes.byref(w), ctypes.byref(c)), "mss_bwd_plan")
    return w.value, c.value


def check(status, op):
    if status != MSS_OK:
        raise MSSError(status, op)
