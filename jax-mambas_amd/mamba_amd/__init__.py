"""mamba_amd — MI355X-native Mamba-1 selective scan (HIP kernels for gfx950 behind a C ABI).

Public API:
  selective_scan      reference-compatible signature (mamba/selective_scan_cuda.py:262-308)
  selective_scan_fn   fused channel-major form (softplus/bias, D, silu(z), states, varlen)
  causal_conv1d_fn    causal depthwise conv1d + silu (the Mamba-1 block's short conv)
  register_hip_kernel load the HIP library (FileNotFoundError if it is not built)
"""
from .conv1d_hip import causal_conv1d_fn  # noqa: F401
from .selective_scan_hip import (  # noqa: F401
    bwd_workspace_bytes,
    register_hip_kernel,
    selective_scan,
    selective_scan_fn,
)

__all__ = ["selective_scan", "selective_scan_fn", "causal_conv1d_fn", "register_hip_kernel",
           "bwd_workspace_bytes"]
