"""Causal depthwise conv1d + SiLU (the Mamba-1 block's short convolution,
mamba/mamba1.py:250-255, 313-329) through the C ABI.

CPU: argument validation before any HIP call. GPU: forward and gradients vs the float64
oracle conv (oracle/mamba1_torch.py, itself checked against torch.conv1d), float32 within
rtol 1e-4 / atol 1e-5 (outputs per element; the weight and bias sums per element against
the sum of the absolute values of their terms), bf16 within 2e-2;
widths 1-4, ragged lengths, channel-outer row layouts, variable lengths, determinism.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mamba_amd import _lib
from mamba_amd.conv1d_hip import causal_conv1d_fn
from oracle import mamba1_torch as ref


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


def conv_args(**kw):
    base = dict(batch=2, dim=3, seqlen=10, width=4, activation=1, x=1, weight=1, y=1)
    base.update(kw)
    return _lib.ConvArgs(**base)


@pytest.mark.parametrize("kw,status", [
    (dict(batch=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(seqlen=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(width=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(width=5), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(activation=2), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(io_dtype=3), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(x=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(y=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dim=70000), _lib.MSS_ERR_UNSUPPORTED),
    (dict(strides=_lib.Strides(io_dim=4)), _lib.MSS_ERR_INVALID_ARGUMENT),
])
def test_conv_fwd_validation(lib, kw, status):
    assert lib.mss_conv_fwd(conv_args(**kw), None) == status


@pytest.mark.parametrize("kw", [dict(dy=None), dict(dx=None), dict(dweight=None), dict(bias=1)])
def test_conv_bwd_validation(lib, kw):
    base = dict(dy=1, dx=1, dweight=1)
    base.update(kw)
    assert lib.mss_conv_bwd(conv_args(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_conv_workspace_depends_on_shapes_only(lib):
    a = conv_args(batch=8, dim=1536, seqlen=2048)
    assert lib.mss_conv_bwd_workspace_bytes(a) == 1536 * 8 * 8 * 5 * 4  # 256-step tiles, K+1 sums
    assert lib.mss_conv_bwd_workspace_bytes(conv_args(width=9)) == 0


def test_conv_python_errors():
    x = torch.randn(2, 3, 10)
    with pytest.raises(ValueError, match="width"):
        causal_conv1d_fn(x, torch.randn(3, 5))
    with pytest.raises(TypeError, match="float32"):
        causal_conv1d_fn(x, torch.randn(3, 4).double())
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        causal_conv1d_fn(x, torch.randn(3, 4), torch.randn(3))


# ------------------------------------------------------------------ GPU parity
def oracle(x, w, b, lens, silu):
    """float64 forward + grads of sum(y * dy) from the oracle conv (B, L, D layout); `pre`
    (the pre-activation, its gradient retained) is returned for the |term| sums."""
    xt = torch.from_numpy(np.swapaxes(x, 1, 2).astype(np.float64)).requires_grad_(True)
    wt = torch.from_numpy(w.astype(np.float64)).requires_grad_(True)
    bt = torch.from_numpy(b.astype(np.float64)).requires_grad_(True)
    pre = ref.causal_depthwise_conv(xt, wt, bt)
    pre.retain_grad()
    y = F.silu(pre) if silu else pre
    if lens is not None:
        mask = (torch.arange(x.shape[2])[None, :, None] < torch.as_tensor(lens)[:, None, None]).double()
        y = y * mask
    return xt, wt, bt, y, pre


def weight_abs_terms(x, w, b, dpre):
    """Per element of dweight and dbias, the sum of the absolute values of the terms summed
    into it: sum over (b, t) of |dpre[t]| |x[t - (K-1) + k]| and of |dpre[t]| (the oracle conv
    run on |x| and contracted with |dpre|)."""
    xa = torch.from_numpy(np.abs(np.swapaxes(x, 1, 2)).astype(np.float64))
    wa = torch.from_numpy(w.astype(np.float64)).requires_grad_(True)
    ba = torch.from_numpy(b.astype(np.float64)).requires_grad_(True)
    (ref.causal_depthwise_conv(xa, wa, ba) * dpre.abs()).sum().backward()
    return wa.grad, ba.grad


def run_case(b, d, l, k, dtype, layout="brl", lens=None, silu=True, seed=0):
    print(f"case conv b={b} d={d} l={l} k={k} {dtype} {layout} lens={lens} silu={silu}", flush=True)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, d, l)).astype(np.float32)
    w = rng.standard_normal((d, k)).astype(np.float32) * 0.5
    bias = rng.standard_normal(d).astype(np.float32)
    dy = rng.standard_normal((b, d, l)).astype(np.float32)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        dy = torch.from_numpy(dy).to(torch.bfloat16).float().numpy()
    if layout == "rbl":
        leaf = torch.from_numpy(np.ascontiguousarray(np.swapaxes(x, 0, 1))).to("cuda", tdt).requires_grad_(True)
        xg = leaf.permute(1, 0, 2)
    else:
        leaf = torch.from_numpy(x).to("cuda", tdt).requires_grad_(True)
        xg = leaf
    wg = torch.from_numpy(w).cuda().requires_grad_(True)
    bg = torch.from_numpy(bias).cuda().requires_grad_(True)
    lens_t = None if lens is None else torch.tensor(lens, dtype=torch.int32, device="cuda")
    y = causal_conv1d_fn(xg, wg, bg, seq_lens=lens_t, activation="silu" if silu else None)
    assert y.stride() == xg.stride() and y.dtype == tdt
    (y.float() * torch.from_numpy(dy).cuda()).sum().backward()
    torch.cuda.synchronize()
    xt, wt, bt, yr, pre = oracle(x, w, bias, lens, silu)
    (yr * torch.from_numpy(np.swapaxes(dy, 1, 2).astype(np.float64))).sum().backward()
    w_abs, b_abs = weight_abs_terms(x, w, bias, pre.grad)
    rtol, atol = (2e-2, 2e-2) if dtype == "bf16" else (1e-4, 1e-5)
    got_y = y.detach().float().cpu().double()
    torch.testing.assert_close(got_y, yr.detach().transpose(1, 2), rtol=rtol, atol=atol)
    dx = leaf.grad.float().cpu().double()
    if layout == "rbl":
        dx = dx.permute(1, 0, 2)
    torch.testing.assert_close(dx, xt.grad.transpose(1, 2), rtol=rtol, atol=atol)
    # dweight / dbias are sums over (batch, step): per element |got - want| <= atol + rtol * s,
    # s the sum of the absolute values of the terms (any summation order stays within it).
    srtol, satol = (2e-2, 1e-3) if dtype == "bf16" else (1e-4, 1e-5)
    for name, got, want, s_abs in (("dweight", wg.grad, wt.grad, w_abs), ("dbias", bg.grad, bt.grad, b_abs)):
        err = (got.cpu().double() - want).abs()
        bound = satol + srtol * s_abs
        ratio = float((err / bound).max())
        print(f"  {name} max_abs={float(err.max()):.3e} worst err/bound={ratio:.3f}", flush=True)
        assert bool(torch.all(err <= bound)), (name, float(err.max()), ratio)
    return y, leaf.grad, wg.grad, bg.grad


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 2, 3, 4])
@pytest.mark.parametrize("l", [1, 3, 7, 300, 2048, 2051])
def test_conv_fp32(k, l):
    run_case(2, 5, l, k, "f32", seed=k * 1000 + l)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["brl", "rbl"])
@pytest.mark.parametrize("l", [64, 1027, 2048])
def test_conv_bf16_layouts(layout, l):
    run_case(3, 16, l, 4, "bf16", layout=layout, seed=l)


@pytest.mark.gpu
def test_conv_fp32_channel_outer_no_silu():
    run_case(4, 6, 1000, 4, "f32", layout="rbl", silu=False)


@pytest.mark.gpu
def test_conv_varlen():
    run_case(4, 8, 2100, 4, "f32", lens=[2100, 1000, 1, 0])


@pytest.mark.gpu
def test_conv_deterministic():
    a = run_case(3, 32, 4096, 4, "bf16", seed=5)
    b = run_case(3, 32, 4096, 4, "bf16", seed=5)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
