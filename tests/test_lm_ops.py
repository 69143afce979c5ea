"""Residual add + RMSNorm over a channel-major stream and bf16 cross-entropy (HIP kernels).

RMSNorm follows mamba/mamba1.py:300-337 (nnx.RMSNorm(epsilon=1e-5) before each block, the
block output added back); the loss is the training step's softmax cross-entropy
(experiments/mamba_inductionheads.py:129-136). CPU: argument validation. GPU: values and
gradients against float64 references on the same inputs — the oracle's rmsnorm
(oracle/mamba1_torch.py, pinned against torch.rms_norm) and torch's cross_entropy; the
one-pass loss + gradient (mss_xent_fwd_grad, taken when the loss will be differentiated)
against the two-pass path: losses within float32 rounding, gradients within one bf16 step.
fp32 activations within rtol 1e-4 / atol 1e-5 (the dweight sums over tokens on the
tensor's scale); bf16 within 2e-2.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mamba_amd import _lib
from mamba_amd.lm_ops import _CrossEntropy, add_rmsnorm, cross_entropy
from oracle import mamba1_torch as ref


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


@pytest.mark.parametrize("kw", [dict(features=0), dict(tokens=0), dict(eps=-1.0), dict(io_dtype=4),
                                dict(h=None), dict(x=None), dict(delta=1, hn=None)])
def test_norm_fwd_validation(lib, kw):
    base = dict(features=8, tokens=10, eps=1e-5, h=1, weight=1, x=1, rstd=1)
    base.update(kw)
    assert lib.mss_norm_fwd(_lib.NormArgs(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_norm_bwd_validation(lib):
    base = dict(features=8, tokens=10, eps=1e-5, h=1, weight=1, rstd=1, dx=1, dhn=1)
    assert lib.mss_norm_bwd(_lib.NormArgs(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT  # no dweight
    # dw partial rows: one per 64-token workgroup of the backward
    assert lib.mss_norm_bwd_workspace_bytes(_lib.NormArgs(features=768, tokens=16384)) == 256 * 768 * 4


@pytest.mark.parametrize("kw", [dict(rows=0), dict(vocab=0), dict(logits=None), dict(loss=None)])
def test_xent_validation(lib, kw):
    base = dict(rows=4, vocab=10, logits=1, targets=1, loss=1, lse=1)
    base.update(kw)
    assert lib.mss_xent_fwd(_lib.XentArgs(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_xent_bwd(_lib.XentArgs(rows=4, vocab=10, logits=1, targets=1, lse=1), None) == \
        _lib.MSS_ERR_INVALID_ARGUMENT  # no grad_scale / dlogits


@pytest.mark.parametrize("kw,status", [
    (dict(dlogits=None), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(grad_scale=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(loss=None), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(vocab=1003), _lib.MSS_ERR_UNSUPPORTED),
    (dict(vocab=65544), _lib.MSS_ERR_UNSUPPORTED), (dict(logits=(1 << 32) + 8), _lib.MSS_ERR_UNSUPPORTED),
    (dict(dlogits=(1 << 32) + 64), _lib.MSS_ERR_INVALID_ARGUMENT),  # overlaps the logits
])
def test_xent_fused_validation(lib, kw, status):
    base = dict(rows=4, vocab=1000, logits=1 << 32, targets=1 << 36, loss=1 << 37, lse=1 << 38, grad_scale=1 << 39,
                dlogits=1 << 40)
    base.update(kw)
    assert lib.mss_xent_fwd_grad(_lib.XentArgs(**base), None) == status
    assert lib.mss_xent_rescale(None, 10, 1 << 39, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_xent_rescale(1 << 40, 10, None, None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_python_errors():
    with pytest.raises(TypeError):
        add_rmsnorm(torch.randn(4, 5, dtype=torch.float64), None, torch.ones(4))
    with pytest.raises(TypeError):
        cross_entropy(torch.randn(3, 5), torch.zeros(3, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        add_rmsnorm(torch.randn(4, 5), None, torch.ones(4))


def _bound_check(name, got, want, rtol, atol, normwise=False):
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    err = (got - want).abs()
    bound = atol + rtol * (want.abs().max() if normwise else want.abs())
    worst = float((err - bound).max())
    print(f"  {name:8s} max_abs={float(err.max()):.3e} ok={worst <= 0}", flush=True)
    assert worst <= 0, name


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("with_delta", [False, True])
# (96, 300), (768, 1024): register-resident kernels (features a multiple of 32, <= 768;
# 300 tokens leave a partial workgroup); (100, 333) and (1024, 320): the two-pass kernels.
@pytest.mark.parametrize("shape", [(96, 300), (768, 1024), (100, 333), (1024, 320)])
def test_add_rmsnorm(dtype, with_delta, shape):
    print(f"case add_rmsnorm {dtype} delta={with_delta} shape={shape}", flush=True)
    f, t = shape
    act = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator().manual_seed(f + t)
    h0 = torch.randn(f, t, generator=g)
    d0 = torch.randn(f, t, generator=g).to(act).float()
    w0 = torch.rand(f, generator=g) + 0.5
    gx = torch.randn(f, t, generator=g).to(act).float()
    gh = torch.randn(f, t, generator=g)
    h = h0.cuda().requires_grad_(True)
    w = w0.cuda().requires_grad_(True)
    delta = d0.to(act).cuda().requires_grad_(True) if with_delta else None
    hn, x = add_rmsnorm(h, delta, w, 1e-5, act)
    assert x.dtype == act
    loss = (x.float() * gx.cuda()).sum() + ((hn * gh.cuda()).sum() if with_delta else 0.0)
    loss.backward()
    torch.cuda.synchronize()
    hr = h0.double().requires_grad_(True)
    wr = w0.double().requires_grad_(True)
    dr = d0.double().requires_grad_(True)
    hnr = hr + dr if with_delta else hr
    xr = ref.rmsnorm(hnr.t(), wr, 1e-5).t()
    lr = (xr * gx.double()).sum() + ((hnr * gh.double()).sum() if with_delta else 0.0)
    lr.backward()
    rtol, atol = (2e-2, 2e-2) if dtype == "bf16" else (1e-4, 1e-5)
    _bound_check("x", x.float(), xr, rtol, atol)
    if with_delta:
        _bound_check("hn", hn, hnr, 1e-6, 1e-6)
        _bound_check("ddelta", delta.grad.float(), dr.grad, rtol, atol)
    _bound_check("dh", h.grad, hr.grad, rtol, atol)
    _bound_check("dw", w.grad, wr.grad, rtol, atol, normwise=True)


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [1000, 1003, 50280])
def test_cross_entropy(vocab):
    print(f"case cross_entropy vocab={vocab}", flush=True)
    rows = 37
    g = torch.Generator().manual_seed(vocab)
    z = (3 * torch.randn(rows, vocab, generator=g)).to(torch.bfloat16)
    tg = torch.randint(0, vocab, (rows,), generator=g)
    zc = z.cuda().requires_grad_(True)
    loss = cross_entropy(zc, tg.cuda())
    (2.5 * loss).backward()
    torch.cuda.synchronize()
    zr = z.double().requires_grad_(True)
    lr = F.cross_entropy(zr, tg)
    (2.5 * lr).backward()
    assert abs(loss.item() - lr.item()) <= 1e-5 * abs(lr.item()) + 1e-5
    # gradients are rounded to bf16 once
    _bound_check("dlogits", zc.grad.float(), zr.grad, 1e-2, 1e-5 * 2.5 / rows)


@pytest.mark.gpu
def test_cross_entropy_bad_target_is_nan():
    z = torch.randn(4, 64, dtype=torch.bfloat16, device="cuda")
    loss = cross_entropy(z, torch.tensor([0, 1, 64, 2], device="cuda"))
    assert torch.isnan(loss).item()


@pytest.mark.gpu
@pytest.mark.parametrize("vocab,rows", [(50280, 64), (1000, 37), (65536, 5), (8, 3)])
def test_cross_entropy_one_pass_matches_two_pass(vocab, rows):
    """The one-pass loss + gradient (a loss that will be differentiated, upstream gradient 1:
    the backward leaves the stored gradient as it is) against the two-pass kernels on the same
    logits: losses within float32 rounding of the row sums, gradients within one bf16 step of
    the value (both are one rounding of the same softmax); against float64 torch as above."""
    print(f"case cross_entropy one pass vocab={vocab} rows={rows}", flush=True)
    g = torch.Generator().manual_seed(vocab + rows)
    z = (3 * torch.randn(rows, vocab, generator=g)).to(torch.bfloat16).cuda()
    tg = torch.randint(0, vocab, (rows,), generator=g).cuda()
    z1 = z.clone().requires_grad_(True)
    l1 = cross_entropy(z1, tg)  # one pass
    l1.backward()
    z2 = z.clone().requires_grad_(True)
    l2 = _CrossEntropy.apply(z2, tg)  # two passes
    l2.backward()
    torch.cuda.synchronize()
    assert abs(l1.item() - l2.item()) <= 1e-6 * abs(l2.item())
    d1, d2 = z1.grad.float(), z2.grad.float()
    assert bool(((d1 - d2).abs() <= 2.0 ** -7 * d2.abs() + 1e-12).all())
    zr = z.cpu().double().requires_grad_(True)
    F.cross_entropy(zr, tg.cpu()).backward()
    _bound_check("dlogits", d1, zr.grad, 1e-2, 1e-5 / rows)


@pytest.mark.gpu
def test_cross_entropy_one_pass_bad_target_is_nan():
    z = torch.randn(4, 64, dtype=torch.bfloat16, device="cuda", requires_grad=True)
    loss = cross_entropy(z, torch.tensor([0, 1, 64, 2], device="cuda"))
    assert torch.isnan(loss).item()
