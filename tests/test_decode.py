"""Single-token recurrent step (decode): S6.step / Mamba.step (mamba/mamba1.py:200-214,
339-363) as HIP kernels, and the model's prefill + step against its own full forward.

CPU: argument validation. GPU: T sequential steps of selective_state_update against the
float64 oracle scan over the same T steps from the same initial state (fp32 within rtol
1e-4 / atol 1e-5), causal_conv1d_update against the oracle conv of [prefix, x], and
MambaLM.prefill + step logits against MambaLM.forward logits on the whole sequence.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mamba_amd import _lib
from mamba_amd import decode
from mamba_amd.decode import (causal_conv1d_update, gemv, gemv_conv_update, gemv_state_update,
                              norm_gemv_conv_update, selective_state_update)
from mamba_amd.lm_ops import add_rmsnorm
from mamba_amd.mamba1 import MambaLM
from oracle import mamba1_torch as ref
from oracle import cscan64, scan64


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


@pytest.mark.parametrize("kw,status", [
    (dict(dstate=17), _lib.MSS_ERR_UNSUPPORTED), (dict(dstate=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(state=None), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(out=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(discretization=3), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(batch=0), _lib.MSS_ERR_INVALID_ARGUMENT),
])
def test_step_validation(lib, kw, status):
    base = dict(batch=2, dim=3, dstate=4, state=1, u=1, delta=1, A=1, B=1, C=1, out=1)
    base.update(kw)
    assert lib.mss_scan_step(_lib.StepArgs(**base), None) == status
    # complex step: same checks, with 8-byte aligned A and state
    base.update(state=64 if base["state"] else None, A=64)
    assert lib.mss_cscan_step(_lib.StepArgs(**base), None) == status


@pytest.mark.parametrize("kw", [dict(state=68), dict(A=4)])
def test_complex_step_alignment(lib, kw):
    base = dict(batch=2, dim=3, dstate=4, state=64, u=64, delta=64, A=64, B=64, C=64, out=64)
    base.update(kw)
    assert lib.mss_cscan_step(_lib.StepArgs(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("kw", [dict(width=0), dict(width=5), dict(conv_state=None), dict(x=None),
                                dict(activation=2)])
def test_conv_step_validation(lib, kw):
    base = dict(batch=2, dim=3, width=4, activation=1, conv_state=1, x=1, weight=1, y=1)
    base.update(kw)
    assert lib.mss_conv_step(_lib.ConvStepArgs(**base), None) == _lib.MSS_ERR_INVALID_ARGUMENT


@pytest.mark.gpu
@pytest.mark.parametrize("zoh", [False, True])
@pytest.mark.parametrize("layout", ["bd", "db"])
def test_state_update_steps_match_oracle_scan(zoh, layout):
    print(f"case state update zoh={zoh} layout={layout}", flush=True)
    rng = np.random.default_rng(11)
    b, d, n, steps = 3, 40, 16, 6
    f = np.float32
    u = rng.standard_normal((b, d, steps)).astype(f)
    dr = rng.standard_normal((b, d, steps)).astype(f)
    z = rng.standard_normal((b, d, steps)).astype(f)
    Bm = rng.standard_normal((b, n, steps)).astype(f)
    Cm = rng.standard_normal((b, n, steps)).astype(f)
    A = (-np.exp(rng.standard_normal((d, n)))).astype(f)
    D = rng.standard_normal(d).astype(f)
    bias = (0.5 * rng.standard_normal(d) - 2.0).astype(f)
    x0 = rng.standard_normal((b, d, n)).astype(f)
    fw = scan64.forward(u, dr, A, Bm, Cm, D=D, z=z, delta_bias=bias, delta_softplus=True, initial_state=x0,
                        discretization="zoh" if zoh else "euler")
    state = torch.from_numpy(x0).cuda()
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    for t in range(steps):
        if layout == "db":  # (dim, batch) activation matrices, as the LM's decode uses them
            ut, dt, zt = (cu(a[:, :, t].T).t() for a in (u, dr, z))
            Bt, Ct = cu(Bm[:, :, t].T).t(), cu(Cm[:, :, t].T).t()
        else:
            ut, dt, zt = (cu(a[:, :, t]) for a in (u, dr, z))
            Bt, Ct = cu(Bm[:, :, t]), cu(Cm[:, :, t])
        out = selective_state_update(state, ut, dt, cu(A), Bt, Ct, D=cu(D), z=zt, delta_bias=cu(bias),
                                     discretization="zoh" if zoh else "euler")
        torch.testing.assert_close(out.double().cpu(), torch.from_numpy(fw["out"][:, :, t]), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state.double().cpu(), torch.from_numpy(fw["last_state"]), rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("zoh", [False, True])
def test_complex_state_update_steps_match_oracle_scan(zoh):
    print(f"case complex state update zoh={zoh}", flush=True)
    rng = np.random.default_rng(12)
    b, d, n, steps = 3, 40, 16, 6
    f = np.float32
    u, dr, z = (rng.standard_normal((b, d, steps)).astype(f) for _ in range(3))
    Bm, Cm = (rng.standard_normal((b, n, steps)).astype(f) for _ in range(2))
    A = (-np.exp(rng.standard_normal((d, n))) + 2j * rng.standard_normal((d, n))).astype(np.complex64)
    D = rng.standard_normal(d).astype(f)
    bias = (0.5 * rng.standard_normal(d) - 2.0).astype(f)
    x0 = (rng.standard_normal((b, d, n)) + 1j * rng.standard_normal((b, d, n))).astype(np.complex64)
    fw = cscan64.forward(u, dr, A, Bm, Cm, D=D, z=z, delta_bias=bias, delta_softplus=True, initial_state=x0,
                         discretization="zoh" if zoh else "euler")
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    state = cu(x0)
    for t in range(steps):
        out = selective_state_update(state, cu(u[:, :, t]), cu(dr[:, :, t]), cu(A), cu(Bm[:, :, t]),
                                     cu(Cm[:, :, t]), D=cu(D), z=cu(z[:, :, t]), delta_bias=cu(bias),
                                     discretization="zoh" if zoh else "euler")
        torch.testing.assert_close(out.double().cpu(), torch.from_numpy(fw["out"][:, :, t]), rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state.cpu().to(torch.complex128), torch.from_numpy(fw["last_state"]),
                               rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("k", [2, 4])
def test_conv_update_matches_full_conv(k):
    print(f"case conv update k={k}", flush=True)
    g = torch.Generator().manual_seed(k)
    b, d, prefix, steps = 2, 24, 9, 5
    x = torch.randn(b, prefix + steps, d, generator=g, dtype=torch.float64)
    w = torch.randn(d, k, generator=g, dtype=torch.float64)
    bias = torch.randn(d, generator=g, dtype=torch.float64)
    want = F.silu(ref.causal_depthwise_conv(x, w, bias))
    state = x[:, prefix - (k - 1):prefix, :].permute(0, 2, 1).contiguous().float().cuda()
    for t in range(steps):
        y = causal_conv1d_update(state, x[:, prefix + t, :].float().cuda(), w.float().cuda(), bias.float().cuda())
        torch.testing.assert_close(y.double().cpu(), want[:, prefix + t, :], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("euler,complex_ssm", [(True, False), (False, False), (True, True), (False, True)])
def test_prefill_and_steps_match_full_forward(euler, complex_ssm):
    print(f"case prefill + steps euler={euler} complex_ssm={complex_ssm}", flush=True)
    torch.manual_seed(5)
    model = MambaLM(16, 64, 2, 2, 16, None, 4, use_euler_barB_approx=euler, complex_ssm=complex_ssm,
                    device="cuda")
    g = torch.Generator().manual_seed(6)
    b, prompt, steps = 3, 37, 6
    tokens = torch.randint(0, 16, (b, prompt + steps), generator=g).cuda()
    with torch.no_grad():
        full = model(tokens, act_dtype=torch.float32).view(b, prompt + steps, -1)
    last, caches = model.prefill(tokens[:, :prompt], act_dtype=torch.float32)
    torch.testing.assert_close(last, full[:, prompt - 1], rtol=1e-4, atol=1e-4)
    for t in range(steps):
        logits = model.step(tokens[:, prompt + t], caches, act_dtype=torch.float32)
        torch.testing.assert_close(logits, full[:, prompt + t], rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
def test_prefill_and_steps_bf16_match_full_forward():
    """The bf16 decode path (shadow weights; in_proj and z_proj as one GEMM) against the
    bf16 full forward: the same bf16 GEMMs and activations, the scan run chunked in one and
    one token at a time in the other (float32 states in both), so logits agree to a few
    bf16 roundings of their scale."""
    print("case prefill + steps bf16", flush=True)
    torch.manual_seed(5)
    model = MambaLM(16, 64, 2, 2, 16, None, 4, device="cuda")
    g = torch.Generator().manual_seed(7)
    b, prompt, steps = 3, 37, 6
    tokens = torch.randint(0, 16, (b, prompt + steps), generator=g).cuda()
    with torch.no_grad():
        full = model(tokens, act_dtype=torch.bfloat16).view(b, prompt + steps, -1).float()
    last, caches = model.prefill(tokens[:, :prompt], act_dtype=torch.bfloat16)
    scale = full.abs().max().item()
    assert (last.float() - full[:, prompt - 1]).abs().max().item() <= 3e-2 * scale
    for t in range(steps):
        logits = model.step(tokens[:, prompt + t], caches, act_dtype=torch.bfloat16).float()
        err = (logits - full[:, prompt + t]).abs().max().item()
        print(f"  step {t}: max abs err {err:.3e} (logit scale {scale:.3e})", flush=True)
        assert err <= 3e-2 * scale


@pytest.mark.gpu
def test_prefill_and_steps_bf16_at_config5_widths():
    """The bf16 decode path at the 130M model's widths (d_model 768, d_inner 1536, dt_rank
    48, vocab 50280, batch 8; two of its 24 layers), so the fused norm + in-projection +
    conv kernel, the x / dt+state / out GEMVs and the 50280-row head run at their real
    shapes: decode logits against the bf16 full forward over the same tokens, as above."""
    print("case prefill + steps bf16 at config-5 widths", flush=True)
    torch.manual_seed(11)
    model = MambaLM(50280, 768, 2, 2, 16, 48, 4, device="cuda")
    g = torch.Generator().manual_seed(12)
    b, prompt, steps = 8, 61, 4
    tokens = torch.randint(0, 50280, (b, prompt + steps), generator=g).cuda()
    with torch.no_grad():
        full = model(tokens, act_dtype=torch.bfloat16).view(b, prompt + steps, -1).float()
    last, caches = model.prefill(tokens[:, :prompt], act_dtype=torch.bfloat16)
    scale = full.abs().max().item()
    assert (last.float() - full[:, prompt - 1]).abs().max().item() <= 3e-2 * scale
    for t in range(steps):
        logits = model.step(tokens[:, prompt + t], caches, act_dtype=torch.bfloat16).float()
        err = (logits - full[:, prompt + t]).abs().max().item()
        print(f"  step {t}: max abs err {err:.3e} (logit scale {scale:.3e})", flush=True)
        assert torch.isfinite(logits).all()
        assert err <= 3e-2 * scale


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(3072, 768, 8), (768, 1536, 8), (80, 1536, 8), (1536, 48, 8),
                                   (300, 4096, 4), (5000, 2560, 2), (40, 2056, 8),
                                   (4099, 768, 4), (5, 8, 1), (257, 136, 2), (4100, 768, 8),
                                   (50280, 768, 8), (4096, 64, 1),
                                   (64, 1024, 1), (200, 1600, 2), (1023, 2048, 4)])
def test_gemv_matches_float32_product(m, k, n):
    """The decode-shaped GEMM against the float32 product of the same bf16 operands: each
    output is one float32 sum over K rounded to bf16 once, so it sits within a bf16
    rounding (plus float32 reordering) of the reference."""
    print(f"case gemv M={m} K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(m + k + n)
    w = torch.randn(m, k, generator=g).to(torch.bfloat16).cuda()
    x = torch.randn(k, n, generator=g).to(torch.bfloat16).cuda()
    y = gemv(w, x)
    torch.cuda.synchronize()
    ref = w.float() @ x.float()
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    err = (y.float() - ref).abs()
    bound = 2.0 ** -8 * ref.abs() + 1e-3 * (k ** 0.5)
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"


def test_gemv_validation(lib):
    ok = dict(M=4, K=8, N=8, ldw=8, W=16, X=16, Y=16)
    assert lib.mss_gemv(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    for kw, status in ((dict(K=12), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(N=3), _lib.MSS_ERR_UNSUPPORTED),
                       (dict(K=8192, ldw=8192), _lib.MSS_ERR_UNSUPPORTED), (dict(X=8), _lib.MSS_ERR_INVALID_ARGUMENT),
                       (dict(ldw=4), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(W=8), _lib.MSS_ERR_INVALID_ARGUMENT),
                       (dict(M=0), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(Y=None), _lib.MSS_ERR_INVALID_ARGUMENT)):
        a = dict(ok, **kw)
        assert lib.mss_gemv(_lib.GemvArgs(**a), None) == status, kw


def test_fused_step_validation(lib):
    """mss_gemv_conv_step / mss_gemv_scan_step check their shapes against each other (CPU,
    invalid arguments only: nothing is launched)."""
    g = _lib.GemvArgs(M=32, K=8, N=4, ldw=8, W=16, X=16, Y=16)
    conv = dict(batch=4, dim=16, width=4, io_dtype=_lib.MSS_BF16, activation=1, conv_state=16, x=None,
                weight=16, bias=None, y=16)
    assert lib.mss_gemv_conv_step(None, _lib.ConvStepArgs(**conv), None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_gemv_conv_step(g, None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    for kw in (dict(batch=2), dict(dim=33), dict(io_dtype=_lib.MSS_F32), dict(y=None), dict(width=5)):
        assert lib.mss_gemv_conv_step(g, _lib.ConvStepArgs(**dict(conv, **kw)), None) == \
            _lib.MSS_ERR_INVALID_ARGUMENT, kw
    # Y is needed for the rows past the conv's
    g_noy = _lib.GemvArgs(M=32, K=8, N=4, ldw=8, W=16, X=16, Y=None)
    assert lib.mss_gemv_conv_step(g_noy, _lib.ConvStepArgs(**conv), None) == _lib.MSS_ERR_INVALID_ARGUMENT
    step = dict(batch=4, dim=32, dstate=16, discretization=_lib.MSS_EULER, delta_softplus=1,
                io_dtype=_lib.MSS_BF16, bc_dtype=_lib.MSS_BF16, state=16, u=16, delta=None, A=16, B=16, C=16,
                out=16)
    assert lib.mss_gemv_scan_step(g, None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    for kw in (dict(batch=8), dict(dim=16), dict(io_dtype=_lib.MSS_F32), dict(bc_dtype=_lib.MSS_F32),
               dict(out=None), dict(discretization=7)):
        assert lib.mss_gemv_scan_step(g, _lib.StepArgs(**dict(step, **kw)), None) == \
            _lib.MSS_ERR_INVALID_ARGUMENT, kw
    assert lib.mss_gemv_scan_step(g, _lib.StepArgs(**dict(step, dstate=17)), None) == _lib.MSS_ERR_UNSUPPORTED
    assert lib.mss_gemv_scan_step(_lib.GemvArgs(M=32, K=8, N=3, ldw=8, W=16, X=16), _lib.StepArgs(**step),
                                  None) == _lib.MSS_ERR_UNSUPPORTED


def test_norm_gemv_conv_step_validation(lib):
    """mss_norm_gemv_conv_step checks the norm against the GEMM and the stream buffers
    against each other (CPU, invalid arguments only: nothing is launched)."""
    g = _lib.GemvArgs(M=32, K=64, N=4, ldw=64, W=16, X=None, Y=16)
    conv = _lib.ConvStepArgs(batch=4, dim=16, width=4, io_dtype=_lib.MSS_BF16, activation=1, conv_state=16,
                             weight=16, y=16)
    stream = 64 * 4 * 4  # bytes of the float32 (64, 4) stream
    norm = dict(features=64, tokens=4, eps=1e-5, io_dtype=_lib.MSS_BF16, h=1 << 20, delta=2 << 20, weight=16,
                hn=3 << 20)
    assert lib.mss_norm_gemv_conv_step(None, g, conv, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_norm_gemv_conv_step(_lib.NormArgs(**norm), None, conv, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_norm_gemv_conv_step(_lib.NormArgs(**norm), g, None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    for kw in (dict(features=72), dict(tokens=2), dict(io_dtype=_lib.MSS_F32), dict(eps=-1.0), dict(h=None),
               dict(weight=None), dict(hn=None), dict(h=(1 << 20) + 8), dict(delta=(2 << 20) + 8),
               dict(hn=(1 << 20) + stream - 16), dict(hn=(2 << 20) - stream + 16), dict(hn=(2 << 20) + 64)):
        assert lib.mss_norm_gemv_conv_step(_lib.NormArgs(**dict(norm, **kw)), g, conv, None) == \
            _lib.MSS_ERR_INVALID_ARGUMENT, kw
    big = _lib.GemvArgs(M=32, K=1032, N=4, ldw=1032, W=16, X=None, Y=16)
    assert lib.mss_norm_gemv_conv_step(_lib.NormArgs(**dict(norm, features=1032)), big, conv, None) == \
        _lib.MSS_ERR_UNSUPPORTED


def _bf16(*shape, scale=1.0, device="cuda"):
    return (torch.randn(*shape, device=device) * scale).to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 2, 4, 8])
@pytest.mark.parametrize("k,act,extra", [(4, "silu", 96), (2, None, 0), (1, "silu", 8), (3, "silu", 40)])
def test_gemv_conv_update_matches_separate_calls(n, k, act, extra):
    """GEMM + fused conv window step == gemv then causal_conv1d_update, bit for bit, over
    three steps in a row (the window state carries between them)."""
    torch.manual_seed(n * 10 + k)
    dim, kin = 200, 136
    w = _bf16(dim + extra, kin, scale=kin ** -0.5)
    weight = torch.randn(dim, k, device="cuda") * 0.5
    bias = torch.randn(dim, device="cuda") * 0.1 if act else None
    s_fused = _bf16(n, dim, k - 1)
    s_ref = s_fused.clone()
    for _ in range(3):
        x = _bf16(kin, n)
        v = gemv(w, x)
        u_ref = causal_conv1d_update(s_ref, v[:dim].t(), weight, bias, act or "none").t()
        u, rest = gemv_conv_update(w, x, s_fused, weight, bias, act or "none")
        assert tuple(u.shape) == (dim, n) and tuple(rest.shape) == (extra, n)
        assert torch.equal(u, u_ref)
        assert torch.equal(rest, v[dim:])
        assert torch.equal(s_fused, s_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 2, 4, 8])
def test_gemv_conv_update_matrix_core_shape(n):
    """The 130M in-projection's shape (M = 3072 rows [x; z], K = 768, K % 64 == 0): the
    conv-fused GEMM sums on the matrix cores, in another order than the plain decode GEMM of
    3072 rows, so its bf16 rows may differ from mss_gemv's by one rounding of the float32 sum.
    With the z rows a copy of the x rows, the z rows the fused call writes are the very rows
    its conv step consumed: the conv window step applied to them by the separate call gives
    the fused u and window state bit for bit, over three steps in a row; and every fused row
    is within one bf16 rounding of mss_gemv's."""
    torch.manual_seed(70 + n)
    dim, kin = 1536, 768
    wx = _bf16(dim, kin, scale=kin ** -0.5)
    w = torch.cat([wx, wx]).contiguous()
    weight = torch.randn(dim, 4, device="cuda") * 0.5
    bias = torch.randn(dim, device="cuda") * 0.1
    s_fused = _bf16(n, dim, 3)
    s_ref = s_fused.clone()
    for _ in range(3):
        x = _bf16(kin, n)
        u, rest = gemv_conv_update(w, x, s_fused, weight, bias, "silu")
        u_ref = causal_conv1d_update(s_ref, rest.t(), weight, bias, "silu").t()
        assert torch.equal(u, u_ref)
        assert torch.equal(s_fused, s_ref)
        v = gemv(w, x)[dim:].float()
        ulp = torch.exp2(torch.floor(torch.log2(v.abs().clamp_min(1e-30))) - 7)
        assert bool(torch.all((rest.float() - v).abs() <= ulp)), float(((rest.float() - v).abs() / ulp).max())


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 2, 4, 8])
@pytest.mark.parametrize("zoh,with_dz,dstate", [(False, True, 16), (True, True, 16), (False, False, 5),
                                                (True, False, 11)])
def test_gemv_state_update_matches_separate_calls(n, zoh, with_dz, dstate):
    """dt GEMM + fused selective-state step == gemv then selective_state_update, bit for
    bit, over three steps in a row (the state carries between them), with the model's
    (features, batch) activation layouts."""
    torch.manual_seed(n * 100 + dstate)
    dim, rank = 160, 48
    disc = "zoh" if zoh else "euler"
    w = _bf16(dim, rank, scale=rank ** -0.5)
    A = -torch.rand(dim, dstate, device="cuda") * 4 - 0.1
    D = torch.randn(dim, device="cuda") if with_dz else None
    bias = torch.randn(dim, device="cuda") * 0.5 if with_dz else None
    st_fused = torch.randn(n, dim, dstate, device="cuda")
    st_ref = st_fused.clone()
    for _ in range(3):
        x = _bf16(rank, n)
        u = _bf16(dim, n)
        z = _bf16(dim, n) if with_dz else None
        bc = _bf16(2 * dstate, n)
        Bt, Ct = bc[:dstate].t(), bc[dstate:].t()
        dt = gemv(w, x)
        y_ref = selective_state_update(st_ref, u.t(), dt.t(), A, Bt, Ct, D, None if z is None else z.t(), bias,
                                       True, disc)
        y = gemv_state_update(w, x, st_fused, u.t(), A, Bt, Ct, D, None if z is None else z.t(), bias, True,
                              disc)
        assert torch.equal(y, y_ref)
        assert torch.equal(st_fused, st_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 2, 4, 8])
@pytest.mark.parametrize("f,with_delta,extra", [(768, True, 1536), (136, True, 40), (1024, False, 8),
                                                (520, True, 0)])
def test_norm_gemv_conv_update_matches_separate_calls(monkeypatch, lib, n, f, with_delta, extra):
    """Residual add + RMSNorm + GEMM + conv window step as one kernel == add_rmsnorm then
    gemv_conv_update, bit for bit (the new stream hn, the conv output, the rows past the
    conv's, the window state, rstd), over three steps in a row; f = 768 is the 130M
    model's d_model (with its 2 x 1536 in/z rows)."""
    print(f"case norm+gemv+conv N={n} features={f} delta={with_delta} extra={extra}", flush=True)
    torch.manual_seed(f + n)
    dim = 96 if extra != 1536 else 1536
    w = _bf16(dim + extra, f, scale=f ** -0.5)
    weight = torch.randn(dim, 4, device="cuda") * 0.5
    bias = torch.randn(dim, device="cuda") * 0.1
    nw = torch.rand(f, device="cuda") + 0.5
    s_fused = _bf16(n, dim, 3)
    s_ref = s_fused.clone()
    for it in range(3):
        h = torch.randn(f, n, device="cuda") * 2
        delta = _bf16(f, n) if with_delta else None
        hn_ref, x = add_rmsnorm(h, delta, nw, 1e-5, torch.bfloat16)
        u_ref, rest_ref = gemv_conv_update(w, x, s_ref, weight, bias)
        with monkeypatch.context() as m:  # the fused kernel, not the fallback's two calls
            m.setattr(decode, "add_rmsnorm", None)
            hn, u, rest = norm_gemv_conv_update(h, delta, nw, 1e-5, w, s_fused, weight, bias)
        assert torch.equal(hn, hn_ref)
        assert torch.equal(u, u_ref)
        assert torch.equal(rest, rest_ref)
        assert torch.equal(s_fused, s_ref)
        if it == 0:  # rstd through the C entry point, against mss_norm_fwd's
            rstd_ref = torch.empty(n, device="cuda")
            xr = torch.empty(f, n, dtype=torch.bfloat16, device="cuda")
            hn2 = torch.empty_like(h)
            na = _lib.NormArgs(features=f, tokens=n, eps=1e-5, io_dtype=_lib.MSS_BF16, h=h.data_ptr(),
                               delta=None if delta is None else delta.data_ptr(), weight=nw.data_ptr(),
                               hn=hn2.data_ptr(), x=xr.data_ptr(), rstd=rstd_ref.data_ptr())
            assert lib.mss_norm_fwd(na, None) == _lib.MSS_OK
            rstd = torch.full((n,), -1.0, device="cuda")
            st = s_fused.clone()
            u2 = torch.empty(dim, n, dtype=torch.bfloat16, device="cuda")
            v2 = torch.empty(dim + extra, n, dtype=torch.bfloat16, device="cuda")
            ca, keep = decode._conv_step_args(st, u2.t(), weight, bias, "silu", u2.t())
            ca.x = None
            na.x, na.rstd, na.hn = None, rstd.data_ptr(), hn2.data_ptr()
            g = _lib.GemvArgs(M=dim + extra, K=f, N=n, ldw=f, W=w.data_ptr(), X=None, Y=v2.data_ptr())
            assert lib.mss_norm_gemv_conv_step(na, g, ca, None) == _lib.MSS_OK
            torch.cuda.synchronize()
            assert torch.equal(rstd, rstd_ref)
            assert torch.equal(xr, x)
