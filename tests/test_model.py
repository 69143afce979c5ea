"""Mamba-1 model plumbing around the scan (callers: mamba/mamba1.py:160-198, 300-337).

CPU: the model oracle's pieces against independent routines (torch conv1d, torch
rms_norm, the float64 scan oracle with its fused extras) and the parameter initialisation.
GPU: the channel-major ``MambaLM`` (HIP scan) against the oracle model in float64 on the
CPU with the same weights, at the reference's CPU-plumbing shape (config 1: 2 layers,
d_model 64, expand 2, N 16, d_conv 4, RMSNorm, tied embeddings, vocab 16, B 8, L 256).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mamba_amd import _lib
from mamba_amd.mamba1 import GraphedTrainStep, MambaLM
from mamba_amd.optim import AdamW
from oracle import mamba1_torch as ref
from oracle import cscan64, scan64

C1 = dict(vocab=16, d_model=64, n_layers=2, expand=2, d_state=16, d_conv=4, batch=8, length=256)
# Config 5: the Mamba-1 130M shape.
C5 = dict(vocab=50280, d_model=768, n_layers=24, expand=2, d_state=16, dt_rank=48, d_conv=4, batch=8,
          length=2048)


def test_oracle_conv_matches_torch_conv1d():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 50, 6, generator=g, dtype=torch.float64)
    w = torch.randn(6, 4, generator=g, dtype=torch.float64)
    b = torch.randn(6, generator=g, dtype=torch.float64)
    got = ref.causal_depthwise_conv(x, w, b)
    want = F.conv1d(F.pad(x.transpose(1, 2), (3, 0)), w[:, None, :], b, groups=6).transpose(1, 2)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    # causality: changing x at step t leaves outputs before t unchanged
    x2 = x.clone()
    x2[:, 20] += 1.0
    assert torch.equal(ref.causal_depthwise_conv(x2, w, b)[:, :20], got[:, :20])


def test_oracle_rmsnorm_matches_torch():
    x = torch.randn(4, 9, 32, dtype=torch.float64)
    w = torch.randn(32, dtype=torch.float64)
    torch.testing.assert_close(ref.rmsnorm(x, w), F.rms_norm(x, (32,), w, eps=1e-5))


def small_params(d_model=8, expand=2, d_state=4, dt_rank=2, vocab=11, n_layers=2, seed=0, complex_ssm=False):
    torch.manual_seed(seed)
    m = MambaLM(vocab, d_model, n_layers, expand, d_state, dt_rank, 4, complex_ssm=complex_ssm)
    return {k: v.detach().double() for k, v in m.state_dict().items()}, m


@pytest.mark.parametrize("euler", [True, False])
def test_oracle_s6_matches_scan64(euler):
    p, _ = small_params()
    pre = "blocks.0.s6."
    rng = np.random.default_rng(1)
    u = torch.from_numpy(rng.standard_normal((2, 30, 16)))
    got = ref.s6(p, pre, u, 2, 4, euler)
    x_dbl = (u @ p[pre + "x_proj"].t()).numpy()
    dt_raw = x_dbl[..., :2] @ p[pre + "dt_proj"].t().numpy()
    sw = lambda a: np.ascontiguousarray(np.swapaxes(a, 1, 2))
    fw = scan64.forward(sw(u.numpy()), sw(dt_raw), -np.exp(p[pre + "A_log"].numpy()), sw(x_dbl[..., 2:6]),
                        sw(x_dbl[..., 6:]), D=p[pre + "D"].numpy(), delta_bias=p[pre + "dt_bias"].numpy(),
                        delta_softplus=True, discretization="euler" if euler else "zoh")
    np.testing.assert_allclose(got.numpy(), np.swapaxes(fw["out"], 1, 2), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("euler", [True, False])
def test_oracle_seq_scan_matches_associative_scan(euler):
    """The oracle model's sequential-scan option (the C oracle's recurrence and adjoint) against
    its associative scan under torch autograd: outputs and every parameter gradient."""
    p, _ = small_params()
    pre = "blocks.0.s6."
    rng = np.random.default_rng(4)
    u0 = torch.from_numpy(rng.standard_normal((2, 40, 16)))
    w = torch.from_numpy(rng.standard_normal((2, 40, 16)))
    outs = []
    for seq in (False, True):
        q = {k: v.clone().requires_grad_(True) for k, v in p.items()}
        u = u0.clone().requires_grad_(True)
        y = ref.s6(q, pre, u, 2, 4, euler, seq_scan=seq)
        (y * w).sum().backward()
        outs.append((y.detach(), u.grad, {k: v.grad for k, v in q.items() if v.grad is not None}))
    torch.testing.assert_close(outs[1][0], outs[0][0], rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(outs[1][1], outs[0][1], rtol=1e-9, atol=1e-11)
    assert outs[1][2].keys() == outs[0][2].keys()
    for k in outs[0][2]:
        torch.testing.assert_close(outs[1][2][k], outs[0][2][k], rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("euler", [True, False])
def test_oracle_complex_s6_matches_cscan64(euler):
    """The oracle model's complex branch (associative scan, mamba/mamba1.py:170-176) against the
    sequential complex oracle, with the reference's complex A initialisation perturbed."""
    p, _ = small_params(complex_ssm=True)
    pre = "blocks.0.s6."
    rng = np.random.default_rng(3)
    p[pre + "A_imag"] = p[pre + "A_imag"] + torch.from_numpy(rng.standard_normal(p[pre + "A_imag"].shape))
    u = torch.from_numpy(rng.standard_normal((2, 30, 16)))
    got = ref.s6(p, pre, u, 2, 4, euler)
    x_dbl = (u @ p[pre + "x_proj"].t()).numpy()
    dt_raw = x_dbl[..., :2] @ p[pre + "dt_proj"].t().numpy()
    sw = lambda a: np.ascontiguousarray(np.swapaxes(a, 1, 2))
    A = -np.exp(p[pre + "A_log"].numpy()) + 1j * p[pre + "A_imag"].numpy()
    fw = cscan64.forward(sw(u.numpy()), sw(dt_raw), A, sw(x_dbl[..., 2:6]), sw(x_dbl[..., 6:]),
                         D=p[pre + "D"].numpy(), delta_bias=p[pre + "dt_bias"].numpy(),
                         delta_softplus=True, discretization="euler" if euler else "zoh")
    np.testing.assert_allclose(got.numpy(), np.swapaxes(fw["out"], 1, 2), rtol=1e-9, atol=1e-12)


def test_complex_parameter_initialisation_follows_reference():
    """A_log + i A_imag = log(1/2 - i n), n = 0..N-1 (mamba/mamba1.py:47), so
    A = -exp(A_log) + i A_imag = -|1/2 - i n| + i atan2(-n, 1/2) (:162)."""
    _, m = small_params(d_model=16, d_state=16, complex_ssm=True)
    a = m.blocks[1].s6.a_matrix().detach()
    assert a.dtype == torch.complex64 and a.shape == (32, 16)
    n = np.arange(16)
    want = -np.sqrt(0.25 + n ** 2) + 1j * np.arctan2(-n, 0.5)
    np.testing.assert_allclose(a[5].numpy(), want, rtol=1e-6)


def test_oracle_block_gate_matches_scan64_gate():
    p, _ = small_params()
    pre = "blocks.1."
    rng = np.random.default_rng(2)
    h = torch.from_numpy(rng.standard_normal((2, 25, 8)))
    got = ref.mamba_block(p, pre, h, 2, 4)
    x = ref.rmsnorm(h, p[pre + "norm.weight"])
    u = F.silu(ref.causal_depthwise_conv(x @ p[pre + "in_proj"].t(), p[pre + "conv_weight"], p[pre + "conv_bias"]))
    z = x @ p[pre + "z_proj"].t()
    s = pre + "s6."
    x_dbl = (u @ p[s + "x_proj"].t()).numpy()
    sw = lambda a: np.ascontiguousarray(np.swapaxes(np.asarray(a), 1, 2))
    fw = scan64.forward(sw(u.numpy()), sw(x_dbl[..., :2] @ p[s + "dt_proj"].t().numpy()),
                        -np.exp(p[s + "A_log"].numpy()), sw(x_dbl[..., 2:6]), sw(x_dbl[..., 6:]),
                        D=p[s + "D"].numpy(), z=sw(z.numpy()), delta_bias=p[s + "dt_bias"].numpy(),
                        delta_softplus=True)
    want = np.swapaxes(fw["out"], 1, 2) @ p[pre + "out_proj"].t().numpy() + h.numpy()
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-9, atol=1e-12)


def test_parameter_initialisation_follows_reference():
    _, m = small_params(d_model=64, d_state=16, dt_rank=None)
    s6 = m.blocks[0].s6
    assert s6.dt_rank == 4  # from d_model: ceil(64 / 16) (mamba/mamba1.py:228-231)
    torch.testing.assert_close(-torch.exp(s6.A_log[3]), -torch.arange(1, 17, dtype=torch.float32))
    dt = F.softplus(s6.dt_bias.detach())
    assert float(dt.min()) >= 1e-4 * 0.999 and float(dt.max()) <= 0.1 * 1.001
    assert torch.equal(s6.D.detach(), torch.ones(128))


@pytest.mark.gpu
@pytest.mark.parametrize("euler,complex_ssm", [(True, False), (False, False), (True, True), (False, True)])
def test_model_matches_oracle_on_gpu(euler, complex_ssm):
    print(f"case model c1 euler={euler} complex_ssm={complex_ssm}", flush=True)
    torch.manual_seed(0)
    cfg = C1
    dev = "cuda"
    model = MambaLM(cfg["vocab"], cfg["d_model"], cfg["n_layers"], cfg["expand"], cfg["d_state"], None,
                    cfg["d_conv"], use_euler_barB_approx=euler, complex_ssm=complex_ssm, device=dev)
    g = torch.Generator().manual_seed(0)
    tokens = torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["length"]), generator=g)
    targets = torch.roll(tokens, -1, dims=1).reshape(-1)
    logits = model(tokens.to(dev), act_dtype=torch.float32)
    loss = F.cross_entropy(logits.float(), targets.to(dev))
    loss.backward()
    torch.cuda.synchronize()

    p = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
    dt_rank = model.blocks[0].s6.dt_rank
    ref_logits = ref.mamba_lm(p, tokens, cfg["n_layers"], dt_rank, cfg["d_state"], euler)
    ref_loss = F.cross_entropy(ref_logits, targets)
    ref_loss.backward()
    torch.testing.assert_close(logits.detach().cpu().double(), ref_logits.detach(), rtol=1e-4, atol=1e-4)
    assert abs(loss.item() - ref_loss.item()) < 1e-5
    named = dict(model.named_parameters())
    for k, v in p.items():
        got = named[k].grad.detach().cpu().double()
        scale = float(v.grad.abs().max())
        err = float((got - v.grad).abs().max())
        print(f"  grad {k:28s} max|g|={scale:.3e} max_err={err:.3e}", flush=True)
        assert err <= 1e-4 * scale + 1e-7, k  # measured <= 7e-6 of scale


@pytest.mark.gpu
def test_bf16_shadow_weights_match_per_use_casts():
    """bf16 training path: weights refreshed once into shadows vs cast at each use. Same
    bf16 weights and products, so identical logits; weight gradients differ only by the
    per-use path's final rounding of each gradient to bf16."""
    print("case model bf16 shadow weights", flush=True)
    torch.manual_seed(1)
    cfg = C1
    model = MambaLM(cfg["vocab"], cfg["d_model"], cfg["n_layers"], cfg["expand"], cfg["d_state"], None,
                    cfg["d_conv"], device="cuda")
    g = torch.Generator().manual_seed(2)
    tokens = torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["length"]), generator=g).cuda()
    targets = torch.roll(tokens, -1, dims=1).reshape(-1)
    grads = []
    logits_all = []
    for shadow in (True, False):
        model.zero_grad(set_to_none=True)
        logits = model(tokens, act_dtype=torch.bfloat16, shadow_weights=shadow)
        F.cross_entropy(logits.float(), targets).backward()
        torch.cuda.synchronize()
        logits_all.append(logits.detach())
        grads.append({k: p.grad.detach().clone() for k, p in model.named_parameters()})
    assert torch.equal(logits_all[0], logits_all[1])
    for k in grads[0]:
        a, b = grads[0][k].double(), grads[1][k].double()
        scale = float(b.abs().max()) + 1e-12
        assert float((a - b).abs().max()) <= 1e-2 * scale, k


@pytest.mark.gpu
@pytest.mark.parametrize("opt", ["torch", "mss"])
def test_graphed_train_step_matches_eager(opt):
    """The HIP-graph training step against eager steps from the same initial weights: the
    loss of every replay and the final weights agree (replays are checked one by one, with
    eager work and synchronisations between them). With torch's fused AdamW, and with
    mss_adamw (mamba_amd.optim.AdamW), which writes the bf16 shadows itself, so neither the
    eager forwards after the first nor the captured one refresh them."""
    print(f"case graphed train step opt={opt}", flush=True)
    from mamba_amd.lm_ops import cross_entropy

    cfg = dict(C1, vocab=256)
    g = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["length"] + 1), generator=g).cuda()
    inp, tgt = tokens[:, :-1].contiguous(), tokens[:, 1:].reshape(-1).contiguous()

    def make():
        torch.manual_seed(4)
        m = MambaLM(cfg["vocab"], cfg["d_model"], cfg["n_layers"], cfg["expand"], cfg["d_state"], None,
                    cfg["d_conv"], device="cuda")
        if opt == "mss":
            return m, AdamW(m.parameters(), lr=1e-3, shadows=m.shadow_weights)
        return m, torch.optim.AdamW(m.parameters(), lr=1e-3, fused=True, capturable=True)

    warm, steps = 3, 4
    m_e, o_e = make()
    eager_losses = []
    for i in range(warm + 1 + steps):
        o_e.zero_grad(set_to_none=True)
        loss = cross_entropy(m_e(inp), tgt)
        loss.backward()
        o_e.step()
        eager_losses.append(loss.item())
    m_g, o_g = make()
    # eager steps on the default stream first (as a benchmark does), dropping their
    # autograd graphs before the capture
    for _ in range(2):
        o_g.zero_grad(set_to_none=True)
        loss = cross_entropy(m_g(inp), tgt)
        loss.backward()
        o_g.step()
    del loss
    torch.cuda.synchronize()
    gs = GraphedTrainStep(m_g, o_g, cross_entropy, inp, tgt, warmup=warm - 2)
    torch.cuda.synchronize()
    # capture does not execute: replay i is step warm + i of the eager run
    graph_losses = []
    for i in range(1 + steps):
        graph_losses.append(gs.step().item())
        torch.cuda.synchronize()
        _ = (m_g.embedding.sum() * 0).item()  # eager work between replays
    print("  eager", [round(x, 5) for x in eager_losses[warm:]], flush=True)
    print("  graph", [round(x, 5) for x in graph_losses], flush=True)
    for a, b in zip(eager_losses[warm:], graph_losses):
        assert abs(a - b) <= 2e-3 * abs(a), (a, b)
    for (k, pe), pg in zip(m_e.named_parameters(), m_g.parameters()):
        scale = float(pe.detach().abs().max()) + 1e-12
        assert float((pe.detach() - pg.detach()).abs().max()) <= 2e-2 * scale, k


def _max_err_over_scale(got, want, rows=2048):
    """max |got - want| and max |want| over (R, C) tensors, in row blocks (bounded memory)."""
    err = scale = 0.0
    for i in range(0, want.shape[0], rows):
        w = want[i:i + rows]
        err = max(err, float((got[i:i + rows].double() - w).abs().max()))
        scale = max(scale, float(w.abs().max()))
    return err, scale


@pytest.mark.gpu
@pytest.mark.slow
@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_c5_widths_one_layer_matches_oracle(act):
    """One block of the config-5 model at its full widths and workload (d_model 768, d_inner
    1536, dt_rank 48, N 16, vocab 50280, B 8, L 2048): logits, loss and every parameter
    gradient against the float64 oracle model (sequential-scan option) on the CPU with the
    same weights. The layer's scan runs the 16-wave backward plan of every config-5 layer.
    f32 activations: the config-1 bars (logits 1e-4, gradients 1e-4 of each tensor's scale);
    bf16 activations (config 5's dtype: bf16 GEMM weights and activations, fp32 scan
    accumulation, fp32 master gradients): logits 1e-2 and gradients 2e-2 of scale (measured:
    at most 7e-6 and 6.2e-3)."""
    print(f"case c5 widths one layer act={act}", flush=True)
    cfg = C5
    st = _lib.Strides(io_batch=cfg["length"], io_dim=cfg["batch"] * cfg["length"], bc_batch=cfg["length"],
                      bc_state=cfg["batch"] * cfg["length"])
    assert _lib.bwd_plan(cfg["batch"], cfg["d_model"] * cfg["expand"], cfg["d_state"], cfg["length"],
                         io_bf16=act == "bf16", strides=st)[0] == 16
    torch.manual_seed(0)
    model = MambaLM(cfg["vocab"], cfg["d_model"], 1, cfg["expand"], cfg["d_state"], cfg["dt_rank"],
                    cfg["d_conv"], device="cuda")
    g = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["length"]), generator=g)
    targets = torch.roll(tokens, -1, dims=1).reshape(-1)
    adt = torch.float32 if act == "f32" else torch.bfloat16
    logits = model(tokens.cuda(), act_dtype=adt)
    loss = F.cross_entropy(logits.float(), targets.cuda())
    loss.backward()
    torch.cuda.synchronize()
    logits = logits.detach().float().cpu()
    named = {k: v.grad.detach().cpu().double() for k, v in model.named_parameters()}
    state = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    del model
    torch.cuda.empty_cache()

    p = {k: v.requires_grad_(True) for k, v in state.items()}
    ref_logits = ref.mamba_lm(p, tokens, 1, cfg["dt_rank"], cfg["d_state"], True, seq_scan=True)
    ref_loss = F.cross_entropy(ref_logits, targets)
    ref_loss.backward()
    err, scale = _max_err_over_scale(logits, ref_logits.detach())
    print(f"  logits max_err={err:.3e} max|ref|={scale:.3e} loss {loss.item():.6f} vs {ref_loss.item():.6f}",
          flush=True)
    lt, gt = (1e-4, 1e-4) if act == "f32" else (1e-2, 2e-2)
    assert err <= lt * scale + (1e-4 if act == "f32" else 0.0)
    assert abs(loss.item() - ref_loss.item()) <= (1e-5 if act == "f32" else 2e-3) * abs(ref_loss.item())
    for k, v in p.items():
        got = named[k]
        sc = float(v.grad.abs().max())
        e = float((got - v.grad).abs().max())
        print(f"  grad {k:28s} max|g|={sc:.3e} max_err={e:.3e} ratio={e / sc:.2e}", flush=True)
        assert e <= gt * sc + 1e-7, k


@pytest.mark.gpu
@pytest.mark.slow
def test_c5_full_train_step_graph_matches_eager():
    """The config-5 training step (24 layers, bf16, mss_adamw writing the bf16 shadows) at its
    workload, as the benchmark runs it: every eager step
    has a finite loss and finite, nonzero gradients, and the HIP-graph step replays the same
    losses and ends at the same weights as the eager steps (replays checked one by one)."""
    print("case c5 full train step graph vs eager", flush=True)
    from mamba_amd.lm_ops import cross_entropy

    cfg = C5
    g = torch.Generator().manual_seed(6)
    tokens = torch.randint(0, cfg["vocab"], (cfg["batch"], cfg["length"] + 1), generator=g).cuda()
    inp, tgt = tokens[:, :-1].contiguous(), tokens[:, 1:].reshape(-1).contiguous()

    def make():
        torch.manual_seed(7)
        m = MambaLM(cfg["vocab"], cfg["d_model"], cfg["n_layers"], cfg["expand"], cfg["d_state"], cfg["dt_rank"],
                    cfg["d_conv"], device="cuda")
        return m, AdamW(m.parameters(), lr=1e-3, shadows=m.shadow_weights)

    warm, steps = 3, 3
    m_e, o_e = make()
    eager_losses = []
    for i in range(warm + 1 + steps):
        o_e.zero_grad(set_to_none=True)
        loss = cross_entropy(m_e(inp), tgt)
        loss.backward()
        for k, prm in m_e.named_parameters():
            assert prm.grad is not None and bool(torch.isfinite(prm.grad).all()), (i, k)
            assert bool((prm.grad != 0).any()), (i, k)
        o_e.step()
        eager_losses.append(loss.item())
        assert np.isfinite(eager_losses[-1])
    del loss
    m_g, o_g = make()
    for _ in range(2):
        o_g.zero_grad(set_to_none=True)
        loss = cross_entropy(m_g(inp), tgt)
        loss.backward()
        o_g.step()
    del loss
    torch.cuda.synchronize()
    gs = GraphedTrainStep(m_g, o_g, cross_entropy, inp, tgt, warmup=warm - 2)
    torch.cuda.synchronize()
    graph_losses = []
    for i in range(1 + steps):
        graph_losses.append(gs.step().item())
        torch.cuda.synchronize()
        _ = (m_g.embedding.sum() * 0).item()  # eager work between replays
    print("  eager", [round(x, 5) for x in eager_losses], flush=True)
    print("  graph", [round(x, 5) for x in graph_losses], flush=True)
    assert eager_losses[0] > eager_losses[-1]
    for a, b in zip(eager_losses[warm:], graph_losses):
        assert abs(a - b) <= 2e-3 * abs(a), (a, b)
    for (k, pe), pg in zip(m_e.named_parameters(), m_g.parameters()):
        scale = float(pe.detach().abs().max()) + 1e-12
        assert float((pe.detach() - pg.detach()).abs().max()) <= 2e-2 * scale, k
