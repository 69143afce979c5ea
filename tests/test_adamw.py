"""AdamW over float32 masters in one HIP launch per step (mss_adamw, mamba_amd.optim.AdamW),
writing the bf16 shadows of the updated weights. No reference counterpart (the reference's
training uses optax, experiments/mamba_inductionheads.py:126-139); the bar is torch's own
single-tensor AdamW (the published algorithm: decoupled weight decay, bias-corrected moments)
on the same gradients: parameters within 2e-6 relative or 4e-6 lr absolute (float32 rounding
of the same operations in another order, over four steps), moments within 1e-5 relative or 1e-6 of the
tensor's largest value (a moment near zero is a difference of rounded terms), every shadow equal to
the updated master cast to bf16 bit for bit (both round to nearest even).

CPU: the C entry point's argument checks (every rejected call returns before any launch), the
optimizer's own checks, and the ShadowWeights bookkeeping that lets a forward skip its refresh.
GPU: the update against torch over shapes with flat tails, partial 64 x 64 tiles, stacked
transposed groups, 1-D and empty parameters, more entries than one launch takes (40), a
parameter without a gradient; the step count in device memory; a captured step's replays.
"""
import ctypes

import pytest
import torch

from mamba_amd import _lib
from mamba_amd.mamba1 import ShadowWeights
from mamba_amd.optim import AdamW


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


_A = 1 << 32  # a 16-byte aligned address that is never dereferenced: every call below is rejected first


def _entry(**kw):
    base = dict(param=_A, grad=_A + 4096, exp_avg=_A + 8192, exp_avg_sq=_A + 12288, step=_A + 16384, shadow=None,
                shadow_t=None, rows=1, cols=64, ld_t=0, numel=64)
    base.update(kw)
    return _lib.AdamWEntry(**base)


def _call(lib, entries, **kw):
    arr = (_lib.AdamWEntry * len(entries))(*entries)
    hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2)
    hp.update(kw)
    args = _lib.AdamWArgs(entries=ctypes.cast(arr, ctypes.c_void_p), n_entries=len(entries), **hp)
    return lib.mss_adamw(ctypes.byref(args), None)


def test_adamw_validation(lib):
    bad = _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_adamw(None, None) == bad
    args = _lib.AdamWArgs(entries=None, n_entries=1, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0)
    assert lib.mss_adamw(ctypes.byref(args), None) == bad
    good = _entry()
    for hp in (dict(lr=-1.0), dict(beta1=1.0), dict(beta1=-0.1), dict(beta2=1.0), dict(eps=0.0), dict(weight_decay=-1.0),
               dict(lr=float("nan")), dict(eps=float("inf"))):
        assert _call(lib, [_entry(numel=0), good], **hp) == bad  # (the bad entry alone is rejected too)
        assert _call(lib, [_entry(param=_A + 2)], **hp) == bad
    for e in (_entry(numel=0), _entry(param=None), _entry(grad=None), _entry(step=None), _entry(param=_A + 8),
              _entry(exp_avg_sq=_A + 12292), _entry(shadow=_A + 4), _entry(numel=1 << 40),
              # transposed shadows: [rows][cols] with rows * cols == numel, cols % 4, ld_t >= rows, % 8, aligned
              _entry(shadow_t=_A, rows=8, cols=8, ld_t=8, numel=63),
              _entry(shadow_t=_A, rows=8, cols=6, ld_t=8, numel=48),
              _entry(shadow_t=_A, rows=16, cols=8, ld_t=8, numel=128),
              _entry(shadow_t=_A, rows=8, cols=8, ld_t=12, numel=64),
              _entry(shadow_t=_A + 8, rows=8, cols=8, ld_t=8, numel=64)):
        assert _call(lib, [good, e]) == bad  # rejected before the first launch
    assert _call(lib, []) == bad


def test_optimizer_checks():
    with pytest.raises(ValueError):
        AdamW([torch.zeros(4)], lr=-1.0)
    with pytest.raises(ValueError):
        AdamW([torch.zeros(4)], betas=(1.0, 0.999))
    with pytest.raises(ValueError):
        AdamW([torch.zeros(4)], eps=0.0)
    p = torch.zeros(4, requires_grad=True)
    p.grad = torch.ones(4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        AdamW([p]).step()


def test_shadow_bookkeeping_on_cpu():
    """refresh() writes the copies once and skips while nothing changed the masters; an
    in-place change, a replaced master or a new dtype makes the next call write again."""
    g = torch.Generator().manual_seed(0)
    ps = [torch.randn(8, 4, generator=g), torch.randn(6, 4, generator=g)]
    sw = ShadowWeights(ps, transposed=[(ps[0], ps[1])])
    assert not sw.is_current()
    sw.refresh(torch.bfloat16)
    assert sw.is_current()
    sw.bufs[0].fill_(7.0)  # a write the next refresh would undo, if it ran
    sw.refresh(torch.bfloat16)
    assert float(sw.bufs[0][0, 0]) == 7.0
    with torch.no_grad():
        ps[0].add_(1.0)  # tracked in-place change
    assert not sw.is_current()
    sw.refresh(torch.bfloat16)
    assert torch.equal(sw.bufs[0], ps[0].to(torch.bfloat16))
    ps[1].data = torch.randn(6, 4, generator=g)  # replaced storage
    assert not sw.is_current()
    sw.refresh(torch.bfloat16)
    assert torch.equal(sw.stacked_t(ps[0], ps[1]), torch.cat(ps).t().to(torch.bfloat16))
    sw.refresh(torch.float16)  # another layout: written again
    assert sw.bufs[0].dtype == torch.float16 and torch.equal(sw.bufs[0], ps[0].to(torch.float16))
    sw.mark_current()
    assert sw.is_current()
    assert sw.targets(ps[0]) is None  # (the optimizer writes bf16 layouts only)


def _bits(t):
    return t.contiguous().view(torch.int16)


def _problem(n_extra=0):
    g = torch.Generator().manual_seed(11)
    shapes = [(192, 128), (64, 128), (128, 192), (80, 128), (37,), (5000,), (4099,), (136, 68), (63, 129), (3, 5, 7),
              (0,), (1,)]
    shapes += [(17 + i, 4) for i in range(n_extra)]
    ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.5).cuda()) for s in shapes]
    gemm = [ps[0], ps[1], ps[2], ps[3], ps[7], ps[8]]
    groups = [(ps[0], ps[1]), (ps[2],), (ps[7],)]
    return ps, gemm, groups


def _grads(ps, step):
    g = torch.Generator().manual_seed(100 + step)
    for i, p in enumerate(ps):
        p.grad = None if i == len(ps) - 1 and step % 2 else (torch.randn(p.shape, generator=g) * 0.1).cuda()


def _check_shadows(sw, gemm, groups):
    for p, b in zip(gemm, sw.bufs):
        assert torch.equal(_bits(b), _bits(p.detach().to(torch.bfloat16)))
    for grp in groups:
        t = sw.stacked_t(*grp)
        assert torch.equal(_bits(t), _bits(torch.cat([w.detach() for w in grp]).t().to(torch.bfloat16)))


@pytest.mark.gpu
@pytest.mark.parametrize("n_extra", [0, 45])
def test_adamw_matches_torch(n_extra):
    """Four steps against torch.optim.AdamW (single-tensor form) on the same gradients, with
    the last parameter's gradient missing every other step (both skip it then). n_extra adds
    small parameters so the call spans two launches of up to 40 entries."""
    print(f"case adamw vs torch n_extra={n_extra}", flush=True)
    ps, gemm, groups = _problem(n_extra)
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    sw = ShadowWeights(gemm, transposed=groups)
    sw.refresh(torch.bfloat16)
    opt = AdamW(ps, lr=3e-3, betas=(0.8, 0.95), eps=1e-6, weight_decay=0.1, shadows=sw)
    opt_ref = torch.optim.AdamW(ref, lr=3e-3, betas=(0.8, 0.95), eps=1e-6, weight_decay=0.1, foreach=False, fused=False)
    for step in range(4):
        _grads(ps, step)
        for p, r in zip(ps, ref):
            r.grad = None if p.grad is None else p.grad.clone()
        assert sw.is_current()
        opt.step()
        opt_ref.step()
        torch.cuda.synchronize()
        assert sw.is_current()  # written by the launch: the next forward would not refresh
        _check_shadows(sw, gemm, groups)
        for i, (p, r) in enumerate(zip(ps, ref)):
            # (atol: a few float32 roundings of updates of size ~lr for parameters near zero)
            torch.testing.assert_close(p.detach(), r.detach(), rtol=2e-6, atol=4e-6 * 3e-3,
                                       msg=lambda m, i=i, step=step: f"param {i} step {step}: {m}")
            if opt_ref.state[r] and p.numel() > 0:
                st, sr = opt.state[p], opt_ref.state[r]
                for k in ("exp_avg", "exp_avg_sq"):  # (a moment near zero is a difference of rounded terms)
                    scale = float(sr[k].abs().max())
                    torch.testing.assert_close(st[k], sr[k], rtol=1e-5, atol=1e-6 * scale,
                                               msg=lambda m, k=k, i=i, step=step: f"{k} {i} step {step}: {m}")
    assert float(opt.state[ps[0]]["step"]) == 4.0
    assert ps[0]._version > 0  # the launch is counted as an in-place update


@pytest.mark.gpu
def test_adamw_graph_replays():
    """A captured optimizer step (the step count advanced inside the graph) replayed three
    times, with eager work between replays, equals three eager steps bit for bit."""
    print("case adamw graph replays", flush=True)
    ps, gemm, groups = _problem()
    ps = ps[:-2]  # (no empty or gradient-less parameters here)
    twin = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    _grads(ps, 0)
    for p, t in zip(ps, twin):
        t.grad = p.grad.clone()
    sw = ShadowWeights(gemm, transposed=groups)
    sw.refresh(torch.bfloat16)
    opt = AdamW(ps, lr=1e-2, shadows=sw)
    opt_e = AdamW(twin, lr=1e-2)
    opt.step()  # state allocated outside the capture
    opt_e.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            opt.step()
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        graph.replay()
        opt_e.step()
        torch.cuda.synchronize()
        _ = float(ps[0].detach().sum())  # eager work between replays
        for p, t in zip(ps, twin):
            assert torch.equal(p.detach(), t.detach())
    _check_shadows(sw, gemm, groups)
    assert float(opt.state[ps[0]]["step"]) == 4.0


@pytest.mark.gpu
def test_adamw_untileable_transposed_shadow():
    """A transposed group whose row count is not a multiple of 8 (the kernel's 16-byte stores):
    the update and the plain shadows are written, the transposed copy is left to the next
    refresh, and the shadows are reported as not current (so a forward refreshes them)."""
    print("case adamw untileable transposed shadow", flush=True)
    g = torch.Generator().manual_seed(5)
    ps = [torch.nn.Parameter(torch.randn(s, generator=g).cuda()) for s in [(130, 68), (70, 68)]]
    ref = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    sw = ShadowWeights(ps[:1], transposed=[(ps[0],)])
    sw.refresh(torch.bfloat16)
    opt = AdamW(ps, lr=1e-2, shadows=sw)
    opt_ref = torch.optim.AdamW(ref, lr=1e-2, foreach=False, fused=False)
    for p, r in zip(ps, ref):
        p.grad = torch.randn(p.shape, generator=g).cuda()
        r.grad = p.grad.clone()
    opt.step()
    opt_ref.step()
    torch.cuda.synchronize()
    for p, r in zip(ps, ref):
        torch.testing.assert_close(p.detach(), r.detach(), rtol=2e-6, atol=1e-9)
    assert torch.equal(_bits(sw.bufs[0]), _bits(ps[0].detach().to(torch.bfloat16)))
    assert not sw.is_current()
    sw.refresh(torch.bfloat16)
    _check_shadows(sw, ps[:1], [(ps[0],)])
