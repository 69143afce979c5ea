"""GPU parity: HIP kernels (through the C ABI) vs the float64 oracle on identical inputs.

Bars (stated by the build target): float32 within rtol 1e-4 / atol 1e-5; bfloat16
inputs with float32 accumulation within rtol 2e-2. Every output and gradient is checked
element by element: |got - ref| <= atol + rtol * s, where s = |ref| for per-step values and,
for the gradients that are sums over channels, batch rows or steps (dA, dB, dC, dD,
ddelta_bias), s = the sum of the absolute values of the terms summed into that element
(returned by the oracle), the scale of the rounding error of any order of summation.
The oracle is the float64 C restatement (oracle/scan64c.c, pinned against the numpy
oracle on the CPU). Cases follow the reference tests
(tests/test_selective_scan_cuda.py: lengths {1, 17, 128, 513} forward, {1, 31, 513, 2051}
VJP, ZOH VJP at 31, reference input recipe) and extend them to the fused extras,
multi-chunk lengths, ragged tails, variable lengths, bf16 and the full config-2 shape.
"""
import ctypes
import os
import sys

import numpy as np
import pytest
import torch

from mamba_amd import _lib
from mamba_amd.configs import C2, C3, C4, ScanConfig, make_scan_inputs
from mamba_amd.selective_scan_hip import selective_scan, selective_scan_fn
from oracle import scan64, scan64c

pytestmark = pytest.mark.gpu

F32_RTOL, F32_ATOL = 1e-4, 1e-5
BF16_RTOL = 2e-2


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def close(name, got, ref, rtol=F32_RTOL, atol=F32_ATOL, scale=None):
    """Elementwise |got - ref| <= atol + rtol * s with s = |ref|, or s = `scale` (same shape:
    the oracle's sum of |terms| of a reduction gradient). Logs the worst err / bound."""
    got = got.detach().float().cpu().numpy() if torch.is_tensor(got) else np.asarray(got)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    s = np.abs(ref) if scale is None else np.asarray(scale, np.float64)
    assert s.shape == ref.shape, (name, s.shape, ref.shape)
    err = np.abs(got - ref)
    bound = atol + rtol * s
    ratio = err / bound
    worst = int(np.argmax(ratio))
    ok = bool(np.all(err <= bound))
    log(f"  {name:16s} max_abs={err.max():.3e} worst err/bound={ratio.flat[worst]:.3f} "
        f"(got={got.flat[worst]:.6e}, ref={ref.flat[worst]:.6e}, scale={s.flat[worst]:.3e}) ok={ok}")
    assert ok, f"{name}: {np.sum(err > bound)} of {err.size} elements outside rtol={rtol}, atol={atol}"
    return float(ratio.flat[worst])


dev = "cuda"


def T(a, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(a)).to(dev, dtype)


def ref_recipe(seed, batch=2, length=17, dim=8, n=16):
    rng = np.random.default_rng(seed)
    A = -np.exp(rng.standard_normal((dim, n)))
    deltas = np.log1p(np.exp(rng.standard_normal((batch, length, dim))))
    Bs = rng.standard_normal((batch, length, n))
    Cs = rng.standard_normal((batch, length, n))
    u = rng.standard_normal((batch, length, dim))
    x0 = rng.standard_normal((batch, dim, n))
    return [a.astype(np.float32) for a in (A, deltas, Bs, Cs, u, x0)]


@pytest.mark.parametrize("length", [1, 17, 128, 513, 2051, 4100])
@pytest.mark.parametrize("euler", [True, False])
def test_reference_api_forward(length, euler):
    log(f"case forward L={length} euler={euler}")
    args = ref_recipe(7, length=length)
    y, fin = selective_scan(*[T(a) for a in args], use_euler_barB_approx=euler)
    torch.cuda.synchronize()
    ey, efin, _ = scan64.reference_api_forward(*args, use_euler_barB_approx=euler)
    close("y", y, ey)
    close("final_x", fin, efin)


@pytest.mark.parametrize("length", [1, 31, 513, 2051])
@pytest.mark.parametrize("euler", [True, False])
def test_reference_api_vjp(length, euler):
    log(f"case vjp L={length} euler={euler}")
    args = ref_recipe(11, batch=1, length=length, dim=4, n=8)
    ts = [T(a).requires_grad_(True) for a in args]
    y, fin = selective_scan(*ts, use_euler_barB_approx=euler)
    loss = (y ** 2).mean() + (fin ** 2).mean()
    loss.backward()
    torch.cuda.synchronize()
    ey, efin, _ = scan64.reference_api_forward(*args, use_euler_barB_approx=euler)
    dy = 2 * ey / ey.size
    dfin = 2 * efin / efin.size
    grads, ab = scan64.reference_api_backward(*args, dy, dfin, use_euler_barB_approx=euler, abs_terms=True)
    for name, t, g in zip(["dA", "ddeltas", "dBs", "dCs", "du", "dinitial_x"], ts, grads):
        close(name, t.grad, g, scale=ab.get(name))


def fused_case(seed, b, d, l, n, dtype="f32", lens=None, zoh=False, extras=True):
    rng = np.random.default_rng(seed)
    f = np.float32
    x = dict(u=rng.standard_normal((b, d, l)).astype(f), delta=rng.standard_normal((b, d, l)).astype(f),
             A=(-np.exp(rng.standard_normal((d, n)))).astype(f), B=rng.standard_normal((b, n, l)).astype(f),
             C=rng.standard_normal((b, n, l)).astype(f))
    if extras:
        x.update(D=rng.standard_normal(d).astype(f), z=rng.standard_normal((b, d, l)).astype(f),
                 delta_bias=(0.5 * rng.standard_normal(d) - 2.0).astype(f),
                 initial_state=rng.standard_normal((b, d, n)).astype(f))
    dout = rng.standard_normal((b, d, l)).astype(f)
    dlast = rng.standard_normal((b, d, n)).astype(f)
    if dtype == "bf16":
        from mamba_amd.configs import round_to_bf16
        for k in ("u", "delta", "B", "C", "z"):
            if k in x:
                x[k] = round_to_bf16(x[k])
        dout = round_to_bf16(dout)
    if lens is not None:
        x["seq_lens"] = np.asarray(lens, np.int32)
    return x, dout, dlast


def run_fused(x, dout, dlast, dtype, zoh, softplus=True):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    io = {"u", "delta", "z", "B", "C"}
    ts = {}
    for k, v in x.items():
        if k == "seq_lens":
            ts[k] = torch.as_tensor(v).to(dev)
        else:
            ts[k] = T(v, tdt if k in io else torch.float32).requires_grad_(True)
    out, last = selective_scan_fn(ts["u"], ts["delta"], ts["A"], ts["B"], ts["C"], D=ts.get("D"), z=ts.get("z"),
                                  delta_bias=ts.get("delta_bias"), delta_softplus=softplus,
                                  return_last_state=True, initial_state=ts.get("initial_state"),
                                  seq_lens=ts.get("seq_lens"), discretization="zoh" if zoh else "euler")
    (out.float() * T(dout)).sum().add_((last * T(dlast)).sum()).backward()
    torch.cuda.synchronize()
    return ts, out, last


def oracle_fused(x, dout, dlast, zoh, softplus=True):
    kw = dict(D=x.get("D"), z=x.get("z"), delta_bias=x.get("delta_bias"), delta_softplus=softplus,
              initial_state=x.get("initial_state"), seq_lens=x.get("seq_lens"),
              discretization="zoh" if zoh else "euler")
    fw = scan64c.forward(x["u"], x["delta"], x["A"], x["B"], x["C"], **kw)
    g = scan64c.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout, dlast_state=dlast, abs_terms=True, **kw)
    return fw, g


GRAD_OF = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
           "delta_bias": "ddelta_bias", "initial_state": "dinitial_state"}


# Gradients that are sums over batch/steps (dA, dD, ddelta_bias) or channels (dB, dC).
REDUCTIONS = {"dA", "dB", "dC", "dD", "ddelta_bias"}


def check_fused(ts, out, last, fw, g, rtol=F32_RTOL, atol=F32_ATOL):
    """Every output and gradient against the oracle; returns {name: worst err / bound}."""
    worst = {"out": close("out", out, fw["out"], rtol, atol),
             "last_state": close("last_state", last, fw["last_state"], rtol, atol)}
    for k, gname in GRAD_OF.items():
        if k in ts:
            scale = g[gname + "_abs"] if gname in REDUCTIONS else None
            worst[gname] = close(gname, ts[k].grad, g[gname], rtol, atol, scale=scale)
    return worst


@pytest.mark.parametrize("l", [1, 7, 250, 1024, 1500, 3000])
@pytest.mark.parametrize("n", [1, 4, 11, 16])
def test_fused_fp32(l, n):
    log(f"case fused fp32 L={l} N={n}")
    x, dout, dlast = fused_case(100 + l + n, 2, 24, l, n)
    ts, out, last = run_fused(x, dout, dlast, "f32", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("zoh", [False, True])
def test_fused_wide_grid(zoh, dtype):
    """2 x 4096 channels: 1024 forward workgroups, more than one pass of the 8-step-per-lane
    launch shape: bf16 rows take the 16-step shape there, float32 rows keep the 8-step one
    over two passes (the other tests' grids are small); 1100 steps give full and ragged
    chunks of either."""
    log(f"case fused wide grid zoh={zoh} {dtype}")
    x, dout, dlast = fused_case(950 + zoh, 2, 4096, 1100, 16, dtype, zoh=zoh)
    ts, out, last = run_fused(x, dout, dlast, dtype, zoh)
    fw, g = oracle_fused(x, dout, dlast, zoh)
    check_fused(ts, out, last, fw, g, *tol(dtype))


def tol(dtype):
    return (BF16_RTOL, BF16_RTOL * 0.05) if dtype == "bf16" else (F32_RTOL, F32_ATOL)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("zoh", [False, True])
@pytest.mark.parametrize("n", [8, 4, 1])
def test_sixteen_wave_state_counts(n, zoh, dtype):
    """1 x 4096 channels: the backward runs 16 waves per workgroup (asserted from the
    library's plan), where N < 16 states give each wave a copy of the rotated dB/dC
    accumulator rows (16 / N copies)."""
    log(f"case sixteen waves N={n} zoh={zoh} {dtype}")
    assert _lib.bwd_plan(1, 4096, n, 600, zoh=zoh, io_bf16=dtype == "bf16")[0] == 16
    x, dout, dlast = fused_case(960 + n + zoh, 1, 4096, 600, n, dtype=dtype, zoh=zoh)
    ts, out, last = run_fused(x, dout, dlast, dtype, zoh)
    fw, g = oracle_fused(x, dout, dlast, zoh)
    check_fused(ts, out, last, fw, g, *tol(dtype))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sixteen_wave_varlen(dtype):
    """Variable lengths on a grid whose backward plan is 16 waves per workgroup: whole chunks
    past a row's length (zero gradients, the adjoint passing through) and an empty row."""
    log(f"case sixteen waves varlen {dtype}")
    assert _lib.bwd_plan(4, 2048, 16, 1100, varlen=True, io_bf16=dtype == "bf16")[0] == 16
    x, dout, dlast = fused_case(970, 4, 2048, 1100, 16, dtype=dtype, lens=[1100, 530, 0, 1])
    ts, out, last = run_fused(x, dout, dlast, dtype, False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g, *tol(dtype))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("l", [32, 544, 1024, 2080])
def test_backward_partial_channel_group(l, dtype):
    """One, two and five chunks (a ragged last one), 40 channels over workgroups of 12 (a
    partial last group), every fused extra, initial state and final-state cotangent."""
    log(f"case backward partial group L={l} {dtype}")
    assert _lib.bwd_plan(3, 40, 16, l, io_bf16=dtype == "bf16") == (12, 12)
    x, dout, dlast = fused_case(1000 + l, 3, 40, l, 16, dtype=dtype)
    ts, out, last = run_fused(x, dout, dlast, dtype, False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g, *tol(dtype))


@pytest.mark.parametrize("lens", [[2080, 600, 0, 31, 545], [512, 513, 1, 1024, 2079]])
def test_varlen_dead_chunks(lens):
    """Variable lengths over five chunks: whole chunks past a row's length (zero gradients,
    the adjoint passing through), a row of length 0, partial chunks; garbage in the
    padding."""
    log(f"case varlen dead chunks lens={lens}")
    x, dout, dlast = fused_case(1100, 5, 40, 2080, 16, lens=lens)
    ts, out, last = run_fused(x, dout, dlast, "f32", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g)


MULTI_ROUND_LENS = [1100, 530, 0, 1, 1099, 512, 513, 700]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("n,zoh", [(16, False), (11, False), (8, True)])
def test_varlen_multi_round(n, zoh, dtype):
    """Variable lengths on a grid whose backward workgroups walk several channel rounds (the
    plan of config 4: more channels per workgroup than waves): per round the adjoint message,
    dA, dD and ddelta_bias bookkeeping restarts from the round's channels, the dead chunks
    past a row's length pass the message through and write zero gradients for every round,
    and rows are handed out longest first. 16 waves x 2 rounds (N = 16, 8) and 12 waves x 2
    rounds (N = 11, two accumulator copies); an empty row, a one-step row, lengths one short
    of / exactly at / one past a 512-step chunk; garbage in the padding; every fused extra."""
    log(f"case varlen multi-round N={n} zoh={zoh} {dtype}")
    waves, cpb = _lib.bwd_plan(8, 1536, n, 1100, varlen=True, zoh=zoh, io_bf16=dtype == "bf16")
    assert cpb >= 2 * waves, (waves, cpb)
    x, dout, dlast = fused_case(1400 + n + zoh, 8, 1536, 1100, n, dtype, lens=MULTI_ROUND_LENS, zoh=zoh)
    ts, out, last = run_fused(x, dout, dlast, dtype, zoh)
    fw, g = oracle_fused(x, dout, dlast, zoh)
    check_fused(ts, out, last, fw, g, *tol(dtype))


PER_ROW = ("u", "delta", "z", "B", "C", "initial_state", "seq_lens")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_varlen_row_permutation(dtype):
    """With lengths the kernels hand rows to workgroups longest first (ties by index). Rows
    permuted give the permuted outputs and per-row gradients bit for bit; the sums over
    rows (dA, dD, ddelta_bias) change only by summation order."""
    log(f"case varlen row permutation {dtype}")
    lens = [2080, 300, 2080, 0, 1500, 700]
    perm = [4, 2, 5, 0, 3, 1]
    x, dout, dlast = fused_case(1300, 6, 40, 2080, 16, dtype, lens=lens)
    xp = {k: (v[perm] if k in PER_ROW else v) for k, v in x.items()}
    a = run_fused(x, dout, dlast, dtype, False)
    b = run_fused(xp, dout[perm], dlast[perm], dtype, False)
    idx = torch.as_tensor(perm, device=dev)
    assert torch.equal(a[1][idx], b[1]) and torch.equal(a[2][idx], b[2])
    for k in PER_ROW[:-1]:
        assert torch.equal(a[0][k].grad[idx], b[0][k].grad), k
    for k in ("A", "D", "delta_bias"):
        ga, gb = a[0][k].grad, b[0][k].grad
        assert torch.allclose(ga, gb, rtol=1e-5, atol=1e-6 * float(ga.abs().max())), k


def test_no_extras_three_chunks_and_determinism():
    """Without D, z, delta bias, softplus or initial state (raw positive delta) over three
    whole chunks, and bit-identical reruns."""
    log("case no extras, three chunks")
    x, dout, dlast = fused_case(1200, 2, 64, 1536, 16, extras=False)
    x["delta"] = np.abs(x["delta"]) * 0.1
    a = run_fused(x, dout, dlast, "f32", False, softplus=False)
    fw, g = oracle_fused(x, dout, dlast, False, softplus=False)
    check_fused(*a, fw, g)
    b = run_fused(x, dout, dlast, "f32", False, softplus=False)
    for k in ("u", "delta", "A", "B", "C"):
        assert torch.equal(a[0][k].grad, b[0][k].grad), k


@pytest.mark.parametrize("l", [5, 300, 2100])
def test_fused_zoh(l):
    log(f"case fused zoh L={l}")
    x, dout, dlast = fused_case(200 + l, 2, 16, l, 8, zoh=True)
    ts, out, last = run_fused(x, dout, dlast, "f32", True)
    fw, g = oracle_fused(x, dout, dlast, True)
    check_fused(ts, out, last, fw, g)


def test_fused_no_extras_no_softplus():
    log("case fused, no extras, raw positive delta")
    x, dout, dlast = fused_case(300, 2, 16, 700, 16, extras=False)
    x["delta"] = np.abs(x["delta"]) * 0.1
    ts, out, last = run_fused(x, dout, dlast, "f32", False, softplus=False)
    fw, g = oracle_fused(x, dout, dlast, False, softplus=False)
    check_fused(ts, out, last, fw, g)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("lens", [None, [600, 333]])
def test_gate_near_zero_z(dtype, lens):
    """The gate's backward takes y sigmoid(z) as out / z except where |z| < 1e-20, where it reads
    y itself, kept by the forward for those elements only: exact zeros of both signs, |z| of
    1e-30 and 9e-21 (kept y), 2e-20 and 1e-6 (out / z), the zero of the gate's slope (z ~ -1.2785)
    and |z| up to 100, scattered over every row, with and without lengths. Per element against
    the oracle."""
    log(f"case gate near zero z {dtype} lens={lens}")
    x, dout, dlast = fused_case(77, 2, 24, 600, 16, dtype, lens=lens)
    flat = x["z"].reshape(-1)
    specials = np.array([0.0, -0.0, 1e-30, -1e-30, 9e-21, -9e-21, 2e-20, -2e-20, 1e-6, -1e-6, -1.2785, 30.0,
                         -30.0, -100.0], np.float32)
    pos = (np.arange(0, flat.size, 7) * 131) % flat.size
    flat[pos] = specials[np.arange(pos.size) % specials.size]
    if dtype == "bf16":
        from mamba_amd.configs import round_to_bf16
        x["z"] = round_to_bf16(x["z"])
    ts, out, last = run_fused(x, dout, dlast, dtype, False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g, *tol(dtype))


def test_gate_output_changed_in_place_raises():
    """With z the backward reads the forward's output (dz from out / z), so an in-place change
    of that output before backward must raise torch's saved-tensor version error instead of
    giving a wrong dz; without z the output is not saved and the same change is allowed."""
    log("case gate output changed in place")
    x, dout, _ = fused_case(78, 1, 8, 256, 4)
    ts = {k: T(v).requires_grad_(True) for k, v in x.items() if k in ("u", "delta", "A", "B", "C", "z")}
    out = selective_scan_fn(ts["u"], ts["delta"], ts["A"], ts["B"], ts["C"], z=ts["z"], delta_softplus=True)
    out.mul_(2.0)
    with pytest.raises(RuntimeError, match="inplace"):
        (out * T(dout)).sum().backward()
    out = selective_scan_fn(ts["u"], ts["delta"], ts["A"], ts["B"], ts["C"], delta_softplus=True)
    out.mul_(2.0)
    (out * T(dout)).sum().backward()
    torch.cuda.synchronize()
    assert torch.isfinite(ts["u"].grad).all()


@pytest.mark.parametrize("lens", [[3000, 1025, 1, 0], [512, 2047, 2048, 2049]])
def test_varlen_fp32(lens):
    log(f"case varlen lens={lens}")
    x, dout, dlast = fused_case(400, 4, 16, 3000, 16, lens=lens)
    # garbage beyond each row's length must not leak
    ts, out, last = run_fused(x, dout, dlast, "f32", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    check_fused(ts, out, last, fw, g)


@pytest.mark.parametrize("l", [64, 1000, 2056])
def test_bf16(l):
    log(f"case bf16 L={l}")
    x, dout, dlast = fused_case(500 + l, 2, 32, l, 16, dtype="bf16")
    ts, out, last = run_fused(x, dout, dlast, "bf16", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    # bf16 outputs are rounded once; fp32 accumulation inside.
    check_fused(ts, out, last, fw, g, rtol=BF16_RTOL, atol=BF16_RTOL * 0.05)


@pytest.mark.parametrize("length", [1024, 999])
def test_bf16_store_rounding_bit_exact(length):
    """bf16 outputs are float32 results rounded to nearest, ties to even, bit for bit: with
    delta = 0 and no softplus every a_bar is 1 and every b_bar*u is 0, so the state stays zero
    and out = D*u is one float32 product, whose bf16 rounding must equal the integer
    round-to-nearest-even of the same product (configs.round_to_bf16). Channels cover exact
    ties (powers of two times 1 + 2^-8, which round down to even), carries into the exponent,
    products past the largest bf16 (round to inf), subnormals and random values; an odd length
    also takes the per-element store path of the last chunk."""
    from mamba_amd.configs import round_to_bf16
    log(f"case bf16 store rounding L={length}")
    b, d, l, n = 2, 8, length, 4
    rng = np.random.default_rng(77 + length)
    f = np.float32
    base = rng.standard_normal((b, d, l)).astype(f)
    u = np.empty((b, d, l), f)
    Dv = np.empty(d, f)
    u[:, 0] = base[:, 0]
    Dv[0] = f(0.7)
    u[:, 1] = base[:, 1] * f(1e3)
    Dv[1] = f(1.0 + 3 * 2.0 ** -9)
    pw = np.ldexp(np.ones((b, l), f), rng.integers(-20, 20, (b, l))).astype(f)
    u[:, 2] = pw * np.where(rng.random((b, l)) < 0.5, f(1), f(-1))
    Dv[2] = f(1.0 + 2.0 ** -8)  # exact ties: round to the even neighbour (down)
    u[:, 3] = (1 + rng.integers(0, 128, (b, l)).astype(f) / 128) * pw
    Dv[3] = f(1.0 + 2.0 ** -8)  # ties, carries, and values just above a tie
    u[:, 4] = np.ldexp(f(1) + rng.integers(120, 128, (b, l)).astype(f) / 128, 127).astype(f)
    Dv[4] = f(1.0 + 2.0 ** -8)  # near the largest bf16: some products round to inf
    u[:, 5] = base[:, 5] * f(2.0 ** -130)  # float32 subnormals
    Dv[5] = f(1.3)
    u[:, 6] = base[:, 6] * f(1e-30)
    Dv[6] = f(1.0 + 2.0 ** -12)
    u[:, 7] = base[:, 7] * f(3e37)
    Dv[7] = f(0.999)
    u = round_to_bf16(u)
    u[u == 0] = 0  # -0 inputs: the state sum adds C*h = +0 to D*u, and -0 + +0 = +0
    with np.errstate(over="ignore"):
        prod = u * Dv[None, :, None]
    want = (round_to_bf16(prod).view(np.uint32) >> 16).astype(np.uint16)
    A = -np.ones((d, n), f)
    Bm = rng.standard_normal((b, n, l)).astype(f)
    Cm = rng.standard_normal((b, n, l)).astype(f)
    out = selective_scan_fn(T(u, torch.bfloat16), T(np.zeros((b, d, l), f), torch.bfloat16), T(A),
                            T(Bm, torch.bfloat16), T(Cm, torch.bfloat16), D=T(Dv), delta_softplus=False)
    torch.cuda.synchronize()
    got = out.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    bad = got != want
    for ch in range(d):
        nb = int(bad[:, ch].sum())
        if nb:
            i = np.argwhere(bad[:, ch])[0]
            log(f"  channel {ch}: {nb} mismatches, e.g. u={u[i[0], ch, i[1]]!r} D={Dv[ch]!r} "
                f"got=0x{int(got[i[0], ch, i[1]]):04x} want=0x{int(want[i[0], ch, i[1]]):04x}")
    assert np.isinf(prod[:, 4]).sum() == 0 and np.isinf(round_to_bf16(prod[:, 4])).any()
    assert not bad.any()


@pytest.mark.parametrize("n,zoh,lens", [(17, False, None), (32, True, None), (40, False, [700, 333]),
                                        (64, False, None), (256, True, None)])
def test_wide_state_fp32(n, zoh, lens):
    """Float32 scans with more than 16 states (the reference C handler's N <= 256): the
    forward keeps every state of a wave in LDS; the backward runs over balanced groups of at
    most 16 states (the first writes dz, dD and the D term, the others add their state sums to
    du, ddelta and ddelta_bias). Every output and gradient against the oracle, with all fused
    extras and a ragged varlen case."""
    log(f"case wide state N={n} zoh={zoh} lens={lens}")
    x, dout, dlast = fused_case(900 + n, 2, 24, 700, n, lens=lens)
    ts, out, last = run_fused(x, dout, dlast, "f32", zoh)
    fw, g = oracle_fused(x, dout, dlast, zoh)
    check_fused(ts, out, last, fw, g)


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes(seed):
    """Seeded random cases across the contract at once: batch 1-4, 1-70 channels (partial
    waves and channel rounds), lengths 1-2600 (ragged chunk tails), 1-16 states (17-40 for
    some float32 cases: the grouped backward), float32 or bf16, Euler or ZOH, with or without
    the fused extras and softplus, with or without variable lengths (zeros and full rows
    included). Every output and gradient against the float64 oracle at the dtype's bar."""
    rng = np.random.default_rng(7000 + seed)
    dtype = "bf16" if rng.random() < 0.35 else "f32"
    b, d = int(rng.integers(1, 5)), int(rng.integers(1, 71))
    l = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 2601))]))
    n = int(rng.integers(17, 41)) if dtype == "f32" and rng.random() < 0.2 else int(rng.integers(1, 17))
    zoh, extras, softplus = bool(rng.random() < 0.4), bool(rng.random() < 0.7), bool(rng.random() < 0.8)
    lens = None
    if rng.random() < 0.4:
        lens = [int(v) for v in rng.integers(0, l + 1, size=b)]
        lens[int(rng.integers(0, b))] = int(rng.choice([0, l]))
    log(f"case random seed={seed}: {dtype} B={b} D={d} L={l} N={n} zoh={zoh} extras={extras} "
        f"softplus={softplus} lens={lens}")
    x, dout, dlast = fused_case(8000 + seed, b, d, l, n, dtype, lens=lens, extras=extras)
    if not softplus:  # raw delta + bias must stay positive (a decaying state)
        x["delta"] = np.abs(x["delta"]) * 0.1
        if dtype == "bf16":
            from mamba_amd.configs import round_to_bf16
            x["delta"] = round_to_bf16(x["delta"])
        if "delta_bias" in x:
            x["delta_bias"] = np.abs(x["delta_bias"]) * 0.01
    ts, out, last = run_fused(x, dout, dlast, dtype, zoh, softplus=softplus)
    fw, g = oracle_fused(x, dout, dlast, zoh, softplus=softplus)
    check_fused(ts, out, last, fw, g, *tol(dtype))


def test_deterministic_rerun():
    log("case determinism")
    x, dout, dlast = fused_case(600, 2, 64, 1500, 16)
    a = run_fused(x, dout, dlast, "f32", False)
    b = run_fused(x, dout, dlast, "f32", False)
    assert torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    for k in ("u", "delta", "z", "A", "B", "C", "D", "delta_bias", "initial_state"):
        assert torch.equal(a[0][k].grad, b[0][k].grad), k


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("l", [37, 1100])
def test_strided_row_layouts(dtype, l):
    """Rows laid out as (R, B*L) activation matrices: u/delta/z channel-outer, B and C row
    slices of one (R + 2N, B*L) projection output. Results equal those of contiguous
    inputs bit for bit (same arithmetic) and match the oracle."""
    log(f"case strided layouts {dtype} L={l}")
    b, d, n, r = 3, 40, 16, 5
    x, dout, dlast = fused_case(700 + l, b, d, l, n, dtype=dtype)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    ts_c, out_c, last_c = run_fused(x, dout, dlast, dtype, False)

    def channel_outer(a):  # (b, d, l) -> leaf (d, b, l) and its (b, d, l) view
        leaf = T(np.ascontiguousarray(np.swapaxes(a, 0, 1)), tdt).requires_grad_(True)
        return leaf, leaf.permute(1, 0, 2)

    leaves = {k: channel_outer(x[k]) for k in ("u", "delta", "z")}
    junk = np.random.default_rng(1).standard_normal((r, b, l)).astype(np.float32)
    proj_np = np.concatenate([junk, np.swapaxes(x["B"], 0, 1), np.swapaxes(x["C"], 0, 1)], axis=0)
    proj = T(proj_np, tdt).requires_grad_(True)
    Bv = proj[r:r + n].permute(1, 0, 2)
    Cv = proj[r + n:].permute(1, 0, 2)
    small = {k: T(x[k]).requires_grad_(True) for k in ("A", "D", "delta_bias", "initial_state")}
    out, last = selective_scan_fn(leaves["u"][1], leaves["delta"][1], small["A"], Bv, Cv, D=small["D"],
                                  z=leaves["z"][1], delta_bias=small["delta_bias"], delta_softplus=True,
                                  return_last_state=True, initial_state=small["initial_state"])
    assert out.stride() == leaves["u"][1].stride()
    (out.float() * T(dout)).sum().add_((last * T(dlast)).sum()).backward()
    torch.cuda.synchronize()
    assert torch.equal(out, out_c) and torch.equal(last, last_c)
    for k in ("u", "delta", "z"):
        assert torch.equal(leaves[k][0].grad.permute(1, 0, 2), ts_c[k].grad), k
    assert torch.equal(proj.grad[r:r + n].permute(1, 0, 2), ts_c["B"].grad)
    assert torch.equal(proj.grad[r + n:].permute(1, 0, 2), ts_c["C"].grad)
    assert torch.count_nonzero(proj.grad[:r]) == 0
    for k in small:
        assert torch.equal(small[k].grad, ts_c[k].grad), k
    fw, g = oracle_fused(x, dout, dlast, False)
    tol = (BF16_RTOL, BF16_RTOL * 0.05) if dtype == "bf16" else (F32_RTOL, F32_ATOL)
    check_fused(ts_c, out_c, last_c, fw, g, *tol)


@pytest.mark.parametrize("length,n", [(2500, 16), (5000, 16), (2500, 32)])
def test_reference_c_entry_points(length, n):
    """mss_scan_fwd / mss_scan_bwd / mss_scan_bwd_ws (the reference FFI handlers'
    counterparts) via ctypes, over two and three 2048-step blocks: the backward re-runs each
    block from the forward's chunk_states. The workspace variant equals mss_scan_bwd bit for
    bit; chunk_states from the float64 oracle give the same gradients to the float32 bar, and
    a corrupted block state changes them (the residual is what the backward starts from)."""
    log(f"case reference C entry points L={length} N={n}")
    lib = _lib.register_hip_kernel()
    A, deltas, Bs, Cs, u, x0 = ref_recipe(13, batch=2, length=length, dim=8, n=n)
    b, l, d = u.shape
    tr = lambda a: T(np.swapaxes(a, 1, 2))  # physical [B][D][L] / [B][N][L]
    tA, td, tB, tC, tu, tx0 = T(A), tr(deltas), tr(Bs), tr(Cs), tr(u), T(x0)
    y = torch.empty(b, d, l, device=dev)
    fin = torch.empty(b, d, n, device=dev)
    cs = torch.empty(b, d, -(-l // 2048), n, 2, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    _lib.check(lib.mss_scan_fwd(st, 0, b, l, d, n, P(tA), P(td), P(tB), P(tC), P(tu), P(tx0), P(y), P(fin), P(cs)),
               "mss_scan_fwd")
    rng = np.random.default_rng(14)
    dy = rng.standard_normal((b, l, d)).astype(np.float32)
    dfin = rng.standard_normal((b, d, n)).astype(np.float32)
    tdy, tdfin = tr(dy), T(dfin)

    def backward(states, ws=None):
        outs = [torch.full_like(t, float("nan")) for t in (tA, td, tB, tC, tu, tx0)]
        args = (st, b, l, d, n, P(tA), P(td), P(tB), P(tC), P(tu), P(tx0), P(states), P(tdy), P(tdfin),
                *[P(o) for o in outs])
        if ws is None:
            _lib.check(lib.mss_scan_bwd(*args), "mss_scan_bwd")
        else:
            _lib.check(lib.mss_scan_bwd_ws(*args, P(ws), ws.numel()), "mss_scan_bwd_ws")
        torch.cuda.synchronize()
        return outs

    outs = backward(cs)
    ws_bytes = int(lib.mss_scan_bwd_workspace_bytes(b, l, d, n))
    outs_ws = backward(cs, torch.empty(ws_bytes, dtype=torch.uint8, device=dev))
    for o, w in zip(outs, outs_ws):
        assert torch.equal(o, w)
    ey, efin, ecs = scan64.reference_api_forward(A, deltas, Bs, Cs, u, x0)
    close("y", y.transpose(1, 2), ey)
    close("final_x", fin, efin)
    close("chunk_states", cs, ecs)
    grads, ab = scan64.reference_api_backward(A, deltas, Bs, Cs, u, x0, dy, dfin, abs_terms=True)
    names = ["dA", "ddeltas", "dBs", "dCs", "du", "dinitial_x"]
    for label, res in (("gpu chunk_states", outs), ("oracle chunk_states", backward(T(ecs)))):
        log(f"  from {label}")
        for name, o, g in zip(names, res, grads):
            got = o if o.shape == g.shape else o.transpose(1, 2)
            close(name, got, g, scale=ab.get(name))
    bad = cs.clone()
    bad[:, :, 0, :, 1] += 1.0  # the state entering block 1
    moved = backward(bad)
    # dC = sum_d g h depends on the forward states: block 1's steps move, block 0's do not
    assert torch.equal(moved[3][:, :, :2048], outs[3][:, :, :2048])
    assert not torch.equal(moved[3][:, :, 2048:4096], outs[3][:, :, 2048:4096])


@pytest.mark.parametrize("seed", range(8))
def test_random_reference_api(seed):
    """Seeded random shapes through the reference's own signatures: the C entry points
    (mss_scan_fwd, then mss_scan_bwd_ws from the forward's chunk_states, Euler as the
    reference handler) and the Python `selective_scan` VJP (Euler or ZOH), batch 1-3, 1-40
    channels, lengths 1-4500 (across 2048-step blocks), 1-16 states (17-40 for some). Every
    output and gradient against the float64 oracle (the Python signature only where its error
    contract admits N)."""
    rng = np.random.default_rng(9000 + seed)
    b, d = int(rng.integers(1, 4)), int(rng.integers(1, 41))
    l = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(2000, 4501))]))
    r = rng.random()
    n = int(rng.integers(17, 41)) if r < 0.25 else int(rng.choice([1, 2, 4, 8, 16])) if r < 0.7 else int(rng.integers(1, 17))
    euler = seed % 2 == 0
    log(f"case random reference API seed={seed}: B={b} D={d} L={l} N={n} euler(python)={euler}")
    A, deltas, Bs, Cs, u, x0 = ref_recipe(9100 + seed, batch=b, length=l, dim=d, n=n)
    dy = rng.standard_normal((b, l, d)).astype(np.float32)
    dfin = rng.standard_normal((b, d, n)).astype(np.float32)
    # C entry points ([B][D][L] / [B][N][L] physical layouts)
    lib = _lib.register_hip_kernel()
    tr = lambda a: T(np.swapaxes(a, 1, 2))
    tA, td, tB, tC, tu, tx0, tdy, tdfin = T(A), tr(deltas), tr(Bs), tr(Cs), tr(u), T(x0), tr(dy), T(dfin)
    y = torch.empty(b, d, l, device=dev)
    fin = torch.empty(b, d, n, device=dev)
    cs = torch.empty(b, d, -(-l // 2048), n, 2, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    _lib.check(lib.mss_scan_fwd(st, _lib.MSS_EULER, b, l, d, n, P(tA), P(td), P(tB), P(tC), P(tu), P(tx0),
                                P(y), P(fin), P(cs)), "mss_scan_fwd")
    outs = [torch.full_like(t, float("nan")) for t in (tA, td, tB, tC, tu, tx0)]
    ws = torch.empty(int(lib.mss_scan_bwd_workspace_bytes(b, l, d, n)), dtype=torch.uint8, device=dev)
    _lib.check(lib.mss_scan_bwd_ws(st, b, l, d, n, P(tA), P(td), P(tB), P(tC), P(tu), P(tx0), P(cs), P(tdy),
                                   P(tdfin), *[P(o) for o in outs], P(ws), ws.numel()), "mss_scan_bwd_ws")
    torch.cuda.synchronize()
    ey, efin, ecs = scan64.reference_api_forward(A, deltas, Bs, Cs, u, x0)
    close("y", y.transpose(1, 2), ey)
    close("final_x", fin, efin)
    close("chunk_states", cs, ecs)
    grads, ab = scan64.reference_api_backward(A, deltas, Bs, Cs, u, x0, dy, dfin, abs_terms=True)
    names = ["dA", "ddeltas", "dBs", "dCs", "du", "dinitial_x"]
    for name, o, g in zip(names, outs, grads):
        close(name, o if o.shape == g.shape else o.transpose(1, 2), g, scale=ab.get(name))
    # the Python reference signature with autograd (its error contract admits N in {1, 2, 4,
    # 8, 16} only, as the reference's _validate_inputs does)
    ts = [T(a).requires_grad_(True) for a in (A, deltas, Bs, Cs, u, x0)]
    if n not in (1, 2, 4, 8, 16):
        with pytest.raises(ValueError, match="N must be one of"):
            selective_scan(*ts, use_euler_barB_approx=euler)
        return
    py, pfin = selective_scan(*ts, use_euler_barB_approx=euler)
    ((py * T(dy)).sum() + (pfin * T(dfin)).sum()).backward()
    torch.cuda.synchronize()
    ey, efin, _ = scan64.reference_api_forward(A, deltas, Bs, Cs, u, x0, use_euler_barB_approx=euler)
    close("py y", py, ey)
    close("py final_x", pfin, efin)
    grads, ab = scan64.reference_api_backward(A, deltas, Bs, Cs, u, x0, dy, dfin, use_euler_barB_approx=euler,
                                              abs_terms=True)
    for name, t, g in zip(names, ts, grads):
        close("py " + name, t.grad, g, scale=ab.get(name))


def config_tensors(cfg, x, dout):
    tdt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    ts = {}
    for k, v in x.items():
        if k == "seq_lens":
            ts[k] = torch.as_tensor(v).to(dev)
        else:
            ts[k] = T(v, tdt if k in ("u", "delta", "z", "B", "C") else torch.float32).requires_grad_(True)
    return ts


@pytest.mark.slow
def test_config2_full_size():
    """Config 2 at its full shape, every output and gradient against the oracle."""
    log("case c2 full size")
    x = make_scan_inputs(C2, seed=0, with_z=True, with_dout=True)
    dout = x.pop("dout")
    dlast = np.random.default_rng(1).standard_normal((C2.batch, C2.dim, C2.dstate)).astype(np.float32)
    ts, out, last = run_fused(x, dout, dlast, "f32", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    worst = check_fused(ts, out, last, fw, g)
    log("  c2 worst err/bound: " + ", ".join(f"{k}={v:.3f}" for k, v in worst.items()))


@pytest.mark.slow
def test_config3_full_size_bf16():
    """Config 3 at its full shape (B=8, D=2048, L=4096, N=16; u/delta/B/C/z/dout in bf16,
    fp32 accumulation): the 16-wave backward plan the config runs, every output and
    gradient against the oracle on the same bf16-rounded inputs."""
    log("case c3 full size")
    assert _lib.bwd_plan(C3.batch, C3.dim, C3.dstate, C3.length, io_bf16=True)[0] == 16
    x = make_scan_inputs(C3, seed=0, with_z=True, with_dout=True)
    dout = x.pop("dout")
    dlast = np.zeros((C3.batch, C3.dim, C3.dstate), np.float32)
    ts, out, last = run_fused(x, dout, dlast, "bf16", False)
    fw, g = oracle_fused(x, dout, dlast, False)
    worst = check_fused(ts, out, last, fw, g, *tol("bf16"))
    log("  c3 worst err/bound: " + ", ".join(f"{k}={v:.3f}" for k, v in worst.items()))


@pytest.mark.slow
@pytest.mark.timeout(900)
def test_config4_full_size():
    """Config 4 at its full shape (B=16, D=2560, L=8192, N=16, float32, seed-0 lengths in
    [512, 8192] right-padded with N(0,1) garbage): the backward plan the config runs (16 waves
    x 80 channels, five channel rounds per workgroup, dead chunks past each row's length), a
    random final-state cotangent, every output and gradient against the float64 oracle."""
    log("case c4 full size")
    assert _lib.bwd_plan(C4.batch, C4.dim, C4.dstate, C4.length, varlen=True) == (16, 80)
    x = make_scan_inputs(C4, seed=0, with_z=True, with_dout=True)
    dout = x.pop("dout")
    log(f"  lengths {x['seq_lens'].tolist()}")
    dlast = np.random.default_rng(1).standard_normal((C4.batch, C4.dim, C4.dstate)).astype(np.float32)
    ts, out, last = run_fused(x, dout, dlast, "f32", False)
    log("  gpu done, running the oracle")
    fw, g = oracle_fused(x, dout, dlast, False)
    worst = check_fused(ts, out, last, fw, g)
    log("  c4 worst err/bound: " + ", ".join(f"{k}={v:.3f}" for k, v in worst.items()))


@pytest.mark.parametrize("zoh", [False, True])
def test_reference_fwd_repeat(zoh):
    """mss_scan_fwd_repeat (the reference benchmark handler's counterpart, which launches the
    forward `repeats` times into the same outputs, native/selective_scan_cuda.cu:470-477):
    three launches leave y, final_x and chunk_states bit for bit as one launch does, and
    those match the float64 oracle (three 2048-step blocks, a ragged last one)."""
    log(f"case reference fwd repeat zoh={zoh}")
    lib = _lib.register_hip_kernel()
    A, deltas, Bs, Cs, u, x0 = ref_recipe(17 + zoh, batch=2, length=4500, dim=8, n=16)
    b, l, d = u.shape
    n = A.shape[1]
    tr = lambda a: T(np.swapaxes(a, 1, 2))
    tA, td, tB, tC, tu, tx0 = T(A), tr(deltas), tr(Bs), tr(Cs), tr(u), T(x0)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: ctypes.c_void_p(t.data_ptr())

    def run(repeats):
        outs = [torch.full((b, d, l), float("nan"), device=dev), torch.full((b, d, n), float("nan"), device=dev),
                torch.full((b, d, -(-l // 2048), n, 2), float("nan"), device=dev)]
        _lib.check(lib.mss_scan_fwd_repeat(st, int(zoh), repeats, b, l, d, n, P(tA), P(td), P(tB), P(tC), P(tu),
                                           P(tx0), *[P(o) for o in outs]), "mss_scan_fwd_repeat")
        torch.cuda.synchronize()
        return outs

    one, three = run(1), run(3)
    for name, o1, o3 in zip(("y", "final_x", "chunk_states"), one, three):
        assert torch.equal(o1, o3), name
    ey, efin, ecs = scan64.reference_api_forward(A, deltas, Bs, Cs, u, x0, use_euler_barB_approx=not zoh)
    close("y", three[0].transpose(1, 2), ey)
    close("final_x", three[1], efin)
    close("chunk_states", three[2], ecs)


@pytest.mark.slow
@pytest.mark.parametrize("zoh", [False, True])
def test_c5_layer_scan_bf16(zoh):
    """The scan of one layer of the config-5 model, as the model calls it: B=8, d_inner=1536,
    L=2048, N=16, bf16, u/delta/z channel-outer ((d_inner, B*L) activation matrices) and B/C
    row slices of the (dt_rank + 2N, B*L) x-projection output (dt_rank 48); the 16-wave
    backward plan; every output and gradient against the oracle."""
    log(f"case c5 layer scan zoh={zoh}")
    b, d, l, n, r = 8, 1536, 2048, 16, 48
    st = _lib.Strides(io_batch=l, io_dim=b * l, bc_batch=l, bc_state=b * l)
    assert _lib.bwd_plan(b, d, n, l, zoh=zoh, io_bf16=True, strides=st)[0] == 16
    cfg = ScanConfig("c5_layer", b, d, l, n, "bf16", None)
    x = make_scan_inputs(cfg, seed=5 + zoh, with_z=True, with_dout=True)
    dout = x.pop("dout")
    dlast = np.zeros((b, d, n), np.float32)
    tdt = torch.bfloat16

    def channel_outer(a):  # (b, d, l) -> leaf (d, b, l) and its (b, d, l) view
        leaf = T(np.ascontiguousarray(np.swapaxes(a, 0, 1)), tdt).requires_grad_(True)
        return leaf, leaf.permute(1, 0, 2)

    leaves = {k: channel_outer(x[k]) for k in ("u", "delta", "z")}
    junk = np.random.default_rng(9).standard_normal((r, b, l)).astype(np.float32)
    proj = T(np.concatenate([junk, np.swapaxes(x["B"], 0, 1), np.swapaxes(x["C"], 0, 1)], axis=0),
             tdt).requires_grad_(True)
    Bv = proj[r:r + n].permute(1, 0, 2)
    Cv = proj[r + n:].permute(1, 0, 2)
    small = {k: T(x[k]).requires_grad_(True) for k in ("A", "D", "delta_bias")}
    out, last = selective_scan_fn(leaves["u"][1], leaves["delta"][1], small["A"], Bv, Cv, D=small["D"],
                                  z=leaves["z"][1], delta_bias=small["delta_bias"], delta_softplus=True,
                                  return_last_state=True, discretization="zoh" if zoh else "euler")
    (out.float() * T(dout)).sum().backward()
    torch.cuda.synchronize()
    assert torch.count_nonzero(proj.grad[:r]) == 0
    ts = {k: leaves[k][0] for k in leaves}
    ts.update(small)
    grads = {k: leaves[k][0].grad.permute(1, 0, 2) for k in leaves}
    grads["B"] = proj.grad[r:r + n].permute(1, 0, 2)
    grads["C"] = proj.grad[r + n:].permute(1, 0, 2)
    grads.update({k: small[k].grad for k in small})
    fw, g = oracle_fused(x, dout, dlast, zoh)
    rt, at = tol("bf16")
    worst = {"out": close("out", out, fw["out"], rt, at), "last_state": close("last_state", last, fw["last_state"], rt, at)}
    for k, gt in grads.items():
        gname = GRAD_OF[k]
        worst[gname] = close(gname, gt, g[gname], rt, at, scale=g[gname + "_abs"] if gname in REDUCTIONS else None)
    log("  c5 layer worst err/bound: " + ", ".join(f"{k}={v:.3f}" for k, v in worst.items()))


@pytest.mark.slow
@pytest.mark.parametrize("cfg", [C4], ids=["c4"])
def test_large_config_channel_slice(cfg):
    """Full L and B of config 4 on a slice of 32 channels (channels are independent;
    dB/dC of the slice are the slice's own sums)."""
    log(f"case {cfg.name} channel slice")
    sl = ScanConfig(cfg.name + "_slice", cfg.batch, 32, cfg.length, cfg.dstate, cfg.dtype, cfg.varlen)
    x = make_scan_inputs(sl, seed=0, with_z=True, with_dout=True)
    dout = x.pop("dout")
    dlast = np.zeros((sl.batch, sl.dim, sl.dstate), np.float32)
    ts, out, last = run_fused(x, dout, dlast, cfg.dtype, False)
    fw, g = oracle_fused(x, dout, dlast, False)
    if cfg.dtype == "bf16":
        check_fused(ts, out, last, fw, g, rtol=BF16_RTOL, atol=BF16_RTOL * 0.05)
    else:
        check_fused(ts, out, last, fw, g)
