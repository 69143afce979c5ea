"""GPU parity of the complex-A scan (mss_cfwd / mss_cbwd through selective_scan_fn with a
complex64 A) against the float64 complex oracle (oracle/cscan64.py), on identical inputs.

Bars: the real scan's — float32 within rtol 1e-4 / atol 1e-5 elementwise for outputs,
states and per-step gradients, sums over many terms (dA, dB, dC, dD, ddelta_bias) on the
scale of the tensor; bfloat16 activations within rtol 2e-2 — plus, per element, the
problem's own float32 sensitivity: 4x the largest change of the float64 oracle when every
input is perturbed by one float32 rounding (relative 2^-24, two random draws). With
rotating states the per-step gradients are sums over the states of terms much larger than
the result (|A| |lambda| |h|), so an input rounding alone moves some elements of ddelta by
more than rtol 1e-4 of their value; a wrong or missing term still shows as an error of the
order of the element. Complex tensors are compared through their (real, imaginary) parts.

Cases: lengths inside one 512-step chunk, across chunks with ragged tails, every state
count class (1, 3, 16), variable lengths (including zero), no extras, bf16, the
reference's own A initialisation (mamba/mamba1.py:47, 162), and a grid with several
channel rounds per backward workgroup and a partial last block.
"""
import sys

import numpy as np
import pytest
import torch

from mamba_amd.selective_scan_hip import selective_scan_fn
from oracle import cscan64

pytestmark = pytest.mark.gpu

F32_RTOL, F32_ATOL = 1e-4, 1e-5
BF16_RTOL = 2e-2
dev = "cuda"
REDUCTIONS = {"dA", "dB", "dC", "dD", "ddelta_bias"}


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def as_real(a):
    a = np.asarray(a)
    return (np.stack([a.real, a.imag], -1) if np.iscomplexobj(a) else a).astype(np.float64)


def close(name, got, ref, rtol=F32_RTOL, atol=F32_ATOL, scale=None, sens=0.0):
    """|got - ref| <= atol + rtol * s + 4 * sens per element, s = |ref| or `scale` (the
    oracle's sum of |terms| of a reduction gradient, real and imaginary parts apart)."""
    if torch.is_tensor(got):
        got = got.detach()
        got = torch.view_as_real(got) if got.is_complex() else got
        got = got.float().cpu().numpy()
    ref = as_real(ref)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    s = np.abs(ref) if scale is None else as_real(scale)
    assert s.shape == ref.shape, (name, s.shape, ref.shape)
    err = np.abs(got - ref)
    bound = atol + rtol * s + 4.0 * sens
    ok = bool(np.all(err <= bound))
    worst = np.argmax(err - bound)
    log(f"  {name:16s} max_abs={err.max():.3e} worst(got={got.flat[worst]:.6e}, "
        f"ref={ref.flat[worst]:.6e}) ok={ok}")
    assert ok, f"{name}: {np.sum(err > bound)} of {err.size} elements outside rtol={rtol}, atol={atol}"


def complex_case(seed, b, d, l, n, dtype="f32", lens=None, extras=True, ref_init=False):
    rng = np.random.default_rng(seed)
    f = np.float32
    if ref_init:
        # A_log = log(1/2 - i*arange(N)), A = -exp(A_log.real) + i*A_log.imag
        a_log = np.log(0.5 - 1j * np.arange(n))
        A = np.broadcast_to(-np.exp(a_log.real) + 1j * a_log.imag, (d, n))
    else:
        A = -np.exp(rng.standard_normal((d, n))) + 2j * rng.standard_normal((d, n))
    x = dict(u=rng.standard_normal((b, d, l)).astype(f), delta=rng.standard_normal((b, d, l)).astype(f),
             A=np.ascontiguousarray(A).astype(np.complex64), B=rng.standard_normal((b, n, l)).astype(f),
             C=rng.standard_normal((b, n, l)).astype(f))
    if extras:
        x.update(D=rng.standard_normal(d).astype(f), z=rng.standard_normal((b, d, l)).astype(f),
                 delta_bias=(0.5 * rng.standard_normal(d) - 2.0).astype(f),
                 initial_state=(rng.standard_normal((b, d, n)) + 1j * rng.standard_normal((b, d, n))
                                ).astype(np.complex64))
    dout = rng.standard_normal((b, d, l)).astype(f)
    dlast = (rng.standard_normal((b, d, n)) + 1j * rng.standard_normal((b, d, n))).astype(np.complex64)
    if dtype == "bf16":
        from mamba_amd.configs import round_to_bf16
        for k in ("u", "delta", "B", "C", "z"):
            if k in x:
                x[k] = round_to_bf16(x[k])
        dout = round_to_bf16(dout)
    if lens is not None:
        x["seq_lens"] = np.asarray(lens, np.int32)
    return x, dout, dlast


def run_complex(x, dout, dlast, dtype, zoh):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    ts = {}
    for k, v in x.items():
        t = torch.as_tensor(np.ascontiguousarray(v)).to(dev)
        if k == "seq_lens":
            ts[k] = t
            continue
        if not t.is_complex():
            t = t.to(tdt if k in ("u", "delta", "z", "B", "C") else torch.float32)
        ts[k] = t.requires_grad_(True)
    out, last = selective_scan_fn(ts["u"], ts["delta"], ts["A"], ts["B"], ts["C"], D=ts.get("D"),
                                  z=ts.get("z"), delta_bias=ts.get("delta_bias"), delta_softplus=True,
                                  return_last_state=True, initial_state=ts.get("initial_state"),
                                  seq_lens=ts.get("seq_lens"), discretization="zoh" if zoh else "euler")
    assert last.dtype == torch.complex64
    dl = torch.as_tensor(dlast).to(dev)
    loss = (out.float() * torch.as_tensor(dout).to(dev)).sum()
    loss = loss + (last.real * dl.real + last.imag * dl.imag).sum()
    loss.backward()
    torch.cuda.synchronize()
    return ts, out, last


GRAD_OF = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
           "delta_bias": "ddelta_bias", "initial_state": "dinitial_state"}


def oracle(x, dout, dlast, zoh):
    kw = dict(D=x.get("D"), z=x.get("z"), delta_bias=x.get("delta_bias"), delta_softplus=True,
              initial_state=x.get("initial_state"), seq_lens=x.get("seq_lens"),
              discretization="zoh" if zoh else "euler")
    fw = cscan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"], **kw)
    g = cscan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout, dlast_state=dlast,
                         abs_terms=True, **kw)
    return {"out": fw["out"], "last_state": fw["last_state"], **g}


def sensitivity(x, dout, dlast, zoh, ref, seed):
    """Largest change of every oracle output under two one-rounding input perturbations."""
    rng = np.random.default_rng(seed)
    sens = {}
    for _ in range(2):
        xp = {k: (v if k == "seq_lens" else v * (1 + 2.0 ** -24 * rng.standard_normal(np.shape(v))))
              for k, v in x.items()}
        r = oracle(xp, dout, dlast, zoh)
        for k, v in r.items():
            if v is not None:
                sens[k] = np.maximum(sens.get(k, 0.0), np.abs(as_real(v) - as_real(ref[k])))
    return sens


def check(x, dout, dlast, zoh, dtype="f32"):
    ts, out, last = run_complex(x, dout, dlast, dtype, zoh)
    ref = oracle(x, dout, dlast, zoh)
    sens = sensitivity(x, dout, dlast, zoh, ref, seed=7)
    rtol, atol = (BF16_RTOL, BF16_RTOL * 0.05) if dtype == "bf16" else (F32_RTOL, F32_ATOL)
    close("out", out, ref["out"], rtol, atol, sens=sens["out"])
    close("last_state", last, ref["last_state"], rtol, atol, sens=sens["last_state"])
    for k, gname in GRAD_OF.items():
        if k in ts:
            close(gname, ts[k].grad, ref[gname], rtol, atol,
                  scale=ref[gname + "_abs"] if gname in REDUCTIONS else None, sens=sens[gname])


@pytest.mark.parametrize("zoh", [False, True])
@pytest.mark.parametrize("l,n", [(1, 4), (17, 16), (513, 3), (1100, 16), (2048, 1)])
def test_complex_fused(l, n, zoh):
    log(f"case complex fused L={l} N={n} zoh={zoh}")
    x, dout, dlast = complex_case(300 + l + n + zoh, 2, 5, l, n)
    check(x, dout, dlast, zoh)


@pytest.mark.parametrize("dtype,lens", [("f32", None), ("f32", [600, 317]), ("bf16", None)])
def test_complex_gate_near_zero_z(dtype, lens):
    """The complex backward takes y sigmoid(z) as out / z except where |z| < 1e-20, where it
    reads y itself, kept by the forward there only: exact zeros of both signs, |z| just under
    and over 1e-20, the zero of the gate's slope and |z| up to 100, scattered over every row."""
    log(f"case complex gate near zero z {dtype} lens={lens}")
    x, dout, dlast = complex_case(79, 2, 13, 600, 8, dtype, lens=lens)
    flat = x["z"].reshape(-1)
    specials = np.array([0.0, -0.0, 1e-30, -1e-30, 9e-21, -9e-21, 2e-20, -2e-20, 1e-6, -1e-6, -1.2785, 30.0,
                         -30.0, -100.0], np.float32)
    pos = (np.arange(0, flat.size, 7) * 131) % flat.size
    flat[pos] = specials[np.arange(pos.size) % specials.size]
    if dtype == "bf16":
        from mamba_amd.configs import round_to_bf16
        x["z"] = round_to_bf16(x["z"])
    check(x, dout, dlast, False, dtype)


@pytest.mark.parametrize("zoh", [False, True])
def test_complex_varlen(zoh):
    log(f"case complex varlen zoh={zoh}")
    x, dout, dlast = complex_case(401 + zoh, 3, 6, 1100, 8, lens=[1100, 530, 0])
    check(x, dout, dlast, zoh)


def test_complex_varlen_row_permutation():
    """Rows go to workgroups longest first: permuted rows give the permuted outputs and
    per-row gradients bit for bit."""
    log("case complex varlen row permutation")
    perm = [2, 0, 3, 1]
    x, dout, dlast = complex_case(405, 4, 6, 1100, 8, lens=[530, 1100, 0, 530])
    per_row = ("u", "delta", "z", "B", "C", "initial_state", "seq_lens")
    xp = {k: (v[perm] if k in per_row else v) for k, v in x.items()}
    a = run_complex(x, dout, dlast, "f32", False)
    b = run_complex(xp, dout[perm], dlast[perm], "f32", False)
    idx = torch.as_tensor(perm, device=dev)
    assert torch.equal(a[1][idx], b[1]) and torch.equal(a[2][idx], b[2])
    for k in per_row[:-1]:
        assert torch.equal(a[0][k].grad[idx], b[0][k].grad), k


@pytest.mark.parametrize("seed", range(6))
def test_complex_random_shapes(seed):
    """Seeded random cases of the complex scan: batch 1-3, 1-30 channels, lengths 1-1500,
    1-16 states, Euler or ZOH, with or without the fused extras and lengths, float32 or bf16;
    every output and gradient against the complex float64 oracle."""
    rng = np.random.default_rng(600 + seed)
    b, d = int(rng.integers(1, 4)), int(rng.integers(1, 31))
    l = int(rng.choice([int(rng.integers(1, 100)), int(rng.integers(100, 1501))]))
    n = int(rng.integers(1, 17))
    zoh, extras = bool(rng.random() < 0.5), bool(rng.random() < 0.7)
    dtype = "bf16" if rng.random() < 0.3 else "f32"
    lens = None
    if rng.random() < 0.4:
        lens = [int(v) for v in rng.integers(0, l + 1, size=b)]
        lens[int(rng.integers(0, b))] = int(rng.choice([0, l]))
    log(f"case complex random seed={seed}: {dtype} B={b} D={d} L={l} N={n} zoh={zoh} extras={extras} lens={lens}")
    x, dout, dlast = complex_case(650 + seed, b, d, l, n, dtype=dtype, lens=lens, extras=extras)
    check(x, dout, dlast, zoh, dtype=dtype)


def test_complex_no_extras():
    log("case complex no extras")
    x, dout, dlast = complex_case(410, 2, 4, 700, 16, extras=False)
    check(x, dout, dlast, False)


@pytest.mark.parametrize("zoh", [False, True])
def test_complex_reference_init(zoh):
    log(f"case complex reference A init zoh={zoh}")
    x, dout, dlast = complex_case(420 + zoh, 2, 8, 600, 16, ref_init=True)
    check(x, dout, dlast, zoh)


def test_complex_bf16():
    log("case complex bf16")
    x, dout, dlast = complex_case(430, 2, 6, 777, 16, dtype="bf16")
    check(x, dout, dlast, True, dtype="bf16")


def test_complex_channel_rounds():
    # batch * ceil(dim / 12) > 256 makes each backward workgroup walk two rounds of 12
    # channels; 1100 = 45 * 24 + 20 leaves the last workgroup with a partial second round.
    log("case complex channel rounds B=4 D=1100 L=64 N=4")
    x, dout, dlast = complex_case(440, 4, 1100, 64, 4)
    check(x, dout, dlast, True)
