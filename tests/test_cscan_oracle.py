"""Pins the complex-SSM float64 oracle (oracle/cscan64.py) before GPU results are compared with it.

Checks chosen so a plausible mistake fails one of them:
  * the reference's own formulation, ``mamba/mamba1.py:143-176`` (complex discretise, affine
    associative scan over (a_bar, B_bar x), einsum with C, ``+ D x``, real part), restated in
    torch complex128 over the odd/even associative scan of oracle/assoc_torch.py — catches a
    conjugation, a dropped imaginary part or a swapped compose;
  * reductions and closed forms: Im(A) = 0 equals the pinned real oracle (forward and every
    gradient); constant complex coefficients are a geometric series; ZOH's b_bar equals the
    integral of exp(sA) over [0, delta] by quadrature; real inputs give conjugate states under
    A -> conj(A), so ``out`` is unchanged;
  * backward: torch complex128 autograd of an independent loop with Re(A), Im(A) and the
    initial state as separate real leaves (no reliance on torch's complex-gradient convention),
    and central finite differences.
"""
import numpy as np
import pytest
import torch
from scipy import integrate

from oracle import assoc_torch, cscan64, scan64


def complex_inputs(rng, b=2, d=3, l=23, n=4, imag_scale=2.0):
    return dict(
        u=rng.standard_normal((b, d, l)), delta=rng.standard_normal((b, d, l)),
        A=-np.exp(rng.standard_normal((d, n))) + 1j * imag_scale * rng.standard_normal((d, n)),
        B=rng.standard_normal((b, n, l)), C=rng.standard_normal((b, n, l)),
        D=rng.standard_normal(d), z=rng.standard_normal((b, d, l)),
        delta_bias=0.5 * rng.standard_normal(d),
        initial_state=rng.standard_normal((b, d, n)) + 1j * rng.standard_normal((b, d, n)))


def reference_formulation(A, deltas, Bs, Cs, x, D, zoh):
    """mamba/mamba1.py:143-176, 195-198 in torch complex128; layouts (B, L, D) / (B, L, N)."""
    T = lambda a: torch.tensor(a)
    A, deltas, Bs, Cs, x = T(A), T(deltas), T(Bs), T(Cs), T(x)
    mul = deltas.to(torch.complex128)[..., None] * A[None, None]
    a_bars = torch.exp(mul)
    if zoh:
        b_bars = ((torch.exp(mul) - 1) / A[None, None]) * Bs[:, :, None, :]
    else:
        b_bars = deltas[..., None] * Bs[:, :, None, :]
    bx = (b_bars * x[..., None]).to(torch.complex128)
    _, xs = assoc_torch.associative_scan(assoc_torch._compose, (a_bars, bx), dim=1)
    ys = torch.einsum("bln,bldn->bld", Cs.to(torch.complex128), xs)
    ys = ys + T(D) * x
    return ys.real.numpy(), xs[:, -1].numpy()


@pytest.mark.parametrize("length", [1, 2, 17, 64])
@pytest.mark.parametrize("zoh", [False, True])
def test_matches_reference_formulation(length, zoh):
    rng = np.random.default_rng(100 + length + zoh)
    x = complex_inputs(rng, l=length)
    dl = np.log1p(np.exp(x["delta"]))
    r = cscan64.forward(x["u"], dl, x["A"], x["B"], x["C"], D=x["D"],
                        discretization="zoh" if zoh else "euler")
    tr = lambda a: np.ascontiguousarray(np.swapaxes(a, 1, 2))
    ys, last = reference_formulation(x["A"], tr(dl), tr(x["B"]), tr(x["C"]), tr(x["u"]), x["D"], zoh)
    np.testing.assert_allclose(r["y"], tr(ys), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(r["last_state"], last, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("disc", ["euler", "zoh"])
def test_real_A_reduces_to_real_scan(disc):
    rng = np.random.default_rng(7)
    x = complex_inputs(rng)
    x["A"] = x["A"].real + 0j
    x["initial_state"] = x["initial_state"].real + 0j
    lens = [23, 9]
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True, seq_lens=lens,
              discretization=disc)
    dout = rng.standard_normal(x["u"].shape)
    dlast = rng.standard_normal(x["initial_state"].shape)
    c = cscan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"],
                        initial_state=x["initial_state"], **kw)
    r = scan64.forward(x["u"], x["delta"], x["A"].real, x["B"], x["C"],
                       initial_state=x["initial_state"].real, **kw)
    np.testing.assert_allclose(c["out"], r["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(c["last_state"], r["last_state"], rtol=1e-12, atol=1e-12)
    gc = cscan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout,
                          initial_state=x["initial_state"], dlast_state=dlast + 0j, abs_terms=True, **kw)
    gr = scan64.backward(x["u"], x["delta"], x["A"].real, x["B"], x["C"], dout,
                         initial_state=x["initial_state"].real, dlast_state=dlast, abs_terms=True, **kw)
    for k in ("du", "ddelta", "dB", "dC", "dD", "dz", "ddelta_bias"):
        np.testing.assert_allclose(gc[k], gr[k], rtol=1e-11, atol=1e-11, err_msg=k)
    np.testing.assert_allclose(gc["dA"].real, gr["dA"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(gc["dinitial_state"], gr["dinitial_state"], rtol=1e-11, atol=1e-11)
    # the |term| sums of the reduction gradients decompose into the real scan's terms too
    for k in ("dB_abs", "dC_abs", "dD_abs", "ddelta_bias_abs"):
        np.testing.assert_allclose(gc[k], gr[k], rtol=1e-11, atol=1e-11, err_msg=k)
    np.testing.assert_allclose(gc["dA_abs"].real, gr["dA_abs"], rtol=1e-11, atol=1e-11)
    assert np.all(gc["dA_abs"].imag == 0)


@pytest.mark.parametrize("zoh", [False, True])
def test_abs_term_sums_bound_the_reduction_gradients(zoh):
    """|sum of terms| <= sum of |terms| for every reduction gradient (real and imaginary
    parts of dA apart), the gradients themselves unchanged by abs_terms, and equality where
    every term has one sign: dD = sum g u with z absent and dout = sign(u)."""
    rng = np.random.default_rng(40 + zoh)
    x = complex_inputs(rng)
    dout = rng.standard_normal(x["u"].shape)
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True, seq_lens=[23, 17],
              initial_state=x["initial_state"], discretization="zoh" if zoh else "euler")
    args = (x["u"], x["delta"], x["A"], x["B"], x["C"], dout)
    g = cscan64.backward(*args, abs_terms=True, **kw)
    g0 = cscan64.backward(*args, **kw)
    for k in g0:
        if g0[k] is not None:
            assert np.array_equal(g[k], g0[k]), k
    for k in ("dB", "dC", "dD", "ddelta_bias"):
        assert np.all(np.abs(g[k]) <= g[k + "_abs"] * (1 + 1e-12)), k
    assert np.all(np.abs(g["dA"].real) <= g["dA_abs"].real * (1 + 1e-12))
    assert np.all(np.abs(g["dA"].imag) <= g["dA_abs"].imag * (1 + 1e-12))
    kw.pop("z")
    g = cscan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], np.sign(x["u"]), abs_terms=True, **kw)
    np.testing.assert_allclose(g["dD"], g["dD_abs"], rtol=1e-12)


def test_constant_coefficients_geometric_series():
    b, d, l, n = 1, 2, 30, 3
    dl = np.full((b, d, l), 0.3)
    A = np.array([[-0.5 + 1.0j, -1.0 - 2.5j, -2.0 + 0.1j], [-0.1 + 3.0j, -0.2, -3.0 - 1.0j]])
    u = np.ones((b, d, l))
    B = np.full((b, n, l), 0.7)
    C = np.ones((b, n, l))
    x0 = np.full((b, d, n), 1.5 - 0.5j)
    r = cscan64.forward(u, dl, A, B, C, initial_state=x0)
    a = np.exp(0.3 * A)[None]
    expect = a ** l * x0 + 0.3 * 0.7 * (1 - a ** l) / (1 - a)
    np.testing.assert_allclose(r["last_state"], expect, rtol=1e-12)


def test_zoh_bbar_is_integral_of_exp():
    rng = np.random.default_rng(9)
    x = complex_inputs(rng, b=1, d=2, l=1, n=3)
    dl = np.abs(x["delta"]) + 0.1
    r = cscan64.forward(x["u"], dl, x["A"], x["B"], x["C"], discretization="zoh")
    for d in range(2):
        for k in range(3):
            a, t = x["A"][d, k], dl[0, d, 0]
            re = integrate.quad(lambda s: np.exp(s * a).real, 0.0, t, epsabs=1e-13)[0]
            im = integrate.quad(lambda s: np.exp(s * a).imag, 0.0, t, epsabs=1e-13)[0]
            expect = (re + 1j * im) * x["B"][0, k, 0] * x["u"][0, d, 0]
            np.testing.assert_allclose(r["last_state"][0, d, k], expect, rtol=1e-10)


def test_conjugate_A_leaves_output_unchanged():
    rng = np.random.default_rng(11)
    x = complex_inputs(rng)
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True,
              discretization="zoh")
    r1 = cscan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"],
                         initial_state=x["initial_state"], **kw)
    r2 = cscan64.forward(x["u"], x["delta"], np.conj(x["A"]), x["B"], x["C"],
                         initial_state=np.conj(x["initial_state"]), **kw)
    np.testing.assert_allclose(r1["out"], r2["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r1["last_state"], np.conj(r2["last_state"]), rtol=1e-12)


def torch_loop_loss(t, dout, dlast, zoh, lens):
    """Independent torch loop; real leaves Ar, Ai, h0r, h0i. Returns the scalar loss."""
    bias = t["delta_bias"]
    xr = t["delta"] + bias[None, :, None]
    dl = torch.nn.functional.softplus(xr)  # threshold 20 as the oracle's
    L = t["u"].shape[-1]
    mask = (torch.arange(L)[None, :] < torch.tensor(lens)[:, None]).double()
    dl = dl * mask[:, None, :]
    A = torch.complex(t["Ar"], t["Ai"])
    h = torch.complex(t["h0r"], t["h0i"])
    ys = []
    for s in range(L):
        w = dl[:, :, s, None] * A[None]
        a = torch.exp(w)
        if zoh:
            bb = (torch.exp(w) - 1) / A[None]
        else:
            bb = dl[:, :, s, None].to(torch.complex128)
        h = a * h + bb * (t["B"][:, None, :, s] * t["u"][:, :, s, None])
        ys.append((t["C"][:, None, :, s] * h.real).sum(-1))
    y = torch.stack(ys, -1) + t["D"][None, :, None] * t["u"]
    out = y * torch.nn.functional.silu(t["z"]) * mask[:, None, :]
    return (out * dout).sum() + (h.real * dlast.real + h.imag * dlast.imag).sum()


@pytest.mark.parametrize("zoh", [False, True])
@pytest.mark.parametrize("lens", [[23, 23], [23, 11]])
def test_backward_matches_autograd(zoh, lens):
    rng = np.random.default_rng(20 + zoh)
    x = complex_inputs(rng)
    dout = rng.standard_normal(x["u"].shape)
    dlast = rng.standard_normal(x["initial_state"].shape) + 1j * rng.standard_normal(x["initial_state"].shape)
    disc = "zoh" if zoh else "euler"
    g = cscan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout, D=x["D"], z=x["z"],
                         delta_bias=x["delta_bias"], delta_softplus=True,
                         initial_state=x["initial_state"], seq_lens=lens, discretization=disc,
                         dlast_state=dlast)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    t = {k: T(x[k]) for k in ("u", "delta", "B", "C", "D", "z", "delta_bias")}
    t.update(Ar=T(x["A"].real), Ai=T(x["A"].imag), h0r=T(x["initial_state"].real),
             h0i=T(x["initial_state"].imag))
    loss = torch_loop_loss(t, torch.tensor(dout), torch.tensor(dlast), zoh, lens)
    loss.backward()
    chk = lambda got, ref, name: np.testing.assert_allclose(got, ref.grad.numpy(), rtol=1e-9,
                                                           atol=1e-10, err_msg=name)
    chk(g["du"], t["u"], "du")
    chk(g["ddelta"], t["delta"], "ddelta")
    chk(g["dB"], t["B"], "dB")
    chk(g["dC"], t["C"], "dC")
    chk(g["dD"], t["D"], "dD")
    chk(g["dz"], t["z"], "dz")
    chk(g["ddelta_bias"], t["delta_bias"], "ddelta_bias")
    chk(g["dA"].real, t["Ar"], "dA.real")
    chk(g["dA"].imag, t["Ai"], "dA.imag")
    chk(g["dinitial_state"].real, t["h0r"], "dh0.real")
    chk(g["dinitial_state"].imag, t["h0i"], "dh0.imag")


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(31)
    x = complex_inputs(rng, b=1, d=2, l=9, n=3)
    dout = rng.standard_normal(x["u"].shape)
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True,
              discretization="zoh")

    def loss(xx):
        r = cscan64.forward(xx["u"], xx["delta"], xx["A"], xx["B"], xx["C"],
                            initial_state=xx["initial_state"],
                            **{**kw, "D": xx["D"], "z": xx["z"], "delta_bias": xx["delta_bias"]})
        return float(np.sum(r["out"] * dout))

    g = cscan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout,
                         initial_state=x["initial_state"], **kw)
    eps = 1e-6
    probes = [("u", (0, 1, 4), None), ("delta", (0, 0, 7), "ddelta"), ("B", (0, 2, 3), None),
              ("C", (0, 1, 8), None), ("A", (1, 2), "re"), ("A", (0, 1), "im"),
              ("initial_state", (0, 1, 2), "re"), ("initial_state", (0, 0, 1), "im")]
    for key, idx, part in probes:
        step = 1j * eps if part == "im" else eps
        xp = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in x.items()}
        xm = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in x.items()}
        xp[key][idx] += step
        xm[key][idx] -= step
        fd = (loss(xp) - loss(xm)) / (2 * eps)
        gk = {"A": "dA", "initial_state": "dinitial_state"}.get(key, "d" + key)
        if part == "ddelta":
            gk = "ddelta"
        got = g[gk][idx]
        got = got.imag if part == "im" else got.real
        np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-8, err_msg=f"{key}{idx}{part}")
