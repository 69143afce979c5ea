"""Pins the float64 oracle (oracle/scan64.py) before any GPU result is compared with it.

Each check is chosen so a plausible mistake (dropped term, wrong sign or index, swapped
operands in the non-commutative compose, off-by-one in the adjoint shift) fails:
  * an independent restatement of the reference's associative scan (oracle/assoc_torch.py,
    mamba/selective_scan_cuda.py:56-90) at the reference test lengths;
  * closed forms: delta = 0, u = 0, A = 0 (cumsum), constant coefficients (geometric
    series), L = 1;
  * invariants: linearity in (u, x0), split invariance through initial/final state,
    variable length == per-row unpadded run, reference chunk residual = (prod a, h);
  * backward: torch float64 autograd of an independent loop, and central differences.
"""
import numpy as np
import pytest
import torch

from oracle import assoc_torch, scan64

RTOL = 2e-5  # tolerance of the reference's own CPU test, tests/test_selective_scan_cuda.py:51-52


def ref_recipe(rng, batch=2, length=17, dim=8, n=16):
    """Input recipe of the reference tests (tests/test_selective_scan_cuda.py:11-19)."""
    A = -np.exp(rng.standard_normal((dim, n)))
    deltas = np.log1p(np.exp(rng.standard_normal((batch, length, dim))))
    Bs = rng.standard_normal((batch, length, n))
    Cs = rng.standard_normal((batch, length, n))
    u = rng.standard_normal((batch, length, dim))
    x0 = rng.standard_normal((batch, dim, n))
    return A, deltas, Bs, Cs, u, x0


@pytest.mark.parametrize("length", [1, 2, 17, 31, 128, 513])
@pytest.mark.parametrize("euler", [True, False])
def test_sequential_matches_associative_reference(length, euler):
    rng = np.random.default_rng(length)
    args = ref_recipe(rng, length=length)
    y, fin, _ = scan64.reference_api_forward(*args, use_euler_barB_approx=euler)
    T = lambda a: torch.tensor(a, dtype=torch.float64)
    y2, fin2 = assoc_torch.selective_scan_reference(*map(T, args), use_euler_barB_approx=euler)
    np.testing.assert_allclose(y, y2.numpy(), rtol=RTOL, atol=RTOL)
    np.testing.assert_allclose(fin, fin2.numpy(), rtol=RTOL, atol=RTOL)


def fused_inputs(rng, b=2, d=3, l=23, n=4):
    return dict(
        u=rng.standard_normal((b, d, l)), delta=rng.standard_normal((b, d, l)),
        A=-np.exp(rng.standard_normal((d, n))), B=rng.standard_normal((b, n, l)),
        C=rng.standard_normal((b, n, l)), D=rng.standard_normal(d), z=rng.standard_normal((b, d, l)),
        delta_bias=0.5 * rng.standard_normal(d), initial_state=rng.standard_normal((b, d, n)))


def test_zero_delta_freezes_state():
    rng = np.random.default_rng(0)
    x = fused_inputs(rng)
    x["delta"][:] = 0.0
    r = scan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"],
                       initial_state=x["initial_state"])
    np.testing.assert_allclose(r["last_state"], x["initial_state"], rtol=1e-15)
    y = np.einsum("bnl,bdn->bdl", x["C"], x["initial_state"]) + x["D"][None, :, None] * x["u"]
    np.testing.assert_allclose(r["y"], y, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("disc", ["euler", "zoh"])
def test_zero_input_is_pure_decay(disc):
    rng = np.random.default_rng(1)
    x = fused_inputs(rng)
    x["u"][:] = 0.0
    dl = np.log1p(np.exp(x["delta"]))
    r = scan64.forward(x["u"], dl, x["A"], x["B"], x["C"], initial_state=x["initial_state"],
                       discretization=disc)
    expect = np.exp(x["A"][None] * dl.sum(-1)[..., None]) * x["initial_state"]
    np.testing.assert_allclose(r["last_state"], expect, rtol=1e-12)


def test_zero_A_euler_is_cumsum():
    rng = np.random.default_rng(2)
    b, d, l = 2, 3, 40
    u = rng.standard_normal((b, d, l))
    dl = np.abs(rng.standard_normal((b, d, l)))
    B = rng.standard_normal((b, 1, l))
    C = np.ones((b, 1, l))
    x0 = rng.standard_normal((b, d, 1))
    r = scan64.forward(u, dl, np.zeros((d, 1)), B, C, initial_state=x0)
    h = x0[..., 0][..., None] + np.cumsum(dl * B * u, axis=-1)
    np.testing.assert_allclose(r["y"], h, rtol=1e-12, atol=1e-12)


def test_constant_coefficients_geometric_series():
    b, d, l, n = 1, 2, 30, 3
    dl = np.full((b, d, l), 0.3)
    A = -np.array([[0.5, 1.0, 2.0], [0.1, 0.2, 3.0]])
    u = np.ones((b, d, l))
    B = np.full((b, n, l), 0.7)
    C = np.ones((b, n, l))
    x0 = np.full((b, d, n), 1.5)
    r = scan64.forward(u, dl, A, B, C, initial_state=x0)
    a = np.exp(0.3 * A)[None]
    bb = 0.3 * 0.7
    t = l
    expect = a ** t * x0 + bb * (1 - a ** t) / (1 - a)
    np.testing.assert_allclose(r["last_state"], expect, rtol=1e-12)


@pytest.mark.parametrize("disc", ["euler", "zoh"])
def test_length_one(disc):
    rng = np.random.default_rng(3)
    x = fused_inputs(rng, l=1)
    dl = np.log1p(np.exp(x["delta"]))
    r = scan64.forward(x["u"], dl, x["A"], x["B"], x["C"], initial_state=x["initial_state"],
                       discretization=disc)
    dA = dl[..., 0][..., None] * x["A"][None]
    bbar = (np.expm1(dA) / x["A"][None]) if disc == "zoh" else dl[..., 0][..., None]
    h = np.exp(dA) * x["initial_state"] + bbar * x["B"][:, None, :, 0] * x["u"][..., 0][..., None]
    np.testing.assert_allclose(r["last_state"], h, rtol=1e-13)


def test_linearity_in_u_and_state():
    rng = np.random.default_rng(4)
    x = fused_inputs(rng)
    dl = np.log1p(np.exp(x["delta"]))
    f = lambda u, x0: scan64.forward(u, dl, x["A"], x["B"], x["C"], initial_state=x0)
    u2 = rng.standard_normal(x["u"].shape)
    s2 = rng.standard_normal(x["initial_state"].shape)
    r1, r2 = f(x["u"], x["initial_state"]), f(u2, s2)
    r12 = f(2.0 * x["u"] - 3.0 * u2, 2.0 * x["initial_state"] - 3.0 * s2)
    np.testing.assert_allclose(r12["y"], 2 * r1["y"] - 3 * r2["y"], rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("split", [1, 7, 22])
def test_split_invariance(split):
    rng = np.random.default_rng(5)
    x = fused_inputs(rng)
    kw = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    full = scan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"],
                          initial_state=x["initial_state"], **kw)
    s = slice(0, split)
    t = slice(split, None)
    p1 = scan64.forward(x["u"][..., s], x["delta"][..., s], x["A"], x["B"][..., s], x["C"][..., s],
                        initial_state=x["initial_state"], **{**kw, "z": x["z"][..., s]})
    p2 = scan64.forward(x["u"][..., t], x["delta"][..., t], x["A"], x["B"][..., t], x["C"][..., t],
                        initial_state=p1["last_state"], **{**kw, "z": x["z"][..., t]})
    np.testing.assert_allclose(np.concatenate([p1["out"], p2["out"]], -1), full["out"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(p2["last_state"], full["last_state"], rtol=1e-12)


def test_varlen_equals_unpadded_rows():
    rng = np.random.default_rng(6)
    x = fused_inputs(rng, b=3, l=29)
    lens = np.array([29, 11, 0])
    kw = dict(D=x["D"], delta_bias=x["delta_bias"], delta_softplus=True)
    r = scan64.forward(x["u"], x["delta"], x["A"], x["B"], x["C"], z=x["z"],
                       initial_state=x["initial_state"], seq_lens=lens, **kw)
    for bi, n_ in enumerate(lens):
        sl = lambda a: a[bi:bi + 1, ..., :n_]
        if n_ == 0:
            np.testing.assert_allclose(r["last_state"][bi], x["initial_state"][bi])
            assert np.all(r["out"][bi] == 0)
            continue
        rr = scan64.forward(sl(x["u"]), sl(x["delta"]), x["A"], sl(x["B"]), sl(x["C"]), z=sl(x["z"]),
                            initial_state=x["initial_state"][bi:bi + 1], **kw)
        np.testing.assert_allclose(r["out"][bi, :, :n_], rr["out"][0], rtol=1e-13, atol=1e-13)
        assert np.all(r["out"][bi, :, n_:] == 0)
        np.testing.assert_allclose(r["last_state"][bi], rr["last_state"][0], rtol=1e-13)


def test_reference_chunk_states():
    rng = np.random.default_rng(7)
    b, d, l, n = 1, 2, 4100, 2
    dl = 0.01 * np.abs(rng.standard_normal((b, d, l)))
    A = -np.abs(rng.standard_normal((d, n)))
    r = scan64.forward(rng.standard_normal((b, d, l)), dl, A, rng.standard_normal((b, n, l)),
                       rng.standard_normal((b, n, l)))
    cs = r["ref_chunk_states"]
    assert cs.shape == (b, d, 3, n, 2)
    ends = [2047, 4095, 4099]
    for c, e in enumerate(ends):
        np.testing.assert_allclose(cs[:, :, c, :, 0], np.exp(A[None] * dl[..., :e + 1].sum(-1)[..., None]), rtol=1e-10)
    np.testing.assert_allclose(cs[:, :, 2, :, 1], r["last_state"])


# --------------------------------------------------------------------------- backward
def torch_loop(u, dr, A, B, C, D, z, bias, x0, lens, softplus, zoh):
    """Independent float64 forward (per-step loop) for autograd."""
    L = u.shape[-1]
    x = dr + bias[None, :, None]
    dl = torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20)))) if softplus else x
    mask = (torch.arange(L)[None, :] < torch.as_tensor(lens)[:, None]).double()
    dl = dl * mask[:, None, :]
    h = x0
    ys = []
    for t in range(L):
        dA = dl[:, :, t, None] * A[None]
        E = torch.expm1(dA) / A[None] if zoh else dl[:, :, t, None]
        h = torch.exp(dA) * h + E * B[:, None, :, t] * u[:, :, t, None]
        ys.append((C[:, None, :, t] * h).sum(-1))
    y = torch.stack(ys, -1) + D[None, :, None] * u
    return y * z * torch.sigmoid(z) * mask[:, None, :], h


@pytest.mark.parametrize("zoh", [False, True])
@pytest.mark.parametrize("lens", [[37, 37], [37, 20], [5, 0]])
def test_backward_matches_autograd(zoh, lens):
    rng = np.random.default_rng(8)
    b, d, l, n = 2, 3, 37, 4
    vals = [rng.standard_normal((b, d, l)), rng.standard_normal((b, d, l)), -np.exp(rng.standard_normal((d, n))),
            rng.standard_normal((b, n, l)), rng.standard_normal((b, n, l)), rng.standard_normal(d),
            rng.standard_normal((b, d, l)), 0.5 * rng.standard_normal(d), rng.standard_normal((b, d, n))]
    dout = rng.standard_normal((b, d, l))
    dlast = rng.standard_normal((b, d, n))
    ts = [torch.tensor(v, requires_grad=True) for v in vals]
    out, h = torch_loop(*ts, lens, True, zoh)
    ((out * torch.tensor(dout)).sum() + (h * torch.tensor(dlast)).sum()).backward()
    u, dr, A, B, C, D, z, bias, x0 = vals
    g = scan64.backward(u, dr, A, B, C, dout, D=D, z=z, delta_bias=bias, delta_softplus=True,
                        initial_state=x0, seq_lens=lens, discretization="zoh" if zoh else "euler",
                        dlast_state=dlast, segment=8)
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias", "dinitial_state"]
    for name, t in zip(names, ts):
        np.testing.assert_allclose(g[name], t.grad.numpy(), rtol=1e-10, atol=1e-10, err_msg=name)


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(9)
    b, d, l, n = 1, 2, 9, 3
    x = dict(u=rng.standard_normal((b, d, l)), delta=rng.standard_normal((b, d, l)),
             A=-np.exp(rng.standard_normal((d, n))), B=rng.standard_normal((b, n, l)),
             C=rng.standard_normal((b, n, l)), D=rng.standard_normal(d), z=rng.standard_normal((b, d, l)),
             delta_bias=0.3 * rng.standard_normal(d), initial_state=rng.standard_normal((b, d, n)))
    dout = rng.standard_normal((b, d, l))
    dlast = rng.standard_normal((b, d, n))

    def loss(v):
        r = scan64.forward(v["u"], v["delta"], v["A"], v["B"], v["C"], D=v["D"], z=v["z"],
                           delta_bias=v["delta_bias"], delta_softplus=True,
                           initial_state=v["initial_state"])
        return np.sum(r["out"] * dout) + np.sum(r["last_state"] * dlast)

    g = scan64.backward(x["u"], x["delta"], x["A"], x["B"], x["C"], dout, D=x["D"], z=x["z"],
                        delta_bias=x["delta_bias"], delta_softplus=True,
                        initial_state=x["initial_state"], dlast_state=dlast)
    key = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
           "delta_bias": "ddelta_bias", "initial_state": "dinitial_state"}
    eps = 1e-6
    for name, gname in key.items():
        flat = x[name].reshape(-1)
        for idx in range(0, flat.size, max(1, flat.size // 5)):
            vp = {k: v.copy() for k, v in x.items()}
            vm = {k: v.copy() for k, v in x.items()}
            vp[name].reshape(-1)[idx] += eps
            vm[name].reshape(-1)[idx] -= eps
            fd = (loss(vp) - loss(vm)) / (2 * eps)
            np.testing.assert_allclose(g[gname].reshape(-1)[idx], fd, rtol=1e-6, atol=1e-7,
                                       err_msg=f"{gname}[{idx}]")


def test_reference_api_backward_shapes_and_layout():
    rng = np.random.default_rng(10)
    A, deltas, Bs, Cs, u, x0 = ref_recipe(rng, batch=1, length=31, dim=4, n=8)
    dy = rng.standard_normal(u.shape)
    dfin = rng.standard_normal(x0.shape)
    dA, dd, dB, dC, du, dx0 = scan64.reference_api_backward(A, deltas, Bs, Cs, u, x0, dy, dfin)
    assert dA.shape == A.shape and dd.shape == deltas.shape and dB.shape == Bs.shape
    assert dC.shape == Cs.shape and du.shape == u.shape and dx0.shape == x0.shape
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    ts = [T(a) for a in (A, deltas, Bs, Cs, u, x0)]
    y, fin = assoc_torch.selective_scan_reference(*ts)
    ((y * torch.tensor(dy)).sum() + (fin * torch.tensor(dfin)).sum()).backward()
    for got, t in zip((dA, dd, dB, dC, du, dx0), ts):
        np.testing.assert_allclose(got, t.grad.numpy(), rtol=1e-10, atol=1e-10)


def _case_inputs(seed, b, d, l, n, extras, lens):
    rng = np.random.default_rng(seed)
    x = dict(u=rng.standard_normal((b, d, l)), delta=rng.standard_normal((b, d, l)),
             A=-np.exp(rng.standard_normal((d, n))), B=rng.standard_normal((b, n, l)),
             C=rng.standard_normal((b, n, l)))
    kw = {}
    if extras:
        kw = dict(D=rng.standard_normal(d), z=rng.standard_normal((b, d, l)),
                  delta_bias=0.5 * rng.standard_normal(d) - 2.0, initial_state=rng.standard_normal((b, d, n)),
                  delta_softplus=True)
    else:
        x["delta"] = np.abs(x["delta"]) * 0.1
    if lens is not None:
        kw["seq_lens"] = np.asarray(lens, np.int32)
    return x, kw, rng.standard_normal((b, d, l)), rng.standard_normal((b, d, n))


@pytest.mark.parametrize("disc", ["euler", "zoh"])
@pytest.mark.parametrize("extras,lens", [(True, None), (True, [300, 17, 0]), (False, None)])
def test_c_oracle_matches_numpy_oracle(disc, extras, lens):
    """The C restatement (oracle/scan64c.c, used by the GPU tests at full size) against the numpy
    oracle: every output, gradient and |term| sum, to float64 rounding."""
    from oracle import scan64c
    x, kw, dout, dlast = _case_inputs(31, 3, 5, 300, 7, extras, lens)
    f1 = scan64.forward(**x, **kw, discretization=disc)
    f2 = scan64c.forward(**x, **kw, discretization=disc)
    for k in ("out", "y", "last_state", "ref_chunk_states"):
        np.testing.assert_allclose(f2[k], f1[k], rtol=1e-12, atol=1e-13 * np.abs(f1[k]).max())
    g1 = scan64.backward(**x, dout=dout, **kw, discretization=disc, dlast_state=dlast, abs_terms=True)
    g2 = scan64c.backward(**x, dout=dout, **kw, discretization=disc, dlast_state=dlast, abs_terms=True)
    assert g1.keys() == g2.keys()
    for k in g1:
        if g1[k] is None:
            assert g2[k] is None, k
            continue
        np.testing.assert_allclose(g2[k], g1[k], rtol=1e-10, atol=1e-12 * np.abs(g1[k]).max(), err_msg=k)


def test_abs_term_sums_bound_the_reduction_gradients():
    """|sum of terms| <= sum of |terms| everywhere, with equality where every term has one sign:
    dD = sum g u with z absent and dout = sign(u) makes every term g u = |u| >= 0."""
    x, kw, dout, dlast = _case_inputs(32, 2, 4, 90, 5, True, None)
    g = scan64.backward(**x, dout=dout, **kw, dlast_state=dlast, abs_terms=True)
    for k in ("dA", "dB", "dC", "dD", "ddelta_bias"):
        assert np.all(np.abs(g[k]) <= g[k + "_abs"] * (1 + 1e-12)), k
        assert np.all(g[k + "_abs"] > 0), k
    kw.pop("z")
    g = scan64.backward(**x, dout=np.sign(x["u"]), **kw, abs_terms=True)
    np.testing.assert_allclose(g["dD"], g["dD_abs"], rtol=1e-12)
