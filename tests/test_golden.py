"""Golden fixtures at the reference tests' lengths (tests/golden/*.npz, written by
tests/golden/make_golden.py from the float64 oracle; inputs follow the reference tests'
recipe, tests/test_selective_scan_cuda.py:11-19, lengths {1, 17, 128, 513} forward and
{1, 31, 513, 2051} VJP, Euler and ZOH).

CPU: the oracle still reproduces every fixture. GPU: the HIP path (reference-signature
Python API with autograd, and the reference-signature C entry point with chunk_states)
against the fixtures: fp32 within rtol 1e-4 / atol 1e-5 per element; for dA/dB/dC (sums over
many terms) the relative part is taken of each element's sum of |terms|, which the float64
oracle returns for the fixture's inputs.
"""
import ctypes
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))
import make_golden  # noqa: E402

CASES = sorted(p.stem for p in (HERE / "golden").glob("*.npz"))


def load(name):
    with np.load(HERE / "golden" / f"{name}.npz") as f:
        return {k: f[k] for k in f.files}


def test_every_case_present():
    assert len(CASES) == 2 * (len(make_golden.FWD_LENGTHS) + len(make_golden.VJP_LENGTHS))


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    kind, disc, lt = name.split("_")
    length, euler = int(lt[1:]), disc == "euler"
    fresh = (make_golden.fwd_case if kind == "fwd" else make_golden.vjp_case)(length, euler)
    stored = load(name)
    assert set(fresh) == set(stored)
    for k in stored:
        np.testing.assert_allclose(stored[k], fresh[k], rtol=1e-12, atol=1e-12, err_msg=k)


def _check(name, got, want, scale=None):
    got = got.detach().double().cpu().numpy() if torch.is_tensor(got) else np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = 1e-5 + 1e-4 * (np.abs(want) if scale is None else np.asarray(scale, np.float64))
    assert np.all(err <= bound), f"{name}: max err {err.max():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_fixture(name):
    print(f"case golden {name}", flush=True)
    from mamba_amd import _lib
    from mamba_amd.selective_scan_hip import selective_scan

    f = load(name)
    euler = "euler" in name
    ts = {k: torch.from_numpy(f[k]).cuda().requires_grad_(True) for k in ("A", "deltas", "Bs", "Cs", "u", "x0")}
    y, fin = selective_scan(ts["A"], ts["deltas"], ts["Bs"], ts["Cs"], ts["u"], ts["x0"],
                            use_euler_barB_approx=euler)
    _check("y", y, f["y"])
    _check("final_x", fin, f["final_x"])
    if name.startswith("vjp"):
        loss = (y * torch.from_numpy(f["dy"]).cuda()).sum() + (fin * torch.from_numpy(f["dfinal_x"]).cuda()).sum()
        loss.backward()
        torch.cuda.synchronize()
        from oracle import scan64
        _, ab = scan64.reference_api_backward(f["A"], f["deltas"], f["Bs"], f["Cs"], f["u"], f["x0"], f["dy"],
                                              f["dfinal_x"], use_euler_barB_approx=euler, abs_terms=True)
        for k, g in (("A", "dA"), ("deltas", "ddeltas"), ("Bs", "dBs"), ("Cs", "dCs"), ("u", "du"), ("x0", "dx0")):
            _check(g, ts[k].grad, f[g], scale=ab.get(g))
    else:
        # reference-signature C entry point: [B][D][L] layouts and chunk_states
        lib = _lib.register_hip_kernel()
        t = lambda a: torch.from_numpy(np.ascontiguousarray(np.swapaxes(a, 1, 2))).cuda()
        b, l, d = f["u"].shape
        n = f["A"].shape[1]
        yk = torch.empty(b, d, l, device="cuda")
        fk = torch.empty(b, d, n, device="cuda")
        ck = torch.empty(b, d, (l + 2047) // 2048, n, 2, device="cuda")
        ins = [torch.from_numpy(f["A"]).cuda(), t(f["deltas"]), t(f["Bs"]), t(f["Cs"]), t(f["u"]),
               torch.from_numpy(f["x0"]).cuda()]
        P = lambda x: ctypes.c_void_p(x.data_ptr())
        st = lib.mss_scan_fwd(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), 0 if euler else 1, b, l, d, n,
                              *[P(x) for x in ins], P(yk), P(fk), P(ck))
        assert st == 0, lib.mss_strerror(st)
        torch.cuda.synchronize()
        _check("y (C ABI)", yk.transpose(1, 2), f["y"])
        _check("chunk_states", ck, f["chunk_states"])
