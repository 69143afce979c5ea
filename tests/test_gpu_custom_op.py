"""The torch.library registration of the scan on the GPU: torch.library.opcheck (schema,
fake implementation, autograd registration) on real and complex A, and a torch.compile
trace (aot_eager: dynamo + AOT autograd over the custom ops, no code generation) that must
give the eager results bit for bit."""
import numpy as np
import pytest
import torch

from mamba_amd.selective_scan_hip import selective_scan_fn

pytestmark = pytest.mark.gpu


def inputs(cplx, seed=0, b=2, d=4, l=70, n=4):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    A = -torch.exp(r(d, n))
    if cplx:
        A = torch.complex(A, 2 * r(d, n))
    x0 = torch.complex(r(b, d, n), r(b, d, n)) if cplx else r(b, d, n)
    t = dict(u=r(b, d, l), delta=r(b, d, l), A=A, B=r(b, n, l), C=r(b, n, l), D=r(d), z=r(b, d, l),
             delta_bias=0.5 * r(d), initial_state=x0)
    return {k: v.cuda().requires_grad_(True) for k, v in t.items()}


@pytest.mark.parametrize("cplx", [False, True])
def test_opcheck(cplx):
    print(f"case opcheck complex={cplx}", flush=True)
    t = inputs(cplx)
    args = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["z"], t["delta_bias"], t["initial_state"],
            None, True, False)
    torch.library.opcheck(torch.ops.mamba_amd.selective_scan_fwd, args,
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


def _run(fn, t, dout):
    out, last = fn(t)
    loss = (out * dout).sum() + (torch.view_as_real(last) if last.is_complex() else last).sum()
    grads = torch.autograd.grad(loss, list(t.values()))
    return out.detach(), last.detach(), [g.detach() for g in grads]


@pytest.mark.parametrize("cplx", [False, True])
def test_compile_matches_eager(cplx):
    print(f"case torch.compile complex={cplx}", flush=True)
    t = inputs(cplx, seed=1)
    dout = torch.randn(t["u"].shape, device="cuda")

    def fn(t):
        return selective_scan_fn(t["u"], t["delta"], t["A"], t["B"], t["C"], D=t["D"], z=t["z"],
                                 delta_bias=t["delta_bias"], delta_softplus=True, return_last_state=True,
                                 initial_state=t["initial_state"])

    eager = _run(fn, t, dout)
    compiled = _run(torch.compile(fn, backend="aot_eager", fullgraph=True), t, dout)
    torch.cuda.synchronize()
    assert torch.equal(eager[0], compiled[0]) and torch.equal(eager[1], compiled[1])
    for a, b in zip(eager[2], compiled[2]):
        assert torch.equal(a, b)
