"""mss_bwd_noalloc: the backward with its workspace in the library's fixed per-device scratch
(for callers that cannot allocate) against mss_bwd with a caller workspace, through the C ABI.

Two calls in a row, the second with a smaller input (the scratch keeps the first call's
contents; nothing in the backward may read what an earlier call left). Every output must
equal mss_bwd's bit for bit: the same kernels run with the same launch plan.
"""
import sys

import numpy as np
import pytest
import torch

from mamba_amd import _lib

pytestmark = pytest.mark.gpu

dev = "cuda"


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(seed, b, d, l, n, lens=None):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(dev)
    x = dict(u=r(b, d, l), delta=r(b, d, l), A=-torch.exp(r(d, n)), B=r(b, n, l), C=r(b, n, l), D=r(d), z=r(b, d, l),
             delta_bias=0.5 * r(d) - 2.0, initial_state=r(b, d, n))
    x["seq_lens"] = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=dev)
    return x, r(b, d, l), r(b, d, n)


def _forward(lib, x, b, d, l, n):
    n_seg = (l + _lib.MSS_SEG_STEPS - 1) // _lib.MSS_SEG_STEPS
    out = torch.empty(b, d, l, device=dev)
    last = torch.empty(b, d, n, device=dev)
    carries = torch.empty(b, d, n, n_seg, device=dev)
    y_pre = torch.empty(b, d, l, device=dev)
    p = lambda t: None if t is None else t.data_ptr()
    fa = _lib.FwdArgs(batch=b, dim=d, seqlen=l, dstate=n, discretization=_lib.MSS_EULER, delta_softplus=1,
                      io_dtype=_lib.MSS_F32, bc_dtype=_lib.MSS_F32, u=p(x["u"]), delta=p(x["delta"]), A=p(x["A"]),
                      B=p(x["B"]), C=p(x["C"]), D=p(x["D"]), z=p(x["z"]), delta_bias=p(x["delta_bias"]),
                      initial_state=p(x["initial_state"]), seq_lens=p(x["seq_lens"]), out=p(out),
                      last_state=p(last), carries=p(carries), y_pre=p(y_pre))
    _lib.check(lib.mss_fwd(fa, None), "mss_fwd")
    return carries, y_pre, out


GRADS = ("du", "ddelta", "dA", "dB", "dC", "dD", "dz", "ddelta_bias", "dinitial_state")


def _backward(lib, fn, x, carries, y_pre, out, dout, dlast, b, d, l, n, workspace=None):
    """Runs `fn` (mss_bwd or mss_bwd_noalloc) into NaN-filled outputs; returns them."""
    shapes = dict(du=(b, d, l), ddelta=(b, d, l), dA=(d, n), dB=(b, n, l), dC=(b, n, l), dD=(d,), dz=(b, d, l),
                  ddelta_bias=(d,), dinitial_state=(b, d, n))
    o = {k: torch.full(shapes[k], float("nan"), device=dev) for k in GRADS}
    p = lambda t: None if t is None else t.data_ptr()
    ba = _lib.BwdArgs(batch=b, dim=d, seqlen=l, dstate=n, discretization=_lib.MSS_EULER, delta_softplus=1,
                      io_dtype=_lib.MSS_F32, bc_dtype=_lib.MSS_F32, u=p(x["u"]), delta=p(x["delta"]), A=p(x["A"]),
                      B=p(x["B"]), C=p(x["C"]), D=p(x["D"]), z=p(x["z"]), delta_bias=p(x["delta_bias"]),
                      initial_state=p(x["initial_state"]), seq_lens=p(x["seq_lens"]), carries=p(carries),
                      y_pre=p(y_pre), out=p(out), dout=p(dout), dlast_state=p(dlast),
                      du=p(o["du"]), ddelta=p(o["ddelta"]), dA=p(o["dA"]), dB=p(o["dB"]), dC=p(o["dC"]),
                      dD=p(o["dD"]), dz=p(o["dz"]), ddelta_bias=p(o["ddelta_bias"]),
                      dinitial_state=p(o["dinitial_state"]))
    if workspace is not None:
        ba.workspace, ba.workspace_bytes = workspace.data_ptr(), workspace.numel()
    _lib.check(fn(ba, None), fn.__name__)
    torch.cuda.synchronize()
    return o


def test_noalloc_backward_matches_workspace_backward():
    lib = _lib.register_hip_kernel()
    # the second call is smaller: fewer rows, channels and steps, and ragged lengths; the third
    # has 32 states (a float32 backward over two groups of 16 in the same scratch)
    for seed, (b, d, l, n), lens in ((1, (4, 1536, 2048, 16), None), (2, (2, 40, 700, 8), [700, 333]),
                                     (3, (2, 48, 600, 32), [600, 257])):
        log(f"case noalloc b={b} d={d} l={l} n={n} lens={lens}")
        x, dout, dlast = _inputs(seed, b, d, l, n, lens)
        carries, y_pre, out = _forward(lib, x, b, d, l, n)
        probe = _lib.BwdArgs(batch=b, dim=d, seqlen=l, dstate=n, seq_lens=None if lens is None else 1)
        ws_bytes = int(lib.mss_bwd_workspace_bytes(probe))
        assert 0 < ws_bytes <= _lib.MSS_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        want = _backward(lib, lib.mss_bwd, x, carries, y_pre, out, dout, dlast, b, d, l, n, workspace=ws)
        got = _backward(lib, lib.mss_bwd_noalloc, x, carries, y_pre, out, dout, dlast, b, d, l, n)
        for k in GRADS:
            assert bool(torch.isfinite(want[k]).all()), k
            assert torch.equal(got[k], want[k]), k
        log("  equal bit for bit")
