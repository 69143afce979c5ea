"""ctypes front-end of the float64 C oracle (``oracle/scan64c.c``) — TEST INFRASTRUCTURE ONLY.

Same call signatures and results as ``oracle.scan64.forward`` / ``backward`` (which it is
checked against in tests/test_oracle.py), for the full-size configurations where the numpy
loop would take minutes. ``backward(..., abs_terms=True)`` also returns, for each reduction
gradient (dA, dB, dC, dD, ddelta_bias), the sum of the absolute values of the terms summed
into it (keys ``dA_abs`` ...): the scale of the rounding error of any summation order.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = None
_PATH = Path(__file__).resolve().parent / "_build" / "libscan64c.so"
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)


def _lib():
    global _LIB
    if _LIB is None:
        if not _PATH.exists():
            from . import build_oracle
            build_oracle.build()
        lib = ctypes.CDLL(str(_PATH))
        lib.scan64c_fwd.restype = ctypes.c_int
        lib.scan64c_bwd.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def _d(a):
    return None if a is None else np.ascontiguousarray(a, np.float64)


def _p(a):
    if a is None:
        return None
    if a.dtype == np.int32:
        return a.ctypes.data_as(_ip)
    return a.ctypes.data_as(_dp)


def _inputs(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens):
    u, delta, A, B, C = (_d(a) for a in (u, delta, A, B, C))
    bsz, dim, L = u.shape
    n = A.shape[1]
    assert delta.shape == (bsz, dim, L) and A.shape == (dim, n)
    assert B.shape == (bsz, n, L) and C.shape == (bsz, n, L)
    lens = None if seq_lens is None else np.ascontiguousarray(seq_lens, np.int32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=_d(D), z=_d(z), bias=_d(delta_bias),
                x0=_d(initial_state), lens=lens), (bsz, dim, L, n)


def forward(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
            initial_state=None, seq_lens=None, discretization="euler"):
    x, (bsz, dim, L, n) = _inputs(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens)
    out = np.empty((bsz, dim, L))
    y = np.empty((bsz, dim, L))
    last = np.empty((bsz, dim, n))
    ref = np.empty((bsz, dim, (L + 2047) // 2048, n, 2))
    s = _lib().scan64c_fwd(bsz, dim, L, n, int(discretization == "zoh"), int(bool(delta_softplus)),
                           _p(x["u"]), _p(x["delta"]), _p(x["A"]), _p(x["B"]), _p(x["C"]), _p(x["D"]),
                           _p(x["z"]), _p(x["bias"]), _p(x["x0"]), _p(x["lens"]), _p(out), _p(y), _p(last),
                           _p(ref))
    if s != 0:
        raise RuntimeError(f"scan64c_fwd failed ({s})")
    return dict(out=out, y=y, last_state=last, ref_chunk_states=ref)


def backward(u, delta, A, B, C, dout, D=None, z=None, delta_bias=None, delta_softplus=False,
             initial_state=None, seq_lens=None, discretization="euler", dlast_state=None,
             abs_terms=False):
    x, (bsz, dim, L, n) = _inputs(u, delta, A, B, C, D, z, delta_bias, initial_state, seq_lens)
    dout = _d(dout)
    dlast = _d(dlast_state)
    g = dict(du=np.empty((bsz, dim, L)), ddelta=np.empty((bsz, dim, L)), dA=np.empty((dim, n)),
             dB=np.empty((bsz, n, L)), dC=np.empty((bsz, n, L)),
             dD=None if D is None else np.empty(dim), dz=None if z is None else np.empty((bsz, dim, L)),
             ddelta_bias=None if delta_bias is None else np.empty(dim),
             dinitial_state=np.empty((bsz, dim, n)))
    ab = {}
    if abs_terms:
        ab = dict(dA_abs=np.empty((dim, n)), dB_abs=np.empty((bsz, n, L)), dC_abs=np.empty((bsz, n, L)),
                  dD_abs=np.empty(dim), ddelta_bias_abs=np.empty(dim))
    s = _lib().scan64c_bwd(bsz, dim, L, n, int(discretization == "zoh"), int(bool(delta_softplus)),
                           _p(x["u"]), _p(x["delta"]), _p(x["A"]), _p(x["B"]), _p(x["C"]), _p(x["D"]),
                           _p(x["z"]), _p(x["bias"]), _p(x["x0"]), _p(x["lens"]), _p(dout), _p(dlast),
                           _p(g["du"]), _p(g["ddelta"]), _p(g["dA"]), _p(g["dB"]), _p(g["dC"]), _p(g["dD"]),
                           _p(g["dz"]), _p(g["ddelta_bias"]), _p(g["dinitial_state"]),
                           _p(ab.get("dA_abs")), _p(ab.get("dB_abs")), _p(ab.get("dC_abs")),
                           _p(ab.get("dD_abs")), _p(ab.get("ddelta_bias_abs")))
    if s != 0:
        raise RuntimeError(f"scan64c_bwd failed ({s})")
    if abs_terms:
        if D is None:
            ab["dD_abs"] = None
        if delta_bias is None:
            ab["ddelta_bias_abs"] = None
    g.update(ab)
    return g
