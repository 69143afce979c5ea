"""C-ABI and host-API checks that need no GPU.

* the library loads and exports every function declared in include/*.h;
* every validation error is returned before any HIP call (reference error contract:
  native/selective_scan_cuda.cu:400-440, native/selective_scan_bwd.cu:45-79,
  mamba/selective_scan_cuda.py:35-40, 93-121);
* the Python API raises the reference's exception types, and refuses CPU tensors
  instead of falling back to a CPU path.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from mamba_amd import _lib
from mamba_amd.configs import C2, algorithmic_bytes, round_to_bf16
from mamba_amd.selective_scan_hip import selective_scan, selective_scan_fn

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    names = []
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mss_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


def test_header_declares_expected_symbols():
    assert set(header_functions()) == set(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_header_symbol(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
    header = (ROOT / "include" / "mamba_selective_scan.h").read_text()
    version = int(re.search(r"#define MSS_ABI_VERSION (\d+)", header).group(1))
    assert lib.mss_abi_version() == version == _lib.MSS_ABI_VERSION
    for name in ("MSS_MAX_DSTATE", "MSS_MAX_DSTATE_WIDE", "MSS_SEG_STEPS", "MSS_REF_CHUNK",
                 "MSS_NORM_GEMV_MAX_FEATURES", "MSS_XENT_FUSED_MAX_VOCAB"):
        value = int(re.search(rf"#define {name} (\d+)", header).group(1))
        assert getattr(_lib, name) == value, name


def test_missing_library_raises_file_not_found(tmp_path):
    saved = _lib._LIBRARY
    try:
        _lib._LIBRARY = None
        with pytest.raises(FileNotFoundError, match="not built"):
            _lib.register_hip_kernel(tmp_path / "nope.so")
    finally:
        _lib._LIBRARY = saved


def fwd_args(**kw):
    base = dict(batch=2, dim=3, seqlen=10, dstate=4, u=1, delta=1, A=1, B=1, C=1, out=1)
    base.update(kw)
    return _lib.FwdArgs(**base)


@pytest.mark.parametrize("kw,status", [
    (dict(batch=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dim=-1), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(seqlen=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dstate=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dstate=257), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dstate=17, io_dtype=_lib.MSS_BF16), _lib.MSS_ERR_UNSUPPORTED),   # wider states: float32 only
    (dict(dstate=17, bc_dtype=_lib.MSS_BF16), _lib.MSS_ERR_UNSUPPORTED),
    (dict(discretization=2), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(delta_softplus=3), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(io_dtype=7), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(bc_dtype=-1), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(u=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(out=None), _lib.MSS_ERR_INVALID_ARGUMENT),
])
def test_fwd_validation(lib, kw, status):
    assert lib.mss_fwd(fwd_args(**kw), None) == status


@pytest.mark.parametrize("strides,status", [
    (dict(io_dim=-10), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(io_dim=5), _lib.MSS_ERR_INVALID_ARGUMENT),                # rows of 10 steps overlap
    (dict(io_batch=10, io_dim=10), _lib.MSS_ERR_INVALID_ARGUMENT),  # (1,0) and (0,1) collide
    (dict(io_batch=10, io_dim=15), _lib.MSS_ERR_INVALID_ARGUMENT),  # [D][B][L] needs io_dim >= 20
    (dict(bc_state=3), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(bc_batch=10, bc_state=10), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(bc_batch=1 << 41), _lib.MSS_ERR_INVALID_ARGUMENT),
])
def test_fwd_stride_validation(lib, strides, status):
    assert lib.mss_fwd(fwd_args(strides=_lib.Strides(**strides)), None) == status
    assert lib.mss_bwd(bwd_args(strides=_lib.Strides(**strides)), None) == status


def test_grid_limit_is_unsupported(lib):
    assert lib.mss_fwd(fwd_args(batch=2048, dstate=16), None) == _lib.MSS_ERR_UNSUPPORTED


def test_struct_layout_matches_header(tmp_path):
    """The ctypes mirrors have the C structs' size and field offsets (compiled with gcc)."""
    structs = {"mss_fwd_args": _lib.FwdArgs, "mss_bwd_args": _lib.BwdArgs, "mss_strides": _lib.Strides,
               "mss_conv_args": _lib.ConvArgs, "mss_norm_args": _lib.NormArgs, "mss_xent_args": _lib.XentArgs,
               "mss_step_args": _lib.StepArgs, "mss_conv_step_args": _lib.ConvStepArgs}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "mamba_selective_scan.h"',
             "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    seen = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, value = line.split()
        seen[(cname, field)] = int(value)
    for cname, cls in structs.items():
        assert seen[(cname, "sizeof")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert seen[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_row_layout_helpers():
    from mamba_amd import selective_scan_hip as ss
    x = torch.empty(3, 5, 7)
    assert ss._layout_of(x) == "brl"
    xt = torch.empty(5, 3, 7).permute(1, 0, 2)
    assert ss._layout_of(xt) == "rbl"
    assert ss._row_strides(xt, "rbl") == (7, 21)
    # a row slice of a bigger (R, B*L) matrix: dense rbl strides, no copy
    big = torch.empty(12, 3 * 7)
    view = big[4:9].view(5, 3, 7).permute(1, 0, 2)
    assert ss._layout_of(view) == "rbl" and ss._conform(view, "rbl") is view
    # a strided view that is neither layout is copied into the requested one
    odd = torch.randn(3, 10, 7)[:, ::2]
    assert ss._layout_of(odd) is None
    c = ss._conform(odd, "rbl")
    assert ss._strides_match(c, "rbl") and torch.equal(c, odd)


def test_null_args(lib):
    assert lib.mss_fwd(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_bwd(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_bwd_workspace_bytes(None) == 0


def bwd_args(**kw):
    base = dict(batch=2, dim=3, seqlen=10, dstate=4, u=1, delta=1, A=1, B=1, C=1, carries=1, dout=1,
                du=1, ddelta=1, dA=1, dB=1, dC=1)
    base.update(kw)
    return _lib.BwdArgs(**base)


@pytest.mark.parametrize("kw", [
    dict(carries=None), dict(dout=None), dict(dB=None), dict(D=1), dict(z=1), dict(delta_bias=1),
    dict(seqlen=0), dict(discretization=5),
    dict(z=1, dz=1, y_pre=1),  # z without the forward's out (dz comes from out / z)
])
def test_bwd_validation(lib, kw):
    assert lib.mss_bwd(bwd_args(**kw), None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_bwd_workspace_too_small(lib):
    a = bwd_args(workspace=1, workspace_bytes=16)
    assert lib.mss_bwd(a, None) == _lib.MSS_ERR_WORKSPACE


def test_noalloc_backward_rejects_shapes_beyond_its_scratch(lib):
    """mss_bwd_noalloc validates like mss_bwd, then refuses shapes whose workspace exceeds its
    fixed scratch (config 3's 129 MiB) before any HIP call; config 2 and the config-5 layers fit."""
    assert lib.mss_bwd_noalloc(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_bwd_noalloc(bwd_args(carries=None), None) == _lib.MSS_ERR_INVALID_ARGUMENT
    big = bwd_args(batch=8, dim=2048, seqlen=4096, dstate=16)
    assert lib.mss_bwd_workspace_bytes(big) > _lib.MSS_NOALLOC_SCRATCH_BYTES
    assert lib.mss_bwd_noalloc(big, None) == _lib.MSS_ERR_SCRATCH_LIMIT
    assert b"mss_bwd_noalloc" in lib.mss_strerror(_lib.MSS_ERR_SCRATCH_LIMIT)
    for b, d, l in ((4, 1536, 2048), (8, 1536, 2048)):
        assert lib.mss_bwd_workspace_bytes(bwd_args(batch=b, dim=d, seqlen=l, dstate=16)) <= \
            _lib.MSS_NOALLOC_SCRATCH_BYTES


def test_workspace_size_depends_on_shapes_only(lib):
    a = bwd_args(batch=4, dim=1536, seqlen=2048, dstate=16)
    n1 = lib.mss_bwd_workspace_bytes(a)
    assert n1 == lib.mss_bwd_workspace_bytes(a) > 0
    # dB/dC partials: at most one per 8-channel octet, at least one per batch row
    assert n1 >= 4 * 2 * 16 * 2048 * 4


def _bwd_blocks(lib, batch, dim, seqlen, dstate):
    """Channel blocks of the backward plan, read back from the workspace size: dB/dC partials
    (blocks x [batch][2][N][L] floats, padded to 64) then dA, dD and dbias partials, each
    rounded up to 256 bytes."""
    a = bwd_args(batch=batch, dim=dim, seqlen=seqlen, dstate=dstate)
    up = lambda x: (x + 255) // 256 * 256
    stride = (batch * 2 * dstate * seqlen + 63) // 64 * 64
    rest = up(batch * dim * dstate * 4) + 2 * up(batch * dim * 4)
    total = lib.mss_bwd_workspace_bytes(a)
    assert (total - rest) % (stride * 4) == 0
    return (total - rest) // (stride * 4)


@pytest.mark.parametrize("shape,waves", [
    ((4, 1536, 2048, 16), 12),   # config 2: 24 channels per CU, 12 waves x 2 rounds
    ((8, 2048, 4096, 16), 16),   # config 3: 16 waves x 4 rounds beat 12 x 6 (232 workgroups)
    ((1, 4096, 600, 8), 16),     # one pass of 16-channel workgroups
    ((1, 4096, 600, 11), 12),    # 16 waves need N to divide 16
    ((2, 24, 64, 16), 12),       # small grids: 12 waves, one round
])
def test_backward_plan(lib, shape, waves):
    """The backward takes 12 or 16 waves per workgroup by a modelled time: workgroup passes
    over 256 CUs x channel rounds x the time of a round (1.2x for 16 waves); the channel
    count per workgroup is the fewest rounds whose grid fits one pass."""
    b, d, l, n = shape
    per_row = -(-d // waves)
    k = max(1, -(-b * per_row // 256))
    while k < per_row and b * (-(-per_row // k)) > 256:
        k += 1
    cpb = min(k, 96 // waves, per_row) * waves
    assert _bwd_blocks(lib, b, d, l, n) == -(-d // cpb)
    assert _lib.bwd_plan(b, d, n, seqlen=l) == (waves, cpb)


def test_backward_plan_of_the_configs(lib):
    """Config 3 and every config-5 layer run the 16-wave backward, config 2 the 12-wave one;
    invalid arguments are rejected."""
    assert _lib.bwd_plan(4, 1536, 16, 2048)[0] == 12
    assert _lib.bwd_plan(8, 2048, 16, 4096, io_bf16=True)[0] == 16
    c5 = _lib.Strides(io_batch=2048, io_dim=8 * 2048, bc_batch=2048, bc_state=8 * 2048)
    assert _lib.bwd_plan(8, 1536, 16, 2048, io_bf16=True, strides=c5)[0] == 16
    w = ctypes.c_int32()
    assert lib.mss_bwd_plan(None, ctypes.byref(w), ctypes.byref(w)) == _lib.MSS_ERR_INVALID_ARGUMENT
    bad = bwd_args(dstate=32, io_dtype=_lib.MSS_BF16)
    assert lib.mss_bwd_plan(bad, ctypes.byref(w), ctypes.byref(w)) == _lib.MSS_ERR_UNSUPPORTED
    assert lib.mss_bwd_plan(bwd_args(dstate=257), ctypes.byref(w), ctypes.byref(w)) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_bwd_plan(bwd_args(), None, ctypes.byref(w)) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_wide_state_backward_groups(lib):
    """Float32 scans with more than 16 states: the backward runs over balanced groups of at
    most 16 states in one workspace, sized for the larger group; the split phases, which
    cannot carry the groups' sums from one call to the next, refuse them before any HIP call."""
    for n, groups in ((17, (9, 8)), (32, (16, 16)), (40, (14, 13)), (256, (16,))):
        got = lib.mss_bwd_workspace_bytes(bwd_args(batch=4, dim=1536, seqlen=2048, dstate=n))
        want = max(lib.mss_bwd_workspace_bytes(bwd_args(batch=4, dim=1536, seqlen=2048, dstate=g)) for g in groups)
        assert got == want > 0, n
        waves, cpb = ctypes.c_int32(), ctypes.c_int32()
        assert lib.mss_bwd_plan(bwd_args(dstate=n), ctypes.byref(waves), ctypes.byref(cpb)) == _lib.MSS_OK
        assert waves.value in (12, 16) and cpb.value % waves.value == 0
        assert lib.mss_bwd_scan(bwd_args(dstate=n), None) == _lib.MSS_ERR_UNSUPPORTED
        assert lib.mss_bwd_reduce(bwd_args(dstate=n), None) == _lib.MSS_ERR_UNSUPPORTED
    assert lib.mss_bwd_workspace_bytes(bwd_args(dstate=17, io_dtype=_lib.MSS_BF16)) == 0
    assert lib.mss_bwd_workspace_bytes(bwd_args(dstate=257)) == 0


def test_reference_entry_points_validate(lib):
    p = ctypes.c_void_p(1)
    assert lib.mss_scan_fwd(None, 0, 0, 10, 3, 4, *[p] * 9) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_fwd(None, 2, 1, 10, 3, 4, *[p] * 9) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_fwd(None, 0, 1, 10, 3, 4, *[p] * 8, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_fwd_repeat(None, 0, 0, 1, 10, 3, 4, *[p] * 9) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_bwd(None, 1, 10, 3, 257, *[p] * 15) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_bwd(None, 1, 10, 3, 4, *[p] * 14, None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_reference_backward_workspace(lib):
    """mss_scan_bwd_ws: its workspace holds the 8-step state carries and mss_bwd's workspace;
    it validates before any HIP call and never allocates."""
    b, l, d, n = 4, 2048, 1536, 16
    carries = b * d * n * (l // 8) * 4
    fused = lib.mss_bwd_workspace_bytes(bwd_args(batch=b, dim=d, seqlen=l, dstate=n))
    assert lib.mss_scan_bwd_workspace_bytes(b, l, d, n) == carries + fused
    assert lib.mss_scan_bwd_workspace_bytes(b, l, d, 257) == 0
    wide = b * d * 40 * (l // 8) * 4 + lib.mss_bwd_workspace_bytes(bwd_args(batch=b, dim=d, seqlen=l, dstate=40))
    assert lib.mss_scan_bwd_workspace_bytes(b, l, d, 40) == wide
    p = ctypes.c_void_p(256)
    args = [None, 1, 64, 3, 4] + [p] * 15
    assert lib.mss_scan_bwd_ws(*args, None, 1 << 30) == _lib.MSS_ERR_WORKSPACE
    assert lib.mss_scan_bwd_ws(*args, p, 16) == _lib.MSS_ERR_WORKSPACE
    assert lib.mss_scan_bwd_ws(*args, ctypes.c_void_p(8), 1 << 30) == _lib.MSS_ERR_WORKSPACE
    assert lib.mss_scan_bwd_ws(None, 1, 64, 3, 257, *[p] * 15, p, 1 << 30) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_scan_bwd_ws(None, 1, 64, 3, 4, *[p] * 14, None, p, 1 << 30) == _lib.MSS_ERR_INVALID_ARGUMENT
    # more 2048-step blocks than the carry rebuild's grid holds
    assert lib.mss_scan_bwd_ws(None, 1, 65535 * 2048 + 1, 3, 4, *[p] * 15, p, 1 << 62) == _lib.MSS_ERR_UNSUPPORTED
    assert lib.mss_scan_bwd(None, 1, 65535 * 2048 + 1, 3, 4, *[p] * 15) == _lib.MSS_ERR_UNSUPPORTED


def test_strerror(lib):
    assert lib.mss_strerror(0) == b"ok"
    assert b"invalid" in lib.mss_strerror(1)
    assert lib.mss_strerror(99) == b"unknown status"


# ------------------------------------------------------------------ Python API errors
def ref_inputs(dtype=torch.float32, b=2, l=17, d=8, n=16):
    g = torch.Generator().manual_seed(7)
    A = -torch.exp(torch.randn(d, n, generator=g))
    return (A.to(dtype), torch.randn(b, l, d, generator=g).to(dtype), torch.randn(b, l, n, generator=g).to(dtype),
            torch.randn(b, l, n, generator=g).to(dtype), torch.randn(b, l, d, generator=g).to(dtype),
            torch.randn(b, d, n, generator=g).to(dtype))


def test_reference_api_rejects_non_float32():
    with pytest.raises(TypeError, match="float32"):
        selective_scan(*ref_inputs(torch.float64))


@pytest.mark.parametrize("n", [3, 32])
def test_reference_api_rejects_state_size(n):
    args = ref_inputs(n=n)
    with pytest.raises(ValueError, match="N must be one of"):
        selective_scan(*args)


def test_reference_api_rejects_zero_length_and_shapes():
    A, d, B, C, u, x0 = ref_inputs()
    with pytest.raises(ValueError, match="positive"):
        selective_scan(A, d[:, :0], B[:, :0], C[:, :0], u[:, :0], x0)
    with pytest.raises(ValueError, match="Bs must have shape"):
        selective_scan(A, d, B[:, :5], C, u, x0)
    with pytest.raises(ValueError, match="initial_x must have shape"):
        selective_scan(A, d, B, C, u, x0[:1])


def test_no_cpu_fallback():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        selective_scan(*ref_inputs())
    u = torch.randn(1, 2, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        selective_scan_fn(u, u, -torch.ones(2, 4), torch.randn(1, 4, 8), torch.randn(1, 4, 8))


def test_fused_api_validation():
    u = torch.randn(1, 2, 8)
    A = -torch.ones(2, 4)
    Bm = torch.randn(1, 4, 8)
    with pytest.raises(TypeError):
        selective_scan_fn(u, u.double(), A, Bm, Bm)
    with pytest.raises(ValueError, match="N must be between 1 and 256"):
        selective_scan_fn(u, u, -torch.ones(2, 257), torch.randn(1, 257, 8), torch.randn(1, 257, 8))
    ub = u.bfloat16()
    with pytest.raises(ValueError, match="N must be between 1 and 16"):
        selective_scan_fn(ub, ub, -torch.ones(2, 17), torch.randn(1, 17, 8).bfloat16(),
                          torch.randn(1, 17, 8).bfloat16())
    with pytest.raises(ValueError, match="N must be between 1 and 16"):
        selective_scan_fn(u, u, -torch.ones(2, 17, dtype=torch.complex64), torch.randn(1, 17, 8),
                          torch.randn(1, 17, 8))
    with pytest.raises(ValueError, match="discretization"):
        selective_scan_fn(u, u, A, Bm, Bm, discretization="rk4")
    with pytest.raises(TypeError, match="float32"):
        selective_scan_fn(u, u, A.double(), Bm, Bm)
    with pytest.raises(ValueError, match="seq_lens"):
        selective_scan_fn(u, u, A, Bm, Bm, seq_lens=torch.tensor([3]))


def test_algorithmic_bytes_match_baseline_table():
    fwd, bwd = algorithmic_bytes(C2)
    assert abs(fwd / 1e6 - 202.9) < 0.1 and abs(bwd / 1e6 - 355.0) < 0.1


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32)
    ours = round_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)


# Complex-A entry points: the same argument blocks; A, the state buffers and the carries
# must be 8-byte aligned (interleaved complex64). Only rejected calls run here (no GPU).
def _aligned(kw, fields):
    return {f: 64 for f in fields} | kw


@pytest.mark.parametrize("kw,status", [
    (dict(batch=0), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(dstate=17), _lib.MSS_ERR_UNSUPPORTED),
    (dict(u=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(discretization=3), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(A=4), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(carries=68), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(last_state=20), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(initial_state=36), _lib.MSS_ERR_INVALID_ARGUMENT),
])
def test_complex_fwd_validation(lib, kw, status):
    args = fwd_args(**_aligned(kw, ("u", "delta", "A", "B", "C", "out")))
    assert lib.mss_cfwd(args, None) == status


@pytest.mark.parametrize("kw,status", [
    (dict(carries=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(carries=12), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(A=4), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(D=64), _lib.MSS_ERR_INVALID_ARGUMENT),     # D without dD
    (dict(z=64), _lib.MSS_ERR_INVALID_ARGUMENT),     # z without dz / y_pre
    (dict(dstate=17), _lib.MSS_ERR_UNSUPPORTED),
])
def test_complex_bwd_validation(lib, kw, status):
    fields = ("u", "delta", "A", "B", "C", "carries", "dout", "du", "ddelta", "dA", "dB", "dC")
    assert lib.mss_cbwd(bwd_args(**_aligned(kw, fields)), None) == status
    assert lib.mss_cfwd(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_cbwd(None, None) == _lib.MSS_ERR_INVALID_ARGUMENT


def test_complex_workspace_bytes(lib):
    assert lib.mss_cbwd_workspace_bytes(None) == 0
    assert lib.mss_cbwd_workspace_bytes(bwd_args(dstate=17)) == 0
    real = lib.mss_bwd_workspace_bytes(bwd_args(batch=4, dim=1100, seqlen=64, dstate=4))
    cplx = lib.mss_cbwd_workspace_bytes(bwd_args(batch=4, dim=1100, seqlen=64, dstate=4))
    # dB/dC partial rows of every channel block (complex blocks hold 2 rounds of 12 channels
    # here: 4 * ceil(1100 / 12) > 256 workgroups for one round) plus complex dA partials
    # [B][D][N][2] and dD / dbias partials [B][D], each 256-byte padded.
    up = lambda x: (x + 255) // 256 * 256
    blocks = (1100 + 23) // 24
    part = (4 * 2 * 4 * 64 + 63) // 64 * 64
    want = up(blocks * part * 4) + up(4 * 1100 * 4 * 2 * 4) + 2 * up(4 * 1100 * 4)
    assert cplx == want
    assert real > 0


# torch.library registration of the scan: fake implementations (no GPU needed) give the
# real ones' shapes, dtypes and row layouts; absent optional results are empty tensors.
def _fake_scan(cplx, layout, with_extras):
    from torch._subclasses.fake_tensor import FakeTensorMode
    b, d, l, n = 2, 3, 40, 4
    with FakeTensorMode():
        if layout == "rbl":
            u = torch.empty(d, b, l, device="cuda").permute(1, 0, 2)
            B = torch.empty(n, b, l, device="cuda").permute(1, 0, 2)
        else:
            u = torch.empty(b, d, l, device="cuda")
            B = torch.empty(b, n, l, device="cuda")
        A = torch.empty(d, n, device="cuda", dtype=torch.complex64 if cplx else torch.float32)
        D = torch.empty(d, device="cuda") if with_extras else None
        z = u if with_extras else None
        x0 = torch.empty(b, d, n, device="cuda", dtype=A.dtype) if with_extras else None
        fw = torch.ops.mamba_amd.selective_scan_fwd(u, u, A, B, B, D, z, D, x0, None, True, False)
        bw = torch.ops.mamba_amd.selective_scan_bwd(u, u, A, B, B, D, z, D, x0, None, fw[2], fw[3],
                                                    fw[0] if z is not None else None, fw[0], fw[1], True, False)
        return u, B, A, fw, bw


@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("layout", ["brl", "rbl"])
@pytest.mark.parametrize("with_extras", [False, True])
def test_custom_op_fake_shapes(cplx, layout, with_extras):
    u, B, A, (out, last, carries, y_pre), bw = _fake_scan(cplx, layout, with_extras)
    sdt = torch.complex64 if cplx else torch.float32
    assert out.shape == u.shape and out.stride() == u.stride() and out.dtype == u.dtype
    assert last.shape == (2, 3, 4) and last.dtype == sdt
    assert carries.shape == (2, 3, 4, 5) and carries.dtype == sdt
    assert (y_pre.numel() > 0) == with_extras
    du, ddelta, dA, dB, dC, dD, dz, dbias, dinit = bw
    assert du.stride() == u.stride() and ddelta.stride() == u.stride()
    assert dA.shape == A.shape and dA.dtype == A.dtype
    assert dB.shape == B.shape and dB.stride() == B.stride() and dC.stride() == B.stride()
    for t in (dD, dz, dbias, dinit):
        assert (t.numel() > 0) == with_extras
    if with_extras:
        assert dz.stride() == u.stride() and dinit.dtype == sdt
