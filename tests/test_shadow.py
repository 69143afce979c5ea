"""bf16 shadows of float32 master weights (mss_shadow_refresh): the copies the training step's
GEMMs read, refreshed once per step, plus contiguous transposed copies of stacked groups for
the input-gradient GEMMs W^T dY. No reference counterpart (its parameters are used in their
own dtype); the bar is torch's own cast: every shadow equals master.to(bfloat16) bit for bit
(both round to nearest even), every transposed shadow cat(group).t().to(bfloat16).

CPU: the C entry point's argument checks, and the torch path of ShadowWeights (CPU tensors).
GPU: the one-launch refresh over shapes with partial 64 x 64 edge tiles, 1-D parameters,
stacked groups, rounding ties, after in-place updates of the masters, and after a master is
replaced (the device table is rebuilt).
"""
import pytest
import torch

from mamba_amd import _lib
from mamba_amd.mamba1 import ShadowWeights


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


def test_shadow_refresh_validation(lib):
    assert lib.mss_shadow_refresh(None, 1, 1, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_shadow_refresh(1 << 32, 0, 1, None) == _lib.MSS_ERR_INVALID_ARGUMENT
    assert lib.mss_shadow_refresh(1 << 32, 1, 0, None) == _lib.MSS_ERR_INVALID_ARGUMENT


def _bits(t):
    return t.contiguous().view(torch.int16)


def _params(dev):
    g = torch.Generator(device="cpu").manual_seed(3)
    shapes = [(1536, 768), (1536, 768), (768, 1536), (80, 1536), (1536, 48), (100, 37), (37,), (64, 64), (63, 129),
              (1, 5), (130, 65)]
    ps = [torch.randn(s, generator=g).to(dev) for s in shapes]
    # exact ties between two bf16 neighbours (round to even), and values that carry into the exponent
    ps[5].view(-1)[:4] = torch.tensor([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 2.0 - 2.0 ** -9])
    return ps


def _check(sw, ps, groups):
    for p, b in zip(ps, sw.bufs):
        assert b.shape == p.shape
        assert torch.equal(_bits(b), _bits(p.to(torch.bfloat16)))
    for grp in groups:
        t = sw.stacked_t(*grp)
        assert t.is_contiguous()
        assert torch.equal(_bits(t), _bits(torch.cat(grp).t().to(torch.bfloat16)))


def test_torch_path_on_cpu():
    ps = _params("cpu")
    groups = [(ps[0], ps[1]), (ps[2],), (ps[9],)]
    sw = ShadowWeights(ps, transposed=groups)
    sw.refresh(torch.bfloat16)
    _check(sw, ps, groups)
    assert sw.stacked_t(ps[3]) is None


@pytest.mark.gpu
def test_native_refresh_matches_casts():
    print("case shadow refresh", flush=True)
    ps = _params("cuda")
    groups = [(ps[0], ps[1]), (ps[2],), (ps[8],), (ps[10],)]
    sw = ShadowWeights(ps, transposed=groups)
    sw.refresh(torch.bfloat16)
    torch.cuda.synchronize()
    assert sw._table is not None  # the HIP launch ran, not the torch copies
    _check(sw, ps, groups)
    with torch.no_grad():  # in-place optimizer-style update: same table, new values
        for p in ps:
            p.mul_(-1.5).add_(0.25)
    sw.refresh(torch.bfloat16)
    torch.cuda.synchronize()
    _check(sw, ps, groups)
    table = sw._table[0]
    ps[3].data = torch.randn(80, 1536, device="cuda")  # a master replaced: the table follows
    sw.refresh(torch.bfloat16)
    torch.cuda.synchronize()
    assert sw._table[0] is not table
    _check(sw, ps, groups)
