"""Projection GEMMs of the training step: mss_proj (the S6 input projections,
mamba/mamba1.py:52-67, 107-124, and their input gradients) and mss_wgrad (the weight
gradients dW = dY X^T of the block's dense projections, float32, tokens split over
workgroups) on the matrix cores.

CPU: argument validation (rejected calls only, before any launch) and the shape gates.
GPU: against float32 products computed on the CPU from the same bf16 values —
  * small-integer operands, whose float32 sums are exact in any order: mss_proj equals the
    bf16 rounding of the exact product (and of old C + product when accumulating) bit for
    bit;
  * random operands: per element |got - ref| <= 2^-8 |ref| + 1e-6 sum|terms| (one bf16
    rounding plus float32 summation-order differences);
  * the weight passed transposed gives the same bits; strided row views (a row slice of a
    wider matrix as X or C); repeated calls bit for bit; the config-5 mixer's four products
    take these kernels.
mss_wgrad, against float32 / float64 products on the CPU: small-integer operands give the
exact product (and old C + product when accumulating) bit for bit, at the config-5 shapes,
with uneven token splits, with the workgroup count not a multiple of the XCD count, and with
one split (no partial planes), with partial edge tiles, on 96 x 96 tiles (a side below 192:
the S6 projections' 80- and 48-wide gradients); random operands within 2^-13 sum|terms| of the float64 product; repeated calls
bit for bit (fixed-order sums); strided views.
"""
import pytest
import torch

from mamba_amd import _lib
from mamba_amd.proj import proj, proj_fits, wgrad, wgrad_fits


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


def _proj_base(**kw):
    # Distinct, 16-byte aligned fake addresses far apart: only rejected calls are made here.
    base = dict(M=80, K=1536, T=4096, accumulate=0, ldw=1536, ldx=4096, ldc=4096,
                W=1 << 32, X=1 << 36, C=1 << 40)
    base.update(kw)
    return _lib.ProjArgs(**base)


@pytest.mark.parametrize("kw,status", [
    (dict(M=0), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(W=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(C=None), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(ldw=1000), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(ldx=4100), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(X=(1 << 36) + 8), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(M=88), _lib.MSS_ERR_UNSUPPORTED), (dict(T=4000, ldx=4000, ldc=4000), _lib.MSS_ERR_UNSUPPORTED),
    (dict(M=144), _lib.MSS_ERR_UNSUPPORTED), (dict(K=1544, ldw=1544), _lib.MSS_ERR_UNSUPPORTED),
    (dict(K=136, ldw=136), _lib.MSS_ERR_UNSUPPORTED),
    (dict(C=(1 << 36) + 4096 * 2 * 8), _lib.MSS_ERR_INVALID_ARGUMENT),  # C inside X
    (dict(w_trans=1, ldw=72), _lib.MSS_ERR_INVALID_ARGUMENT),  # W^T rows hold M = 80 values
])
def test_proj_validation(lib, kw, status):
    assert lib.mss_proj(_proj_base(**kw), None) == status


def test_fits_gates_cpu_tensors():
    w = torch.zeros(80, 1536, dtype=torch.bfloat16)
    x = torch.zeros(1536, 4096, dtype=torch.bfloat16)
    assert not proj_fits(w, x)  # not on a GPU


def _wgrad_base(lib, **kw):
    M, N, K = kw.get("M", 3072), kw.get("N", 768), kw.get("K", 16384)
    base = dict(M=M, N=N, K=K, accumulate=0, lda=16384, ldb=16384, ldc=768, A=1 << 32, B=1 << 36, C=1 << 40,
                workspace=1 << 41, workspace_bytes=int(lib.mss_wgrad_workspace_bytes(M, N, K)))
    base.update(kw)
    return _lib.WgradArgs(**base)


@pytest.mark.parametrize("kw,status", [
    (dict(M=0), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(A=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(C=None), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(lda=1000), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(ldc=700), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(ldc=770), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(ldb=16388), _lib.MSS_ERR_INVALID_ARGUMENT), (dict(B=(1 << 36) + 8), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(N=702), _lib.MSS_ERR_UNSUPPORTED),
    (dict(K=16100), _lib.MSS_ERR_UNSUPPORTED),
    (dict(workspace=None), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(workspace_bytes=1 << 20), _lib.MSS_ERR_INVALID_ARGUMENT),
    (dict(C=(1 << 32) + 4096), _lib.MSS_ERR_INVALID_ARGUMENT),  # C inside A
    (dict(C=(1 << 41) + 4096), _lib.MSS_ERR_INVALID_ARGUMENT),  # C inside the workspace
])
def test_wgrad_validation(lib, kw, status):
    assert lib.mss_wgrad(_wgrad_base(lib, **kw), None) == status


def test_wgrad_workspace_bytes(lib):
    """splits x M x N float32 partial planes, the split count filling the 256 CUs once with
    at least 4 k-stages per split (192 x 192 tiles with 64-deep stages; 96 x 96 when a side is
    below 192, with 128-deep stages when K allows); 0 for one split and for unsupported shapes."""
    assert lib.mss_wgrad_workspace_bytes(3072, 768, 16384) == 4 * 3072 * 768 * 4      # 64 tiles x 4
    assert lib.mss_wgrad_workspace_bytes(768, 1536, 16384) == 8 * 768 * 1536 * 4      # 32 tiles x 8
    assert lib.mss_wgrad_workspace_bytes(960, 1152, 4160) == 9 * 960 * 1152 * 4       # 30 tiles x 9
    assert lib.mss_wgrad_workspace_bytes(576, 384, 8192) == 32 * 576 * 384 * 4        # 6 tiles, 128 stages
    assert lib.mss_wgrad_workspace_bytes(192, 1920, 320) == 0                          # 5 stages: 1 split
    # a side below 192: 96 x 96 tiles
    assert lib.mss_wgrad_workspace_bytes(80, 1536, 16384) == 16 * 80 * 1536 * 4       # 1 x 16 partial tiles
    assert lib.mss_wgrad_workspace_bytes(1536, 48, 16384) == 16 * 1536 * 48 * 4      # 16 x 1
    assert lib.mss_wgrad_workspace_bytes(150, 1000, 4096) == 8 * 150 * 1000 * 4       # 2 x 11, 32 stages of 128
    assert lib.mss_wgrad_workspace_bytes(100, 196, 576) == 2 * 100 * 196 * 4          # 9 stages of 64
    assert lib.mss_wgrad_workspace_bytes(3000, 768, 16384) == 4 * 3000 * 768 * 4      # 16 x 4 tiles
    assert lib.mss_wgrad_workspace_bytes(192, 702, 16384) == 0                         # N % 4
    assert lib.mss_wgrad_workspace_bytes(192, 192, 100) == 0


def test_wgrad_fits_gates_cpu_tensors():
    assert not wgrad_fits(torch.zeros(3072, 1024, dtype=torch.bfloat16), torch.zeros(768, 1024, dtype=torch.bfloat16))


# ------------------------------------------------------------------------------ GPU
def _ints(shape, gen, lo=-4, hi=4):
    return torch.randint(lo, hi + 1, shape, generator=gen).to(torch.bfloat16)


def _randn(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)


def _check_bf16(got, W, X, old=None):
    ref = W.float() @ X.float()
    terms = W.float().abs() @ X.float().abs()
    if old is not None:
        ref = ref + old.float()
        terms = terms + old.float().abs()
    bound = 2.0 ** -8 * ref.abs() + 1e-6 * terms
    err = (got.float().cpu() - ref).abs()
    assert bool((err <= bound).all()), f"max err/bound {float((err / bound.clamp_min(1e-30)).max()):.3g}"


PROJ_SHAPES = [  # (M, K, T): reduce kernel (K % 64, M <= 128) and expand kernel (K <= 128)
    (80, 1536, 4096), (48, 1536, 2048), (16, 64, 64), (128, 192, 128), (112, 256, 320),
    (1536, 48, 2048), (1536, 80, 4096), (1552, 16, 128), (16, 128, 64), (32, 112, 192),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,T", PROJ_SHAPES)
def test_proj_exact_small_integers(M, K, T):
    gen = torch.Generator().manual_seed(M * 7 + K * 3 + T)
    W, X = _ints((M, K), gen), _ints((K, T), gen)
    want = (W.float() @ X.float()).to(torch.bfloat16)
    got = proj(W.cuda(), X.cuda())
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    old = _ints((M, T), gen, -1000, 1000)
    want = (old.float() + W.float() @ X.float()).to(torch.bfloat16)
    out = old.cuda()
    proj(W.cuda(), X.cuda(), out=out, accumulate=True)
    assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,T", PROJ_SHAPES)
def test_proj_random(M, K, T):
    gen = torch.Generator().manual_seed(1000 + M + K + T)
    W, X = _randn((M, K), gen, K ** -0.5), _randn((K, T), gen)
    got = proj(W.cuda(), X.cuda())
    _check_bf16(got, W, X)
    again = proj(W.cuda(), X.cuda())
    assert torch.equal(got.view(torch.int16), again.view(torch.int16))
    old = _randn((M, T), gen)
    out = old.cuda()
    proj(W.cuda(), X.cuda(), out=out, accumulate=True)
    _check_bf16(out, W, X, old)
    # the weight passed as the transposed view of its (K, M) transpose: same sums, same bits
    Wt = W.t().contiguous().cuda()
    assert torch.equal(proj(Wt.t(), X.cuda()).view(torch.int16), got.view(torch.int16))
    out_t = old.cuda()
    proj(Wt.t(), X.cuda(), out=out_t, accumulate=True)
    assert torch.equal(out_t.view(torch.int16), out.view(torch.int16))


@pytest.mark.gpu
def test_proj_row_views():
    """X and C as row slices of wider matrices (the model's x_dbl[:R] / dx_dbl[:R])."""
    gen = torch.Generator().manual_seed(5)
    T = 2048
    big = _randn((80, T), gen).cuda()
    W = _randn((1536, 48), gen, 48 ** -0.5)
    got = proj(W.cuda(), big[:48])
    _check_bf16(got, W, big[:48].cpu())
    W2 = _randn((48, 1536), gen, 1536 ** -0.5)
    X2 = _randn((1536, T), gen)
    sink = torch.full((80, T), 7.0, dtype=torch.bfloat16, device="cuda")
    proj(W2.cuda(), X2.cuda(), out=sink[:48])
    _check_bf16(sink[:48], W2, X2)
    assert bool((sink[48:] == 7.0).all())  # rows past the view untouched


@pytest.mark.gpu
def test_model_projection_shapes_take_the_kernels():
    """The config-5 mixer's four projection products fit the kernels (so the model runs
    them, not the library GEMM)."""
    dev = "cuda"
    T, di, r, n = 16384, 1536, 48, 16
    u = torch.empty(di, T, dtype=torch.bfloat16, device=dev)
    x_dbl = torch.empty(r + 2 * n, T, dtype=torch.bfloat16, device=dev)
    w_x = torch.empty(r + 2 * n, di, dtype=torch.bfloat16, device=dev)
    w_dt = torch.empty(di, r, dtype=torch.bfloat16, device=dev)
    assert proj_fits(w_x, u) and proj_fits(w_dt, x_dbl[:r])
    assert proj_fits(w_dt.t(), u, x_dbl[:r]) and proj_fits(w_x.t(), x_dbl, u)


WGRAD_SHAPES = [  # (M, N, K): config-5 in_proj / out_proj / x_proj / dt_proj gradients;
    # uneven splits and a workgroup count that is not a multiple of 8 (960 x 1152: 30 tiles x
    # 9 splits over 65 stages); one split (direct store); tall and wide tile grids; partial
    # edge tiles on either side or both
    (3072, 768, 16384), (768, 1536, 16384), (80, 1536, 16384), (1536, 48, 16384), (960, 1152, 4160),
    (192, 192, 64), (192, 1920, 320), (576, 384, 8192), (1536, 192, 640), (100, 196, 640), (1, 4, 64),
    (200, 388, 1024), (150, 1000, 4096), (100, 196, 576),
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", WGRAD_SHAPES)
def test_wgrad_exact_small_integers(M, N, K):
    gen = torch.Generator().manual_seed(M * 5 + N * 3 + K)
    A, B = _ints((M, K), gen), _ints((N, K), gen)
    want = A.float() @ B.float().t()  # exact: |sums| < 2^24
    got = wgrad(A.cuda(), B.cuda())
    assert torch.equal(got.cpu(), want)
    old = _ints((M, N), gen, -1000, 1000).float()
    out = old.cuda()
    wgrad(A.cuda(), B.cuda(), out=out, accumulate=True)
    assert torch.equal(out.cpu(), old + want)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(768, 1536, 16384), (960, 1152, 4160), (192, 1920, 320), (80, 1536, 16384),
                                   (200, 388, 1024), (1536, 48, 16384), (150, 1000, 4096)])
def test_wgrad_random(M, N, K):
    gen = torch.Generator().manual_seed(2000 + M + N + K)
    A, B = _randn((M, K), gen), _randn((N, K), gen)
    ref = A.double() @ B.double().t()
    terms = A.double().abs() @ B.double().abs().t()
    got = wgrad(A.cuda(), B.cuda())
    err = (got.cpu().double() - ref).abs()
    assert bool((err <= 2.0 ** -13 * terms).all()), float((err / terms).max())
    again = wgrad(A.cuda(), B.cuda())
    assert torch.equal(got, again)  # the partial tiles are added in a fixed order


@pytest.mark.gpu
def test_wgrad_views_and_fits():
    """dY as a row slice of a wider matrix (the model's dxz rows), C as a column block of a
    wider float32 matrix (ldc > N): the columns outside it untouched; the config-5 in- and
    out-projection gradients take the kernel, the S6 projections' (80 and 48 wide, faster on
    the library GEMM) do not."""
    gen = torch.Generator().manual_seed(9)
    K = 1024
    big = _ints((768, K), gen).cuda()
    X = _ints((384, K), gen).cuda()
    sink = torch.full((384, 384 + 64), 5.0, device="cuda")
    wgrad(big[192:576], X, out=sink[:, :384])
    assert torch.equal(sink[:, :384].cpu(), big[192:576].cpu().float() @ X.cpu().float().t())
    assert bool((sink[:, 384:] == 5.0).all())
    T = 16384
    dxz = torch.empty(3072, T, dtype=torch.bfloat16, device="cuda")
    x = torch.empty(768, T, dtype=torch.bfloat16, device="cuda")
    dy = torch.empty(768, T, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(1536, T, dtype=torch.bfloat16, device="cuda")
    u = torch.empty(1536, T, dtype=torch.bfloat16, device="cuda")
    dx_dbl = torch.empty(80, T, dtype=torch.bfloat16, device="cuda")
    assert wgrad_fits(dxz, x) and wgrad_fits(dy, y)
    assert not wgrad_fits(dx_dbl, u) and not wgrad_fits(u, dx_dbl[:48])
    assert not wgrad_fits(dxz, torch.empty(462, T, dtype=torch.bfloat16, device="cuda"))  # N % 4
