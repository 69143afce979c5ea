"""Token embedding gathered into the channel-major stream (mss_embed_cm) and its gradient
(mss_embed_cm_backward), behind mamba_amd.lm_ops.embed_cm. Reference behaviour: the LM's input
embedding, nnx.Embed (mamba/mamba1.py:378-380), whose table the output head shares; the bar is
torch's own gather (bit for bit: a copy) and its scatter-add gradient (float32, the run of each
token summed in another association: within 2^-20 of the sum of |terms| per element, plus the
same for a gradient already held for the tied head), and determinism (two runs bit for bit).

CPU: the C entry points' argument checks (each rejected call returns before any launch).
GPU: shapes with partial 64 x 64 tiles, out-of-range tokens (NaN columns, skipped in the
gradient), runs of equal tokens longer than the kernel's linear probe (its binary search), the
tied-head holder, and the LM's gradients against the plain gather at the config-1 shape.
"""
import pytest
import torch

from mamba_amd import _lib
from mamba_amd.lm_ops import GradHolder, embed_cm


@pytest.fixture(scope="module")
def lib():
    return _lib.register_hip_kernel()


_A = 1 << 32  # 16-byte aligned, never dereferenced: every call below is rejected first


def test_embed_validation(lib):
    bad, uns = _lib.MSS_ERR_INVALID_ARGUMENT, _lib.MSS_ERR_UNSUPPORTED
    f = lib.mss_embed_cm
    assert f(None, 64, _A, 10, 8, _A + (1 << 20), 64, None) == bad
    assert f(_A, 0, _A + 4096, 10, 8, _A + (1 << 20), 64, None) == bad
    assert f(_A, 64, _A + 4096, 0, 8, _A + (1 << 20), 64, None) == bad
    assert f(_A, 64, _A + 4096, 10, 8, _A + (1 << 20), 63, None) == bad    # ldh < T
    assert f(_A, 64, _A + 4096, 10, 8, _A + 4096 + 64, 64, None) == bad    # h overlaps E
    assert f(_A, 1 << 31, _A + 4096, 10, 8, _A + (1 << 40), 1 << 31, None) == bad
    b = lib.mss_embed_cm_backward
    ok = dict(dh=_A, ldh=64, st=_A + (1 << 20), order=_A + (2 << 20), T=64, V=10, D=8, dE=_A + (3 << 20),
              ws=_A + (4 << 20), wsb=64 * 8 * 4)

    def call(**kw):
        a = dict(ok, **kw)
        return b(a["dh"], a["ldh"], a["st"], a["order"], a["T"], a["V"], a["D"], a["dE"], a["ws"], a["wsb"], None)

    assert call(dh=None) == bad and call(order=None) == bad and call(ws=None) == bad
    assert call(T=0) == bad and call(V=0) == bad and call(ldh=63) == bad
    assert call(D=6) == uns and call(D=1028) == uns                        # D % 4, D <= 1024
    assert call(wsb=64 * 8 * 4 - 1) == bad                                  # workspace too small
    assert call(dE=_A + (3 << 20) + 8) == bad                               # dE alignment
    assert call(dE=_A + 16) == bad                                          # dE overlaps dh
    assert call(ws=_A + (3 << 20) + 64) == bad                              # workspace overlaps dE


def _case(V, D, T, seed, lo=0, hi=None):
    g = torch.Generator().manual_seed(seed)
    table = torch.randn(V, D, generator=g)
    tokens = torch.randint(lo, V if hi is None else hi, (T,), generator=g)
    dh = torch.randn(D, T, generator=g)
    return table, tokens, dh


@pytest.mark.gpu
@pytest.mark.parametrize("V,D,T", [(50, 64, 64), (1000, 100, 1100), (7, 768, 4096), (50280, 768, 2048), (3, 4, 70)])
def test_embed_forward_matches_gather(V, D, T):
    print(f"case embed fwd V={V} D={D} T={T}", flush=True)
    table, tokens, _ = _case(V, D, T, V + D + T)
    h = embed_cm(table.cuda(), tokens.cuda())
    assert h.shape == (D, T) and h.is_contiguous()
    assert torch.equal(h.cpu(), table[tokens].t())


@pytest.mark.gpu
def test_embed_forward_out_of_range_tokens():
    print("case embed fwd out of range", flush=True)
    table, tokens, _ = _case(20, 8, 130, 1)
    tokens[[0, 65, 129]] = torch.tensor([-1, 20, 1 << 40])
    h = embed_cm(table.cuda(), tokens.cuda()).cpu()
    bad = torch.zeros(130, dtype=torch.bool)
    bad[[0, 65, 129]] = True
    assert bool(torch.isnan(h[:, bad]).all())
    assert torch.equal(h[:, ~bad], table[tokens[~bad]].t())


def _reference_grad(V, D, tokens, dh, held=None):
    """Float64 scatter-add of dh's columns by token, plus a held gradient, and the sum of
    |terms| per element for the tolerance."""
    ok = (tokens >= 0) & (tokens < V)
    ref = torch.zeros(V, D, dtype=torch.float64)
    mag = torch.zeros(V, D, dtype=torch.float64)
    ref.index_add_(0, tokens[ok], dh.t()[ok].double())
    mag.index_add_(0, tokens[ok], dh.t()[ok].double().abs())
    if held is not None:
        ref += held.double()
        mag += held.double().abs()
    return ref, mag


@pytest.mark.gpu
@pytest.mark.parametrize("V,D,T,hi", [(1000, 100, 1100, None), (7, 768, 4096, None), (50280, 768, 16384, None),
                                      (50, 64, 3000, 2), (5, 4, 64, None)])
@pytest.mark.parametrize("held", [False, True])
def test_embed_backward_matches_scatter_add(V, D, T, hi, held):
    """hi=2: two tokens share 3000 positions (runs far past the linear probe)."""
    print(f"case embed bwd V={V} D={D} T={T} hi={hi} held={held}", flush=True)
    table, tokens, dh = _case(V, D, T, 7 * V + D + T, hi=hi)
    tokens[T // 2] = V + 3  # skipped
    g = torch.Generator().manual_seed(3)
    h0 = torch.randn(V, D, generator=g) if held else None
    outs = []
    for _ in range(2):
        t = table.cuda().requires_grad_(True)
        holder = GradHolder()
        if held:
            holder.put(h0.cuda())
        h = embed_cm(t, tokens.cuda(), holder)
        h.backward(dh.cuda())
        assert holder.grad is None  # taken by the backward
        outs.append(t.grad.cpu())
    assert torch.equal(outs[0], outs[1])  # deterministic
    ref, mag = _reference_grad(V, D, tokens, dh, h0)
    err = (outs[0].double() - ref).abs()
    assert bool((err <= 2.0 ** -20 * mag).all()), float((err / mag.clamp_min(1e-30)).max())


@pytest.mark.gpu
def test_lm_gradients_with_native_embedding():
    """The config-1 LM (bf16 activations, shadows, tied head) with the HIP gather against the
    same weights with torch's gather: logits bit for bit, the embedding gradient (head + gather
    through the holder vs two autograd edges) within float32 rounding of its scale, every
    other gradient bit for bit."""
    print("case lm gradients native embedding", flush=True)
    from mamba_amd.lm_ops import cross_entropy
    from mamba_amd.mamba1 import MambaLM
    import mamba_amd.mamba1 as m1

    torch.manual_seed(5)
    model = MambaLM(256, 64, 2, 2, 16, None, 4, device="cuda")
    tokens = torch.randint(0, 256, (8, 257), device="cuda")
    inp, tgt = tokens[:, :-1].contiguous(), tokens[:, 1:].reshape(-1)
    grads = []
    for native in (True, False):
        model.zero_grad(set_to_none=True)
        saved = m1.embed_cm, m1.GradHolder
        if not native:  # torch's gather, and the head's gradient on its own autograd edge
            m1.embed_cm = lambda table, tok, holder=None: table[tok.reshape(-1)].t().contiguous()
            m1.GradHolder = lambda: None
        try:
            logits = model(inp)
            loss = cross_entropy(logits, tgt)
            loss.backward()
        finally:
            m1.embed_cm, m1.GradHolder = saved
        grads.append((logits.detach().clone(), {k: p.grad.clone() for k, p in model.named_parameters()}))
    (la, ga), (lb, gb) = grads
    assert torch.equal(la, lb)
    for k in ga:
        if k == "embedding":
            scale = float(gb[k].abs().max())
            assert float((ga[k] - gb[k]).abs().max()) <= 1e-6 * scale, k
        else:
            assert torch.equal(ga[k], gb[k]), k
