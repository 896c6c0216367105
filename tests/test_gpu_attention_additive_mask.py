"""Additive (floating) attention masks on the fused kernels (GPU) vs the CPU oracle.

The reference's general attention adds a floating ``attn_mask`` to the scores, so
to their constant order (/root/reference/src/polytensors/_decompositions.py:38-40),
and its tests run an additive mask with -inf entries and a row with no
admissible key (/root/reference/tests/test_attention.py:49-55,60-91). Here the
forward and the gradient series of that case, and of larger ones, are checked
against ``oracle.attention`` / ``oracle.attention_backward`` (pinned against jets
in tests/test_oracle_pins.py) in float64 on the same (upcast) inputs. A row with
no admissible key gets output zero and finite zero gradients (the fused-kernel
convention; the general rule's softmax gives NaN there, so the oracle is compared
on the other rows). Per-order tolerance max|got - want| / max|want|: 1e-10
float64, 1e-4 float32, 2e-2 bfloat16 (the reference's half-type tolerance,
/root/reference/tests/test_fused_kernels.py:64-72).
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _series(shape, degree, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]


def _additive(L, S, seed, window=None, empty_rows=()):
    """Normal values with -inf outside a band (key j admissible for query i when
    0 <= i + 10 - j <= window) and on ``empty_rows``."""
    g = torch.Generator().manual_seed(seed)
    mask = torch.randn(L, S, generator=g, dtype=torch.float64)
    if window is not None:
        i, j = torch.arange(L)[:, None], torch.arange(S)[None, :]
        band = (i + 10 - j >= 0) & (i + 10 - j <= window)
        mask = mask.masked_fill(~band, float("-inf"))
    for r in empty_rows:
        mask[r] = float("-inf")
    return mask


def _kept(mask):
    return ~torch.isneginf(mask).all(-1)


def _check(got, want, dtype, rows=None, what=""):
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.detach().cpu().double(), b.double()
        if rows is not None:
            a, b = a[..., rows, :], b[..., rows, :]
        err = rel_err(a, b)
        assert err <= TOL[dtype], f"{what} order {k}: {err:.3e}"


def _poly(cs, dtype, grad=False):
    return PolyTensor(tuple(c.to(dtype).cuda() for c in cs), requires_grad=grad)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("window", [None, 37])
@pytest.mark.parametrize("degree", [1, 3, 8])
def test_forward_matches_oracle(monkeypatch, dtype, window, degree):
    calls = []
    original = _ops.taylor_attention_fwd
    monkeypatch.setattr(_ops, "taylor_attention_fwd", lambda *a, **k: calls.append(1) or original(*a, **k))
    shape = (2, 3, 150, 64)
    Q, K, V = (_series(shape, degree, 10 + i) for i in range(3))
    mask = _additive(150, 150, 20, window=window, empty_rows=(7,))
    with torch.no_grad(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(_poly(Q, dtype), _poly(K, dtype), _poly(V, dtype),
                                             attn_mask=mask.to(dtype).cuda())
    assert calls == [1] and out.degree == degree and out.dtype == dtype
    up = [[c.to(dtype).double() for c in s] for s in (Q, K, V)]
    want = oracle.attention(*up, attn_mask=mask.to(dtype).double())
    _check(out.coeffs, want, dtype, rows=_kept(mask))
    assert all(c[..., 7, :].abs().max().item() == 0 for c in out.coeffs)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("L,S", [(1, 16), (65, 33), (130, 47)])
@pytest.mark.parametrize("plain_q", [False, True])
def test_forward_ragged_lengths_and_lse(dtype, L, S, plain_q):
    # every order given (the 16-bit pipelined kernel) and an ordinary query (the staged kernels);
    # 16-bit operands take the mask's float32 values directly
    degree = 2
    Q = _series((2, L, 32), degree, 30)[:1 if plain_q else None]
    K, V = (_series((2, S, 32), degree, 31 + i) for i in range(2))
    mask = _additive(L, S, 33, window=20)
    q, k, v = ([c.to(dtype).cuda() for c in s] for s in (Q, K, V))
    out, lse = _ops.taylor_attention_fwd(q, k, v, mask.to(dtype).cuda(), False, 0.3, degree)
    assert out.dtype == dtype and lse.dtype == (torch.float64 if dtype == torch.float64 else torch.float32)
    up = [oracle.paths.lift([c.to(dtype).double() for c in s], degree) for s in (Q, K, V)]
    madd = mask.to(dtype).double()   # the mask's values as the kernel received them
    want = oracle.attention(*up, attn_mask=madd, scale=0.3)
    _check(out.unbind(0), want, dtype, rows=_kept(mask))
    # lse series of the admissible scores (the constant order shifted by the mask)
    scores = oracle.series.cauchy([c * 0.3 for c in up[0]], [c.transpose(-2, -1) for c in up[1]], matmul=True)
    keep = ~torch.isneginf(madd)
    scores = [torch.where(keep, s + (madd if i == 0 else 0.0), torch.full((), float("-inf") if i == 0 else 0.0,
                                                                         dtype=s.dtype))
              for i, s in enumerate(scores)]
    want_lse = oracle.series.softmax_family(scores, -1)[2]
    rows = _kept(mask)
    for i in range(degree + 1):
        a, b = lse[i].cpu().double()[:, rows], want_lse[i][..., 0][:, rows]
        assert rel_err(a, b) <= TOL[dtype], f"lse order {i}"


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("degree", [0, 2, 4])
def test_gradient_series_match_oracle(dtype, degree):
    bh, L, d = 3, 150, 64
    Q, K, V, G = (_series((bh, L, d), degree, 100 + i) for i in range(4))
    mask = _additive(L, L, 40, window=21, empty_rows=(3, 90))
    q, k, v, g = ([c.to(dtype).cuda() for c in s] for s in (Q, K, V, G))
    m = mask.to(dtype).cuda()
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, m, False, scale, degree)
    for materialize in (-1, 1):   # the additive mask always recomputes; materialize is ignored
        got = _ops.taylor_attention_bwd(q, k, v, out, lse, g, m, False, scale, materialize)
        up = [[c.to(dtype).double() for c in s] for s in (Q, K, V, G)]
        want = oracle.attention_backward(*up, attn_mask=mask)
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.isfinite(a).all(), name
            _check(a.unbind(0), b, dtype, what=name)


@pytest.mark.parametrize("degree", [3, 8])
@pytest.mark.parametrize("d", [16, 128])
def test_float64_every_head_dim_through_autograd(degree, d):
    # wrapper autograd through F.scaled_dot_product_attention: forward and gradient series
    L = 83
    Q, K, V, G = (_series((2, L, d), degree, 120 + i) for i in range(4))
    mask = _additive(L, L, 50, window=30, empty_rows=(0,))
    q, k, v = (_poly(s, torch.float64, grad=True) for s in (Q, K, V))
    with PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda())
        out.backward(_poly(G, torch.float64))
    want = oracle.attention(Q, K, V, attn_mask=mask)
    _check(out.coeffs, want, torch.float64, rows=_kept(mask))
    grads = oracle.attention_backward(Q, K, V, G, attn_mask=mask)
    for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), grads):
        _check(x.grad.coeffs, b, torch.float64, what=name)


def test_reference_case():
    # the data and additive mask of /root/reference/tests/test_attention.py:13-17,53-54 (seed 27,
    # [1, 1, 3, 2] values / 3, directions / 4, degree 3), the head dim zero-padded to 16 (zero
    # columns change neither the scores nor the other output columns)
    g = torch.Generator().manual_seed(27)
    values = [torch.randn(1, 1, 3, 2, generator=g, dtype=torch.float64) / 3 for _ in range(3)]
    directions = [torch.randn(c.shape, generator=g, dtype=c.dtype) / 4 for c in values]
    inf = float("-inf")
    mask = torch.tensor([[inf] * 3, [0.2, inf, -0.1], [0.1, -0.3, 0.0]], dtype=torch.float64)
    pad = lambda t: F.pad(t, (0, 14))   # noqa: E731
    series = [oracle.paths.lift([x, d], 3) for x, d in zip(values, directions)]
    q, k, v = (PolyTensor(tuple(pad(c).cuda() for c in s), requires_grad=True) for s in series)
    with PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda(), scale=1 / math.sqrt(2))
        G = [2 * c.detach() for c in out.coeffs]   # cotangent of sum(out^2) at the constant order
        out.backward(PolyTensor(tuple(G)))
    want = oracle.attention(*series, attn_mask=mask)
    for c in out.coeffs:
        assert torch.equal(c[..., 0, :].cpu(), torch.zeros_like(c[..., 0, :].cpu()))
        assert c[..., 2:].abs().max().item() == 0
    _check([c[..., :2] for c in out.coeffs], want, torch.float64, rows=torch.tensor([False, True, True]))
    grads = oracle.attention_backward(*series, [g[..., :2].cpu() for g in G], attn_mask=mask)
    for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), grads):
        for c in x.grad.coeffs:
            assert torch.isfinite(c).all()
        _check([c[..., :2] for c in x.grad.coeffs], b, torch.float64, what=name)
