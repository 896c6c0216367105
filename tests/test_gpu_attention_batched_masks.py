"""Attention masks that differ over the batch (GPU) vs the CPU oracle.

The reference's general rule broadcasts ``attn_mask`` against the scores
(/root/reference/src/polytensors/_decompositions.py:36-41), so a mask may be
(L, S) or carry batch dimensions: one per batch entry ([B, 1, L, S], a padding
mask), one per head ([1, H, L, S]), one per (batch, head), or another rank of
batch. The kernels take such a mask as a set of (L, S) masks with a map from
heads to masks (the ``mask_map`` of the attention entry points). Checked: the
forward series of boolean and additive masks of every such shape, the gradient
series through autograd, bfloat16 operands, a mask together with is_causal, a
mask set with an explicit map against one mask per head (outputs and lse), and
the operator's refusal of a map that sends a head past the masks given. The oracle
(``oracle.attention`` / ``oracle.attention_backward``, whose broadcast masks match
per-entry calls exactly: tests/test_oracle_pins.py) runs in float64 on the same
(upcast) inputs; rows with no admissible key are compared as zero (the fused
convention) and left out of the oracle comparison (NaN in its general rule).
Per-order tolerance max|got - want| / max|want|: 1e-10 float64, 1e-4 float32,
2e-2 bfloat16.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _series(shape, degree, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]


def _band_masks(shape, L, S, seed):
    """Boolean masks of ``shape`` (..., L, S): a band of a different width per entry, and one
    row per entry with no admissible key."""
    g = torch.Generator().manual_seed(seed)
    lead = shape[:-2]
    n = 1
    for x in lead:
        n *= x
    i, j = torch.arange(L)[:, None], torch.arange(S)[None, :]
    masks = []
    for e in range(n):
        w = int(torch.randint(5, 60, (1,), generator=g))
        m = (i + 3 - j >= 0) & (i + 3 - j <= w)
        m[int(torch.randint(0, L, (1,), generator=g))] = False
        masks.append(m)
    return torch.stack(masks).reshape(shape)


def _empty_rows(mask, batch):
    """[*batch, L] True where a query row has no admissible key."""
    keep = mask if mask.dtype == torch.bool else ~torch.isneginf(mask)
    return (~keep.any(-1)).expand(*batch, keep.shape[-2])


def _check(got, want, empty, dtype, what=""):
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.detach().cpu().double(), b.double()
        assert a[empty].abs().max().item() == 0 if empty.any() else True, f"{what} order {k}: empty rows"
        a, b = a[~empty], b[~empty]
        err = rel_err(a, b)
        assert err <= TOL[dtype], f"{what} order {k}: {err:.3e}"


def _poly(cs, dtype, grad=False):
    return PolyTensor(tuple(c.to(dtype).cuda() for c in cs), requires_grad=grad)


MASK_SHAPES = [(2, 1, 150, 150), (1, 3, 150, 150), (3, 150, 150), (2, 3, 150, 150)]


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("additive", [False, True])
@pytest.mark.parametrize("mshape", MASK_SHAPES)
def test_forward_matches_oracle(monkeypatch, dtype, additive, mshape):
    calls = []
    original = _ops.taylor_attention_fwd
    monkeypatch.setattr(_ops, "taylor_attention_fwd", lambda *a, **k: calls.append(1) or original(*a, **k))
    degree, shape = 2, (2, 3, 150, 64)
    Q, K, V = (_series(shape, degree, 10 + i) for i in range(3))
    mask = _band_masks(mshape, 150, 150, 20)
    if additive:
        g = torch.Generator().manual_seed(21)
        mask = torch.randn(mshape, generator=g, dtype=torch.float64).masked_fill(~mask, float("-inf"))
        mask = mask.to(dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(_poly(Q, dtype), _poly(K, dtype), _poly(V, dtype),
                                             attn_mask=mask.cuda())
    assert calls == [1] and out.dtype == dtype
    up = [[c.to(dtype).double() for c in s] for s in (Q, K, V)]
    want = oracle.attention(*up, attn_mask=mask.double() if additive else mask)
    _check(out.coeffs, want, _empty_rows(mask, shape[:-2]), dtype)


def test_five_dimensional_batch():
    # batch (2, 2, 3) with a mask over the first batch dimension only: one mask per head
    degree, shape = 1, (2, 2, 3, 70, 32)
    Q, K, V = (_series(shape, degree, 30 + i) for i in range(3))
    mask = _band_masks((2, 1, 1, 70, 70), 70, 70, 33)
    with torch.no_grad(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(_poly(Q, torch.float64), _poly(K, torch.float64),
                                             _poly(V, torch.float64), attn_mask=mask.cuda())
    want = oracle.attention(Q, K, V, attn_mask=mask)
    _check(out.coeffs, want, _empty_rows(mask, shape[:-2]), torch.float64)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("additive", [False, True])
@pytest.mark.parametrize("mshape", [(2, 1, 96, 96), (1, 3, 96, 96), (2, 3, 96, 96)])
def test_gradient_series_through_autograd(dtype, additive, mshape):
    degree, shape = 2, (2, 3, 96, 64)
    Q, K, V, G = (_series(shape, degree, 40 + i) for i in range(4))
    mask = _band_masks(mshape, 96, 96, 44)
    if additive:
        g = torch.Generator().manual_seed(45)
        mask = torch.randn(mshape, generator=g, dtype=torch.float64).masked_fill(~mask, float("-inf")).to(dtype)
    q, k, v = (_poly(s, dtype, grad=True) for s in (Q, K, V))
    with PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda())
        out.backward(_poly(G, dtype))
    up = [[c.to(dtype).double() for c in s] for s in (Q, K, V, G)]
    m = mask.double() if additive else mask
    empty = _empty_rows(mask, shape[:-2])
    _check(out.coeffs, oracle.attention(*up[:3], attn_mask=m), empty, dtype)
    grads = oracle.attention_backward(*up, attn_mask=m)
    none = torch.zeros(shape[:-2] + (96,), dtype=torch.bool)   # gradients: every row compared
    for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), grads):
        _check(x.grad.coeffs, b, none, dtype, what=name)


def test_operator_mask_sets_and_maps():
    degree, bh, L, d = 1, 6, 40, 16
    Q, K, V = (_series((bh, L, d), degree, 50 + i) for i in range(3))
    q, k, v = ([c.cuda() for c in s] for s in (Q, K, V))
    masks = _band_masks((2, L, L), L, L, 53)
    # heads 0-2 use mask 0, heads 3-5 mask 1 (a [2, 1, L, L] mask over 3 heads)
    out, lse = _ops.taylor_attention_fwd(q, k, v, masks.cuda(), False, 0.25, degree, mask_map=[3, 1, 0])
    per_head = masks.repeat_interleave(3, dim=0)
    out2, lse2 = _ops.taylor_attention_fwd(q, k, v, per_head.cuda(), False, 0.25, degree)   # one mask per head
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    want = oracle.attention(Q, K, V, attn_mask=per_head, scale=0.25)
    _check(out.unbind(0), want, _empty_rows(per_head, (bh,)), torch.float64)
    with pytest.raises(ValueError, match="past"):
        _ops.taylor_attention_fwd(q, k, v, masks.cuda(), False, 0.25, degree, mask_map=[2, 1, 0])
    with pytest.raises(ValueError, match="one mask per head"):
        _ops.taylor_attention_fwd(q, k, v, masks.cuda(), False, 0.25, degree)
    with pytest.raises(ValueError, match="mask_map"):
        _ops.taylor_attention_fwd(q, k, v, masks[0].cuda(), False, 0.25, degree, mask_map=[1, 1, 0])


@pytest.mark.parametrize("additive", [False, True])
def test_causal_together_with_a_mask(additive):
    # the general rule applies both (/root/reference/src/polytensors/_decompositions.py:36-41)
    degree, shape = 2, (2, 3, 100, 32)
    Q, K, V, G = (_series(shape, degree, 60 + i) for i in range(4))
    g = torch.Generator().manual_seed(64)
    mask = torch.rand(2, 1, 100, 100, generator=g) < 0.6
    if additive:
        mask = torch.randn(2, 1, 100, 100, generator=g, dtype=torch.float64).masked_fill(~mask, float("-inf"))
    q, k, v = (_poly(s, torch.float64, grad=True) for s in (Q, K, V))
    with PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda(), is_causal=True)
        out.backward(_poly(G, torch.float64))
    keep = (mask if not additive else ~torch.isneginf(mask)) & torch.ones(100, 100, dtype=torch.bool).tril()
    empty = (~keep.any(-1)).expand(2, 3, 100)
    _check(out.coeffs, oracle.attention(Q, K, V, attn_mask=mask, is_causal=True), empty, torch.float64)
    grads = oracle.attention_backward(Q, K, V, G, attn_mask=mask, is_causal=True)
    none = torch.zeros(2, 3, 100, dtype=torch.bool)
    for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), grads):
        _check(x.grad.coeffs, b, none, torch.float64, what=name)
