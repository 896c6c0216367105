"""Attention gradient series with bfloat16 / float16 operands (GPU) vs the CPU oracle.

The 16-bit backward kernels take Q, K, V and the cotangent series G as stored
into 16x16x32 MFMAs with fp32 accumulation; the probability and dS series are
rounded to the storage type as operands of the products that contract them
(a hi + lo pair from degree 5), and every gradient is rounded once. The oracle
(``oracle.attention_backward``, pinned against jets of torch.func.vjp in
tests/test_oracle_pins.py) runs in float64 on the same stored 16-bit inputs,
upcast. Both paths run: P and dS recomputed by the dK / dV kernels, and stored by
the dQ kernel (degrees 1..4, materialize=1; elsewhere the request falls back to
recomputing). Cases: every degree 0..8 and head dim, causal / boolean window /
unmasked / additive masks, unequal and ragged lengths, a single query, skipped
blocks, masks over the batch through autograd, one gradient not wanted (NULL
outputs through the C ABI, here and for float32), and the full config-3 shape (one
head against the oracle, linearity in G over all heads).
Tolerance per order, max|got - want| / max|want|: 2e-2 (the north star's
bf16-input / fp32-accumulate bound; the reference compares its half-type
gradients with float32 at 5e-2, /root/reference/tests/test_fused_kernels.py:64-72).
"""

import ctypes
import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _lib, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

HALF = [torch.bfloat16, torch.float16]
TOL = 2e-2


def _series(shape, degree, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k).to(dtype)
            for k in range(degree + 1)]


def _up(cs):
    return [c.double() for c in cs]


def _window_mask(L, S, window):
    i, j = torch.arange(L)[:, None], torch.arange(S)[None, :]
    return (i >= j) & (i - j <= window)


def _check(got, want, what, floor=0.0, tol=TOL):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.detach().cpu().double(), b.double()
        err = (a - b).abs().max().item() / max(b.abs().max().item(), floor) if b.numel() else 0.0
        assert err <= tol, f"{what} order {k}: {err:.3e} > {tol:.0e}"


def _grads(Q, K, V, G, mask=None, causal=False, materialize=-1):
    """Forward then the 16-bit backward on [bh, T, d] series (mask: bool or float (L, S));
    materialize 1: the dQ kernel stores the P and dS series and the dK / dV kernels read them
    (degrees 1..4), 0: the scores are recomputed, -1: the operator's choice."""
    q, k, v, g = ([c.cuda() for c in s] for s in (Q, K, V, G))
    degree, scale = len(q) - 1, 1 / math.sqrt(q[0].shape[-1])
    m = None if mask is None else (mask.cuda() if mask.dtype == torch.bool else mask.float().cuda())
    out, lse = _ops.taylor_attention_fwd(q, k, v, m, causal, scale, degree)
    dq, dk, dv = _ops.taylor_attention_bwd(q, k, v, out, lse, g, m, causal, scale, materialize)
    assert dq.dtype == dk.dtype == dv.dtype == q[0].dtype
    return dq.unbind(0), dk.unbind(0), dv.unbind(0)


def _compare(Q, K, V, G, mask=None, causal=False, what="", materialize=-1):
    got = _grads(Q, K, V, G, mask=mask, causal=causal, materialize=materialize)
    want = oracle.attention_backward(_up(Q), _up(K), _up(V), _up(G),
                                     attn_mask=mask if mask is None or mask.dtype == torch.bool else mask.double(),
                                     is_causal=causal)
    # a row with one admissible key has softmax 1 and dQ exactly 0: scale by the inputs instead
    floor = 1.0 if K[0].shape[-2] == 1 or Q[0].shape[-2] == 1 else 0.0
    for name, a, b in zip(("dq", "dk", "dv"), got, want):
        _check(a, b, f"{what} {name}", floor=floor)


@pytest.mark.parametrize("materialize", [0, 1])
@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("degree", range(9))
@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_every_degree_and_head_dim(dtype, degree, d, materialize):
    Q, K, V, G = (_series((2, 80, d), degree, 10 + i, dtype) for i in range(4))
    _compare(Q, K, V, G, causal=True, what=f"K={degree} d={d}", materialize=materialize)


@pytest.mark.parametrize("materialize", [0, 1])
@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("mode", ["none", "causal", "window", "additive"])
@pytest.mark.parametrize("L,S", [(150, 150), (70, 33), (33, 70), (1, 40), (130, 96)])
@pytest.mark.parametrize("degree", [1, 4, 6])
def test_masks_and_lengths(dtype, mode, L, S, degree, materialize):
    Q, K, V, G = (_series((3, T, 64), degree, 20 + i, dtype) for i, T in enumerate((L, S, S, L)))
    mask, causal = None, mode == "causal"
    if mode == "window":
        mask = _window_mask(L, S, 37)
    elif mode == "additive":
        g = torch.Generator().manual_seed(29)
        keep = torch.rand(L, S, generator=g) < 0.7
        keep[:, 0] = True   # every row admits a key (the oracle's NaN rows are covered elsewhere)
        mask = torch.randn(L, S, generator=g, dtype=torch.float64).masked_fill(~keep, float("-inf"))
    _compare(Q, K, V, G, mask=mask, causal=causal, what=f"{mode} L={L} S={S} K={degree}", materialize=materialize)


@pytest.mark.parametrize("materialize", [0, 1])
@pytest.mark.parametrize("dtype", HALF)
def test_rows_and_columns_without_admissible_pairs(dtype, materialize):
    # a window with a query block masked out and a key block that no query admits: skipped blocks
    # of both kernels; their gradients are zero
    L, d, degree = 320, 32, 2
    mask = _window_mask(L, L, 50)
    mask[64:128] = False
    mask[:, 192:256] = False
    Q, K, V, G = (_series((2, L, d), degree, 30 + i, dtype) for i in range(4))
    dq, dk, dv = _grads(Q, K, V, G, mask=mask, materialize=materialize)
    for o in range(degree + 1):
        assert dq[o][:, 64:128].abs().max().item() == 0
        assert dk[o][:, 192:256].abs().max().item() == 0 and dv[o][:, 192:256].abs().max().item() == 0
    _compare(Q, K, V, G, mask=mask, what="skipped blocks", materialize=materialize)


@pytest.mark.parametrize("dtype", HALF)
def test_through_autograd_with_masks_over_the_batch(dtype):
    # F.scaled_dot_product_attention on 16-bit series, a [B, 1, L, S] padding-style mask
    degree, shape = 2, (2, 3, 96, 64)
    Q, K, V, G = (_series(shape, degree, 40 + i, dtype) for i in range(4))
    g = torch.Generator().manual_seed(45)
    mask = torch.rand(2, 1, 96, 96, generator=g) < 0.7
    mask[..., 0] = True
    q, k, v = (PolyTensor(tuple(c.cuda() for c in s), requires_grad=True) for s in (Q, K, V))
    with PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda())
        out.backward(PolyTensor(tuple(c.cuda() for c in G)))
    want = oracle.attention_backward(_up(Q), _up(K), _up(V), _up(G), attn_mask=mask)
    for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), want):
        assert x.grad.dtype == dtype
        _check(x.grad.coeffs, b, name)


def _abi_bwd(q, k, v, out, lse, g, dtype, materialize, want_q=True, want_k=True, want_v=True):
    """pt_taylor_attention_bwd through ctypes with the gradients not wanted passed as NULL."""
    lib = _lib.load()
    degree = len(q) - 1
    bh, L, d = q[0].shape
    S = k[0].shape[1]
    outs = [torch.full((degree + 1, bh, T, d), float("nan"), dtype=dtype, device="cuda") for T in (L, S, S)]
    code = _lib.DTYPE_CODES[dtype]
    ws = torch.empty(max(1, lib.pt_taylor_attention_bwd_workspace_size(code, degree, bh, L, S, materialize)),
                     dtype=torch.uint8, device="cuda")
    arrays = [_lib.ptr_array(list(t.unbind(0))) if want else None
              for t, want in zip(outs, (want_q, want_k, want_v))]
    status = lib.pt_taylor_attention_bwd(
        code, degree, _lib.ptr_array(q), _lib.ptr_array(k), _lib.ptr_array(v), _lib.ptr_array(list(out.unbind(0))),
        _lib.ptr_array(list(lse.unbind(0))), _lib.ptr_array(g), *arrays, ws.data_ptr(), materialize, bh, L, S, d,
        1, None, None, None, None, 1 / math.sqrt(d), _lib.stream_of(q[0].device))
    _lib.check(status, "taylor_attention_bwd")
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("dtype,materialize", [(torch.bfloat16, 0), (torch.float16, 0), (torch.bfloat16, 1),
                                               (torch.float16, 1), (torch.float32, 0), (torch.float32, 1)])
@pytest.mark.parametrize("d", [32, 128])
def test_gradients_not_wanted_are_not_written(dtype, materialize, d):
    # NULL dq / dk / dv: the other outputs equal the full call's bit for bit and the NULL one's buffer
    # is untouched (head dim 32: the dK/dV pass is fused when both are wanted)
    degree = 2
    q, k, v, g = ([c.cuda() for c in _series((2, 100, d), degree, 50 + i, dtype)] for i in range(4))
    out, lse = _ops.taylor_attention_fwd(q, k, v, None, True, 1 / math.sqrt(d), degree)
    full = _abi_bwd(q, k, v, out, lse, g, dtype, materialize)
    assert all(torch.isfinite(t).all() for t in full)
    for wants in [(True, False, True), (True, True, False), (False, True, True), (False, False, True)]:
        got = _abi_bwd(q, k, v, out, lse, g, dtype, materialize, *wants)
        for want, a, b in zip(wants, got, full):
            if want:
                assert torch.equal(a, b)
            else:
                assert torch.isnan(a).all()


@pytest.mark.parametrize("dtype", HALF)
def test_close_to_float32(dtype):
    # /root/reference/tests/test_fused_kernels.py:64-72 at degrees 1 and 3: the 16-bit gradient
    # series against the float32 kernels' on the same stored inputs, within 5e-2
    for degree in (1, 3):
        Q, K, V, G = (_series((2, 256, 128), degree, 60 + i, dtype, scale=0.5) for i in range(4))
        half = _grads(Q, K, V, G, causal=True)
        full = _grads(*([c.float() for c in s] for s in (Q, K, V, G)), causal=True)
        for a, b in zip(half, full):
            for x, y in zip(a, b):
                assert rel_err(x.float().cpu(), y.cpu()) < 5e-2


@pytest.mark.parametrize("materialize", [0, 1])
@pytest.mark.parametrize("dtype", HALF)
def test_full_size_config3(dtype, materialize):
    # benchmark config 3's shape (B=4 H=16 L=2048 d=128, K=4, causal, line inputs) in 16-bit storage
    # with a random cotangent series: one head against the oracle; on every head, linearity in G
    # (bwd(G1 + G2) = bwd(G1) + bwd(G2) within twice the rounding tolerance)
    B, H, L, d, degree = 4, 16, 2048, 128, 4
    gen = torch.Generator(device="cuda").manual_seed(5)

    def line():
        base = torch.randn(B * H, L, d, generator=gen, device="cuda") / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=gen, device="cuda")
        return [base.to(dtype), direction.to(dtype)] + [torch.zeros_like(base, dtype=dtype) for _ in range(degree - 1)]

    def cot():
        return [(torch.randn(B * H, L, d, generator=gen, device="cuda") * 0.5 ** k).to(dtype) for k in range(degree + 1)]

    q, k, v = line(), line(), line()
    g1, g2 = cot(), cot()
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, None, True, scale, degree)
    r1 = _ops.taylor_attention_bwd(q, k, v, out, lse, g1, None, True, scale, materialize)
    head = 21
    want = oracle.attention_backward(*([c[head].cpu().double() for c in s] for s in (q, k, v, g1)), is_causal=True)
    for name, got, w in zip(("dq", "dk", "dv"), r1, want):
        _check([c[head] for c in got], w, name)
    r2 = _ops.taylor_attention_bwd(q, k, v, out, lse, g2, None, True, scale, materialize)
    r12 = _ops.taylor_attention_bwd(q, k, v, out, lse, [a + b for a, b in zip(g1, g2)], None, True, scale,
                                    materialize)
    for name, a, b, ab in zip(("dq", "dk", "dv"), r1, r2, r12):
        for o in range(degree + 1):
            lhs, rhs = ab[o].double(), a[o].double() + b[o].double()
            err = ((lhs - rhs).abs().amax(dim=(1, 2)) / rhs.abs().amax(dim=(1, 2))).max().item()
            assert err <= 2 * TOL, f"{name} order {o}: linearity {err:.3e}"
