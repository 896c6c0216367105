"""Gradient series of the fused attention (GPU) vs the CPU oracle.

The backward kernels compute, for an output cotangent series G(t), the series
of the vector-Jacobian product J(x(t))^T G(t) for query, key and value
(/root/reference/src/polytensors/_fused_attention.py:267-295 at degree 1,
/root/reference/tests/test_fused_kernels.py:136-160 for its gradient check).
The oracle is ``oracle.attention_backward`` (pinned against jets of
torch.func.vjp in tests/test_oracle_pins.py) in float64 on the same (upcast)
inputs. Cases: every degree 0..8, every head dim, causal / boolean window /
unmasked, ragged and unequal query and key lengths, rows and columns with no
admissible pair, empty sequences, the autograd path through
F.scaled_dot_product_attention with ordinary operands, and the full-size
headline shape (one head against the oracle, linearity in G on all heads).
Per-order tolerance max|got - want| / max|want|: 1e-10 float64, 1e-4 float32.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4}


def _series(shape, degree, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]


def _window_mask(L, S, window):
    i, j = torch.arange(L)[:, None], torch.arange(S)[None, :]
    return (i >= j) & (i - j <= window)


def _check(got, want, dtype, what="", floor=0.0):
    """Per-order error relative to max|want|, or to ``floor`` where the exact series is ~0."""
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.detach().cpu().double(), b.double()
        err = (a - b).abs().max().item() / max(b.abs().max().item(), floor) if b.numel() else 0.0
        assert err <= TOL[dtype], f"{what} order {k}: {err:.3e} > {TOL[dtype]:.0e}"


def _kernel(Q, K, V, G, dtype, mask=None, causal=False, scale=None, materialize=-1):
    """Forward then backward kernels on [bh, T, d] series; returns (dq, dk, dv) as lists."""
    q, k, v, g = ([c.to(dtype).cuda().contiguous() for c in s] for s in (Q, K, V, G))
    degree = len(q) - 1
    scale = 1 / math.sqrt(q[0].shape[-1]) if scale is None else scale
    m = None if mask is None else mask.cuda()
    out, lse = _ops.taylor_attention_fwd(q, k, v, m, causal, scale, degree)
    dq, dk, dv = _ops.taylor_attention_bwd(q, k, v, out, lse, g, m, causal, scale, materialize)
    return list(dq.unbind(0)), list(dk.unbind(0)), list(dv.unbind(0))


def _oracle(Q, K, V, G, dtype, **kwargs):
    up = [[c.to(dtype).double() for c in s] for s in (Q, K, V, G)]
    return oracle.attention_backward(*up, **kwargs)


# The stored-tile path (materialize=1) is float32 only: a float64 run of it (degree 8, head dim 64)
# took a GPU memory fault whose cause is not established, and the library refuses it for float64.
FP64_MATERIALIZE = "the stored-tile backward is float32 only (float64 fault, cause not established)"


def _compare(Q, K, V, G, dtype, mask=None, causal=False, scale=None, materialize=-1):
    if dtype == torch.float64 and materialize == 1:
        pytest.skip(FP64_MATERIALIZE)
    got = _kernel(Q, K, V, G, dtype, mask=mask, causal=causal, scale=scale, materialize=materialize)
    want = _oracle(Q, K, V, G, dtype, attn_mask=mask, is_causal=causal, scale=scale)
    # with a single admissible key per row the softmax is 1 and dQ is exactly zero: scale by the
    # (order-one) inputs instead
    floor = 1.0 if K[0].shape[-2] == 1 or (causal and Q[0].shape[-2] == 1) else 0.0
    for name, a, b in zip(("dq", "dk", "dv"), got, want):
        _check(a, b, dtype, name, floor=floor)


# materialize 1: P and dS tiles stored by the dQ kernel and read by the dK/dV kernel; 0: recomputed
@pytest.mark.parametrize("materialize", [1, 0])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("causal,window", [(True, None), (False, 21), (False, None)])
@pytest.mark.parametrize("degree", [0, 1, 2, 4])
def test_matches_oracle(dtype, causal, window, degree, materialize):
    bh, L, d = 3, 150, 64
    Q, K, V, G = (_series((bh, L, d), degree, 100 + i) for i in range(4))
    mask = None if window is None else _window_mask(L, L, window)
    _compare(Q, K, V, G, dtype, mask=mask, causal=causal, materialize=materialize)


# Every degree and head dim, including the head-dim slices and separate dK/dV passes of the
# high-degree launches, and (float64 at d=128 from degree 4) the two operand tiles of a block
# taking turns in one LDS buffer.
@pytest.mark.parametrize("materialize", [1, 0])
@pytest.mark.parametrize("degree", [3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_every_degree_and_head_dim(dtype, d, degree, materialize):
    Q, K, V, G = (_series((2, 83, d), degree, 110 + i) for i in range(4))
    _compare(Q, K, V, G, dtype, causal=True, materialize=materialize)


@pytest.mark.parametrize("L,S", [(50, 96), (100, 32), (1, 64), (64, 1), (17, 130)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cross_lengths(dtype, L, S):
    degree = 3
    Q, G = _series((2, L, 32), degree, 120), _series((2, L, 32), degree, 121)
    K, V = _series((2, S, 32), degree, 122), _series((2, S, 32), degree, 123)
    for causal in (False, True):
        for materialize in ((1, 0) if dtype == torch.float32 else (0,)):
            _compare(Q, K, V, G, dtype, causal=causal, scale=0.3, materialize=materialize)


def test_rows_and_columns_without_admissible_pairs():
    # rows 3 and 40 see no key, keys 10 and 11 are seen by no query: zero gradient series there
    L, S, degree = 48, 40, 2
    mask = _window_mask(L, S, 5)
    mask[3] = False
    mask[40] = False
    mask[:, 10:12] = False
    Q, G = _series((2, L, 16), degree, 130), _series((2, L, 16), degree, 131)
    K, V = _series((2, S, 16), degree, 132), _series((2, S, 16), degree, 133)
    for dtype in (torch.float32, torch.float64):
        dq, dk, dv = _kernel(Q, K, V, G, dtype, mask=mask, materialize=int(dtype == torch.float32))
        for c in dq:
            assert torch.equal(c[:, [3, 40]].cpu(), torch.zeros_like(c[:, [3, 40]].cpu()))
        for c in dk + dv:
            assert torch.equal(c[:, 10:12].cpu(), torch.zeros_like(c[:, 10:12].cpu()))
        if dtype == torch.float32:
            _compare(Q, K, V, G, dtype, mask=mask, materialize=1)
        _compare(Q, K, V, G, dtype, mask=mask, materialize=0)


def test_empty_sequences():
    for dtype in (torch.float32, torch.float64):  # materialize=1 for float32 only (see FP64_MATERIALIZE)
        q = [torch.randn(2, 5, 32, dtype=dtype, device="cuda") for _ in range(3)]
        kv = [torch.empty(2, 0, 32, dtype=dtype, device="cuda") for _ in range(3)]
        out, lse = _ops.taylor_attention_fwd(q, kv, kv, None, False, 0.1, 2)
        for materialize in ((1, 0) if dtype == torch.float32 else (0,)):
            dq, dk, dv = _ops.taylor_attention_bwd(q, kv, kv, out, lse, q, None, False, 0.1, materialize)
            assert torch.equal(dq, torch.zeros_like(dq)) and dk.numel() == 0 and dv.numel() == 0
        # no queries: key and value gradients are zero
        qe = [torch.empty(2, 0, 32, dtype=dtype, device="cuda") for _ in range(3)]
        out, lse = _ops.taylor_attention_fwd(qe, q, q, None, False, 0.1, 2)
        for materialize in ((1, 0) if dtype == torch.float32 else (0,)):
            dq, dk, dv = _ops.taylor_attention_bwd(qe, q, q, out, lse, qe, None, False, 0.1, materialize)
            assert dq.numel() == 0 and torch.equal(dk, torch.zeros_like(dk)) and torch.equal(dv, torch.zeros_like(dv))


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("degree", [1, 4])
def test_autograd_through_sdpa(dtype, degree):
    # PolyTensor operands requiring grad: F.scaled_dot_product_attention records the series
    # attention, and torch.autograd.grad with a series cotangent runs the backward kernels.
    shape = (2, 3, 70, 32)
    Q, K, V, G = (_series(shape, degree, 140 + i) for i in range(4))
    mask = _window_mask(70, 70, 9)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        q, k, v = (PolyTensor(tuple(c.to(dtype).cuda() for c in s), requires_grad=True) for s in (Q, K, V))
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask.cuda())
        grad = PolyTensor(tuple(c.to(dtype).cuda() for c in G))
        dq, dk, dv = torch.autograd.grad(out, (q, k, v), grad)
    flat = [[c.reshape(6, *c.shape[-2:]) for c in s] for s in (Q, K, V, G)]
    want = _oracle(*flat, dtype, attn_mask=mask)
    for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert isinstance(got, PolyTensor) and got.degree == degree
        _check([c.reshape(6, *c.shape[-2:]) for c in got.coeffs], w, dtype, name)


def test_autograd_with_an_ordinary_key():
    # an ordinary key is a constant series (zero higher orders) and gets no gradient
    degree, shape = 3, (1, 2, 40, 16)
    Q, V, G = (_series(shape, degree, 150 + i) for i in range(3))
    key = torch.randn(shape, generator=torch.Generator().manual_seed(153), dtype=torch.float64)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        q, v = (PolyTensor(tuple(c.cuda() for c in s), requires_grad=True) for s in (Q, V))
        out = F.scaled_dot_product_attention(q, key.cuda(), v, is_causal=True)
        dq, dv = torch.autograd.grad(out, (q, v), PolyTensor(tuple(c.cuda() for c in G)))
    flat = [[c.reshape(2, *c.shape[-2:]) for c in s] for s in (Q, [key], V, G)]
    want = oracle.attention_backward(*flat, is_causal=True)
    _check([c.reshape(2, 40, 16) for c in dq.coeffs], want[0], torch.float64, "dq")
    _check([c.reshape(2, 40, 16) for c in dv.coeffs], want[2], torch.float64, "dv")


def test_float64_materialize_is_refused():
    q = [torch.randn(1, 16, 16, dtype=torch.float64, device="cuda") for _ in range(2)]
    out, lse = _ops.taylor_attention_fwd(q, q, q, None, True, 0.25, 1)
    with pytest.raises(Exception, match="not available for float64"):
        _ops.taylor_attention_bwd(q, q, q, out, lse, q, None, True, 0.25, 1)


def test_full_size_config3_backward():
    # benchmark config 3 shape (B=4 H=16 L=2048 d=128, K=4, fp32, causal) with line inputs and a
    # random cotangent series: one head against the oracle; on every head, linearity in the
    # cotangent (bwd(G1 + G2) = bwd(G1) + bwd(G2)), a size-independent property.
    B, H, L, d, degree = 4, 16, 2048, 128, 4
    gen = torch.Generator(device="cuda").manual_seed(3)

    def line():
        base = torch.randn(B * H, L, d, generator=gen, device="cuda") / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=gen, device="cuda")
        return [base, direction] + [torch.zeros_like(base) for _ in range(degree - 1)]

    def cot():
        return [torch.randn(B * H, L, d, generator=gen, device="cuda") * 0.5 ** k for k in range(degree + 1)]

    q, k, v = line(), line(), line()
    g1, g2 = cot(), cot()
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, None, True, scale, degree)
    r1 = _ops.taylor_attention_bwd(q, k, v, out, lse, g1, None, True, scale)
    head = 21
    want = oracle.attention_backward(*([c[head].cpu().double() for c in s] for s in (q, k, v, g1)), is_causal=True)
    for name, got, w in zip(("dq", "dk", "dv"), r1, want):
        _check([c[head] for c in got], w, torch.float32, name)
    r2 = _ops.taylor_attention_bwd(q, k, v, out, lse, g2, None, True, scale)
    r12 = _ops.taylor_attention_bwd(q, k, v, out, lse, [a + b for a, b in zip(g1, g2)], None, True, scale)
    for name, a, b, ab in zip(("dq", "dk", "dv"), r1, r2, r12):
        for o in range(degree + 1):
            err = rel_err((a[o] + b[o]).cpu(), ab[o].cpu())
            assert err <= TOL[torch.float32], f"{name} order {o}: linearity {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sliding_window_skips_blocks(dtype):
    # narrow window: whole key blocks (dQ) and query blocks (dK, dV) lie outside the mask ranges,
    # plus a query block with no admissible key and a key block that no query admits
    L, d, degree = 640, 32, 2
    mask = _window_mask(L, L, 50)
    mask[192:256] = False
    mask[:, 448:512] = False
    Q, K, V, G = (_series((2, L, d), degree, 160 + i) for i in range(4))
    if dtype == torch.float32:
        _compare(Q, K, V, G, dtype, mask=mask, materialize=1)
    _compare(Q, K, V, G, dtype, mask=mask, materialize=0)
