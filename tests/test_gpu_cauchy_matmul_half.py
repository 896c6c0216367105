"""Cauchy-product matmul with bfloat16 / float16 series (GPU).

The 16-bit kernel takes the operands as stored into 16x16x32 MFMAs, accumulates
every product of an order in fp32 and rounds each element of C_k to the storage
type once. The oracle forms the reference's (K+1)(K+2)/2 matmuls
(/root/reference/src/polytensors/_plain.py:118-128) in float64 on the same
stored inputs. Per-order tolerance max|got - want| / max|want|: one rounding of
the result is at most 2^-9 (bfloat16) / 2^-12 (float16) of it; the bound is
twice that, and far inside the north star's bf16 tier of 2e-2 (the
reference's own half-type tests use 2e-2, /root/reference/tests/test_fused_kernels.py:64-72).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

HALF = [torch.bfloat16, torch.float16]
TOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def _series(shape, degree, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * 0.5 ** k).to(dtype) for k in range(degree + 1)]


def _poly(cs):
    return PolyTensor(tuple(c.cuda() for c in cs))


def _up(cs):
    return [c.double() for c in cs]


def _check(got, want, dtype, tol=None):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        assert a.dtype == dtype
        err = rel_err(a.cpu(), b)
        assert err <= (tol or TOL[dtype]), f"order {k}: {err:.3e}"


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("m,kd,n", [(64, 64, 64), (128, 256, 192), (100, 72, 88), (1, 32, 8),
                                    (70, 37, 29), (257, 129, 65), (31, 3, 200), (64, 1, 64)])
@pytest.mark.parametrize("degree", [1, 4])
def test_matches_oracle(monkeypatch, dtype, m, kd, n, degree):
    # ragged contraction / column counts are zero-padded to multiples of 8 on the way in
    calls = []
    original = _ops.cauchy_matmul
    monkeypatch.setattr(_ops, "cauchy_matmul", lambda *a, **k: calls.append(1) or original(*a, **k))
    A, B = _series((m, kd), degree, 1, dtype), _series((kd, n), degree, 2, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c = _poly(A) @ _poly(B)
    assert calls == [1] and c.shape == (m, n) and c.degree == degree and c.dtype == dtype
    _check(c.coeffs, oracle.matmul(_up(A), _up(B)), dtype)


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("degree", [0, 2, 3, 5, 6, 7, 8])
@pytest.mark.parametrize("trans_b", [False, True])
def test_every_degree_both_layouts(dtype, degree, trans_b):
    A = _series((96, 80), degree, 3, dtype)
    B = _series((112, 80) if trans_b else (80, 112), degree, 4, dtype)
    flat = lambda cs: [c.unsqueeze(0).cuda() for c in cs]
    C = _ops.cauchy_matmul(flat(A), flat(B), degree, trans_b)
    want = oracle.matmul(_up(A), [b.t() for b in _up(B)] if trans_b else _up(B))
    _check([c[0] for c in C], want, dtype)


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("degree", [0, 1, 2, 4])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("orders", ["both", "left", "right"])
@pytest.mark.parametrize("m,kd,n", [(256, 64, 256), (300, 136, 264), (520, 40, 392)])
def test_wide_tile_ragged_edges(dtype, degree, trans_b, orders, m, kd, n):
    # outputs of at least 256 x 256 at degree <= 4 run the 128 x 128 workgroup tile; these shapes
    # leave partial tiles on both output sides and a partial last contraction chunk
    A = _series((m, kd), degree if orders != "right" else 0, 7, dtype)
    B = _series((n, kd) if trans_b else (kd, n), degree if orders != "left" else 0, 8, dtype)
    flat = lambda cs: [c.unsqueeze(0).cuda() for c in cs]
    C = _ops.cauchy_matmul(flat(A), flat(B), degree, trans_b)
    want = oracle.matmul(_up(A), [b.t() for b in _up(B)] if trans_b else _up(B))
    want += [torch.zeros_like(want[0])] * (degree + 1 - len(want))
    _check([c[0] for c in C], want, dtype)


@pytest.mark.parametrize("dtype", HALF)
@pytest.mark.parametrize("side", ["left", "right"])
def test_plain_operand_uses_one_order(dtype, side):
    degree = 4
    A, B = _series((70, 48), degree, 5, dtype), _series((48, 66), degree, 6, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        if side == "left":
            c = A[0].cuda() @ _poly(B)
            want = oracle.matmul(_up(A[:1]), _up(B))
        else:
            c = _poly(A) @ B[0].cuda()
            want = oracle.matmul(_up(A), _up(B[:1]))
    _check(c.coeffs, want, dtype)


@pytest.mark.parametrize("dtype", HALF)
def test_two_ordinary_operands(dtype):
    # C_0 = A B and the higher orders zero
    degree = 3
    A, B = _series((40, 32), 0, 5, dtype), _series((32, 24), 0, 6, dtype)
    C = _ops.cauchy_matmul([A[0].cuda()[None]], [B[0].cuda()[None]], degree, False)
    _check([C[0][0]], oracle.matmul(_up(A), _up(B)), dtype)
    assert all(torch.count_nonzero(C[k]) == 0 for k in range(1, degree + 1))


@pytest.mark.parametrize("dtype", HALF)
def test_batched_broadcast_and_linear(dtype):
    degree = 3
    A = _series((2, 3, 40, 24), degree, 7, dtype)
    B = _series((24, 56), degree, 8, dtype)
    Bb = _series((2, 3, 24, 56), degree, 9, dtype)
    W = _series((40, 24), degree, 10, dtype)
    bias = torch.randn(40, generator=torch.Generator().manual_seed(11)).to(dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c1 = _poly(A) @ _poly(B)
        c2 = _poly(A) @ _poly(Bb)
        y = F.linear(_poly(A), _poly(W), bias.cuda())
    _check(c1.coeffs, oracle.matmul(_up(A), _up(B)), dtype)
    _check(c2.coeffs, oracle.matmul(_up(A), _up(Bb)), dtype)
    want = oracle.matmul(_up(A), [w.t() for w in _up(W)])
    want = [want[0] + bias.double()] + want[1:]
    # the bias is added in the storage type after the product (a second rounding)
    _check(y.coeffs, want, dtype, tol=2 * TOL[dtype])


@pytest.mark.parametrize("dtype", HALF)
def test_gradient_series(dtype):
    degree = 3
    A, B, G = _series((48, 40), degree, 20, dtype), _series((40, 56), degree, 21, dtype), \
        _series((48, 56), degree, 22, dtype)
    a = PolyTensor(tuple(c.cuda() for c in A), requires_grad=True)
    b = PolyTensor(tuple(c.cuda() for c in B), requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        c = a @ b
        da, db = torch.autograd.grad(c, (a, b), _poly(G))
    # contraction over 56 (dA) and 48 (dB): the backward's own products of the same kernel
    _check(da.coeffs, oracle.matmul(_up(G), [m.T for m in _up(B)]), dtype)
    _check(db.coeffs, oracle.matmul([m.T for m in _up(A)], _up(G)), dtype)


@pytest.mark.parametrize("dtype", HALF)
def test_offset_views_are_realigned(dtype):
    # operands at a storage offset that is not 16-byte aligned are copied before the DMA
    degree = 2
    big = [x.cuda() for x in _series((40 * 24 + 3,), degree, 30, dtype)]
    A = [x[3:].view(40, 24) for x in big]
    assert all(a.data_ptr() % 16 != 0 for a in A)
    B = _series((24, 16), degree, 31, dtype)
    C = _ops.cauchy_matmul([a[None] for a in A], [b.cuda()[None] for b in B], degree, False)
    _check([c[0] for c in C], oracle.matmul([a.cpu().double() for a in A], _up(B)), dtype)


@pytest.mark.parametrize("dtype", HALF)
def test_full_size_config2_sampled_rows(dtype):
    # benchmark config 2's shape (A, B [5, 4096, 4096], coefficient k scaled by 0.5^k) in 16-bit storage:
    # sampled rows against the oracle, and linearity in A over the whole product
    degree, n = 4, 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    A = [(torch.randn(1, n, n, generator=g, device="cuda") * 0.5 ** k).to(dtype) for k in range(degree + 1)]
    B = [(torch.randn(1, n, n, generator=g, device="cuda") * 0.5 ** k).to(dtype) for k in range(degree + 1)]
    C = _ops.cauchy_matmul(A, B, degree, False)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(2))[:4]
    want = oracle.matmul([a[0][rows].cpu().double() for a in A], [b[0].cpu().double() for b in B])
    _check([c[0][rows.cuda()] for c in C], want, dtype)
    A2 = [a.flip(-1) for a in A]
    lhs = _ops.cauchy_matmul([(x.double() + y.double()).to(dtype) for x, y in zip(A, A2)], B, degree, False)
    rhs = [c.double() + d.double() for c, d in zip(C, _ops.cauchy_matmul(A2, B, degree, False))]
    # A + A' is rounded to the storage type before the product; three output roundings
    for k in range(degree + 1):
        assert rel_err(lhs[k].double().cpu(), rhs[k].cpu()) <= 8 * TOL[dtype]
