"""Cauchy-product matmul kernel vs the CPU oracle (GPU).

``a @ b`` on PolyTensors inside plain_range() runs C_k = sum_{i+j=k} A_i B_j in
one MFMA launch; the oracle forms the reference's (K+1)(K+2)/2 matmuls
(/root/reference/src/polytensors/_plain.py:118-128) in float64. Per-order
tolerance max|got - want| / max|want|: 1e-10 float64, 1e-4 float32 (fp32 MFMA,
no TF32 anywhere).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4}


def _series(shape, degree, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * 0.5 ** k).to(dtype) for k in range(degree + 1)]


def _poly(cs):
    return PolyTensor(tuple(c.cuda() for c in cs))


def _check(got, want, dtype):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.cpu(), b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e}"


@pytest.mark.parametrize("m,kd,n", [(64, 64, 64), (128, 256, 192), (100, 70, 90), (1, 33, 5), (257, 129, 65),
                                    (31, 3, 200), (64, 1, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("degree", [1, 4])
def test_matches_oracle(monkeypatch, m, kd, n, dtype, degree):
    calls = []
    original = _ops.cauchy_matmul
    monkeypatch.setattr(_ops, "cauchy_matmul", lambda *a, **k: calls.append(1) or original(*a, **k))
    A, B = _series((m, kd), degree, 1, dtype), _series((kd, n), degree, 2, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c = _poly(A) @ _poly(B)
    assert calls == [1] and c.shape == (m, n) and c.degree == degree
    _check(c.coeffs, oracle.matmul([a.double() for a in A], [b.double() for b in B]), dtype)


@pytest.mark.parametrize("degree", [0, 2, 3, 5, 6, 7, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_every_degree(degree, dtype):
    A, B = _series((96, 80), degree, 3, dtype), _series((80, 112), degree, 4, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c = torch.matmul(_poly(A), _poly(B))
    _check(c.coeffs, oracle.matmul([a.double() for a in A], [b.double() for b in B]), dtype)


@pytest.mark.parametrize("side", ["left", "right"])
def test_plain_operand_uses_one_order(side):
    degree, dtype = 4, torch.float32
    A, B = _series((70, 48), degree, 5, dtype), _series((48, 66), degree, 6, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        if side == "left":
            c = A[0].cuda() @ _poly(B)
            want = oracle.matmul([A[0].double()], [b.double() for b in B])
        else:
            c = _poly(A) @ B[0].cuda()
            want = oracle.matmul([a.double() for a in A], [B[0].double()])
    _check(c.coeffs, want, dtype)


def test_batched_and_broadcast():
    degree, dtype = 3, torch.float32
    A = _series((2, 3, 40, 24), degree, 7, dtype)
    B = _series((24, 56), degree, 8, dtype)
    Bb = _series((2, 3, 24, 56), degree, 9, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c1 = _poly(A) @ _poly(B)
        c2 = _poly(A) @ _poly(Bb)
        c3 = torch.bmm(_poly([a.reshape(6, 40, 24) for a in A]), _poly([b.reshape(6, 24, 56) for b in Bb]))
    _check(c1.coeffs, oracle.matmul([a.double() for a in A], [b.double() for b in B]), dtype)
    _check(c2.coeffs, oracle.matmul([a.double() for a in A], [b.double() for b in Bb]), dtype)
    _check([c.reshape(2, 3, 40, 56) for c in c3.coeffs], oracle.matmul([a.double() for a in A], [b.double() for b in Bb]),
           dtype)


@pytest.mark.parametrize("bias", [False, True])
def test_linear_uses_transposed_weight(bias):
    degree, dtype = 3, torch.float32
    X = _series((5, 7, 48), degree, 10, dtype)
    W = _series((40, 48), degree, 11, dtype)
    b = torch.randn(40, generator=torch.Generator().manual_seed(12)).to(dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.linear(_poly(X), _poly(W), b.cuda() if bias else None)
    want = oracle.matmul([x.double() for x in X], [w.double().t() for w in W])
    if bias:
        want = [want[0] + b.double()] + want[1:]
    _check(y.coeffs, want, dtype)


@pytest.mark.parametrize("plain_b", [False, True])
def test_matmul_by_transposed_view(plain_b):
    # x @ W.t() with W contiguous [n, k]: the kernel reads W in place (its transposed-B mode)
    degree, dtype = 2, torch.float32
    X = _series((3, 33, 48), degree, 15, dtype)
    W = _series((40, 48), 0 if plain_b else degree, 16, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        w = W[0].cuda().t() if plain_b else PolyTensor(tuple(c.cuda().t() for c in W))
        y = _poly(X) @ w
    want = oracle.matmul([x.double() for x in X], [c.double().t() for c in W])
    _check(y.coeffs, want, dtype)


def test_vector_operands():
    degree, dtype = 2, torch.float64
    A, v = _series((30, 20), degree, 13, dtype), _series((20,), degree, 14, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        c = _poly(A) @ _poly(v)
        d = _poly(v) @ _poly([a.t().contiguous() for a in A])
    _check(c.coeffs, oracle.matmul([a.double() for a in A], [x.double() for x in v]), dtype)
    _check(d.coeffs, oracle.matmul([x.double() for x in v], [a.double().t() for a in A]), dtype)


def test_known_answer_real_analog():
    # /root/reference/tests/test_dispatch.py:63-70 with real directions: a = (I, J), b = (2I, 2J), J = ones(2, 2)
    eye, ones = torch.eye(2, dtype=torch.float64), torch.ones(2, 2, dtype=torch.float64)
    a = PolyTensor((eye.cuda(), ones.cuda()), degree=2)
    b = PolyTensor(((2 * eye).cuda(), (2 * ones).cuda()), degree=2)
    with torch.no_grad(), PolyTensor.plain_range():
        c = a @ b
    assert torch.equal(c.coeffs[0].cpu(), 2 * eye)
    assert torch.equal(c.coeffs[1].cpu(), 4 * ones)
    assert torch.equal(c.coeffs[2].cpu(), 4 * ones)     # J @ 2J = 4J


def test_full_size_config_sampled_rows():
    # benchmark config 2: A, B [5, 4096, 4096] fp32, coefficient k scaled by 0.5^k. Rows of C are checked
    # on a seeded sample; the full product's linearity is checked through C(A + A') = C(A) + C(A').
    degree, n = 4, 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    A = [torch.randn(1, n, n, generator=g, device="cuda") * 0.5 ** k for k in range(degree + 1)]
    B = [torch.randn(1, n, n, generator=g, device="cuda") * 0.5 ** k for k in range(degree + 1)]
    C = _ops.cauchy_matmul(A, B, degree, False)
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(2))[:8]
    want = oracle.matmul([a[0][rows].cpu().double() for a in A], [b[0].cpu().double() for b in B])
    _check([c[0][rows.cuda()] for c in C], want, torch.float32)
    A2 = [a.flip(-1) for a in A]
    lhs = _ops.cauchy_matmul([x + y for x, y in zip(A, A2)], B, degree, False)
    rhs = C + _ops.cauchy_matmul(A2, B, degree, False)
    for k in range(degree + 1):
        assert rel_err(lhs[k].cpu(), rhs[k].cpu()) <= 1e-5
