"""Reverse mode through the series kernels (GPU).

For a series map y = f(x) the gradient series is the Taylor series of the
vector-Jacobian product along the curve, J(x(t))^T G(t)
(/root/reference/docs/api.md:148-153, /root/reference/src/polytensors/_fused_attention.py:18-22).
These tests run torch.autograd.grad / PolyTensor.backward through the
kernels inside plain_range() and retain_wrappers(), as the reference's
/root/reference/tests/test_fused_activation.py:10-26 does at degree 1, and
compare every order with the oracle's backward series, or with nested
forward-mode derivatives of torch.func.vjp / torch.func.grad along the curve
(tests/jets.py) in float64. Per-order tolerance max|got - want| / max|want|:
1e-10 float64, 1e-4 float32, 2e-2 bfloat16.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err, taylor

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2}
FUNCTIONS = {
    "gelu": F.gelu,
    "gelu_tanh": lambda x: F.gelu(x, approximate="tanh"),
    "tanh": torch.tanh,
    "sigmoid": torch.sigmoid,
    "silu": F.silu,
    "exp": torch.exp,
    "log": torch.log,
}


def _series(shape, degree, seed, scale=1.0, positive=False):
    g = torch.Generator().manual_seed(seed)
    cs = [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]
    if positive:
        cs[0] = cs[0].abs() + 0.5
    return cs


def _poly(cs, dtype, requires_grad=False):
    return PolyTensor(tuple(c.to(dtype).cuda() for c in cs), requires_grad=requires_grad)


def _check(got, want, dtype):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.detach().cpu(), b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e} > {TOL[dtype]:.0e}"


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("degree", [1, 3, 6])
@pytest.mark.parametrize("kind", sorted(FUNCTIONS))
def test_activation_value_and_gradient_series(kind, degree, dtype):
    X = _series((3, 1027), degree, seed=18, scale=1.5, positive=kind == "log")
    G = _series((3, 1027), degree, seed=19)
    X = [c.to(dtype).double() for c in X]   # the values the kernel sees
    G = [c.to(dtype).double() for c in G]
    x = _poly(X, dtype, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        y = FUNCTIONS[kind](x)
        (dx,) = torch.autograd.grad(y, x, _poly(G, dtype))
    assert isinstance(dx, PolyTensor) and dx.degree == degree and dx.dtype == dtype
    _check(y.coeffs, oracle.activation(X, kind), dtype)
    if kind == "exp":
        want = oracle.cauchy(G, oracle.activation(X, "exp"))
    elif kind == "log":
        want = oracle.quotient(G, X)
    else:
        saved = oracle.activation(X, kind) if kind in ("tanh", "sigmoid") else X
        want = oracle.activation_backward(G, saved, kind)
    _check(dx.coeffs, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("degree", [1, 4])
def test_matmul_gradient_series(degree, dtype):
    A = _series((48, 40), degree, seed=20)
    B = _series((40, 56), degree, seed=21)
    G = _series((48, 56), degree, seed=22)
    a, b = _poly(A, dtype, True), _poly(B, dtype, True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        c = a @ b
        da, db = torch.autograd.grad(c, (a, b), _poly(G, dtype))
    _check(c.coeffs, oracle.matmul(A, B), dtype)
    _check(da.coeffs, oracle.matmul(G, [m.T for m in B]), dtype)
    _check(db.coeffs, oracle.matmul([m.T for m in A], G), dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
def test_series_product_and_quotient(dtype):
    A = [c.to(dtype).double() for c in _series((5, 333), 4, seed=23)]
    B = [c.to(dtype).double() for c in _series((5, 333), 4, seed=24, positive=True)]
    with torch.no_grad(), PolyTensor.plain_range():
        prod = _poly(A, dtype) * _poly(B, dtype)
        quot = _poly(A, dtype) / _poly(B, dtype)
        recip = 1.0 / _poly(B, dtype)
    _check(prod.coeffs, oracle.cauchy(A, B), dtype)
    _check(quot.coeffs, oracle.quotient(A, B), dtype)
    ones = [torch.ones_like(B[0])] + [torch.zeros_like(b) for b in B[1:]]
    _check(recip.coeffs, oracle.quotient(ones, B), dtype)


def test_mlp_gradient_series_matches_jets_of_grad():
    # loss(x) = sum(gelu(x @ W1) @ W2 * c): PolyTensor.backward seeds (1, 0, ..., 0), and the gradient
    # series of x must equal the Taylor series of grad loss(x(t)) along the curve.
    degree = 4
    X = _series((6, 24), degree, seed=25)
    g = torch.Generator().manual_seed(26)
    W1 = torch.randn(24, 32, generator=g, dtype=torch.float64) / 5
    W2 = torch.randn(32, 8, generator=g, dtype=torch.float64) / 5
    cvec = torch.randn(6, 8, generator=g, dtype=torch.float64)

    def loss(x):
        return (F.gelu(x @ W1) @ W2 * cvec).sum()

    x = _poly(X, torch.float64, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = loss_gpu = (F.gelu(x @ W1.cuda()) @ W2.cuda() * cvec.cuda()).sum()
        out.backward()
        grad = x.grad
    _check(loss_gpu.coeffs, taylor(loss, [X], degree), torch.float64)
    _check(grad.coeffs, taylor(lambda z: torch.func.grad(loss)(z), [X], degree), torch.float64)


@pytest.mark.parametrize("n", [64, 4096, 999])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("degree", [1, 4, 8])
@pytest.mark.parametrize("layer", [False, True])
def test_norm_gradient_series(layer, degree, dtype, n):
    # RMSNorm / LayerNorm value and gradient series (register paths for n = 64, 4096; the
    # streaming path for n = 999), as /root/reference/tests/test_fused_norm.py:14-35 at degree K.
    X = [c.to(dtype).double() for c in _series((6, n), degree, seed=27, scale=2.0)]
    G = [c.to(dtype).double() for c in _series((6, n), degree, seed=28)]
    x = _poly(X, dtype, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        y = F.layer_norm(x, (n,), eps=1e-5) if layer else F.rms_norm(x, (n,), eps=1e-5)
        (dx,) = torch.autograd.grad(y, x, _poly(G, dtype))
    if layer:
        want_y, want_dx = oracle.layer_norm(X, (n,), eps=1e-5), oracle.layer_norm_backward(X, G, (n,), eps=1e-5)
    else:
        want_y, want_dx = oracle.rms_norm(X, (n,), eps=1e-5), oracle.rms_norm_backward(X, G, (n,), eps=1e-5)
    _check(y.coeffs, want_y, dtype)
    _check(dx.coeffs, want_dx, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_norm_with_series_weight_gradients(dtype):
    # The weight multiplies as a separate series product (as the reference's
    # /root/reference/src/polytensors/_fused_norm.py:69), so its gradient is sum_rows g (*) normalized.
    degree, n = 3, 256
    X = _series((8, n), degree, seed=29, scale=2.0)
    W = _series((n,), degree, seed=30)
    W[0] = W[0] + 1.0
    G = _series((8, n), degree, seed=31)
    x, w = _poly(X, dtype, True), _poly(W, dtype, True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        y = F.rms_norm(x, (n,), weight=w, eps=1e-6)
        dx, dw = torch.autograd.grad(y, (x, w), _poly(G, dtype))
    normalized = oracle.rms_norm(X, (n,), eps=1e-6)
    _check(y.coeffs, oracle.cauchy(normalized, W), dtype)
    _check(dx.coeffs, oracle.rms_norm_backward(X, oracle.cauchy(G, W), (n,), eps=1e-6), dtype)
    _check(dw.coeffs, [c.sum(0) for c in oracle.cauchy(G, normalized)], dtype)


@pytest.mark.parametrize("softcap,strided", [(None, False), (15.0, True)])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("degree", [1, 4])
def test_cross_entropy_gradient_series(degree, dtype, reduction, softcap, strided):
    # /root/reference/tests/test_fused_kernels.py:142-164,186-211 (ignored targets, all reductions,
    # softcap on a padded row slice) with value and gradient series at degree K.
    N, C, pad = 150, 3000, 64 if strided else 0
    full = [c.to(dtype).double() for c in _series((N, C + pad), degree, seed=32, scale=40.0 if softcap else 3.0)]
    g = torch.Generator().manual_seed(33)
    y = torch.randint(0, C, (N,), generator=g)
    y[::7] = -1
    logits = _poly(full, dtype, requires_grad=True)
    gshape = (N,) if reduction == "none" else ()
    Gs = [c.double() for c in _series(gshape, degree, seed=34)]
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        z = logits[:, :C] if strided else logits
        loss = PolyTensor.cross_entropy(z, y.cuda(), softcap=softcap, ignore_index=-1, reduction=reduction)
        (dz,) = torch.autograd.grad(loss, logits, _poly(Gs, acc))
    Z = [c[:, :C] for c in full]
    _check(loss.coeffs, oracle.cross_entropy(Z, y, ignore_index=-1, reduction=reduction, softcap=softcap), dtype)
    count = (y != -1).sum().double()
    rows = [c if reduction == "none" else (c / count if reduction == "mean" else c).expand(N) for c in Gs]
    want = oracle.cross_entropy_backward(Z, y, rows, ignore_index=-1, softcap=softcap)
    got = [c[:, :C] for c in dz.coeffs]
    if strided:
        assert all(float(c[:, C:].abs().max()) == 0 for c in dz.coeffs)
    _check(got, want, dtype)
