"""Differentiating through updates, and reverse mode with complex directions (GPU).

The first five cases restate the reference's training examples
(/root/reference/tests/test_training.py:33-160) on the HIP device: forward mode
through plain SGD on a PolyTensor parameter (real and complex directions),
an input direction with a closed form, and coefficient autograd (real and
complex directions). Their expected coefficients come from PyTorch's own
reverse AD of ordinary functional SGD on the CPU (the higher derivatives of
the updated weight with respect to its initial value, times v^k / k!), which
shares no code with the series rules.

The remaining cases take complex directions through the fused kernels in reverse
mode: the gradient series of LayerNorm -> GELU -> linear -> cross entropy and of
causal attention, by PolyTensor.backward and by coefficient autograd, against the
Taylor series of torch.func.grad of the same composite along x + t (u + i w)
(tests/jets.py:taylor_complex, polarized nested jvp; reference semantics
/root/reference/docs/api.md:69-92), at 1e-10 in complex128. Then second-order
coefficient autograd ("further reverse derivatives remain supported",
/root/reference/docs/api.md:137-139): through the Cauchy matmul and the series
product against reverse AD of the explicit coefficient sums, and through the norms,
cross entropy, attention and tanh/sigmoid/silu/gelu/gelu_tanh against reverse AD
of plain-torch jets (tests/jets.py:taylor), at 1e-10 in float64.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from polytensors_amd import PolyTensor
from tests.jets import rel_err, taylor, taylor_complex

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _sgd_coefficients(initial, direction, degree, steps=2, rate=0.1):
    """Coefficients of w_steps(initial + t direction) for SGD on (w - 1)^4 / 4, by reverse AD."""
    start = initial.detach().double().requires_grad_()
    w = start
    for _ in range(steps):
        g = torch.autograd.grad((w - 1).pow(4) / 4, w, create_graph=True)[0]
        w = w - rate * g
    out = [w.detach()]
    deriv = w
    for k in range(1, degree + 1):
        deriv = torch.autograd.grad(deriv, start, create_graph=True)[0]
        out.append(deriv.detach() * direction.pow(k) / math.factorial(k))
    return out


def _close(actual, expected, dtype):
    tol = 1e-10 if dtype in (torch.float64, torch.complex128) else 1e-5
    a = actual.detach().cpu().to(torch.complex128)
    b = expected.detach().cpu().to(torch.complex128)
    assert (a - b).abs().max().item() <= tol * max(1.0, b.abs().max().item()), (a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_forward_through_sgd_matches_independent_higher_derivatives(dtype):
    initial, direction, degree = torch.tensor(0.5, dtype=dtype), torch.tensor(0.3, dtype=dtype), 4
    weight = PolyTensor((initial.to(DEV), direction.to(DEV)), degree=degree, requires_grad=True)
    opt = torch.optim.SGD([weight], lr=0.1, foreach=False)
    with PolyTensor.plain_range():
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            with PolyTensor.retain_wrappers():
                loss = (weight - 1).pow(4) / 4
                torch.autograd.backward(loss, torch.ones_like(loss))
                assert isinstance(weight.grad, PolyTensor)
                opt.step()
    expected = _sgd_coefficients(initial, direction.double(), degree)
    for got, want in zip(weight.coeffs, expected):
        _close(got, want, dtype)


def test_forward_through_sgd_with_real_base_and_complex_direction():
    initial = torch.tensor(0.5, dtype=torch.float64)
    direction = torch.tensor(0.3 + 0.2j, dtype=torch.complex128)
    degree = 4
    weight = PolyTensor((initial.to(DEV), direction.to(DEV)), degree=degree, requires_grad=True)
    opt = torch.optim.SGD([weight], lr=0.1, foreach=False)
    with PolyTensor.plain_range():
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            with PolyTensor.retain_wrappers():
                loss = (weight - 1).pow(4) / 4
                torch.autograd.backward(loss, torch.ones_like(loss))
                opt.step()
    expected = _sgd_coefficients(initial, direction, degree)
    assert all(c.is_complex() for c in weight.coeffs[1:])
    for got, want in zip(weight.coeffs, expected):
        _close(got, want, torch.complex128)


def test_training_input_direction_matches_closed_form_quadratic():
    initial, value, direction = (torch.tensor(x, dtype=torch.float64) for x in (0.2, 1.0, 0.4))
    target = PolyTensor((value.to(DEV), direction.to(DEV)), degree=3)
    weight = PolyTensor((initial.to(DEV),), degree=3, requires_grad=True)
    opt = torch.optim.SGD([weight], lr=0.1, foreach=False)
    with PolyTensor.plain_range():
        for _ in range(3):
            opt.zero_grad(set_to_none=True)
            with PolyTensor.retain_wrappers():
                loss = (weight - target).square() / 2
                torch.autograd.backward(loss, torch.ones_like(loss))
                opt.step()
    decay = 0.9 ** 3
    _close(weight.coeffs[0], decay * initial + (1 - decay) * value, torch.float64)
    _close(weight.coeffs[1], (1 - decay) * direction, torch.float64)
    for c in weight.coeffs[2:]:
        _close(c, torch.zeros(()), torch.float64)


@pytest.mark.parametrize("complex_direction", [False, True])
def test_coefficient_autograd_training_matches_independent_higher_derivatives(complex_direction):
    initial = torch.tensor(0.5, dtype=torch.float64)
    direction = torch.tensor(0.3 + 0.2j if complex_direction else 0.3,
                             dtype=torch.complex128 if complex_direction else torch.float64)
    degree = 4
    coeffs = (initial.to(DEV), direction.to(DEV)) + tuple(torch.zeros_like(direction).to(DEV)
                                                         for _ in range(degree - 1))
    with PolyTensor.plain_range():
        for _ in range(2):
            coeffs = tuple(c.detach().requires_grad_() for c in coeffs)
            weight = PolyTensor(coeffs)
            with PolyTensor.coefficient_autograd():
                loss = (weight - 1).pow(4) / 4
            assert not loss.requires_grad
            grads = []
            for c in loss.coeffs:
                g = torch.autograd.grad(c.real, coeffs[0], retain_graph=True)[0]
                if c.is_complex():
                    g = torch.complex(g, torch.autograd.grad(c.imag, coeffs[0], retain_graph=True)[0])
                grads.append(g)
            coeffs = tuple(c - 0.1 * g for c, g in zip(coeffs, grads))
    expected = _sgd_coefficients(initial, direction, degree)
    for got, want in zip(coeffs, expected):
        _close(got, want, torch.complex128)


def test_coefficient_autograd_treats_taylor_coefficients_as_independent_inputs():
    values = (0.2, -0.3, 0.4, 0.1)
    coeffs = tuple(torch.tensor(v, dtype=torch.float64, device=DEV, requires_grad=True) for v in values)
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        result = torch.exp(PolyTensor(coeffs))
    b, c1, c2, c3 = (torch.tensor(v, dtype=torch.float64) for v in values)
    expected = (b.exp(), b.exp() * c1, b.exp() * (c2 + c1 ** 2 / 2), b.exp() * (c3 + c1 * c2 + c1 ** 3 / 6))
    for got, want in zip(result.coeffs, expected):
        _close(got, want, torch.float64)


# ---------------------------------------------------------------------------
# Complex directions through the fused kernels in reverse mode

def _layer_norm(x, eps=1e-5):
    # written out: torch's native layer_norm has wrong nested forward-mode derivatives of order >= 2
    mu = x.mean(-1, keepdim=True)
    c = x - mu
    return c * torch.rsqrt((c * c).mean(-1, keepdim=True) + eps)


def _mlp_case(seed=0):
    g = torch.Generator().manual_seed(seed)
    x0 = torch.randn(6, 32, generator=g, dtype=torch.float64)
    u, w = (torch.randn(6, 32, generator=g, dtype=torch.float64) * 0.5 for _ in range(2))
    W = torch.randn(32, 11, generator=g, dtype=torch.float64) / 6
    y = torch.randint(0, 11, (6,), generator=g)
    return x0, u, w, W, y


@pytest.mark.parametrize("degree", [1, 3])
def test_complex_direction_gradient_series_through_norm_gelu_linear_cross_entropy(degree):
    x0, u, w, W, y = _mlp_case()

    def loss(x):
        return F.cross_entropy(F.gelu(_layer_norm(x)) @ W, y)

    x = PolyTensor((x0.to(DEV), torch.complex(u, w).to(DEV)), degree=degree, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = F.cross_entropy(F.gelu(F.layer_norm(x, (32,))) @ W.to(DEV), y.to(DEV))
        out.backward()
    want_loss = taylor_complex(loss, [x0], [u], [w], degree)
    want_grad = taylor_complex(lambda z: torch.func.grad(loss)(z), [x0], [u], [w], degree)
    for k in range(degree + 1):
        assert rel_err(out.coeffs[k].cpu(), want_loss[k]) <= 1e-10, f"loss order {k}"
        assert rel_err(x.grad.coeffs[k].cpu(), want_grad[k]) <= 1e-10, f"gradient order {k}"


def _attention_case(seed=1):
    g = torch.Generator().manual_seed(seed)
    shape = (1, 2, 40, 16)
    bases = [torch.randn(shape, generator=g, dtype=torch.float64) / 2 for _ in range(3)]
    reals = [torch.randn(shape, generator=g, dtype=torch.float64) / 2 for _ in range(3)]
    imags = [torch.randn(shape, generator=g, dtype=torch.float64) / 2 for _ in range(3)]
    R = torch.randn(shape, generator=g, dtype=torch.float64)
    return bases, reals, imags, R


def _math_attention(q, k, v):
    s = (q / 4) @ k.transpose(-2, -1)
    keep = torch.ones(s.shape[-2:], dtype=torch.bool).tril()
    return torch.softmax(s.masked_fill(~keep, float("-inf")), -1) @ v


@pytest.mark.parametrize("degree", [2, 3])
def test_complex_direction_gradient_series_through_attention(degree):
    bases, reals, imags, R = _attention_case()

    def loss(q, k, v):
        return (_math_attention(q, k, v) * R).sum()

    q, k, v = (PolyTensor((b.to(DEV), torch.complex(r, i).to(DEV)), degree=degree, requires_grad=True)
               for b, r, i in zip(bases, reals, imags))
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = (F.scaled_dot_product_attention(q, k, v, is_causal=True) * R.to(DEV)).sum()
        out.backward()
    for which, x in enumerate((q, k, v)):
        want = taylor_complex(lambda *t, j=which: torch.func.grad(loss, argnums=j)(*t), bases, reals, imags, degree)
        for order in range(degree + 1):
            assert rel_err(x.grad.coeffs[order].cpu(), want[order]) <= 1e-10, f"{'qkv'[which]} order {order}"


def test_complex_direction_coefficient_autograd_through_fused_ops():
    # coefficient autograd: d(loss_k)/d(x_0) is coefficient k of the gradient series; for a
    # complex loss coefficient its real and imaginary parts are differentiated separately
    degree = 3
    x0, u, w, W, y = _mlp_case(seed=2)

    def loss(x):
        return F.cross_entropy(F.gelu(_layer_norm(x)) @ W, y)

    base = x0.to(DEV).requires_grad_()
    direction = torch.complex(u, w).to(DEV).requires_grad_()
    rest = [torch.zeros_like(direction) for _ in range(degree - 1)]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        out = F.cross_entropy(F.gelu(F.layer_norm(PolyTensor((base, direction, *rest)), (32,))) @ W.to(DEV),
                              y.to(DEV))
    want = taylor_complex(lambda z: torch.func.grad(loss)(z), [x0], [u], [w], degree)
    for k, c in enumerate(out.coeffs):
        g = torch.autograd.grad(c.real, base, retain_graph=True)[0]
        if c.is_complex():
            g = torch.complex(g, torch.autograd.grad(c.imag, base, retain_graph=True)[0])
        assert rel_err(g.cpu(), want[k]) <= 1e-10, f"order {k}"


# ---------------------------------------------------------------------------
# Second-order coefficient autograd (matmul, series product)

def test_second_order_coefficient_autograd_through_matmul_and_product():
    degree = 3
    g = torch.Generator().manual_seed(3)
    A = [torch.randn(5, 7, generator=g, dtype=torch.float64) * 0.5 ** k for k in range(degree + 1)]
    B = torch.randn(7, 4, generator=g, dtype=torch.float64)
    R = torch.randn(5, 4, generator=g, dtype=torch.float64)

    def explicit(a):   # coefficient `degree` of sum((A @ B) (*) (A @ B) (*) R), plain torch
        c = [x @ B for x in a]
        return sum((c[i] * c[degree - i] * R).sum() for i in range(degree + 1))

    # d loss_3 / d A_1 = 2 (A_2 B o R) B^T depends on A_2: differentiate its square by A_2
    leaves = [x.clone().requires_grad_() for x in A]
    first = torch.autograd.grad(explicit(leaves), leaves[1], create_graph=True)[0]
    want = torch.autograd.grad((first * first).sum(), leaves[2])[0]

    cl = [x.to(DEV).requires_grad_() for x in A]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        c = PolyTensor(tuple(cl)) @ B.to(DEV)
        out = (c * c * R.to(DEV)).sum()
    first = torch.autograd.grad(out.coeffs[degree], cl[1], create_graph=True)[0]
    got = torch.autograd.grad((first * first).sum(), cl[2])[0]
    assert rel_err(got.cpu(), want) <= 1e-10


def _second_order(fn, series_fn, X, degree, wrt=(0, 0)):
    """d/dX_b of |d coefficient_degree / dX_a|^2 (a, b = wrt): plain-torch jets of ``fn`` on the CPU
    against coefficient autograd through ``series_fn`` on a PolyTensor of X."""
    a, b = wrt

    def explicit(xs):
        return taylor(fn, [xs], degree)[degree].sum()

    leaves = [c.clone().requires_grad_() for c in X]
    first = torch.autograd.grad(explicit(leaves), leaves[a], create_graph=True)[0]
    want = torch.autograd.grad((first * first).sum(), leaves[b])[0]
    cl = [c.to(DEV).requires_grad_() for c in X]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        out = series_fn(PolyTensor(tuple(cl)))
    first = torch.autograd.grad(out.coeffs[degree].sum(), cl[a], create_graph=True)[0]
    got = torch.autograd.grad((first * first).sum(), cl[b])[0]
    assert rel_err(got.cpu(), want) <= 1e-10


def test_second_order_coefficient_autograd_through_the_quotient():
    # the quotient's backward reads its saved output, which must keep its graph: saved as a view
    # made in the autograd setup, it entered a second derivative as a constant
    degree = 2
    X = _series_input((3, 6), degree, 37)
    R = torch.randn(3, 6, generator=torch.Generator().manual_seed(38), dtype=torch.float64)

    def f(x, r):
        e = x.exp()
        return e / e.sum(-1, keepdim=True) * r

    _second_order(lambda x: f(x, R), lambda x: f(x, R.to(DEV)), X, degree)
    _second_order(lambda x: 1.0 / (x * x + 1.0) * R, lambda x: 1.0 / (x * x + 1.0) * R.to(DEV), X, degree)


def _series_input(shape, degree, seed, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale ** k for k in range(degree + 1)]


@pytest.mark.parametrize("layer", (False, True))
def test_second_order_coefficient_autograd_through_the_norms(layer):
    # the fused kernel's gradient is a kernel without its own derivative; asked for a graph of it,
    # the norm is recomposed from series operations and differentiated. The CPU side is the
    # norms' definition in plain operations (torch's nested jvp of native_layer_norm gives a
    # wrong second coefficient: the sum of a layer norm's outputs came out -1.84, not 0), weighted
    # by R (a layer norm's plain sum vanishes)
    degree = 2
    X = _series_input((3, 8), degree, 31)
    R = torch.randn(3, 8, generator=torch.Generator().manual_seed(36), dtype=torch.float64)

    def plain(x):
        if layer:
            x = x - x.mean(-1, keepdim=True)
            return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-5) * R
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * R

    def series(x):
        y = F.layer_norm(x, (8,), eps=1e-5) if layer else F.rms_norm(x, (8,), eps=1e-6)
        return y * R.to(DEV)

    _second_order(plain, series, X, degree)
    _second_order(plain, series, X, degree, wrt=(1, 0))


def test_second_order_coefficient_autograd_through_cross_entropy():
    degree = 2
    Z = _series_input((5, 7), degree, 32)
    y = torch.tensor([0, 3, 6, 2, 3])
    _second_order(lambda z: F.cross_entropy(z, y), lambda z: F.cross_entropy(z, y.to(DEV)), Z, degree)


@pytest.mark.parametrize("causal", (False, True))
def test_second_order_coefficient_autograd_through_attention(causal):
    degree = 2
    Q = _series_input((1, 2, 6, 16), degree, 33)
    g = torch.Generator().manual_seed(34)
    Kp, Vp = (torch.randn(1, 2, 6, 16, generator=g, dtype=torch.float64) for _ in range(2))
    keep = torch.ones(6, 6, dtype=torch.bool).tril() if causal else torch.ones(6, 6, dtype=torch.bool)

    def plain(q):   # (torch's CPU attention has no forward AD: its definition in plain operations)
        s = (q @ Kp.transpose(-2, -1)) / math.sqrt(16)
        return torch.softmax(s.masked_fill(~keep, float("-inf")), -1) @ Vp

    _second_order(plain, lambda q: F.scaled_dot_product_attention(q, Kp.to(DEV), Vp.to(DEV), is_causal=causal),
                  Q, degree)


@pytest.mark.parametrize("kind", ("tanh", "sigmoid", "silu", "gelu", "gelu_tanh"))
def test_second_order_coefficient_autograd_through_activations(kind):
    degree = 3
    X = _series_input((4, 5), degree, 35)
    fn = {"tanh": torch.tanh, "sigmoid": torch.sigmoid, "silu": F.silu, "gelu": F.gelu,
          "gelu_tanh": lambda x: F.gelu(x, approximate="tanh")}[kind]
    _second_order(fn, fn, X, degree)
    _second_order(fn, fn, X, degree, wrt=(2, 1))
