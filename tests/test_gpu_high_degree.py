"""Degrees above 8 and the elementwise functions sin, cos, sqrt, rsqrt, reciprocal (GPU).

The elementwise kernels (activation series, series product and quotient) run up
to degree 16, and the Cauchy matmul runs above its kernel's degree 8 in blocks of
orders. The checks:
* the reference's closed forms along a line x + t v at degrees 1, 3, 12 (and 16)
  with real and complex directions (/root/reference/tests/test_series.py:15-46:
  exp, log, reciprocal, rsqrt, sin, cos; sqrt by the same binomial series),
  rtol 2e-13 elementwise for real directions as there, and the contract's
  per-order 1e-10 for complex directions (evaluated at real nodes and recombined);
* the reference's round trips (/root/reference/tests/test_series.py:93-109):
  exp(log x), 1/(1/x), sqrt(x)^2 and rsqrt(x)^2 x on a dense degree-5 series;
* dense random series at degrees 9, 12 and 16 for every activation against the
  oracle's restatements (pinned by jets at lower degrees) and, for sin, cos,
  sqrt and rsqrt, against the oracle's exp and log series (exp(i x), exp(log(x)/2)),
  1e-10 in float64;
* series product and quotient at degree 16 and the matmul at degrees 9..16
  against the oracle's Cauchy sums (1e-10 float64, 1e-4 float32, 2e-2 bfloat16);
* gradients of the new functions: reverse mode through sin/cos/sqrt/rsqrt
  against jets of torch.func.grad, and their second-order coefficient autograd;
* above degree 8 the norms, cross entropy and attention are composed from series operations
  (the reference's decompositions); at degree 12 they match the oracle's restatements at
  1e-10 in float64, and degree 17 is refused.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor
from tests.jets import rel_err, taylor

pytestmark = pytest.mark.gpu

OPS = ("exp", "log", "reciprocal", "rsqrt", "sqrt", "sin", "cos")


def _line(base, direction, degree):
    return PolyTensor((base.cuda(), direction.cuda()), degree=degree)


def _closed_form(operation, base, direction, order):
    if operation == "exp":
        return torch.exp(base) * direction ** order / math.factorial(order)
    if operation == "log":
        return ((-1) ** (order - 1) / order) * (direction / base) ** order
    if operation == "reciprocal":
        return torch.reciprocal(base) * (-direction / base) ** order
    if operation in ("rsqrt", "sqrt"):
        p = -0.5 if operation == "rsqrt" else 0.5
        binomial = math.prod((p - i) / (i + 1) for i in range(order))
        return binomial * base ** p * (direction / base) ** order
    derivative = ((torch.sin(base), torch.cos(base), -torch.sin(base), -torch.cos(base)) if operation == "sin" else
                  (torch.cos(base), -torch.sin(base), -torch.cos(base), torch.sin(base)))[order % 4]
    return derivative * direction ** order / math.factorial(order)


@pytest.mark.parametrize("degree", (1, 3, 12, 16))
@pytest.mark.parametrize("complex_direction", (False, True))
@pytest.mark.parametrize("operation", OPS)
def test_line_coefficients_match_analytic_derivatives(operation, complex_direction, degree):
    base = torch.tensor([1.7, 0.6, 2.9], dtype=torch.float64)
    direction = torch.tensor([0.2 + 0.3j, -0.1 + 0.05j, 0.3 - 0.2j] if complex_direction else [0.2, -0.1, 0.3],
                             dtype=torch.complex128 if complex_direction else torch.float64)
    with torch.no_grad(), PolyTensor.plain_range():
        result = getattr(torch, operation)(_line(base, direction, degree))
    assert result.degree == degree
    torch.testing.assert_close(result.coeffs[0].cpu(), getattr(torch, operation)(base), rtol=1e-15, atol=0)
    for order in range(1, degree + 1):
        want = _closed_form(operation, base, direction, order)
        if complex_direction:
            # complex directions run as K+1 real evaluations recombined by Lagrange weights, whose
            # rounding grows with the order: the contract's per-order bound for complex128 up to
            # degree 12; above, the interpolation's amplification (up to 1e-9 elementwise at
            # degree 16) is bounded at 1e-8
            bound = 1e-10 if degree <= 12 else 1e-8
            assert rel_err(result.coeffs[order].cpu(), want) <= bound, f"order {order}"
        else:
            torch.testing.assert_close(result.coeffs[order].cpu(), want, rtol=2e-13, atol=1e-28)


@pytest.mark.parametrize("degree", (1, 3, 12))
@pytest.mark.parametrize("operation", ("exp", "log", "rsqrt", "sqrt", "sin", "cos"))
def test_complex_base_line_coefficients_match_analytic_derivatives(operation, degree):
    # a complex constant term (the reference's complex arithmetic, docs/notes.md:74-77): the same
    # closed forms with complex base and direction (principal branches, as torch's)
    base = torch.tensor([1.7 + 0.4j, 0.6 - 1.1j, -2.9 + 0.8j], dtype=torch.complex128)
    direction = torch.tensor([0.2 + 0.3j, -0.1 + 0.05j, 0.3 - 0.2j], dtype=torch.complex128)
    with torch.no_grad(), PolyTensor.plain_range():
        result = getattr(torch, operation)(_line(base, direction, degree))
    assert result.degree == degree
    want0 = getattr(torch, operation)(base)
    assert rel_err(result.coeffs[0].cpu(), want0) <= 1e-14
    for order in range(1, degree + 1):
        assert rel_err(result.coeffs[order].cpu(), _closed_form(operation, base, direction, order)) <= 1e-10, \
            f"order {order}"


@pytest.mark.parametrize("kind", ("tanh", "sigmoid", "silu", "gelu_tanh"))
def test_complex_base_activations_match_jets(kind):
    degree = 6
    g = torch.Generator().manual_seed(960)
    X = [torch.complex(torch.randn(4, 5, generator=g, dtype=torch.float64),
                       torch.randn(4, 5, generator=g, dtype=torch.float64)) * 0.5 ** k for k in range(degree + 1)]
    c, a = math.sqrt(2.0 / math.pi), 0.044715
    plain = {"tanh": torch.tanh, "sigmoid": torch.sigmoid, "silu": lambda z: z * torch.sigmoid(z),
             "gelu_tanh": lambda z: 0.5 * z * (1 + torch.tanh(c * (z + a * z ** 3)))}[kind]
    series = {"tanh": torch.tanh, "sigmoid": torch.sigmoid, "silu": F.silu,
              "gelu_tanh": lambda z: F.gelu(z, approximate="tanh")}[kind]
    with torch.no_grad(), PolyTensor.plain_range():
        out = series(PolyTensor(tuple(x.cuda() for x in X)))
    want = taylor(plain, [X], degree)
    for k in range(degree + 1):
        assert rel_err(out.coeffs[k].cpu(), want[k]) <= 1e-10, f"{kind} order {k}"


def test_nonlinear_input_series_round_trips():
    coefficients = tuple(torch.tensor([v, v / 2], dtype=torch.float64)
                         for v in (1.5, 0.2, -0.1, 0.03, 0.0, -0.002))
    value = PolyTensor(tuple(c.cuda() for c in coefficients))
    with torch.no_grad(), PolyTensor.plain_range():
        results = (torch.exp(torch.log(value)), torch.reciprocal(torch.reciprocal(value)), torch.sqrt(value).square())
        identity = torch.rsqrt(value).square() * value
    for result in results:
        for actual, expected in zip(result.coeffs, coefficients):
            torch.testing.assert_close(actual.cpu(), expected, rtol=2e-13, atol=1e-15)
    for order, actual in enumerate(identity.coeffs):
        expected = torch.ones(2, dtype=torch.float64) if order == 0 else torch.zeros(2, dtype=torch.float64)
        torch.testing.assert_close(actual.cpu(), expected, rtol=2e-13, atol=1e-15)


_FNS = {"gelu": F.gelu, "gelu_tanh": lambda x: F.gelu(x, approximate="tanh"), "tanh": torch.tanh,
        "sigmoid": torch.sigmoid, "silu": F.silu, "exp": torch.exp, "log": torch.log, "sin": torch.sin,
        "cos": torch.cos, "sqrt": torch.sqrt, "rsqrt": torch.rsqrt}


def _dense(shape, degree, seed, positive=False, scale=0.5):
    g = torch.Generator().manual_seed(seed)
    cs = [torch.randn(shape, generator=g, dtype=torch.float64) * scale ** k for k in range(degree + 1)]
    if positive:
        cs[0] = cs[0].abs() + 1.0
    return cs


@pytest.mark.parametrize("degree", (9, 12, 16))
@pytest.mark.parametrize("kind", ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu", "exp", "log"))
def test_dense_series_above_degree_eight_match_the_oracle(kind, degree):
    # the oracle's restatements of the reference's rules (pinned against jets at lower degrees in
    # tests/test_oracle_activation_pins.py) hold at any degree
    X = _dense((3, 41), degree, 700 + degree, positive=kind == "log")
    with torch.no_grad(), PolyTensor.plain_range():
        out = _FNS[kind](PolyTensor(tuple(c.cuda() for c in X)))
    want = oracle.activation(X, kind)
    for k in range(degree + 1):
        assert rel_err(out.coeffs[k].cpu(), want[k]) <= 1e-10, f"{kind} order {k}"


def _exp_of(series):
    return oracle.exp_series(series)


@pytest.mark.parametrize("degree", (9, 12, 16))
def test_dense_sin_cos_sqrt_rsqrt_above_degree_eight(degree):
    # independent routes through the oracle's exp and log series: cos x + i sin x = exp(i x),
    # sqrt x = exp(log(x) / 2), rsqrt x = exp(-log(x) / 2)
    X = _dense((3, 41), degree, 760 + degree)
    P = _dense((3, 41), degree, 761 + degree, positive=True)
    with torch.no_grad(), PolyTensor.plain_range():
        x, p = (PolyTensor(tuple(c.cuda() for c in s)) for s in (X, P))
        got = {"sin": torch.sin(x), "cos": torch.cos(x), "sqrt": torch.sqrt(p), "rsqrt": torch.rsqrt(p)}
    e = _exp_of([c * 1j for c in X])
    logs = oracle.log_series(P)
    want = {"sin": [c.imag for c in e], "cos": [c.real for c in e],
            "sqrt": _exp_of([c * 0.5 for c in logs]), "rsqrt": _exp_of([c * -0.5 for c in logs])}
    for kind in got:
        for k in range(degree + 1):
            assert rel_err(got[kind].coeffs[k].cpu(), want[kind][k]) <= 1e-10, f"{kind} order {k}"


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-4)])
def test_series_product_and_quotient_at_degree_sixteen(dtype, tol):
    degree = 16
    A = _dense((5, 37), degree, 710)
    B = _dense((5, 37), degree, 711, positive=True)
    a, b = (PolyTensor(tuple(c.to(dtype).cuda() for c in s)) for s in (A, B))
    up = lambda s: [c.to(dtype).double() for c in s]   # noqa: E731
    with torch.no_grad(), PolyTensor.plain_range():
        for got, want, what in ((a * b, oracle.cauchy(up(A), up(B)), "a * b"),
                                (a / b, oracle.quotient(up(A), up(B)), "a / b")):
            for k in range(degree + 1):
                assert rel_err(got.coeffs[k].cpu(), want[k]) <= tol, f"{what} order {k}"


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("degree", (9, 12, 16))
def test_matmul_above_the_kernel_degree(dtype, tol, degree):
    A = _dense((2, 33, 40), degree, 720 + degree)
    B = _dense((40, 24), degree, 721 + degree)
    W = _dense((24, 40), 0, 722)[0]
    up = lambda s: [c.to(dtype).double() for c in s]   # noqa: E731
    a, b = (PolyTensor(tuple(c.to(dtype).cuda() for c in s)) for s in (A, B))
    with torch.no_grad(), PolyTensor.plain_range():
        cases = ((a @ b, oracle.matmul(up(A), up(B)), "series @ series"),
                 (a @ B[0].to(dtype).cuda(), oracle.matmul(up(A), up(B[:1])), "series @ plain"),
                 (F.linear(a, W.to(dtype).cuda()), oracle.matmul(up(A), [W.t().to(dtype).double()]), "linear"))
        for got, want, what in cases:
            for k in range(degree + 1):
                assert rel_err(got.coeffs[k].cpu(), want[k]) <= tol, f"{what} order {k}"


def test_matmul_above_the_kernel_degree_with_complex_directions():
    degree = 10
    A = _dense((20, 16), degree, 730)
    Ai = _dense((20, 16), degree, 731)
    B = _dense((16, 12), degree, 732)
    Ac = [A[0]] + [torch.complex(x, y) for x, y in zip(A[1:], Ai[1:])]
    with torch.no_grad(), PolyTensor.plain_range():
        got = PolyTensor(tuple(c.cuda() for c in Ac)) @ PolyTensor(tuple(c.cuda() for c in B))
    want = oracle.matmul(Ac, [c.to(torch.complex128) for c in B])
    for k in range(degree + 1):
        assert rel_err(got.coeffs[k].cpu(), want[k]) <= 1e-10, f"order {k}"


@pytest.mark.parametrize("kind", ("sin", "cos", "sqrt", "rsqrt"))
def test_reverse_mode_through_the_new_functions(kind):
    degree = 4
    X = _dense((3, 5), degree, 740, positive=kind in ("sqrt", "rsqrt"))
    R = torch.randn(3, 5, generator=torch.Generator().manual_seed(741), dtype=torch.float64)

    def loss(x):
        return (_FNS[kind](x) * R).sum()

    x = PolyTensor(tuple(c.cuda() for c in X), requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = (_FNS[kind](x) * R.cuda()).sum()
        out.backward()
    want = taylor(lambda z: torch.func.grad(loss)(z), [X], degree)
    for k in range(degree + 1):
        assert rel_err(x.grad.coeffs[k].cpu(), want[k]) <= 1e-10, f"{kind} gradient order {k}"


@pytest.mark.parametrize("kind", ("sin", "cos", "sqrt", "rsqrt"))
def test_second_order_coefficient_autograd_of_the_new_functions(kind):
    degree = 3
    X = _dense((4,), degree, 750, positive=kind in ("sqrt", "rsqrt"))
    fn = _FNS[kind]

    def explicit(xs):   # coefficient `degree` of fn(x(t)), by nested jvp in t (plain torch)
        return taylor(fn, [xs], degree)[degree].sum()

    leaves = [c.clone().requires_grad_() for c in X]
    first = torch.autograd.grad(explicit(leaves), leaves[0], create_graph=True)[0]
    want = torch.autograd.grad((first * first).sum(), leaves[0])[0]
    cl = [c.cuda().requires_grad_() for c in X]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        out = fn(PolyTensor(tuple(cl))).sum()
    first = torch.autograd.grad(out.coeffs[degree], cl[0], create_graph=True)[0]
    got = torch.autograd.grad((first * first).sum(), cl[0])[0]
    assert rel_err(got.cpu(), want) <= 1e-10


def _poly(coeffs):
    return PolyTensor(tuple(c.cuda() for c in coeffs))


def _check(out, want, what):
    got = out.coeffs if isinstance(out, PolyTensor) else (out,)
    assert len(got) == len(want), what
    for k, (g, w) in enumerate(zip(got, want)):
        assert rel_err(g.cpu(), w) <= 1e-10, f"{what}: order {k}"


def test_norms_compose_above_degree_eight():
    degree = 12
    X = _dense((6, 40), degree, 901)
    W, B = _dense((40,), degree, 902), _dense((40,), degree, 903)
    W[0] = W[0] + 2.0
    with torch.no_grad(), PolyTensor.plain_range():
        rms = F.rms_norm(_poly(X), (40,), _poly(W), eps=1e-6)
        layer = F.layer_norm(_poly(X), (40,), _poly(W), _poly(B), eps=1e-5)
        plain_w = F.rms_norm(_poly(X), (40,), W[0].cuda())
    assert rms.degree == layer.degree == degree
    _check(rms, oracle.rms_norm(X, (40,), W, eps=1e-6), "rms_norm")
    _check(layer, oracle.layer_norm(X, (40,), W, B, eps=1e-5), "layer_norm")
    _check(plain_w, oracle.rms_norm(X, (40,), [W[0]]), "rms_norm, ordinary weight")


@pytest.mark.parametrize("layer", (False, True))
def test_reverse_mode_through_the_composed_norms(layer):
    # the composed norm is recorded by autograd as its series operations; the gradient series for
    # the cotangent (R, 0, ..., 0) of a plain-weighted sum is the oracle's
    degree = 10
    X = _dense((5, 24), degree, 930)
    R = torch.randn(5, 24, generator=torch.Generator().manual_seed(931), dtype=torch.float64)
    x = PolyTensor(tuple(c.cuda() for c in X), requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = F.layer_norm(x, (24,), eps=1e-5) if layer else F.rms_norm(x, (24,), eps=1e-6)
        (out * R.cuda()).sum().backward()
    G = [R] + [torch.zeros_like(R) for _ in range(degree)]
    want = (oracle.layer_norm_backward(X, G, (24,), eps=1e-5) if layer else
            oracle.rms_norm_backward(X, G, (24,), eps=1e-6))
    _check(x.grad, want, "layer_norm gradient" if layer else "rms_norm gradient")


@pytest.mark.parametrize("mask", ("causal", "bool", "float"))
def test_attention_composes_above_degree_eight(mask):
    degree = 12
    Q, K, V = (_dense((2, 3, 24, 16), degree, 910 + i, scale=0.3) for i in range(3))
    g = torch.Generator().manual_seed(915)
    attn_mask, causal = None, mask == "causal"
    if mask == "bool":
        attn_mask = torch.rand(24, 24, generator=g) < 0.7
        attn_mask |= torch.eye(24, dtype=torch.bool)   # every row keeps a key
    elif mask == "float":
        attn_mask = torch.randn(2, 1, 24, 24, generator=g, dtype=torch.float64)
    with torch.no_grad(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(_poly(Q), _poly(K), _poly(V), is_causal=causal,
                                             attn_mask=None if attn_mask is None else attn_mask.cuda())
    assert out.degree == degree
    _check(out, oracle.attention(Q, K, V, attn_mask=attn_mask, is_causal=causal), f"attention, {mask}")


@pytest.mark.parametrize("case", ("mean", "none_ignored", "weighted_smoothed", "softcap"))
def test_cross_entropy_composes_above_degree_eight(case):
    degree = 12
    Z = _dense((7, 33), degree, 920)
    g = torch.Generator().manual_seed(921)
    target = torch.randint(0, 33, (7,), generator=g)
    kwargs, want_kwargs = {}, {}
    if case == "none_ignored":
        target[2] = -100
        kwargs = want_kwargs = {"reduction": "none"}
    elif case == "weighted_smoothed":
        target[4] = -100
        weight = torch.rand(33, generator=g, dtype=torch.float64) + 0.5
        kwargs = {"weight": weight.cuda(), "label_smoothing": 0.1}
        want_kwargs = {"weight": weight, "label_smoothing": 0.1}
    with torch.no_grad(), PolyTensor.plain_range():
        if case == "softcap":
            out = PolyTensor.cross_entropy(_poly(Z), target.cuda(), softcap=5.0)
            want = oracle.cross_entropy(Z, target, softcap=5.0)
        else:
            out = F.cross_entropy(_poly(Z), target.cuda(), **kwargs)
            want = oracle.cross_entropy(Z, target, **want_kwargs)
    assert out.degree == degree
    _check(out, want, f"cross_entropy, {case}")


def test_row_and_mfma_operations_refuse_degree_seventeen():
    x = PolyTensor(tuple(torch.randn(4, 16, dtype=torch.float64, device="cuda") for _ in range(18)))
    q = PolyTensor(tuple(torch.randn(1, 1, 8, 16, dtype=torch.float64, device="cuda") for _ in range(18)))
    y = torch.zeros(4, dtype=torch.int64, device="cuda")
    with torch.no_grad(), PolyTensor.plain_range():
        for call in (lambda: F.layer_norm(x, (16,)), lambda: F.rms_norm(x, (16,)),
                     lambda: F.cross_entropy(x, y), lambda: F.scaled_dot_product_attention(q, q, q)):
            with pytest.raises(NotImplementedError, match="exceeds"):
                call()
