"""Coefficient autograd through the fused kernels (GPU).

Inside ``PolyTensor.coefficient_autograd()`` the coefficient tensors are
ordinary autograd leaves and every fused operation records a graph on them
(/root/reference/src/polytensors/_tensor.py:291-323). The expected gradients
come from ordinary autograd through the CPU oracle in float64: the oracle is
the reference's plain-range rules restated in plain torch operations, so
differentiating it gives the exact coefficient Jacobians. Every input order
is a leaf and the loss weights every output order, so all Jacobian blocks
dy_k / dx_j (j <= k) are exercised. Mirrors the reference's
test_fused_kernels.py:75-93 (attention against wrapper autograd),
test_fused_norm.py:55 and test_fused_activation.py:29 (gradients of an order-1
coefficient against autograd of a jvp). Tolerance: relative 1e-12 in float64,
1e-4 in float32.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor
from tests.jets import rel_err

pytestmark = pytest.mark.gpu


def _leaves(shape, degree, seed, dtype=torch.float64, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k).to(dtype)
            for k in range(degree + 1)]


def _weights(degree, seed):
    g = torch.Generator().manual_seed(1000 + seed)
    return torch.randn(degree + 1, generator=g, dtype=torch.float64)


def _loss(coeffs, w, probe):
    """sum_k w_k <probe_k, y_k>: every output order contributes."""
    return sum(w[k] * (c * p).sum() for k, (c, p) in enumerate(zip(coeffs, probe)))


def _probes(like, seed):
    g = torch.Generator().manual_seed(2000 + seed)
    return [torch.randn(c.shape, generator=g, dtype=torch.float64) for c in like]


def _compare(device_fn, cpu_fn, inputs, seed, tol=1e-12):
    """Gradients of the weighted loss w.r.t. every input coefficient: fused (GPU) vs oracle (CPU)."""
    degree = len(inputs[0]) - 1
    w = _weights(degree, seed)
    gpu_leaves = [[c.cuda().requires_grad_() for c in s] for s in inputs]
    cpu_leaves = [[c.double().clone().requires_grad_() for c in s] for s in inputs]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        out = device_fn(*(PolyTensor(tuple(s), requires_grad=False) for s in gpu_leaves))
    want_out = cpu_fn(*cpu_leaves)
    probe = _probes(want_out, seed)
    got_loss = _loss([c.double() for c in out.coeffs], w.cuda(), [p.cuda() for p in probe])
    want_loss = _loss(want_out, w, probe)
    got = torch.autograd.grad(got_loss, [c for s in gpu_leaves for c in s], allow_unused=True)
    want = torch.autograd.grad(want_loss, [c for s in cpu_leaves for c in s], allow_unused=True)
    for i, (a, b) in enumerate(zip(got, want)):
        if b is None:
            assert a is None or a.abs().max() == 0, i
            continue
        assert a is not None, f"no gradient for input coefficient {i}"
        err = rel_err(a.cpu(), b)
        assert err <= tol, f"input coefficient {i}: {err:.3e}"
    return out


@pytest.mark.parametrize("degree", [1, 3])
@pytest.mark.parametrize("mode", ["causal", "window", "none"])
def test_attention(degree, mode):
    shape = (1, 2, 40, 32)
    inputs = [_leaves(shape, degree, 10 + i, scale=0.5) for i in range(3)]
    i = torch.arange(40)
    mask = (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] <= 9) if mode == "window" else None
    kwargs = dict(is_causal=mode == "causal")

    def dev(q, k, v):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=None if mask is None else mask.cuda(), **kwargs)

    def cpu(q, k, v):
        return oracle.attention(q, k, v, attn_mask=mask, **kwargs)

    _compare(dev, cpu, inputs, seed=degree)


def test_attention_matches_wrapper_autograd_like_the_reference():
    # /root/reference/tests/test_fused_kernels.py:75-93: the gradient of sum(out_1) w.r.t. the order-0
    # coefficients equals order 1 of the wrapper gradient series for G = (1, 0).
    shape = (1, 2, 96, 32)
    coefficients = [[c.cuda().requires_grad_() for c in _leaves(shape, 1, 20 + i, scale=0.5)] for i in range(3)]
    q, k, v = (PolyTensor(tuple(c), requires_grad=False) for c in coefficients)
    with PolyTensor.coefficient_autograd(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    first = torch.autograd.grad(out.coeffs[1].sum(), [c[0] for c in coefficients])
    q2, k2, v2 = (PolyTensor(tuple(x.detach() for x in c), requires_grad=True) for c in coefficients)
    with PolyTensor.retain_wrappers(), PolyTensor.plain_range():
        out2 = F.scaled_dot_product_attention(q2, k2, v2, is_causal=True)
        out2.backward(PolyTensor.constant(torch.ones_like(out2.value), 1))
    for x, g in zip((q2, k2, v2), first):
        assert rel_err(g.cpu(), x.grad.coeffs[1].cpu()) < 1e-12
    assert rel_err(out.coeffs[1].cpu(), out2.coeffs[1].cpu()) < 1e-12


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("affine", ["none", "plain", "series"])
def test_norms(layer, affine):
    degree, shape, n = 3, (6, 48), 48
    x = _leaves(shape, degree, 30)
    g = torch.Generator().manual_seed(31)
    inputs = [x]
    if affine == "plain":
        inputs.append([1 + 0.1 * torch.randn(n, generator=g, dtype=torch.float64)])
    elif affine == "series":
        inputs.append([(1 if k == 0 else 0.1) * torch.randn(n, generator=g, dtype=torch.float64)
                       for k in range(degree + 1)])
    if layer and affine != "none":
        inputs.append([0.1 * torch.randn(n, generator=g, dtype=torch.float64) for _ in inputs[-1]])

    def dev(*xs):
        w = None if affine == "none" else (xs[1] if affine == "series" else xs[1].coeffs[0])
        if layer:
            b = None if affine == "none" else (xs[2] if affine == "series" else xs[2].coeffs[0])
            return F.layer_norm(xs[0], (n,), w, b, eps=1e-5)
        return F.rms_norm(xs[0], (n,), w, eps=1e-5)

    def cpu(*xs):
        w = None if affine == "none" else xs[1]
        if layer:
            return oracle.layer_norm(xs[0], (n,), weight=w, bias=None if affine == "none" else xs[2], eps=1e-5)
        return oracle.rms_norm(xs[0], (n,), weight=w, eps=1e-5)

    if affine == "plain":   # an ordinary weight/bias leaf: one coefficient
        _compare_plain(dev, cpu, inputs, seed=32 + layer)
    else:
        _compare(dev, cpu, inputs, seed=32 + layer)


def _compare_plain(device_fn, cpu_fn, inputs, seed):
    """_compare for operands given as one-coefficient lists (ordinary tensors on the device side)."""
    degree = len(inputs[0]) - 1
    w = _weights(degree, seed)
    gpu = [[c.cuda().requires_grad_() for c in s] for s in inputs]
    cpu = [[c.double().clone().requires_grad_() for c in s] for s in inputs]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        wrapped = [PolyTensor(tuple(gpu[0]), requires_grad=False)] + [
            PolyTensor((s[0],), degree=degree, requires_grad=False) for s in gpu[1:]]
        out = device_fn(*wrapped)
    want_out = cpu_fn(*cpu)
    probe = _probes(want_out, seed)
    got = torch.autograd.grad(_loss([c.double() for c in out.coeffs], w.cuda(), [p.cuda() for p in probe]),
                              [c for s in gpu for c in s])
    want = torch.autograd.grad(_loss(want_out, w, probe), [c for s in cpu for c in s])
    for i, (a, b) in enumerate(zip(got, want)):
        assert rel_err(a.cpu(), b) <= 1e-12, f"input coefficient {i}"


def test_rms_norm_like_the_reference():
    # /root/reference/tests/test_fused_norm.py:55-62 pattern: gradients of y_1 w.r.t. (x0, x1) against
    # autograd of the jvp of the ordinary function
    x0 = torch.randn(2, 4, device="cuda", dtype=torch.float64, requires_grad=True)
    x1 = torch.randn_like(x0, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        y = F.rms_norm(PolyTensor((x0, x1)), (4,), eps=0.1)
        actual = torch.autograd.grad(y.coeffs[1].sum(), (x0, x1))
    _, expected_y = torch.func.jvp(lambda x: F.rms_norm(x, (4,), eps=0.1), (x0,), (x1,))
    expected = torch.autograd.grad(expected_y.sum(), (x0, x1))
    for a, b in zip(actual, expected):
        assert rel_err(a.cpu(), b.cpu()) <= 1e-12


@pytest.mark.parametrize("kind", ["gelu", "gelu_tanh", "tanh", "sigmoid", "silu", "exp", "log"])
def test_activations(kind):
    degree = 3
    x = _leaves((5, 37), degree, 40)
    if kind == "log":
        x[0] = x[0].abs() + 0.5
    fn = {"gelu": F.gelu, "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"), "tanh": torch.tanh,
          "sigmoid": torch.sigmoid, "silu": F.silu, "exp": torch.exp, "log": torch.log}[kind]
    _compare(fn, lambda xs: oracle.activation(xs, kind), [x], seed=41)


@pytest.mark.parametrize("function", [F.gelu, torch.tanh, torch.sigmoid])
def test_activation_like_the_reference(function):
    # /root/reference/tests/test_fused_activation.py:29-38
    x0 = torch.randn(2, 3, device="cuda", dtype=torch.float64, requires_grad=True)
    x1 = torch.randn_like(x0, requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        y = function(PolyTensor((x0, x1)))
        actual = torch.autograd.grad(y.coeffs[1].sum(), (x0, x1))
    _, expected_y = torch.func.jvp(function, (x0,), (x1,))
    expected = torch.autograd.grad(expected_y.sum(), (x0, x1))
    for a, b in zip(actual, expected):
        assert rel_err(a.cpu(), b.cpu()) <= 1e-12


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_cross_entropy(reduction):
    degree = 3
    z = _leaves((20, 50), degree, 50, scale=2.0)
    y = torch.randint(0, 50, (20,), generator=torch.Generator().manual_seed(51))
    y[::4] = -100

    def dev(logits):
        return F.cross_entropy(logits, y.cuda(), reduction=reduction)

    def cpu(zs):
        return oracle.cross_entropy(zs, y, reduction=reduction)

    _compare(dev, cpu, [z], seed=52)


@pytest.mark.parametrize("case", ["series@series", "series@plain", "linear", "batched"])
def test_matmul(case):
    degree = 3
    if case == "series@series":
        inputs = [_leaves((7, 9), degree, 60), _leaves((9, 5), degree, 61)]
        _compare(lambda a, b: a @ b, lambda a, b: oracle.matmul(a, b), inputs, seed=62)
    elif case == "batched":
        inputs = [_leaves((3, 7, 9), degree, 63), _leaves((9, 5), degree, 64)]
        _compare(lambda a, b: torch.matmul(a, b), lambda a, b: oracle.matmul(a, b), inputs, seed=65)
    elif case == "series@plain":
        inputs = [_leaves((7, 9), degree, 66), [torch.randn(9, 5, dtype=torch.float64)]]
        _compare_plain(lambda a, b: a @ b.coeffs[0], lambda a, b: oracle.matmul(a, b), inputs, seed=67)
    else:
        g = torch.Generator().manual_seed(68)
        inputs = [_leaves((2, 4, 9), degree, 69), [torch.randn(5, 9, generator=g, dtype=torch.float64)],
                  [torch.randn(5, generator=g, dtype=torch.float64)]]

        def dev(x, w, b):
            return F.linear(x, w.coeffs[0], b.coeffs[0])

        def cpu(x, w, b):
            out = oracle.matmul(x, [w[0].transpose(0, 1)])
            return [out[0] + b[0]] + out[1:]

        _compare_plain(dev, cpu, inputs, seed=70)


@pytest.mark.parametrize("op", ["mul", "div"])
def test_series_product_and_quotient(op):
    degree = 3
    a = _leaves((4, 11), degree, 80)
    b = _leaves((4, 11), degree, 81)
    b[0] = b[0].abs() + 1.0
    if op == "mul":
        _compare(lambda x, y: x * y, lambda x, y: oracle.cauchy(x, y), [a, b], seed=82)
    else:
        _compare(lambda x, y: x / y, lambda x, y: oracle.quotient(x, y), [a, b], seed=83)


def test_float32_attention_and_cross_entropy_pipeline():
    # a small float32 model: attention -> linear -> cross entropy, every coefficient a leaf
    degree = 2
    shape = (1, 1, 32, 16)
    qkv = [_leaves(shape, degree, 90 + i, dtype=torch.float32, scale=0.5) for i in range(3)]
    W = torch.randn(16, 10, generator=torch.Generator().manual_seed(93), dtype=torch.float64).float()
    y = torch.randint(0, 10, (32,), generator=torch.Generator().manual_seed(94))

    def dev(q, k, v):
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return F.cross_entropy(out.reshape(32, 16) @ W.cuda(), y.cuda())

    def cpu(q, k, v):
        out = oracle.attention(q, k, v, is_causal=True)
        logits = oracle.matmul([o.reshape(32, 16) for o in out], [W.double()])
        return oracle.cross_entropy(logits, y)

    _compare(dev, cpu, qkv, seed=95, tol=1e-4)
