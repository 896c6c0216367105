"""Complex directions (GPU): real constant term, complex higher coefficients.

The reference extends the derivatives of the real computation multilinearly to
complex directions (/root/reference/docs/notes.md:59-76). polytensors_amd
computes them with its real kernels, either by evaluating at K+1 real nodes and
interpolating at i, or by splitting bilinear products into real and imaginary
parts (polytensors_amd/_complex.py). The oracle instead runs the reference's
recurrences in complex arithmetic (complex128 on upcast inputs), so agreement
pins both. Every fused operation is covered, plus the config-5 GPT decoder
(bench.gpt_forward) at reduced size, at full width, and at full size through
properties. Per-order tolerance max|got - want| / max|want|: 1e-10 complex128,
1e-4 complex64.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor
import bench
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4}


def _series(shape, degree, seed, scale=1.0, positive=False):
    """Real order 0, complex orders 1..degree (float64 / complex128 on the CPU)."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(shape, generator=g, dtype=torch.float64) * scale
    if positive:
        base = base.abs() + 0.5
    rest = [torch.complex(torch.randn(shape, generator=g, dtype=torch.float64),
                          torch.randn(shape, generator=g, dtype=torch.float64)) * scale * 0.5 ** k
            for k in range(1, degree + 1)]
    return [base] + rest


def _cast(cs, dtype):
    cdt = {torch.float32: torch.complex64, torch.float64: torch.complex128}[dtype]
    return [c.to(cdt if c.is_complex() else dtype) for c in cs]


def _poly(cs, dtype):
    return PolyTensor(tuple(c.cuda() for c in _cast(cs, dtype)))


def _up(cs, dtype):
    return [c.to(torch.complex128 if c.is_complex() else torch.float64) for c in _cast(cs, dtype)]


def _check(got, want, dtype):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        a = a.detach().cpu()
        assert (a.is_complex() or k == 0), f"order {k} lost its imaginary part"
        err = rel_err(a, b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e} > {TOL[dtype]:.0e}"


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("numel", [1, 6, 4099])
def test_plane_kernels_round_trip(dtype, numel):
    # real variants at every node, recombined with the interpolation weights, give back the complex
    # planes (the identity map is a polynomial of degree 1 in lam); a real/imaginary split likewise
    from polytensors_amd import _complex, _ops

    cdt = torch.complex64 if dtype == torch.float32 else torch.complex128
    planes = [torch.randn(numel, dtype=cdt, device="cuda") for _ in range(3)]
    nodes, weights = _complex.nodes_and_weights(3)
    var = _ops.complex_to_real(planes, [1.0] * 4, list(nodes))
    for v, lam in enumerate(nodes):
        for o in range(3):
            want = planes[o].real + lam * planes[o].imag
            assert torch.allclose(var[v, o], want, rtol=1e-6 if dtype == torch.float32 else 1e-14, atol=1e-6)
    back = _ops.real_to_complex([p for v in var.unbind(0) for p in v.unbind(0)], 3,
                                [w.real for w in weights], [w.imag for w in weights])
    for o in range(3):
        assert (back[o] - planes[o]).abs().max() <= (1e-5 if dtype == torch.float32 else 1e-13)
    split = _ops.complex_to_real(planes, [1.0, 0.0], [0.0, 1.0])
    assert torch.equal(split[0, 1], planes[1].real) and torch.equal(split[1, 2], planes[2].imag)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("both", [False, True])
def test_matmul_and_linear(dtype, both):
    degree = 3
    A = _series((3, 40, 24), degree, 1)
    B = _series((24, 33), degree, 2) if both else [torch.randn(24, 33, dtype=torch.float64)]
    bias = torch.randn(33, dtype=torch.float64)
    with torch.no_grad(), PolyTensor.plain_range():
        a = _poly(A, dtype)
        b = _poly(B, dtype) if both else B[0].to(dtype).cuda()
        got = a @ b
        lin = F.linear(a, b.transpose(0, 1) if not both else b.transpose(0, 1).contiguous(), bias.to(dtype).cuda())
    want = oracle.matmul(_up(A, dtype), _up(B, dtype))
    _check(got.coeffs, want, dtype)
    want_lin = [want[0] + bias.to(dtype).double()] + want[1:]
    _check(lin.coeffs, want_lin, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_series_product_and_quotient(dtype):
    degree = 4
    A = _series((5, 37), degree, 3)
    B = _series((5, 37), degree, 4, positive=True)
    R = [torch.randn(5, 37, dtype=torch.float64)] + [torch.randn(5, 37, dtype=torch.float64) for _ in range(degree)]
    with torch.no_grad(), PolyTensor.plain_range():
        a, b = _poly(A, dtype), _poly(B, dtype)
        r = PolyTensor(tuple(c.to(dtype).cuda() for c in R))
        prod, quot, mixed = a * b, a / b, a * r
    _check(prod.coeffs, oracle.cauchy(_up(A, dtype), _up(B, dtype)), dtype)
    _check(quot.coeffs, oracle.quotient(_up(A, dtype), _up(B, dtype)), dtype)
    _check(mixed.coeffs, oracle.cauchy(_up(A, dtype), [c.to(dtype).double() for c in R]), dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kind", ["gelu", "gelu_tanh", "tanh", "sigmoid", "silu", "exp", "log"])
def test_activations(kind, dtype):
    degree = 3
    X = _series((4, 257), degree, 5, positive=kind == "log")
    fn = {"gelu": F.gelu, "gelu_tanh": lambda x: F.gelu(x, approximate="tanh"), "tanh": torch.tanh,
          "sigmoid": torch.sigmoid, "silu": F.silu, "exp": torch.exp, "log": torch.log}[kind]
    with torch.no_grad(), PolyTensor.plain_range():
        got = fn(_poly(X, dtype))
    _check(got.coeffs, oracle.activation(_up(X, dtype), kind), dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("layer", [False, True])
def test_norms(layer, dtype):
    degree = 3
    X = _series((6, 96), degree, 6)
    w = 1 + 0.1 * torch.randn(96, dtype=torch.float64)
    b = 0.1 * torch.randn(96, dtype=torch.float64)
    with torch.no_grad(), PolyTensor.plain_range():
        x = _poly(X, dtype)
        if layer:
            got = F.layer_norm(x, (96,), w.to(dtype).cuda(), b.to(dtype).cuda())
        else:
            got = F.rms_norm(x, (96,), w.to(dtype).cuda(), eps=1e-6)
    wd, bd = [w.to(dtype).double()], [b.to(dtype).double()]
    want = (oracle.layer_norm(_up(X, dtype), (96,), weight=wd, bias=bd) if layer
            else oracle.rms_norm(_up(X, dtype), (96,), weight=wd, eps=1e-6))
    _check(got.coeffs, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("masking", ["causal", "window"])
def test_attention(dtype, masking):
    degree, L, d = 3, 70, 32
    Q, K, V = (_series((2, 2, L, d), degree, 7 + i, scale=0.5) for i in range(3))
    i = torch.arange(L)
    window = (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] <= 20)
    kw = dict(is_causal=True) if masking == "causal" else dict(attn_mask=window)
    with torch.no_grad(), PolyTensor.plain_range():
        got = F.scaled_dot_product_attention(
            _poly(Q, dtype), _poly(K, dtype), _poly(V, dtype),
            **({k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}))
    _check(got.coeffs, oracle.attention(_up(Q, dtype), _up(K, dtype), _up(V, dtype), **kw), dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_cross_entropy(reduction, dtype):
    degree = 3
    Z = _series((40, 300), degree, 8, scale=2.0)
    y = torch.randint(0, 300, (40,), generator=torch.Generator().manual_seed(9))
    y[::7] = -100
    with torch.no_grad(), PolyTensor.plain_range():
        got = F.cross_entropy(_poly(Z, dtype), y.cuda(), reduction=reduction)
    _check(got.coeffs, oracle.cross_entropy(_up(Z, dtype), y, reduction=reduction), dtype)


def test_complex_base_is_refused():
    # gelu's erf form has no complex form here (the other activations take a complex constant term,
    # tests/test_gpu_high_degree.py); reverse mode with complex directions is covered by
    # tests/test_gpu_training.py
    with PolyTensor.plain_range():
        x = PolyTensor((torch.randn(4, 8, dtype=torch.complex64, device="cuda"),
                        torch.randn(4, 8, dtype=torch.complex64, device="cuda")))
        with pytest.raises(NotImplementedError, match="complex base"):
            F.gelu(x)


def _decoder_case(layers, d, heads, vocab, batch, seq, degree, seed):
    params = bench.gpt_init_params(layers, d, vocab, seq, seed=seed, dtype=torch.float64)
    g = torch.Generator().manual_seed(seed + 1)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g)
    targets = torch.randint(0, vocab, (batch, seq), generator=g)
    base = bench.gpt_embed(params, tokens)
    direction = torch.complex(torch.randn(batch, seq, d, generator=g, dtype=torch.float64),
                              torch.randn(batch, seq, d, generator=g, dtype=torch.float64))
    return params, base, direction, targets


def _decoder_gpu(params, base, direction, targets, heads, degree, dtype):
    cdt = torch.complex64 if dtype == torch.float32 else torch.complex128
    gp = {k: v for k, v in params.items()}
    gp["blocks"] = [{k: v.to(dtype).cuda() for k, v in blk.items()} for blk in params["blocks"]]
    for k in ("wte", "wpe", "lnf_w", "lnf_b", "head"):
        gp[k] = params[k].to(dtype).cuda()
    with torch.no_grad(), PolyTensor.plain_range():
        x = PolyTensor((base.to(dtype).cuda(), direction.to(cdt).cuda()), degree=degree)
        return bench.gpt_forward(gp, x, targets.cuda(), heads)


def _decoder_oracle(params, base, direction, targets, heads, degree, dtype):
    cdt = torch.complex64 if dtype == torch.float32 else torch.complex128
    up = lambda t: t.to(dtype).double() if not t.is_complex() else t.to(cdt).to(torch.complex128)  # noqa: E731
    op = {k: v for k, v in params.items()}
    op["blocks"] = [{k: up(v) for k, v in blk.items()} for blk in params["blocks"]]
    for k in ("wte", "wpe", "lnf_w", "lnf_b", "head"):
        op[k] = up(params[k])
    X = [up(base), up(direction)] + [torch.zeros(base.shape, dtype=torch.complex128) for _ in range(degree - 1)]
    return oracle.gpt_forward(op, X, targets, heads)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_decoder_small(dtype):
    layers, d, heads, vocab, batch, seq, degree = 2, 64, 4, 96, 2, 32, 3
    case = _decoder_case(layers, d, heads, vocab, batch, seq, degree, seed=11)
    got = _decoder_gpu(*case, heads, degree, dtype)
    want = _decoder_oracle(*case, heads, degree, dtype)
    assert got.degree == degree and all(c.is_complex() for c in got.coeffs[1:])
    for k, (a, b) in enumerate(zip(got.coeffs, want)):
        err = abs(a.item() - b.item()) / max(abs(b.item()), 1e-30)
        assert err <= TOL[dtype], f"order {k}: {a.item()} vs {b.item()} ({err:.2e})"


def test_decoder_full_width():
    # config 5's network (12 layers, d 768, 12 heads, vocab 32000, K=3, complex64 directions) on one
    # sequence of 64 tokens against the oracle
    layers, d, heads, vocab, batch, seq, degree = 12, 768, 12, 32000, 1, 64, 3
    case = _decoder_case(layers, d, heads, vocab, batch, seq, degree, seed=12)
    got = _decoder_gpu(*case, heads, degree, torch.float32)
    want = _decoder_oracle(*case, heads, degree, torch.float32)
    for k, (a, b) in enumerate(zip(got.coeffs, want)):
        err = abs(a.item() - b.item()) / max(abs(b.item()), 1e-30)
        assert err <= TOL[torch.float32], f"order {k}: {a.item()} vs {b.item()} ({err:.2e})"


def test_decoder_config5_full_size_properties():
    # config 5 exactly (batch 8, seq 1024) on the GPU: order 0 is the ordinary model's loss, and
    # order 1 is linear in the direction: loss_1(u + i w) = loss_1(u) + i loss_1(w) with the
    # real-direction runs computed separately
    layers, d, heads, vocab, batch, seq, degree = 12, 768, 12, 32000, 8, 1024, 3
    params = bench.gpt_init_params(layers, d, vocab, seq, seed=5, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(6)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g, device="cuda")
    targets = torch.randint(0, vocab, (batch, seq), generator=g, device="cuda")
    base = bench.gpt_embed(params, tokens)
    u = torch.randn(batch, seq, d, generator=g, device="cuda")
    w = torch.randn(batch, seq, d, generator=g, device="cuda")
    with torch.no_grad(), PolyTensor.plain_range():
        z = bench.gpt_forward(params, PolyTensor((base, torch.complex(u, w)), degree=degree), targets, heads)
        zu = bench.gpt_forward(params, PolyTensor((base, u), degree=degree), targets, heads)
        zw = bench.gpt_forward(params, PolyTensor((base, w), degree=degree), targets, heads)
        plain = bench.gpt_forward(params, base, targets, heads)
    assert math.isfinite(z.coeffs[0].item()) and abs(z.coeffs[0].item() - plain.item()) <= 1e-4 * abs(plain.item())
    first = complex(zu.coeffs[1].item(), zw.coeffs[1].item())
    assert abs(z.coeffs[1].item() - first) <= 1e-4 * abs(first)
    # a real computation has conjugate-symmetric coefficients: loss_k(u - i w) = conj(loss_k(u + i w))
    with torch.no_grad(), PolyTensor.plain_range():
        zc = bench.gpt_forward(params, PolyTensor((base, torch.complex(u, -w)), degree=degree), targets, heads)
    for k in range(1, degree + 1):
        a, b = zc.coeffs[k].item(), z.coeffs[k].item().conjugate()
        assert abs(a - b) <= 1e-4 * max(abs(b), 1e-30), k


@pytest.mark.parametrize("degree", [5, 6, 7, 8])
def test_complex64_at_high_degree(degree):
    # the interpolation at lam = i amplifies the real runs' rounding most at high degree; complex64
    # must still meet the float32 tolerance (1e-4 per order) at every supported degree
    dt = torch.float32
    Q, K, V = (_series((2, 2, 70, 32), degree, 7 + i, scale=0.5) for i in range(3))
    X = _series((6, 96), degree, 6)
    Z = _series((40, 300), degree, 8, scale=2.0)
    y = torch.randint(0, 300, (40,), generator=torch.Generator().manual_seed(9))
    A, B = _series((5, 37), degree, 3), _series((5, 37), degree, 4, positive=True)
    with torch.no_grad(), PolyTensor.plain_range():
        att = F.scaled_dot_product_attention(_poly(Q, dt), _poly(K, dt), _poly(V, dt), is_causal=True)
        ln = F.layer_norm(_poly(X, dt), (96,))
        ge = F.gelu(_poly(X, dt))
        ce = F.cross_entropy(_poly(Z, dt), y.cuda())
        qu = _poly(A, dt) / _poly(B, dt)
    _check(att.coeffs, oracle.attention(_up(Q, dt), _up(K, dt), _up(V, dt), is_causal=True), dt)
    _check(ln.coeffs, oracle.layer_norm(_up(X, dt), (96,)), dt)
    _check(ge.coeffs, oracle.activation(_up(X, dt), "gelu"), dt)
    _check(ce.coeffs, oracle.cross_entropy(_up(Z, dt), y), dt)
    _check(qu.coeffs, oracle.quotient(_up(A, dt), _up(B, dt)), dt)


# ---------------------------------------------------------------------------
# A complex constant term (complex base): complex arithmetic in the bilinear products
# (/root/reference/docs/notes.md:74-77: "a complex constant coefficient uses PyTorch's complex
# semantics"), against the oracle's complex arithmetic (torch.matmul and elementwise products of
# complex tensors, /root/reference/src/polytensors/_plain.py:118-128).

def _complex_series(shape, degree, seed, dtype=torch.complex128):
    g = torch.Generator().manual_seed(seed)
    return [torch.complex(torch.randn(shape, generator=g, dtype=torch.float64),
                          torch.randn(shape, generator=g, dtype=torch.float64)).to(dtype) * 0.5 ** k
            for k in range(degree + 1)]


def _check_series(got, want, tol, what):
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.detach().cpu(), b)
        assert err <= tol, f"{what} order {k}: {err:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.complex128, 1e-10), (torch.complex64, 1e-4)])
@pytest.mark.parametrize("degree", [1, 3])
def test_complex_base_matmul(dtype, tol, degree):
    A = _complex_series((2, 17, 24), degree, 300, dtype)
    B = _complex_series((24, 9), degree, 301, dtype)
    W = _complex_series((24, 9), 0, 302, dtype)[0]
    real = torch.float64 if dtype == torch.complex128 else torch.float32
    Breal = [torch.randn(24, 9, generator=torch.Generator().manual_seed(303 + k), dtype=real) for k in range(degree + 1)]
    a, b, breal = (PolyTensor(tuple(c.cuda() for c in s)) for s in (A, B, Breal))
    up = lambda s: [c.to(torch.complex128) for c in s]   # noqa: E731
    with torch.no_grad(), PolyTensor.plain_range():
        _check_series((a @ b).coeffs, oracle.matmul(up(A), up(B)), tol, "series @ series")
        _check_series((a @ W.cuda()).coeffs, oracle.matmul(up(A), [W.to(torch.complex128)]), tol, "series @ plain")
        _check_series((a @ breal).coeffs, oracle.matmul(up(A), [c.to(torch.complex128) for c in Breal]), tol,
                      "complex base @ real series")
        _check_series(F.linear(a, W.t().contiguous().cuda()).coeffs,
                      oracle.matmul(up(A), [W.to(torch.complex128)]), tol, "linear")


@pytest.mark.parametrize("degree", [2, 4])
def test_complex_base_elementwise_product_quotient_and_powers(degree):
    X = _complex_series((7, 33), degree, 310)
    Y = _complex_series((7, 33), degree, 311)
    Y[0] = Y[0] + 3.0   # keep the divisor away from zero
    g = torch.Generator().manual_seed(312)
    R = [torch.randn(7, 33, generator=g, dtype=torch.float64) * 0.5 ** k for k in range(degree + 1)]
    R[0] = R[0].abs() + 1.0
    D = [R[0]] + [torch.complex(torch.randn(7, 33, generator=g, dtype=torch.float64),
                                torch.randn(7, 33, generator=g, dtype=torch.float64)) for _ in range(degree)]
    x, y, r, d = (PolyTensor(tuple(c.cuda() for c in s)) for s in (X, Y, R, D))
    with torch.no_grad(), PolyTensor.plain_range():
        _check_series((x * y).coeffs, oracle.cauchy(X, Y), 1e-10, "x * y")
        _check_series((x * r).coeffs, oracle.cauchy(X, R), 1e-10, "x * real series")
        _check_series((x * d).coeffs, oracle.cauchy(X, [c.to(torch.complex128) for c in D]), 1e-10,
                      "x * complex-direction series")
        _check_series((x / y).coeffs, oracle.quotient(X, Y), 1e-10, "x / y")
        _check_series((x / r).coeffs, oracle.quotient(X, R), 1e-10, "x / real series")
        _check_series((r / y).coeffs, oracle.quotient([c.to(torch.complex128) for c in R], Y), 1e-10,
                      "real series / y")
        cube = oracle.cauchy(oracle.cauchy(X, X), X)
        _check_series(x.pow(3).coeffs, cube, 1e-10, "x ** 3")
        _check_series(x.pow(-2).coeffs, oracle.quotient([torch.ones_like(X[0])] + [torch.zeros_like(c) for c in X[1:]],
                                                         oracle.cauchy(X, X)), 1e-10, "x ** -2")


def test_complex_base_coefficient_autograd_matches_autograd_of_the_oracle():
    degree = 2
    A = _complex_series((5, 12), degree, 320)
    B = _complex_series((12, 4), degree, 321)
    Wt = _complex_series((5, 4), degree, 322)

    def loss(a):   # real loss of the complex product's coefficients
        y = oracle.matmul(a, B)
        return sum((yk * wk).real.sum() for yk, wk in zip(y, Wt))

    leaves = [c.clone().requires_grad_() for c in A]
    want = torch.autograd.grad(loss(leaves), leaves)
    cl = [c.cuda().requires_grad_() for c in A]
    with PolyTensor.plain_range(), PolyTensor.coefficient_autograd():
        y = PolyTensor(tuple(cl)) @ PolyTensor(tuple(c.cuda() for c in B))
    total = sum((yk * wk.cuda()).real.sum() for yk, wk in zip(y.coeffs, Wt))
    got = torch.autograd.grad(total, cl)
    for k, (a, b) in enumerate(zip(got, want)):
        assert rel_err(a.cpu(), b) <= 1e-10, f"gradient of coefficient {k}"


def test_complex_base_refusals():
    with PolyTensor.plain_range():
        x = PolyTensor(tuple(c.cuda() for c in _complex_series((4, 8), 2, 330)), requires_grad=True)
        w = torch.randn(8, 3, dtype=torch.complex128, device="cuda")
        with pytest.raises(NotImplementedError, match="reverse mode with a complex constant term"):
            x @ w
        with torch.no_grad(), pytest.raises(NotImplementedError, match="complex base"):
            F.gelu(x)
        with torch.no_grad(), pytest.raises(NotImplementedError, match="complex base"):
            F.layer_norm(x, (8,))
