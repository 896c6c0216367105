"""Activation-series kernel vs the CPU oracle (GPU).

Mirrors /root/reference/tests/test_fused_activation.py:10-26 (value and
gradient series of gelu/tanh/sigmoid on transposed (non-contiguous) inputs in
four dtypes) at degree K, and adds gelu's tanh form, silu, exp and log, every
degree 0..8, the backward operations, and the large-|x| sigmoid derivative of
/root/reference/tests/test_primitives.py:215-234. Inputs are generated on the
CPU with seeded generators; the oracle runs in float64 on the (upcast) inputs.
Per-order tolerance max|got - want| / max|want|: 1e-10 float64, 1e-4 float32,
2e-2 bfloat16 and float16.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}
KINDS = ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu", "exp", "log")
FUNCTIONS = {
    "gelu": F.gelu,
    "gelu_tanh": lambda x: F.gelu(x, approximate="tanh"),
    "tanh": torch.tanh,
    "sigmoid": torch.sigmoid,
    "silu": F.silu,
    "exp": torch.exp,
    "log": torch.log,
}
BACKWARD_OPS = {
    "gelu": lambda g, s: torch.ops.aten.gelu_backward(g, s),
    "gelu_tanh": lambda g, s: torch.ops.aten.gelu_backward(g, s, approximate="tanh"),
    "tanh": torch.ops.aten.tanh_backward,
    "sigmoid": torch.ops.aten.sigmoid_backward,
    "silu": torch.ops.aten.silu_backward,
}


def _series(shape, degree, seed, kind="gelu", scale=1.5, transpose=False):
    g = torch.Generator().manual_seed(seed)
    cs = [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]
    if kind == "log":
        cs[0] = cs[0].abs() + 0.5
    if transpose:
        cs = [c.T for c in cs]
    return cs


def _cast(cs, dtype):
    return [c.to(dtype) for c in cs]


def _poly(cs):
    return PolyTensor(tuple(c.cuda() for c in cs))


def _check(got, want, dtype):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.cpu(), b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e} > {TOL[dtype]:.0e}"


class _Spy:
    def __init__(self, monkeypatch, name):
        self.calls = 0
        original = getattr(_ops, name)

        def spy(*args, **kwargs):
            self.calls += 1
            return original(*args, **kwargs)

        monkeypatch.setattr(_ops, name, spy)


SHAPES = [((3, 1027), True), ((4096,), False), ((5, 33), False), ((1000003,), False)]


@pytest.mark.parametrize("shape,transpose", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("degree", [1, 4])
@pytest.mark.parametrize("kind", KINDS)
def test_forward_matches_oracle(monkeypatch, kind, degree, dtype, shape, transpose):
    spy = _Spy(monkeypatch, "activation_series")
    X = _cast(_series(shape, degree, seed=3, kind=kind, transpose=transpose), dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        y = FUNCTIONS[kind](_poly(X))
    assert spy.calls == 1
    assert y.degree == degree and y.dtype == dtype and y.shape == X[0].shape
    _check(y.coeffs, oracle.activation([c.double() for c in X], kind), dtype)


@pytest.mark.parametrize("degree", [0, 2, 3, 5, 6, 7, 8])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("kind", KINDS)
def test_every_degree(kind, dtype, degree):
    X = _cast(_series((7, 129), degree, seed=4, kind=kind), dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        y = FUNCTIONS[kind](_poly(X))
    _check(y.coeffs, oracle.activation([c.double() for c in X], kind), dtype)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("degree", [1, 4, 8])
@pytest.mark.parametrize("kind", sorted(BACKWARD_OPS))
def test_backward_matches_oracle(monkeypatch, kind, degree, dtype, transpose):
    spy = _Spy(monkeypatch, "activation_series_backward")
    X = _series((3, 1027), degree, seed=5, transpose=transpose)
    G = _series((3, 1027), degree, seed=6, scale=1.0, transpose=transpose)
    # tanh/sigmoid backward take the forward output, as aten does.
    saved = oracle.activation(X, kind) if kind in ("tanh", "sigmoid") else X
    saved, G = _cast(saved, dtype), _cast(G, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        dx = BACKWARD_OPS[kind](_poly(G), _poly(saved))
    assert spy.calls == 1 and dx.degree == degree and dx.dtype == dtype
    want = oracle.activation_backward([g.double() for g in G], [s.double() for s in saved], kind)
    _check(dx.coeffs, want, dtype)


def test_plain_operand_of_backward_is_lifted():
    X = _series((64,), 3, seed=7)
    g0 = torch.randn(64, dtype=torch.float64)
    with torch.no_grad(), PolyTensor.plain_range():
        dx = torch.ops.aten.gelu_backward(g0.cuda(), _poly(X))
    want = oracle.activation_backward([g0, *(torch.zeros_like(g0) for _ in range(3))], X, "gelu")
    _check(dx.coeffs, want, torch.float64)


def test_rounded_sigmoid_keeps_its_small_derivative():
    # /root/reference/tests/test_primitives.py:215-228: for |x| up to ~25 a float32
    # sigmoid rounds to 0 or 1, yet the first order must stay accurate per element.
    g = torch.Generator().manual_seed(11)
    x0 = 5 * torch.randn((32, 1536), generator=g)
    x1 = torch.randn(x0.shape, generator=g)
    with torch.no_grad(), PolyTensor.plain_range():
        y = torch.sigmoid(_poly([x0, x1]))
    tail = torch.exp(-x0.double().abs())
    first = (tail / (1 + tail).square() * x1.double()).float()
    torch.testing.assert_close(y.coeffs[1].cpu(), first, rtol=2e-6, atol=0)
    torch.testing.assert_close(y.coeffs[0].cpu(), torch.sigmoid(x0.double()).float(), rtol=4e-7, atol=0)


def test_full_size_bench_shape_rows_sample():
    # The bench workload (gelu of a degree-4 bf16 [8192, 4096] series), checked on sampled rows.
    g = torch.Generator().manual_seed(12)
    X = [(torch.randn(8192, 4096, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(5)]
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.gelu(_poly(X))
    rows = torch.randint(0, 8192, (48,), generator=g)
    want = oracle.activation([c[rows].double() for c in X], "gelu")
    _check([c[rows.cuda()] for c in y.coeffs], want, torch.bfloat16)


def test_errors_are_loud():
    X = _series((8,), 2, seed=13)
    x = _poly(X)
    with pytest.raises(NotImplementedError, match="plain_range"):
        with torch.no_grad():
            torch.tanh(x)
    with PolyTensor.plain_range(), torch.no_grad():
        with pytest.raises(ValueError, match="approximate"):
            torch.ops.aten.gelu(x, approximate="erf")
        with pytest.raises(NotImplementedError, match="HIP"):
            torch.tanh(PolyTensor(tuple(X)))
        with pytest.raises(NotImplementedError, match="broadcast"):
            torch.ops.aten.tanh_backward(x, _poly([c[:1] for c in X]))
