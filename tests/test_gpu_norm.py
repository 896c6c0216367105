"""RMSNorm / LayerNorm series kernels vs the CPU oracle (GPU).

Mirrors the reference's fused-norm tests (/root/reference/tests/test_fused_norm.py:14-35):
F.rms_norm on a PolyTensor inside plain_range() must take the fused path and
match independent series at every order. Inputs are generated on the CPU with a
seeded generator and copied to the device, so kernel and oracle see the same
bits; the oracle runs in float64 on the (upcast) inputs. Per-order tolerance is
max|got - want| / max|want|: 1e-10 float64, 1e-4 float32, 2e-2 bfloat16 and
float16 (float32 arithmetic on 16-bit storage).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor, _fused_norm, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _series(shape, degree, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k).to(dtype)
            for k in range(degree + 1)]


def _poly(cpu_coeffs):
    return PolyTensor(tuple(c.cuda() for c in cpu_coeffs))


class _Spy:
    def __init__(self, monkeypatch):
        self.calls = 0
        original = _ops.norm_series

        def spy(*args, **kwargs):
            self.calls += 1
            return original(*args, **kwargs)

        monkeypatch.setattr(_ops, "norm_series", spy)


def _check(got, want, dtype):
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.cpu(), b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e} > {TOL[dtype]:.0e}"


# (shape, normalized): register paths with 64 and 256 threads per row and 1/2/4 chunks,
# the streaming path (rows too long, or not a multiple of the vector width), several rows.
SHAPES = [((3, 17), (17,)), ((2, 3, 4), (3, 4)), ((5, 64), (64,)), ((7, 256), (256,)),
          ((6, 1024), (1024,)), ((4, 2048), (2048,)), ((4, 4096), (4096,)), ((3, 12288), (12288,)),
          ((2, 5, 1000), (1000,)), ((9, 384), (384,))]


@pytest.mark.parametrize("shape,normalized", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("degree", [1, 4])
def test_rms_norm_matches_oracle(monkeypatch, shape, normalized, dtype, degree):
    spy = _Spy(monkeypatch)
    X = _series(shape, degree, seed=1, dtype=dtype)
    x = _poly(X)
    with torch.no_grad(), PolyTensor.plain_range():
        assert _fused_norm.eligible(x, normalized)
        y = F.rms_norm(x, normalized, eps=1e-5)
    assert spy.calls == 1
    assert y.degree == degree and y.dtype == dtype and all(c.dtype == dtype for c in y.coeffs)
    want = oracle.rms_norm([c.double() for c in X], normalized, eps=1e-5)
    _check(y.coeffs, want, dtype)


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 5, 6, 7, 8])
@pytest.mark.parametrize("n", [96, 4096])
def test_rms_norm_every_degree(degree, n):
    X = _series((6, n), degree, seed=2, dtype=torch.float32)
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.rms_norm(_poly(X), (n,), eps=1e-6)
    want = oracle.rms_norm([c.double() for c in X], (n,), eps=1e-6)
    _check(y.coeffs, want, torch.float32)


@pytest.mark.parametrize("weight_kind", ["plain", "series", "other_dtype"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_weight(weight_kind, dtype):
    degree, n = 3, 512
    X = _series((8, n), degree, seed=3, dtype=dtype)
    g = torch.Generator().manual_seed(4)
    if weight_kind == "series":
        Wc = [(1 + 0.02 * torch.randn(n, generator=g, dtype=torch.float64)).to(dtype)] + \
             [(0.1 * torch.randn(n, generator=g, dtype=torch.float64)).to(dtype) for _ in range(degree)]
        w = _poly(Wc)
    else:
        wdtype = torch.float64 if weight_kind == "other_dtype" else dtype
        Wc = [(1 + 0.02 * torch.randn(n, generator=g, dtype=torch.float64)).to(wdtype)]
        w = Wc[0].cuda()
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.rms_norm(_poly(X), (n,), weight=w, eps=1e-6)
    want = oracle.rms_norm([c.double() for c in X], (n,), weight=[c.double() for c in Wc], eps=1e-6)
    _check(y.coeffs, want, dtype)


def test_rms_norm_default_eps_and_plain_operands():
    X = _series((4, 32), 2, seed=5, dtype=torch.float32)
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.rms_norm(_poly(X), (32,))
    want = oracle.rms_norm([c.double() for c in X], (32,), eps=torch.finfo(torch.float32).eps)
    _check(y.coeffs, want, torch.float32)


@pytest.mark.parametrize("affine", ["none", "plain", "series"])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [200, 768, 4096])
def test_layer_norm_matches_oracle(affine, dtype, n):
    degree = 3
    X = _series((5, n), degree, seed=6, dtype=dtype, scale=2.0)
    X[0] = (X[0].double() + 3.0).to(dtype)     # a mean to remove
    g = torch.Generator().manual_seed(7)
    W = B = None
    if affine == "plain":
        W = [(1 + 0.1 * torch.randn(n, generator=g, dtype=torch.float64)).to(dtype)]
        B = [(0.1 * torch.randn(n, generator=g, dtype=torch.float64)).to(dtype)]
    elif affine == "series":
        W = _series((n,), degree, seed=8, dtype=dtype)
        B = _series((n,), degree, seed=9, dtype=dtype)
    to_arg = lambda s: None if s is None else (s[0].cuda() if len(s) == 1 else _poly(s))
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.layer_norm(_poly(X), (n,), to_arg(W), to_arg(B), eps=1e-5)
    dbl = lambda s: None if s is None else [c.double() for c in s]
    want = oracle.layer_norm(dbl(X), (n,), dbl(W), dbl(B), eps=1e-5)
    _check(y.coeffs, want, dtype)


def test_noncontiguous_input_and_rows_from_a_stacked_buffer():
    degree, n = 4, 1024
    X = _series((n, 6), degree, seed=10, dtype=torch.float32)
    stacked = torch.stack([c.cuda() for c in X]).transpose(-1, -2)     # [K+1, 6, n] non-contiguous
    x = PolyTensor(tuple(stacked.unbind(0)))
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.rms_norm(x, (n,), eps=1e-5)
    want = oracle.rms_norm([c.double().t() for c in X], (n,), eps=1e-5)
    _check(y.coeffs, want, torch.float32)


def test_full_size_config_rows_sample():
    # benchmark config 4a: [5, 8192, 4096] bf16, eps 1e-6, weight 1 + 0.02 N(0,1). Checked on a
    # seeded sample of rows against the oracle, and for the row mean-square identity of order 0.
    degree, rows, n = 4, 8192, 4096
    g = torch.Generator().manual_seed(3)
    X = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(degree + 1)]
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(torch.bfloat16)
    with torch.no_grad(), PolyTensor.plain_range():
        y = F.rms_norm(_poly(X), (n,), weight=w.cuda(), eps=1e-6)
    pick = torch.randperm(rows, generator=g)[:48]
    want = oracle.rms_norm([c[pick].double() for c in X], (n,), weight=[w.double()], eps=1e-6)
    _check([c[pick.cuda()] for c in y.coeffs], want, torch.bfloat16)
    ms = (y.coeffs[0].float() / w.cuda().float()).pow(2).mean(-1)
    assert torch.allclose(ms, torch.ones_like(ms), atol=2e-2)
