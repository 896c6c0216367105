"""Pins of the oracle's activation series (CPU only).

``oracle.activation`` restates the reference's plain-range activation rule
(derivatives at the constant term composed by Faa di Bruno,
/root/reference/src/polytensors/_plain.py:174-259) and its default-mode silu /
gelu_tanh jets (/root/reference/src/polytensors/_activations.py:89-115). The
checks here fix the answer independently of those rules: nested forward-mode
derivatives of torch's own activation along the curve (tests/jets.py), and,
for the backward operations, forward-over-reverse derivatives of torch.func.vjp
-- the pattern of /root/reference/tests/test_fused_activation.py:10-26 taken to
degree K. Planted mistakes in copies of the composition must be caught.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import activations
from tests.jets import rel_err, taylor

FUNCTIONS = {
    "gelu": F.gelu,
    "gelu_tanh": lambda x: F.gelu(x, approximate="tanh"),
    "tanh": torch.tanh,
    "sigmoid": torch.sigmoid,
    "silu": F.silu,
    "exp": torch.exp,
    "log": torch.log,
}


def _series(shape, degree, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]


def _inputs(kind, degree, seed):
    X = _series((3, 5), degree, seed, scale=1.5)
    if kind == "log":
        X[0] = X[0].abs() + 0.5
    return X


def _check(got, want, tol):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a, b)
        assert err <= tol, f"order {k}: {err:.3e} > {tol:.0e}"


@pytest.mark.parametrize("degree", (1, 4, 5))
@pytest.mark.parametrize("kind", sorted(FUNCTIONS))
def test_activation_matches_jets(kind, degree):
    X = _inputs(kind, degree, seed=60 + degree)
    _check(oracle.activation(X, kind), taylor(FUNCTIONS[kind], [X], degree), 1e-10)


@pytest.mark.parametrize("degree", (1, 4))
@pytest.mark.parametrize("kind", ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu"))
def test_activation_backward_matches_jets(kind, degree):
    X = _inputs(kind, degree, seed=70 + degree)
    G = _series((3, 5), degree, seed=80 + degree)
    saved = oracle.activation(X, kind) if kind in ("tanh", "sigmoid") else X
    f = FUNCTIONS[kind]

    def vjp(x, g):
        return torch.func.vjp(f, x)[1](g)[0]

    _check(oracle.activation_backward(G, saved, kind), taylor(vjp, [X, G], degree), 1e-10)


def test_degree_one_matches_the_reference_fused_kernel_formulas():
    # The degree-1 values the reference's Triton kernel computes
    # (/root/reference/src/polytensors/_activation_kernels.py:15-36): y1 = f'(x0) x1.
    x0, x1 = _series((4, 7), 1, seed=90)
    phi = torch.exp(-0.5 * x0 * x0) / math.sqrt(2 * math.pi)
    cdf = 0.5 * (1 + torch.erf(x0 / math.sqrt(2)))
    expected = {
        "gelu": (x0 * cdf, (cdf + x0 * phi) * x1),
        "tanh": (torch.tanh(x0), (1 - torch.tanh(x0) ** 2) * x1),
        "sigmoid": (torch.sigmoid(x0), torch.sigmoid(x0) * (1 - torch.sigmoid(x0)) * x1),
    }
    for kind, (y0, y1) in expected.items():
        got = oracle.activation([x0, x1], kind)
        torch.testing.assert_close(got[0], y0, rtol=1e-14, atol=1e-15)
        torch.testing.assert_close(got[1], y1, rtol=1e-12, atol=1e-14)


# --- planted mistakes -------------------------------------------------------------------------

def _compose_plain_factorial(derivatives, X):
    degree = len(X) - 1
    h = [torch.zeros_like(X[0])] + list(X[1:])
    out = [derivatives[0]] + [torch.zeros_like(X[0]) for _ in range(degree)]
    power = h
    for j in range(1, degree + 1):
        coefficient = derivatives[j] / j           # planted: j instead of j!
        for k in range(j, degree + 1):
            out[k] = out[k] + coefficient * power[k]
        if j < degree:
            power = activations.cauchy(power, h)
    return out


def _compose_no_power_update(derivatives, X):
    degree = len(X) - 1
    h = [torch.zeros_like(X[0])] + list(X[1:])
    out = [derivatives[0]] + [torch.zeros_like(X[0]) for _ in range(degree)]
    factorial = 1.0
    for j in range(1, degree + 1):
        factorial *= j
        for k in range(j, degree + 1):
            out[k] = out[k] + derivatives[j] / factorial * h[k]   # planted: h instead of h^j
    return out


@pytest.mark.parametrize("mutant", [_compose_plain_factorial, _compose_no_power_update])
def test_planted_composition_mistakes_are_caught(monkeypatch, mutant):
    monkeypatch.setattr(activations, "compose", mutant)
    with pytest.raises(AssertionError):
        test_activation_matches_jets("gelu", 4)
    with pytest.raises(AssertionError):
        test_activation_matches_jets("tanh", 4)
