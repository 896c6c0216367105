"""Elementwise activation series of the oracle (test infrastructure only; see oracle/__init__.py).

gelu, tanh and sigmoid follow the reference's plain-range rule: the
derivatives of the activation at the constant term, composed with the
series' higher orders by Faa di Bruno
(/root/reference/src/polytensors/_plain.py:174-259). silu and gelu_tanh have
no plain-range rule in the reference; they follow its default-mode jets
(/root/reference/src/polytensors/_activations.py:89-115): normalized
derivatives of x*sigmoid(x) and x*sigmoid(2c(x + 0.044715 x^3)) at the
constant term, composed the same way. exp and log are plain_exp/plain_log
(_plain.py:153-171). Backward rules are _plain.py:310-325 (gelu, tanh,
sigmoid) and the derivative jets of the same functions (silu, gelu_tanh).
"""

import math

import torch

from .series import cauchy, exp_series, log_series


def compose(derivatives, X):
    """f(X(t)) from the derivatives f^(j)(X_0), j = 0..K (Faa di Bruno via powers of h).

    /root/reference/src/polytensors/_plain.py:174-188 (_compose): h = (0, X_1, .., X_K),
    out_k = sum_j f^(j)/j! (h^j)_k.
    """
    degree = len(X) - 1
    h = [torch.zeros_like(X[0])] + list(X[1:])
    out = [derivatives[0]] + [torch.zeros_like(X[0]) for _ in range(degree)]
    power = h
    factorial = 1.0
    for j in range(1, degree + 1):
        factorial *= j
        coefficient = derivatives[j] / factorial
        for k in range(j, degree + 1):
            out[k] = out[k] + coefficient * power[k]
        if j < degree:
            power = cauchy(power, h)
    return out


def _hermite(x, count):
    """Probabilists' Hermite polynomials He_0..He_{count-1}, /root/reference/src/polytensors/_plain.py:191-196."""
    values = [torch.ones_like(x), x]
    for n in range(1, count - 1):
        values.append(x * values[n] - n * values[n - 1])
    return values[:count]


def _gelu_derivatives(x, count, offset=0):
    """(x Phi(x))^(n), n = offset..offset+count-1, /root/reference/src/polytensors/_plain.py:199-219."""
    phi = torch.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)
    Phi = 0.5 * (1 + torch.erf(x / math.sqrt(2)))
    he = _hermite(x, offset + count + 1)

    def Phi_derivative(m):
        if m == 0:
            return Phi
        sign = -1.0 if (m - 1) % 2 else 1.0
        return sign * he[m - 1] * phi

    return [x * Phi if n == 0 else x * Phi_derivative(n) + n * Phi_derivative(n - 1)
            for n in range(offset, offset + count)]


def _output_polynomial_derivatives(y, count, offset, g):
    """Derivatives P_n(y) of a function with f' = g(f): P_0 = y, P_{n+1} = P_n'(y) g(y).

    /root/reference/src/polytensors/_plain.py:221-244; ``g`` lists polynomial
    coefficients in increasing powers.
    """
    polynomial = [0.0, 1.0]
    polynomials = [polynomial]
    for _ in range(offset + count - 1):
        derivative = [i * c for i, c in enumerate(polynomial)][1:] or [0.0]
        product = [0.0] * (len(derivative) + len(g) - 1)
        for i, a in enumerate(derivative):
            for j, b in enumerate(g):
                product[i + j] += a * b
        polynomial = product
        polynomials.append(polynomial)
    out = []
    for p in polynomials[offset:offset + count]:
        value = torch.zeros_like(y)
        for c in reversed(p):
            value = value * y + c
        out.append(value)
    return out


def derivatives(kind, x, count, offset=0):
    """f^(n)(x) for n = offset..offset+count-1, /root/reference/src/polytensors/_plain.py:246-253."""
    if kind == "gelu":
        return _gelu_derivatives(x, count, offset)
    if kind == "tanh":
        return _output_polynomial_derivatives(torch.tanh(x), count, offset, [1.0, 0.0, -1.0])
    if kind == "sigmoid":
        return _output_polynomial_derivatives(torch.sigmoid(x), count, offset, [0.0, 1.0, -1.0])
    if kind in ("silu", "gelu_tanh"):
        jet = _product_jet(kind, x, offset + count - 1)
        return [jet[n] * math.factorial(n) for n in range(offset, offset + count)]
    raise ValueError(kind)


def _normalized_compose(jet, delta):
    """sum_n jet[n] (delta^n)_k for a zero-constant series delta, /root/reference/src/polytensors/_activations.py:26-36."""
    degree = len(delta) - 1
    power = [torch.ones_like(jet[0])] + [torch.zeros_like(jet[0]) for _ in range(degree)]
    result = [torch.zeros_like(jet[0]) for _ in range(degree + 1)]
    for n in range(degree + 1):
        for k in range(n, degree + 1):
            result[k] = result[k] + jet[n] * power[k]
        if n < degree:
            power = cauchy(power, delta)
    return result


def _sigmoid_jet(x, degree):
    """Normalized derivatives sigmoid^(n)(x)/n!, n = 0..degree, by the recurrence of
    /root/reference/src/polytensors/_activations.py:39-60 (_sigmoid_taylor) in plain arithmetic:
    r = exp(-|x|), v_0 = sigmoid(x) from r, q_0 = r / (1 + r)^2 and, from y' = y - y^2,
    q_n = v_n (1 - 2 v_0) - sum_{i=1..n-1} v_i v_{n-i},  v_{n+1} = q_n / (n + 1).
    """
    sign = torch.where(x >= 0, 1.0, -1.0).to(x.dtype)
    r = torch.exp(-sign * x)
    denominator = 1 + r
    root = (sign > 0).to(x.dtype) - sign * (r / denominator)
    values = [root]
    q = [r / (denominator * denominator)]
    for n in range(degree):
        if n:
            coefficient = values[n] * (1 - 2 * root)
            for i in range(1, n):
                coefficient = coefficient - values[i] * values[n - i]
            q.append(coefficient)
        values.append(q[n] / (n + 1))
    return values


def _product_jet(kind, x, degree):
    """Normalized derivatives f^(n)(x)/n!, n = 0..degree, of silu and gelu_tanh.

    /root/reference/src/polytensors/_activations.py:89-115: with s_n the
    normalized sigmoid jet of the inner argument, f_0 = x s_0, f_n = x s_n + s_{n-1}.
    """
    if kind == "silu":
        inner = _sigmoid_jet(x, degree)
    else:
        scale = 2 * math.sqrt(2 / math.pi)
        cubic = 0.044715
        argument = scale * x * (1 + cubic * x * x)
        sigmoid = _sigmoid_jet(argument, degree)
        delta = [torch.zeros_like(x) for _ in range(degree + 1)]
        if degree >= 1:
            delta[1] = scale * (1 + 3 * cubic * x * x)
        if degree >= 2:
            delta[2] = scale * 3 * cubic * x
        if degree >= 3:
            delta[3] = torch.full_like(x, scale * cubic)
        inner = _normalized_compose(sigmoid, delta)
    return [x * inner[0]] + [x * inner[n] + inner[n - 1] for n in range(1, degree + 1)]


def activation(X, kind):
    """Series of f(X(t)) for gelu, gelu_tanh, tanh, sigmoid, silu, exp, log."""
    if kind == "exp":
        return exp_series(X)
    if kind == "log":
        return log_series(X)
    degree = len(X) - 1
    return compose(derivatives(kind, X[0], degree + 1), X)


def activation_backward(G, S, kind):
    """Gradient series of the native backward: G (*) f'(X(t)).

    ``S`` is the forward input X for gelu, gelu_tanh, silu, and the forward
    output Y for tanh and sigmoid (as aten.tanh_backward takes it):
      gelu     G (*) f'(X) with f' composed from derivatives at offset 1 (_plain.py:310-315);
      tanh     G (*) (1 - Y (*) Y)                                        (_plain.py:316-320);
      sigmoid  G (*) (Y (*) (1 - Y))                                      (_plain.py:321-325);
      silu, gelu_tanh: G (*) f'(X), f' from the same derivative jets.
    """
    degree = len(S) - 1
    if kind == "tanh":
        one_minus = [1 - y if k == 0 else -y for k, y in enumerate(cauchy(S, S))]
        return cauchy(G, one_minus)
    if kind == "sigmoid":
        one_minus = [1 - y if k == 0 else -y for k, y in enumerate(S)]
        return cauchy(G, cauchy(S, one_minus))
    if kind in ("gelu", "silu", "gelu_tanh"):
        return cauchy(G, compose(derivatives(kind, S[0], degree + 1, offset=1), S))
    raise ValueError(f"no backward series for {kind}")
