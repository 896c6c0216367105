"""Fused elementwise activation series (any degree up to 16) on gfx950.

The reference fuses first-order GELU/tanh/sigmoid and their native backward
operations (/root/reference/src/polytensors/_fused_activation.py:5-24, Triton
kernel _activation_kernels.py:8-38) and otherwise composes the derivatives of
the activation at the constant term (/root/reference/src/polytensors/_plain.py:174-259,
plain_rule :276-355). Here one kernel computes the whole series of
gelu (erf and tanh forms), tanh, sigmoid, silu, exp, log, sin, cos, sqrt and
rsqrt, and the gradient series of the gelu/tanh/sigmoid/silu backward
operations, at any degree up to 16.
Inputs are made contiguous first, as the reference's fused path does (:17).
Half and bfloat16 compute in float32, float64 in float64.
"""

import math

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)
BACKWARD_KINDS = ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu")


def why_ineligible(*operands, complex_ok=False, complex_base_ok=False):
    # Reached from __torch_dispatch__ only: autograd above has recorded the native
    # backward operation (gelu_backward, tanh_backward, ...), which routes here too.
    reason = _gate.common_reason(operands, below_autograd=True, complex_ok=complex_ok,
                                 complex_base_ok=complex_base_ok, max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    polys = [x for x in operands if isinstance(x, PolyTensor)]
    dtype = _gate.real_dtype(polys[0].dtype)
    if dtype not in _DTYPES or any(_gate.real_dtype(c.dtype) != dtype for p in polys for c in p.coeffs):
        return "activation series need float16/bfloat16/float32/float64 in every order"
    if any(not isinstance(x, PolyTensor) and (x.dtype != dtype) for x in operands if isinstance(x, torch.Tensor)):
        return "an ordinary operand must have the series' dtype"
    shape = polys[0].shape
    if any(tuple(x.shape) != tuple(shape) for x in operands if isinstance(x, torch.Tensor)):
        return "operands must have one shape (no broadcasting)"
    return None


def _coeffs(x, degree):
    if isinstance(x, PolyTensor):
        return [c.contiguous() for c in x.coeffs]
    base = x.contiguous()
    return [base] + [torch.zeros_like(base) for _ in range(degree)]


# kinds taken with a complex constant term (gelu's erf has no complex form here)
COMPLEX_BASE_KINDS = ("exp", "log", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid", "silu", "gelu_tanh")


def _mul(a, b):
    from ._fused_elementwise import binary

    return binary(a, b, "mul")


def _div(a, b):
    from ._fused_elementwise import binary

    return binary(a, b, "div")


def _lin(*terms):
    """sum of scale * series (scale a Python number, real or complex), order by order."""
    return PolyTensor(tuple(sum(w * x.coeffs[k] for w, x in terms) for k in range(terms[0][1].degree + 1)))


def _shift(x, value):
    """x + value on the constant order."""
    return PolyTensor((x.coeffs[0] + value,) + tuple(x.coeffs[1:]))


def _complex_exp(z):
    """exp(x + i y) = e^x (cos y + i sin y): the real kernels for exp, cos, sin and the product."""
    x, y = _complex._split(z)
    if y is None:
        return activation(x, "exp")
    ex = activation(x, "exp")
    return _complex._join(_mul(ex, activation(y, "cos")), _mul(ex, activation(y, "sin")))


def _complex_log(z):
    """log z = log(x^2 + y^2) / 2 + i arg z. The argument series integrates its derivative along
    t, (x y' - y x') / (x^2 + y^2) (real products and a quotient), from arg z_0 (torch.atan2: the
    principal branch, as torch's complex log)."""
    x, y = _complex._split(z)
    if y is None:
        return activation(x, "log")
    degree = z.degree

    def derivative(s):   # coefficient k: (k + 1) s_{k+1}; the last order has none
        cs = s.coeffs
        return PolyTensor(tuple((k + 1) * cs[k + 1] for k in range(degree)) + (torch.zeros_like(cs[0]),))

    r2 = _lin((1.0, _mul(x, x)), (1.0, _mul(y, y)))
    slope = _div(_lin((1.0, _mul(x, derivative(y))), (-1.0, _mul(y, derivative(x)))), r2)
    arg = PolyTensor((torch.atan2(y.coeffs[0], x.coeffs[0]),) +
                     tuple(slope.coeffs[k - 1] / k for k in range(1, degree + 1)))
    return _complex._join(_lin((0.5, activation(r2, "log"))), arg)


def _complex_reciprocal_of(z):
    """1 / z for a complex series (the complex quotient of the real kernels)."""
    one = PolyTensor((torch.ones_like(z.coeffs[0]),) + tuple(torch.zeros_like(c) for c in z.coeffs[1:]))
    return _complex.complex_quotient(_div, _mul, one, z)


def _complex_base(z, kind):
    """``kind`` of a series with a complex constant term, in complex arithmetic over the real
    kernels (the reference's general rules take complex arithmetic, /root/reference/docs/notes.md:74-77):
    exp and log as above; sqrt z = exp(log z / 2), rsqrt z = exp(-log z / 2); sin and cos from
    exp(+-i z); tanh z = 1 - 2 / (exp(2 z) + 1); sigmoid z = 1 / (1 + exp(-z)); silu z = z sigmoid z;
    gelu_tanh z = z (1 + tanh(c (z + a z^3))) / 2. Principal branches, as torch's."""
    if kind == "exp":
        return _complex_exp(z)
    if kind == "log":
        return _complex_log(z)
    if kind in ("sqrt", "rsqrt"):
        return _complex_exp(_lin((0.5 if kind == "sqrt" else -0.5, _complex_log(z))))
    if kind in ("sin", "cos"):
        up, down = _complex_exp(_lin((1j, z))), _complex_exp(_lin((-1j, z)))
        return _lin((-0.5j, up), (0.5j, down)) if kind == "sin" else _lin((0.5, up), (0.5, down))
    if kind == "tanh":
        return _lin((1.0, _shift(_lin((0.0, z)), 1.0)),
                    (-2.0, _complex_reciprocal_of(_shift(_complex_exp(_lin((2.0, z))), 1.0))))
    if kind in ("sigmoid", "silu"):
        sg = _complex_reciprocal_of(_shift(_complex_exp(_lin((-1.0, z))), 1.0))
        return sg if kind == "sigmoid" else _complex.complex_product(_mul, z, sg)
    c, a = math.sqrt(2.0 / math.pi), 0.044715   # gelu_tanh
    cube = _complex.complex_product(_mul, _complex.complex_product(_mul, z, z), z)
    t = _complex_base(_lin((c, z), (c * a, cube)), "tanh")
    return _lin((0.5, _complex.complex_product(_mul, z, _shift(t, 1.0))))


def activation(x, kind):
    """Series of ``f(x)`` for ``kind`` in gelu, gelu_tanh, tanh, sigmoid, silu, exp, log, sin, cos,
    sqrt, rsqrt."""
    reason = why_ineligible(x, complex_ok=True, complex_base_ok=kind in COMPLEX_BASE_KINDS)
    if reason is not None:
        raise NotImplementedError(f"{kind}: {reason}")
    if _complex.has_complex_base(x):
        return _complex_base(x, kind)
    if _complex.has_complex(x):
        return _complex.at_real_nodes_below_autograd(activation, kind, x, kind)
    out = _ops.activation_series(_coeffs(x, x.degree), kind)
    return PolyTensor.from_stacked(out)


def backward(grad, saved, kind):
    """Gradient series ``grad * f'(x)`` of the native ``<kind>_backward`` operation.

    ``saved`` is the forward input for gelu, gelu_tanh and silu and the forward
    output for tanh and sigmoid, as the aten backward operations take them.
    """
    if kind not in BACKWARD_KINDS:
        raise NotImplementedError(f"{kind}_backward has no series kernel")
    reason = why_ineligible(grad, saved, complex_ok=True)
    if reason is not None:
        raise NotImplementedError(f"{kind}_backward: {reason}")
    if _complex.has_complex(grad, saved):
        return _complex.at_real_nodes_below_autograd(backward, f"{kind}_backward", grad, saved, kind)
    degree = next(x.degree for x in (grad, saved) if isinstance(x, PolyTensor))
    out = _ops.activation_series_backward(_coeffs(grad, degree), _coeffs(saved, degree), kind)
    return PolyTensor.from_stacked(out)
