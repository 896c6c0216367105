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

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)
BACKWARD_KINDS = ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu")


def why_ineligible(*operands, complex_ok=False):
    # Reached from __torch_dispatch__ only: autograd above has recorded the native
    # backward operation (gelu_backward, tanh_backward, ...), which routes here too.
    reason = _gate.common_reason(operands, below_autograd=True, complex_ok=complex_ok,
                                 max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    polys = [x for x in operands if isinstance(x, PolyTensor)]
    dtype = polys[0].dtype
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


def activation(x, kind):
    """Series of ``f(x)`` for ``kind`` in gelu, gelu_tanh, tanh, sigmoid, silu, exp, log, sin, cos,
    sqrt, rsqrt."""
    reason = why_ineligible(x, complex_ok=True)
    if reason is not None:
        raise NotImplementedError(f"{kind}: {reason}")
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
