"""Elementwise product and quotient of two series (any degree up to 16) on gfx950.

The reference multiplies and divides series elementwise by its general rules
(/root/reference/src/polytensors/_range_ops.py:133-149): the Cauchy product
(_plain.py:118-128) and the quotient recurrence (_range_ops.py:86-93). An
ordinary operand of ``*`` or ``/ ordinary`` takes the constant-operand path
(:109-132) in ``_dispatch``; this module handles series (*) series, series /
series and ordinary / series. Operands broadcast as in torch (materialised
when their shapes differ). Reached from ``__torch_dispatch__``, under autograd.
"""

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def why_ineligible(a, b):
    reason = _gate.common_reason((a, b), below_autograd=True, complex_ok=True, complex_base_ok=True,
                                 max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    coeffs = [c for x in (a, b) for c in _gate.coefficients(x, 0)]
    dtype = _gate.real_dtype(coeffs[0].dtype)
    if dtype not in _DTYPES or any(_gate.real_dtype(c.dtype) != dtype for c in coeffs):
        return "series operands must share one float16/bfloat16/float32/float64 dtype"
    return None


def binary(a, b, op):
    """Series of ``a * b`` (op "mul") or ``a / b`` (op "div")."""
    reason = why_ineligible(a, b)
    if reason is not None:
        raise NotImplementedError(f"series {op}: {reason}")
    if _complex.has_complex_base(a, b):
        mul = lambda x, y: binary(x, y, "mul")   # noqa: E731
        if op == "mul":
            return _complex.complex_product(mul, a, b)
        return _complex.complex_quotient(lambda x, y: binary(x, y, "div"), mul, a, b)
    if _complex.has_complex(a, b):
        if op == "mul":
            return _complex.bilinear(binary, "series mul", a, b, op)
        return _complex.at_real_nodes_below_autograd(binary, "series div", a, b, op)
    degree = next(x.degree for x in (a, b) if isinstance(x, PolyTensor))
    shape = torch.broadcast_shapes(a.shape, b.shape)

    def series(x):
        coeffs = list(_gate.coefficients(x, degree))
        coeffs = [c.expand(shape).contiguous() for c in coeffs]
        return coeffs + [torch.zeros_like(coeffs[0]) for _ in range(degree + 1 - len(coeffs))]

    return PolyTensor.from_stacked(_ops.series_binary(series(a), series(b), op))
