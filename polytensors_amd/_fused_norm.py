"""Fused RMSNorm / LayerNorm series (degrees up to 8 in one kernel, 9..16 composed) on gfx950.

``rms_norm`` mirrors /root/reference/src/polytensors/_fused_norm.py:63-69: the
normalisation runs in one kernel pass and ``eps`` defaults to
``finfo(dtype).eps`` (:64). The reference then multiplies by the weight as a
separate PolyTensor operation (:69); here an ordinary or series weight of the
normalised shape and input dtype is applied inside the kernel, and any other
weight falls back to that separate multiply. Half and bfloat16 inputs compute in
float32, float64 in float64 (as the reference's kernel, _norm_kernels.py:12-13).

``layer_norm`` has no reference counterpart (native layer norm has no rule
there, /root/reference/docs/notes.md:33-35); it is the series of
``(x - mean(x)) * rsqrt(mean((x - mean(x))**2) + eps) * w + b``.
"""

import math

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def why_ineligible(input, normalized_shape, weight=None, bias=None, allow_grad=False,
                   max_degree=_gate.MAX_DEGREE):
    """Why the norm kernel cannot take this call (None if it can); ``max_degree`` the composed
    path's limit for degrees above the kernel's."""
    reason = _gate.common_reason((input, weight, bias), allow_plain_grad=allow_grad, complex_ok=True,
                                 max_degree=max_degree)
    if reason is not None:
        return reason
    if not isinstance(input, torch.Tensor) or input.dtype not in _DTYPES:
        return "input must be a float16/bfloat16/float32/float64 tensor"
    polys = [x for x in (input, weight, bias) if isinstance(x, PolyTensor)]
    if any(_gate.real_dtype(c.dtype) != input.dtype for p in polys for c in p.coeffs):
        return "all series coefficients must have the input's dtype"
    shape = tuple(normalized_shape)
    if not shape or tuple(input.shape[-len(shape):]) != shape:
        return "normalized_shape must match the input's trailing dimensions"
    if math.prod(shape) == 0 or input.numel() == 0:
        return "empty normalisation"
    return None


def eligible(input, normalized_shape, weight=None, bias=None):
    return why_ineligible(input, normalized_shape, weight, bias) is None


def _series_coeffs(x, degree):
    if isinstance(x, PolyTensor):
        return [c.contiguous() for c in x.coeffs]
    return [x.contiguous()] + [torch.zeros_like(x, memory_format=torch.contiguous_format)
                               for _ in range(degree)]


def _affine_coeffs(a, input, shape):
    """Kernel-side coefficients of a weight/bias, or None if it must be applied separately."""
    if a is None:
        return []
    coeffs = a.coeffs if isinstance(a, PolyTensor) else (a,)
    if any(c.dtype != input.dtype or tuple(c.shape) != shape or c.device != input.device for c in coeffs):
        return None
    return [c.contiguous().reshape(-1) for c in coeffs]


def _needs_grad(*values):
    return _gate.wrapper_grad(*values)


class _SeriesNorm(torch.autograd.Function):
    """The normalization (no affine terms) with its degree-K gradient series.

    As /root/reference/src/polytensors/_fused_norm.py:43-60 (_SeriesNorm): the
    forward kernel, and a backward kernel computing J(x(t))^T g(t); the weight
    and bias are separate operations under autograd, so their gradients follow
    from the elementwise rules.
    """

    @staticmethod
    def forward(ctx, input, shape, eps, layer):
        ctx.save_for_backward(input)
        ctx.shape, ctx.eps, ctx.layer = shape, eps, layer
        x = _series_coeffs(input, input.degree)
        return _from_stacked(_ops.norm_series(x, [], [], math.prod(shape), eps, layer))

    @staticmethod
    def backward(ctx, gradient):
        from ._plain import _plain_range

        if torch.is_grad_enabled():
            raise NotImplementedError("second-order reverse mode through the fused norm is not implemented")
        (input,) = ctx.saved_tensors
        token = _plain_range.set(True)   # the engine's thread does not see the caller's context
        try:
            x = _series_coeffs(input, input.degree)
            g = _series_coeffs(gradient, input.degree)
            dx = _from_stacked(_ops.norm_series_backward(x, g, math.prod(ctx.shape), ctx.eps, ctx.layer))
        finally:
            _plain_range.reset(token)
        return dx, None, None, None


def _from_stacked(stacked):
    return PolyTensor.from_stacked(stacked)


def _composed(input, shape, weight, bias, eps, layer):
    """Degrees 9..16, above the row kernel's register plan (K+1 <= 9 accumulator sets).

    The reference's decomposition of the norm (/root/reference/src/polytensors/
    _decompositions.py:14-22): ``x * rsqrt(mean(x*x) + eps)``, layer_norm centring x first,
    in series operations: the products and rsqrt run the elementwise series kernels (to degree
    16) and the means act on each coefficient.
    """
    dims = tuple(range(-len(shape), 0))
    x = input
    if layer:
        x = x - x.mean(dim=dims, keepdim=True)
    y = x * ((x * x).mean(dim=dims, keepdim=True) + eps).rsqrt()
    if weight is not None:
        y = y * weight
    if layer and bias is not None:
        y = y + bias
    return y


def _run(input, normalized_shape, weight, bias, eps, layer):
    shape = tuple(normalized_shape)
    degree = max((x.degree for x in (input, weight, bias) if isinstance(x, PolyTensor)), default=0)
    if degree > _gate.MAX_DEGREE and isinstance(input, PolyTensor):
        reason = why_ineligible(input, shape, weight, bias, allow_grad=_needs_grad(input, weight, bias),
                                max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
        if reason is not None:
            raise NotImplementedError(f"{'layer_norm' if layer else 'rms_norm'}: {reason}")
        return _composed(input, shape, weight, bias, eps, layer)
    grads = _needs_grad(input, weight, bias)
    reason = why_ineligible(input, shape, weight, bias, allow_grad=grads)
    if reason is not None:
        raise NotImplementedError(f"{'layer_norm' if layer else 'rms_norm'}: {reason}")
    if _complex.has_complex(input, weight, bias):
        return _complex.at_real_nodes(_run, "layer_norm" if layer else "rms_norm", input, normalized_shape,
                                      weight, bias, eps, layer)
    if grads:
        if not isinstance(input, PolyTensor):
            raise NotImplementedError("reverse mode through the fused norm needs a PolyTensor input")
        result = _SeriesNorm.apply(input, shape, float(eps), layer)
        if weight is not None:
            result = result * weight
        if layer and bias is not None:
            result = result + bias
        return result
    degree = next(x.degree for x in (input, weight, bias) if isinstance(x, PolyTensor))
    x = _series_coeffs(input, degree)
    w = _affine_coeffs(weight, input, shape)
    b = _affine_coeffs(bias, input, shape) if layer else []
    # a coefficient graph differentiates the affine terms as separate series operations
    fused_affine = w is not None and b is not None and not _gate.coefficient_graph(input, weight, bias)
    out = _ops.norm_series(x, w if fused_affine else [], b if fused_affine else [], math.prod(shape),
                           float(eps), layer)
    result = PolyTensor.from_stacked(out)
    if not fused_affine:
        if weight is not None:
            result = result * weight
        if layer and bias is not None:
            result = result + bias
    return result


def rms_norm(input, normalized_shape, weight=None, eps=None):
    """Degree-K series of ``torch.nn.functional.rms_norm``."""
    eps = torch.finfo(input.dtype).eps if eps is None else eps
    return _run(input, normalized_shape, weight, None, eps, layer=False)


def layer_norm(input, normalized_shape, weight=None, bias=None, eps=1e-5):
    """Degree-K series of ``torch.nn.functional.layer_norm``."""
    return _run(input, normalized_shape, weight, bias, eps, layer=True)
