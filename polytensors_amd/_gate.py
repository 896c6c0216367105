"""Conditions every fused entry point shares, as reason strings.

A ``None`` reason means the call can run on the gfx950 kernels. The reference's
``eligible`` functions (/root/reference/src/polytensors/_fused_attention.py:227-256,
_fused_norm.py:11-21, _fused_cross_entropy.py:131-147) return False and let the
caller use the general rules; this package has no general rules, so callers
turn a reason into NotImplementedError. A missing kernel library on a HIP
device is never a reason: it raises LibraryMissingError.
"""

import torch

from . import _lib
from ._plain import plain_range_enabled
from ._tensor import PolyTensor, _coefficient_autograd_enabled

MAX_DEGREE = 8
# the elementwise kernels (activations, series product and quotient) and the Cauchy matmul, which
# runs above MAX_DEGREE in blocks of orders
MAX_ELEMENTWISE_DEGREE = 16
_REAL_OF = {torch.complex32: torch.float16, torch.complex64: torch.float32, torch.complex128: torch.float64}


def real_dtype(dtype):
    """The real dtype of a (possibly complex) coefficient dtype."""
    return _REAL_OF.get(dtype, dtype)


def coefficients(x, degree):
    """The coefficient tuple of a PolyTensor, or (x,) for an ordinary tensor (a plain operand)."""
    if isinstance(x, PolyTensor):
        return tuple(x.coeffs)
    return (x,)


def common_reason(values, *, allow_plain_grad=False, below_autograd=False, complex_ok=False,
                  complex_base_ok=False, max_degree=MAX_DEGREE):
    """Shared conditions over the tensor operands of one fused call.

    ``below_autograd``: the call comes from ``__torch_dispatch__``, under the
    autograd layer, which has already recorded the operation's native backward;
    operands requiring grad are then fine (the backward operations have rules too).
    ``complex_ok``: the entry point runs complex directions through its real kernel
    (polytensors_amd._complex). ``complex_base_ok``: it also takes a complex constant
    term, in complex arithmetic (the bilinear products); reverse mode at the wrapper
    level, which would follow torch's conjugating complex autograd, is refused there.
    ``max_degree``: the entry point's largest degree (MAX_DEGREE for the MFMA and row
    kernels, MAX_ELEMENTWISE_DEGREE for the elementwise ones and the matmul).
    """
    tensors = [v for v in values if isinstance(v, torch.Tensor)]
    polys = [v for v in tensors if isinstance(v, PolyTensor)]
    if not polys:
        return "no PolyTensor operand"
    if not plain_range_enabled():
        return ("extended-range (default) mode is not implemented by polytensors_amd; "
                "run the series inside PolyTensor.plain_range()")
    degree = polys[0].degree
    if any(p.degree != degree for p in polys):
        return "PolyTensor operands must have the same degree"
    if degree > max_degree:
        return f"degree {degree} exceeds this kernel's maximum {max_degree}"
    plain = [t for t in tensors if not isinstance(t, PolyTensor)]
    # A series' orders share one device, its higher orders one dtype (the coercion rules of
    # PolyTensor), so the constant and the last order stand for every coefficient below.
    complex_dirs = any(p.coeffs[-1].is_complex() for p in polys) or any(t.is_complex() for t in plain)
    if _coefficient_autograd_enabled.get():
        # the custom ops carry coefficient-level autograd (polytensors_amd._ops); the wrappers
        # stay outside autograd, so only wrapper gradients are refused
        if any(p.requires_grad for p in polys):
            return ("coefficient_autograd differentiates the coefficient tensors: build the PolyTensor "
                    "wrappers with requires_grad=False")
    elif torch.is_grad_enabled() and not below_autograd:
        grads = any(t.requires_grad for t in tensors) or any(
            c.requires_grad for p in polys for c in p.coeffs)
        if grads and not allow_plain_grad:
            return ("this operation has no wrapper-level gradient; use torch.no_grad(), or build a "
                    "coefficient graph inside PolyTensor.coefficient_autograd()")
    if any(t.is_complex() for t in plain) or any(p.coeffs[0].is_complex() for p in polys):
        if not complex_base_ok:
            return ("a complex constant term (complex base) is implemented for the bilinear products "
                    "(matmul, series product and quotient, integer powers) only; this kernel is real-valued, "
                    "complex directions need a real base")
        if wrapper_grad(*tensors) or (torch.is_grad_enabled() and not _coefficient_autograd_enabled.get() and
                                      any(c.requires_grad for p in polys for c in p.coeffs)):
            return ("reverse mode with a complex constant term (torch's conjugating complex autograd) is not "
                    "implemented; use coefficient_autograd or complex directions over a real base")
    if not complex_ok and complex_dirs:
        return "complex directions are not implemented for this operation"
    if not (all(p.coeffs[0].is_cuda for p in polys) and all(t.is_cuda for t in plain)):
        return "polytensors_amd runs on HIP (cuda) devices only"
    _lib.load()   # loud failure if the kernels are not built
    return None


def coefficient_graph(*values):
    """Whether this call builds a coefficient-level autograd graph: coefficient_autograd is on,
    grad mode is enabled and some coefficient (or ordinary tensor operand) requires grad."""
    if not (_coefficient_autograd_enabled.get() and torch.is_grad_enabled()):
        return False
    return any((c.requires_grad for c in v.coeffs) if isinstance(v, PolyTensor) else
               (isinstance(v, torch.Tensor) and v.requires_grad) for v in values)


def wrapper_grad(*values):
    """Whether this call is recorded by wrapper-level (PolyTensor) autograd: grad mode is enabled,
    coefficient_autograd is off and some operand requires grad."""
    if _coefficient_autograd_enabled.get() or not torch.is_grad_enabled():
        return False
    return any(isinstance(v, torch.Tensor) and v.requires_grad for v in values)
