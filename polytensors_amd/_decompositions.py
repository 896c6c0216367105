"""Routing of composite operations on PolyTensors to the fused kernels.

Mirrors ``maybe_decompose`` of the reference
(/root/reference/src/polytensors/_decompositions.py:52-99): rms_norm,
cross_entropy and scaled_dot_product_attention are intercepted above autograd
and sent to their fused entry point when ``eligible``; LayerNorm and the
matrix products (torch.matmul, @, mm, bmm, F.linear) are intercepted here too,
so they reach the Cauchy-product kernel without the copies the
CompositeImplicit matmul decomposition makes. Where the reference falls back to
its general series rules, this package raises NotImplementedError with the
reason (it has no general rules).
"""

import torch
import torch.nn.functional as F

from ._tensor import PolyTensor
from . import _fused_attention, _fused_cross_entropy, _fused_matmul, _fused_norm

_RMS_NORM = frozenset((F.rms_norm, torch.rms_norm))
_LAYER_NORM = frozenset((F.layer_norm, torch.layer_norm))
_ATTENTION = frozenset((F.scaled_dot_product_attention,))
_CROSS_ENTROPY = frozenset((F.cross_entropy,))
_CROSS_ENTROPY_ARGS = ("input", "target", "weight", "size_average", "ignore_index", "reduce", "reduction",
                       "label_smoothing")
_MATMUL = frozenset((torch.matmul, torch.Tensor.matmul, torch.Tensor.__matmul__, torch.Tensor.__rmatmul__,
                     torch.mm, torch.Tensor.mm, torch.bmm, torch.Tensor.bmm, F.linear))


def _has_poly(values):
    return any(isinstance(v, PolyTensor) for v in values)


def _needs_grad(args, kwargs):
    from ._gate import wrapper_grad

    return wrapper_grad(*args, *kwargs.values())


def maybe_decompose(function, args, kwargs):
    """The fused result, or NotImplemented to continue with ordinary dispatch."""
    if function in _RMS_NORM or function in _LAYER_NORM:
        layer = function in _LAYER_NORM
        names = ("input", "normalized_shape", "weight", "bias", "eps") if layer else \
            ("input", "normalized_shape", "weight", "eps")
        bound = dict(zip(names, args))
        bound.update(kwargs)
        if not _has_poly((bound.get("input"), bound.get("weight"), bound.get("bias"))):
            return NotImplemented

        shape = tuple(bound["normalized_shape"]) if not isinstance(bound["normalized_shape"], int) \
            else (bound["normalized_shape"],)
        if layer:
            return _fused_norm.layer_norm(bound["input"], shape, bound.get("weight"), bound.get("bias"),
                                          bound.get("eps", 1e-5))
        return _fused_norm.rms_norm(bound["input"], shape, bound.get("weight"), bound.get("eps"))

    if function in _CROSS_ENTROPY:
        bound = dict(zip(_CROSS_ENTROPY_ARGS, args))
        bound.update(kwargs)
        if not _has_poly(bound.values()):
            return NotImplemented
        if bound.get("size_average") is not None or bound.get("reduce") is not None:
            raise NotImplementedError("cross_entropy: the deprecated size_average/reduce arguments are not supported")

        loss = _fused_cross_entropy.fused_or_raise(
            bound["input"], bound["target"], weight=bound.get("weight"),
            ignore_index=bound.get("ignore_index", -100), reduction=bound.get("reduction", "mean"),
            label_smoothing=bound.get("label_smoothing", 0.0))
        # F.cross_entropy returns the input's dtype.
        return loss if loss.dtype == bound["input"].dtype else loss.to(bound["input"].dtype)

    if function in _ATTENTION:
        names = ("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale", "enable_gqa")
        bound = dict(zip(names, args))
        bound.update(kwargs)
        if not _has_poly(bound.values()):
            return NotImplemented

        _fused_attention.require_eligible(bound["query"], bound["key"], bound["value"], bound.get("attn_mask"),
                                          bound.get("dropout_p", 0.0), bound.get("is_causal", False),
                                          bound.get("enable_gqa", False))
        return _fused_attention.attention_checked(bound["query"], bound["key"], bound["value"],
                                          attn_mask=bound.get("attn_mask"), is_causal=bound.get("is_causal", False),
                                          scale=bound.get("scale"))

    if function in _MATMUL:
        if _needs_grad(args, kwargs):
            # Let autograd record mm/bmm/addmm; they reach the kernel through __torch_dispatch__,
            # and so do the products of their backward.
            return NotImplemented
        if function is F.linear:
            names = ("input", "weight", "bias")
            bound = dict(zip(names, args))
            bound.update(kwargs)
            return _fused_matmul.linear(bound["input"], bound["weight"], bound.get("bias"))
        if function is torch.Tensor.__rmatmul__:
            return _fused_matmul.matmul(args[1], args[0])
        return _fused_matmul.matmul(args[0], args[1])
    return NotImplemented
