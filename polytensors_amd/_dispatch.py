"""aten-level rules of ``PolyTensor`` (the ``__torch_dispatch__`` hook).

Only the rules the hot path needs exist here:
  * shape, view, copy and conversion operations, applied to every coefficient
    (as /root/reference/src/polytensors/_range_ops.py:224-257), and the
    factories autograd uses (_dispatch.py:769-790);
  * linear arithmetic: series +/- series, and +, -, *, / with an ordinary
    operand (the constant-operand fast path, _range_ops.py:109-132), sum and
    mean (_range_ops.py:178-193);
  * series (*) series and series / series (and ordinary / series), the
    elementwise Cauchy product and quotient kernel (_range_ops.py:133-149), and
    pow with a scalar exponent built from them (or from exp and log);
  * the matrix products mm/bmm/addmm/mv/dot, which run the Cauchy-product
    kernel (_range_ops.py:160-176 -> convolution(matrix=True), :78-84);
  * the elementwise activations gelu (erf and tanh forms), tanh, sigmoid,
    silu, exp, log, sin, cos, sqrt, rsqrt and the gelu/tanh/sigmoid/silu
    backward operations, which
    run the activation-series kernel (the reference's rules,
    /root/reference/src/polytensors/_plain.py:276-355 and
    /root/reference/src/polytensors/_dispatch.py:460-473,612-638).
Every other operation raises NotImplementedError (as the reference does for
operations without a rule, /root/reference/src/polytensors/_dispatch.py:852):
nonlinear series arithmetic outside the fused operations is not part of this
package.
"""

import torch
from torch.utils._python_dispatch import return_and_correct_aliasing

from ._tensor import PolyTensor
from . import _fused_activation, _fused_elementwise, _fused_matmul

aten = torch.ops.aten

_VIEW_OPS = {
    aten.t.default, aten.transpose.int, aten.permute.default, aten.view.default,
    aten._unsafe_view.default, aten.reshape.default, aten.flatten.using_ints, aten.slice.Tensor,
    aten.select.int, aten.unsqueeze.default, aten.squeeze.dim, aten.squeeze.dims, aten.squeeze.default,
    aten.expand.default, aten.alias.default, aten.unbind.int, aten.split.Tensor, aten.chunk.default,
    aten.narrow.default, aten.unfold.default, aten.diagonal.default, aten.as_strided.default,
    aten.view_as_real.default, aten.view_as_complex.default,
}
_COERCED_VIEWS = {aten.as_strided.default, aten.view_as_real.default, aten.view_as_complex.default}
_COPY_OPS = {
    aten.clone.default, aten.detach.default, aten._to_copy.default, aten.contiguous.default,
    aten.index_select.default, aten.gather.default, aten.index.Tensor, aten.flip.default,
    aten.roll.default, aten.repeat.default,
    # embedding of a series weight, per order (/root/reference/src/polytensors/_dispatch.py:530-532)
    aten.embedding.default,
    # the (linear) backward operations of views and gathers, per coefficient
    aten.slice_backward.default, aten.select_backward.default, aten.diagonal_backward.default,
    aten.index_add.default, aten.scatter_add.default, aten.unfold_backward.default,
}
# In-place arithmetic: the out-of-place rule, written into the target's coefficients
# (/root/reference/src/polytensors/_range_ops.py:95-103, write).
_IN_PLACE = {aten.add_.Tensor: aten.add.Tensor, aten.add_.Scalar: aten.add.Scalar,
             aten.sub_.Tensor: aten.sub.Tensor, aten.sub_.Scalar: aten.sub.Scalar,
             aten.mul_.Tensor: aten.mul.Tensor, aten.mul_.Scalar: aten.mul.Scalar,
             aten.div_.Tensor: aten.div.Tensor, aten.div_.Scalar: aten.div.Scalar}
_ADD = {aten.add.Tensor, aten.add.Scalar}
_SUB = {aten.sub.Tensor, aten.sub.Scalar}
_MUL = {aten.mul.Tensor, aten.mul.Scalar}
_DIV = {aten.div.Tensor, aten.div.Scalar}
_MATMUL = {aten.mm.default, aten.bmm.default, aten.mv.default, aten.dot.default, aten.matmul.default}
_ACTIVATION = {aten.tanh.default: "tanh", aten.sigmoid.default: "sigmoid", aten.silu.default: "silu",
               aten.exp.default: "exp", aten.log.default: "log", aten.sin.default: "sin", aten.cos.default: "cos",
               aten.sqrt.default: "sqrt", aten.rsqrt.default: "rsqrt"}
# (grad_output, output) for tanh/sigmoid, (grad_output, self) for silu
_ACTIVATION_BACKWARD = {aten.tanh_backward.default: "tanh", aten.sigmoid_backward.default: "sigmoid",
                        aten.silu_backward.default: "silu"}


def _gelu_kind(approximate):
    if approximate not in ("none", "tanh"):
        raise ValueError("GELU approximate must be 'none' or 'tanh'")
    return "gelu" if approximate == "none" else "gelu_tanh"


def _is_poly(x):
    return type(x) is PolyTensor


def _collect(x, out):
    if _is_poly(x):
        out.append(x)
    elif isinstance(x, (tuple, list)):
        for y in x:
            _collect(y, out)
    elif isinstance(x, dict):
        for y in x.values():
            _collect(y, out)


def _wrap(coeffs):
    return PolyTensor(tuple(coeffs), requires_grad=False)


def _wrap_views(coeffs):
    return PolyTensor._wrap(tuple(coeffs))


def _per_order(args, k):
    """The k-th coefficient of every PolyTensor in a nested argument structure."""
    if _is_poly(args):
        return args.coeffs[k]
    if isinstance(args, tuple):
        return tuple(_per_order(a, k) for a in args)
    if isinstance(args, list):
        return [_per_order(a, k) for a in args]
    if isinstance(args, dict):
        return {key: _per_order(v, k) for key, v in args.items()}
    return args


def _to_copy_kwargs(coefficient, kwargs):
    dtype = kwargs.get("dtype")
    if dtype is None or not coefficient.is_complex() or dtype.is_complex:
        return kwargs
    complex_dtype = {torch.float16: torch.complex32, torch.float32: torch.complex64,
                     torch.float64: torch.complex128}.get(dtype)
    if complex_dtype is None:
        raise TypeError(f"{dtype} cannot hold complex PolyTensor directions")
    return {**kwargs, "dtype": complex_dtype}


def _power(x, exponent):
    """Series of ``x ** exponent`` for a Python scalar exponent: an integral exponent by series
    products (square and multiply; a negative one as the quotient 1 / x^|n|), any other as
    exp(exponent * log x), as the reference's rules compose it from products, quotients and the
    exp/log series (/root/reference/src/polytensors/_range_ops.py:133-149, _plain.py:153-171)."""
    if isinstance(exponent, complex) or isinstance(exponent, bool):
        raise NotImplementedError("PolyTensor pow takes a real exponent")
    head = x.coeffs[0]
    if float(exponent).is_integer():
        n = int(exponent)
        if n == 0:
            return _wrap((torch.ones_like(head), *(torch.zeros_like(c) for c in x.coeffs[1:])))
        result, base, m = None, x, abs(n)
        while m:
            if m & 1:
                result = base if result is None else _fused_elementwise.binary(result, base, "mul")
            m >>= 1
            if m:
                base = _fused_elementwise.binary(base, base, "mul")
        if result is x:
            result = _wrap(c.clone() for c in x.coeffs)
        if n < 0:
            result = _fused_elementwise.binary(torch.ones_like(head), result, "div")
        return result
    if exponent in (0.5, -0.5):
        return _fused_activation.activation(x, "sqrt" if exponent > 0 else "rsqrt")
    logs = _fused_activation.activation(x, "log")
    return _fused_activation.activation(_wrap(c * exponent for c in logs.coeffs), "exp")


def dispatch(func, types, args=(), kwargs=None):
    kwargs = {} if kwargs is None else kwargs
    polys = []
    _collect(args, polys)
    _collect(kwargs, polys)
    if not polys:
        return func(*args, **kwargs)
    from ._plain import _plain_range, in_backward, plain_range_enabled

    if not plain_range_enabled() and in_backward():
        token = _plain_range.set(True)
        try:
            return _dispatch(func, types, args, kwargs, polys)
        finally:
            _plain_range.reset(token)
    return _dispatch(func, types, args, kwargs, polys)


def _dispatch(func, types, args, kwargs, polys):
    for p in polys:
        if not hasattr(p, "coeffs"):
            raise RuntimeError("PolyTensor wrapper reached dispatch without coefficient storage; "
                               "keep PolyTensor wrappers alive (PolyTensor.retain_wrappers())")
    degree = polys[0].degree
    if any(p.degree != degree for p in polys[1:]):
        raise ValueError("PolyTensor operands must have the same degree")
    count = degree + 1
    schema = getattr(func, "_schema", None)
    mutable = bool(getattr(schema, "is_mutable", False))
    if mutable and args and not _is_poly(args[0]):
        raise RuntimeError(f"cannot update a regular Tensor in-place with a PolyTensor ({func})")

    if func in _IN_PLACE:
        target = args[0]
        result = dispatch(_IN_PLACE[func], types, args, kwargs)
        for dest, src in zip(target.coeffs, result.coeffs):
            if src.is_complex() and not dest.is_complex():
                raise RuntimeError("cannot write complex PolyTensor coefficients into real storage")
            dest.copy_(src)
        return target

    if func in _VIEW_OPS:
        source = args[0]
        if len(polys) == 1 and source is polys[0]:
            rest = args[1:]
            results = [func(c, *rest, **kwargs) for c in source.coeffs]
        else:
            results = [func(*_per_order(args, k), **_per_order(kwargs, k)) for k in range(count)]
        # A view of each order lies inside that order's memory, so the views of well-formed
        # coefficients are disjoint, of one shape, dtype and device: wrapped as they are. The
        # views that may leave their coefficient's memory (as_strided) or change the dtype go
        # through the coercion rules.
        wrap = _wrap if func in _COERCED_VIEWS else _wrap_views
        if isinstance(results[0], (tuple, list)):
            out = type(results[0])(wrap([r[i] for r in results]) for i in range(len(results[0])))
        else:
            out = wrap(results)
        del source
        return return_and_correct_aliasing(func, args, kwargs, out)

    if func in _COPY_OPS:
        if func is aten._to_copy.default:
            results = [func(c, **_to_copy_kwargs(c, kwargs)) for c in args[0].coeffs]
        else:
            results = [func(*_per_order(args, k), **_per_order(kwargs, k)) for k in range(count)]
        return _wrap(results)

    if func in (aten.copy_.default,):
        target, source = args[0], args[1]
        sources = source.coeffs if _is_poly(source) else (source,) + (None,) * degree
        for dest, src in zip(target.coeffs, sources):
            if src is None:
                dest.zero_()
            else:
                if src.is_complex() and not dest.is_complex():
                    raise RuntimeError("cannot copy complex PolyTensor coefficients into real storage")
                dest.copy_(src)
        return target
    if func is aten.zero_.default:
        for c in args[0].coeffs:
            c.zero_()
        return args[0]

    # Autograd and optimizer plumbing (/root/reference/src/polytensors/_dispatch.py:769-790): a
    # constant fill is a constant series; empty/zero factories act on every coefficient.
    if func in (aten.ones_like.default, aten.full_like.default, aten.new_ones.default, aten.new_full.default):
        head = func(args[0].coeffs[0], *args[1:], **kwargs)
        return _wrap((head, *(torch.zeros_like(head) for _ in range(degree))))
    if func in (aten.zeros_like.default, aten.empty_like.default, aten.new_empty_strided.default,
                aten.new_empty.default, aten.new_zeros.default):
        return _wrap(func(c, *args[1:], **kwargs) for c in args[0].coeffs)
    if func is aten.fill_.Scalar:
        args[0].coeffs[0].fill_(args[1])
        for c in args[0].coeffs[1:]:
            c.zero_()
        return args[0]
    if func is aten.detach_.default:
        args[0]._set_coeffs(tuple(c.detach() for c in args[0].coeffs))
        return args[0]

    if func is aten.neg.default:
        return _wrap(-c for c in args[0].coeffs)
    if func is aten.rsub.Scalar:
        # other - alpha * x (/root/reference/src/polytensors/_range_ops.py:151-155)
        x, other = args[0], args[1]
        alpha = kwargs.get("alpha", 1)
        return _wrap((other - alpha * x.coeffs[0], *(-alpha * c for c in x.coeffs[1:])))
    if func is aten.reciprocal.default:
        # quotient(1, x) (/root/reference/src/polytensors/_range_ops.py:86-93,157-158)

        return _fused_elementwise.binary(torch.ones_like(args[0].coeffs[0]), args[0], "div")

    if func is aten.pow.Tensor_Scalar:
        return _power(args[0], args[1])

    if func in _ADD or func in _SUB:
        a, b = args[0], args[1]
        alpha = kwargs.get("alpha", 1)
        sign = alpha if func in _ADD else -alpha
        if _is_poly(a) and _is_poly(b):
            return _wrap(torch.add(x, y, alpha=sign) for x, y in zip(a.coeffs, b.coeffs))
        if _is_poly(a):
            return _wrap((torch.add(a.coeffs[0], b, alpha=sign), *(c.clone() for c in a.coeffs[1:])))
        return _wrap((torch.add(a, b.coeffs[0], alpha=sign), *(sign * c for c in b.coeffs[1:])))

    if func in _MUL or func in _DIV:
        a, b = args[0], args[1]
        if func in _DIV and kwargs.get("rounding_mode") is not None:
            raise NotImplementedError("PolyTensor does not implement rounded division")
        if (_is_poly(a) and _is_poly(b)) or (func in _DIV and _is_poly(b)):
            if not isinstance(a, torch.Tensor):
                a = torch.as_tensor(a, dtype=b.dtype, device=b.device)
            return _fused_elementwise.binary(a, b, "mul" if func in _MUL else "div")
        if _is_poly(a):
            return _wrap((c * b if func in _MUL else c / b) for c in a.coeffs)
        return _wrap(a * c for c in b.coeffs)

    if func in (aten.sum.default, aten.sum.dim_IntList, aten.mean.default, aten.mean.dim):
        return _wrap(func(*_per_order(args, k), **kwargs) for k in range(count))

    if func in _MATMUL or func is aten.addmm.default:
        return _fused_matmul.from_dispatch(func, args, kwargs)

    if func in _ACTIVATION or func is aten.gelu.default:
        if func is aten.gelu.default:
            kind = _gelu_kind(args[1] if len(args) > 1 else kwargs.get("approximate", "none"))
        else:
            kind = _ACTIVATION[func]
        return _fused_activation.activation(args[0], kind)

    if func in _ACTIVATION_BACKWARD or func is aten.gelu_backward.default:
        if func is aten.gelu_backward.default:
            kind = _gelu_kind(args[2] if len(args) > 2 else kwargs.get("approximate", "none"))
        else:
            kind = _ACTIVATION_BACKWARD[func]
        return _fused_activation.backward(args[0], args[1], kind)

    raise NotImplementedError(
        f"PolyTensor has no rule for {func}: polytensors_amd implements the fused Taylor hot path "
        "(matmul, scaled_dot_product_attention, rms_norm/layer_norm, cross_entropy, elementwise "
        "activations) and linear shape/arithmetic operations only")
