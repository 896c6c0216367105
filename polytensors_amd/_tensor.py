"""``PolyTensor``: a truncated power series of tensors in one scalar variable.

The public surface mirrors the reference's class
(/root/reference/src/polytensors/_tensor.py:23-418): construction from K+1
coefficients with the same coercion rules (:38-96), ``.coeffs``, ``.value``,
``.tangent``, ``.degree``, ``constant``, the context managers
``retain_wrappers``, ``plain_range``, ``fused_attention``,
``fused_cross_entropy``, ``coefficient_autograd``, the static
``cross_entropy``, and the two routing hooks ``__torch_function__`` (composite
operations, :345-368) and ``__torch_dispatch__`` (aten operations, :370-418).

What differs is what sits behind the hooks: the four hot-path operations
(Cauchy-product matmul, scaled-dot-product attention, RMSNorm/LayerNorm,
cross entropy) run the gfx950 kernels at any degree up to 8 on HIP devices,
and there are no general series rules: a call the kernels cannot take raises
``NotImplementedError`` naming the reason instead of decomposing.
"""

import contextlib
import contextvars
import operator

import torch

_retention_scopes = contextvars.ContextVar("polytensors_amd_retention_scopes", default=())
_coefficient_autograd_enabled = contextvars.ContextVar("polytensors_amd_coefficient_autograd", default=False)
_DK = torch._C.DispatchKey
_COEFFICIENT_AUTOGRAD_KEYS = (_DK.Conjugate, _DK.Negative, _DK.ADInplaceOrView, _DK.Autograd,
                              _DK.AutogradFunctionality, _DK.AutogradOther, _DK.AutogradCPU, _DK.AutogradCUDA)
_COMPLEX_OF = {torch.float16: torch.complex32, torch.float32: torch.complex64, torch.float64: torch.complex128}


def _extent(t):
    """[start, end) byte addresses of a strided tensor's elements (conservative for gaps)."""
    n = t.numel()
    if n == 0:
        return 0, 0
    size = t.element_size()
    start = t.data_ptr()
    if t.is_contiguous():
        return start, start + n * size
    span = 1 + sum((d - 1) * abs(st) for d, st in zip(t.shape, t.stride()))
    start -= size * sum((d - 1) * abs(st) for d, st in zip(t.shape, t.stride()) if st < 0)
    return start, start + span * size


def _overlaps(a, b):
    """Whether two coefficients may share memory.

    ``torch._C._overlaps`` (which the reference uses, _tensor.py:93,124) reports any two views of
    one storage as overlapping, so it would clone every order of a coefficient-stacked buffer.
    This compares the byte addresses the two tensors span instead (live allocations never share
    addresses): exact for the disjoint slices of a stacked [K+1, ...] buffer, conservative for
    interleaved strided views.
    """
    if a.device != b.device:
        return False
    (s0, e0), (s1, e1) = _extent(a), _extent(b)
    return s0 < e1 and s1 < e0


def _as_coefficient(value, like):
    if isinstance(value, torch.Tensor):
        return value
    probe = torch.as_tensor(value)
    return torch.as_tensor(value, device=like.device, dtype=torch.promote_types(like.dtype, probe.dtype))


def _coerce_coeffs(coeffs, degree=None):
    """Normalise a coefficient sequence (the rules of _tensor.py:38-96 of the reference)."""
    if isinstance(coeffs, PolyTensor):
        coeffs = coeffs.coeffs
    coeffs = tuple(coeffs)
    if degree is None and _well_formed(coeffs):
        return coeffs
    if not coeffs:
        raise ValueError("at least one coefficient is required")
    if degree is not None:
        if isinstance(degree, bool):
            raise TypeError("degree must be a nonnegative integer")
        degree = operator.index(degree)
        if degree < 0:
            raise ValueError("degree must be nonnegative")
    head = coeffs[0]
    if not isinstance(head, torch.Tensor):
        head = torch.as_tensor(head)
        if not (head.is_floating_point() or head.is_complex()):
            head = head.to(torch.get_default_dtype())
    coeffs = (head,) + tuple(_as_coefficient(c, head) for c in coeffs[1:])
    for c in coeffs:
        if isinstance(c, PolyTensor):
            raise TypeError("nested PolyTensor coefficients are not supported")
        if c.layout != torch.strided:
            raise TypeError("coefficients must be dense strided tensors")
        if not (c.is_floating_point() or c.is_complex()):
            raise TypeError("tensor coefficients must have floating-point or complex dtype")
        if c.device != head.device:
            raise ValueError("all coefficients must be on the same device")
    common = coeffs[0].dtype
    for c in coeffs[1:]:
        common = torch.promote_types(common, c.dtype)
    real = torch.empty((), dtype=common).real.dtype
    complex_directions = any(c.is_complex() for c in coeffs[1:])
    coeffs = tuple(c.to(common if (c.is_complex() or (k > 0 and complex_directions)) else real)
                   for k, c in enumerate(coeffs))
    if degree is not None:
        if degree < len(coeffs) - 1:
            raise ValueError("degree must be at least the degree of coeffs")
        template = coeffs[-1] if len(coeffs) > 1 else coeffs[0]
        coeffs = coeffs + tuple(torch.zeros_like(template) for _ in range(degree + 1 - len(coeffs)))
    shape = torch.broadcast_shapes(*(c.shape for c in coeffs))
    coeffs = tuple(c if c.shape == shape else c.expand(shape).clone() for c in coeffs)
    # Orders must not share memory: an in-place update of one order would
    # otherwise change another.
    kept = []
    for c in coeffs:
        if any(_overlaps(c, other) for other in kept):
            c = c.clone()
        kept.append(c)
    return tuple(kept)


def _well_formed(coeffs):
    """True when ``coeffs`` already satisfy every coercion rule (the common case for kernel outputs)."""
    if not coeffs:
        return False
    head = coeffs[0]
    if type(head) is not torch.Tensor or head.layout != torch.strided:
        return False
    if not (head.dtype.is_floating_point or head.dtype.is_complex):
        return False
    higher = None
    for c in coeffs[1:]:
        if type(c) is not torch.Tensor or c.layout != torch.strided:
            return False
        if c.shape != head.shape or c.device != head.device:
            return False
        if higher is None:
            higher = c.dtype
            if higher != head.dtype and _COMPLEX_OF.get(head.dtype) != higher:
                return False
        elif c.dtype != higher:
            return False
    for i in range(1, len(coeffs)):
        for j in range(i):
            if _overlaps(coeffs[i], coeffs[j]):
                return False
    return True


class PolyTensor(torch.Tensor):
    """A truncated tensor-valued power series ``sum_k coeffs[k] * t**k``.

    ``PolyTensor((x, v), degree=n)`` represents ``x + t*v`` through order ``n``.
    After a supported function ``f``, coefficient ``k`` is the order-k
    directional derivative of ``f`` at ``x`` along ``v`` divided by ``k!``.
    """

    @staticmethod
    def __new__(cls, coeffs, *, degree=None, requires_grad=False):
        return cls._wrap(_coerce_coeffs(coeffs, degree), requires_grad)

    def __init__(self, coeffs, *, degree=None, requires_grad=False):
        pass

    @classmethod
    def from_stacked(cls, stacked, requires_grad=False):
        """Wrap a coefficient-stacked ``[K+1, ...]`` tensor without copying.

        The orders of a contiguous real stack (every kernel's output) are disjoint slices of one
        shape, device and dtype, so they satisfy every coercion rule as they are and skip the
        checks; any other stack goes through them."""
        coeffs = tuple(stacked.unbind(0))
        if (type(stacked) is torch.Tensor and stacked.layout == torch.strided and stacked.is_contiguous()
                and stacked.dtype.is_floating_point and stacked.dim() >= 1 and stacked.shape[0] >= 1):
            return cls._wrap(coeffs, requires_grad)
        return cls(coeffs, requires_grad=requires_grad)

    @classmethod
    def _wrap(cls, coeffs, requires_grad=False):
        """A PolyTensor over coefficients already known to satisfy the coercion rules."""
        head = coeffs[0]
        out = torch.Tensor._make_wrapper_subclass(
            cls, head.shape, strides=head.stride(), storage_offset=head.storage_offset(),
            dtype=head.dtype, layout=head.layout, device=head.device, requires_grad=requires_grad)
        out.coeffs = coeffs
        out.degree = len(coeffs) - 1
        for scope in _retention_scopes.get():
            scope.append(out)
        return out

    def _set_coeffs(self, coeffs):
        self.coeffs = _coerce_coeffs(coeffs)
        self.degree = len(self.coeffs) - 1

    @property
    def value(self):
        return self.coeffs[0]

    @property
    def tangent(self):
        """Coefficient 1 (the first directional derivative)."""
        if self.degree == 0:
            raise ValueError("a degree-zero PolyTensor has no tangent")
        return self.coeffs[1]

    @classmethod
    def constant(cls, x, degree):
        """A series whose higher coefficients are all zero."""
        return cls((x,), degree=degree)

    @classmethod
    @contextlib.contextmanager
    def retain_wrappers(cls, isolated=False):
        """Keep every PolyTensor created in the scope alive until the scope exits.

        Nested scopes also retain into their outer scopes unless ``isolated``.
        The yielded list is for diagnostics (e.g. counting retained wrappers).
        """
        refs = []
        token = _retention_scopes.set((refs,) if isolated else (*_retention_scopes.get(), refs))
        try:
            yield refs
        finally:
            _retention_scopes.reset(token)
            refs.clear()

    @classmethod
    @contextlib.contextmanager
    def plain_range(cls):
        """Ordinary floating-point range for coefficient arithmetic (required by the fused kernels)."""
        from ._plain import _plain_range

        token = _plain_range.set(True)
        try:
            yield
        finally:
            _plain_range.reset(token)

    @classmethod
    @contextlib.contextmanager
    def fused_attention(cls, enabled=True):
        """Enable or disable the fused attention kernel (default: enabled)."""
        from ._fused_attention import _enabled

        token = _enabled.set(bool(enabled))
        try:
            yield
        finally:
            _enabled.reset(token)

    @classmethod
    @contextlib.contextmanager
    def fused_cross_entropy(cls, enabled=True):
        """Enable or disable the fused cross-entropy kernel (default: enabled)."""
        from ._fused_cross_entropy import _enabled

        token = _enabled.set(bool(enabled))
        try:
            yield
        finally:
            _enabled.reset(token)

    @classmethod
    @contextlib.contextmanager
    def coefficient_autograd(cls):
        """Build an ordinary autograd graph for the coefficient tensors
        (/root/reference/src/polytensors/_tensor.py:291-323).

        Make the coefficients autograd leaves and wrap them with ``requires_grad=False``;
        inside the scope every operation records ``grad_fn`` nodes on the coefficients,
        the fused kernels included (their coefficient gradients are the backward
        kernels' gradient series of the reversed cotangents). The gradient of loss
        coefficient k with respect to a parameter's coefficient 0 is coefficient k of
        the parameter's gradient series. Complex directions are not supported here.
        """
        token = _coefficient_autograd_enabled.set(True)
        try:
            yield
        finally:
            _coefficient_autograd_enabled.reset(token)

    @staticmethod
    def cross_entropy(logits, target, softcap=None, ignore_index=-100, reduction="mean"):
        """Cross entropy of (N, C) logits; returns at least float32 (as the reference's
        /root/reference/src/polytensors/_fused_cross_entropy.py:173-187)."""
        from ._fused_cross_entropy import cross_entropy

        return cross_entropy(logits, target, softcap=softcap, ignore_index=ignore_index, reduction=reduction)

    def backward(self, gradient=None, retain_graph=None, create_graph=False, inputs=None):
        """Reverse mode through the series (/root/reference/src/polytensors/_tensor.py:325-338).

        A scalar output seeds the cotangent series (1, 0, ..., 0); an ordinary
        ``gradient`` is lifted to a constant series. Gradients of the fused
        operations are their degree-K backward kernels.
        """
        if gradient is None:
            if self.numel() != 1:
                raise RuntimeError("grad can be implicitly created only for scalar outputs")
            if self.is_complex():
                raise RuntimeError("an explicit gradient is required for a complex output")
            gradient = PolyTensor.constant(torch.ones_like(self.value), self.degree)
        elif not isinstance(gradient, PolyTensor):
            gradient = PolyTensor.constant(gradient, self.degree)
        torch.autograd.backward(self, gradient, retain_graph=retain_graph, create_graph=create_graph,
                                inputs=inputs)

    def __repr__(self):
        if not hasattr(self, "coeffs"):
            return f"PolyTensor(<uninitialized>, requires_grad={self.requires_grad})"
        return f"PolyTensor({self.coeffs}, requires_grad={self.requires_grad})"

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = {} if kwargs is None else kwargs
        # The routed paths run with this hook disabled too: their reads of the operands' shape,
        # dtype and flags then go straight to the tensor instead of back through this method, and
        # the torch calls they make on PolyTensors (none of them routed) reach __torch_dispatch__
        # as they would from the default branch.
        with torch._C.DisableTorchFunctionSubclass():
            result = maybe_decompose(func, args, kwargs)
            if result is not NotImplemented:
                return result
            return func(*args, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        if _coefficient_autograd_enabled.get():
            # Subclass dispatch runs below the wrapper's autograd layer; re-include the
            # autograd keys so the rules' operations on the coefficient tensors (and the
            # kernels' custom ops) record their own graph, as the reference's
            # /root/reference/src/polytensors/_tensor.py:370-400 does.
            with contextlib.ExitStack() as stack:
                for key in _COEFFICIENT_AUTOGRAD_KEYS:
                    stack.enter_context(torch._C._SetExcludeDispatchKeyGuard(key, False))
                return dispatch(func, types, args, kwargs)
        return dispatch(func, types, args, kwargs)


# The routing modules import PolyTensor themselves, so they come after the class.
from ._decompositions import maybe_decompose  # noqa: E402
from ._dispatch import dispatch  # noqa: E402
