"""Complex directions through the real gfx950 kernels.

A PolyTensor may carry complex higher coefficients over a real constant term;
the reference defines the result as the derivatives of the real computation
extended multilinearly to complex vectors (/root/reference/docs/notes.md:59-76,
coercion /root/reference/src/polytensors/_tensor.py:72-80). Coefficient k of any
fused operation is a polynomial in the operands' higher coefficients whose
monomials have at most k factors. Substituting ``c_j -> Re c_j + lam * Im c_j`` in
every operand at once therefore gives a real-valued polynomial P_k(lam) of
degree <= k, and the complex coefficient is P_k(i). It is recovered exactly
from K+1 real evaluations at nodes lam_0..lam_K (Lagrange interpolation at
lam = i): each evaluation is one run of the real kernel on real-direction
series, so every real kernel serves complex directions unchanged. Order 0 is the
same in every run.

Operations that are bilinear in the series (the Cauchy matmul and the
elementwise series product) use the exact split
``A (*) B = A_R (*) B_R - A_I (*) B_I + i (A_R (*) B_I + A_I (*) B_R)`` instead,
two real runs when one operand is real (the reference's own linear split of
complex coefficients, /root/reference/src/polytensors/_dispatch.py:12-26, in
bilinear form).

Nodes are equispaced on [-r, r] with r chosen per degree to keep sum_m |w_m| r^K
small (about 6 at K = 3, 11 at K = 4, 170 at K = 8: the factor by which the real
runs' rounding errors can grow in the complex result); above degree 12, r = 3
(measured on the exponential series: relative errors of the combination about
3e-5 from float32 runs and 1e-13 from float64 runs at degree 16, against 3e-4 and
1e-12 with r = 2; Chebyshev nodes measured worse at every radius tried).
"""

import contextlib
import functools

import torch

from . import _gate, _ops
from ._tensor import PolyTensor

_NODE_RADIUS = {1: 1.0, 2: 1.5, 3: 1.5}


@functools.lru_cache(maxsize=None)
def nodes_and_weights(degree):
    """Real nodes lam_m and the complex Lagrange weights w_m = l_m(i) (Python floats/complex)."""
    n = degree + 1
    r = _NODE_RADIUS.get(degree, 2.0 if degree <= 12 else 3.0)
    nodes = [0.0] if n == 1 else [r * (2 * m / (n - 1) - 1) for m in range(n)]
    weights = []
    for m, xm in enumerate(nodes):
        w = 1 + 0j
        for j, xj in enumerate(nodes):
            if j != m:
                w *= (1j - xj) / (xm - xj)
        weights.append(w)
    return tuple(nodes), tuple(weights)


def _is_complex_series(x):
    # the higher orders share one dtype, complex when any order is (PolyTensor's coercion rules)
    return isinstance(x, PolyTensor) and x.coeffs[-1].is_complex()


def has_complex(*values):
    """Whether any operand (nested in lists/tuples/dicts) is a series with complex coefficients."""
    for v in values:
        if isinstance(v, (list, tuple)):
            if has_complex(*v):
                return True
        elif isinstance(v, dict):
            if has_complex(*v.values()):
                return True
        elif _is_complex_series(v):
            return True
    return False


def _check(values, what):
    for v in values:
        if isinstance(v, PolyTensor) and v.coeffs[0].is_complex():
            raise NotImplementedError(f"{what}: a complex constant coefficient (complex base) is not implemented; "
                                      "complex directions need a real constant term")


def _flatten(values):
    out = []
    for v in values:
        if isinstance(v, (list, tuple)):
            out.extend(_flatten(v))
        elif isinstance(v, dict):
            out.extend(_flatten(list(v.values())))
        else:
            out.append(v)
    return out


def _planes(x):
    """The contiguous complex planes (orders 1..K) of a complex-direction series."""
    return [c.contiguous() for c in x.coeffs[1:]]


def _variants(x, alpha, beta):
    """Real-direction series alpha_v Re + beta_v Im of x's higher orders (order 0 shared), one per v."""
    planes = _ops.complex_to_real(_planes(x), list(alpha), list(beta))
    return [PolyTensor((x.coeffs[0],) + tuple(v.unbind(0))) for v in planes.unbind(0)]


def _substitute(x, table):
    """x with every complex-direction series replaced by its variant from ``table``."""
    if isinstance(x, (list, tuple)):
        return type(x)(_substitute(v, table) for v in x)
    if isinstance(x, dict):
        return {k: _substitute(v, table) for k, v in x.items()}
    return table.get(id(x), x)


def _combine(outputs, weights):
    """Complex series sum_m w_m Y_m in the higher orders; order 0 of the first run."""
    first = outputs[0]
    orders = first.degree
    if orders == 0:
        return first
    src = [y.coeffs[k].contiguous() for y in outputs for k in range(1, orders + 1)]
    planes = _ops.real_to_complex(src, orders, [w.real for w in weights], [w.imag for w in weights])
    return PolyTensor((first.coeffs[0],) + tuple(planes.unbind(0)))


@contextlib.contextmanager
def _in_plain_range():
    from ._plain import _plain_range

    token = _plain_range.set(True)
    try:
        yield
    finally:
        _plain_range.reset(token)


class _Variants(torch.autograd.Function):
    """The real variants of a complex-direction series at the interpolation nodes, under
    wrapper-level (PolyTensor) autograd.

    Reverse mode needs the gradient series J(x(t))^T G(t) extended multilinearly to
    complex x and G, as the forward is (/root/reference/docs/api.md:69-76). Its
    coefficient k is again a polynomial of degree <= k in the substitution
    c_j -> Re c_j + lam Im c_j applied to x's and G's higher orders (G_0 is real), so it
    is the Lagrange combination of the real gradient series at the nodes, each formed
    at the node's variants of x and of G. Hence the backward of "variants" is the
    combination, and the backward of the combination (``_Combination``) is the
    cotangent's variants: each node's real graph runs the real backward kernels.
    """

    @staticmethod
    def forward(ctx, x):
        nodes, weights = nodes_and_weights(x.degree)
        ctx.weights = weights
        return tuple(_variants(x, [1.0] * len(nodes), nodes))

    @staticmethod
    def backward(ctx, *grads):
        with _in_plain_range():   # the engine's thread does not see the caller's context
            return _combine(list(grads), ctx.weights)


class _Shared(torch.autograd.Function):
    """A real operand (series or ordinary tensor) that requires grad, handed unchanged to every
    node under wrapper-level autograd: its gradient series is the Lagrange combination of the
    nodes' gradients (complex in general), not their sum."""

    @staticmethod
    def forward(ctx, x, degree):
        nodes, weights = nodes_and_weights(degree)
        ctx.weights = weights
        return tuple(x.view_as(x) for _ in nodes)

    @staticmethod
    def backward(ctx, *grads):
        if all(isinstance(g, PolyTensor) for g in grads):
            with _in_plain_range():
                return _combine(list(grads), ctx.weights), None
        return grads[0], None   # an ordinary gradient (order 0 only) is the same at every node


class _Combination(torch.autograd.Function):
    """The complex series sum_m w_m Y_m of the node outputs, under wrapper-level autograd
    (see ``_Variants``): its backward hands each node the variant of the cotangent series."""

    @staticmethod
    def forward(ctx, *outputs):
        ctx.degree = outputs[0].degree
        return _combine(list(outputs), nodes_and_weights(ctx.degree)[1])

    @staticmethod
    def backward(ctx, grad):
        nodes, _ = nodes_and_weights(ctx.degree)
        if not _is_complex_series(grad):   # a real cotangent series is its own variant at every node
            return tuple(grad for _ in nodes)
        _check([grad], "reverse mode")
        with _in_plain_range():
            return tuple(_variants(grad, [1.0] * len(nodes), nodes))


def at_real_nodes(fn, what, *args, **kwargs):
    """``fn(*args, **kwargs)`` for complex-direction series from K+1 runs on real directions.

    ``fn`` returns one PolyTensor. The real variants of every complex-direction
    operand are formed in one pass per operand (all nodes at once). Called above
    autograd (the fused norm, cross entropy and attention) under wrapper-level
    autograd, the variants and the combination are recorded (``_Variants``,
    ``_Combination``), so that reverse mode runs each node's real backward
    kernels; in coefficient autograd the plumbing operators record their own
    (linear) gradients.
    """
    values = _flatten(list(args) + list(kwargs.values()))
    return _nodes(fn, what, args, kwargs, values, _gate.wrapper_grad(*values))


def at_real_nodes_below_autograd(fn, what, *args, **kwargs):
    """``at_real_nodes`` for a rule reached from ``__torch_dispatch__`` (under the autograd layer,
    which has recorded the operation's own backward): nothing is recorded here."""
    values = _flatten(list(args) + list(kwargs.values()))
    return _nodes(fn, what, args, kwargs, values, False)


def _nodes(fn, what, args, kwargs, values, recorded):
    _check(values, what)
    degree = next(v.degree for v in values if isinstance(v, PolyTensor))
    nodes, weights = nodes_and_weights(degree)
    ones = [1.0] * len(nodes)
    variants = {id(v): (_Variants.apply(v) if recorded else _variants(v, ones, nodes))
                for v in values if _is_complex_series(v)}
    if recorded:
        for v in values:
            if isinstance(v, torch.Tensor) and v.requires_grad and id(v) not in variants:
                variants[id(v)] = _Shared.apply(v, degree)
    outputs = []
    for m in range(len(nodes)):
        table = {key: vs[m] for key, vs in variants.items()}
        out = fn(*_substitute(list(args), table), **_substitute(kwargs, table))
        if not isinstance(out, PolyTensor):
            raise TypeError(f"{what}: a series operation returned {type(out).__name__}")
        outputs.append(out)
    del variants
    if recorded and any(out.requires_grad for out in outputs):
        return _Combination.apply(*outputs)
    return _combine(outputs, weights)


def has_complex_base(*values):
    """Whether any operand is complex in its constant term: a series with a complex order 0, or a
    complex ordinary tensor."""
    for v in _flatten(list(values)):
        if isinstance(v, PolyTensor):
            if v.coeffs[0].is_complex():
                return True
        elif isinstance(v, torch.Tensor) and v.is_complex():
            return True
    return False


def _split(x):
    """(real part, imaginary part or None) of an operand, every order split (views)."""
    if isinstance(x, PolyTensor):
        if not x.coeffs[-1].is_complex() and not x.coeffs[0].is_complex():
            return x, None
        re = tuple(c.real if c.is_complex() else c for c in x.coeffs)
        im = tuple(c.imag if c.is_complex() else torch.zeros_like(c) for c in x.coeffs)
        return PolyTensor._wrap(re), PolyTensor._wrap(im)
    if isinstance(x, torch.Tensor) and x.is_complex():
        return x.real, x.imag
    return x, None


def _join(real, imag):
    """The series real + i imag (either may be None: zero)."""
    if imag is None:
        return real
    return PolyTensor(tuple(torch.complex(r, i) for r, i in zip(real.coeffs, imag.coeffs)))


def _add(x, y, sign=1.0):
    if x is None:
        return y if sign > 0 or y is None else PolyTensor._wrap(tuple(-c for c in y.coeffs))
    if y is None:
        return x
    return PolyTensor._wrap(tuple(a + sign * b for a, b in zip(x.coeffs, y.coeffs)))


def complex_product(fn, a, b, *rest, **kwargs):
    """``fn(a, b, ...)`` for a product bilinear in a and b when some operand has a complex constant
    term (complex arithmetic, /root/reference/docs/notes.md:74-77): the real runs
    fn(a_R, b_R) - fn(a_I, b_I) + i (fn(a_R, b_I) + fn(a_I, b_R)) of the real kernel, each operand
    split order by order into its real and imaginary parts (a real operand has none)."""
    ar, ai = _split(a)
    br, bi = _split(b)
    real = fn(ar, br, *rest, **kwargs)
    imag = None
    if ai is not None and bi is not None:
        real = _add(real, fn(ai, bi, *rest, **kwargs), -1.0)
    if bi is not None:
        imag = fn(ar, bi, *rest, **kwargs)
    if ai is not None:
        imag = _add(imag, fn(ai, br, *rest, **kwargs))
    return _join(real, imag)


def complex_quotient(divide, multiply, a, b):
    """a / b elementwise when some operand has a complex constant term: a conj(b) / (b conj(b)),
    where b conj(b) = b_R (*) b_R + b_I (*) b_I is a real series (conj taken order by order, the
    conjugate of b(t) for real t), so the quotient is two real quotient runs."""
    br, bi = _split(b)
    if bi is None:   # a real divisor: each part of a over b
        ar, ai = _split(a)
        return _join(divide(ar, b), None if ai is None else divide(ai, b))
    conj_b = _join(br, PolyTensor._wrap(tuple(-c for c in bi.coeffs)))
    numerator = complex_product(multiply, a, conj_b)
    denominator = _add(multiply(br, br), multiply(bi, bi))
    nr, ni = _split(numerator)
    return _join(divide(nr, denominator), None if ni is None else divide(ni, denominator))


def bilinear(fn, what, a, b, *rest, **kwargs):
    """``fn(a, b, ...)`` for an operation bilinear in the series a, b (Cauchy products).

    With one complex-direction series and one ordinary tensor, the imaginary run
    takes the imaginary planes as a series of degree K-1 (orders shifted down by
    one: an ordinary operand does not mix orders), so it forms K products, not
    K+1. Two series operands use the four real runs of the complex product. An
    operand with a complex constant term takes the general split
    (``complex_product``).
    """
    if has_complex_base(a, b):
        return complex_product(fn, a, b, *rest, **kwargs)
    _check([a, b], what)
    ac, bc = _is_complex_series(a), _is_complex_series(b)
    if ac != bc and not isinstance(b if ac else a, PolyTensor):
        x = a if ac else b
        real, imag = _ops.complex_to_real(_planes(x), [1.0, 0.0], [0.0, 1.0]).unbind(0)
        xr = PolyTensor((x.coeffs[0],) + tuple(real.unbind(0)))
        xi = PolyTensor(tuple(imag.unbind(0)))
        yr = fn(xr, b, *rest, **kwargs) if ac else fn(a, xr, *rest, **kwargs)
        yi = fn(xi, b, *rest, **kwargs) if ac else fn(a, xi, *rest, **kwargs)
        # orders 1..K of the result: real from yr's orders 1..K, imaginary from yi's orders 0..K-1
        return _combine_parts(yr, list(yi.coeffs))
    def parts(x):
        if not _is_complex_series(x):
            return x, None
        r, i = _ops.complex_to_real(_planes(x), [1.0, 0.0], [0.0, 1.0]).unbind(0)
        return (PolyTensor((x.coeffs[0],) + tuple(r.unbind(0))),
                PolyTensor((torch.zeros_like(x.coeffs[0]),) + tuple(i.unbind(0))))

    ar, ai = parts(a)
    br, bi = parts(b)
    real = fn(ar, br, *rest, **kwargs)
    imag = None
    if ai is not None:
        imag = fn(ai, br, *rest, **kwargs)
    if bi is not None:
        t = fn(ar, bi, *rest, **kwargs)
        imag = t if imag is None else PolyTensor(tuple(x + y for x, y in zip(imag.coeffs, t.coeffs)))
        if ai is not None:
            t = fn(ai, bi, *rest, **kwargs)
            real = PolyTensor(tuple(x - y for x, y in zip(real.coeffs, t.coeffs)))
    return _combine_parts(real, list(imag.coeffs[1:]))


def _combine_parts(real, imag_orders):
    """Series with order 0 of ``real`` and orders k >= 1 = real_k + i imag_orders[k-1]."""
    orders = real.degree
    if orders == 0:
        return real
    src = [c.contiguous() for c in real.coeffs[1:]] + [c.contiguous() for c in imag_orders[:orders]]
    planes = _ops.real_to_complex(src, orders, [1.0, 0.0], [0.0, 1.0])
    return PolyTensor((real.coeffs[0],) + tuple(planes.unbind(0)))
