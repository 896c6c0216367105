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
runs' rounding errors can grow in the complex result).
"""

import functools

import torch

_NODE_RADIUS = {1: 1.0, 2: 1.5, 3: 1.5}


@functools.lru_cache(maxsize=None)
def nodes_and_weights(degree):
    """Real nodes lam_m and the complex Lagrange weights w_m = l_m(i) (Python floats/complex)."""
    n = degree + 1
    r = _NODE_RADIUS.get(degree, 2.0)
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
    from ._tensor import PolyTensor

    return isinstance(x, PolyTensor) and any(c.is_complex() for c in x.coeffs)


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
    from ._tensor import PolyTensor

    for v in values:
        if isinstance(v, PolyTensor) and v.coeffs[0].is_complex():
            raise NotImplementedError(f"{what}: a complex constant coefficient (complex base) is not implemented; "
                                      "complex directions need a real constant term")
    if torch.is_grad_enabled() and any(isinstance(v, torch.Tensor) and v.requires_grad for v in values):
        raise NotImplementedError(f"{what}: reverse mode with complex directions is not implemented")


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


def _real_part(x, lam):
    """The real-direction series Re c_j + lam Im c_j (orders >= 1); other values unchanged."""
    from ._tensor import PolyTensor

    if isinstance(x, (list, tuple)):
        return type(x)(_real_part(v, lam) for v in x)
    if isinstance(x, dict):
        return {k: _real_part(v, lam) for k, v in x.items()}
    if not _is_complex_series(x):
        return x
    head = x.coeffs[0]
    return PolyTensor((head,) + tuple(torch.add(c.real, c.imag, alpha=lam) if c.is_complex() else c
                                      for c in x.coeffs[1:]))


def _combine(outputs, weights):
    """Complex series sum_m w_m Y_m in the higher orders; order 0 of the first run."""
    from ._tensor import PolyTensor

    first = outputs[0]
    coeffs = [first.coeffs[0]]
    for k in range(1, first.degree + 1):
        re = im = None
        for w, y in zip(weights, outputs):
            c = y.coeffs[k]
            re = c * w.real if re is None else re.add_(c, alpha=w.real)
            im = c * w.imag if im is None else im.add_(c, alpha=w.imag)
        coeffs.append(torch.complex(re, im))
    return PolyTensor(tuple(coeffs))


def at_real_nodes(fn, what, *args, **kwargs):
    """``fn(*args, **kwargs)`` for complex-direction series from K+1 runs on real directions.

    ``fn`` returns one PolyTensor; its real runs are made one at a time (the
    working set is one real variant of the operands).
    """
    from ._tensor import PolyTensor

    values = _flatten(list(args) + list(kwargs.values()))
    _check(values, what)
    degree = next(v.degree for v in values if isinstance(v, PolyTensor))
    nodes, weights = nodes_and_weights(degree)
    outputs = []
    for lam in nodes:
        out = fn(*_real_part(list(args), lam), **_real_part(kwargs, lam))
        if not isinstance(out, PolyTensor):
            raise TypeError(f"{what}: a series operation returned {type(out).__name__}")
        outputs.append(out)
    return _combine(outputs, weights)


def _parts(x):
    """(real part, imaginary part or None) of a series operand: A_R = [A_0, Re A_1, ...],
    A_I = [0, Im A_1, ...]; ordinary tensors are real."""
    from ._tensor import PolyTensor

    if not _is_complex_series(x):
        return x, None
    head = x.coeffs[0]
    real = PolyTensor((head,) + tuple(c.real.contiguous() if c.is_complex() else c for c in x.coeffs[1:]))
    imag = PolyTensor((torch.zeros_like(head),) + tuple(c.imag.contiguous() if c.is_complex() else torch.zeros_like(c)
                                                       for c in x.coeffs[1:]))
    return real, imag


def bilinear(fn, what, a, b, *rest, **kwargs):
    """``fn(a, b, ...)`` for an operation bilinear in the series a, b (Cauchy products)."""
    from ._tensor import PolyTensor

    _check([a, b], what)
    ar, ai = _parts(a)
    br, bi = _parts(b)
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
    coeffs = [real.coeffs[0]] + [torch.complex(r, i) for r, i in zip(real.coeffs[1:], imag.coeffs[1:])]
    return PolyTensor(tuple(coeffs))
