"""Independent Taylor coefficients by nested forward-mode AD (test helper).

For a function ``f`` and polynomial curves ``x_j(t) = sum_k c_jk t^k``, the
order-k coefficient of ``f(x(t))`` at t = 0 is ``g^(k)(0) / k!`` with
``g(t) = f(x(t))``; ``taylor`` computes it with k nested ``torch.func.jvp``
calls on the scalar t, exactly as the reference's tests derive their expected
values (/root/reference/tests/test_attention.py:33-46,
/root/reference/tests/test_plain_range.py:103-115). It shares no code with the
series recurrences it checks.
"""

import math

import torch


def curve(coeffs, t):
    """Horner evaluation of sum_k coeffs[k] t^k (no t**0, whose derivative at 0 is NaN)."""
    out = coeffs[-1]
    for c in reversed(coeffs[:-1]):
        out = c + t * out
    return out


def taylor(f, series, degree, dtype=torch.float64):
    """Coefficients 0..degree of f(*curves) along t; ``series`` is a list of coefficient lists."""
    t0 = torch.zeros((), dtype=dtype)

    def g(t):
        return f(*(curve(list(s), t) for s in series))

    out = []
    fn = g
    for k in range(degree + 1):
        value = fn(t0)
        if isinstance(value, tuple):
            out.append(tuple(v / math.factorial(k) for v in value))
        else:
            out.append(value / math.factorial(k))
        prev = fn

        def fn(t, prev=prev):
            return torch.func.jvp(prev, (t,), (torch.ones_like(t),))[1]
    return out


def taylor_complex(f, bases, reals, imags, degree, dtype=torch.float64):
    """Coefficients 0..degree of f along x_j + t (u_j + i w_j), a complex direction over a real base.

    By multilinearity (/root/reference/docs/notes.md:59-76) coefficient k is
    sum_b C(k, b) i^b d_s^{k-b} d_t^b g(0, 0) / k! with g(s, t) = f(x + s u + t w), a
    real function; its mixed partials are nested torch.func.jvp calls on s and t.
    """
    s0 = torch.zeros((), dtype=dtype)

    def g(s, t):
        return f(*(x + s * u + t * w for x, u, w in zip(bases, reals, imags)))

    def mixed(a, b):
        fn = g
        for _ in range(a):
            def fn(s, t, prev=fn):
                return torch.func.jvp(lambda s_: prev(s_, t), (s,), (torch.ones_like(s),))[1]
        for _ in range(b):
            def fn(s, t, prev=fn):
                return torch.func.jvp(lambda t_: prev(s, t_), (t,), (torch.ones_like(t),))[1]
        return fn(s0, s0)

    out = []
    for k in range(degree + 1):
        total = None
        for b in range(k + 1):
            term = mixed(k - b, b) * (math.comb(k, b) * (1j ** b))
            total = term if total is None else total + term
        out.append(total / math.factorial(k) if k else total.real)
    return out


def rel_err(got, want):
    """max |got - want| / max |want| (the per-order tolerance metric); complex values compare whole."""
    dtype = torch.complex128 if (got.is_complex() or want.is_complex()) else torch.float64
    got = got.to(dtype)
    want = want.to(dtype)
    scale = want.abs().max().item()
    err = (got - want).abs().max().item()
    return err / scale if scale > 0 else err


def norm_rel_err(got, want):
    """||got - want|| / ||want|| (the reference's _relative, tests/test_fused_kernels.py:44-45)."""
    dtype = torch.complex128 if (got.is_complex() or want.is_complex()) else torch.float64
    got = got.to(dtype)
    want = want.to(dtype)
    return ((got - want).norm() / want.norm()).item()
