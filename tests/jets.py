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


def rel_err(got, want):
    """max |got - want| / max |want| (the per-order tolerance metric)."""
    got = got.to(torch.float64)
    want = want.to(torch.float64)
    scale = want.abs().max().item()
    err = (got - want).abs().max().item()
    return err / scale if scale > 0 else err


def norm_rel_err(got, want):
    """||got - want|| / ||want|| (the reference's _relative, tests/test_fused_kernels.py:44-45)."""
    got = got.to(torch.float64)
    want = want.to(torch.float64)
    return ((got - want).norm() / want.norm()).item()
