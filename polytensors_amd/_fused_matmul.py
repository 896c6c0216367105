"""Cauchy-product matrix products of degree-K series on gfx950.

``C_k = sum_{i+j=k} A_i @ B_j`` for all k in one kernel launch: the reference
computes the same product as (K+1)(K+2)/2 separate matmuls
(/root/reference/src/polytensors/_plain.py:118-128, reached from the
mm/bmm/matmul/linear/addmm rules of /root/reference/src/polytensors/_range_ops.py:160-176).
An ordinary-tensor operand is a series with one order (the reference lifts it
with zero orders, _range_ops.py:37-45), so only K+1 products are formed.
Batch dimensions broadcast as in torch.matmul; float32 and float64, and
bfloat16 / float16 with fp32 accumulation and one rounding per element. Above
the kernel's degree (8, up to 16) the product runs in blocks of 9 orders.
"""

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_DTYPES = (torch.float32, torch.float64, torch.bfloat16, torch.float16)
# the 16-bit kernel addresses each (column-padded) operand matrix with 32-bit byte offsets
_HALF_MATRIX_LIMIT = 1 << 29


def why_ineligible(a, b, below_autograd=False):
    reason = _gate.common_reason((a, b), below_autograd=below_autograd, complex_ok=True, complex_base_ok=True,
                                 max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    coeffs = [c for x in (a, b) for c in _gate.coefficients(x, 0)]
    dtype = _gate.real_dtype(coeffs[0].dtype)
    if dtype not in _DTYPES or any(_gate.real_dtype(c.dtype) != dtype for c in coeffs):
        return "operands must share one dtype, float32, float64, bfloat16 or float16"
    if a.ndim == 0 or b.ndim == 0:
        return "matmul of a 0-d tensor"
    if dtype in (torch.bfloat16, torch.float16):
        for x in (a, b):
            rows = x.shape[-2] if x.ndim > 1 else 1
            if rows * (-(-x.shape[-1] // 8) * 8) >= _HALF_MATRIX_LIMIT:
                return "16-bit operand matrices must stay below 2^29 elements"
    return None


def _cauchy(A, B, degree, trans_b):
    """The Cauchy-product kernel's stacked [K+1, batch, m, n] result for operand coefficient lists
    A (1 or K+1 orders) and B; above the kernel's degree, in blocks of its orders.

    With blocks of m = MAX_DEGREE + 1 orders, X = sum_p t^(m p) X^(p) and
    A (*) B = sum_{p,q} t^(m (p+q)) A^(p) (*) B^(q), each block product being the full product of two
    degree-(m-1) series: its orders 0..m-1 are one kernel launch, and its orders m..2m-2 another on
    the blocks with their orders reversed (order r of the reversed product is order 2m-2-r of the
    forward one). An ordinary operand needs no blocking of its own: C_k = A_k B_0 per block of A.
    """
    cap = _gate.MAX_DEGREE
    if degree <= cap:
        return _ops.cauchy_matmul(A, B, degree, trans_b)
    m = cap + 1

    def block(X, p):   # orders m p .. m p + m - 1, zero past the given ones
        part = list(X[m * p: m * (p + 1)])
        return part + [torch.zeros_like(X[0]) for _ in range(m - len(part))]

    out = [None] * (degree + 1)

    def add(k, value):
        out[k] = value if out[k] is None else out[k] + value

    blocks = -(-(degree + 1) // m)
    if len(A) == 1 or len(B) == 1:
        for p in range(blocks):
            low = _ops.cauchy_matmul(block(A, p) if len(A) > 1 else A, block(B, p) if len(B) > 1 else B, cap, trans_b)
            for j in range(m):
                if m * p + j <= degree:
                    add(m * p + j, low[j])
    else:
        for p in range(blocks):
            for q in range(blocks):
                base = m * (p + q)
                if base > degree:
                    continue
                ap, bq = block(A, p), block(B, q)
                low = _ops.cauchy_matmul(ap, bq, cap, trans_b)
                for j in range(min(m, degree - base + 1)):
                    add(base + j, low[j])
                if base + m <= degree:
                    # orders 0..cap-1 of the reversed blocks give orders 2 cap .. cap + 1 of the block product
                    high = _ops.cauchy_matmul(ap[::-1][:cap], bq[::-1][:cap], cap - 1, trans_b)
                    for r in range(m - 1):
                        k = base + 2 * cap - r
                        if k <= degree:
                            add(k, high[r])
    zero = None
    for k in range(degree + 1):
        if out[k] is None:
            zero = torch.zeros_like(out[0]) if zero is None else zero
            out[k] = zero
    return torch.stack(out)


def eligible(a, b):
    return why_ineligible(a, b) is None


def _degree(*xs):
    return next(x.degree for x in xs if isinstance(x, PolyTensor))


def matmul(a, b, below_autograd=False):
    """Series of ``torch.matmul(a, b)``."""
    reason = why_ineligible(a, b, below_autograd)
    if reason is not None:
        raise NotImplementedError(f"matmul: {reason}")
    if _complex.has_complex(a, b) or _complex.has_complex_base(a, b):
        return _complex.bilinear(matmul, "matmul", a, b, below_autograd=below_autograd)
    degree = _degree(a, b)
    A = list(_gate.coefficients(a, degree))
    B = list(_gate.coefficients(b, degree))
    squeeze_m = A[0].ndim == 1
    squeeze_n = B[0].ndim == 1
    if squeeze_m:
        A = [c.unsqueeze(0) for c in A]
    if squeeze_n:
        B = [c.unsqueeze(-1) for c in B]
    m, kd = A[0].shape[-2:]
    kb, n = B[0].shape[-2:]
    if kd != kb:
        raise RuntimeError(f"matmul: inner dimensions differ ({kd} vs {kb})")
    batch_a, batch_b = A[0].shape[:-2], B[0].shape[:-2]
    batch = batch_a if batch_a == batch_b or not batch_b else \
        batch_b if not batch_a else torch.broadcast_shapes(batch_a, batch_b)

    def flat(coeffs, rows, cols):
        own = coeffs[0].shape[:-2]
        if len(own) == 0 or (tuple(own) != tuple(batch) and all(s == 1 for s in own)):
            return [c.view(1, rows, cols) if c.is_contiguous() else c.reshape(1, rows, cols).contiguous()
                    for c in coeffs]
        if own == batch:
            return [c.view(-1, rows, cols) if c.is_contiguous() else c.reshape(-1, rows, cols).contiguous()
                    for c in coeffs]
        return [c.expand(*batch, rows, cols).reshape(-1, rows, cols).contiguous() for c in coeffs]

    if all(c.ndim == 2 and not c.is_contiguous() and c.t().is_contiguous() for c in B):
        # a transposed [n, k] matrix (a linear layer's weight): the kernel reads it in place
        out = _cauchy(flat(A, m, kd), [c.t().reshape(1, n, kd) for c in B], degree, True)
    else:
        out = _cauchy(flat(A, m, kd), flat(B, kd, n), degree, False)
    out = out.view(degree + 1, *batch, m, n)
    if squeeze_m:
        out = out.squeeze(-2)
    if squeeze_n:
        out = out.squeeze(-1)
    return PolyTensor.from_stacked(out)


def linear(x, weight, bias=None):
    """Series of ``torch.nn.functional.linear``: x @ weight^T (+ bias)."""
    reason = why_ineligible(x, weight)
    if reason is not None:
        raise NotImplementedError(f"linear: {reason}")
    if _complex.has_complex(x, weight) or _complex.has_complex_base(x, weight):
        result = _complex.bilinear(linear, "linear", x, weight)
        return result if bias is None else result + bias
    degree = _degree(x, weight, *([bias] if isinstance(bias, PolyTensor) else []))
    X = list(_gate.coefficients(x, degree))
    W = list(_gate.coefficients(weight, degree))
    if W[0].ndim != 2:
        raise RuntimeError("linear: weight must be 2-D")
    out_features, in_features = W[0].shape
    lead = X[0].shape[:-1]
    X = [c.reshape(1, -1, in_features).contiguous() for c in X]
    W = [c.reshape(1, out_features, in_features).contiguous() for c in W]
    out = _cauchy(X, W, degree, True)
    result = PolyTensor.from_stacked(out.view(degree + 1, *lead, out_features))
    if bias is not None:
        result = result + bias
    return result


def from_dispatch(func, args, kwargs):
    """mm/bmm/mv/dot/matmul/addmm reaching ``__torch_dispatch__`` (under autograd, whose
    recorded backward runs these same products on the cotangent series)."""
    aten = torch.ops.aten
    if func is aten.addmm.default:
        bias, a, b = args[:3]
        beta, alpha = kwargs.get("beta", 1), kwargs.get("alpha", 1)
        product = matmul(a, b, below_autograd=True)
        if alpha != 1:
            product = product * alpha
        if beta == 0:
            return product
        return product + (bias * beta if beta != 1 else bias)
    return matmul(args[0], args[1], below_autograd=True)
