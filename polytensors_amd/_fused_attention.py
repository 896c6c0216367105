"""Fused flash-style attention of degree-K series on gfx950.

For query, key and value series Q(t), K(t), V(t):
    S(t) = scale * Q(t) K(t)^T  (masked),  P(t) = softmax(S(t)),  O(t) = P(t) V(t),
the series of the reference's plain-range decomposition
/root/reference/src/polytensors/_decompositions.py:28-43, computed block by block
without forming the L x S score series: the online max and rescale use the
constant-order scores only, the exponential series of the higher orders is
formed from ``k E_k = sum_j j S_j E_{k-j}`` (/root/reference/src/polytensors/_plain.py:153-159),
and the output is the series quotient of the accumulated numerator and row sum.
Eligibility and conventions follow the degree-1 kernel of the reference
(/root/reference/src/polytensors/_fused_attention.py:188-316): causal, a mask or
both (as the general rule, which applies each), no dropout or GQA, default scale 1/sqrt(d), and a query row with no
admissible key gets output zero. The mask is (..., L, S), broadcasting over the
batch as in the reference's general rule (one shared mask, one per batch entry,
one per head, or any mix of these). A floating mask is added to the
scores, so to their constant order, as the reference's general rule does
(/root/reference/src/polytensors/_decompositions.py:38-40); its -inf entries
exclude their keys (16-bit operands with such a mask run the float32 kernel).

Under autograd (a PolyTensor operand requiring grad) the call records
``_SeriesAttention``, whose backward is the degree-K gradient series kernel
(the reference's _SeriesAttention, _fused_attention.py:267-295, at any degree).
"""

import contextvars
import math

import torch

from . import _complex, _gate, _ops
from ._tensor import PolyTensor

_enabled = contextvars.ContextVar("polytensors_amd_fused_attention", default=True)
_HEAD_DIMS = {torch.float32: (16, 32, 64, 128), torch.float64: (16, 32, 64, 128),
              torch.bfloat16: (16, 32, 64, 128), torch.float16: (16, 32, 64, 128)}


def default_scale(head_dim):
    return 1 / math.sqrt(head_dim)


def _kernel_mask(attn_mask, batch, L, S):
    """The mask as the kernels take it, ``(mask, mask_map)``: ``(None, None)`` without one, an
    (L, S) mask shared by every head with map None, or a set of masks (n, L, S) with the map
    (div, outer, inner) of heads to masks (head b of the flattened batch uses mask
    ``(b // div) * outer + (b % div) * inner``). The mask broadcasts against the batch
    dimensions ``batch`` as in torch's scaled_dot_product_attention. NotImplemented for a mask
    that is neither boolean nor floating or does not broadcast."""
    if attn_mask is None:
        return None, None
    if not (attn_mask.dtype == torch.bool or attn_mask.dtype.is_floating_point) or attn_mask.ndim < 2 or \
            tuple(attn_mask.shape[-2:]) != (L, S) or attn_mask.ndim - 2 > len(batch):
        return NotImplemented
    lead = (1,) * (len(batch) - (attn_mask.ndim - 2)) + tuple(attn_mask.shape[:-2])
    if any(m not in (1, b) for m, b in zip(lead, batch)):
        return NotImplemented
    if all(m == 1 for m in lead):
        return attn_mask.reshape(L, S), None
    if len(batch) >= 2 and all(m == 1 for m in lead[:-2]):
        H = batch[-1]
        if lead[-1] == 1 and math.prod(batch[:-2]) == 1:   # a mask per batch entry, over its H heads
            return attn_mask.reshape(lead[-2], L, S), (H, 1, 0)
        if lead[-2] == 1:   # a mask per head, the same in every batch entry
            return attn_mask.reshape(lead[-1], L, S), (H, 0, 1)
    # otherwise a mask per head of the flattened batch
    return attn_mask.expand(*batch, L, S).reshape(-1, L, S), (1, 1, 0)


def _needs_grad(*values):
    return _gate.wrapper_grad(*values)


def why_ineligible(query, key, value, attn_mask, dropout_p, is_causal, enable_gqa):
    if not _enabled.get():
        return ("the fused attention kernel is disabled (PolyTensor.fused_attention(False)) and "
                "polytensors_amd has no general series rules")
    if dropout_p != 0.0:
        return "dropout is not supported"
    if enable_gqa:
        return "GQA is not supported"
    tensors = (query, key, value)
    if not all(isinstance(x, torch.Tensor) for x in tensors):
        return "query, key and value must be tensors"
    if isinstance(attn_mask, PolyTensor):
        return "the mask must be an ordinary tensor"
    if attn_mask is not None and attn_mask.requires_grad and torch.is_grad_enabled():
        return "a mask that requires grad is not supported (no gradient flows to attn_mask)"
    grads = _needs_grad(*tensors)
    # (degrees above the kernels' are composed from series operations, to the elementwise limit)
    reason = _gate.common_reason(tensors, allow_plain_grad=grads, complex_ok=True,
                                 max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    if grads and any(not isinstance(x, PolyTensor) and x.requires_grad for x in tensors):
        # as the reference's gate (_fused_attention.py:242-243): the gradient of an
        # ordinary operand would be a series, which autograd cannot hand to it
        return "an ordinary (non-PolyTensor) operand requires grad"
    dtype = query.dtype
    for x in tensors:   # (a series' higher orders share one dtype: its last order stands for them)
        coeffs = _gate.coefficients(x, 0)
        if coeffs[0].dtype != dtype or _gate.real_dtype(coeffs[-1].dtype) != dtype:
            return "query, key and value coefficients must share one dtype"
    if dtype not in _HEAD_DIMS:
        return f"dtype {dtype} is not supported (float32, float64, bfloat16 or float16)"
    qs, ks = query.shape, key.shape
    if len(qs) < 3 or ks != value.shape or qs[:-2] != ks[:-2]:
        return "shapes must be (..., L, d) and (..., S, d) with equal batch dimensions"
    d = qs[-1]
    if d != ks[-1] or d not in _HEAD_DIMS[dtype]:
        return f"head dim {d} not in {_HEAD_DIMS[dtype]}"
    if attn_mask is not None and _kernel_mask(attn_mask, tuple(qs[:-2]), qs[-2], ks[-2]) is NotImplemented:
        return "the mask must be boolean or floating, of shape (..., L, S) broadcasting over the batch"
    return None


def eligible(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, enable_gqa=False):
    return why_ineligible(query, key, value, attn_mask, dropout_p, is_causal, enable_gqa) is None


def require_eligible(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, enable_gqa=False):
    reason = why_ineligible(query, key, value, attn_mask, dropout_p, is_causal, enable_gqa)
    if reason is not None:
        raise NotImplementedError(f"scaled_dot_product_attention: {reason}")


def _flat(coeffs, shape):
    """[bh, T, d] contiguous coefficients (no copy when already contiguous)."""
    rows, d = shape[-2], shape[-1]
    return [c.view(-1, rows, d) if c.shape == shape and c.is_contiguous() else
            c.expand(shape).reshape(-1, rows, d).contiguous() for c in coeffs]


def _contiguous(coeffs):
    return [c if c.is_contiguous() else c.contiguous() for c in coeffs]


def _full(x, degree, shape):
    """K+1 flattened [bh, T, d] coefficients; an ordinary tensor gets zero higher orders."""
    if isinstance(x, PolyTensor):
        return _flat(x.coeffs, shape)
    base = _flat([x], shape)[0]
    return [base] + [torch.zeros_like(base) for _ in range(degree)]


class _SeriesAttention(torch.autograd.Function):
    """Degree-K attention with its gradient series.

    As /root/reference/src/polytensors/_fused_attention.py:267-295 (_SeriesAttention):
    the forward kernel saves the log-sum-exp series, and the backward computes
    the gradient series of query, key and value (coefficient j = sum_{k<=j}
    J_{j-k}^T G_k) with the degree-K backward kernels. Ordinary operands get no
    gradient.
    """

    @staticmethod
    def forward(ctx, query, key, value, mask, causal, scale):   # mask: (mask, mask_map) of _kernel_mask
        degree = next(x.degree for x in (query, key, value) if isinstance(x, PolyTensor))
        q = _full(query, degree, query.shape)
        k = _full(key, degree, key.shape)
        v = _full(value, degree, value.shape)
        out, lse = _ops.taylor_attention_fwd(q, k, v, mask[0], causal, scale, degree, mask_map=mask[1])
        ctx.save_for_backward(*q, *k, *v, out, lse)
        ctx.meta = (degree, mask, causal, scale, query.shape, key.shape)
        ctx.poly = tuple(isinstance(x, PolyTensor) for x in (query, key, value))
        return PolyTensor.from_stacked(out.view(degree + 1, *query.shape))

    @staticmethod
    def backward(ctx, gradient):
        from ._plain import _plain_range
        if torch.is_grad_enabled():
            raise NotImplementedError("second-order reverse mode through the fused attention is not implemented")
        degree, mask, causal, scale, shape_q, shape_k = ctx.meta
        saved = ctx.saved_tensors
        n = degree + 1
        q, k, v = list(saved[:n]), list(saved[n:2 * n]), list(saved[2 * n:3 * n])
        out, lse = saved[3 * n], saved[3 * n + 1]
        token = _plain_range.set(True)   # the engine's thread does not see the caller's context
        try:
            g = _full(gradient, degree, shape_q)
            dq, dk, dv = _ops.attention_gradient_series(q, k, v, out, lse, g, mask[0], causal, scale, mask[1])
            grads = (PolyTensor.from_stacked(dq.view(n, *shape_q)), PolyTensor.from_stacked(dk.view(n, *shape_k)),
                     PolyTensor.from_stacked(dv.view(n, *shape_k)))
        finally:
            _plain_range.reset(token)
        return (*(gr if is_poly else None for gr, is_poly in zip(grads, ctx.poly)), None, None, None)


def attention(query, key, value, attn_mask=None, is_causal=False, scale=None):
    """Fused degree-K attention of an eligible call (see ``eligible``)."""
    require_eligible(query, key, value, attn_mask, 0.0, is_causal, False)
    return attention_checked(query, key, value, attn_mask, is_causal, scale)


def _masked(scores, excluded):
    """A masked score is (-inf, 0, ..., 0): masked_fill of the lifted -inf
    (/root/reference/src/polytensors/_range_ops.py:271-277 with _plain.py:70-75)."""
    return PolyTensor(tuple(torch.where(excluded, torch.full((), float("-inf") if k == 0 else 0.0, dtype=c.dtype,
                                                             device=c.device), c)
                            for k, c in enumerate(scores.coeffs)))


def _composed(query, key, value, attn_mask, is_causal, scale):
    """Degrees 9..16, above the attention kernels' register plans.

    The reference's decomposition (/root/reference/src/polytensors/_decompositions.py:28-43) in
    series operations: the score and value products run the Cauchy matmul (above its degree 8 in
    blocks of orders); the softmax (/root/reference/src/polytensors/_plain.py:262-273) runs the
    elementwise series kernels (exp, and the quotient by the row sums) on the scores less the row
    maximum of their constant order, which changes only that order. A masked score is
    (-inf, 0, ..., 0) and a float mask adds to the constant order. A row without an admissible key
    is NaN, as in the reference's general rule.
    """
    L, S = query.shape[-2], key.shape[-2]
    scores = (query * scale) @ key.transpose(-2, -1)
    if is_causal:
        keep = torch.ones(L, S, dtype=torch.bool, device=scores.coeffs[0].device).tril()
        scores = _masked(scores, ~keep)
    if attn_mask is not None:
        scores = _masked(scores, ~attn_mask) if attn_mask.dtype == torch.bool else scores + attn_mask
    top = scores.coeffs[0].detach().amax(-1, keepdim=True)
    e = (scores - top).exp()
    return (e / e.sum(-1, keepdim=True)) @ value


def attention_checked(query, key, value, attn_mask=None, is_causal=False, scale=None):
    """``attention`` for a call whose eligibility (including dropout and GQA) the caller checked."""
    if _complex.has_complex(query, key, value):
        return _complex.at_real_nodes(attention, "scaled_dot_product_attention", query, key, value,
                                      attn_mask=attn_mask, is_causal=is_causal, scale=scale)
    degree = next(x.degree for x in (query, key, value) if isinstance(x, PolyTensor))
    if degree > _gate.MAX_DEGREE:
        scale = default_scale(query.shape[-1]) if scale is None else scale
        return _composed(query, key, value, attn_mask, is_causal, scale)
    L, S = query.shape[-2], key.shape[-2]
    if is_causal and attn_mask is not None:
        # both: the causal rule applied to the mask (the general rule masks the scores with each,
        # /root/reference/src/polytensors/_decompositions.py:36-41)
        keep = torch.ones(L, S, dtype=torch.bool, device=attn_mask.device).tril()
        attn_mask = attn_mask & keep if attn_mask.dtype == torch.bool else attn_mask.masked_fill(~keep, float("-inf"))
        is_causal = False
    mask = _kernel_mask(attn_mask, tuple(query.shape[:-2]), L, S)   # (mask, mask_map)
    scale = default_scale(query.shape[-1]) if scale is None else scale
    if _needs_grad(query, key, value):
        return _SeriesAttention.apply(query, key, value, mask, bool(is_causal), float(scale))
    # the operator takes [..., T, d] coefficients (batch dimensions flattened to heads in order)
    q = _contiguous(_gate.coefficients(query, degree))
    k = _contiguous(_gate.coefficients(key, degree))
    v = _contiguous(_gate.coefficients(value, degree))
    out, _ = _ops.taylor_attention_fwd(q, k, v, mask[0], bool(is_causal), float(scale), degree, mask_map=mask[1])
    return PolyTensor.from_stacked(out)
