"""Fused cross entropy of degree-K series of (N, C) (or (N, C, d1, ...)) logits on gfx950.

For logits ``z(t) = sum_k z_k t^k`` and integer targets ``y``, one streaming
pass per row computes the log-sum-exp series ``lse(t)`` of the row, and the
loss series is ``lse_k - z_k[y]`` (the log-softmax series of
/root/reference/src/polytensors/_plain.py:262-273 read at the target, the
per-order NLL of /root/reference/src/polytensors/_dispatch.py:537-543). Rows
whose target is ``ignore_index`` have zero loss; ``mean`` divides by the
number of other rows, as ``torch.nn.functional.cross_entropy`` and the
reference's reductions (/root/reference/src/polytensors/_fused_cross_entropy.py:163-170).
Arithmetic is float32 (float64 for float64 logits).
"""

import contextvars

import torch

from . import _complex, _gate, _lib, _ops
from ._tensor import PolyTensor

_enabled = contextvars.ContextVar("polytensors_amd_fused_cross_entropy", default=True)
_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def why_ineligible(input, target, weight=None, reduction="mean", label_smoothing=0.0, softcap=None,
                   allow_grad=False):
    if not _enabled.get():
        return ("the fused cross-entropy kernel is disabled (PolyTensor.fused_cross_entropy(False)) and "
                "polytensors_amd has no general series rules")
    if not isinstance(input, PolyTensor):
        return "logits must be a PolyTensor"
    if isinstance(weight, torch.Tensor) and weight.requires_grad and torch.is_grad_enabled():
        return "class weights that require grad are not supported (no gradient flows to weight)"
    # (degrees above the kernel's are composed from series operations, to the elementwise limit)
    reason = _gate.common_reason((input,), allow_plain_grad=allow_grad, complex_ok=True,
                                 max_degree=_gate.MAX_ELEMENTWISE_DEGREE)
    if reason is not None:
        return reason
    if input.ndim < 2:
        return "logits must be (N, C) or (N, C, d1, ...)"
    if input.dtype not in _DTYPES or any(_gate.real_dtype(c.dtype) != input.dtype for c in input.coeffs):
        return "logits must be float16/bfloat16/float32/float64 in every order"
    if isinstance(target, PolyTensor) or not isinstance(target, torch.Tensor) or target.dtype != torch.int64:
        return "targets must be an ordinary int64 tensor (class indices)"
    if target.shape != input.shape[:1] + input.shape[2:] or target.device != input.device:
        return "targets must be (N,) (or (N, d1, ...)) on the logits' device"
    if weight is not None and (isinstance(weight, PolyTensor) or not isinstance(weight, torch.Tensor) or
                               weight.shape != input.shape[1:2] or not weight.dtype.is_floating_point or
                               weight.device != input.device):
        return "class weights must be an ordinary floating (C,) tensor on the logits' device"
    if not 0.0 <= label_smoothing <= 1.0:
        return "label_smoothing must be in [0, 1]"
    if softcap is not None and (weight is not None or label_smoothing != 0.0):
        return "softcap with class weights or label smoothing is not implemented"
    if reduction not in _lib.REDUCTIONS:
        return f"unknown reduction {reduction!r}"
    if softcap is not None and not (isinstance(softcap, (int, float)) and 0 < softcap < float("inf")):
        return "softcap must be a positive finite number"
    return None


def eligible(input, target, weight=None, reduction="mean", label_smoothing=0.0, softcap=None):
    return why_ineligible(input, target, weight, reduction, label_smoothing, softcap) is None


def _rows(coeffs):
    """Coefficients whose rows are unit-stride with one common row stride (a padded slice is fine).

    Rows that overlap (a row stride below the row length, such as the stride 0
    of an expanded row) are made contiguous: the kernels read rows at
    ``row_stride >= classes`` apart.
    """
    first = coeffs[0]
    rows, classes = first.shape
    if (first.stride(-1) == 1 and (rows <= 1 or first.stride(0) >= classes)
            and all(c.stride() == first.stride() for c in coeffs)):
        return list(coeffs)
    return [c.contiguous() for c in coeffs]


class _SeriesCrossEntropy(torch.autograd.Function):
    """Per-row loss series with their degree-K gradient series.

    As /root/reference/src/polytensors/_fused_cross_entropy.py:101-128
    (_SeriesCrossEntropy): the forward kernel gives the per-row losses (and the
    lse series, saved); the backward kernel computes J(z(t))^T c(t) per row.
    Reductions are ordinary series operations on the per-row losses.
    """

    @staticmethod
    def forward(ctx, logits, target, ignore_index, softcap):
        z = _rows(logits.coeffs)
        target = target.contiguous()
        loss, lse = _ops.cross_entropy_series(z, target, int(ignore_index), 0, float(softcap or 0.0))
        ctx.save_for_backward(logits, target, lse)
        ctx.ignore_index, ctx.softcap = int(ignore_index), float(softcap or 0.0)
        return PolyTensor.from_stacked(loss)

    @staticmethod
    def backward(ctx, gradient):
        from ._plain import _plain_range
        if torch.is_grad_enabled():
            raise NotImplementedError("second-order reverse mode through the fused cross entropy is not implemented")
        logits, target, lse = ctx.saved_tensors
        degree = logits.degree
        coeffs = gradient.coeffs if isinstance(gradient, PolyTensor) else (gradient,)
        cot = [c.to(lse.dtype).expand(lse.shape[1:]).contiguous() for c in coeffs]
        cot += [torch.zeros_like(cot[0]) for _ in range(degree + 1 - len(cot))]
        token = _plain_range.set(True)   # the engine's thread does not see the caller's context
        try:
            dz = _ops.cross_entropy_series_backward(_rows(logits.coeffs), target, ctx.ignore_index, ctx.softcap,
                                                    lse, cot)
            dz = PolyTensor.from_stacked(dz)
        finally:
            _plain_range.reset(token)
        return dz, None, None, None


def fused(input, target, ignore_index=-100, reduction="mean", softcap=None, weight=None, label_smoothing=0.0):
    """Loss series (a PolyTensor in float32, or float64 for float64 logits).

    ``softcap`` caps the logit series as ``softcap * tanh(z / softcap)`` inside the
    kernel, as the reference's fused pass does at degree 1
    (/root/reference/src/polytensors/_cross_entropy_kernels.py:7-17). Under grad the
    per-row losses come from ``_SeriesCrossEntropy`` and the reduction is a series
    sum (and division by the count of kept rows), as the reference's
    /root/reference/src/polytensors/_fused_cross_entropy.py:163-170. Logits
    (N, C, d1, ...) are rows of C classes (moved last); class weights and label
    smoothing are ``_weighted``.
    """
    if _complex.has_complex(input):
        return _complex.at_real_nodes(fused, "cross_entropy", input, target, ignore_index=ignore_index,
                                      reduction=reduction, softcap=softcap, weight=weight,
                                      label_smoothing=label_smoothing)
    if input.ndim > 2:
        classes = input.shape[1]
        flat = fused(input.movedim(1, -1).reshape(-1, classes), target.reshape(-1), ignore_index, reduction, softcap,
                     weight, label_smoothing)
        return flat.reshape(target.shape) if reduction == "none" else flat
    if weight is not None or label_smoothing != 0.0:
        return _weighted(input, target, ignore_index, reduction, weight, label_smoothing)
    if input.degree > _gate.MAX_DEGREE or _gate.wrapper_grad(input):
        if input.degree > _gate.MAX_DEGREE:
            losses = _composed_losses(input, target, ignore_index, softcap)
        else:
            losses = _SeriesCrossEntropy.apply(input, target, ignore_index, softcap)
        if reduction == "none":
            return losses
        total = losses.sum()
        if reduction == "sum":
            return total
        count = (target != ignore_index).sum().to(losses.dtype)
        return total / count
    z = _rows(input.coeffs)
    loss, _ = _ops.cross_entropy_series(z, target.contiguous(), int(ignore_index), _lib.REDUCTIONS[reduction],
                                        float(softcap) if softcap is not None else 0.0)
    return PolyTensor.from_stacked(loss)


def _composed_losses(input, target, ignore_index, softcap):
    """Per-row loss series lse - z_y (zero for ignored rows) of (N, C) logits at degrees 9..16,
    above the row kernel's register plan.

    torch's cross_entropy as the reference's general rules decompose it (log-sum-exp and a gather,
    /root/reference/src/polytensors/_fused_cross_entropy.py:142 and _plain.py:262-273) in series
    operations: exp and log run the elementwise series kernels on the logits less the row maximum
    of their constant order (which changes only that order), the row sums and the gather act on
    each coefficient. The loss dtype is the kernel's: float32, or float64 for float64 logits.
    """
    dtype = torch.float64 if input.dtype == torch.float64 else torch.float32
    z = input if input.dtype == dtype else input.to(dtype)
    if softcap is not None:
        z = (z / softcap).tanh() * softcap
    top = z.coeffs[0].detach().amax(1, keepdim=True)
    lse = (z - top).exp().sum(1).log() + top.squeeze(1)
    keep = target != ignore_index
    safe = torch.where(keep, target, torch.zeros((), dtype=target.dtype, device=target.device))
    return (lse - z.gather(1, safe[:, None]).squeeze(1)) * keep.to(dtype)


def _weighted(input, target, ignore_index, reduction, weight, label_smoothing):
    """``F.cross_entropy`` with class weights w and label smoothing eps on (N, C) logits.

    The reference has no fused rule for these (/root/reference/src/polytensors/_fused_cross_entropy.py:142):
    torch's cross_entropy decomposes into log_softmax and linear loss terms, which
    its general rules apply to every order. Per kept row, with lse the row's
    log-sum-exp series and the kernel's loss l = lse - z_y:
        (1 - eps) w_y l + (eps / C) sum_c w_c (lse - z_c)
    (w = 1 without weights); ignored rows are zero, and "mean" divides by the kept
    rows' total target weight (their count without weights), as torch's
    cross_entropy. The smoothing sum is formed from the differences lse - z_c, which
    do not change when an order of the logits is shifted by a constant (as torch's
    sum of w_c (-log_softmax_c)); W lse - sum_c w_c z_c would subtract two sums that
    grow with such a shift. The terms beyond l are series operations on the logits
    (gather, broadcast difference, weighted row sums), so autograd records them as
    it does the kernel's losses.
    """
    losses = fused(input, target, ignore_index=ignore_index, reduction="none")
    dtype = losses.dtype
    keep = target != ignore_index
    safe = torch.where(keep, target, torch.zeros((), dtype=target.dtype, device=target.device))
    kept = keep.to(dtype)
    w = None if weight is None else weight.to(dtype)
    wy = kept if w is None else w[safe] * kept
    per_row = losses * wy
    if label_smoothing != 0.0:
        classes = input.shape[1]
        z = input if input.dtype == dtype else input.to(dtype)
        zy = z.gather(1, safe[:, None]).squeeze(1)
        gap = (losses + zy).unsqueeze(1) - z   # lse - z_c, every class
        smooth = (gap.sum(1) if w is None else (gap * w).sum(1)) * kept
        per_row = per_row * (1.0 - label_smoothing) + smooth * (label_smoothing / classes)
    if reduction == "none":
        return per_row
    total = per_row.sum()
    if reduction == "sum":
        return total
    return total / wy.sum()


def fused_or_raise(input, target, weight=None, ignore_index=-100, reduction="mean", label_smoothing=0.0):
    reason = why_ineligible(input, target, weight, reduction, label_smoothing,
                            allow_grad=_gate.wrapper_grad(input))
    if reason is not None:
        raise NotImplementedError(f"cross_entropy: {reason}")
    return fused(input, target, ignore_index=ignore_index, reduction=reduction, weight=weight,
                 label_smoothing=label_smoothing)


def cross_entropy(logits, target, softcap=None, ignore_index=-100, reduction="mean"):
    """``PolyTensor.cross_entropy``: series logits use the fused kernel (at least float32 out);
    ordinary tensors use the composite, as /root/reference/src/polytensors/_fused_cross_entropy.py:173-187."""
    if isinstance(logits, PolyTensor):
        reason = why_ineligible(logits, target, None, reduction, 0.0, softcap,
                                allow_grad=_gate.wrapper_grad(logits))
        if reason is not None:
            raise NotImplementedError(f"cross_entropy: {reason}")
        return fused(logits, target, ignore_index=ignore_index, reduction=reduction, softcap=softcap)
    logits = logits.to(torch.promote_types(logits.dtype, torch.float32))
    if softcap is not None:
        logits = softcap * torch.tanh(logits / softcap)
    return torch.nn.functional.cross_entropy(logits, target, ignore_index=ignore_index, reduction=reduction)
