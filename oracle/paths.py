"""The four hot-path operations of the oracle (test infrastructure only; see oracle/__init__.py).

Each restates the reference's plain-range general path, operation for
operation, on lists of K+1 CPU coefficient tensors. An ordinary operand is a
list of one tensor; ``lift`` pads it with zero orders as the reference does
(/root/reference/src/polytensors/_range_ops.py:37-45).
"""

import math

import torch
import torch.nn.functional as F

from .series import cauchy, rsqrt_series, softmax_family


def lift(x, degree):
    x = list(x)
    return x + [torch.zeros_like(x[0]) for _ in range(degree + 1 - len(x))]


def _mean(X, dims):
    # sum then divide by the element count: /root/reference/src/polytensors/_range_ops.py:178-193
    divisor = 1
    for d in dims:
        divisor *= X[0].shape[d]
    return [c.sum(dim=dims, keepdim=True) / divisor for c in X]


def _add_to_order0(X, value):
    # constant operand: only order 0 changes, /root/reference/src/polytensors/_range_ops.py:122-132
    return [X[0] + value] + [c.clone() for c in X[1:]]


def _affine(out, weight, bias):
    if weight is not None:
        out = [c * weight[0] for c in out] if len(weight) == 1 else cauchy(out, lift(weight, len(out) - 1))
    if bias is not None:
        out = _add_to_order0(out, bias[0]) if len(bias) == 1 else [c + b for c, b in zip(out, bias)]
    return out


def rms_norm(X, normalized_shape, weight=None, eps=None):
    """Series of ``input * rsqrt(mean(input*input) + eps) [* weight]``.

    /root/reference/src/polytensors/_decompositions.py:14-22 (_rms_norm); eps
    defaults to finfo(dtype).eps (:16-17); input*input and input*r are Cauchy
    products (_range_ops.py:143-144); rsqrt is _series.py:83-96. ``weight`` is a
    list of 1 (ordinary) or K+1 coefficients.
    """
    dims = tuple(range(-len(normalized_shape), 0))
    eps = torch.finfo(X[0].dtype).eps if eps is None else eps
    s = _add_to_order0(_mean(cauchy(X, X), dims), eps)
    out = cauchy(X, rsqrt_series(s))
    return _affine(out, weight, None)


def layer_norm(X, normalized_shape, weight=None, bias=None, eps=1e-5):
    """Series of ``(x - mean x) * rsqrt(mean((x - mean x)^2) + eps) [* w] [+ b]``.

    The reference has no layer-norm rule (/root/reference/docs/notes.md:33-35);
    this is the composite of its rules: mean (_range_ops.py:178-193), series
    subtraction (:140-142), Cauchy products (:143-144) and rsqrt (_series.py:83-96).
    """
    dims = tuple(range(-len(normalized_shape), 0))
    mu = _mean(X, dims)
    C = [x - m for x, m in zip(X, mu)]
    s = _add_to_order0(_mean(cauchy(C, C), dims), eps)
    out = cauchy(C, rsqrt_series(s))
    return _affine(out, weight, bias)


def rms_norm_backward(X, G, normalized_shape, eps=None):
    """Gradient series of the RMSNorm normalization (no weight): the series of
    ``g * r - x * r**3 * mean(x * g)``, r = rsqrt(mean(x*x) + eps), every product a
    Cauchy product -- the reference's backward formula
    /root/reference/src/polytensors/_fused_norm.py:52-56 evaluated on series.
    """
    dims = tuple(range(-len(normalized_shape), 0))
    eps = torch.finfo(X[0].dtype).eps if eps is None else eps
    r = rsqrt_series(_add_to_order0(_mean(cauchy(X, X), dims), eps))
    r3 = cauchy(cauchy(r, r), r)
    dot = _mean(cauchy(X, G), dims)
    return [a - b for a, b in zip(cauchy(G, r), cauchy(X, cauchy(r3, dot)))]


def layer_norm_backward(X, G, normalized_shape, eps=1e-5):
    """Gradient series of the LayerNorm normalization (no affine terms): with
    d = x - mean(x) and r = rsqrt(mean(d*d) + eps), the series of
    ``r * (g - mean(g)) - d * r**3 * mean(d * g)`` (Cauchy products), the composite
    rules' VJP (the reference has no layer-norm rule, docs/notes.md:33-35).
    """
    dims = tuple(range(-len(normalized_shape), 0))
    D = [x - m for x, m in zip(X, _mean(X, dims))]
    r = rsqrt_series(_add_to_order0(_mean(cauchy(D, D), dims), eps))
    r3 = cauchy(cauchy(r, r), r)
    Gc = [g - m for g, m in zip(G, _mean(G, dims))]
    dot = _mean(cauchy(D, G), dims)
    return [a - b for a, b in zip(cauchy(r, Gc), cauchy(D, cauchy(r3, dot)))]


def attention(Q, K, V, attn_mask=None, is_causal=False, scale=None):
    """Series of ``softmax((Q*scale) @ K^T masked) @ V``.

    /root/reference/src/polytensors/_decompositions.py:28-43 (_attention):
    scale defaults to 1/sqrt(d); a masked score becomes (-inf, 0, ..., 0)
    (masked_fill of the lifted -inf, _range_ops.py:271-277 with _plain.py:70-75);
    a float mask is added to order 0; softmax is _plain.py:262-273; both
    products are Cauchy matmuls (_plain.py:118-128). A row with no admissible
    key is NaN here, as in the reference's general rule.
    """
    degree = max(len(Q), len(K), len(V)) - 1
    Q, K, V = lift(Q, degree), lift(K, degree), lift(V, degree)
    L, S = Q[0].shape[-2], K[0].shape[-2]
    scale = 1 / math.sqrt(Q[0].shape[-1]) if scale is None else scale
    scores = cauchy([q * scale for q in Q], [k.transpose(-2, -1) for k in K], matmul=True)

    def masked_fill(series, excluded):
        return [torch.where(excluded, torch.full((), float("-inf") if k == 0 else 0.0, dtype=c.dtype), c)
                for k, c in enumerate(series)]

    if is_causal:
        keep = torch.ones(L, S, dtype=torch.bool).tril(diagonal=0)
        scores = masked_fill(scores, ~keep)
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            scores = masked_fill(scores, ~attn_mask)
        else:
            scores = _add_to_order0(scores, attn_mask)
    probabilities = softmax_family(scores, -1)[0]
    return cauchy(probabilities, V, matmul=True)


def attention_backward(Q, K, V, G, attn_mask=None, is_causal=False, scale=None):
    """Gradient series (dQ, dK, dV) of ``attention`` for the output cotangent series ``G``.

    The vector-Jacobian product of softmax(scale Q K^T) V evaluated on series,
    every product a Cauchy product: P = softmax series of the masked scores
    (_plain.py:262-273), dV = P^T G, dP = G V^T, dS = P (dP - rowsum(P dP)),
    dQ = scale dS K, dK = scale dS^T Q -- the reference's degree-1 backward
    (/root/reference/src/polytensors/_attention_kernels.py:85-201) at degree K.
    A float mask is added to the order-0 scores (as in ``attention``); its -inf
    entries exclude their keys. A query row with no admissible key has P = 0, as
    in the fused kernels (lse = +inf, _attention_kernels.py:80-81).
    """
    degree = max(len(Q), len(K), len(V), len(G)) - 1
    Q, K, V, G = (lift(x, degree) for x in (Q, K, V, G))
    L, S = Q[0].shape[-2], K[0].shape[-2]
    scale = 1 / math.sqrt(Q[0].shape[-1]) if scale is None else scale
    scores = cauchy([q * scale for q in Q], [k.transpose(-2, -1) for k in K], matmul=True)
    keep = torch.ones(L, S, dtype=torch.bool)
    if is_causal:
        keep = keep.tril(diagonal=0)
    if attn_mask is not None and attn_mask.dtype == torch.bool:
        keep = keep & attn_mask
    elif attn_mask is not None:
        keep = keep & ~torch.isneginf(attn_mask)
        scores = _add_to_order0(scores, torch.where(keep, attn_mask, torch.zeros((), dtype=attn_mask.dtype)))
    scores = [torch.where(keep, c, torch.full((), float("-inf") if k == 0 else 0.0, dtype=c.dtype))
              for k, c in enumerate(scores)]
    empty = ~keep.any(-1, keepdim=True)
    P = [torch.where(empty, torch.zeros((), dtype=p.dtype), p) for p in softmax_family(scores, -1)[0]]
    Pt = [p.transpose(-2, -1) for p in P]
    dV = cauchy(Pt, G, matmul=True)
    dP = cauchy(G, [v.transpose(-2, -1) for v in V], matmul=True)
    row = [x.sum(-1, keepdim=True) for x in cauchy(P, dP)]
    dS = cauchy(P, [a - b for a, b in zip(dP, row)])
    dQ = [scale * x for x in cauchy(dS, K, matmul=True)]
    dK = [scale * x for x in cauchy([d.transpose(-2, -1) for d in dS], Q, matmul=True)]
    return dQ, dK, dV


def cross_entropy(Z, target, ignore_index=-100, reduction="mean", softcap=None, weight=None, label_smoothing=0.0):
    """Per-order loss series of ``F.cross_entropy(z, target)`` on (N, C) logits.

    The log-softmax series (/root/reference/src/polytensors/_plain.py:262-273)
    followed by native NLL on every order (/root/reference/src/polytensors/_dispatch.py:537-543).
    With ``softcap`` the logits are first ``softcap * tanh(z / softcap)``, the
    composite of /root/reference/src/polytensors/_fused_cross_entropy.py:184-187:
    per-coefficient scalar division and product around the plain-range tanh
    rule (_plain.py:256-259, 303-304). With class weights or label smoothing the
    reference has no fused rule (_fused_cross_entropy.py:142) and torch's
    cross_entropy decomposes into log_softmax and its linear loss terms
    (/root/reference/src/polytensors/_decompositions.py:66-67), applied here to
    every order of the log-softmax series (``_smoothed``).
    """
    if softcap is not None:
        from .activations import activation

        Z = [softcap * t for t in activation([z / softcap for z in Z], "tanh")]
    _, log_softmax, _ = softmax_family(Z, 1)
    if weight is None and label_smoothing == 0.0:
        return [_nll(lp, target, ignore_index, reduction) for lp in log_softmax]
    return [_smoothed(lp, target, weight, ignore_index, reduction, label_smoothing) for lp in log_softmax]


def _smoothed(lp, target, weight, ignore_index, reduction, eps):
    """torch's cross-entropy terms of one order of log-probabilities ``lp`` (N, C): (1 - eps) times
    the weighted NLL -w_y lp_y plus eps / C times -sum_c w_c lp_c, both zero on ignored rows;
    "mean" divides by the kept rows' total target weight (the count without weights)."""
    C = lp.shape[1]
    keep = target != ignore_index
    safe = torch.where(keep, target, torch.zeros((), dtype=target.dtype))
    w = torch.ones(C, dtype=lp.real.dtype) if weight is None else weight.to(lp.real.dtype)
    wy = torch.where(keep, w[safe], torch.zeros((), dtype=w.dtype))
    nll = -lp.gather(1, safe[:, None]).squeeze(1) * wy
    smooth = torch.where(keep, -(lp * w).sum(1), torch.zeros((), dtype=lp.dtype))
    per_row = (1 - eps) * nll + (eps / C) * smooth
    if reduction == "none":
        return per_row
    if reduction == "sum":
        return per_row.sum()
    return per_row.sum() / wy.sum()


def _nll(lp, target, ignore_index, reduction):
    """Native NLL of one order; a complex order is split into its real and imaginary parts (NLL is
    linear), as /root/reference/src/polytensors/_dispatch.py:12-26,537-543."""
    if lp.is_complex():
        return torch.complex(F.nll_loss(lp.real, target, ignore_index=ignore_index, reduction=reduction),
                             F.nll_loss(lp.imag, target, ignore_index=ignore_index, reduction=reduction))
    return F.nll_loss(lp, target, ignore_index=ignore_index, reduction=reduction)


def cross_entropy_backward(Z, target, C, ignore_index=-100, softcap=None):
    """Gradient series of the per-row losses w.r.t. (N, C) logits for per-row cotangents C:
    c (*) (softmax(z) - e_y) per kept row, zero for ignored rows, times the series of
    1 - tanh(z / cap)^2 with a softcap -- the reference's degree-1 backward
    (/root/reference/src/polytensors/_cross_entropy_kernels.py:58-85) in series arithmetic,
    with the softmax series of _plain.py:262-273.
    """
    from .activations import activation

    if softcap is not None:
        T = activation([z / softcap for z in Z], "tanh")
        Zc = [softcap * t for t in T]
        dT = [(1 if k == 0 else 0) - s for k, s in enumerate(cauchy(T, T))]
    else:
        Zc = Z
    p = softmax_family(Zc, 1)[0]
    onehot = torch.zeros_like(p[0])
    keep = target != ignore_index
    onehot[keep.nonzero().squeeze(1), target[keep]] = 1
    p = [p[0] - onehot] + p[1:]
    Cr = [torch.where(keep, c, torch.zeros_like(c)).unsqueeze(1) for c in C]
    dz = cauchy(Cr, p)
    return cauchy(dz, dT) if softcap is not None else dz


def logsumexp(Z, dim=-1):
    """Log-sum-exp series along ``dim`` (keepdim squeezed), /root/reference/src/polytensors/_plain.py:262-273."""
    return [c.squeeze(dim) for c in softmax_family(Z, dim)[2]]


def matmul(A, B):
    """Cauchy-product matmul, /root/reference/src/polytensors/_plain.py:118-128."""
    degree = max(len(A), len(B)) - 1
    return cauchy(lift(A, degree), lift(B, degree), matmul=True)
