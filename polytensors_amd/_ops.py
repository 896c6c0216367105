"""The ``polytensors_amd::*`` operators of the gfx950 Taylor kernels.

The operators are registered from C++ (``csrc/torch_ops.cpp``, built into
``_lib/libpolytaylor_torch.so``): TORCH_LIBRARY schemas and CUDA (HIP)
implementations that check their arguments, allocate the result and launch the
C-ABI entry points of ``libpolytaylor.so`` on the current HIP stream. Each takes
the K+1 coefficient tensors of a series as a ``Tensor[]`` (the reference's tuple
storage, passed without stacking copies) and returns one coefficient-stacked
tensor ``[K+1, ...]``; on any other device the dispatcher raises. This module
adds what belongs in Python: the fake (shape) implementations and the
coefficient-level autograd of every operator. Outputs never alias inputs.
"""

import math

import torch

from . import _lib

NAMESPACE = "polytensors_amd"

# The operators' schemas, as csrc/torch_ops.cpp defines them (tests/test_capi.py checks that
# the two agree). Without the built extension these alone are defined, with a HIP
# implementation that raises LibraryMissingError, so that every call fails loudly.
SCHEMAS = {
    "norm_series": "(Tensor[] x, Tensor[] weight, Tensor[] bias, int n, float eps, bool layer) -> Tensor",
    "norm_series_backward": "(Tensor[] x, Tensor[] grad, int n, float eps, bool layer) -> Tensor",
    "cross_entropy_series": ("(Tensor[] z, Tensor target, int ignore_index, int reduction, float softcap) "
                             "-> (Tensor, Tensor)"),
    "cross_entropy_series_backward": ("(Tensor[] z, Tensor target, int ignore_index, float softcap, Tensor lse, "
                                      "Tensor[] cot) -> Tensor"),
    "cauchy_matmul": "(Tensor[] a, Tensor[] b, int degree, bool trans_b) -> Tensor",
    "taylor_attention_fwd": ("(Tensor[] q, Tensor[] k, Tensor[] v, Tensor? mask, bool causal, float scale, "
                             "int degree, int[]? mask_map=None) -> (Tensor, Tensor)"),
    "taylor_attention_bwd": ("(Tensor[] q, Tensor[] k, Tensor[] v, Tensor out, Tensor lse, Tensor[] grad, "
                             "Tensor? mask, bool causal, float scale, int materialize=-1, int[]? mask_map=None) "
                             "-> (Tensor, Tensor, Tensor)"),
    "complex_to_real": "(Tensor[] src, float[] alpha, float[] beta) -> Tensor",
    "real_to_complex": "(Tensor[] src, int orders, float[] wre, float[] wim) -> Tensor",
    "activation_series": "(Tensor[] x, str kind) -> Tensor",
    "activation_series_backward": "(Tensor[] grad, Tensor[] saved, str kind) -> Tensor",
    "series_binary": "(Tensor[] a, Tensor[] b, str op) -> Tensor",
}

_fallback = []   # the Python library object of the stand-in schemas (kept alive)


def _register():
    if _lib.load_torch_ops():
        return True
    lib = torch.library.Library(NAMESPACE, "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(name + schema)

        def missing(*args, _name=name, **kwargs):
            _lib.load()   # raises LibraryMissingError naming the library to build
            raise _lib.LibraryMissingError(f"{_lib.TORCH_LIB_PATH} is not loaded: build it with "
                                           f"`python -m polytensors_amd.build` ({NAMESPACE}::{_name})")

        lib.impl(name, missing, "CUDA")
    _fallback.append(lib)
    return False


NATIVE = _register()   # True: the C++ extension registered the operators


_below_autograd = torch._C._AutoDispatchBelowAutograd


def _op(name):
    """The operator ``polytensors_amd::name``. With grad mode off no graph can be recorded, so the
    call goes straight to the HIP implementation, past the Python autograd kernel (which would
    only redispatch below itself)."""
    overload = getattr(getattr(torch.ops, NAMESPACE), name).default
    grad_enabled = torch.is_grad_enabled

    def call(*args, **kwargs):
        if grad_enabled():
            return overload(*args, **kwargs)
        with _below_autograd():
            return overload(*args, **kwargs)

    call.__name__ = call.__qualname__ = name
    call.overload = overload
    return call


def _acc_dtype(dtype):
    return torch.float64 if dtype == torch.float64 else torch.float32


# ---------------------------------------------------------------------------
# RMSNorm / LayerNorm series

norm_series = _op("norm_series")


@torch.library.register_fake(f"{NAMESPACE}::norm_series")
def _(x, weight, bias, n, eps, layer):
    return x[0].new_empty((len(x), *x[0].shape))


# ---------------------------------------------------------------------------
# Cross-entropy series

cross_entropy_series = _op("cross_entropy_series")


@torch.library.register_fake(f"{NAMESPACE}::cross_entropy_series")
def _(z, target, ignore_index, reduction, softcap):
    rows = z[0].shape[0]
    loss = z[0].new_empty((len(z), rows) if reduction == 0 else (len(z),), dtype=_acc_dtype(z[0].dtype))
    lse = z[0].new_empty((len(z), rows), dtype=_acc_dtype(z[0].dtype))
    return loss, lse


# ---------------------------------------------------------------------------
# Cauchy-product matmul

cauchy_matmul = _op("cauchy_matmul")


@torch.library.register_fake(f"{NAMESPACE}::cauchy_matmul")
def _(a, b, degree, trans_b):
    ba, m, _ = a[0].shape
    bb = b[0].shape[0]
    n = b[0].shape[1] if trans_b else b[0].shape[2]
    return a[0].new_empty((degree + 1, max(ba, bb), m, n))


# ---------------------------------------------------------------------------
# Taylor flash attention forward

def _mask_ranges(mask, lq, lk):
    """Block ranges of a bool (L, S) mask on its device, as the attention operators compute
    them internally (pt_attention_mask_ranges; a direct handle for tests)."""
    lib = _lib.load()
    ranges = torch.empty(max(lib.pt_attention_mask_ranges_count(lq, lk), 1), dtype=torch.int32, device=mask.device)
    _lib.check(lib.pt_attention_mask_ranges(mask.data_ptr(), 1, lq, lk, ranges.data_ptr(), _lib.stream_of(mask.device)),
               "attention_mask_ranges")
    return ranges


taylor_attention_fwd = _op("taylor_attention_fwd")


@torch.library.register_fake(f"{NAMESPACE}::taylor_attention_fwd")
def _(q, k, v, mask, causal, scale, degree, mask_map=None):
    *batch, lq, d = q[0].shape   # batch dimensions, flattened to bh heads in the lse series
    return (q[0].new_empty((degree + 1, *batch, lq, d)),
            q[0].new_empty((degree + 1, math.prod(batch), lq), dtype=_acc_dtype(q[0].dtype)))


def attention_gradient_series(q, k, v, out, lse, grad, mask, causal, scale, mask_map=None):
    """Gradient series (dq, dk, dv) of the attention forward for every operand dtype.

    bfloat16/float16 operands run the 16-bit backward kernels (16-bit MFMA
    operands, float32 accumulation; the forward's lse series is float32), as the
    reference's half-type backward accumulates in float32
    (/root/reference/src/polytensors/_fused_attention.py:72-78, tolerance 5e-2
    against float32, tests/test_fused_kernels.py:64-72).
    """
    return taylor_attention_bwd(q, k, v, out, lse, grad, mask, causal, scale, mask_map=mask_map)


taylor_attention_bwd = _op("taylor_attention_bwd")


@torch.library.register_fake(f"{NAMESPACE}::taylor_attention_bwd")
def _(q, k, v, out, lse, grad, mask, causal, scale, materialize=-1, mask_map=None):
    return (q[0].new_empty((len(q), *q[0].shape)), k[0].new_empty((len(k), *k[0].shape)),
            k[0].new_empty((len(k), *k[0].shape)))


# ---------------------------------------------------------------------------
# Complex directions: real variants and their recombination

_REAL_OF = {torch.complex64: torch.float32, torch.complex128: torch.float64}


complex_to_real = _op("complex_to_real")


@torch.library.register_fake(f"{NAMESPACE}::complex_to_real")
def _(src, alpha, beta):
    return src[0].new_empty((len(alpha), len(src), *src[0].shape), dtype=_REAL_OF[src[0].dtype])


real_to_complex = _op("real_to_complex")


@torch.library.register_fake(f"{NAMESPACE}::real_to_complex")
def _(src, orders, wre, wim):
    cplx = torch.complex64 if src[0].dtype == torch.float32 else torch.complex128
    return src[0].new_empty((orders, *src[0].shape), dtype=cplx)


# ---------------------------------------------------------------------------
# Elementwise activation series

activation_series = _op("activation_series")


@torch.library.register_fake(f"{NAMESPACE}::activation_series")
def _(x, kind):
    return x[0].new_empty((len(x), *x[0].shape))


activation_series_backward = _op("activation_series_backward")


@torch.library.register_fake(f"{NAMESPACE}::activation_series_backward")
def _(grad, saved, kind):
    return grad[0].new_empty((len(grad), *grad[0].shape))


# ---------------------------------------------------------------------------
# Elementwise series product / quotient

series_binary = _op("series_binary")


@torch.library.register_fake(f"{NAMESPACE}::series_binary")
def _(a, b, op):
    return a[0].new_empty((len(a), *a[0].shape))


norm_series_backward = _op("norm_series_backward")


@torch.library.register_fake(f"{NAMESPACE}::norm_series_backward")
def _(x, grad, n, eps, layer):
    return x[0].new_empty((len(x), *x[0].shape))


cross_entropy_series_backward = _op("cross_entropy_series_backward")


@torch.library.register_fake(f"{NAMESPACE}::cross_entropy_series_backward")
def _(z, target, ignore_index, softcap, lse, cot):
    return z[0].new_empty((len(z), *z[0].shape))


# ---------------------------------------------------------------------------
# Coefficient-level autograd (PolyTensor.coefficient_autograd).
#
# Each op above maps input coefficients to output coefficients, y_k being
# coefficient k of f(x(t)). Perturbing x_j by d adds d t^j to x(t), so
# dy_k/dx_j = J_{k-j}, coefficient k-j of the Jacobian along the curve, and the
# vector-Jacobian product with output cotangents c_0..c_K is
#     dL/dx_i = sum_{k>=i} J_{k-i}^T c_k,
# which is coefficient K-i of the gradient series J(x(t))^T G(t) for the
# reversed cotangents G_k = c_{K-k}: the backward kernels' own product, read in
# reverse (at degree 1 the reference's "VJP with cotangents (G1, G0) and orders
# swapped", /root/reference/docs/api.md:148-153). An operand given with one
# order (an ordinary tensor) gets coefficient K. The backwards of the Cauchy
# matmul, the series product and quotient, exp and log are themselves products
# of those operators, so they differentiate again (further reverse derivatives,
# as the reference's general rules allow, /root/reference/docs/api.md:137-139).
# The norm, cross-entropy, attention and other activation backwards are single
# gradient-series kernels without a kernel for their own derivative. When a graph
# of the gradient is asked for (create_graph), the norm, cross entropy and
# attention are recomposed from series operations and differentiated
# (``_regraded``), and tanh, sigmoid, silu, gelu and gelu_tanh form G (*) f' from
# series products (``_series_derivative``).

def _reversed(grad):
    """Cotangents of a stacked [K+1, ...] output in reverse order, as a coefficient list."""
    return list(grad.flip(0).unbind(0))


def _read_back(series, orders):
    """Gradients of an operand with ``orders`` coefficients from a gradient series of reversed cotangents."""
    top = series.shape[0] - 1
    return [series[top - i] for i in range(orders)]


def _grads_flag(tensors):
    return any(t.requires_grad for t in tensors)


def _returned(ctx, *grads):
    """``grads`` padded with None to the number of arguments the call passed: torch matches the
    backward's return to the arguments given (defaulted ones excluded, and so is a keyword
    argument passed at its default), whose structure ``ctx.needs_input_grad`` has here."""
    return tuple(grads) + (None,) * (len(ctx.needs_input_grad) - len(grads))


def _once(what):
    if torch.is_grad_enabled():
        raise NotImplementedError(f"{what}: second-order coefficient autograd through the fused kernels "
                                  "is not implemented")


def _regraded(inputs, cotangents, compose):
    """A fused operation's gradient as a graph (create_graph), for further reverse derivatives.

    The operation is recomputed from its saved input coefficients by ``compose`` in series
    operations whose backwards are products of the series kernels (the compositions of the degree
    9..16 paths, as the reference's general rules), and differentiated with create_graph: the
    gradient is then a function of the inputs and cotangents that autograd can differentiate
    again. ``inputs`` are lists of coefficient tensors; returns one list of gradients per list
    (zeros where a coefficient takes no part).
    """
    from ._plain import _plain_range
    from ._tensor import _coefficient_autograd_enabled

    flat = [t for xs in inputs for t in xs]
    wanted = [t for t in flat if t.requires_grad]
    tokens = (_plain_range.set(True), _coefficient_autograd_enabled.set(True))
    try:
        pairs = [(y, c) for y, c in zip(compose(*inputs), cotangents) if y.requires_grad]
        got = torch.autograd.grad([y for y, _ in pairs], wanted, [c for _, c in pairs], create_graph=True,
                                  allow_unused=True) if wanted and pairs else [None] * len(wanted)
    finally:
        _coefficient_autograd_enabled.reset(tokens[1])
        _plain_range.reset(tokens[0])
    by_id = {id(t): g for t, g in zip(wanted, got)}
    result = []
    for xs in inputs:
        result.append([by_id.get(id(t)) if by_id.get(id(t)) is not None else torch.zeros_like(t) for t in xs])
    return result


def _poly(coeffs, degree=None):
    """A PolyTensor of coefficient tensors (an operand with fewer orders padded with zeros)."""
    from ._tensor import PolyTensor

    return PolyTensor(tuple(coeffs), degree=degree)


def _norm_setup(ctx, inputs, output):
    x, weight, bias, n, eps, layer = inputs
    ctx.save_for_backward(*x)
    ctx.meta = (n, eps, layer, bool(weight) or bool(bias))
    ctx.n_inputs = len(inputs)


def _norm_backward(ctx, grad):
    n, eps, layer, affine = ctx.meta
    if affine:
        raise NotImplementedError("norm_series: the fused weight/bias has no coefficient gradient; under "
                                  "autograd apply them as separate series operations")
    x = list(ctx.saved_tensors)
    if torch.is_grad_enabled():   # a graph of the gradient: the composed norm, differentiated
        from ._fused_norm import _composed

        def compose(xs):
            y = _composed(_poly([c.reshape(-1, n) for c in xs]), (n,), None, None, eps, layer)
            return [c.reshape(xs[0].shape) for c in y.coeffs]

        (dx,) = _regraded([x], list(grad.unbind(0)), compose)
        return _returned(ctx, dx, [], [])
    dx = norm_series_backward(x, _reversed(grad), n, eps, layer)
    return _returned(ctx, _read_back(dx, len(x)), [], [])


torch.library.register_autograd(f"{NAMESPACE}::norm_series", _norm_backward, setup_context=_norm_setup)


def _ce_setup(ctx, inputs, output):
    z, target, ignore_index, reduction, softcap = inputs
    ctx.mark_non_differentiable(output[1])
    ctx.save_for_backward(*z, target, output[1])
    ctx.meta = (len(z), ignore_index, reduction, softcap)
    ctx.n_inputs = len(inputs)


def _ce_backward(ctx, grad_loss, grad_lse):
    n, ignore_index, reduction, softcap = ctx.meta
    saved = ctx.saved_tensors
    z, target, lse = list(saved[:n]), saved[n], saved[n + 1]
    if torch.is_grad_enabled():   # a graph of the gradient: the composed loss, differentiated
        from ._fused_cross_entropy import _composed_losses

        def compose(zs):
            losses = _composed_losses(_poly(zs), target, ignore_index, softcap or None)
            if reduction != 0:
                losses = losses.sum()
                if reduction == 1:
                    losses = losses / (target != ignore_index).sum().to(losses.dtype)
            return [c.to(grad_loss.dtype) for c in losses.coeffs]

        (dz,) = _regraded([z], list(grad_loss.unbind(0)), compose)
        return _returned(ctx, dz)
    rows = z[0].shape[0]
    cot = grad_loss.to(lse.dtype)
    if reduction != 0:   # per-row cotangents of the sum (ignored rows have zero loss and gradient)
        cot = cot[:, None].expand(n, rows)
        if reduction == 1:
            cot = cot / (target != ignore_index).sum().to(lse.dtype)
    dz = cross_entropy_series_backward(z, target, ignore_index, softcap, lse,
                                       [c.contiguous() for c in cot.flip(0).unbind(0)])
    return _returned(ctx, _read_back(dz, n))


torch.library.register_autograd(f"{NAMESPACE}::cross_entropy_series", _ce_backward, setup_context=_ce_setup)


def _mm_setup(ctx, inputs, output):
    a, b, degree, trans_b = inputs
    ctx.save_for_backward(*a, *b)
    ctx.meta = (len(a), len(b), degree, trans_b, _grads_flag(a), _grads_flag(b))
    ctx.n_inputs = len(inputs)


def _mm_backward(ctx, grad):
    na, nb, degree, trans_b, need_a, need_b = ctx.meta
    saved = ctx.saved_tensors
    a, b = list(saved[:na]), list(saved[na:])
    c = _reversed(grad)                     # [batch, m, n] each
    batch = grad.shape[1]
    ga = gb = None
    if need_a:   # dA = C (*) B^T
        da = cauchy_matmul(c, b, degree, not trans_b)
        if a[0].shape[0] == 1 and batch > 1:
            da = da.sum(1, keepdim=True)
        ga = _read_back(da, na)
    if need_b:   # dB = A^T (*) C, or its transpose for a [batch, n, k] operand
        if trans_b:
            db = cauchy_matmul([x.transpose(-1, -2).contiguous() for x in c], a, degree, False)
        else:
            db = cauchy_matmul([x.transpose(-1, -2).contiguous() for x in a], c, degree, False)
        if b[0].shape[0] == 1 and batch > 1:
            db = db.sum(1, keepdim=True)
        gb = _read_back(db, nb)
    return _returned(ctx, ga if ga is not None else [None] * na, gb if gb is not None else [None] * nb)


torch.library.register_autograd(f"{NAMESPACE}::cauchy_matmul", _mm_backward, setup_context=_mm_setup)


def _attn_setup(ctx, inputs, output):
    q, k, v, mask, causal, scale, degree = inputs[:7]
    mask_map = inputs[7] if len(inputs) > 7 else None
    out, lse = output
    ctx.mark_non_differentiable(lse)
    ctx.save_for_backward(*q, *k, *v, out, lse, *([] if mask is None else [mask]))
    ctx.meta = (len(q), len(k), len(v), mask is not None, causal, scale, degree, mask_map)
    ctx.n_inputs = len(inputs)


def _attn_backward(ctx, grad_out, grad_lse):
    nq, nk, nv, has_mask, causal, scale, degree, mask_map = ctx.meta
    s = ctx.saved_tensors
    q, k, v = list(s[:nq]), list(s[nq:nq + nk]), list(s[nq + nk:nq + nk + nv])
    out, lse = s[nq + nk + nv], s[nq + nk + nv + 1]
    mask = s[-1] if has_mask else None

    shape_q, shape_k = q[0].shape, k[0].shape   # [..., L, d], [..., S, d]: flattened to [bh, T, d] here
    if torch.is_grad_enabled():   # a graph of the gradient: the composed attention, differentiated
        from ._fused_attention import _composed

        bh = math.prod(shape_q[:-2])
        full_mask = None
        if mask is not None:   # the mask of every flattened head (bool or additive)
            if mask_map is None:
                full_mask = mask.reshape(mask.shape[-2:])
            else:
                div, outer, inner = mask_map
                heads = torch.arange(bh, device=mask.device)
                full_mask = mask[(heads // div) * outer + (heads % div) * inner]

        def compose(qs, ks, vs):
            flat = lambda xs: _poly([x.reshape(-1, *x.shape[-2:]) for x in xs], degree)   # noqa: E731
            y = _composed(flat(qs), flat(ks), flat(vs), full_mask, causal, scale)
            return [c.reshape(shape_q) for c in y.coeffs]

        dq, dk, dv = _regraded([q, k, v], list(grad_out.unbind(0)), compose)
        return _returned(ctx, dq, dk, dv)

    def full(xs):   # the backward kernels take every order; an ordinary operand has zero higher orders
        xs = [x.reshape(-1, *x.shape[-2:]) for x in xs]
        return xs + [torch.zeros_like(xs[0]) for _ in range(degree + 1 - len(xs))]

    dq, dk, dv = attention_gradient_series(full(q), full(k), full(v), out.reshape(degree + 1, -1, *shape_q[-2:]),
                                           lse, full(_reversed(grad_out)), mask, causal, scale, mask_map)
    return _returned(ctx, _read_back(dq.view(degree + 1, *shape_q), nq), _read_back(dk.view(degree + 1, *shape_k), nk),
                     _read_back(dv.view(degree + 1, *shape_k), nv))


torch.library.register_autograd(f"{NAMESPACE}::taylor_attention_fwd", _attn_backward, setup_context=_attn_setup)

# the derivative's saved series: the input, or the output where the backward operation takes it
_ACT_SAVES_OUTPUT = ("tanh", "sigmoid", "exp", "sqrt", "rsqrt")
# kinds whose gradient series is a product of forward series (differentiable again)
_ACT_PRODUCT_BACKWARD = ("exp", "log", "sin", "cos", "sqrt", "rsqrt")


def _act_setup(ctx, inputs, output):
    x, kind = inputs
    ctx.kind = kind
    ctx.n_inputs = len(inputs)
    if kind in _ACT_SAVES_OUTPUT:
        ctx.save_for_backward(output)
    else:
        ctx.save_for_backward(*x)


def _series_derivative(kind, saved):
    """The derivative series f'(x(t)) of tanh, sigmoid, silu, gelu and gelu_tanh from series
    products, sums, the forward kernels and per-coefficient torch operations (so that the gradient
    series G (*) f' differentiates again): tanh' = 1 - y^2 and sigmoid' = y - y^2 from the saved
    output y; silu' = s + x s (1 - s) with s = sigmoid(x); gelu' = Phi(x) + x phi(x), the normal
    density phi from the exp kernel and the normal distribution Phi from its ODE
    (Phi' = phi: k Phi_k = sum_j j x_j phi_{k-j}); gelu_tanh' = (1 + t) / 2 + x (1 - t^2) c (1 + 3 a x^2) / 2
    with t = tanh(c (x + a x^3)), c = sqrt(2 / pi), a = 0.044715."""
    def mul(a, b):
        return list(series_binary(a, b, "mul").unbind(0))

    def affine(series, scale, shift):   # scale * series + shift (the shift on the constant order)
        return [scale * c + (shift if k == 0 else 0.0) for k, c in enumerate(series)]

    def add(a, b):
        return [x + y for x, y in zip(a, b)]

    if kind == "tanh":
        return affine(mul(saved, saved), -1.0, 1.0)
    if kind == "sigmoid":
        return add(saved, affine(mul(saved, saved), -1.0, 0.0))
    x = saved
    if kind == "gelu":   # Phi(x) + x phi(x), phi = exp(-x^2 / 2) / sqrt(2 pi), Phi by its ODE k Phi_k = sum j x_j phi_{k-j}
        phi = [c / math.sqrt(2.0 * math.pi) for c in activation_series(affine(mul(x, x), -0.5, 0.0), "exp").unbind(0)]
        cdf = [torch.special.ndtr(x[0])]
        for k in range(1, len(x)):
            cdf.append(sum(j * x[j] * phi[k - j] for j in range(1, k + 1)) / k)
        return add(cdf, mul(x, phi))
    if kind == "silu":
        sg = list(activation_series(x, "sigmoid").unbind(0))
        return add(sg, mul(x, mul(sg, affine(sg, -1.0, 1.0))))
    c, a = math.sqrt(2.0 / math.pi), 0.044715
    x2 = mul(x, x)
    t = list(activation_series(affine(add(x, affine(mul(x2, x), a, 0.0)), c, 0.0), "tanh").unbind(0))
    slope = mul(affine(mul(t, t), -1.0, 1.0), affine(x2, 3.0 * a * c, c))
    return add(affine(t, 0.5, 0.5), affine(mul(x, slope), 0.5, 0.0))


def _act_backward(ctx, grad):
    kind = ctx.kind
    regraph = torch.is_grad_enabled() and kind in ("tanh", "sigmoid", "silu", "gelu", "gelu_tanh")
    if kind not in _ACT_PRODUCT_BACKWARD and not regraph:
        _once(f"activation_series ({kind})")
    saved = ctx.saved_tensors
    saved = list(saved[0].unbind(0)) if kind in _ACT_SAVES_OUTPUT else list(saved)
    g = _reversed(grad)
    if regraph:            # a graph of the gradient: G (*) f' in differentiable series operations
        dx = series_binary(g, _series_derivative(kind, saved), "mul")
    elif kind == "exp":    # exp' = exp: the gradient series is G (*) y
        dx = series_binary(g, saved, "mul")
    elif kind == "log":    # log' = 1/x: G / x
        dx = series_binary(g, saved, "div")
    elif kind == "sin":    # sin' = cos
        dx = series_binary(g, list(activation_series(saved, "cos").unbind(0)), "mul")
    elif kind == "cos":    # cos' = -sin
        dx = -series_binary(g, list(activation_series(saved, "sin").unbind(0)), "mul")
    elif kind == "sqrt":   # sqrt' = 1 / (2 y)
        dx = 0.5 * series_binary(g, saved, "div")
    elif kind == "rsqrt":  # rsqrt' = -y^3 / 2
        y2 = list(series_binary(saved, saved, "mul").unbind(0))
        y3 = list(series_binary(y2, saved, "mul").unbind(0))
        dx = -0.5 * series_binary(g, y3, "mul")
    else:
        dx = activation_series_backward(g, saved, kind)
    return _returned(ctx, _read_back(dx, len(saved)))


torch.library.register_autograd(f"{NAMESPACE}::activation_series", _act_backward, setup_context=_act_setup)


def _binary_setup(ctx, inputs, output):
    a, b, op = inputs
    ctx.op = op
    ctx.n = len(a)
    ctx.n_inputs = len(inputs)
    # (the quotient's output saved whole: a view of it made here would be saved without its
    # graph, and a second derivative would treat it as a constant)
    ctx.save_for_backward(*a, *b, *([output] if op == "div" else []))


def _binary_backward(ctx, grad):
    n, op = ctx.n, ctx.op
    s = ctx.saved_tensors
    a, b = list(s[:n]), list(s[n:2 * n])
    g = _reversed(grad)
    if op == "mul":        # d(a b) = b da + a db
        da, db = series_binary(g, b, "mul"), series_binary(g, a, "mul")
    else:                  # d(a / b) = da / b - (a / b) db / b
        y = list(s[2 * n].unbind(0))
        da = series_binary(g, b, "div")
        db = -series_binary(list(series_binary(g, y, "mul").unbind(0)), b, "div")
    return _returned(ctx, _read_back(da, n), _read_back(db, n))


torch.library.register_autograd(f"{NAMESPACE}::series_binary", _binary_backward, setup_context=_binary_setup)


# The complex-direction plumbing is linear in its inputs. Its gradients follow torch's
# convention for complex tensors (the gradient of a real loss L with respect to a complex z is
# dL/dRe z + i dL/dIm z), since in coefficient autograd the complex higher coefficients are
# ordinary complex leaves: for v_a = alpha_a Re p + beta_a Im p the gradient of plane p is
# sum_a (alpha_a + i beta_a) g_a; for y_k = sum_m w_m x_{m,k} with real x it is Re(conj(w_m) g_k).
# Both are written with torch operations, so they differentiate again.

def _c2r_setup(ctx, inputs, output):
    src, alpha, beta = inputs
    ctx.meta = (len(src), list(alpha), list(beta))
    ctx.n_inputs = len(inputs)


def _c2r_backward(ctx, grad):
    planes, alpha, beta = ctx.meta
    shape = (len(alpha),) + (1,) * (grad.dim() - 1)
    a = torch.tensor(alpha, dtype=grad.dtype, device=grad.device).view(shape)
    b = torch.tensor(beta, dtype=grad.dtype, device=grad.device).view(shape)
    gp = torch.complex((a * grad).sum(0), (b * grad).sum(0))   # [planes, ...]
    return _returned(ctx, list(gp.unbind(0)))


torch.library.register_autograd(f"{NAMESPACE}::complex_to_real", _c2r_backward, setup_context=_c2r_setup)


def _r2c_setup(ctx, inputs, output):
    src, orders, wre, wim = inputs
    ctx.meta = (len(src), orders, list(wre), list(wim))
    ctx.n_inputs = len(inputs)


def _r2c_backward(ctx, grad):
    n, orders, wre, wim = ctx.meta
    re, im = grad.real, grad.imag   # [orders, ...]
    grads = []
    for m in range(n // orders):
        for k in range(orders):
            grads.append(wre[m] * re[k] + wim[m] * im[k])
    return _returned(ctx, grads)


torch.library.register_autograd(f"{NAMESPACE}::real_to_complex", _r2c_backward, setup_context=_r2c_setup)
