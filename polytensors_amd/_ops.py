"""``torch.library`` custom ops of the gfx950 Taylor kernels.

Each op takes the K+1 coefficient tensors of a series as a ``Tensor[]`` (the
reference's tuple storage, passed without stacking copies), launches the C-ABI
entry point of ``libpolytaylor.so`` on the current HIP stream, and returns the
result as one coefficient-stacked tensor ``[K+1, ...]``. The ops are registered
for the CUDA (HIP) device only, with fake implementations for shape
propagation; on any other device the dispatcher raises. Outputs never alias
inputs.
"""

from typing import List, Optional, Tuple

import torch

from . import _lib

NAMESPACE = "polytensors_amd"


def _acc_dtype(dtype):
    return torch.float64 if dtype == torch.float64 else torch.float32


def _require(cond, message):
    if not cond:
        raise ValueError(message)


def _check_series(name, coeffs, dtype=None):
    _require(len(coeffs) >= 1, f"{name}: at least one coefficient is required")
    first = coeffs[0]
    dtype = first.dtype if dtype is None else dtype
    for c in coeffs:
        _require(c.dtype == dtype, f"{name}: coefficient dtypes differ ({c.dtype} vs {dtype})")
        _require(c.device == first.device, f"{name}: coefficients on different devices")
        _require(c.shape == first.shape, f"{name}: coefficient shapes differ")
        _require(c.is_contiguous(), f"{name}: coefficients must be contiguous")
    _require(dtype in _lib.DTYPE_CODES, f"{name}: unsupported dtype {dtype}")


# ---------------------------------------------------------------------------
# RMSNorm / LayerNorm series

@torch.library.custom_op(f"{NAMESPACE}::norm_series", mutates_args=(), device_types="cuda")
def norm_series(x: List[torch.Tensor], weight: List[torch.Tensor], bias: List[torch.Tensor],
                n: int, eps: float, layer: bool) -> torch.Tensor:
    """y = (Layer|RMS)Norm series over the last ``n`` elements of each coefficient."""
    _check_series("norm_series", x)
    degree = len(x) - 1
    numel = x[0].numel()
    _require(n >= 1 and numel % n == 0, "norm_series: n must divide the element count")
    for name, aff in (("weight", weight), ("bias", bias)):
        _require(len(aff) in (0, 1, degree + 1), f"norm_series: {name} needs 0, 1 or degree+1 coefficients")
        for c in aff:
            _require(c.dtype == x[0].dtype and c.device == x[0].device and c.numel() == n
                     and c.is_contiguous(), f"norm_series: {name} coefficients must be contiguous [n] of the input dtype")
    _require(layer or not bias, "norm_series: bias is a LayerNorm argument")
    out = torch.empty((degree + 1, *x[0].shape), dtype=x[0].dtype, device=x[0].device)
    lib = _lib.load()
    ys = list(out.unbind(0))
    args = (_lib.DTYPE_CODES[x[0].dtype], degree, _lib.ptr_array(x),
            _lib.ptr_array(weight) if weight else None, len(weight))
    if layer:
        status = lib.pt_layer_norm_series_fwd(*args, _lib.ptr_array(bias) if bias else None, len(bias),
                                              _lib.ptr_array(ys), numel // n, n, float(eps),
                                              _lib.stream_of(x[0].device))
    else:
        status = lib.pt_rms_norm_series_fwd(*args, _lib.ptr_array(ys), numel // n, n, float(eps),
                                            _lib.stream_of(x[0].device))
    _lib.check(status, "layer_norm_series" if layer else "rms_norm_series")
    return out


@norm_series.register_fake
def _(x, weight, bias, n, eps, layer):
    return x[0].new_empty((len(x), *x[0].shape))


# ---------------------------------------------------------------------------
# Cross-entropy series

@torch.library.custom_op(f"{NAMESPACE}::cross_entropy_series", mutates_args=(), device_types="cuda")
def cross_entropy_series(z: List[torch.Tensor], target: torch.Tensor, ignore_index: int,
                         reduction: int, softcap: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-order cross entropy of (N, C) logit series; returns (loss, lse).

    loss: [K+1, N] (reduction none) or [K+1] (mean/sum), and lse: [K+1, N], both in
    float32 (float64 for float64 logits). ``softcap`` > 0 caps the logit series as
    softcap * tanh(z / softcap) first; 0 for none. (No argument has a default: the
    autograd registration below expects every argument passed.)
    """
    _require(len(z) >= 1, "cross_entropy_series: at least one coefficient is required")
    first = z[0]
    _require(first.dim() == 2, "cross_entropy_series: logits must be (N, C)")
    _require(first.dtype in _lib.DTYPE_CODES, f"cross_entropy_series: unsupported dtype {first.dtype}")
    for c in z:
        _require(c.dtype == first.dtype and c.device == first.device and c.shape == first.shape,
                 "cross_entropy_series: coefficients must share dtype, device and shape")
        _require(c.stride() == first.stride() and c.stride(1) == 1,
                 "cross_entropy_series: coefficient rows must be contiguous with one common row stride")
    _require(target.dtype == torch.int64 and target.shape == first.shape[:1] and target.is_contiguous()
             and target.device == first.device, "cross_entropy_series: target must be contiguous int64 [N]")
    _require(reduction in (0, 1, 2), "cross_entropy_series: reduction must be 0, 1 or 2")
    _require(softcap >= 0.0 and softcap != float("inf"), "cross_entropy_series: softcap must be 0 or a positive cap")
    degree = len(z) - 1
    rows, classes = first.shape
    dtype = first.dtype
    lse = torch.empty((degree + 1, rows), dtype=_acc_dtype(dtype), device=first.device)
    loss = torch.empty((degree + 1, rows) if reduction == 0 else (degree + 1,), dtype=_acc_dtype(dtype),
                       device=first.device)
    lib = _lib.load()
    code = _lib.DTYPE_CODES[dtype]
    wbytes = lib.pt_cross_entropy_series_workspace_size(code, degree, rows, reduction)
    workspace = torch.empty((max(1, wbytes),), dtype=torch.uint8, device=first.device)
    status = lib.pt_cross_entropy_series_fwd(
        code, degree, _lib.ptr_array(z), rows, classes, first.stride(0) if rows else classes,
        target.data_ptr(), ignore_index, float(softcap), reduction, _lib.ptr_array(list(loss.unbind(0))),
        _lib.ptr_array(list(lse.unbind(0))), workspace.data_ptr(), _lib.stream_of(first.device))
    _lib.check(status, "cross_entropy_series")
    return loss, lse


@cross_entropy_series.register_fake
def _(z, target, ignore_index, reduction, softcap):
    rows = z[0].shape[0]
    loss = z[0].new_empty((len(z), rows) if reduction == 0 else (len(z),), dtype=_acc_dtype(z[0].dtype))
    lse = z[0].new_empty((len(z), rows), dtype=_acc_dtype(z[0].dtype))
    return loss, lse


# ---------------------------------------------------------------------------
# Cauchy-product matmul

@torch.library.custom_op(f"{NAMESPACE}::cauchy_matmul", mutates_args=(), device_types="cuda")
def cauchy_matmul(a: List[torch.Tensor], b: List[torch.Tensor], degree: int, trans_b: bool) -> torch.Tensor:
    """C_k = sum_{i+j=k} A_i @ B_j for [batch, m, k] x [batch, k, n] (or [batch, n, k] if trans_b).

    ``a`` and ``b`` hold 1 (plain operand) or degree+1 coefficients; a batch
    dimension of size 1 broadcasts. Returns [degree+1, batch, m, n].
    """
    for name, s in (("a", a), ("b", b)):
        _require(len(s) in (1, degree + 1), f"cauchy_matmul: {name} needs 1 or degree+1 coefficients")
        _check_series(f"cauchy_matmul {name}", s)
        _require(s[0].dim() == 3, f"cauchy_matmul: {name} must be 3-D [batch, rows, cols]")
    dtype = a[0].dtype
    _require(b[0].dtype == dtype and b[0].device == a[0].device, "cauchy_matmul: operand dtype/device differ")
    _require(dtype in _MATMUL_DTYPES, "cauchy_matmul: float32, float64, bfloat16 or float16")
    ba, m, kd = a[0].shape
    if trans_b:
        bb, n, kb = b[0].shape
    else:
        bb, kb, n = b[0].shape
    _require(kb == kd, "cauchy_matmul: inner dimensions differ")
    _require(ba == bb or ba == 1 or bb == 1, "cauchy_matmul: batch dimensions do not broadcast")
    batch = max(ba, bb)
    n_out = n
    if dtype in _HALF_DTYPES:
        # the 16-bit kernel moves 16-byte chunks: zero-pad the contraction (which leaves every
        # product unchanged) and, for B stored [k, n], the columns to multiples of 8, and give
        # it 16-byte aligned operands
        a = _aligned16([_pad_dim(c, -1, 8) for c in a])
        b = _aligned16([_pad_dim(c, -1 if trans_b else -2, 8) for c in b])
        if not trans_b:
            b = [_pad_dim(c, -1, 8) for c in b]
            n = b[0].shape[-1]
        kd = a[0].shape[-1]
    out = torch.empty((degree + 1, batch, m, n), dtype=dtype, device=a[0].device)
    lib = _lib.load()
    status = lib.pt_cauchy_matmul(
        _lib.DTYPE_CODES[dtype], degree, _lib.ptr_array(a), len(a), _lib.ptr_array(b), len(b),
        _lib.ptr_array(list(out.unbind(0))), batch, m, n, kd,
        0 if ba == 1 else m * kd, 0 if bb == 1 else n * kd, int(trans_b), _lib.stream_of(a[0].device))
    _lib.check(status, "cauchy_matmul")
    return out if n == n_out else out[..., :n_out].contiguous()


_HALF_DTYPES = (torch.bfloat16, torch.float16)
_MATMUL_DTYPES = (torch.float32, torch.float64) + _HALF_DTYPES


def _pad_dim(x, dim, multiple):
    """x zero-padded at the end of ``dim`` to a multiple of ``multiple`` (x itself if it is one)."""
    extra = -x.shape[dim] % multiple
    if extra == 0:
        return x
    pad = [0, 0] * (x.dim() - 1 - (dim % x.dim())) + [0, extra]
    return torch.nn.functional.pad(x, pad)


def _aligned16(coeffs):
    return [c if c.data_ptr() % 16 == 0 else c.clone() for c in coeffs]


@cauchy_matmul.register_fake
def _(a, b, degree, trans_b):
    ba, m, _ = a[0].shape
    bb = b[0].shape[0]
    n = b[0].shape[1] if trans_b else b[0].shape[2]
    return a[0].new_empty((degree + 1, max(ba, bb), m, n))


# ---------------------------------------------------------------------------
# Taylor flash attention forward

def _mask_ranges(mask, lq, lk):
    """Block ranges of a bool (L, S) mask on its device (skipped key/query blocks), or None."""
    if mask is None:
        return None
    lib = _lib.load()
    ranges = torch.empty(max(lib.pt_attention_mask_ranges_count(lq, lk), 1), dtype=torch.int32, device=mask.device)
    _lib.check(lib.pt_attention_mask_ranges(mask.data_ptr(), lq, lk, ranges.data_ptr(), _lib.stream_of(mask.device)),
               "attention_mask_ranges")
    return ranges


@torch.library.custom_op(f"{NAMESPACE}::taylor_attention_fwd", mutates_args=(), device_types="cuda")
def taylor_attention_fwd(q: List[torch.Tensor], k: List[torch.Tensor], v: List[torch.Tensor],
                         mask: Optional[torch.Tensor], causal: bool, scale: float,
                         degree: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Degree-K attention of [bh, L, d] query and [bh, S, d] key/value series.

    Each of q, k, v holds 1 (plain operand) or degree+1 coefficients. ``mask``
    is an optional (L, S) bool tensor (True = admissible). Returns
    (out [degree+1, bh, L, d], lse [degree+1, bh, L]).
    """
    for name, s in (("q", q), ("k", k), ("v", v)):
        _require(len(s) in (1, degree + 1), f"taylor_attention: {name} needs 1 or degree+1 coefficients")
        _check_series(f"taylor_attention {name}", s)
        _require(s[0].dim() == 3, f"taylor_attention: {name} must be [bh, length, d]")
    dtype = q[0].dtype
    _require(dtype in (torch.float32, torch.float64, torch.bfloat16, torch.float16),
             "taylor_attention: float32, float64, bfloat16 or float16")
    bh, lq, d = q[0].shape
    _require(k[0].shape == v[0].shape and k[0].shape[0] == bh and k[0].shape[2] == d,
             "taylor_attention: key/value shapes must be [bh, S, d] matching the query")
    _require(k[0].dtype == dtype and v[0].dtype == dtype, "taylor_attention: dtypes differ")
    lk = k[0].shape[1]
    if mask is not None:
        _require(mask.dtype == torch.bool and mask.shape == (lq, lk) and mask.device == q[0].device,
                 "taylor_attention: mask must be a bool (L, S) tensor on the query's device")
        _require(not causal, "taylor_attention: mask and causal are exclusive")
        mask = mask.contiguous()
    out = torch.empty((degree + 1, bh, lq, d), dtype=dtype, device=q[0].device)
    lse = torch.empty((degree + 1, bh, lq), dtype=_acc_dtype(dtype), device=q[0].device)
    ranges = _mask_ranges(mask, lq, lk)
    lib = _lib.load()
    status = lib.pt_taylor_attention_fwd(
        _lib.DTYPE_CODES[dtype], degree, _lib.ptr_array(q), len(q), _lib.ptr_array(k), len(k),
        _lib.ptr_array(v), len(v), _lib.ptr_array(list(out.unbind(0))), _lib.ptr_array(list(lse.unbind(0))),
        bh, lq, lk, d, int(causal), None if mask is None else mask.data_ptr(),
        None if ranges is None else ranges.data_ptr(), float(scale),
        _lib.stream_of(q[0].device))
    _lib.check(status, "taylor_attention_fwd")
    return out, lse


@taylor_attention_fwd.register_fake
def _(q, k, v, mask, causal, scale, degree):
    bh, lq, d = q[0].shape
    return (q[0].new_empty((degree + 1, bh, lq, d)),
            q[0].new_empty((degree + 1, bh, lq), dtype=_acc_dtype(q[0].dtype)))


def attention_gradient_series(q, k, v, out, lse, grad, mask, causal, scale):
    """Gradient series (dq, dk, dv) of the attention forward for every operand dtype.

    float32/float64 call ``taylor_attention_bwd``. bfloat16/float16 operands run
    the float32 backward kernels on float32 copies of q, k, v, the forward's
    output and the cotangents (the forward's lse series is already float32) and
    round the gradients to the operand dtype: the reference's half-type backward
    likewise accumulates in float32 (/root/reference/src/polytensors/_fused_attention.py:72-78,
    tolerance 5e-2 against float32, tests/test_fused_kernels.py:64-72).
    """
    dtype = q[0].dtype
    if dtype in (torch.bfloat16, torch.float16):
        def up(xs):
            return [x.float() for x in xs]

        dq, dk, dv = taylor_attention_bwd(up(q), up(k), up(v), out.float(), lse, up(grad), mask, causal, scale)
        return dq.to(dtype), dk.to(dtype), dv.to(dtype)
    return taylor_attention_bwd(q, k, v, out, lse, grad, mask, causal, scale)


@torch.library.custom_op(f"{NAMESPACE}::taylor_attention_bwd", mutates_args=(), device_types="cuda")
def taylor_attention_bwd(q: List[torch.Tensor], k: List[torch.Tensor], v: List[torch.Tensor], out: torch.Tensor,
                         lse: torch.Tensor, grad: List[torch.Tensor], mask: Optional[torch.Tensor], causal: bool,
                         scale: float, materialize: int = -1) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradient series (dq, dk, dv) of ``taylor_attention_fwd`` for the cotangent series ``grad``.

    q, k, v and grad hold degree+1 coefficients each ([bh, L, d] and [bh, S, d]);
    ``out`` [degree+1, bh, L, d] and ``lse`` [degree+1, bh, L] are the forward's
    outputs. Returns three [degree+1, ...] tensors in the operands' dtype.
    ``materialize``: 1 stores the P and dS tiles (5 series products per pair;
    float32 only), 0 recomputes them (8 products, no L x S workspace), -1
    chooses 1 for float32 when that workspace is at most a quarter of the
    device's memory.
    """
    degree = len(q) - 1
    for name, s in (("q", q), ("k", k), ("v", v), ("grad", grad)):
        _require(len(s) == degree + 1, f"taylor_attention_bwd: {name} needs degree+1 coefficients")
        _check_series(f"taylor_attention_bwd {name}", s)
        _require(s[0].dim() == 3, f"taylor_attention_bwd: {name} must be [bh, length, d]")
    dtype = q[0].dtype
    _require(dtype in (torch.float32, torch.float64), "taylor_attention_bwd: float32 or float64 only")
    bh, lq, d = q[0].shape
    _require(k[0].shape == v[0].shape and k[0].shape[0] == bh and k[0].shape[2] == d,
             "taylor_attention_bwd: key/value shapes must be [bh, S, d] matching the query")
    _require(grad[0].shape == q[0].shape, "taylor_attention_bwd: grad must have the query's shape")
    _require(all(s[0].dtype == dtype for s in (k, v, grad)), "taylor_attention_bwd: dtypes differ")
    _require(out.dtype == dtype and out.is_contiguous() and tuple(out.shape) == (degree + 1, bh, lq, d),
             "taylor_attention_bwd: out must be the forward's contiguous [K+1, bh, L, d] output")
    _require(lse.dtype == _acc_dtype(dtype) and lse.is_contiguous() and tuple(lse.shape) == (degree + 1, bh, lq),
             "taylor_attention_bwd: lse must be the forward's contiguous [K+1, bh, L] output")
    lk = k[0].shape[1]
    if mask is not None:
        _require(mask.dtype == torch.bool and mask.shape == (lq, lk) and mask.device == q[0].device,
                 "taylor_attention_bwd: mask must be a bool (L, S) tensor on the query's device")
        _require(not causal, "taylor_attention_bwd: mask and causal are exclusive")
        mask = mask.contiguous()
    device = q[0].device
    dq = torch.empty((degree + 1, bh, lq, d), dtype=dtype, device=device)
    dk = torch.empty((degree + 1, bh, lk, d), dtype=dtype, device=device)
    dv = torch.empty_like(dk)
    ranges = _mask_ranges(mask, lq, lk)
    lib = _lib.load()
    code = _lib.DTYPE_CODES[dtype]
    if materialize < 0:   # float32 only: the library refuses the stored-tile path for float64
        size = lib.pt_taylor_attention_bwd_workspace_size(code, degree, bh, lq, lk, 1)
        materialize = int(dtype == torch.float32 and
                          size <= torch.cuda.get_device_properties(device).total_memory // 4)
    workspace = torch.empty(max(lib.pt_taylor_attention_bwd_workspace_size(code, degree, bh, lq, lk,
                                                                           int(materialize)), 1),
                            dtype=torch.uint8, device=device)
    status = lib.pt_taylor_attention_bwd(
        code, degree, _lib.ptr_array(q), _lib.ptr_array(k), _lib.ptr_array(v),
        _lib.ptr_array(list(out.unbind(0))), _lib.ptr_array(list(lse.unbind(0))), _lib.ptr_array(grad),
        _lib.ptr_array(list(dq.unbind(0))), _lib.ptr_array(list(dk.unbind(0))), _lib.ptr_array(list(dv.unbind(0))),
        workspace.data_ptr(), int(materialize), bh, lq, lk, d, int(causal), None if mask is None else mask.data_ptr(),
        None if ranges is None else ranges.data_ptr(), float(scale),
        _lib.stream_of(device))
    _lib.check(status, "taylor_attention_bwd")
    return dq, dk, dv


@taylor_attention_bwd.register_fake
def _(q, k, v, out, lse, grad, mask, causal, scale, materialize=-1):
    return (q[0].new_empty((len(q), *q[0].shape)), k[0].new_empty((len(k), *k[0].shape)),
            k[0].new_empty((len(k), *k[0].shape)))


# ---------------------------------------------------------------------------
# Complex directions: real variants and their recombination

_REAL_OF = {torch.complex64: torch.float32, torch.complex128: torch.float64}


@torch.library.custom_op(f"{NAMESPACE}::complex_to_real", mutates_args=(), device_types="cuda")
def complex_to_real(src: List[torch.Tensor], alpha: List[float], beta: List[float]) -> torch.Tensor:
    """[len(alpha), len(src), *shape] real planes alpha[v] Re(src[o]) + beta[v] Im(src[o])."""
    _require(len(src) >= 1 and len(alpha) == len(beta) >= 1, "complex_to_real: planes and variants required")
    first = src[0]
    _require(first.dtype in _REAL_OF, "complex_to_real: complex64 or complex128 planes")
    for c in src:
        _require(c.dtype == first.dtype and c.shape == first.shape and c.device == first.device and c.is_contiguous(),
                 "complex_to_real: planes must share dtype, shape and device and be contiguous")
    real = _REAL_OF[first.dtype]
    out = torch.empty((len(alpha), len(src), *first.shape), dtype=real, device=first.device)
    lib = _lib.load()
    dst = [p for v in out.unbind(0) for p in v.unbind(0)]
    status = lib.pt_complex_to_real(_lib.DTYPE_CODES[real], len(src), _lib.ptr_array(src), len(alpha),
                                    _lib.double_array(alpha), _lib.double_array(beta), _lib.ptr_array(dst),
                                    first.numel(), _lib.stream_of(first.device))
    _lib.check(status, "complex_to_real")
    return out


@complex_to_real.register_fake
def _(src, alpha, beta):
    return src[0].new_empty((len(alpha), len(src), *src[0].shape), dtype=_REAL_OF[src[0].dtype])


@torch.library.custom_op(f"{NAMESPACE}::real_to_complex", mutates_args=(), device_types="cuda")
def real_to_complex(src: List[torch.Tensor], orders: int, wre: List[float], wim: List[float]) -> torch.Tensor:
    """[orders, *shape] complex planes sum_v (wre[v] + i wim[v]) src[v * orders + o]."""
    variants = len(wre)
    _require(variants >= 1 and len(wim) == variants and len(src) == variants * orders and orders >= 1,
             "real_to_complex: src must hold variants x orders planes")
    first = src[0]
    _require(first.dtype in (torch.float32, torch.float64), "real_to_complex: float32 or float64 planes")
    for c in src:
        _require(c.dtype == first.dtype and c.shape == first.shape and c.device == first.device and c.is_contiguous(),
                 "real_to_complex: planes must share dtype, shape and device and be contiguous")
    cplx = torch.complex64 if first.dtype == torch.float32 else torch.complex128
    out = torch.empty((orders, *first.shape), dtype=cplx, device=first.device)
    lib = _lib.load()
    status = lib.pt_real_to_complex(_lib.DTYPE_CODES[first.dtype], orders, variants, _lib.ptr_array(src),
                                    _lib.double_array(wre), _lib.double_array(wim),
                                    _lib.ptr_array(list(out.unbind(0))), first.numel(), _lib.stream_of(first.device))
    _lib.check(status, "real_to_complex")
    return out


@real_to_complex.register_fake
def _(src, orders, wre, wim):
    cplx = torch.complex64 if src[0].dtype == torch.float32 else torch.complex128
    return src[0].new_empty((orders, *src[0].shape), dtype=cplx)


# ---------------------------------------------------------------------------
# Elementwise activation series

@torch.library.custom_op(f"{NAMESPACE}::activation_series", mutates_args=(), device_types="cuda")
def activation_series(x: List[torch.Tensor], kind: str) -> torch.Tensor:
    """f(x(t)) for f in _lib.ACTIVATIONS; returns [K+1, *x.shape]."""
    _check_series("activation_series", x)
    _require(kind in _lib.ACTIVATIONS, f"activation_series: unknown kind {kind!r}")
    degree = len(x) - 1
    out = torch.empty((degree + 1, *x[0].shape), dtype=x[0].dtype, device=x[0].device)
    lib = _lib.load()
    status = lib.pt_activation_series_fwd(_lib.DTYPE_CODES[x[0].dtype], degree, _lib.ACTIVATIONS[kind],
                                          _lib.ptr_array(x), _lib.ptr_array(list(out.unbind(0))),
                                          x[0].numel(), _lib.stream_of(x[0].device))
    _lib.check(status, f"activation_series({kind})")
    return out


@activation_series.register_fake
def _(x, kind):
    return x[0].new_empty((len(x), *x[0].shape))


@torch.library.custom_op(f"{NAMESPACE}::activation_series_backward", mutates_args=(), device_types="cuda")
def activation_series_backward(grad: List[torch.Tensor], saved: List[torch.Tensor], kind: str) -> torch.Tensor:
    """grad(t) * f'(x(t)); ``saved`` is the forward input (gelu, gelu_tanh, silu) or output (tanh, sigmoid)."""
    _check_series("activation_series_backward grad", grad)
    _check_series("activation_series_backward saved", saved)
    _require(len(grad) == len(saved) and grad[0].shape == saved[0].shape and grad[0].dtype == saved[0].dtype
             and grad[0].device == saved[0].device,
             "activation_series_backward: grad and saved series must match in degree, shape, dtype and device")
    _require(kind in ("gelu", "gelu_tanh", "tanh", "sigmoid", "silu"),
             f"activation_series_backward: no backward for kind {kind!r}")
    degree = len(grad) - 1
    out = torch.empty((degree + 1, *grad[0].shape), dtype=grad[0].dtype, device=grad[0].device)
    lib = _lib.load()
    status = lib.pt_activation_series_bwd(_lib.DTYPE_CODES[grad[0].dtype], degree, _lib.ACTIVATIONS[kind],
                                          _lib.ptr_array(grad), _lib.ptr_array(saved),
                                          _lib.ptr_array(list(out.unbind(0))), grad[0].numel(),
                                          _lib.stream_of(grad[0].device))
    _lib.check(status, f"activation_series_backward({kind})")
    return out


@activation_series_backward.register_fake
def _(grad, saved, kind):
    return grad[0].new_empty((len(grad), *grad[0].shape))


# ---------------------------------------------------------------------------
# Elementwise series product / quotient

@torch.library.custom_op(f"{NAMESPACE}::series_binary", mutates_args=(), device_types="cuda")
def series_binary(a: List[torch.Tensor], b: List[torch.Tensor], op: str) -> torch.Tensor:
    """a (*) b or a / b of two series of one shape; returns [K+1, *shape]."""
    _check_series("series_binary a", a)
    _check_series("series_binary b", b)
    _require(len(a) == len(b) and a[0].shape == b[0].shape and a[0].dtype == b[0].dtype
             and a[0].device == b[0].device, "series_binary: operands must match in degree, shape, dtype and device")
    _require(op in _lib.BINARY_OPS, f"series_binary: unknown operation {op!r}")
    degree = len(a) - 1
    out = torch.empty((degree + 1, *a[0].shape), dtype=a[0].dtype, device=a[0].device)
    lib = _lib.load()
    status = lib.pt_series_binary(_lib.DTYPE_CODES[a[0].dtype], degree, _lib.BINARY_OPS[op], _lib.ptr_array(a),
                                  _lib.ptr_array(b), _lib.ptr_array(list(out.unbind(0))), a[0].numel(),
                                  _lib.stream_of(a[0].device))
    _lib.check(status, f"series_binary({op})")
    return out


@series_binary.register_fake
def _(a, b, op):
    return a[0].new_empty((len(a), *a[0].shape))


@torch.library.custom_op(f"{NAMESPACE}::norm_series_backward", mutates_args=(), device_types="cuda")
def norm_series_backward(x: List[torch.Tensor], grad: List[torch.Tensor], n: int, eps: float,
                         layer: bool) -> torch.Tensor:
    """Gradient series of the (Layer|RMS)Norm normalization over the last ``n`` elements."""
    _check_series("norm_series_backward x", x)
    _check_series("norm_series_backward grad", grad)
    _require(len(x) == len(grad) and x[0].shape == grad[0].shape and x[0].dtype == grad[0].dtype
             and x[0].device == grad[0].device, "norm_series_backward: x and grad series must match")
    degree = len(x) - 1
    numel = x[0].numel()
    _require(n >= 1 and numel % n == 0, "norm_series_backward: n must divide the element count")
    out = torch.empty((degree + 1, *x[0].shape), dtype=x[0].dtype, device=x[0].device)
    lib = _lib.load()
    entry = lib.pt_layer_norm_series_bwd if layer else lib.pt_rms_norm_series_bwd
    status = entry(_lib.DTYPE_CODES[x[0].dtype], degree, _lib.ptr_array(x), _lib.ptr_array(grad),
                   _lib.ptr_array(list(out.unbind(0))), numel // n, n, float(eps), _lib.stream_of(x[0].device))
    _lib.check(status, "layer_norm_series_bwd" if layer else "rms_norm_series_bwd")
    return out


@norm_series_backward.register_fake
def _(x, grad, n, eps, layer):
    return x[0].new_empty((len(x), *x[0].shape))


@torch.library.custom_op(f"{NAMESPACE}::cross_entropy_series_backward", mutates_args=(), device_types="cuda")
def cross_entropy_series_backward(z: List[torch.Tensor], target: torch.Tensor, ignore_index: int, softcap: float,
                                  lse: torch.Tensor, cot: List[torch.Tensor]) -> torch.Tensor:
    """Gradient series of the per-row losses w.r.t. (N, C) logits; ``lse`` [K+1, N] from the
    forward, ``cot`` the K+1 per-row cotangents. Returns [K+1, N, C] in the logits' dtype."""
    _require(len(z) >= 1 and len(cot) == len(z) and lse.shape[0] == len(z),
             "cross_entropy_series_backward: z, lse and cot need the same number of orders")
    first = z[0]
    for c in z:
        _require(c.dtype == first.dtype and c.device == first.device and c.shape == first.shape
                 and c.stride() == first.stride() and c.stride(1) == 1,
                 "cross_entropy_series_backward: logit rows must be unit-stride with one common row stride")
    rows, classes = first.shape
    acc = _acc_dtype(first.dtype)
    _require(lse.dtype == acc and lse.is_contiguous() and tuple(lse.shape[1:]) == (rows,),
             "cross_entropy_series_backward: lse must be contiguous [K+1, N] of the arithmetic type")
    for c in cot:
        _require(c.dtype == acc and c.is_contiguous() and tuple(c.shape) == (rows,),
                 "cross_entropy_series_backward: cotangents must be contiguous [N] of the arithmetic type")
    _require(target.dtype == torch.int64 and target.is_contiguous() and tuple(target.shape) == (rows,),
             "cross_entropy_series_backward: target must be contiguous int64 [N]")
    degree = len(z) - 1
    out = torch.empty((degree + 1, rows, classes), dtype=first.dtype, device=first.device)
    lib = _lib.load()
    status = lib.pt_cross_entropy_series_bwd(
        _lib.DTYPE_CODES[first.dtype], degree, _lib.ptr_array(z), rows, classes,
        first.stride(0) if rows else classes, target.data_ptr(), ignore_index, float(softcap),
        _lib.ptr_array(list(lse.unbind(0))), _lib.ptr_array(cot), _lib.ptr_array(list(out.unbind(0))),
        _lib.stream_of(first.device))
    _lib.check(status, "cross_entropy_series_bwd")
    return out


@cross_entropy_series_backward.register_fake
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
# order (an ordinary tensor) gets coefficient K. These backward functions are
# not themselves differentiable (as the reference's once_differentiable fused
# Functions, /root/reference/src/polytensors/_fused_attention.py:166-185).

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
    """``grads`` padded with None to the number of arguments the call passed (torch matches the
    backward's return to the arguments given, defaulted ones excluded)."""
    return tuple(grads) + (None,) * (ctx.n_inputs - len(grads))


def _once(what):
    if torch.is_grad_enabled():
        raise NotImplementedError(f"{what}: second-order coefficient autograd through the fused kernels "
                                  "is not implemented")


def _norm_setup(ctx, inputs, output):
    x, weight, bias, n, eps, layer = inputs
    ctx.save_for_backward(*x)
    ctx.meta = (n, eps, layer, bool(weight) or bool(bias))
    ctx.n_inputs = len(inputs)


def _norm_backward(ctx, grad):
    _once("norm_series")
    n, eps, layer, affine = ctx.meta
    if affine:
        raise NotImplementedError("norm_series: the fused weight/bias has no coefficient gradient; under "
                                  "autograd apply them as separate series operations")
    x = list(ctx.saved_tensors)
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
    _once("cross_entropy_series")
    n, ignore_index, reduction, softcap = ctx.meta
    saved = ctx.saved_tensors
    z, target, lse = list(saved[:n]), saved[n], saved[n + 1]
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
    _once("cauchy_matmul")
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
    q, k, v, mask, causal, scale, degree = inputs
    out, lse = output
    ctx.mark_non_differentiable(lse)
    ctx.save_for_backward(*q, *k, *v, out, lse, *([] if mask is None else [mask]))
    ctx.meta = (len(q), len(k), len(v), mask is not None, causal, scale, degree)
    ctx.n_inputs = len(inputs)


def _attn_backward(ctx, grad_out, grad_lse):
    _once("taylor_attention_fwd")
    nq, nk, nv, has_mask, causal, scale, degree = ctx.meta
    s = ctx.saved_tensors
    q, k, v = list(s[:nq]), list(s[nq:nq + nk]), list(s[nq + nk:nq + nk + nv])
    out, lse = s[nq + nk + nv], s[nq + nk + nv + 1]
    mask = s[-1] if has_mask else None

    def full(xs):   # the backward kernels take every order; an ordinary operand has zero higher orders
        return xs + [torch.zeros_like(xs[0]) for _ in range(degree + 1 - len(xs))]

    dq, dk, dv = attention_gradient_series(full(q), full(k), full(v), out, lse, _reversed(grad_out), mask, causal,
                                           scale)
    return _returned(ctx, _read_back(dq, nq), _read_back(dk, nk), _read_back(dv, nv))


torch.library.register_autograd(f"{NAMESPACE}::taylor_attention_fwd", _attn_backward, setup_context=_attn_setup)

# the derivative's saved series: the input, or the output where the backward operation takes it
_ACT_SAVES_OUTPUT = ("tanh", "sigmoid", "exp")


def _act_setup(ctx, inputs, output):
    x, kind = inputs
    ctx.kind = kind
    ctx.n_inputs = len(inputs)
    if kind in _ACT_SAVES_OUTPUT:
        ctx.save_for_backward(output)
    else:
        ctx.save_for_backward(*x)


def _act_backward(ctx, grad):
    _once("activation_series")
    kind = ctx.kind
    saved = ctx.saved_tensors
    saved = list(saved[0].unbind(0)) if kind in _ACT_SAVES_OUTPUT else list(saved)
    g = _reversed(grad)
    if kind == "exp":      # exp' = exp: the gradient series is G (*) y
        dx = series_binary(g, saved, "mul")
    elif kind == "log":    # log' = 1/x: G / x
        dx = series_binary(g, saved, "div")
    else:
        dx = activation_series_backward(g, saved, kind)
    return _returned(ctx, _read_back(dx, len(saved)))


torch.library.register_autograd(f"{NAMESPACE}::activation_series", _act_backward, setup_context=_act_setup)


def _binary_setup(ctx, inputs, output):
    a, b, op = inputs
    ctx.op = op
    ctx.n = len(a)
    ctx.n_inputs = len(inputs)
    ctx.save_for_backward(*a, *b, *(list(output.unbind(0)) if op == "div" else []))


def _binary_backward(ctx, grad):
    _once("series_binary")
    n, op = ctx.n, ctx.op
    s = ctx.saved_tensors
    a, b = list(s[:n]), list(s[n:2 * n])
    g = _reversed(grad)
    if op == "mul":        # d(a b) = b da + a db
        da, db = series_binary(g, b, "mul"), series_binary(g, a, "mul")
    else:                  # d(a / b) = da / b - (a / b) db / b
        y = list(s[2 * n:])
        da = series_binary(g, b, "div")
        db = -series_binary(list(series_binary(g, y, "mul").unbind(0)), b, "div")
    return _returned(ctx, _read_back(da, n), _read_back(db, n))


torch.library.register_autograd(f"{NAMESPACE}::series_binary", _binary_backward, setup_context=_binary_setup)
