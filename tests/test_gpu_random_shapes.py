"""Seeded random cases of every fused operation through the PolyTensor API (GPU) vs the CPU oracle.

The other GPU tests pin chosen shapes and edge cases; here one seeded generator
draws degrees, dtypes, sizes (ragged, not multiples of the kernels' tiles) and
options per case, so that combinations nobody listed get exercised too:
attention (causal / boolean / additive / per-batch masks, cross lengths,
plain operands) with its gradient series (the 16-bit backward kernels for bfloat16),
Cauchy matmul with broadcast batches
and plain operands, RMSNorm / LayerNorm with series weights, cross entropy with
ignored rows, weights and label smoothing, and the elementwise activations.
The oracle runs in float64 on the same (rounded) inputs. Per-order tolerance
is the contract's: max|got - want| / max|want| <= 1e-10 float64, 1e-4 float32,
2e-2 bfloat16, each order normalised by its own largest value. An order whose
exact value is zero everywhere must come out zero to within that tolerance in
absolute terms. The one floor is where an order's exact value is zero
analytically but its computed value is rounding noise (attention's key gradient
with a single key; see the case).
"""

import random

import pytest
import torch
import torch.nn.functional as F

import oracle
from polytensors_amd import PolyTensor

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2}
CASES = 40
MODES = ("causal", "bool", "additive", "batched", "none")


def _series(shape, degree, g, scale=1.0):
    return [torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k for k in range(degree + 1)]


def _rounded(S, dtype):
    return [c.to(dtype).double() for c in S]


def _poly(S, dtype, grad=False):
    return PolyTensor(tuple(c.to(dtype).cuda() for c in S), requires_grad=grad)


def _check(got, want, dtype, what, rows=None, floor=0.0):
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.detach().cpu().double(), b.double()
        if rows is not None:
            a, b = a[rows], b[rows]
        if not b.numel():
            continue
        scale = max(b.abs().max().item(), floor)
        diff = (a - b).abs().max().item()
        err = diff / scale if scale > 0 else diff
        assert err <= TOL[dtype], f"{what}: order {k} error {err:.3e} (scale {scale:.3e})"


@pytest.mark.parametrize("case", range(CASES))
def test_attention(case):
    rnd = random.Random(1000 + case)
    g = torch.Generator().manual_seed(1000 + case)
    dtype = rnd.choice([torch.float64, torch.float32, torch.bfloat16])
    degree = rnd.randint(0, 5)
    d = rnd.choice([16, 32, 64, 128])
    B, H = rnd.randint(1, 2), rnd.randint(1, 3)
    L, S = rnd.randint(1, 140), rnd.randint(1, 140)
    mode = MODES[case % len(MODES)]
    grad = rnd.random() < 0.6
    Q, K, V = (_series((B, H, T, d), degree, g) for T in (L, S, S))
    mask, causal = None, False
    if mode == "causal":
        causal = True
    elif mode in ("bool", "additive", "batched"):
        shape = (B, 1, L, S) if mode == "batched" else (L, S)
        keep = torch.rand(shape, generator=g) < 0.75
        mask = keep if mode != "additive" else \
            torch.randn(shape, generator=g, dtype=torch.float64).masked_fill(~keep, float("-inf")).to(dtype)
    q, k, v = (_poly(X, dtype, grad) for X in (Q, K, V))
    with PolyTensor.plain_range():
        ctx = torch.enable_grad() if grad else torch.no_grad()
        with ctx:
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=None if mask is None else mask.cuda(),
                                                 is_causal=causal)
            if grad:
                Gs = _series((B, H, L, d), degree, g)
                out.backward(_poly(Gs, dtype))
    up = [_rounded(X, dtype) for X in (Q, K, V)]
    m = mask if mask is None or mask.dtype == torch.bool else mask.double()
    want = oracle.attention(*up, attn_mask=m, is_causal=causal)
    keep = torch.ones(L, S, dtype=torch.bool).tril() if causal else torch.ones(L, S, dtype=torch.bool)
    if m is not None:
        keep = keep & (m if m.dtype == torch.bool else ~torch.isneginf(m))
    rows = keep.any(-1).expand(B, H, L)   # rows with an admissible key (the others are zero here, NaN there)
    what = f"attention {dtype} K={degree} d={d} B={B} H={H} L={L} S={S} {mode}"
    _check(out.coeffs, want, dtype, what, rows=rows)
    for c in out.coeffs:
        assert c.detach()[~rows.cuda()].abs().max().item() == 0 if (~rows).any() else True, f"{what}: empty rows"
    if grad:
        grads = oracle.attention_backward(*up, _rounded(Gs, dtype), attn_mask=m, is_causal=causal)
        for name, x, b in zip(("dq", "dk", "dv"), (q, k, v), grads):
            # With one key the softmax is identically 1, so dS = 0 and dq, dk are exactly zero;
            # the kernels' values there are rounding noise of G.V - Delta, measured against the
            # scale of the cotangent (1) rather than against zero.
            _check(x.grad.coeffs, b, dtype, f"{what} {name}", floor=1.0 if S == 1 and name != "dv" else 0.0)


@pytest.mark.parametrize("case", range(CASES))
def test_matmul(case):
    rnd = random.Random(2000 + case)
    g = torch.Generator().manual_seed(2000 + case)
    dtype = rnd.choice([torch.float64, torch.float32, torch.bfloat16])
    degree = rnd.randint(0, 6)
    m, kd, n = rnd.randint(1, 150), 8 * rnd.randint(1, 20), rnd.randint(1, 150)
    batch_a, batch_b = rnd.choice([((), ()), ((3,), ()), ((2, 1), (3,)), ((1,), (2,))])
    A = _series(batch_a + (m, kd), degree, g)
    plain_b = rnd.random() < 0.4
    Bm = [torch.randn(batch_b + (kd, n), generator=g, dtype=torch.float64)] if plain_b else _series(batch_b + (kd, n),
                                                                                                     degree, g)
    a = _poly(A, dtype)
    b = Bm[0].to(dtype).cuda() if plain_b else _poly(Bm, dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        out = a @ b
    want = oracle.matmul(_rounded(A, dtype), _rounded(Bm, dtype))
    _check(out.coeffs, want, dtype, f"matmul {dtype} K={degree} {batch_a}{(m, kd)} @ {batch_b}{(kd, n)}")


@pytest.mark.parametrize("case", range(CASES))
def test_norms(case):
    rnd = random.Random(3000 + case)
    g = torch.Generator().manual_seed(3000 + case)
    dtype = rnd.choice([torch.float64, torch.float32, torch.bfloat16])
    degree = rnd.randint(0, 8)
    rows, n = rnd.randint(1, 70), rnd.randint(1, 3000)
    layer = rnd.random() < 0.5
    X = _series((rows, n), degree, g)
    W = _series((n,), degree, g) if rnd.random() < 0.5 else None
    Bias = _series((n,), degree, g) if layer and rnd.random() < 0.5 else None
    with torch.no_grad(), PolyTensor.plain_range():
        x = _poly(X, dtype)
        w = None if W is None else _poly(W, dtype)
        if layer:
            out = F.layer_norm(x, (n,), w, None if Bias is None else _poly(Bias, dtype), eps=1e-5)
        else:
            out = F.rms_norm(x, (n,), w, eps=1e-6)
    Xr = _rounded(X, dtype)
    Wr = None if W is None else _rounded(W, dtype)
    if layer:
        want = oracle.layer_norm(Xr, (n,), Wr, None if Bias is None else _rounded(Bias, dtype), eps=1e-5)
    else:
        want = oracle.rms_norm(Xr, (n,), Wr, eps=1e-6)
    _check(out.coeffs, want, dtype, f"{'layer' if layer else 'rms'}_norm {dtype} K={degree} [{rows}, {n}]")


@pytest.mark.parametrize("case", range(CASES))
def test_cross_entropy(case):
    rnd = random.Random(4000 + case)
    g = torch.Generator().manual_seed(4000 + case)
    dtype = rnd.choice([torch.float64, torch.float32, torch.bfloat16])
    degree = rnd.randint(0, 8)
    rows, classes = rnd.randint(1, 90), rnd.randint(2, 5000)
    reduction = rnd.choice(["none", "mean", "sum"])
    Z = _series((rows, classes), degree, g, scale=2.0)
    y = torch.randint(0, classes, (rows,), generator=g)
    y[torch.rand(rows, generator=g) < 0.15] = -100
    if (y == -100).all():
        y[0] = 0
    weight = (torch.rand(classes, generator=g, dtype=torch.float64) + 0.5) if rnd.random() < 0.3 else None
    smoothing = rnd.choice([0.0, 0.0, 0.1])
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(_poly(Z, dtype), y.cuda(), weight=None if weight is None else weight.to(dtype).cuda(),
                               reduction=reduction, label_smoothing=smoothing)
    want = oracle.cross_entropy(_rounded(Z, dtype), y, reduction=reduction,
                                weight=None if weight is None else weight.to(dtype).double(), label_smoothing=smoothing)
    _check(loss.coeffs, want, dtype, f"cross_entropy {dtype} K={degree} [{rows}, {classes}] {reduction} "
           f"w={weight is not None} eps={smoothing}")


@pytest.mark.parametrize("case", range(CASES))
def test_activations(case):
    rnd = random.Random(5000 + case)
    g = torch.Generator().manual_seed(5000 + case)
    dtype = rnd.choice([torch.float64, torch.float32, torch.bfloat16])
    degree = rnd.randint(0, 8)
    kind = rnd.choice(["gelu", "gelu_tanh", "tanh", "sigmoid", "silu", "exp"])
    X = _series((rnd.randint(1, 300), rnd.randint(1, 300)), degree, g, scale=0.7)
    fn = {"gelu": F.gelu, "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"), "tanh": torch.tanh,
          "sigmoid": torch.sigmoid, "silu": F.silu, "exp": torch.exp}[kind]
    with torch.no_grad(), PolyTensor.plain_range():
        out = fn(_poly(X, dtype))
    want = oracle.activation(_rounded(X, dtype), kind)
    _check(out.coeffs, want, dtype, f"{kind} {dtype} K={degree}")
