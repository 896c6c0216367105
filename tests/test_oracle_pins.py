"""Pins of the CPU oracle (CPU only).

The oracle restates the reference's plain-range series rules; these tests check
it against what fixes the answer independently of those rules:
  * nested forward-mode derivatives of the plain composite function along the
    curve (tests/jets.py), the reference's own oracle pattern;
  * closed forms along a line and round trips (/root/reference/tests/test_series.py:18-46,83-98,113-120);
  * known-answer values from the reference's tests
    (/root/reference/tests/test_tensor.py:70-76, /root/reference/tests/test_dispatch.py:63-70);
  * the reference's finite-difference checks on its fixed data
    (/root/reference/tests/test_primitives.py:115-146,245-273).
The last group plants plausible mistakes in copies of oracle functions and
checks that these pins catch them.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import paths, series
from tests.jets import rel_err, taylor

torch.set_default_dtype(torch.float32)


def _series(shape, degree, seed, scale=1.0, decay=0.5, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=dtype) * scale * (decay ** k) for k in range(degree + 1)]


# --- known answers -----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64,
                                   torch.complex64, torch.complex128])
def test_square_plus_one_known_answer(dtype):
    # /root/reference/tests/test_tensor.py:70-76: (x*x + 1) for x = 2 + t is (5, 4, 1, 0).
    X = paths.lift([torch.tensor(2.0, dtype=dtype), torch.tensor(1.0, dtype=dtype)], 3)
    out = paths._add_to_order0(series.cauchy(X, X), 1)
    assert [c.item() for c in out] == [5, 4, 1, 0]


def test_complex_matrix_known_answer():
    # /root/reference/tests/test_dispatch.py:63-70
    eye = torch.eye(2, dtype=torch.float64)
    A = paths.lift([eye, torch.full((2, 2), 1j, dtype=torch.complex128)], 2)
    B = paths.lift([eye * 2, torch.full((2, 2), 2j, dtype=torch.complex128)], 2)
    C = oracle.matmul(A, B)
    torch.testing.assert_close(C[0], 2 * eye)   # real base stays real
    torch.testing.assert_close(C[1], torch.full((2, 2), 4j, dtype=torch.complex128))
    torch.testing.assert_close(C[2], torch.full((2, 2), -4 + 0j, dtype=torch.complex128))


# --- closed forms ------------------------------------------------------------------------------

@pytest.mark.parametrize("degree", (1, 3, 12))
@pytest.mark.parametrize("complex_direction", (False, True))
@pytest.mark.parametrize("operation", ("exp", "log", "rsqrt"))
def test_line_closed_forms(operation, complex_direction, degree):
    # /root/reference/tests/test_series.py:18-46
    base = torch.tensor(1.7, dtype=torch.float64)
    direction = torch.tensor(0.2 + 0.3j if complex_direction else 0.2,
                             dtype=torch.complex128 if complex_direction else torch.float64)
    X = [base, direction] + [torch.zeros_like(direction) for _ in range(degree - 1)]
    result = {"exp": series.exp_series, "log": series.log_series, "rsqrt": series.rsqrt_series}[operation](X)
    binomial = 1.0
    for order in range(1, degree + 1):
        if operation == "exp":
            expected = torch.exp(base) * direction ** order / math.factorial(order)
        elif operation == "log":
            expected = ((-1) ** (order - 1) / order) * (direction / base) ** order
        else:
            binomial *= (-0.5 - (order - 1)) / order
            expected = binomial * torch.rsqrt(base) * (direction / base) ** order
        torch.testing.assert_close(result[order], expected, rtol=2e-13, atol=1e-28)


def test_round_trips():
    # /root/reference/tests/test_series.py:83-98
    X = [torch.tensor(v, dtype=torch.float64) for v in (1.5, 0.2, -0.1, 0.03, 0.0, -0.002)]
    back = series.exp_series(series.log_series(X))
    for a, b in zip(back, X):
        torch.testing.assert_close(a, b, rtol=2e-13, atol=1e-15)
    r = series.rsqrt_series(X)
    identity = series.cauchy(series.cauchy(r, r), X)
    for k, c in enumerate(identity):
        torch.testing.assert_close(c, torch.tensor(1.0 if k == 0 else 0.0, dtype=torch.float64),
                                   rtol=2e-13, atol=1e-15)


@pytest.mark.parametrize("dtype", (torch.float32, torch.float64))
def test_logsumexp_large_common_offset(dtype):
    # /root/reference/tests/test_series.py:113-120: a line along ones adds t exactly.
    base = torch.full((2,), 1e20, dtype=dtype)
    X = [base, torch.ones_like(base)] + [torch.zeros_like(base) for _ in range(4)]
    lse = paths.logsumexp(X, 0)
    assert torch.equal(lse[0], torch.logsumexp(base, 0))
    assert lse[1].item() == 1.0
    for c in lse[2:]:
        assert c.item() == 0.0


# --- the reference's finite-difference checks on its fixed data ---------------------------------

_FD_LOGITS = [[0.2, -1.3, 2.1], [3.0, -4.0, 0.1]]
_FD_DIRECTION = [[0.7, -0.2, 0.4], [-0.8, 0.5, 0.3]]


def _fd(function, x0, direction, step=2e-3):
    # five-point differences, /root/reference/tests/test_primitives.py:17-29
    f0 = function(x0)
    plus, minus = function(x0 + step * direction), function(x0 - step * direction)
    plus2, minus2 = function(x0 + 2 * step * direction), function(x0 - 2 * step * direction)
    return (f0, (plus - minus) / (2 * step), (plus - 2 * f0 + minus) / (2 * step ** 2),
            (plus2 - 2 * plus + 2 * minus - minus2) / (12 * step ** 3))


def test_cross_entropy_degree3_finite_differences():
    # /root/reference/tests/test_primitives.py:115-146 (targets [2, 0], reduction sum)
    x0 = torch.tensor(_FD_LOGITS, dtype=torch.float64)
    d = torch.tensor(_FD_DIRECTION, dtype=torch.float64)
    y = torch.tensor([2, 0])
    got = oracle.cross_entropy(paths.lift([x0, d], 3), y, reduction="sum")
    want = _fd(lambda v: F.cross_entropy(v, y, reduction="sum"), x0, d)
    assert torch.equal(got[0], want[0])
    for k in range(1, 4):
        torch.testing.assert_close(got[k], want[k], atol=5e-8, rtol=0.0)


@pytest.mark.parametrize("which", ("softmax", "log_softmax", "logsumexp"))
def test_softmax_family_degree3_finite_differences(which):
    # /root/reference/tests/test_primitives.py:245-273
    x0 = torch.tensor(_FD_LOGITS, dtype=torch.float64)
    d = torch.tensor(_FD_DIRECTION, dtype=torch.float64)
    sm, lsm, lse = series.softmax_family(paths.lift([x0, d], 3), -1)
    got = {"softmax": sm, "log_softmax": lsm, "logsumexp": [c.squeeze(-1) for c in lse]}[which]
    fn = {"softmax": lambda v: torch.softmax(v, -1), "log_softmax": lambda v: torch.log_softmax(v, -1),
          "logsumexp": lambda v: torch.logsumexp(v, -1)}[which]
    want = _fd(fn, x0, d)
    assert torch.equal(got[0], want[0])
    for k in range(1, 4):
        torch.testing.assert_close(got[k], want[k], atol=5e-8, rtol=0.0)


# --- independent jets of the composite functions -------------------------------------------------

def _check(got, want, tol):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        assert rel_err(a, b) <= tol, (k, rel_err(a, b))


def test_rms_norm_line_matches_higher_derivatives():
    # /root/reference/tests/test_plain_range.py:103-115 (shape (4,), eps 1e-5, degree 4)
    g = torch.Generator().manual_seed(7)
    base, direction = torch.randn(4, generator=g, dtype=torch.float64), torch.randn(4, generator=g, dtype=torch.float64)
    got = oracle.rms_norm(paths.lift([base, direction], 4), (4,), eps=1e-5)
    want = taylor(lambda x: F.rms_norm(x, (4,), eps=1e-5), [[base, direction]], 4)
    _check(got, want, 1e-12)


@pytest.mark.parametrize("weight_kind", ("none", "plain", "series"))
def test_rms_norm_general_series(weight_kind):
    X = _series((3, 5, 16), 4, seed=11)
    W = {"none": None, "plain": [1 + 0.1 * torch.randn(16, dtype=torch.float64)],
         "series": _series((16,), 4, seed=12)}[weight_kind]
    got = oracle.rms_norm(X, (16,), weight=W, eps=1e-3)
    if W is None:
        want = taylor(lambda x: F.rms_norm(x, (16,), eps=1e-3), [X], 4)
    else:
        want = taylor(lambda x, w: F.rms_norm(x, (16,), eps=1e-3) * w, [X, W], 4)
    _check(got, want, 1e-12)


def test_rms_norm_default_eps_is_dtype_eps():
    X = _series((2, 8), 2, seed=13, dtype=torch.float32)
    explicit = oracle.rms_norm(X, (8,), eps=torch.finfo(torch.float32).eps)
    default = oracle.rms_norm(X, (8,))
    for a, b in zip(explicit, default):
        assert torch.equal(a, b)


@pytest.mark.parametrize("affine", (False, True))
def test_layer_norm_general_series(affine):
    X = _series((4, 24), 4, seed=21, scale=2.0)
    W = _series((24,), 4, seed=22) if affine else None
    B = _series((24,), 4, seed=23) if affine else None
    got = oracle.layer_norm(X, (24,), W, B, eps=1e-4)

    # The explicit composite: torch's native layer_norm gives wrong orders >= 2 under nested
    # forward-mode AD (its forward derivative does not track the derivative of its saved rstd).
    def composite(x):
        c = x - x.mean(-1, keepdim=True)
        return c * torch.rsqrt((c * c).mean(-1, keepdim=True) + 1e-4)

    if affine:
        want = taylor(lambda x, w, b: composite(x) * w + b, [X, W, B], 4)
    else:
        want = taylor(composite, [X], 4)
    _check(got, want, 1e-12)


def _math_attention(q, k, v, excluded=None, scale=None, additive=None):
    s = (1 / math.sqrt(q.shape[-1]) if scale is None else scale) * (q @ k.transpose(-2, -1))
    if additive is not None:
        s = s + additive
    if excluded is not None:
        s = s.masked_fill(excluded, float("-inf"))
    return torch.softmax(s, -1) @ v


def test_attention_reference_case_boolean_mask():
    # data and mask of /root/reference/tests/test_attention.py:13-17,52; rows with no admissible
    # key are NaN in the plain-range general rule (softmax of an all -inf row)
    g = torch.Generator().manual_seed(27)
    values = [torch.randn(1, 1, 3, 2, generator=g, dtype=torch.float64) / 3 for _ in range(3)]
    directions = [torch.randn(c.shape, generator=g, dtype=c.dtype) / 4 for c in values]
    mask = torch.tensor([[False, False, False], [True, False, True], [True, True, True]])
    Q, K, V = (paths.lift([x, d], 3) for x, d in zip(values, directions))
    got = oracle.attention(Q, K, V, attn_mask=mask)
    want = taylor(lambda q, k, v: _math_attention(q, k, v, excluded=~mask),
                  [[values[i], directions[i]] for i in range(3)], 3)
    for k in range(4):
        assert torch.isnan(got[k][..., 0, :]).all()
        torch.testing.assert_close(got[k][..., 1:, :], want[k][..., 1:, :], atol=2e-14, rtol=2e-12)


@pytest.mark.parametrize("mode", ("causal", "window", "none", "additive"))
def test_attention_general_series(mode):
    L, S, d, degree = 9, 9, 4, 4
    Q, K, V = (_series((2, 2, L, d), degree, seed=30 + i) for i in range(3))
    i = torch.arange(L)
    window = (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] <= 3)
    additive = torch.randn(L, S, generator=torch.Generator().manual_seed(39), dtype=torch.float64)
    kwargs = {"causal": dict(is_causal=True), "window": dict(attn_mask=window), "none": {},
              "additive": dict(attn_mask=additive)}[mode]
    got = oracle.attention(Q, K, V, scale=0.3, **kwargs)
    excluded = {"causal": ~torch.ones(L, S, dtype=torch.bool).tril(), "window": ~window}.get(mode)
    want = taylor(lambda q, k, v: _math_attention(q, k, v, excluded=excluded, scale=0.3,
                                                  additive=additive if mode == "additive" else None),
                  [Q, K, V], degree)
    _check(got, want, 1e-12)


@pytest.mark.parametrize("reduction", ("none", "mean", "sum"))
def test_cross_entropy_general_series(reduction):
    Z = _series((12, 37), 4, seed=40, scale=2.0)
    y = torch.randint(0, 37, (12,), generator=torch.Generator().manual_seed(41))
    y[::5] = -1
    got = oracle.cross_entropy(Z, y, ignore_index=-1, reduction=reduction)
    want = taylor(lambda z: F.cross_entropy(z, y, ignore_index=-1, reduction=reduction), [Z], 4)
    _check(got, want, 1e-12)


@pytest.mark.parametrize("reduction", ("none", "mean", "sum"))
@pytest.mark.parametrize("weighted,smoothing", ((True, 0.0), (False, 0.1), (True, 0.25)))
def test_cross_entropy_weights_and_label_smoothing(reduction, weighted, smoothing):
    # torch's own cross_entropy with class weights / label smoothing, differentiated along the curve
    Z = _series((12, 37), 4, seed=44, scale=2.0)
    y = torch.randint(0, 37, (12,), generator=torch.Generator().manual_seed(45))
    y[::5] = -1
    w = torch.rand(37, generator=torch.Generator().manual_seed(46), dtype=torch.float64) + 0.5 if weighted else None
    got = oracle.cross_entropy(Z, y, ignore_index=-1, reduction=reduction, weight=w, label_smoothing=smoothing)
    want = taylor(lambda z: F.cross_entropy(z, y, weight=w, ignore_index=-1, reduction=reduction,
                                            label_smoothing=smoothing), [Z], 4)
    _check(got, want, 1e-12)


@pytest.mark.parametrize("reduction", ("none", "mean"))
def test_cross_entropy_softcap_general_series(reduction):
    # the composite of /root/reference/src/polytensors/_fused_cross_entropy.py:184-187
    Z = _series((12, 37), 4, seed=42, scale=20.0)
    y = torch.randint(0, 37, (12,), generator=torch.Generator().manual_seed(43))
    y[::4] = -1
    cap = 15.0
    got = oracle.cross_entropy(Z, y, ignore_index=-1, reduction=reduction, softcap=cap)
    want = taylor(lambda z: F.cross_entropy(cap * torch.tanh(z / cap), y, ignore_index=-1, reduction=reduction),
                  [Z], 4)
    _check(got, want, 1e-12)


@pytest.mark.parametrize("degree", (1, 4))
def test_rms_norm_backward_series_matches_jets_of_vjp(degree):
    X = _series((5, 16), degree, seed=54)
    G = _series((5, 16), degree, seed=55)

    def vjp(x, g):
        return torch.func.vjp(lambda z: F.rms_norm(z, (16,), eps=1e-5), x)[1](g)[0]

    _check(oracle.rms_norm_backward(X, G, (16,), eps=1e-5), taylor(vjp, [X, G], degree), 1e-12)


@pytest.mark.parametrize("degree", (1, 4))
def test_layer_norm_backward_series_matches_jets_of_vjp(degree):
    X = _series((5, 16), degree, seed=56)
    G = _series((5, 16), degree, seed=57)

    def layer_norm(z):   # the explicit composite (torch's native layer_norm has wrong higher jets)
        d = z - z.mean(-1, keepdim=True)
        return d * torch.rsqrt((d * d).mean(-1, keepdim=True) + 1e-5)

    def vjp(x, g):
        return torch.func.vjp(layer_norm, x)[1](g)[0]

    _check(oracle.layer_norm_backward(X, G, (16,), eps=1e-5), taylor(vjp, [X, G], degree), 1e-12)


@pytest.mark.parametrize("softcap", (None, 3.0))
def test_cross_entropy_backward_series_matches_jets_of_vjp(softcap):
    degree = 4
    Z = _series((6, 11), degree, seed=58, scale=2.0)
    C = _series((6,), degree, seed=59)
    y = torch.randint(0, 11, (6,), generator=torch.Generator().manual_seed(60))
    y[2] = -1

    def per_row(z):
        if softcap is not None:
            z = softcap * torch.tanh(z / softcap)
        return F.cross_entropy(z, y, ignore_index=-1, reduction="none")

    def vjp(z, c):
        return torch.func.vjp(per_row, z)[1](c)[0]

    got = oracle.cross_entropy_backward(Z, y, C, ignore_index=-1, softcap=softcap)
    _check(got, taylor(vjp, [Z, C], degree), 1e-12)


def test_attention_reference_case_additive_mask():
    # data and additive mask of /root/reference/tests/test_attention.py:13-17,53-54: -inf entries
    # exclude their keys, the others add to the constant-order scores; row 0 has no admissible key
    g = torch.Generator().manual_seed(27)
    values = [torch.randn(1, 1, 3, 2, generator=g, dtype=torch.float64) / 3 for _ in range(3)]
    directions = [torch.randn(c.shape, generator=g, dtype=c.dtype) / 4 for c in values]
    inf = float("-inf")
    mask = torch.tensor([[inf] * 3, [0.2, inf, -0.1], [0.1, -0.3, 0.0]], dtype=torch.float64)
    Q, K, V = (paths.lift([x, d], 3) for x, d in zip(values, directions))
    got = oracle.attention(Q, K, V, attn_mask=mask)
    finite = torch.where(torch.isneginf(mask), torch.zeros(()), mask)
    want = taylor(lambda q, k, v: _math_attention(q, k, v, excluded=torch.isneginf(mask), additive=finite),
                  [[values[i], directions[i]] for i in range(3)], 3)
    for k in range(4):
        assert torch.isnan(got[k][..., 0, :]).all()
        torch.testing.assert_close(got[k][..., 1:, :], want[k][..., 1:, :], atol=2e-14, rtol=2e-12)


@pytest.mark.parametrize("mode,degree", (("causal", 1), ("causal", 3), ("window", 2), ("none", 3),
                                         ("additive", 3)))
def test_attention_backward_series_matches_jets_of_vjp(mode, degree):
    L, S, d = 7, 9, 4
    Q = _series((2, L, d), degree, seed=61)
    K, V = (_series((2, S, d), degree, seed=62 + i) for i in range(2))
    G = _series((2, L, d), degree, seed=64)
    i, j = torch.arange(L)[:, None], torch.arange(S)[None, :]
    window = (i + 2 >= j) & (i + 2 - j <= 3)
    window[3] = False                                      # a query row with no admissible key
    additive = torch.randn(L, S, generator=torch.Generator().manual_seed(65), dtype=torch.float64)
    additive = additive.masked_fill(~window, float("-inf"))
    mask = {"causal": None, "window": window, "none": None, "additive": additive}[mode]
    excluded = {"causal": ~torch.ones(L, S, dtype=torch.bool).tril(), "window": ~window,
                "additive": ~window}.get(mode)
    finite = additive.masked_fill(~window, 0.0) if mode == "additive" else 0.0

    def vjp(q, k, v, g):
        def f(a, b, c):
            s = 0.4 * (a @ b.transpose(-2, -1)) + finite
            if excluded is None:
                return torch.softmax(s, -1) @ c
            empty = excluded.all(-1, keepdim=True)          # such a row: zero output, no gradient
            p = torch.softmax(s.masked_fill(excluded & ~empty, float("-inf")), -1)
            return torch.where(empty, torch.zeros((), dtype=p.dtype), p) @ c
        return torch.func.vjp(f, q, k, v)[1](g)

    got = oracle.attention_backward(Q, K, V, G, attn_mask=mask, is_causal=mode == "causal", scale=0.4)
    want = taylor(vjp, [Q, K, V, G], degree)
    for which in range(3):
        _check(got[which], [w[which] for w in want], 1e-12)


def test_elementwise_product_and_quotient_series():
    # /root/reference/src/polytensors/_range_ops.py:86-93,143-144
    A = _series((4, 9), 5, seed=52)
    B = _series((4, 9), 5, seed=53)
    B[0] = B[0].abs() + 0.5
    _check(series.cauchy(A, B), taylor(lambda a, b: a * b, [A, B], 5), 1e-13)
    _check(oracle.quotient(A, B), taylor(lambda a, b: a / b, [A, B], 5), 1e-12)


def test_matmul_general_series():
    A = _series((3, 6, 5), 4, seed=50)
    B = _series((5, 7), 4, seed=51)
    got = oracle.matmul(A, B)
    want = taylor(lambda a, b: a @ b, [A, B], 4)
    _check(got, want, 1e-13)
    plain = oracle.matmul(A, [B[0]])
    want = taylor(lambda a: a @ B[0], [A], 4)
    _check(plain, want, 1e-13)


# --- planted mistakes: the pins above must catch them ---------------------------------------------

def _rsqrt_dropped_term(X):
    Y = [torch.rsqrt(X[0])]
    n = [None] + [x / X[0] for x in X[1:]]
    for k in range(1, len(X)):
        acc = ((2 * k - 1) / (2 * k)) * n[1] * Y[k - 1]
        for i in range(2, k):          # planted: the i = k term is dropped
            acc = acc + ((2 * k - i) / (2 * k)) * n[i] * Y[k - i]
        Y.append(-acc)
    return Y


def _exp_wrong_weight(X):
    Y = [torch.exp(X[0])]
    for k in range(1, len(X)):
        acc = sum((1 / k) * X[i] * Y[k - i] for i in range(1, k + 1))   # planted: i/k -> 1/k
        Y.append(acc)
    return Y


def _cauchy_wrong_index(left, right, matmul=False):
    out = []
    for k in range(len(left)):
        total = 0
        for i in range(k + 1):
            a, b = left[i], right[max(0, k - i - (1 if i == 0 and k > 1 else 0))]   # planted index slip
            total = total + (a @ b if matmul else a * b)
        out.append(total)
    return out


@pytest.mark.parametrize("target,mutant", [
    ("rsqrt_series", _rsqrt_dropped_term),
    ("exp_series", _exp_wrong_weight),
    ("cauchy", _cauchy_wrong_index),
])
def test_planted_mistakes_are_caught(monkeypatch, target, mutant):
    monkeypatch.setattr(paths, target, mutant, raising=False)
    monkeypatch.setattr(series, target, mutant)
    checks = [
        lambda: test_rms_norm_general_series("series"),
        lambda: test_cross_entropy_general_series("mean"),
        lambda: test_attention_general_series("causal"),
        lambda: test_matmul_general_series(),
    ]
    failures = 0
    for check in checks:
        try:
            check()
        except AssertionError:
            failures += 1
    assert failures >= 1, f"no pin caught the planted mistake in {target}"


# --- complex directions over a real base (config 5) ------------------------------------------------

def _complex_line(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))


def _line_series(x, u, w, degree):
    return [x, torch.complex(u, w)] + [torch.zeros(x.shape, dtype=torch.complex128) for _ in range(degree - 1)]


def _check_complex(got, want, tol):
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        err = (a - b).abs().max().item() / max(b.abs().max().item(), 1e-300)
        assert err <= tol, (k, err)


def _composite_layer_norm(z, shape, weight=None, bias=None, eps=1e-5):
    # torch's native layer_norm has wrong higher-order forward-mode jets; the explicit composite
    d = z - z.mean(-1, keepdim=True)
    out = d * torch.rsqrt((d * d).mean(-1, keepdim=True) + eps)
    return out * weight + bias if weight is not None else out


def test_complex_direction_attention_norm_activation_ce():
    # the oracle's recurrences in complex arithmetic vs mixed real partials (tests/jets.py)
    from tests.jets import taylor_complex

    degree = 3
    q, k, v = (_complex_line((1, 2, 6, 4), 70 + i) for i in range(3))
    got = oracle.attention(*(_line_series(*t, degree) for t in (q, k, v)), is_causal=True)
    excluded = ~torch.ones(6, 6, dtype=torch.bool).tril()
    want = taylor_complex(lambda a, b, c: _math_attention(a, b, c, excluded=excluded),
                          [q[0], k[0], v[0]], [q[1], k[1], v[1]], [q[2], k[2], v[2]], degree)
    _check_complex(got, want, 1e-12)

    x, u, w = _complex_line((5, 16), 73)
    weight, bias = torch.randn(16, dtype=torch.float64), torch.randn(16, dtype=torch.float64)
    got = oracle.layer_norm(_line_series(x, u, w, degree), (16,), weight=[weight], bias=[bias])
    want = taylor_complex(lambda z: _composite_layer_norm(z, (16,), weight, bias), [x], [u], [w], degree)
    _check_complex(got, want, 1e-12)

    got = oracle.activation(_line_series(x, u, w, degree), "gelu_tanh")
    want = taylor_complex(lambda z: F.gelu(z, approximate="tanh"), [x], [u], [w], degree)
    _check_complex(got, want, 1e-12)

    y = torch.randint(0, 16, (5,), generator=torch.Generator().manual_seed(74))
    y[1] = -100
    got = oracle.cross_entropy(_line_series(x, u, w, degree), y)
    want = taylor_complex(lambda z: F.cross_entropy(z, y), [x], [u], [w], degree)
    _check_complex(got, want, 1e-12)


def test_decoder_oracle_matches_complex_jets(monkeypatch):
    # the config-5 network (bench.gpt_forward) at toy size: the oracle composite with a complex
    # embedding direction vs mixed real partials of the same network (math attention)
    import bench
    from tests.jets import taylor_complex

    degree, d, heads, vocab, seq = 3, 16, 2, 11, 5
    params = bench.gpt_init_params(2, d, vocab, seq, seed=3, dtype=torch.float64)
    params["blocks"][0]["ln1_w"] = params["blocks"][0]["ln1_w"] + 0.1   # non-trivial affine terms
    g = torch.Generator().manual_seed(4)
    tokens = torch.randint(0, vocab, (1, seq), generator=g)
    targets = torch.randint(0, vocab, (1, seq), generator=g)
    base = bench.gpt_embed(params, tokens)
    u, w = (torch.randn(base.shape, generator=g, dtype=torch.float64) for _ in range(2))

    def math_sdpa(q, k, v, is_causal):
        L = q.shape[-2]
        return _math_attention(q, k, v, excluded=~torch.ones(L, L, dtype=torch.bool).tril())

    monkeypatch.setattr(F, "layer_norm", _composite_layer_norm)
    got = oracle.gpt_forward(params, _line_series(base, u, w, degree), targets, heads)
    want = taylor_complex(lambda x: bench.gpt_forward(params, x, targets, heads, attention=math_sdpa),
                          [base], [u], [w], degree)
    _check_complex(got, want, 1e-10)


def test_attention_oracle_broadcast_masks_match_per_entry_calls():
    # a mask over the batch ([B, 1, L, S], [1, H, L, S], [B, H, L, S], boolean and additive) gives
    # each (batch, head) entry what the pinned (L, S) path gives it with that entry's mask
    B, H, L, S, d, degree = 2, 3, 7, 9, 4, 2
    Q = _series((B, H, L, d), degree, seed=70)
    K, V, G = (_series((B, H, S, d), degree, seed=71 + i) for i in range(3))
    G = _series((B, H, L, d), degree, seed=74)
    g = torch.Generator().manual_seed(75)
    for shape in ((B, 1, L, S), (1, H, L, S), (B, H, L, S)):
        keep = torch.rand(shape, generator=g) < 0.7
        keep[..., 2, :] = False                            # rows with no admissible key
        additive = torch.randn(shape, generator=g, dtype=torch.float64).masked_fill(~keep, float("-inf"))
        for mask in (keep, additive):
            got = oracle.attention(Q, K, V, attn_mask=mask, scale=0.4)
            grads = oracle.attention_backward(Q, K, V, G, attn_mask=mask, scale=0.4)
            for b in range(B):
                for h in range(H):
                    m = mask[b % mask.shape[0], h % mask.shape[1]]
                    pick = lambda X: [x[b:b + 1, h:h + 1] for x in X]   # noqa: E731
                    want = oracle.attention(pick(Q), pick(K), pick(V), attn_mask=m, scale=0.4)
                    for a, w in zip(got, want):
                        torch.testing.assert_close(a[b:b + 1, h:h + 1], w, equal_nan=True, rtol=0, atol=0)
                    want_g = oracle.attention_backward(pick(Q), pick(K), pick(V), pick(G), attn_mask=m, scale=0.4)
                    for gs, ws in zip(grads, want_g):
                        for a, w in zip(gs, ws):
                            torch.testing.assert_close(a[b:b + 1, h:h + 1], w, rtol=0, atol=0)
