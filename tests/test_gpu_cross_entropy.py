"""Cross-entropy series kernel vs the CPU oracle (GPU).

Mirrors the reference's fused cross-entropy tests
(/root/reference/tests/test_fused_kernels.py:142-181): N=300, C=5000 logits with
every 7th target ignored, all three reductions, F.cross_entropy inside
plain_range() taking the fused path. The oracle (log-softmax series + per-order
NLL) runs in float64 on the same (upcast) inputs. Per-order tolerance
max|got - want| / max|want|: 1e-10 float64, 1e-4 float32, 2e-2 bfloat16/float16.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import paths
from polytensors_amd import PolyTensor, _fused_cross_entropy, _ops

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _logits(N, C, degree, seed, dtype, base_scale=3.0, pad=0):
    g = torch.Generator().manual_seed(seed)
    full = [(torch.randn(N, C + pad, generator=g, dtype=torch.float64) * (base_scale if k == 0 else 0.5 ** k))
            .to(dtype) for k in range(degree + 1)]
    target = torch.randint(0, C, (N,), generator=g)
    return full, target


def _check(got, want, dtype, inputs=None):
    # max |got - want| / max |want|. A loss coefficient is lse_k - z_k[y]; when it vanishes
    # identically (one class) both results are the rounding of cancelling O(|z_k|) terms, so the
    # scale is floored at the order's input scale max |z_k| when the inputs are given.
    for k, (a, b) in enumerate(zip(got, want)):
        a, b = a.cpu().double(), b.double()
        scale = b.abs().max().item()
        if inputs is not None:
            scale = max(scale, inputs[k].double().abs().max().item())
        err = (a - b).abs().max().item() / scale
        assert err <= TOL[dtype], f"order {k}: {err:.3e}"


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("degree", [1, 4])
def test_matches_oracle_with_ignored_rows(monkeypatch, reduction, degree):
    calls = []
    original = _ops.cross_entropy_series
    monkeypatch.setattr(_ops, "cross_entropy_series", lambda *a, **k: calls.append(1) or original(*a, **k))
    Z, y = _logits(300, 5000, degree, seed=0, dtype=torch.float32)
    y[::7] = -1
    logits = PolyTensor(tuple(c.cuda() for c in Z))
    with torch.no_grad(), PolyTensor.plain_range():
        assert _fused_cross_entropy.eligible(logits, y.cuda(), None, reduction, 0.0)
        loss = F.cross_entropy(logits, y.cuda(), ignore_index=-1, reduction=reduction)
    assert calls == [1]
    assert loss.dtype == torch.float32 and loss.degree == degree
    want = oracle.cross_entropy([c.double() for c in Z], y, ignore_index=-1, reduction=reduction)
    _check(loss.coeffs, want, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("degree", [0, 2, 3, 5, 8])
def test_dtypes_and_degrees(dtype, degree):
    Z, y = _logits(64, 1000, degree, seed=1, dtype=dtype)
    with torch.no_grad(), PolyTensor.plain_range():
        loss = PolyTensor.cross_entropy(PolyTensor(tuple(c.cuda() for c in Z)), y.cuda(), reduction="none")
    assert loss.dtype == torch.promote_types(dtype, torch.float32)   # PolyTensor.cross_entropy: at least float32
    want = oracle.cross_entropy([c.double() for c in Z], y, reduction="none")
    _check(loss.coeffs, want, dtype)


@pytest.mark.parametrize("C,pad", [(3000, 64), (777, 0), (5, 3), (1, 0), (257, 1), (40000, 0)])
def test_row_strides_and_class_counts(C, pad):
    # a sliced (padded) row stride stays a zero-copy view; odd strides take the scalar path
    degree = 3
    full, y = _logits(50, C, degree, seed=2, dtype=torch.float32, pad=pad)
    dev = [c.cuda() for c in full]
    logits = PolyTensor(tuple(c[:, :C] for c in dev))
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(logits, y.cuda(), reduction="none")
    want = oracle.cross_entropy([c[:, :C].double() for c in full], y, reduction="none")
    _check(loss.coeffs, want, torch.float32, inputs=[c[:, :C] for c in full])


def test_lse_series_output():
    degree = 4
    Z, y = _logits(40, 2000, degree, seed=3, dtype=torch.float32)
    _, lse = _ops.cross_entropy_series([c.cuda() for c in Z], y.cuda(), -100, 0, 0.0)
    want = paths.logsumexp([c.double() for c in Z], 1)
    _check(list(lse.unbind(0)), want, torch.float32)


def test_all_ignored_mean_is_nan_like_torch():
    Z, y = _logits(8, 100, 2, seed=4, dtype=torch.float32)
    y[:] = -100
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(PolyTensor(tuple(c.cuda() for c in Z)), y.cuda())
    native = F.cross_entropy(Z[0], y)
    assert math.isnan(native.item())
    assert all(torch.isnan(c).item() for c in loss.coeffs)


def test_large_common_offset_keeps_higher_orders_exact():
    # /root/reference/tests/test_series.py:113-120 through the kernel: logits 1e20 + t.
    base = torch.full((3, 2), 1e20, dtype=torch.float32)
    coeffs = (base, torch.ones_like(base), *(torch.zeros_like(base) for _ in range(3)))
    _, lse = _ops.cross_entropy_series([c.cuda() for c in coeffs], torch.zeros(3, dtype=torch.int64).cuda(), -100, 0, 0.0)
    lse = lse.cpu()
    assert torch.equal(lse[1], torch.ones(3))
    assert torch.equal(lse[2:], torch.zeros(3, 3))


def test_full_size_config_rows_sample():
    # benchmark config 4b: [5, 8192, 32000] fp32, base N(0, 2^2), order k N(0,1) 0.5^k; the mean must
    # equal the mean of the per-row losses, and a seeded sample of rows must match the oracle.
    degree, N, C = 4, 8192, 32000
    g = torch.Generator(device="cuda").manual_seed(4)
    Z = [torch.randn(N, C, generator=g, device="cuda") * (2.0 if k == 0 else 0.5 ** k) for k in range(degree + 1)]
    y = torch.randint(0, C, (N,), generator=g, device="cuda")
    rows, _ = _ops.cross_entropy_series(Z, y, -100, 0, 0.0)
    mean, _ = _ops.cross_entropy_series(Z, y, -100, 1, 0.0)
    for k in range(degree + 1):
        assert abs(mean[k].item() - rows[k].double().mean().item()) <= 1e-5 * max(1.0, abs(mean[k].item()))
    pick = torch.randperm(N, generator=torch.Generator().manual_seed(5))[:32].cuda()
    want = oracle.cross_entropy([c[pick].cpu().double() for c in Z], y[pick].cpu(), reduction="none")
    _check([r[pick] for r in rows], want, torch.float32)


@pytest.mark.parametrize("strided", [False, True])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("degree", [1, 4])
def test_softcap_matches_oracle(monkeypatch, degree, dtype, strided):
    # /root/reference/tests/test_fused_kernels.py:186-211: N=200, C=3000 logits of scale 40, cap 15,
    # every 5th target ignored, optionally a padded (strided) row slice; the kernel caps on the fly.
    calls = []
    original = _ops.cross_entropy_series
    monkeypatch.setattr(_ops, "cross_entropy_series", lambda *a, **k: calls.append(1) or original(*a, **k))
    N, C, pad, cap = 200, 3000, 64 if strided else 0, 15.0
    g = torch.Generator().manual_seed(1)
    full = [(torch.randn(N, C + pad, generator=g, dtype=torch.float64) * 40 * 0.5 ** k).to(dtype)
            for k in range(degree + 1)]
    y = torch.randint(0, C, (N,), generator=g)
    y[::5] = -1
    logits = PolyTensor(tuple(c.cuda() for c in full))
    with torch.no_grad(), PolyTensor.plain_range():
        sliced = logits[:, :C]
        loss = PolyTensor.cross_entropy(sliced, y.cuda(), softcap=cap, ignore_index=-1, reduction="none")
    assert calls == [1] and loss.degree == degree
    Z = [c[:, :C].double() for c in full]
    want = oracle.cross_entropy(Z, y, ignore_index=-1, reduction="none", softcap=cap)
    capped = [cap * t for t in oracle.activation([z / cap for z in Z], "tanh")]
    _check(loss.coeffs, want, dtype, inputs=capped)


def test_softcap_mean_and_lse_at_degree_eight():
    N, C, cap = 64, 1000, 7.5
    Z, y = _logits(N, C, 8, seed=9, dtype=torch.float64, base_scale=10.0)
    out, lse = _ops.cross_entropy_series([c.cuda() for c in Z], y.cuda(), -100, 1, cap)
    want = oracle.cross_entropy(Z, y, reduction="mean", softcap=cap)
    _check(list(out), want, torch.float64)
    capped = [cap * t for t in oracle.activation([z / cap for z in Z], "tanh")]
    want_lse = paths.logsumexp(capped, dim=1)
    _check(list(lse), want_lse, torch.float64)


def test_softcap_must_be_positive():
    Z, y = _logits(4, 16, 1, seed=10, dtype=torch.float32)
    with torch.no_grad(), PolyTensor.plain_range():
        with pytest.raises(NotImplementedError, match="softcap"):
            PolyTensor.cross_entropy(PolyTensor(tuple(c.cuda() for c in Z)), y.cuda(), softcap=-1.0)


def test_expanded_logits_rows_are_materialized():
    # an expanded (broadcast) row has row stride 0; the glue must copy it rather than hand the
    # kernel overlapping rows
    degree = 2
    g = torch.Generator().manual_seed(5)
    row = [torch.randn(1, 300, generator=g, dtype=torch.float64).mul(0.5 ** k).float() for k in range(degree + 1)]
    y = torch.randint(0, 300, (6,), generator=g)
    logits = PolyTensor(tuple(c.cuda().expand(6, 300) for c in row))
    assert logits.coeffs[0].stride(0) == 0
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(logits, y.cuda(), reduction="none")
    want = oracle.cross_entropy([c.double().expand(6, 300) for c in row], y, reduction="none")
    _check(loss.coeffs, want, torch.float32)


# Class weights and label smoothing: the reference's general rule (torch's cross_entropy decomposed
# into log_softmax and its linear terms, /root/reference/src/polytensors/_decompositions.py:66-67);
# the oracle restates those terms per order and is pinned by jets of torch's own cross_entropy.
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("weighted,smoothing", [(True, 0.0), (False, 0.1), (True, 0.3)])
def test_weights_and_label_smoothing(dtype, reduction, weighted, smoothing):
    degree = 3
    Z, y = _logits(200, 700, degree, seed=60, dtype=dtype)
    y[::9] = -1
    w = (torch.rand(700, generator=torch.Generator().manual_seed(61), dtype=torch.float64) + 0.5).to(dtype) \
        if weighted else None
    logits = PolyTensor(tuple(c.cuda() for c in Z))
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(logits, y.cuda(), weight=None if w is None else w.cuda(), ignore_index=-1,
                               reduction=reduction, label_smoothing=smoothing)
    assert loss.dtype == dtype and loss.degree == degree
    want = oracle.cross_entropy([c.double() for c in Z], y, ignore_index=-1, reduction=reduction,
                                weight=None if w is None else w.double(), label_smoothing=smoothing)
    _check(loss.coeffs, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("weighted", [False, True])
def test_label_smoothing_with_a_large_common_offset(dtype, weighted):
    # logits shifted by +100 over C = 32000 classes: the smoothing term sum_c w_c (lse - z_c) does
    # not depend on such a shift and must not lose precision to it. (A shift of the higher orders
    # is another matter: the plain-range log-sum-exp series of [z_0, z_1 + c, ...] cancels terms of
    # size c^k in every formulation, the reference's included, so it is not part of this case.)
    degree, N, C = 3, 48, 32000
    Z, y = _logits(N, C, degree, seed=65, dtype=torch.float64, base_scale=2.0)
    Z = [(c + (100.0 if k == 0 else 0.0)).to(dtype) for k, c in enumerate(Z)]
    y[::5] = -100
    w = (torch.rand(C, generator=torch.Generator().manual_seed(66), dtype=torch.float64) + 0.5).to(dtype) \
        if weighted else None
    logits = PolyTensor(tuple(c.cuda() for c in Z))
    for reduction in ("none", "mean"):
        with torch.no_grad(), PolyTensor.plain_range():
            loss = F.cross_entropy(logits, y.cuda(), weight=None if w is None else w.cuda(), reduction=reduction,
                                   label_smoothing=0.1)
        want = oracle.cross_entropy([c.double() for c in Z], y, reduction=reduction,
                                    weight=None if w is None else w.double(), label_smoothing=0.1)
        _check(loss.coeffs, want, dtype)


@pytest.mark.parametrize("reduction", ["none", "mean"])
def test_logits_with_extra_dimensions(reduction):
    # (N, C, d1, d2) logits with (N, d1, d2) targets: rows of C classes, as torch's cross_entropy
    degree, N, C = 2, 3, 40
    g = torch.Generator().manual_seed(62)
    Z = [torch.randn(N, C, 5, 7, generator=g, dtype=torch.float64) * 0.5 ** k for k in range(degree + 1)]
    y = torch.randint(0, C, (N, 5, 7), generator=g)
    y[0, 1] = -100
    logits = PolyTensor(tuple(c.cuda() for c in Z))
    with torch.no_grad(), PolyTensor.plain_range():
        loss = F.cross_entropy(logits, y.cuda(), reduction=reduction, label_smoothing=0.2)
    rows = [z.movedim(1, -1).reshape(-1, C) for z in Z]
    want = oracle.cross_entropy(rows, y.reshape(-1), reduction=reduction, label_smoothing=0.2)
    if reduction == "none":
        want = [x.reshape(N, 5, 7) for x in want]
    _check(loss.coeffs, want, torch.float64)


@pytest.mark.parametrize("weighted,smoothing", [(True, 0.0), (False, 0.15), (True, 0.15)])
def test_weights_and_label_smoothing_gradient_series(weighted, smoothing):
    # PolyTensor.backward of the mean loss: the gradient series of the logits must be the Taylor
    # series of torch.func.grad of torch's own cross_entropy along the curve
    from tests.jets import taylor

    degree = 3
    Z, y = _logits(40, 60, degree, seed=63, dtype=torch.float64, base_scale=1.5)
    y[::6] = -1
    w = torch.rand(60, generator=torch.Generator().manual_seed(64), dtype=torch.float64) + 0.5 if weighted else None

    def loss(z):
        return F.cross_entropy(z, y, weight=w, ignore_index=-1, label_smoothing=smoothing)

    x = PolyTensor(tuple(c.cuda() for c in Z), requires_grad=True)
    with PolyTensor.plain_range(), PolyTensor.retain_wrappers():
        out = F.cross_entropy(x, y.cuda(), weight=None if w is None else w.cuda(), ignore_index=-1,
                              label_smoothing=smoothing)
        out.backward()
    _check(out.coeffs, taylor(loss, [Z], degree), torch.float64)
    _check(x.grad.coeffs, taylor(lambda z: torch.func.grad(loss)(z), [Z], degree), torch.float64)
