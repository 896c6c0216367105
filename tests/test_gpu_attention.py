"""Taylor flash-attention kernel vs the CPU oracle (GPU).

Mirrors the reference's fused-attention tests (/root/reference/tests/test_fused_kernels.py:48-134):
shape (2, 3, 150, 64), causal, a window-37 boolean mask and unmasked, explicit
scale, plain operands, F.scaled_dot_product_attention inside plain_range()
taking the fused path, here at degrees up to 8. The oracle is the reference's
plain-range decomposition (softmax series of the masked Cauchy-product scores,
then the Cauchy product with V) in float64 on the same (upcast) inputs.
Per-order tolerance max|got - want| / max|want|: 1e-10 float64, 1e-4 float32.
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import paths, series
from polytensors_amd import PolyTensor, _fused_attention, _ops
from tests.jets import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float64: 1e-10, torch.float32: 1e-4}


def _series(shape, degree, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g, dtype=torch.float64) * scale * 0.5 ** k).to(dtype)
            for k in range(degree + 1)]


def _poly(cs):
    return PolyTensor(tuple(c.cuda() for c in cs))


def _window_mask(L, window):
    i = torch.arange(L)
    return (i[:, None] >= i[None, :]) & (i[:, None] - i[None, :] <= window)


def _check(got, want, dtype):
    for k, (a, b) in enumerate(zip(got, want)):
        err = rel_err(a.cpu(), b)
        assert err <= TOL[dtype], f"order {k}: {err:.3e}"


def _run(q, k, v, **kwargs):
    with torch.no_grad(), PolyTensor.plain_range():
        return F.scaled_dot_product_attention(q, k, v, **kwargs)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("causal,window", [(True, None), (False, 37), (False, None)])
@pytest.mark.parametrize("degree", [1, 4])
def test_matches_oracle(monkeypatch, dtype, causal, window, degree):
    calls = []
    original = _ops.taylor_attention_fwd
    monkeypatch.setattr(_ops, "taylor_attention_fwd", lambda *a, **k: calls.append(1) or original(*a, **k))
    shape = (2, 3, 150, 64)
    Q, K, V = (_series(shape, degree, 10 + i, dtype) for i in range(3))
    mask = None if window is None else _window_mask(150, window)
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=None if mask is None else mask.cuda(), is_causal=causal)
    assert calls == [1] and out.degree == degree and out.dtype == dtype
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                            attn_mask=mask, is_causal=causal)
    _check(out.coeffs, want, dtype)


@pytest.mark.parametrize("degree", [0, 2, 3, 5, 6, 7, 8])
@pytest.mark.parametrize("d", [16, 32, 128])
def test_every_degree_and_head_dim(degree, d):
    shape = (1, 2, 70, d)
    Q, K, V = (_series(shape, degree, 20 + i, torch.float32) for i in range(3))
    out = _run(_poly(Q), _poly(K), _poly(V), is_causal=True)
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V], is_causal=True)
    _check(out.coeffs, want, torch.float32)


@pytest.mark.parametrize("case", ["moderate", "rising", "orthogonal_norms"])
@pytest.mark.parametrize("causal", [True, False])
def test_running_maximum_of_the_pipelined_kernel(case, causal):
    # The float32 pipelined kernel shifts the exponentials by a running maximum of the order-0
    # scores, raised only when a key block's maximum exceeds it by more than 8, with the output
    # accumulators and row sums rescaled then. The output must not depend on the shift.
    # "moderate": order-0 scores three times larger. "rising": one query dimension at 8 and the
    # keys' ramping from 0 to 80 along the sequence, so the scores climb about 8.5 per 16-key block
    # and the maximum rises (rescaling the accumulators) block after block, up to scores near 80.
    # "orthogonal_norms": |q| and |k| near 400 in dimensions the other operand leaves at zero.
    shape = (1, 2, 150, 64)
    Q, K, V = (_series(shape, 3, 50 + i, torch.float32) for i in range(3))
    if case == "moderate":
        Q[0], K[0] = Q[0] * 3, K[0] * 3
    elif case == "rising":
        Q[0][..., 0] = 8.0
        K[0][..., 0] = torch.linspace(0.0, 80.0, 150)
    else:
        Q[0][..., 0], Q[0][..., 1] = 400.0, 0.0
        K[0][..., 0], K[0][..., 1] = 0.0, 400.0
    mask = None if causal else _window_mask(150, 37)
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=None if mask is None else mask.cuda(), is_causal=causal)
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                            attn_mask=mask, is_causal=causal)
    _check(out.coeffs, want, torch.float32)


@pytest.mark.parametrize("L,S", [(1, 16), (17, 16), (65, 33), (130, 47)])
@pytest.mark.parametrize("mode", ["causal", "mask_with_empty_row", "none"])
def test_pipelined_kernel_short_and_ragged(L, S, mode):
    # float32, full orders: the pipelined kernel. With few key blocks, rows past L and rows with no
    # admissible key (whose running maximum never leaves -inf) must come out as in the oracle
    # (empty rows: zero, the fused-kernel convention).
    Q = _series((1, 2, L, 64), 2, 70, torch.float32)
    K, V = (_series((1, 2, S, 64), 2, 71 + i, torch.float32) for i in range(2))
    mask = None
    if mode == "mask_with_empty_row":
        g = torch.Generator().manual_seed(73)
        mask = torch.rand(L, S, generator=g) < 0.6
        mask[L // 2] = False
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=None if mask is None else mask.cuda(),
               is_causal=mode == "causal")
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                            attn_mask=mask, is_causal=mode == "causal")
    if mask is not None:   # the plain-range rule gives NaN on a row with no admissible key; the kernels 0
        empty = ~mask.any(-1)
        want = [torch.where(empty[:, None], torch.zeros_like(w), w) for w in want]
        for c in out.coeffs:
            assert torch.equal(c.cpu()[..., empty, :], torch.zeros_like(c.cpu()[..., empty, :]))
    _check(out.coeffs, want, torch.float32)


def test_scale_argument_and_default():
    shape = (1, 2, 40, 64)
    Q, K, V = (_series(shape, 3, 30 + i, torch.float64) for i in range(3))
    out = _run(_poly(Q), _poly(K), _poly(V), is_causal=True, scale=0.3)
    want = oracle.attention([c for c in Q], [c for c in K], [c for c in V], is_causal=True, scale=0.3)
    _check(out.coeffs, want, torch.float64)
    assert math.isclose(_fused_attention.default_scale(64), 0.125)


def test_plain_operands():
    # /root/reference/tests/test_fused_kernels.py:112-122: an ordinary key tensor has a zero tangent
    shape = (2, 2, 64, 32)
    Q, V = _series(shape, 2, 40, torch.float64), _series(shape, 2, 41, torch.float64)
    k = torch.randn(shape, generator=torch.Generator().manual_seed(42), dtype=torch.float64)
    out = _run(_poly(Q), k.cuda(), _poly(V), is_causal=True)
    want = oracle.attention(Q, [k], V, is_causal=True)
    _check(out.coeffs, want, torch.float64)


def test_cross_attention_lengths():
    Q = _series((1, 2, 50, 64), 3, 43, torch.float32)
    K, V = _series((1, 2, 90, 64), 3, 44, torch.float32), _series((1, 2, 90, 64), 3, 45, torch.float32)
    for causal in (False, True):
        out = _run(_poly(Q), _poly(K), _poly(V), is_causal=causal)
        want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                                is_causal=causal)
        _check(out.coeffs, want, torch.float32)


def test_fully_masked_row_is_zero_with_infinite_lse():
    # The reference's fused kernel convention (/root/reference/src/polytensors/_attention_kernels.py:70-76):
    # a row with no admissible key gets output zero and lse = +inf.
    L = 24
    Q, K, V = (_series((1, 1, L, 32), 2, 50 + i, torch.float64) for i in range(3))
    mask = _window_mask(L, 3)
    mask[5, :] = False
    out, lse = _ops.taylor_attention_fwd([c.cuda().reshape(1, L, 32) for c in Q],
                                         [c.cuda().reshape(1, L, 32) for c in K],
                                         [c.cuda().reshape(1, L, 32) for c in V], mask.cuda(), False, 0.2, 2)
    assert torch.equal(out[:, 0, 5].cpu(), torch.zeros(3, 32, dtype=torch.float64))
    assert lse[0, 0, 5].item() == math.inf and lse[1:, 0, 5].abs().max().item() == 0
    keep = torch.ones(L, dtype=torch.bool)
    keep[5] = False
    want = oracle.attention(Q, K, V, attn_mask=mask, scale=0.2)
    _check([o[0][keep] for o in out], [w[0, 0][keep] for w in want], torch.float64)


def test_lse_series_output():
    L, d, degree = 48, 64, 3
    Q, K, V = (_series((1, 1, L, d), degree, 60 + i, torch.float64) for i in range(3))
    _, lse = _ops.taylor_attention_fwd([c.cuda().reshape(1, L, d) for c in Q], [c.cuda().reshape(1, L, d) for c in K],
                                       [c.cuda().reshape(1, L, d) for c in V], None, True, 0.125, degree)
    scores = series.cauchy([q * 0.125 for q in Q], [k.transpose(-2, -1) for k in K], matmul=True)
    excluded = ~torch.ones(L, L, dtype=torch.bool).tril()
    scores = [torch.where(excluded, torch.tensor(-math.inf if o == 0 else 0.0, dtype=torch.float64), s)
              for o, s in enumerate(scores)]
    want = paths.logsumexp(scores, -1)
    _check([x.reshape(1, 1, L) for x in lse.unbind(0)], want, torch.float64)


def test_config1_fp64_attention_and_projected_cross_entropy():
    # benchmark config 1: K=3, fp64, Q/K/V [1,1,128,64] = x + t v with x, v ~ N(0,1)/8 (seed 0), causal;
    # logits = out.view(128, 64) @ W with W ~ N(0,1)/8 [64, 256], integer targets in [0, 256), mean CE.
    g = torch.Generator().manual_seed(0)
    shape = (1, 1, 128, 64)
    lines = [(torch.randn(shape, generator=g, dtype=torch.float64) / 8,
              torch.randn(shape, generator=g, dtype=torch.float64) / 8) for _ in range(3)]
    W = torch.randn(64, 256, generator=g, dtype=torch.float64) / 8
    y = torch.randint(0, 256, (128,), generator=g)
    q, k, v = (PolyTensor((x.cuda(), d.cuda()), degree=3) for x, d in lines)
    with torch.no_grad(), PolyTensor.plain_range():
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        logits = out.reshape(128, 64) @ W.cuda()
        loss = F.cross_entropy(logits, y.cuda())
    Qs, Ks, Vs = (paths.lift([x, d], 3) for x, d in lines)
    want = oracle.attention(Qs, Ks, Vs, is_causal=True)
    _check(out.coeffs, want, torch.float64)
    want_logits = oracle.matmul([w.reshape(128, 64) for w in want], [W])
    _check(logits.coeffs, want_logits, torch.float64)
    want_loss = oracle.cross_entropy(want_logits, y)
    for k_, (a, b) in enumerate(zip(loss.coeffs, want_loss)):
        assert abs(a.item() - b.item()) <= 1e-10 * max(1.0, abs(b.item())), k_


def test_full_size_config3_one_head():
    # benchmark config 3: B=4 H=16 L=2048 d=128, K=4, fp32, causal; line inputs (x + t v). One (b, h) of
    # the full launch is checked against the oracle; every head's order-0 output is checked against
    # torch's own fp32 attention (the ordinary softmax attention that order 0 equals).
    B, H, L, d, degree = 4, 16, 2048, 128, 4
    g = torch.Generator(device="cuda").manual_seed(2)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device="cuda") / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device="cuda")
        return [base, direction] + [torch.zeros_like(base) for _ in range(degree - 1)]

    q, k, v = line(), line(), line()
    out, _ = _ops.taylor_attention_fwd(q, k, v, None, True, 1 / math.sqrt(d), degree)
    head = 37
    want = oracle.attention([c[head].cpu().double() for c in q], [c[head].cpu().double() for c in k],
                            [c[head].cpu().double() for c in v], is_causal=True)
    _check([o[head] for o in out], want, torch.float32)
    torch.backends.cuda.matmul.allow_tf32 = False
    ref0 = torch.softmax((q[0] @ k[0].transpose(-1, -2).contiguous() / math.sqrt(d)).masked_fill(
        ~torch.ones(L, L, dtype=torch.bool, device="cuda").tril(), -math.inf), -1) @ v[0]
    assert rel_err(out[0].cpu(), ref0.cpu()) <= 1e-4


def test_full_size_config3_all_heads_linear_in_the_value_series():
    # benchmark config 3's full launch (B=4 H=16 L=2048 d=128, K=4, fp32, causal, line inputs): every
    # head and every order of O(t) = softmax(S(t)) V(t) is linear in the value series, so
    # O[V + 2 W] = O[V] + 2 O[W] holds for all 64 heads at once (each side a separate launch).
    B, H, L, d, degree = 4, 16, 2048, 128, 4
    g = torch.Generator(device="cuda").manual_seed(21)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device="cuda") / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device="cuda")
        return [base, direction] + [torch.zeros_like(base) for _ in range(degree - 1)]

    q, k, v, w = line(), line(), line(), line()
    scale = 1 / math.sqrt(d)
    o_v, _ = _ops.taylor_attention_fwd(q, k, v, None, True, scale, degree)
    o_w, _ = _ops.taylor_attention_fwd(q, k, w, None, True, scale, degree)
    o_sum, _ = _ops.taylor_attention_fwd(q, k, [a + 2 * b for a, b in zip(v, w)], None, True, scale, degree)
    want = o_v + 2 * o_w
    for order in range(degree + 1):
        for head in range(B * H):
            err = ((o_sum[order, head] - want[order, head]).abs().max() / want[order, head].abs().max()).item()
            assert err <= 1e-4, f"order {order}, head {head}: {err:.3e}"


# The pipelined fp32 kernel runs for full-order operands with a key length that is a multiple of 16
# (and two K/V tiles within LDS); these shapes exercise it.
@pytest.mark.parametrize("d,degree", [(16, 1), (16, 8), (32, 4), (64, 4), (64, 8), (128, 1), (128, 4)])
@pytest.mark.parametrize("causal,window", [(True, None), (False, 21), (False, None)])
def test_pipelined_kernel_shapes(d, degree, causal, window):
    shape = (2, 3, 144, d)
    Q, K, V = (_series(shape, degree, 70 + i, torch.float32) for i in range(3))
    mask = None if window is None else _window_mask(144, window)
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=None if mask is None else mask.cuda(), is_causal=causal)
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                            attn_mask=mask, is_causal=causal)
    _check(out.coeffs, want, torch.float32)


@pytest.mark.parametrize("L,S", [(50, 96), (100, 32), (16, 16), (1, 64)])
def test_pipelined_kernel_cross_lengths(L, S):
    Q = _series((1, 2, L, 128), 4, 80, torch.float32)
    K, V = _series((1, 2, S, 128), 4, 81, torch.float32), _series((1, 2, S, 128), 4, 82, torch.float32)
    for causal in (False, True):
        out = _run(_poly(Q), _poly(K), _poly(V), is_causal=causal)
        want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                                is_causal=causal)
        _check(out.coeffs, want, torch.float32)


def test_empty_key_length_gives_empty_rows():
    # zero keys: every row is empty (zero output, +inf order-0 log-sum-exp) on both fp32 paths' dispatch
    for dtype in (torch.float32, torch.float64):
        q = [torch.randn(2, 5, 32, dtype=dtype, device="cuda") for _ in range(5)]
        kv = [torch.empty(2, 0, 32, dtype=dtype, device="cuda") for _ in range(5)]
        for causal in (False, True):
            out, lse = _ops.taylor_attention_fwd(q, kv, kv, None, causal, 0.1, 4)
            assert torch.equal(out, torch.zeros_like(out))
            assert torch.isinf(lse[0]).all() and (lse[1:] == 0).all()


def _ranges_reference(mask, block=64):
    # per query block / key block, first and one-past-last admissible index (0, 0 if none), the
    # definition of /root/reference/src/polytensors/_fused_attention.py:81-99 at block 64
    L, S = mask.shape
    out = []
    for r0 in range(0, L, block):
        cols = mask[r0:r0 + block].any(0).nonzero().flatten()
        out += [int(cols[0]), int(cols[-1]) + 1] if len(cols) else [0, 0]
    for c0 in range(0, S, block):
        rows = mask[:, c0:c0 + block].any(1).nonzero().flatten()
        out += [int(rows[0]), int(rows[-1]) + 1] if len(rows) else [0, 0]
    return out


@pytest.mark.parametrize("L,S", [(150, 150), (64, 200), (300, 37), (1, 1), (256, 320), (130, 208), (96, 272)])
def test_mask_ranges_kernel(L, S):
    # (S a multiple of 16: the kernel's 16-byte path; (96, 272): one admissible key per row, at a
    # random column, so the first and last admissible byte of each chunk are checked exactly)
    g = torch.Generator().manual_seed(L + S)
    if (L, S) == (96, 272):
        mask = torch.zeros(L, S, dtype=torch.bool)
        mask[torch.arange(L), torch.randint(0, S, (L,), generator=g)] = True
    else:
        mask = _window_mask(max(L, S), 23)[:L, :S] & (torch.rand(L, S, generator=g) > 0.3)
    if L > 70:
        mask[64:128] = False          # a query block with no admissible key
    if S > 70:
        mask[:, 64:128] = False       # a key block no query admits
    got = _ops._mask_ranges(mask.cuda(), L, S)
    assert got.cpu().tolist()[:len(_ranges_reference(mask))] == _ranges_reference(mask)


# Sliding windows much narrower than the sequence: the kernels skip the key blocks outside each
# query block's range (and, in the pipelined kernel, keep one fully masked block for a query block
# with no admissible key).
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sliding_window_skips_blocks(dtype):
    L, d, degree = 704, 64, 2
    mask = _window_mask(L, 60)
    mask[256:320] = False
    Q, K, V = (_series((1, 2, L, d), degree, 90 + i, dtype) for i in range(3))
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=mask.cuda())
    want = oracle.attention([c.double() for c in Q], [c.double() for c in K], [c.double() for c in V],
                            attn_mask=mask)
    for k, (a, b) in enumerate(zip(out.coeffs, want)):
        a = a.cpu()
        assert torch.equal(a[..., 256:320, :], torch.zeros_like(a[..., 256:320, :]))
        keep = torch.ones(L, dtype=torch.bool)
        keep[256:320] = False
        assert rel_err(a[..., keep, :], b[..., keep, :]) <= TOL[dtype], k


@pytest.mark.parametrize("degree", range(9))
@pytest.mark.parametrize("d", [64, 128])
def test_float64_every_degree_with_output_slices(degree, d):
    # float64 splits the output head dims over workgroups at head dim 128 from degree 3 and 64
    # from degree 6, and stages K then V through one LDS buffer at head dim 128 from degree 7
    shape = (1, 2, 70, d)
    Q, K, V = (_series(shape, degree, 140 + i, torch.float64) for i in range(3))
    mask = _window_mask(70, 23) if degree % 2 else None
    out = _run(_poly(Q), _poly(K), _poly(V), attn_mask=None if mask is None else mask.cuda(), is_causal=mask is None)
    want = oracle.attention(Q, K, V, attn_mask=mask, is_causal=mask is None)
    _check(out.coeffs, want, torch.float64)


def test_float64_plain_key_with_output_slices():
    degree, shape = 5, (1, 2, 40, 128)
    Q, V = (_series(shape, degree, 150 + i, torch.float64) for i in range(2))
    Kp = _series(shape, 0, 152, torch.float64)[0]
    out = _run(_poly(Q), Kp.cuda(), _poly(V), is_causal=True)
    Ks = [Kp] + [torch.zeros_like(Kp) for _ in range(degree)]
    _check(out.coeffs, oracle.attention(Q, Ks, V, is_causal=True), torch.float64)


def test_float64_head_dim_128_gradients_at_degree_4():
    # wrapper autograd through the forward's output slices and the backward's shared tile buffer,
    # against the oracle's VJP series (G = the all-ones constant series)
    degree, shape = 4, (1, 1, 40, 128)
    Q, K, V = (_series(shape, degree, 160 + i, torch.float64) for i in range(3))
    xs = [PolyTensor(tuple(c.cuda() for c in X), requires_grad=True) for X in (Q, K, V)]
    with PolyTensor.retain_wrappers(), PolyTensor.plain_range():
        assert _fused_attention.eligible(*xs, is_causal=True)
        out = F.scaled_dot_product_attention(*xs, is_causal=True)
        out.backward(PolyTensor.constant(torch.ones_like(out.value), degree))
    G = [torch.ones(shape, dtype=torch.float64)] + [torch.zeros(shape, dtype=torch.float64)] * degree
    want = oracle.attention_backward(Q, K, V, G, is_causal=True)
    for x, w in zip(xs, want):
        _check(x.grad.coeffs, w, torch.float64)


@pytest.mark.parametrize("dtype,L,S,causal,masked", [(torch.float64, 128, 128, True, False),
                                                    (torch.float64, 96, 150, False, True),
                                                    (torch.float32, 128, 70, True, False),
                                                    (torch.float64, 1, 300, False, False)])
def test_key_split_launch_matches_the_unsplit_one(dtype, L, S, causal, masked):
    # launches of few workgroups divide each key range over several workgroups and merge their
    # partial sums (pt_taylor_attention_fwd_ws, which the operator calls); the plain entry point runs
    # the same launch unsplit
    from polytensors_amd import _lib

    degree, d, bh = 3, 64, 1
    Q = _series((bh, L, d), degree, 170, dtype)
    K, V = (_series((bh, S, d), degree, 171 + i, dtype) for i in range(2))
    mask = (torch.rand(L, S, generator=torch.Generator().manual_seed(9)) < 0.5) if masked else None
    lib = _lib.load()
    code = _lib.DTYPE_CODES[dtype]
    assert lib.pt_taylor_attention_fwd_workspace_size(code, degree, degree + 1, degree + 1, degree + 1, bh, L, S, d) > 0
    q, k, v = ([c.cuda() for c in X] for X in (Q, K, V))
    m = None if mask is None else mask.cuda()
    out, lse = _ops.taylor_attention_fwd(q, k, v, m, causal, 0.125, degree)
    ref_out = torch.empty_like(out)
    ref_lse = torch.empty_like(lse)
    ranges = None if m is None else _ops._mask_ranges(m, L, S)
    _lib.check(lib.pt_taylor_attention_fwd(code, degree, _lib.ptr_array(q), len(q), _lib.ptr_array(k), len(k),
                                           _lib.ptr_array(v), len(v), _lib.ptr_array(list(ref_out.unbind(0))),
                                           _lib.ptr_array(list(ref_lse.unbind(0))), bh, L, S, d, int(causal),
                                           None if m is None else m.data_ptr(),
                                           None if ranges is None else ranges.data_ptr(), 0.125,
                                           _lib.stream_of(out.device)), "unsplit")
    torch.cuda.synchronize()
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for k_ in range(degree + 1):
        assert rel_err(out[k_].cpu(), ref_out[k_].cpu()) <= tol
        finite = torch.isfinite(ref_lse[k_])
        assert torch.equal(torch.isfinite(lse[k_]), finite)
        assert rel_err(lse[k_][finite].cpu(), ref_lse[k_][finite].cpu()) <= tol
    want = oracle.attention([c.unsqueeze(0).double() for c in Q], [c.unsqueeze(0).double() for c in K],
                            [c.unsqueeze(0).double() for c in V], attn_mask=mask, is_causal=causal, scale=0.125)
    empty = torch.zeros(L, dtype=torch.bool) if mask is None else ~mask.any(-1)
    want = [torch.where(empty[:, None], torch.zeros_like(w[0]), w[0]) for w in want]
    _check([o for o in out], want, dtype)
