"""Benchmark of the gfx950 truncated-Taylor kernels on benchmark configs 2-5 (shapes in each workload).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload attention|attention_dense|attention_bf16|attention_fp64|attention_window|
                                attention_bf16_additive|attention_bwd|attention_bwd_bf16|attention_bwd_window|
                                matmul|matmul_bf16|
                                matmul_fp64|norm|ce|activation|norm_bwd|ce_bwd|config1|decoder]
                    [--no-cpu-baseline] [--no-components] [--no-ceiling] [--component-seconds S]
                    [--copy-calibration]

One step is one launch of the workload's fused kernel on one batch of synthetic
input already resident in HBM (inputs are generated on the device with a
seeded generator before the timed region). The launch-bound ``config1``
workload (benchmark config 1) times its whole pipeline through the PolyTensor
API per step, and again as the replay of a HIP graph holding one step
(``graph``: ms per replay and the graph's kernel count, the launches per step). The timed region is K back-to-back
steps on the current stream, after at least W warm-up steps lasting at least
0.3 s (the clock ramps up after idle), bracketed by torch.cuda.synchronize() and timed
with HIP events on that stream (``ms_per_step``, the mean); ``ms_median`` is the
median over 21 further steps of each step's own event interval. ``value`` is the
workload's throughput (from the mean) and
``roofline`` compares it to MI355X's published peak (fp32 MFMA 157.3 TFLOP/s,
fp64 MFMA 78.6 TFLOP/s, bf16 MFMA 2.5 PFLOP/s, HBM 8 TB/s). ``cpu_baseline``
times the CPU oracle (the op-for-op restatement of the reference's general
path) on a bounded sample of the same workload on this host: the median of
three timings after one warm-up run. For memory-bound workloads ``roofline.stream_ceiling`` is the measured rate
of a plain streaming read or copy of the same byte count on the same GPU (the
library's probe kernels), a practical HBM ceiling beside the published peak. Rank 0 prints one JSON line.
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ms & TFLOP/s per degree-K Taylor attention fwd; GB/s norm/CE; % roofline"
PEAK_FP32_MFMA = 157.3   # TFLOP/s, dense
PEAK_FP64_MFMA = 78.6    # TFLOP/s, dense
PEAK_BF16_MFMA = 2500.0  # TFLOP/s, dense (bf16 and fp16)
PEAK_HBM = 8000.0        # GB/s


def _gen(seed, device):
    import torch

    return torch.Generator(device=device).manual_seed(seed)


# ---------------------------------------------------------------------------
# The config-5 network: a GPT-style decoder written with ordinary torch.nn.functional
# calls (layer_norm, linear, scaled_dot_product_attention, gelu, cross_entropy). Given
# PolyTensor hidden states it runs the whole forward plus loss in Taylor mode through
# polytensors_amd's kernels. Pre-LayerNorm blocks with tanh-GELU MLPs (GPT-2 layout) and
# an untied head; weights N(0, 0.02) are ordinary tensors (zero higher coefficients).

def gpt_init_params(layers, d, vocab, seq, seed=0, device="cpu", dtype=None):
    import torch

    dtype = torch.float32 if dtype is None else dtype
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=dtype) * 0.02

    def zeros(*shape):
        return torch.zeros(*shape, device=device, dtype=dtype)

    def ones(*shape):
        return torch.ones(*shape, device=device, dtype=dtype)

    blocks = [dict(ln1_w=ones(d), ln1_b=zeros(d), attn_w=normal(3 * d, d), attn_b=zeros(3 * d),
                   proj_w=normal(d, d), proj_b=zeros(d), ln2_w=ones(d), ln2_b=zeros(d),
                   fc_w=normal(4 * d, d), fc_b=zeros(4 * d), fc2_w=normal(d, 4 * d), fc2_b=zeros(d))
              for _ in range(layers)]
    return dict(blocks=blocks, wte=normal(vocab, d), wpe=normal(seq, d), lnf_w=ones(d), lnf_b=zeros(d),
                head=normal(vocab, d))


def gpt_embed(params, tokens):
    """Token plus position embeddings (ordinary tensors): the base of the perturbed series."""
    return params["wte"][tokens] + params["wpe"][: tokens.shape[1]]


def gpt_forward(params, x, targets, heads, attention=None):
    """Mean next-token cross entropy of hidden states x [B, T, d] (a PolyTensor in Taylor mode).

    ``attention(q, k, v, is_causal=True)`` defaults to F.scaled_dot_product_attention
    (tests pass a math version to differentiate).
    """
    import torch.nn.functional as F

    attention = F.scaled_dot_product_attention if attention is None else attention
    B, T, d = x.shape
    hd = d // heads
    for blk in params["blocks"]:
        h = F.layer_norm(x, (d,), blk["ln1_w"], blk["ln1_b"])
        q, k, v = F.linear(h, blk["attn_w"], blk["attn_b"]).split(d, dim=-1)
        q, k, v = (t.reshape(B, T, heads, hd).transpose(1, 2) for t in (q, k, v))
        y = attention(q, k, v, is_causal=True)
        x = x + F.linear(y.transpose(1, 2).reshape(B, T, d), blk["proj_w"], blk["proj_b"])
        h = F.layer_norm(x, (d,), blk["ln2_w"], blk["ln2_b"])
        h = F.gelu(F.linear(h, blk["fc_w"], blk["fc_b"]), approximate="tanh")
        x = x + F.linear(h, blk["fc2_w"], blk["fc2_b"])
    x = F.layer_norm(x, (d,), params["lnf_w"], params["lnf_b"])
    logits = F.linear(x, params["head"])
    return F.cross_entropy(logits.reshape(B * T, -1), targets.reshape(-1))


# ---------------------------------------------------------------------------
# Workloads: each returns a dict with the step closure and its algorithmic work.

def wl_attention(device, dense_orders=False):
    """benchmark config 3: B=4 H=16 L=2048 d=128, K=4, fp32, causal, scale 1/sqrt(128)."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(2, device)

    def series():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        rest = [torch.randn(B * H, L, d, generator=g, device=device) * 0.5 ** k if dense_orders
                else torch.zeros(B * H, L, d, device=device) for k in range(2, K + 1)]
        return [base, direction, *rest]

    q, k, v = series(), series(), series()
    scale = 1 / math.sqrt(d)

    def step():
        return _ops.taylor_attention_fwd(q, k, v, None, True, scale, K)

    pairs = (K + 1) * (K + 2) // 2
    flops = 2 * pairs * 2 * d * B * H * L * (L + 1) / 2    # dense-series count, causal
    nbytes = 4 * (K + 1) * B * H * L * d * 4                 # q, k, v read + out written (fp32)
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_FP32_MFMA,
                bytes=nbytes, kernel="taylor_attention", dtype="fp32",
                workload=f"taylor_attention_fwd B={B} H={H} L={L} d={d} K={K} fp32 causal"
                         + (" dense orders" if dense_orders else " line inputs (orders 2..4 zero)"),
                cpu=lambda: cpu_attention(L, d, K))


def wl_attention_window(device):
    """Config 3's shape with a boolean sliding-window mask (key j admissible for query i iff
    0 <= i - j < 256) instead of causal: the kernel visits only the key blocks in each query
    block's mask range. Work is the dense-series count over the admissible pairs."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K, W = 4, 16, 2048, 128, 4, 256
    g = _gen(9, device)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [base, direction] + [torch.zeros(B * H, L, d, device=device) for _ in range(2, K + 1)]

    q, k, v = line(), line(), line()
    i = torch.arange(L, device=device)
    mask = ((i[:, None] - i[None, :]) >= 0) & ((i[:, None] - i[None, :]) < W)
    scale = 1 / math.sqrt(d)

    def step():
        return _ops.taylor_attention_fwd(q, k, v, mask, False, scale, K)

    pairs = (K + 1) * (K + 2) // 2
    admissible = W * (W + 1) // 2 + (L - W) * W
    flops = 2 * pairs * 2 * d * B * H * admissible
    nbytes = 4 * (K + 1) * B * H * L * d * 4 + L * L
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_FP32_MFMA,
                bytes=nbytes, kernel="taylor_attention_window", dtype="fp32",
                workload=f"taylor_attention_fwd B={B} H={H} L={L} d={d} K={K} fp32 sliding window {W} (bool mask)",
                cpu=lambda: cpu_attention_window(L, d, K, W))


def wl_attention_bwd(device):
    """Attention gradient series on config 3's shape (B=4 H=16 L=2048 d=128, K=4, fp32, causal, line
    inputs) for a random cotangent series G_k ~ N(0,1) 0.5^k: the dQ, dK and dV series."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(8, device)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [base, direction] + [torch.zeros(B * H, L, d, device=device) for _ in range(2, K + 1)]

    q, k, v = line(), line(), line()
    cot = [torch.randn(B * H, L, d, generator=g, device=device) * 0.5 ** o for o in range(K + 1)]
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, None, True, scale, K)

    def step():
        return _ops.taylor_attention_bwd(q, k, v, out, lse, cot, None, True, scale)

    pairs = (K + 1) * (K + 2) // 2
    # five series products over the causal pairs: S (recomputed), dP, dV, dK, dQ
    flops = 5 * pairs * 2 * d * B * H * L * (L + 1) / 2
    nbytes = 8 * (K + 1) * B * H * L * d * 4               # q, k, v, out, G read; dq, dk, dv written
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_FP32_MFMA,
                bytes=nbytes, kernel="taylor_attention_bwd", dtype="fp32",
                workload=f"taylor_attention_bwd B={B} H={H} L={L} d={d} K={K} fp32 causal line inputs",
                cpu=lambda: cpu_attention_bwd(L, d, K))


def wl_attention_bwd_bf16(device):
    """``attention_bwd`` (config 3's shape, K=4, causal, line inputs, cotangent series G_k ~ N(0,1) 0.5^k)
    with every operand stored in bfloat16: the 16-bit backward kernels (bf16 MFMA operands, fp32
    accumulation, lse and Delta in fp32). Work is the same five-product count; the roofline is the
    bf16 MFMA peak."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(8, device)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [x.to(torch.bfloat16) for x in [base, direction] + [torch.zeros_like(base) for _ in range(2, K + 1)]]

    q, k, v = line(), line(), line()
    cot = [(torch.randn(B * H, L, d, generator=g, device=device) * 0.5 ** o).to(torch.bfloat16) for o in range(K + 1)]
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, None, True, scale, K)

    def step():
        return _ops.attention_gradient_series(q, k, v, out, lse, cot, None, True, scale)

    pairs = (K + 1) * (K + 2) // 2
    flops = 5 * pairs * 2 * d * B * H * L * (L + 1) / 2
    nbytes = 8 * (K + 1) * B * H * L * d * 2               # q, k, v, out, G read; dq, dk, dv written
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_MFMA,
                bytes=nbytes, kernel="taylor_attention_bwd_bf16", dtype="bf16 (fp32 accumulate)",
                workload=f"taylor_attention_bwd B={B} H={H} L={L} d={d} K={K} bf16 causal line inputs",
                cpu=lambda: cpu_attention_bwd(L, d, K, heads=2, dtype="bf16"))


def wl_attention_bwd_window(device):
    """The attention gradient series of ``attention_bwd`` with the boolean sliding-window mask of
    ``attention_window`` (0 <= i - j < 256) instead of causal. Work: five series products over
    the admissible pairs."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K, W = 4, 16, 2048, 128, 4, 256
    g = _gen(12, device)

    def line():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [base, direction] + [torch.zeros(B * H, L, d, device=device) for _ in range(2, K + 1)]

    q, k, v = line(), line(), line()
    cot = [torch.randn(B * H, L, d, generator=g, device=device) * 0.5 ** o for o in range(K + 1)]
    i = torch.arange(L, device=device)
    mask = ((i[:, None] - i[None, :]) >= 0) & ((i[:, None] - i[None, :]) < W)
    scale = 1 / math.sqrt(d)
    out, lse = _ops.taylor_attention_fwd(q, k, v, mask, False, scale, K)

    def step():
        return _ops.taylor_attention_bwd(q, k, v, out, lse, cot, mask, False, scale)

    pairs = (K + 1) * (K + 2) // 2
    admissible = W * (W + 1) // 2 + (L - W) * W
    flops = 5 * pairs * 2 * d * B * H * admissible
    nbytes = 8 * (K + 1) * B * H * L * d * 4 + L * L
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_FP32_MFMA,
                bytes=nbytes, kernel="taylor_attention_bwd_window", dtype="fp32",
                workload=f"taylor_attention_bwd B={B} H={H} L={L} d={d} K={K} fp32 sliding window {W} (bool mask)",
                cpu=lambda: cpu_attention_bwd(L, d, K, window=W))


def wl_decoder(device):
    """benchmark config 5: GPT-style decoder forward plus mean cross entropy in Taylor mode. 12 layers,
    d_model 768, 12 heads, seq 1024, batch 8, vocab 32000, K=3; weights N(0, 0.02) (ordinary tensors:
    zero higher coefficients); a complex64 direction N(0,1) + i N(0,1) on the token embeddings."""
    import torch
    from polytensors_amd import PolyTensor

    layers, d, heads, vocab, batch, seq, K = 12, 768, 12, 32000, 8, 1024, 3
    params = gpt_init_params(layers, d, vocab, seq, seed=10, device=device)
    g = _gen(11, device)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g, device=device)
    targets = torch.randint(0, vocab, (batch, seq), generator=g, device=device)
    base = gpt_embed(params, tokens)
    direction = torch.complex(torch.randn(batch, seq, d, generator=g, device=device),
                              torch.randn(batch, seq, d, generator=g, device=device))

    def step():
        with torch.no_grad(), PolyTensor.plain_range():
            x = PolyTensor((base, direction), degree=K)
            return gpt_forward(params, x, targets, heads)

    return dict(step=step, work=batch * seq, unit="tokens/s", bound=None, peak=None, bytes=None,
                kernel="gpt_decoder", dtype="fp32 (complex64 directions)",
                workload=f"gpt_decoder_taylor layers={layers} d={d} heads={heads} seq={seq} batch={batch} "
                         f"vocab={vocab} K={K} complex64 directions, forward + mean CE",
                cpu=lambda: cpu_decoder(layers, d, heads, vocab, K))


def wl_attention_bf16(device):
    """Config 3's shape and inputs (B=4 H=16 L=2048 d=128, K=4, causal, line inputs, scale 1/sqrt(128))
    stored in bfloat16: the 16-bit kernel (bf16 MFMA operands, fp32 accumulation). Work is the same
    dense-series count; the roofline is the bf16 MFMA peak."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(2, device)

    def series():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [x.to(torch.bfloat16) for x in [base, direction] + [torch.zeros_like(base) for _ in range(2, K + 1)]]

    q, k, v = series(), series(), series()
    scale = 1 / math.sqrt(d)

    def step():
        return _ops.taylor_attention_fwd(q, k, v, None, True, scale, K)

    pairs = (K + 1) * (K + 2) // 2
    flops = 2 * pairs * 2 * d * B * H * L * (L + 1) / 2
    nbytes = 4 * (K + 1) * B * H * L * d * 2
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_MFMA,
                bytes=nbytes, kernel="taylor_attention_bf16", dtype="bf16 (fp32 accumulate)",
                workload=f"taylor_attention_fwd B={B} H={H} L={L} d={d} K={K} bf16 causal line inputs",
                cpu=lambda: cpu_attention(L, d, K, heads=8, dtype="bf16"))


def wl_attention_fp64(device):
    """Config 3's shape and inputs (B=4 H=16 L=2048 d=128, K=4, causal, line inputs, scale 1/sqrt(128))
    in float64: the fp64 MFMA kernels (v_mfma_f64_16x16x4_f64, fp64 scores, series and accumulators).
    Work is the same dense-series count; the roofline is the fp64 MFMA peak (78.6 TFLOP/s)."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(2, device)

    def series():
        base = torch.randn(B * H, L, d, generator=g, device=device, dtype=torch.float64) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device, dtype=torch.float64)
        return [base, direction] + [torch.zeros_like(base) for _ in range(2, K + 1)]

    q, k, v = series(), series(), series()
    scale = 1 / math.sqrt(d)

    def step():
        return _ops.taylor_attention_fwd(q, k, v, None, True, scale, K)

    pairs = (K + 1) * (K + 2) // 2
    flops = 2 * pairs * 2 * d * B * H * L * (L + 1) / 2
    nbytes = 4 * (K + 1) * B * H * L * d * 8
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_FP64_MFMA,
                bytes=nbytes, kernel="taylor_attention_fp64", dtype="fp64",
                workload=f"taylor_attention_fwd B={B} H={H} L={L} d={d} K={K} fp64 causal line inputs",
                cpu=lambda: cpu_attention(L, d, K, heads=16, dtype="fp64"))


def wl_attention_bf16_additive(device):
    """Config 3's shape in bfloat16 (B=4 H=16 L=2048 d=128, K=4, line inputs, scale 1/sqrt(128)) with a
    padding-style floating mask instead of causal: batch entry b admits keys j < 2048 - 256 b (mask value
    0) and excludes the rest (-inf), a [B, 1, L, S] bfloat16 mask over the H heads of each entry. The
    16-bit kernels take the mask's float32 values; one step includes the operator's mask preparation
    (float32 values, admissible entries, block ranges). Work is the dense-series count over the
    admissible pairs."""
    import torch
    from polytensors_amd import _ops

    B, H, L, d, K = 4, 16, 2048, 128, 4
    g = _gen(13, device)

    def series():
        base = torch.randn(B * H, L, d, generator=g, device=device) / math.sqrt(d)
        direction = torch.randn(B * H, L, d, generator=g, device=device)
        return [x.to(torch.bfloat16) for x in [base, direction] + [torch.zeros_like(base) for _ in range(2, K + 1)]]

    q, k, v = series(), series(), series()
    lengths = [L - 256 * b for b in range(B)]
    j = torch.arange(L, device=device)
    mask = torch.stack([torch.where(j < n, 0.0, float("-inf")).expand(L, L) for n in lengths]).to(torch.bfloat16)
    scale = 1 / math.sqrt(d)

    def step():
        return _ops.taylor_attention_fwd(q, k, v, mask, False, scale, K, [H, 1, 0])

    pairs = (K + 1) * (K + 2) // 2
    admissible = H * L * sum(lengths)
    flops = 2 * pairs * 2 * d * admissible
    nbytes = 4 * (K + 1) * B * H * L * d * 2 + B * L * L * 2
    return dict(step=step, work=flops, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_MFMA,
                bytes=nbytes, kernel="taylor_attention_bf16_additive", dtype="bf16 (fp32 accumulate)",
                workload=f"taylor_attention_fwd B={B} H={H} L={L} d={d} K={K} bf16 padding float mask "
                         f"(key lengths {lengths}) line inputs",
                cpu=lambda: cpu_attention_padding(L, d, K, lengths[1], heads=4))


def wl_attention_dense(device):
    """Config 3 with dense random orders 2..4 (N(0,1) 0.5^k) instead of a line: the same kernel
    and work count, with no zero input orders."""
    w = wl_attention(device, dense_orders=True)
    w["kernel"] = "taylor_attention_dense"
    return w


def wl_config1(device):
    """benchmark config 1: degree-3 fp64 causal attention on Q, K, V [1,1,128,64] (x + t v with x, v
    ~ N(0,1)/8, seed 0, scale 1/8), logits = out.view(128, 64) @ W with W ~ N(0,1)/8 [64, 256], mean
    cross entropy over 256 classes. One step is that whole pipeline through the PolyTensor API
    (F.scaled_dot_product_attention, @, F.cross_entropy): launch-bound, so the step is also captured
    in a HIP graph and replayed (``graph``)."""
    import torch
    import torch.nn.functional as F
    from polytensors_amd import PolyTensor

    K, L, d, C = 3, 128, 64, 256
    g = torch.Generator().manual_seed(0)   # the seeded CPU inputs of the parity test, copied to the device
    lines = [(torch.randn(1, 1, L, d, generator=g, dtype=torch.float64) / 8,
              torch.randn(1, 1, L, d, generator=g, dtype=torch.float64) / 8) for _ in range(3)]
    W = (torch.randn(d, C, generator=g, dtype=torch.float64) / 8).to(device)
    y = torch.randint(0, C, (L,), generator=g).to(device)
    q, k, v = (PolyTensor((x.to(device), u.to(device)), degree=K) for x, u in lines)

    def step():
        with torch.no_grad(), PolyTensor.plain_range():
            out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            logits = out.reshape(L, d) @ W
            return F.cross_entropy(logits, y)

    pairs = (K + 1) * (K + 2) // 2
    flops = 2 * pairs * 2 * d * L * (L + 1) / 2 + 2 * (K + 1) * L * d * C   # attention + series @ plain W
    return dict(step=step, work=None, unit="ms", bound=None, peak=None, bytes=None, graph=True,
                flops=flops, kernel="config1", dtype="fp64",
                workload=f"config1: taylor attention [1,1,{L},{d}] K={K} fp64 causal -> @ W [{d},{C}] -> mean CE",
                cpu=lambda: cpu_config1(L, d, C, K))


def wl_matmul(device):
    """benchmark config 2: A, B [5, 4096, 4096] fp32 (K=4), coefficient k scaled by 0.5^k."""
    import torch
    from polytensors_amd import _ops

    K, n = 4, 4096
    g = _gen(1, device)
    a = [torch.randn(1, n, n, generator=g, device=device) * 0.5 ** k for k in range(K + 1)]
    b = [torch.randn(1, n, n, generator=g, device=device) * 0.5 ** k for k in range(K + 1)]

    def step():
        return _ops.cauchy_matmul(a, b, K, False)

    pairs = (K + 1) * (K + 2) // 2
    return dict(step=step, work=2 * pairs * n ** 3, unit="TFLOP/s", bound="mfma", peak=PEAK_FP32_MFMA,
                bytes=3 * (K + 1) * n * n * 4, kernel="cauchy_matmul", dtype="fp32",
                workload=f"cauchy_matmul [{K + 1},{n},{n}] x [{K + 1},{n},{n}] fp32",
                cpu=lambda: cpu_matmul(n, K))


def wl_matmul_bf16(device):
    """Config 2's shape and inputs ([5, 4096, 4096] x [5, 4096, 4096], K=4, coefficient k scaled by
    0.5^k) stored in bfloat16: the 16-bit kernel (bf16 MFMA operands, fp32 accumulation, one rounding
    per output element). The roofline is the bf16 MFMA peak."""
    import torch
    from polytensors_amd import _ops

    K, n = 4, 4096
    g = _gen(1, device)
    a = [(torch.randn(1, n, n, generator=g, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    b = [(torch.randn(1, n, n, generator=g, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]

    def step():
        return _ops.cauchy_matmul(a, b, K, False)

    pairs = (K + 1) * (K + 2) // 2
    return dict(step=step, work=2 * pairs * n ** 3, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_MFMA,
                bytes=3 * (K + 1) * n * n * 2, kernel="cauchy_matmul_bf16", dtype="bf16 (fp32 accumulate)",
                workload=f"cauchy_matmul [{K + 1},{n},{n}] x [{K + 1},{n},{n}] bf16",
                cpu=lambda: cpu_matmul(n, K, dtype="bf16"))


def wl_matmul_fp64(device):
    """Config 2's shape and inputs ([5, 4096, 4096] x [5, 4096, 4096], K=4, coefficient k scaled by
    0.5^k) in float64: the fp64 MFMA kernel (v_mfma_f64_16x16x4_f64, fp64 accumulation). The roofline
    is the fp64 MFMA peak (78.6 TFLOP/s)."""
    import torch
    from polytensors_amd import _ops

    K, n = 4, 4096
    g = _gen(1, device)
    a = [torch.randn(1, n, n, generator=g, device=device, dtype=torch.float64) * 0.5 ** k for k in range(K + 1)]
    b = [torch.randn(1, n, n, generator=g, device=device, dtype=torch.float64) * 0.5 ** k for k in range(K + 1)]

    def step():
        return _ops.cauchy_matmul(a, b, K, False)

    pairs = (K + 1) * (K + 2) // 2
    return dict(step=step, work=2 * pairs * n ** 3, unit="TFLOP/s", bound="mfma", peak=PEAK_FP64_MFMA,
                bytes=3 * (K + 1) * n * n * 8, kernel="cauchy_matmul_fp64", dtype="fp64",
                workload=f"cauchy_matmul [{K + 1},{n},{n}] x [{K + 1},{n},{n}] fp64",
                cpu=lambda: cpu_matmul(n, K, dtype="fp64"))


def wl_norm(device):
    """benchmark config 4a: RMSNorm series x [5, 8192, 4096] bf16, eps 1e-6, weight 1+0.02 N(0,1)."""
    import torch
    from polytensors_amd import _ops

    K, rows, n = 4, 8192, 4096
    g = _gen(3, device)
    x = [(torch.randn(rows, n, generator=g, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    w = (1 + 0.02 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

    def step():
        return _ops.norm_series(x, [w], [], n, 1e-6, False)

    nbytes = 2 * (K + 1) * rows * n * 2 + n * 2
    return dict(step=step, work=nbytes, unit="GB/s", bound="hbm", pattern="copy", streams=(K + 1, K + 1), peak=PEAK_HBM,
                bytes=nbytes, kernel="norm_series", dtype="bf16",
                workload=f"rms_norm_series [{K + 1},{rows},{n}] bf16 weight eps=1e-6",
                cpu=lambda: cpu_norm(rows, n, K))


def wl_ce(device):
    """benchmark config 4b: logits [5, 8192, 32000] fp32, base N(0,2^2), order k N(0,1) 0.5^k, mean."""
    import torch
    from polytensors_amd import _ops

    K, rows, classes = 4, 8192, 32000
    g = _gen(4, device)
    z = [torch.randn(rows, classes, generator=g, device=device) * (2.0 if k == 0 else 0.5 ** k)
         for k in range(K + 1)]
    y = torch.randint(0, classes, (rows,), generator=g, device=device)

    def step():
        return _ops.cross_entropy_series(z, y, -100, 1, 0.0)

    nbytes = (K + 1) * rows * classes * 4 + rows * 8 + (K + 1) * rows * 4
    return dict(step=step, work=nbytes, unit="GB/s", bound="hbm", pattern="read", peak=PEAK_HBM,
                bytes=nbytes, kernel="cross_entropy_series", dtype="fp32",
                workload=f"cross_entropy_series [{K + 1},{rows},{classes}] fp32 mean",
                cpu=lambda: cpu_ce(rows, classes, K))


def wl_activation(device):
    """Activation series: GELU (erf form) of a degree-4 bf16 [8192, 4096] series (config 4a's shape)."""
    import torch
    from polytensors_amd import _ops

    K, rows, n = 4, 8192, 4096
    g = _gen(5, device)
    x = [(torch.randn(rows, n, generator=g, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]

    def step():
        return _ops.activation_series(x, "gelu")

    nbytes = 2 * (K + 1) * rows * n * 2
    return dict(step=step, work=nbytes, unit="GB/s", bound="hbm", pattern="copy", streams=(K + 1, K + 1), peak=PEAK_HBM,
                bytes=nbytes, kernel="activation_series", dtype="bf16",
                workload=f"gelu_series [{K + 1},{rows},{n}] bf16",
                cpu=lambda: cpu_activation(rows, n, K))


def wl_norm_bwd(device):
    """RMSNorm gradient series on config 4a's shape: x, g [5, 8192, 4096] bf16, eps 1e-6."""
    import torch
    from polytensors_amd import _ops

    K, rows, n = 4, 8192, 4096
    gen = _gen(6, device)
    x = [(torch.randn(rows, n, generator=gen, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    g = [(torch.randn(rows, n, generator=gen, device=device) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]

    def step():
        return _ops.norm_series_backward(x, g, n, 1e-6, False)

    nbytes = 3 * (K + 1) * rows * n * 2
    return dict(step=step, work=nbytes, unit="GB/s", bound="hbm", pattern="copy", streams=(2 * (K + 1), K + 1), peak=PEAK_HBM,
                bytes=nbytes, kernel="norm_series_bwd", dtype="bf16",
                workload=f"rms_norm_series_backward [{K + 1},{rows},{n}] bf16",
                cpu=lambda: cpu_norm_bwd(rows, n, K))


def wl_ce_bwd(device):
    """Cross-entropy gradient series on config 4b's shape: logits [5, 8192, 32000] fp32, per-row cotangents."""
    import torch
    from polytensors_amd import _ops

    K, rows, classes = 4, 8192, 32000
    gen = _gen(7, device)
    z = [torch.randn(rows, classes, generator=gen, device=device) * (2.0 if k == 0 else 0.5 ** k)
         for k in range(K + 1)]
    y = torch.randint(0, classes, (rows,), generator=gen, device=device)
    _, lse = _ops.cross_entropy_series(z, y, -100, 0, 0.0)
    cot = [torch.randn(rows, generator=gen, device=device) * 0.5 ** k for k in range(K + 1)]

    def step():
        return _ops.cross_entropy_series_backward(z, y, -100, 0.0, lse, cot)

    nbytes = 2 * (K + 1) * rows * classes * 4 + rows * 8 + 2 * (K + 1) * rows * 4
    return dict(step=step, work=nbytes, unit="GB/s", bound="hbm", pattern="copy", streams=(K + 1, K + 1), peak=PEAK_HBM,
                bytes=nbytes, kernel="cross_entropy_series_bwd", dtype="fp32",
                workload=f"cross_entropy_series_backward [{K + 1},{rows},{classes}] fp32",
                cpu=lambda: cpu_ce_bwd(rows, classes, K))


WORKLOADS = {"attention": wl_attention, "matmul": wl_matmul, "matmul_bf16": wl_matmul_bf16,
             "matmul_fp64": wl_matmul_fp64, "attention_fp64": wl_attention_fp64, "norm": wl_norm,
             "ce": wl_ce,
             "activation": wl_activation, "norm_bwd": wl_norm_bwd, "ce_bwd": wl_ce_bwd,
             "attention_bwd": wl_attention_bwd, "attention_bwd_bf16": wl_attention_bwd_bf16,
             "attention_window": wl_attention_window,
             "attention_bwd_window": wl_attention_bwd_window,
             "attention_dense": wl_attention_dense, "attention_bf16": wl_attention_bf16,
             "attention_bf16_additive": wl_attention_bf16_additive, "config1": wl_config1,
             "decoder": wl_decoder}


# ---------------------------------------------------------------------------
# CPU baseline: the oracle (the reference's general path restated op for op) on a bounded sample.

def _cpu_time(fn, reps=3):
    fn()   # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_attention(L, d, K, heads=64, dtype=None):
    import torch
    import oracle

    g = torch.Generator().manual_seed(2)
    q, k, v = ([torch.randn(1, 1, L, d, generator=g) * (0.5 ** o) for o in range(K + 1)] for _ in range(3))
    if dtype in ("bf16", "fp64"):   # the reference's general path on bf16 / fp64 coefficients
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float64
        q, k, v = ([c.to(tdt) for c in s] for s in (q, k, v))

    def all_heads():   # one head at a time (the L x L series of all heads would not fit in host memory)
        for _ in range(heads):
            oracle.attention(q, k, v, is_causal=True)

    t = _cpu_time(all_heads, reps=3)
    flops = heads * 2 * ((K + 1) * (K + 2) // 2) * 2 * d * L * (L + 1) / 2
    return dict(value=flops / t / 1e12, unit="TFLOP/s",
                sample=f"{heads} of 64 (b,h) heads one at a time, L={L} d={d} K={K} {dtype or 'fp32'} causal",
                seconds=t)


def cpu_attention_window(L, d, K, W, heads=16):
    import torch
    import oracle

    g = torch.Generator().manual_seed(9)
    q, k, v = ([torch.randn(1, 1, L, d, generator=g) * (0.5 ** o) for o in range(K + 1)] for _ in range(3))
    i = torch.arange(L)
    mask = ((i[:, None] - i[None, :]) >= 0) & ((i[:, None] - i[None, :]) < W)

    def some_heads():
        for _ in range(heads):
            oracle.attention(q, k, v, attn_mask=mask)

    t = _cpu_time(some_heads, reps=3)
    flops = heads * 2 * ((K + 1) * (K + 2) // 2) * 2 * d * (W * (W + 1) // 2 + (L - W) * W)
    return dict(value=flops / t / 1e12, unit="TFLOP/s",
                sample=f"{heads} of 64 (b,h) heads one at a time, L={L} d={d} K={K} fp32 window {W}", seconds=t)


def cpu_attention_padding(L, d, K, length, heads=4):
    """The reference's general path on bf16 coefficients with an additive padding mask (keys past
    ``length`` at -inf), one head at a time."""
    import torch
    import oracle

    g = torch.Generator().manual_seed(13)
    q, k, v = ([(torch.randn(1, 1, L, d, generator=g) * (0.5 ** o)).to(torch.bfloat16) for o in range(K + 1)]
               for _ in range(3))
    mask = torch.where(torch.arange(L) < length, 0.0, float("-inf")).expand(L, L).to(torch.bfloat16)

    def some_heads():
        for _ in range(heads):
            oracle.attention(q, k, v, attn_mask=mask)

    t = _cpu_time(some_heads, reps=3)
    flops = heads * 2 * ((K + 1) * (K + 2) // 2) * 2 * d * L * length
    return dict(value=flops / t / 1e12, unit="TFLOP/s",
                sample=f"{heads} heads one at a time, L={L} d={d} K={K} bf16, padding mask of {length} keys",
                seconds=t)


def cpu_attention_bwd(L, d, K, heads=16, window=None, dtype=None):
    import torch
    import oracle

    g = torch.Generator().manual_seed(8)
    q, k, v, cot = ([torch.randn(1, 1, L, d, generator=g) * (0.5 ** o) for o in range(K + 1)] for _ in range(4))
    if dtype == "bf16":   # the reference's general path on bf16 coefficients (torch's CPU bf16 ops)
        q, k, v, cot = ([c.to(torch.bfloat16) for c in s] for s in (q, k, v, cot))
    mask = None
    if window is not None:
        i = torch.arange(L)
        mask = ((i[:, None] - i[None, :]) >= 0) & ((i[:, None] - i[None, :]) < window)

    def some_heads():
        for _ in range(heads):
            oracle.attention_backward(q, k, v, cot, attn_mask=mask, is_causal=mask is None)

    t = _cpu_time(some_heads, reps=3)
    pairs = L * (L + 1) / 2 if window is None else window * (window + 1) // 2 + (L - window) * window
    flops = heads * 5 * ((K + 1) * (K + 2) // 2) * 2 * d * pairs
    what = "causal" if window is None else f"window {window}"
    return dict(value=flops / t / 1e12, unit="TFLOP/s",
                sample=f"{heads} of 64 (b,h) heads one at a time, L={L} d={d} K={K} {dtype or 'fp32'} {what}",
                seconds=t)


def cpu_decoder(layers, d, heads, vocab, K, seq=64):
    import torch
    import oracle

    params = gpt_init_params(layers, d, vocab, seq, seed=10)
    g = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, vocab, (1, seq), generator=g)
    targets = torch.randint(0, vocab, (1, seq), generator=g)
    base = gpt_embed(params, tokens)
    direction = torch.complex(torch.randn(1, seq, d, generator=g), torch.randn(1, seq, d, generator=g))
    X = [base, direction] + [torch.zeros(1, seq, d, dtype=torch.complex64) for _ in range(K - 1)]
    t = _cpu_time(lambda: oracle.gpt_forward(params, X, targets, heads), reps=3)
    return dict(value=seq / t, unit="tokens/s", seconds=t,
                sample=f"one sequence of {seq} tokens (attention cost grows with seq), full width, K={K} complex64")


def cpu_config1(L, d, C, K):
    import torch
    import oracle
    from oracle import paths

    g = torch.Generator().manual_seed(0)
    lines = [(torch.randn(1, 1, L, d, generator=g, dtype=torch.float64) / 8,
              torch.randn(1, 1, L, d, generator=g, dtype=torch.float64) / 8) for _ in range(3)]
    W = torch.randn(d, C, generator=g, dtype=torch.float64) / 8
    y = torch.randint(0, C, (L,), generator=g)
    Q, Kk, V = (paths.lift([x, u], K) for x, u in lines)

    def pipeline():
        out = oracle.attention(Q, Kk, V, is_causal=True)
        logits = oracle.matmul([o.reshape(L, d) for o in out], [W])
        return oracle.cross_entropy(logits, y)

    reps = 20
    t = _cpu_time(lambda: [pipeline() for _ in range(reps)], reps=3) / reps
    return dict(value=t * 1e3, unit="ms", sample=f"the whole config-1 pipeline, {reps} runs per timing", seconds=t * reps)


def cpu_matmul(n, K, dtype="fp32"):
    import torch
    import oracle

    rows = n // 4
    tdt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp64": torch.float64}[dtype]
    g = torch.Generator().manual_seed(1)
    a = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(tdt) for k in range(K + 1)]
    b = [(torch.randn(n, n, generator=g) * 0.5 ** k).to(tdt) for k in range(K + 1)]
    t = _cpu_time(lambda: oracle.matmul(a, b), reps=3)
    flops = 2 * ((K + 1) * (K + 2) // 2) * rows * n * n
    return dict(value=flops / t / 1e12, unit="TFLOP/s", sample=f"{rows} of {n} rows of A, K={K} {dtype}",
                seconds=t)


def cpu_norm(rows, n, K):
    import torch
    import oracle

    g = torch.Generator().manual_seed(3)
    x = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    w = [(1 + 0.02 * torch.randn(n, generator=g)).to(torch.bfloat16)]
    t = _cpu_time(lambda: oracle.rms_norm(x, (n,), weight=w, eps=1e-6))
    nbytes = 2 * (K + 1) * rows * n * 2
    return dict(value=nbytes / t / 1e9, unit="GB/s", sample=f"all {rows} rows, n={n} K={K} bf16", seconds=t)


def cpu_ce(rows, classes, K):
    import torch
    import oracle

    rows = rows // 8
    g = torch.Generator().manual_seed(4)
    z = [torch.randn(rows, classes, generator=g) * (2.0 if k == 0 else 0.5 ** k) for k in range(K + 1)]
    y = torch.randint(0, classes, (rows,), generator=g)
    t = _cpu_time(lambda: oracle.cross_entropy(z, y))
    nbytes = (K + 1) * rows * classes * 4
    return dict(value=nbytes / t / 1e9, unit="GB/s", sample=f"{rows} of 8192 rows, C={classes} K={K} fp32", seconds=t)


def cpu_activation(rows, n, K):
    import torch
    import oracle

    g = torch.Generator().manual_seed(5)
    x = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    t = _cpu_time(lambda: oracle.activation(x, "gelu"))
    nbytes = 2 * (K + 1) * rows * n * 2
    return dict(value=nbytes / t / 1e9, unit="GB/s", sample=f"all {rows} rows, n={n} K={K} bf16", seconds=t)


def cpu_norm_bwd(rows, n, K):
    import torch
    import oracle

    g = torch.Generator().manual_seed(6)
    x = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    gr = [(torch.randn(rows, n, generator=g) * 0.5 ** k).to(torch.bfloat16) for k in range(K + 1)]
    t = _cpu_time(lambda: oracle.rms_norm_backward(x, gr, (n,), eps=1e-6))
    nbytes = 3 * (K + 1) * rows * n * 2
    return dict(value=nbytes / t / 1e9, unit="GB/s", sample=f"all {rows} rows, n={n} K={K} bf16", seconds=t)


def cpu_ce_bwd(rows, classes, K):
    import torch
    import oracle

    rows = rows // 8
    g = torch.Generator().manual_seed(7)
    z = [torch.randn(rows, classes, generator=g) * (2.0 if k == 0 else 0.5 ** k) for k in range(K + 1)]
    y = torch.randint(0, classes, (rows,), generator=g)
    cot = [torch.randn(rows, generator=g) * 0.5 ** k for k in range(K + 1)]
    t = _cpu_time(lambda: oracle.cross_entropy_backward(z, y, cot))
    nbytes = 2 * (K + 1) * rows * classes * 4
    return dict(value=nbytes / t / 1e9, unit="GB/s", sample=f"{rows} of 8192 rows, C={classes} K={K} fp32", seconds=t)


# ---------------------------------------------------------------------------

def profiled_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of this workload, if any."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_bench.txt")
    try:
        for line in open(path):
            if line.startswith("HBM traffic per launch"):
                return float(line.rsplit("=", 1)[1].split()[0]) * 1e6
    except OSError:
        pass
    return None


def _progress(message):
    """One line per finished measurement on stderr (the JSON line alone goes to stdout)."""
    print(f"[bench] {message}", file=sys.stderr, flush=True)


SETTLE_SECONDS = 0.3   # warm-up lasts at least this long: the GPU clock ramps up over ~30 ms of work
_warmup_done = [0]     # warm-up steps the last time_steps call ran (profile summaries index the trace by it)


def time_steps(step, steps, warmup, settle=SETTLE_SECONDS):
    """Mean ms per step over ``steps`` back-to-back steps, after ``warmup`` untimed steps (continued
    until ``settle`` seconds of warm-up have passed: the first launches after an idle period run at
    lower clocks, up to 35% slower for a 1.4 ms kernel)."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t0 < settle:
        step()
        done += 1
        if done % 4 == 0:   # bounds how far the host runs ahead of the GPU
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    _warmup_done[0] = done
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_median(step, reps=21):
    """Median over ``reps`` steps of each step's own HIP-event interval (events recorded between
    consecutive steps on the current stream, launched back to back)."""
    import torch

    events = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    events[0].record()
    for i in range(reps):
        step()
        events[i + 1].record()
    torch.cuda.synchronize()
    times = sorted(events[i].elapsed_time(events[i + 1]) for i in range(reps))
    return times[reps // 2]


def cpu_model():
    """The host CPU's model name (as lscpu reports it), for the CPU baseline."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def stream_ceiling(device, pattern, nbytes, steps=10, warmup=2, streams=None):
    """Measured HBM ceiling for a workload moving ``nbytes`` algorithmic bytes.

    pattern "read": pt_stream_read over nbytes; "copy": pt_stream_copy of nbytes / 2
    each way (read + write). The probes use the series kernels' access pattern
    (16-byte non-temporal accesses); the best over grid sizes and two layouts (a
    contiguous chunk per block, a grid-stride walk) is reported, beside torch's own
    copy for "copy".

    ``streams`` = (sources, destinations): the same bytes over that many separate
    buffers with the series kernels' own pattern (one 16-byte vector of every order per
    thread, pt_stream_series), reported as ``series_rate``: the ceiling of the
    kernels' multi-order access pattern, the median of five timings.
    """
    import torch
    from polytensors_amd import _lib

    lib = _lib.load()
    stream = _lib.stream_of(device)
    each = (nbytes // 2 if pattern == "copy" else nbytes) // 16 * 16
    src = torch.empty(each // 4, device=device).fill_(1.0)
    dst = torch.empty_like(src) if pattern == "copy" else None
    out = torch.empty(65536, dtype=torch.int32, device=device)
    moved = 2 * each if pattern == "copy" else each
    best, best_how = 0.0, ""
    for chunked in (1, 0):
        for blocks in (1024, 2048, 4096, 8192, 16384):
            if pattern == "copy":
                def fn(blocks=blocks, chunked=chunked):
                    _lib.check(lib.pt_stream_copy(src.data_ptr(), dst.data_ptr(), each, blocks, chunked, stream),
                               "stream copy")
            else:
                def fn(blocks=blocks, chunked=chunked):
                    _lib.check(lib.pt_stream_read(src.data_ptr(), each, blocks, chunked, out.data_ptr(), stream),
                               "stream read")
            reps = max(steps, math.ceil(50.0 / max(time_steps(fn, 2, warmup, settle=0.0), 1e-3)))   # >= 50 ms
            rate = moved / (time_steps(fn, reps, 1, settle=0.0) * 1e-3) / 1e9
            if rate > best:
                best, best_how = rate, f"{blocks} blocks of 256, {'chunked' if chunked else 'grid-stride'}"
    entry = {"pattern": pattern, "bytes": moved, "rate": round(best, 1), "unit": "GB/s",
             "how": f"pt_stream_{pattern} ({best_how}; best of a sweep of grids and layouts)"}
    if pattern == "copy":
        reps = max(steps, math.ceil(50.0 / max(time_steps(lambda: dst.copy_(src), 2, warmup, settle=0.0), 1e-3)))
        entry["torch_copy"] = round(moved / (time_steps(lambda: dst.copy_(src), reps, 1, settle=0.0) * 1e-3) / 1e9, 1)
    del src, dst, out
    torch.cuda.empty_cache()
    if streams is not None:
        ns, nd = streams
        each = nbytes // (ns + nd) // 16 * 16
        srcs = [torch.empty(each // 4, device=device).fill_(1.0) for _ in range(ns)]
        dsts = [torch.empty(each // 4, device=device) for _ in range(nd)]
        blk = torch.empty(max(1, lib.pt_stream_series_blocks(each)), dtype=torch.int32, device=device)
        sp, dp = _lib.ptr_array(srcs), _lib.ptr_array(dsts) if nd else None

        def fn():
            _lib.check(lib.pt_stream_series(sp, ns, dp, nd, each, blk.data_ptr(), stream), "stream series")

        reps = max(steps, math.ceil(50.0 / max(time_steps(fn, 2, warmup, settle=0.0), 1e-3)))
        rates = sorted(each * (ns + nd) / (time_steps(fn, reps, 1, settle=0.0) * 1e-3) / 1e9 for _ in range(5))
        entry["series_rate"] = round(rates[2], 1)
        entry["series_how"] = (f"pt_stream_series: {ns} source and {nd} destination buffers of {each} bytes, "
                               "one 16-byte vector of each per thread (median of 5)")
        del srcs, dsts, blk
        torch.cuda.empty_cache()
    return entry


def graph_nodes(graph):
    """Node counts by type of a captured HIP graph (hipGraphGetNodes / hipGraphNodeGetType on the
    runtime torch loaded): {"kernel": n, "memset": n, ...}."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")
    raw = ctypes.c_void_p(graph.raw_cuda_graph())
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(raw, None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * max(1, count.value))()
    if hip.hipGraphGetNodes(raw, nodes, ctypes.byref(count)) != 0:
        return None
    names = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty"}
    kinds = {}
    for i in range(count.value):
        kind = ctypes.c_int(-1)
        hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kind))
        name = names.get(kind.value, f"type{kind.value}")
        kinds[name] = kinds.get(name, 0) + 1
    return kinds


def graph_replay(step, steps, warmup):
    """The step captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed: ms per replay,
    the graph's node counts, and whether the last replay reproduces the eager result bit for bit.
    A graph holding memset nodes is not timed (such nodes have given wrong results on replay)."""
    import torch

    eager = step()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        captured = step()
    nodes = graph_nodes(graph)
    graph.instantiate()
    if nodes is None or nodes.get("memset", 0):
        return {"nodes": nodes, "ms": None, "matches_eager": None}
    ms = time_steps(graph.replay, steps, warmup)
    torch.cuda.synchronize()
    same = all(torch.equal(a, b) for a, b in zip(eager.coeffs, captured.coeffs))
    return {"nodes": nodes, "ms": ms, "matches_eager": same, "warmup_done": _warmup_done[0]}


def measure(name, device, steps, warmup, min_seconds=0.0):
    """Time ``steps`` steps (raised so the timed region lasts at least ``min_seconds``)."""
    w = WORKLOADS[name](device)
    if min_seconds > 0:
        estimate = time_steps(w["step"], 3, warmup)
        steps = max(steps, math.ceil(min_seconds * 1e3 / max(estimate, 1e-3)))
        warmup = 1
    ms = time_steps(w["step"], steps, warmup)   # warm-up of at least SETTLE_SECONDS
    w["steps"], w["warmup_done"] = steps, _warmup_done[0]
    w["ms_median"] = time_median(w["step"])
    if w["unit"] == "ms":   # launch-bound workloads report time per step
        achieved = ms
    else:
        scale = {"TFLOP/s": 1e12, "GB/s": 1e9}.get(w["unit"], 1.0)
        achieved = w["work"] / (ms * 1e-3) / scale
    w.update(ms=ms, achieved=achieved)
    if w.get("graph"):
        w["graph_result"] = graph_replay(w["step"], steps, warmup)
    return w


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--workload", default="attention", choices=sorted(WORKLOADS))
    parser.add_argument("--no-components", action="store_true", help="skip timing the other three kernels")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-ceiling", action="store_true", help="skip the measured HBM ceilings (profiling runs)")
    parser.add_argument("--component-seconds", type=float, default=0.2,
                        help="minimum timed duration of each component kernel (0: steps/2 steps)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run a plain 1 GiB device copy (scales rocprof FETCH_SIZE/WRITE_SIZE)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the Taylor kernels are single-GPU "
              "in this build (each path shards over heads, rows or output tiles; that sharding is not built)", file=sys.stderr)
        sys.exit(2)

    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    device = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(1 << 28, device=device)          # 1 GiB of float32
        dst = torch.empty_like(src)
        ms = time_steps(lambda: dst.copy_(src), max(1, args.steps), args.warmup)
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "ms": round(ms, 4),
                          "GB/s": round(2 * src.numel() * 4 / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return
    w = measure(args.workload, device, args.steps, args.warmup)
    _progress(f"{args.workload}: {w['ms']:.4f} ms per step; {w['warmup_done']} warm-up steps"
              + (f", graph warm-up {w['graph_result'].get('warmup_done')} replays" if "graph_result" in w else "")
              + f"; work per step {w.get('work') or 0:.6e}, algorithmic HBM bytes {w.get('bytes') or 0:.6e}")
    line = {
        "metric": METRIC,
        "value": round(w["achieved"], 3),
        "unit": w["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(w["ms"], 4),
        "ms_median": round(w["ms_median"], 4),
        "higher_is_better": w["unit"] != "ms",
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic (seeded torch.randn on device)",
        "config": {"workload": w["workload"], "parallelism": "none (1 GPU)"},
        "roofline": {"bound": w["bound"], "achieved": round(w["achieved"], 3), "peak": w["peak"],
                     "unit": w["unit"], "frac": round(w["achieved"] / w["peak"], 4) if w["peak"] else None,
                     "traffic": profiled_traffic(w["kernel"]) if w["peak"] else None},
    }
    if w["bound"] == "hbm" and not args.no_ceiling:
        ceil = stream_ceiling(device, w["pattern"], w["bytes"], streams=w.get("streams"))
        ceil["frac"] = round(w["achieved"] / ceil["rate"], 4)
        if "series_rate" in ceil:
            ceil["series_frac"] = round(w["achieved"] / ceil["series_rate"], 4)
        line["roofline"]["stream_ceiling"] = ceil
    if "graph_result" in w:
        gr = w["graph_result"]
        line["graph"] = {"ms": round(gr["ms"], 4) if gr["ms"] is not None else None, "nodes": gr["nodes"],
                         "matches_eager": gr["matches_eager"], "launches_per_step": (gr["nodes"] or {}).get("kernel")}
    cpu_samplers = {}
    if not args.no_components:
        comps = {}
        for name in sorted(WORKLOADS):
            if name == args.workload:
                continue
            c = measure(name, device, max(3, args.steps // 2), 2, min_seconds=args.component_seconds)
            comps[name] = {"workload": c["workload"], "ms": round(c["ms"], 4), "ms_median": round(c["ms_median"], 4),
                           "steps": c["steps"],
                           "achieved": round(c["achieved"], 3), "unit": c["unit"],
                           "frac": round(c["achieved"] / c["peak"], 4) if c["peak"] else None,
                           "traffic": profiled_traffic(c["kernel"]) if c["peak"] else None}
            if "graph_result" in c:
                gr = c["graph_result"]
                comps[name]["graph"] = {"ms": round(gr["ms"], 4) if gr["ms"] is not None else None,
                                        "nodes": gr["nodes"], "matches_eager": gr["matches_eager"],
                                        "launches_per_step": (gr["nodes"] or {}).get("kernel")}
            if c["bound"] == "hbm" and not args.no_ceiling:
                ceil = stream_ceiling(device, c["pattern"], c["bytes"], streams=c.get("streams"))
                ceil["frac"] = round(c["achieved"] / ceil["rate"], 4)
                if "series_rate" in ceil:
                    ceil["series_frac"] = round(c["achieved"] / ceil["series_rate"], 4)
                comps[name]["stream_ceiling"] = ceil
            cpu_samplers[name] = c["cpu"]
            _progress(f"component {name}: {c['ms']:.4f} ms ({c['achieved']:.1f} {c['unit']})")
            del c
            torch.cuda.empty_cache()
        line["components"] = comps
    if not args.no_cpu_baseline:
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)

        model = cpu_model()

        def cpu_entry(sampler):
            cpu = sampler()
            return {"value": round(cpu["value"], 6), "unit": cpu["unit"], "cores": torch.get_num_threads(),
                    "kind": "port", "sample": cpu["sample"], "seconds": round(cpu["seconds"], 3),
                    "timing": "median of 3 timings after one warm-up run", "cpu_model": model}

        line["cpu_baseline"] = cpu_entry(w["cpu"])
        _progress(f"cpu baseline {args.workload}: {line['cpu_baseline']['value']} {line['cpu_baseline']['unit']}")
        for name, sampler in cpu_samplers.items():   # the reference's CPU path beside each component
            line["components"][name]["cpu_baseline"] = cpu_entry(sampler)
            _progress(f"cpu baseline {name}: {line['components'][name]['cpu_baseline']['value']}")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
