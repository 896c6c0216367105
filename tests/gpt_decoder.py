"""GPT-style decoder of benchmark config 5, as a workload and a parity case (test helper).

``forward`` is written with ordinary torch.nn.functional calls (layer_norm,
linear, scaled_dot_product_attention, gelu, cross_entropy); given PolyTensor
hidden states it runs the whole forward plus loss in Taylor mode through
polytensors_amd's kernels. ``oracle_forward`` is the same network on lists of
CPU coefficients through the oracle (the reference's plain-range rules).

Config 5: 12 layers, d_model 768, 12 heads, seq 1024, batch 8, vocab 32000,
degree 3; weights N(0, 0.02) with zero higher coefficients (ordinary tensors);
the series enters as a complex perturbation direction on the token embeddings.
Pre-LayerNorm blocks with tanh-GELU MLPs (GPT-2 layout) and an untied head.
"""

import torch
import torch.nn.functional as F


def init_params(layers, d, vocab, seq, seed=0, device="cpu", dtype=torch.float32):
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


def embed(params, tokens):
    """Token plus position embeddings (ordinary tensors): the base of the perturbed series."""
    return params["wte"][tokens] + params["wpe"][: tokens.shape[1]]


def forward(params, x, targets, heads, attention=F.scaled_dot_product_attention):
    """Mean next-token cross entropy of hidden states x [B, T, d] (a PolyTensor in Taylor mode).

    ``attention(q, k, v, is_causal=True)`` is replaceable (tests differentiate a math version).
    """
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


def oracle_forward(params, X, targets, heads):
    """``forward`` on coefficient lists through the oracle (CPU, any dtype incl. complex)."""
    import oracle

    def linear(S, w, b=None):
        out = oracle.matmul(S, [w.transpose(0, 1)])
        if b is not None:
            out = [out[0] + b] + out[1:]
        return out

    B, T, d = X[0].shape
    hd = d // heads
    for blk in params["blocks"]:
        H = oracle.layer_norm(X, (d,), weight=[blk["ln1_w"]], bias=[blk["ln1_b"]])
        QKV = linear(H, blk["attn_w"], blk["attn_b"])
        parts = [[c.split(d, dim=-1)[i].reshape(B, T, heads, hd).transpose(1, 2) for c in QKV] for i in range(3)]
        Y = oracle.attention(*parts, is_causal=True)
        Y = [c.transpose(1, 2).reshape(B, T, d) for c in Y]
        X = [a + b for a, b in zip(X, linear(Y, blk["proj_w"], blk["proj_b"]))]
        H = oracle.layer_norm(X, (d,), weight=[blk["ln2_w"]], bias=[blk["ln2_b"]])
        H = oracle.activation(linear(H, blk["fc_w"], blk["fc_b"]), "gelu_tanh")
        X = [a + b for a, b in zip(X, linear(H, blk["fc2_w"], blk["fc2_b"]))]
    X = oracle.layer_norm(X, (d,), weight=[params["lnf_w"]], bias=[params["lnf_b"]])
    logits = linear(X, params["head"])
    return oracle.cross_entropy([c.reshape(B * T, -1) for c in logits], targets.reshape(-1))
