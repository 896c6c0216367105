"""The config-5 GPT-style decoder on coefficient lists (CPU, any dtype incl. complex).

The network of ``bench.gpt_forward`` (pre-LayerNorm blocks, tanh-GELU MLPs, an
untied head, mean cross entropy) evaluated through this package's restatements
of the reference's plain-range rules: the Cauchy matmul of linear layers
(/root/reference/src/polytensors/_plain.py:118-128 via _range_ops.py:160-176),
the LayerNorm composite (_range_ops.py:133-149,178-193, _series.py:83-96), the
attention decomposition (_decompositions.py:28-43), the tanh-GELU series and the
cross-entropy series (_dispatch.py:537-543). Test infrastructure: the checker of
the decoder tests and the timed CPU baseline of the decoder bench workload.
"""

from .activations import activation
from .paths import attention, cross_entropy, layer_norm, matmul


def gpt_forward(params, X, targets, heads):
    """Mean cross-entropy series of hidden-state coefficients X (a list of [B, T, d] tensors)."""

    def linear(S, w, b=None):
        out = matmul(S, [w.transpose(0, 1)])
        if b is not None:
            out = [out[0] + b] + out[1:]
        return out

    B, T, d = X[0].shape
    hd = d // heads
    for blk in params["blocks"]:
        H = layer_norm(X, (d,), weight=[blk["ln1_w"]], bias=[blk["ln1_b"]])
        QKV = linear(H, blk["attn_w"], blk["attn_b"])
        parts = [[c.split(d, dim=-1)[i].reshape(B, T, heads, hd).transpose(1, 2) for c in QKV] for i in range(3)]
        Y = attention(*parts, is_causal=True)
        Y = [c.transpose(1, 2).reshape(B, T, d) for c in Y]
        X = [a + b for a, b in zip(X, linear(Y, blk["proj_w"], blk["proj_b"]))]
        H = layer_norm(X, (d,), weight=[blk["ln2_w"]], bias=[blk["ln2_b"]])
        H = activation(linear(H, blk["fc_w"], blk["fc_b"]), "gelu_tanh")
        X = [a + b for a, b in zip(X, linear(H, blk["fc2_w"], blk["fc2_b"]))]
    X = layer_norm(X, (d,), weight=[params["lnf_w"]], bias=[params["lnf_b"]])
    logits = linear(X, params["head"])
    return cross_entropy([c.reshape(B * T, -1) for c in logits], targets.reshape(-1))
