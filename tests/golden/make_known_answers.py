"""Writes tests/golden/known_answers.json: known-answer vectors for the series path.

Inputs are the fixed data of the reference's own tests (cited per case) or
benchmark config 1's seeded inputs; expected outputs are independent Taylor
coefficients from nested ``torch.func.jvp`` (tests/jets.py) in float64, or the
closed-form answers those tests assert. Nothing here imports or runs the
reference. Run from the repository root:

    python -m tests.golden.make_known_answers
"""

import json
import math
import os

import torch
import torch.nn.functional as F

from tests.jets import taylor

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")


def enc(x):
    """Nested lists of floats; complex values as [re, im] pairs."""
    if isinstance(x, torch.Tensor):
        if x.is_complex():
            return [enc(x.real), enc(x.imag)]
        return x.tolist()
    return x


def math_attention(q, k, v, excluded=None, is_causal=False, scale=None):
    L, S = q.shape[-2], k.shape[-2]
    s = (1 / math.sqrt(q.shape[-1]) if scale is None else scale) * (q @ k.transpose(-2, -1))
    if is_causal:
        excluded = ~torch.ones(L, S, dtype=torch.bool).tril()
    if excluded is not None:
        s = s.masked_fill(excluded, float("-inf"))
    return torch.softmax(s, -1) @ v


def config1_inputs():
    """benchmark config 1 (seed 0, float64): Q/K/V = x + t v with x, v ~ N(0,1)/8, W ~ N(0,1)/8."""
    g = torch.Generator().manual_seed(0)
    shape = (1, 1, 128, 64)
    lines = [(torch.randn(shape, generator=g, dtype=torch.float64) / 8,
              torch.randn(shape, generator=g, dtype=torch.float64) / 8) for _ in range(3)]
    W = torch.randn(64, 256, generator=g, dtype=torch.float64) / 8
    y = torch.randint(0, 256, (128,), generator=g)
    return lines, W, y


def checksum(t):
    return [t.sum().item(), (t * t).sum().item()]


def main():
    cases = {}

    # /root/reference/tests/test_tensor.py:70-76: x = 2 + t, x * x + 1 = 5 + 4t + t^2
    cases["square_plus_one"] = {
        "source": "tests/test_tensor.py:70-76", "degree": 3,
        "x": [2.0, 1.0, 0.0, 0.0], "expected": [5.0, 4.0, 1.0, 0.0]}

    # /root/reference/tests/test_dispatch.py:63-70: (I + i 1 t) @ (2I + 2i 1 t), degree 2
    eye = torch.eye(2, dtype=torch.float64)
    ones = torch.ones(2, 2, dtype=torch.float64)
    cases["complex_matmul"] = {
        "source": "tests/test_dispatch.py:63-70", "degree": 2,
        "a": [enc(eye), enc(ones * 1j)], "b": [enc(2 * eye), enc(ones * 2j)],
        "expected": [enc(2 * eye + 0j), enc(ones * 4j), enc(-4 * ones + 0j)]}

    # /root/reference/tests/test_primitives.py:115-146 and :245-273: fixed logits and direction
    x0 = torch.tensor([[0.2, -1.3, 2.1], [3.0, -4.0, 0.1]], dtype=torch.float64)
    d = torch.tensor([[0.7, -0.2, 0.4], [-0.8, 0.5, 0.3]], dtype=torch.float64)
    y = torch.tensor([2, 0])
    ce = taylor(lambda v: F.cross_entropy(v, y, reduction="sum"), [[x0, d]], 3)
    cases["cross_entropy_line"] = {
        "source": "tests/test_primitives.py:115-146", "degree": 3, "reduction": "sum",
        "x": enc(x0), "direction": enc(d), "target": y.tolist(), "expected": [c.item() for c in ce]}
    fam = {
        "softmax": taylor(lambda v: torch.softmax(v, -1), [[x0, d]], 3),
        "log_softmax": taylor(lambda v: torch.log_softmax(v, -1), [[x0, d]], 3),
        "logsumexp": taylor(lambda v: torch.logsumexp(v, -1), [[x0, d]], 3)}
    cases["softmax_family_line"] = {
        "source": "tests/test_primitives.py:245-273", "degree": 3, "x": enc(x0), "direction": enc(d),
        "expected": {k: [enc(c) for c in v] for k, v in fam.items()}}

    # /root/reference/tests/test_plain_range.py:103-115: RMSNorm of a shape-(4,) line, eps 1e-5, degree 4
    g = torch.Generator().manual_seed(7)
    base, direction = (torch.randn(4, generator=g, dtype=torch.float64) for _ in range(2))
    rn = taylor(lambda x: F.rms_norm(x, (4,), eps=1e-5), [[base, direction]], 4)
    cases["rms_norm_line"] = {
        "source": "tests/test_plain_range.py:103-115", "degree": 4, "eps": 1e-5,
        "x": enc(base), "direction": enc(direction), "expected": [enc(c) for c in rn]}

    # /root/reference/tests/test_attention.py:13-17,52: seed 27, (1,1,3,2), values / 3, directions / 4,
    # boolean mask (True = admissible); row 0 admits no key (plain range: NaN, fused kernels: 0)
    g = torch.Generator().manual_seed(27)
    values = [torch.randn(1, 1, 3, 2, generator=g, dtype=torch.float64) / 3 for _ in range(3)]
    directions = [torch.randn(c.shape, generator=g, dtype=c.dtype) / 4 for c in values]
    mask = torch.tensor([[False, False, False], [True, False, True], [True, True, True]])
    at = taylor(lambda q, k, v: math_attention(q, k, v, excluded=~mask),
                [[values[i], directions[i]] for i in range(3)], 3)
    cases["attention_masked"] = {
        "source": "tests/test_attention.py:13-55", "degree": 3, "mask": mask.tolist(),
        "q": [enc(values[0]), enc(directions[0])], "k": [enc(values[1]), enc(directions[1])],
        "v": [enc(values[2]), enc(directions[2])],
        "expected_rows_1_2": [enc(c[..., 1:, :]) for c in at]}

    # benchmark config 1: causal attention, logits = out.view(128, 64) @ W, mean cross entropy, degree 3.
    # The inputs are regenerated from the seed; their checksums guard against generator drift.
    lines, W, y = config1_inputs()
    def loss_fn(q, k, v):
        out = math_attention(q, k, v, is_causal=True)
        return F.cross_entropy(out.reshape(128, 64) @ W, y)
    series = [[x, dv] for x, dv in lines]
    att = taylor(lambda q, k, v: math_attention(q, k, v, is_causal=True), series, 3)
    loss = taylor(loss_fn, series, 3)
    cases["config1"] = {
        "source": "BASELINE config 1 (seed 0)", "degree": 3,
        "input_checksums": [checksum(t) for line in lines for t in line] + [checksum(W), [float(y.sum())]],
        "attention_checksums": [checksum(c) for c in att],
        "loss": [c.item() for c in loss]}

    meta = {"torch": torch.__version__, "how": "tests/golden/make_known_answers.py (nested torch.func.jvp, float64)"}
    with open(OUT, "w") as f:
        json.dump({"meta": meta, "cases": cases}, f, indent=1)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
