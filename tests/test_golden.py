"""The CPU oracle against the committed known-answer vectors (tests/golden/known_answers.json).

The vectors hold the fixed inputs of the reference's own tests (and benchmark
config 1's seeded inputs) with expected coefficients from nested forward-mode
AD; tests/golden/make_known_answers.py writes them. The GPU kernels are checked
against the same file in tests/test_gpu_golden.py.
"""

import json
import os

import pytest
import torch

import oracle
from oracle import paths, series
from tests.golden.make_known_answers import checksum, config1_inputs

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "known_answers.json")


def load():
    with open(FIXTURE) as f:
        return json.load(f)["cases"]


def dec(x):
    return torch.tensor(x, dtype=torch.float64)


def dec_complex(x):
    """The generator stores a complex tensor as [real part, imaginary part]."""
    re, im = x
    return torch.complex(torch.tensor(re, dtype=torch.float64), torch.tensor(im, dtype=torch.float64))


def close(got, want, tol=1e-12):
    got, want = (torch.as_tensor(x, dtype=torch.float64) if not isinstance(x, torch.Tensor) else x.double()
                 for x in (got, want))
    scale = max(want.abs().max().item(), 1e-300)
    assert (got - want).abs().max().item() <= tol * scale, ((got - want).abs().max().item(), scale)


def test_fixture_cases_present():
    assert set(load()) == {"square_plus_one", "complex_matmul", "cross_entropy_line", "softmax_family_line",
                           "rms_norm_line", "attention_masked", "config1"}


def test_square_plus_one():
    c = load()["square_plus_one"]
    X = [torch.tensor(v, dtype=torch.float64) for v in c["x"]]
    out = paths._add_to_order0(series.cauchy(X, X), 1)
    assert [o.item() for o in out] == c["expected"]


def test_complex_matmul():
    c = load()["complex_matmul"]
    A = paths.lift([dec(c["a"][0]), dec_complex(c["a"][1])], c["degree"])
    B = paths.lift([dec(c["b"][0]), dec_complex(c["b"][1])], c["degree"])
    C = oracle.matmul(A, B)
    for got, want in zip(C, c["expected"]):
        assert torch.equal(got.to(torch.complex128), dec_complex(want))


def test_cross_entropy_line():
    c = load()["cross_entropy_line"]
    Z = paths.lift([dec(c["x"]), dec(c["direction"])], c["degree"])
    got = oracle.cross_entropy(Z, torch.tensor(c["target"]), reduction=c["reduction"])
    for g, w in zip(got, c["expected"]):
        close(g, w)


@pytest.mark.parametrize("which", ("softmax", "log_softmax", "logsumexp"))
def test_softmax_family_line(which):
    c = load()["softmax_family_line"]
    sm, lsm, lse = series.softmax_family(paths.lift([dec(c["x"]), dec(c["direction"])], c["degree"]), -1)
    got = {"softmax": sm, "log_softmax": lsm, "logsumexp": [x.squeeze(-1) for x in lse]}[which]
    for g, w in zip(got, c["expected"][which]):
        close(g, dec(w))


def test_rms_norm_line():
    c = load()["rms_norm_line"]
    got = oracle.rms_norm(paths.lift([dec(c["x"]), dec(c["direction"])], c["degree"]), (4,), eps=c["eps"])
    for g, w in zip(got, c["expected"]):
        close(g, dec(w))


def test_attention_masked():
    c = load()["attention_masked"]
    Q, K, V = (paths.lift([dec(c[n][0]), dec(c[n][1])], c["degree"]) for n in "qkv")
    got = oracle.attention(Q, K, V, attn_mask=torch.tensor(c["mask"]))
    for g, w in zip(got, c["expected_rows_1_2"]):
        assert torch.isnan(g[..., 0, :]).all()   # plain range: softmax of a row with no admissible key
        close(g[..., 1:, :], dec(w))


def test_config1_inputs_reproduce():
    c = load()["config1"]
    lines, W, y = config1_inputs()
    got = [checksum(t) for line in lines for t in line] + [checksum(W), [float(y.sum())]]
    assert got == c["input_checksums"]


def test_config1_oracle():
    c = load()["config1"]
    lines, W, y = config1_inputs()
    Q, K, V = (paths.lift([x, d], c["degree"]) for x, d in lines)
    att = oracle.attention(Q, K, V, is_causal=True)
    for g, w in zip(att, c["attention_checksums"]):
        close(checksum(g)[0], w[0], 1e-10)
        close(checksum(g)[1], w[1], 1e-10)
    logits = oracle.matmul([a.reshape(128, 64) for a in att], [W])
    loss = oracle.cross_entropy(logits, y)
    for g, w in zip(loss, c["loss"]):
        close(g, w, 1e-10)
