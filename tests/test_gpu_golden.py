"""The gfx950 kernels against the committed known-answer vectors (tests/golden/known_answers.json).

Each case runs through the PolyTensor API on the GPU in float64 (the reference's
fixed test data, benchmark config 1) and is compared with the stored expected
coefficients at 1e-10 relative to each order's largest value. The attention
case pads the head dim from 2 to 16 with zeros (the kernels take 16..128; zero
columns change neither the scores nor the kept output columns) and, as the
reference's fused kernels do, returns zeros for the row with no admissible key.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from polytensors_amd import PolyTensor
from tests.golden.make_known_answers import checksum, config1_inputs
from tests.test_golden import close, dec, dec_complex, load

pytestmark = pytest.mark.gpu

TOL = 1e-10


def _poly(coeffs, degree):
    return PolyTensor(tuple(c.cuda() for c in coeffs), degree=degree)


def test_square_plus_one():
    c = load()["square_plus_one"]
    with torch.no_grad(), PolyTensor.plain_range():
        x = _poly([torch.tensor([v], dtype=torch.float64) for v in c["x"]], c["degree"])
        out = x * x + 1
    assert [o.item() for o in out.coeffs] == c["expected"]


def test_complex_matmul():
    c = load()["complex_matmul"]
    with torch.no_grad(), PolyTensor.plain_range():
        a = _poly([dec(c["a"][0]), dec_complex(c["a"][1])], c["degree"])
        b = _poly([dec(c["b"][0]), dec_complex(c["b"][1])], c["degree"])
        out = a @ b
    for got, want in zip(out.coeffs, c["expected"]):
        close(got.cpu().to(torch.complex128).real, dec_complex(want).real, TOL)
        close(got.cpu().to(torch.complex128).imag, dec_complex(want).imag, TOL)


def test_cross_entropy_line():
    c = load()["cross_entropy_line"]
    with torch.no_grad(), PolyTensor.plain_range():
        z = _poly([dec(c["x"]), dec(c["direction"])], c["degree"])
        out = F.cross_entropy(z, torch.tensor(c["target"]).cuda(), reduction=c["reduction"])
    for got, want in zip(out.coeffs, c["expected"]):
        close(got.cpu(), want, TOL)


def test_rms_norm_line():
    c = load()["rms_norm_line"]
    with torch.no_grad(), PolyTensor.plain_range():
        x = _poly([dec(c["x"]), dec(c["direction"])], c["degree"])
        out = F.rms_norm(x, (4,), eps=c["eps"])
    for got, want in zip(out.coeffs, c["expected"]):
        close(got.cpu(), dec(want), TOL)


def test_attention_masked_padded_head_dim():
    c = load()["attention_masked"]

    def padded(name):
        return [F.pad(dec(x), (0, 14)) for x in c[name]]

    with torch.no_grad(), PolyTensor.plain_range():
        q, k, v = (_poly(padded(n), c["degree"]) for n in "qkv")
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=torch.tensor(c["mask"]).cuda(), scale=1 / math.sqrt(2))
    for got, want in zip(out.coeffs, c["expected_rows_1_2"]):
        got = got.cpu()
        assert torch.equal(got[..., 0, :], torch.zeros_like(got[..., 0, :]))   # no admissible key
        assert torch.equal(got[..., 2:], torch.zeros_like(got[..., 2:]))       # zero V columns
        close(got[..., 1:, :2], dec(want), TOL)


def test_config1():
    c = load()["config1"]
    lines, W, y = config1_inputs()
    assert [checksum(t) for line in lines for t in line] + [checksum(W), [float(y.sum())]] == c["input_checksums"]
    with torch.no_grad(), PolyTensor.plain_range():
        q, k, v = (_poly([x, d], c["degree"]) for x, d in lines)
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        loss = F.cross_entropy(out.reshape(128, 64) @ W.cuda(), y.cuda())
    for got, want in zip(out.coeffs, c["attention_checksums"]):
        s, s2 = checksum(got.cpu())
        close(s, want[0], TOL)
        close(s2, want[1], TOL)
    for got, want in zip(loss.coeffs, c["loss"]):
        close(got.cpu(), want, TOL)
