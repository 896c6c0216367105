"""PolyTensor surface and routing (CPU only).

The coercion rules follow /root/reference/src/polytensors/_tensor.py:38-126 (and its tests,
/root/reference/tests/test_tensor.py); the fused entry points must refuse loudly, never fall
back, when a call is outside what the kernels implement.
"""

import pytest
import torch
import torch.nn.functional as F

from polytensors_amd import PolyTensor
from polytensors_amd import _fused_attention, _fused_cross_entropy, _fused_matmul, _fused_norm
from polytensors_amd._plain import plain_range_enabled


def test_degree_padding_and_broadcast():
    # /root/reference/tests/test_tensor.py:60-66: coefficients broadcast to one shape
    x = PolyTensor([torch.tensor([1.0, 2.0]), torch.tensor(3.0)], degree=2)
    assert x.degree == 2 and all(c.shape == (2,) for c in x.coeffs)
    assert torch.equal(x.coeffs[1], torch.tensor([3.0, 3.0]))
    assert torch.equal(x.coeffs[2], torch.zeros(2))
    assert torch.equal(x.value, torch.tensor([1.0, 2.0])) and torch.equal(x.tangent, x.coeffs[1])


def test_dtype_promotion_and_complex_directions():
    x = PolyTensor((torch.ones(3, dtype=torch.float32), torch.ones(3, dtype=torch.float64)))
    assert x.dtype == torch.float64 and x.coeffs[1].dtype == torch.float64
    z = PolyTensor((torch.ones(2), torch.full((2,), 1j, dtype=torch.complex64)), degree=3)
    assert z.value.dtype == torch.float32
    assert all(c.dtype == torch.complex64 for c in z.coeffs[1:])


def test_rejections():
    with pytest.raises(ValueError):
        PolyTensor(())
    with pytest.raises(TypeError):
        PolyTensor((torch.ones(2, dtype=torch.int64),))
    with pytest.raises(ValueError):
        PolyTensor((torch.ones(2), torch.ones(2)), degree=0)
    with pytest.raises(TypeError):
        PolyTensor((torch.ones(2),), degree=True)


def test_overlapping_orders_are_cloned_and_stacked_views_are_not():
    z = torch.zeros(4)
    x = PolyTensor((z, z, z))
    ptrs = {c.data_ptr() for c in x.coeffs}
    assert len(ptrs) == 3
    stacked = torch.randn(3, 4)
    y = PolyTensor.from_stacked(stacked)
    assert [c.data_ptr() for c in y.coeffs] == [stacked[i].data_ptr() for i in range(3)]


def test_constant_and_context_switches_are_context_local():
    c = PolyTensor.constant(torch.ones(2), 3)
    assert c.degree == 3 and all(torch.equal(k, torch.zeros(2)) for k in c.coeffs[1:])
    assert not plain_range_enabled()
    with PolyTensor.plain_range():
        assert plain_range_enabled()
    assert not plain_range_enabled()
    with PolyTensor.fused_attention(False):
        assert not _fused_attention._enabled.get()
    assert _fused_attention._enabled.get()
    with PolyTensor.fused_cross_entropy(False):
        assert not _fused_cross_entropy._enabled.get()


def test_retain_wrappers_scopes():
    # /root/reference/tests/test_primitives.py:31-60
    x = PolyTensor.constant(torch.tensor([0.1, -0.2]), degree=3)
    with PolyTensor.retain_wrappers() as outer:
        with PolyTensor.retain_wrappers() as inner:
            y = x + 0.4
            assert any(item is y for item in inner) and any(item is y for item in outer)
        assert inner == []
        with PolyTensor.retain_wrappers(isolated=True) as alone:
            w = x * 2.0
            assert any(item is w for item in alone) and not any(item is w for item in outer)
    assert outer == []


def test_linear_rules_are_per_coefficient():
    x = PolyTensor((torch.tensor([1.0, 2.0]), torch.tensor([3.0, 4.0]), torch.tensor([5.0, 6.0])))
    y = PolyTensor((torch.tensor([1.0, 1.0]), torch.tensor([1.0, 1.0]), torch.tensor([1.0, 1.0])))
    s = x + y
    assert [c.tolist() for c in s.coeffs] == [[2, 3], [4, 5], [6, 7]]
    d = 2 * x - 1
    assert [c.tolist() for c in d.coeffs] == [[1, 3], [6, 8], [10, 12]]
    m = x.sum()
    assert [c.item() for c in m.coeffs] == [3, 7, 11]
    t = PolyTensor((torch.arange(6.0).reshape(2, 3), torch.ones(2, 3))).transpose(0, 1).reshape(6)
    assert t.shape == (6,) and t.coeffs[0].tolist() == [0, 3, 1, 4, 2, 5]


def test_nonlinear_series_without_a_kernel_raise():
    x = PolyTensor((torch.ones(2), torch.ones(2)))
    with pytest.raises(NotImplementedError):
        torch.exp(x)
    with pytest.raises(NotImplementedError):
        x * x


@pytest.mark.parametrize("op", ["rms_norm", "layer_norm", "attention", "cross_entropy", "matmul"])
def test_fused_calls_refuse_instead_of_falling_back(op):
    x = PolyTensor((torch.randn(2, 1, 8, 16), torch.randn(2, 1, 8, 16)))
    z = PolyTensor((torch.randn(4, 10), torch.randn(4, 10)))
    y = torch.randint(0, 10, (4,))
    calls = {
        "rms_norm": lambda: F.rms_norm(x, (16,)),
        "layer_norm": lambda: F.layer_norm(x, (16,)),
        "attention": lambda: F.scaled_dot_product_attention(x, x, x, is_causal=True),
        "cross_entropy": lambda: F.cross_entropy(z, y),
        "matmul": lambda: z @ z.transpose(0, 1),
    }
    for scope in (None, PolyTensor.plain_range):
        with pytest.raises(NotImplementedError) as info:
            if scope is None:
                calls[op]()
            else:
                with scope():
                    calls[op]()
        reason = str(info.value)
        assert ("extended-range" in reason) if scope is None else ("HIP" in reason)


def test_eligibility_reasons():
    x = PolyTensor((torch.randn(1, 1, 8, 16), torch.randn(1, 1, 8, 16)))
    with PolyTensor.plain_range():
        assert not _fused_norm.eligible(x, (16,))
        assert "HIP" in _fused_norm.why_ineligible(x, (16,))
        assert "dropout" in _fused_attention.why_ineligible(x, x, x, None, 0.5, False, False)
        assert "GQA" in _fused_attention.why_ineligible(x, x, x, None, 0.0, False, True)
        with PolyTensor.fused_attention(False):
            assert "disabled" in _fused_attention.why_ineligible(x, x, x, None, 0.0, False, False)
        assert not _fused_matmul.eligible(x, x)
    deep = PolyTensor((torch.randn(3, 4),), degree=9)
    with PolyTensor.plain_range():
        assert "exceeds" in _fused_norm.why_ineligible(deep, (4,))


def test_backward_seeds_the_constant_series_and_accumulates():
    # /root/reference/src/polytensors/_tensor.py:325-338: a scalar output seeds (1, 0, ..., 0).
    x = PolyTensor((torch.ones(3, dtype=torch.float64), torch.full((3,), 2.0, dtype=torch.float64)),
                   requires_grad=True)
    with PolyTensor.retain_wrappers():
        y = (x * 3.0 + 1.0).sum()
        y.backward()
        assert isinstance(x.grad, PolyTensor) and x.grad.degree == 1
        assert [c.tolist() for c in x.grad.coeffs] == [[3.0] * 3, [0.0] * 3]
        (x * 2.0).sum().backward()          # a second pass accumulates
        assert [c.tolist() for c in x.grad.coeffs] == [[5.0] * 3, [0.0] * 3]


def test_backward_with_an_ordinary_gradient_lifts_it():
    x = PolyTensor((torch.ones(2, dtype=torch.float64), torch.ones(2, dtype=torch.float64)), requires_grad=True)
    with PolyTensor.retain_wrappers():
        (x * 4.0).backward(torch.tensor([1.0, 2.0], dtype=torch.float64))
        assert [c.tolist() for c in x.grad.coeffs] == [[4.0, 8.0], [0.0, 0.0]]


def test_backward_needs_a_scalar_or_a_gradient():
    x = PolyTensor((torch.ones(3), torch.ones(3)), requires_grad=True)
    with PolyTensor.retain_wrappers(), pytest.raises(RuntimeError, match="scalar"):
        (x * 2.0).backward()


def test_plain_tensor_cross_entropy_with_softcap_matches_composite():
    # /root/reference/tests/test_fused_kernels.py:214-220 on ordinary tensors
    z = torch.randn(10, 50)
    y = torch.randint(0, 50, (10,))
    expected = F.cross_entropy(15 * torch.tanh(z / 15), y)
    assert torch.allclose(PolyTensor.cross_entropy(z, y, softcap=15.0), expected)


def test_masks_and_class_weights_that_require_grad_are_refused():
    # no gradient flows to attn_mask or to class weights: such calls are refused, not silently cut
    from polytensors_amd import _fused_attention, _fused_cross_entropy

    x = PolyTensor((torch.randn(1, 1, 8, 16), torch.randn(1, 1, 8, 16)))
    mask = torch.zeros(8, 8, requires_grad=True)
    assert "requires grad" in _fused_attention.why_ineligible(x, x, x, mask, 0.0, False, False)
    z = PolyTensor((torch.randn(4, 10), torch.randn(4, 10)))
    y = torch.randint(0, 10, (4,))
    w = torch.ones(10, requires_grad=True)
    assert "require grad" in _fused_cross_entropy.why_ineligible(z, y, w)
    with torch.no_grad():
        assert "requires grad" not in (_fused_attention.why_ineligible(x, x, x, mask, 0.0, False, False) or "")
