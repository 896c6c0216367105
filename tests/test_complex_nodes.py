"""Real-node evaluation of complex directions (CPU): the interpolation weights.

polytensors_amd/_complex.py recovers a complex-direction coefficient P_k(i) from
real evaluations P_k(lam_m), P_k a real polynomial of degree <= k <= K. These
tests check the weights against the defining identity on monomials and on a
random polynomial, and that the real-variant construction keeps order 0.
"""

import torch

from polytensors_amd import PolyTensor, _complex


def test_weights_evaluate_every_monomial_at_i():
    for degree in range(0, 9):
        nodes, weights = _complex.nodes_and_weights(degree)
        assert len(set(nodes)) == degree + 1 and all(isinstance(x, float) for x in nodes)
        for j in range(degree + 1):
            got = sum(w * lam ** j for w, lam in zip(weights, nodes))
            assert abs(got - 1j ** j) < 1e-9 * max(1.0, max(abs(x) for x in nodes) ** j)


def test_weights_on_a_random_polynomial():
    g = torch.Generator().manual_seed(0)
    for degree in (1, 3, 5):
        coeffs = torch.randn(degree + 1, generator=g, dtype=torch.float64).tolist()
        nodes, weights = _complex.nodes_and_weights(degree)
        p = lambda z: sum(c * z ** j for j, c in enumerate(coeffs))  # noqa: E731
        assert abs(sum(w * p(x) for w, x in zip(weights, nodes)) - p(1j)) < 1e-12 * sum(abs(c) for c in coeffs) * 2 ** degree


def test_real_variant_and_combination_round_trip():
    # the real variants at every node, recombined, give back the complex series itself (identity map)
    x = PolyTensor((torch.randn(3, 4, dtype=torch.float64),
                    torch.randn(3, 4, dtype=torch.complex128), torch.randn(3, 4, dtype=torch.complex128)))
    assert _complex.has_complex(x) and not _complex.has_complex(x.coeffs[0], [1, 2])
    out = _complex.at_real_nodes(lambda s: s, "identity", x)
    assert torch.equal(out.coeffs[0], x.coeffs[0])
    for a, b in zip(out.coeffs[1:], x.coeffs[1:]):
        assert (a - b).abs().max() < 1e-13
