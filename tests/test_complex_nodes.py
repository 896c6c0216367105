"""Real-node evaluation of complex directions (CPU): the interpolation weights.

polytensors_amd/_complex.py recovers a complex-direction coefficient P_k(i) from
real evaluations P_k(lam_m), P_k a real polynomial of degree <= k <= K. These
tests check the weights against the defining identity on monomials and on a
random polynomial (the GPU round trip through the plane kernels is in
tests/test_gpu_complex.py).
"""

import torch

from polytensors_amd import _complex


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
