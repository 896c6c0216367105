"""polytensors_amd: MI355X (gfx950) kernels for PolyTensors' truncated-Taylor hot path.

``PolyTensor`` keeps the reference library's public surface
(/root/reference/src/polytensors/__init__.py:1-5, _tensor.py:23-418); inside
``PolyTensor.plain_range()`` on HIP devices, matmul, scaled-dot-product
attention, RMSNorm/LayerNorm and cross entropy of degree-K series (K <= 8) run
hand-written HIP kernels through the C ABI of ``include/polytaylor.h``.
"""

from ._tensor import PolyTensor

__all__ = ["PolyTensor"]
