"""The plain-range switch (/root/reference/src/polytensors/_plain.py:15-19).

Inside ``PolyTensor.plain_range()`` coefficients are ordinary tensors in their
dtype's range; the fused kernels run only there, as in the reference.
"""

import contextvars

_plain_range = contextvars.ContextVar("polytensors_amd_plain_range", default=False)


def plain_range_enabled():
    return _plain_range.get()
