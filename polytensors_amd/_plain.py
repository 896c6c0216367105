"""The plain-range switch (/root/reference/src/polytensors/_plain.py:15-19).

Inside ``PolyTensor.plain_range()`` coefficients are ordinary tensors in their
dtype's range; the fused kernels run only there, as in the reference.
"""

import contextvars

_plain_range = contextvars.ContextVar("polytensors_amd_plain_range", default=False)


def plain_range_enabled():
    return _plain_range.get()


def in_backward():
    """Whether the calling thread is running an autograd graph task.

    The engine runs a CUDA graph's backward on its own device thread, where the
    caller's ``plain_range()`` context variable is not set. The reference's rules
    then fall back to its default mode; this package has no other mode (its
    forward operations run in plain range only, so every graph reaching backward
    was recorded there), so backward operations run in plain range
    (``_dispatch.dispatch``), as if the context had travelled with the graph.
    """
    import torch

    return torch._C._current_graph_task_id() != -1
