"""CPU oracle of the truncated-Taylor hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in plain PyTorch on the CPU, of the reference's plain-range
general series rules for the four fused operations (Cauchy-product matmul,
scaled-dot-product attention, RMSNorm/LayerNorm, cross entropy) and of the
elementwise activation series (oracle/activations.py). Each function
cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline. The product (``polytensors_amd``) never imports or calls it.

Pinning (tests/test_oracle_pins.py): every function here is checked against
independent derivatives (nested autograd / torch.func.jvp on the composite
function along the curve, in float64), against closed forms and known-answer
values the reference's own tests hold, and against brute-force sums.
"""

from .series import cauchy, exp_series, log_series, quotient, rsqrt_series, softmax_family  # noqa: F401
from .paths import attention, cross_entropy, layer_norm, layer_norm_backward, matmul, rms_norm  # noqa: F401
from .paths import attention_backward, cross_entropy_backward, rms_norm_backward  # noqa: F401
from .activations import activation, activation_backward  # noqa: F401
from .decoder import gpt_forward  # noqa: F401
