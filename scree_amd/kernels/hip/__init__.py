"""MI355X (gfx950) HIP kernels for the varlen path.

Counterpart of the reference's ``scree.kernels.triton`` package
(``src/scree/kernels/triton/__init__.py:10-31``): :data:`HIP_AVAILABLE` plays
the role of ``TRITON_AVAILABLE``.  The functions are always importable; when
the library is missing they raise ``HipUnavailableError`` on call.

The reference's own names are exported too, as aliases of the HIP launchers
(``varlen_attention_triton`` and friends, ``triton/__init__.py:17-29`` and
``triton/_backward.py:288``), so a caller of ``scree.kernels.triton`` changes
only its import line.  ``TRITON_AVAILABLE`` there reports whether the HIP
library loaded; nothing in this package uses Triton.
"""

from ._autograd import VarlenAttentionHip, varlen_attention_hip_autograd
from ._ffi import HIP_AVAILABLE, HipUnavailableError, ScreeHipError
from .attention import (
    attention_schedule,
    needs_schedule,
    prepare_workspace,
    schedule_items,
    varlen_attention_hip,
    varlen_attention_hip_backward,
)
from .norms import (
    varlen_add_rmsnorm_hip,
    varlen_add_rmsnorm_hip_backward,
    varlen_layernorm_hip,
    varlen_layernorm_hip_autograd,
    varlen_layernorm_hip_backward,
    varlen_rmsnorm_hip,
    varlen_rmsnorm_hip_autograd,
    varlen_rmsnorm_hip_backward,
)
from .softmax import varlen_softmax_hip, varlen_softmax_hip_backward

# The reference's names, bound to the HIP launchers (same arguments, same
# returns): src/scree/kernels/triton/varlen_attention.py:165,
# _backward.py:288, _autograd.py:51, varlen_rmsnorm.py:49,
# varlen_layernorm.py:52.
varlen_attention_triton = varlen_attention_hip
varlen_attention_triton_backward = varlen_attention_hip_backward
varlen_attention_triton_autograd = varlen_attention_hip_autograd
varlen_rmsnorm_triton = varlen_rmsnorm_hip
varlen_layernorm_triton = varlen_layernorm_hip
TRITON_AVAILABLE = HIP_AVAILABLE

__all__ = [
    "HIP_AVAILABLE",
    "TRITON_AVAILABLE",
    "HipUnavailableError",
    "ScreeHipError",
    "VarlenAttentionHip",
    "attention_schedule",
    "needs_schedule",
    "prepare_workspace",
    "schedule_items",
    "varlen_add_rmsnorm_hip",
    "varlen_add_rmsnorm_hip_backward",
    "varlen_attention_hip",
    "varlen_attention_hip_autograd",
    "varlen_attention_hip_backward",
    "varlen_layernorm_hip",
    "varlen_layernorm_hip_autograd",
    "varlen_layernorm_hip_backward",
    "varlen_rmsnorm_hip",
    "varlen_rmsnorm_hip_autograd",
    "varlen_rmsnorm_hip_backward",
    "varlen_softmax_hip",
    "varlen_softmax_hip_backward",
    "varlen_attention_triton",
    "varlen_attention_triton_autograd",
    "varlen_attention_triton_backward",
    "varlen_layernorm_triton",
    "varlen_rmsnorm_triton",
]
