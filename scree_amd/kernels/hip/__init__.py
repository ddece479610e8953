"""MI355X (gfx950) HIP kernels for the varlen path.

Counterpart of the reference's ``scree.kernels.triton`` package
(``src/scree/kernels/triton/__init__.py:10-31``): :data:`HIP_AVAILABLE` plays
the role of ``TRITON_AVAILABLE``.  The functions are always importable; when
the library is missing they raise ``HipUnavailableError`` on call.
"""

from ._autograd import VarlenAttentionHip, varlen_attention_hip_autograd
from ._ffi import HIP_AVAILABLE, HipUnavailableError, ScreeHipError
from .attention import (
    attention_schedule,
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

__all__ = [
    "HIP_AVAILABLE",
    "HipUnavailableError",
    "ScreeHipError",
    "VarlenAttentionHip",
    "attention_schedule",
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
]
