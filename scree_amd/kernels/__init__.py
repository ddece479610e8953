"""Array-level varlen kernels on the HIP path.

Same signatures as the reference's ``scree.kernels.reference`` functions
(``src/scree/kernels/reference/varlen_attention.py:10``,
``varlen_rmsnorm.py:18``, ``varlen_layernorm.py:14``, ``varlen_softmax.py:13``),
taking and returning
:class:`scree_amd.Array`.  They run only on ROCm device tensors -- there is no
CPU implementation here; a host array raises ``TypeError``.  Outputs reuse
the input's offsets, as the reference does, and are built without
re-validating them, so none of these calls reads device memory on the host
(no host synchronisation; tested under ``torch.cuda.set_sync_debug_mode``).
"""

from __future__ import annotations

from .._core import Array, _is_torch


def _require_device(values, fn: str) -> None:
    if not (_is_torch(values) and values.is_cuda):
        raise TypeError(f"{fn}: the HIP kernels need ROCm device tensors, got {type(values).__name__}"
                        f"{' on ' + str(values.device) if _is_torch(values) else ''}")


def varlen_attention(q: Array, k: Array, v: Array, causal: bool = False) -> Array:
    """Per-sequence self-attention of packed ``(total, heads, head_dim)`` arrays.

    ``k`` / ``v`` may carry fewer heads than ``q`` (grouped-query attention:
    a divisor of the query heads, each K/V head serving consecutive query
    heads); the reference requires equal head counts.

    Offsets must be identical for q, k, v (``ValueError`` otherwise, as the
    reference, ``reference/varlen_attention.py:118-119``).  When all three
    Arrays share one offsets tensor the check is an identity test; distinct
    tensors are compared on the device, which reads the result on the host.
    Offsets that decrease somewhere (overlapping sequences; ``Array`` checks
    only the two ends) make every output and gradient NaN: the device
    scheduler checks them, so no host read of the offsets is needed.

    Values may be fp16 or bf16 (the matrix-instruction kernels, as the
    reference's Triton launcher takes, ``triton/varlen_attention.py:215``) or
    fp32, which the reference's Array-level torch branch also computes
    (``reference/varlen_attention.py:90-113``): fp32 runs on kernels that
    keep every operand in fp32.  q, k and v must share the dtype; any other
    dtype raises ``TypeError``.  The result supports autograd in every case.
    """
    import torch

    from .hip import VarlenAttentionHip

    _require_device(q.values, "varlen_attention")
    for name, a in (("q", q), ("k", k), ("v", v)):
        if a.values.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise TypeError(f"varlen_attention: {name} is {a.values.dtype}; the HIP kernels take "
                            "float16, bfloat16 or float32")
    if not (q.values.dtype == k.values.dtype == v.values.dtype):
        raise TypeError("varlen_attention: q, k and v must share a dtype")
    if not (q.offsets is k.offsets and q.offsets is v.offsets):
        if not (torch.equal(q.offsets, k.offsets) and torch.equal(q.offsets, v.offsets)):
            raise ValueError("q, k, v must have identical offsets")
    if q.ragged_dim != 0:
        raise NotImplementedError("varlen_attention supports ragged_dim=0 only")
    out = VarlenAttentionHip.apply(q.values, k.values, v.values, q.offsets, causal)
    return Array._trusted(out, q.offsets, 0)


def varlen_rmsnorm(arr: Array, weight=None, eps: float = 1e-6) -> Array:
    """RMSNorm over the last axis of a packed array."""
    from .hip import varlen_rmsnorm_hip

    _require_device(arr.values, "varlen_rmsnorm")
    return Array._trusted(varlen_rmsnorm_hip(arr.values, weight, eps), arr.offsets, arr.ragged_dim)


def varlen_layernorm(arr: Array, weight=None, bias=None, eps: float = 1e-5) -> Array:
    """LayerNorm over the last axis of a packed array."""
    from .hip import varlen_layernorm_hip

    _require_device(arr.values, "varlen_layernorm")
    return Array._trusted(varlen_layernorm_hip(arr.values, weight, bias, eps), arr.offsets,
                          arr.ragged_dim)


def varlen_add_rmsnorm(arr: Array, residual, weight=None, eps: float = 1e-6):
    """Fused ``h = arr + residual`` and ``y = varlen_rmsnorm(h)``; returns ``(h, y)`` as Arrays.

    ``residual`` is an :class:`Array` with the same offsets or a tensor of the
    values' shape.  Same results, bit for bit, as adding then calling
    :func:`varlen_rmsnorm` (the reference block's two steps,
    ``examples/03_train_step.py:46-48``).
    """
    import torch

    from .hip import varlen_add_rmsnorm_hip

    _require_device(arr.values, "varlen_add_rmsnorm")
    if isinstance(residual, Array):
        if residual.offsets is not arr.offsets and not torch.equal(residual.offsets, arr.offsets):
            raise ValueError("arr and residual must have identical offsets")
        residual = residual.values
    h, y = varlen_add_rmsnorm_hip(arr.values, residual, weight, eps)
    return (Array._trusted(h, arr.offsets, arr.ragged_dim),
            Array._trusted(y, arr.offsets, arr.ragged_dim))


def varlen_softmax(arr: Array) -> Array:
    """Softmax along the ragged dimension, per sequence (``varlen_softmax.py:13-63``)."""
    from .hip import varlen_softmax_hip

    if arr.ragged_dim != 0:
        raise NotImplementedError("varlen_softmax supports ragged_dim=0 only in v0.1")
    _require_device(arr.values, "varlen_softmax")
    return Array._trusted(varlen_softmax_hip(arr.values, arr.offsets), arr.offsets, 0)


__all__ = ["varlen_add_rmsnorm", "varlen_attention", "varlen_layernorm", "varlen_rmsnorm",
           "varlen_softmax"]
