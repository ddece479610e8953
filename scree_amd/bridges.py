"""HuggingFace ``(hidden_states, attention_mask)`` <-> :class:`scree_amd.Array`.

Same functions and conventions as the reference's bridge
(``src/scree/bridges/_hf_padded.py:15-46``): ``attention_mask`` is 1 for real
tokens and 0 for padding, int64 on the way out; right padding.  On ROCm
tensors both directions run the device kernels through
:func:`scree_amd.to_padded` / :func:`scree_amd.from_padded`.
"""

from __future__ import annotations

from typing import Any, Tuple

from ._core import Array, _is_torch, from_padded, to_padded


def from_hf_padded(hidden_states: Any, attention_mask: Any) -> Array:
    if _is_torch(attention_mask):
        import torch

        mask = attention_mask.to(dtype=torch.bool)
    else:
        mask = attention_mask.astype(bool)
    return from_padded(hidden_states, mask)


def to_hf_padded(arr: Array) -> Tuple[Any, Any]:
    padded, mask = to_padded(arr, side="right")
    if _is_torch(mask):
        import torch

        return padded, mask.to(dtype=torch.int64)
    import numpy as np

    return padded, mask.astype(np.int64)


__all__ = ["from_hf_padded", "to_hf_padded"]
