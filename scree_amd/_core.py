"""The packed ``values + offsets + ragged_dim`` value type and its constructors.

This is the contract the varlen kernels consume: ``offsets`` is an int32
vector of length ``B + 1`` with ``offsets[0] == 0`` and
``offsets[-1] == values.shape[ragged_dim]`` -- exactly FlashAttention's
``cu_seqlens``.  Behaviour follows ``src/scree/_core.py`` of the reference
(invariants ``:44-62``, ``pack`` ``:97-141``, ``unpack`` ``:144-158``,
``to_padded`` / ``from_padded`` ``:161-301``, ``from_cu_seqlens``
``:304-309``), restricted to the two backends this package runs on: numpy
(host) and torch (host or ROCm device).  Error messages are kept word for word
so callers matching on them keep working.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Tuple

import numpy as np


def _is_torch(x: Any) -> bool:
    return type(x).__module__.startswith("torch")


def _offsets_from_lengths_np(lengths: List[int]) -> np.ndarray:
    """int32 ``[0, cumsum(lengths)]`` (reference ``_core.py:137-138``)."""
    offsets = np.zeros(len(lengths) + 1, dtype=np.int32)
    if lengths:
        offsets[1:] = np.cumsum(np.asarray(lengths, dtype=np.int64)).astype(np.int32)
    return offsets


@dataclass(frozen=True)
class Array:
    """A packed array with one variable-length dimension.

    Three sequences of lengths ``[4, 2, 5]`` with feature dim 8 are stored as
    ``values`` of shape ``(11, 8)`` and ``offsets = [0, 4, 6, 11]``.
    """

    values: Any
    offsets: Any
    ragged_dim: int = 0

    def __post_init__(self) -> None:
        if self.values.ndim < 1:
            raise ValueError(f"values must be at least 1-D, got {self.values.ndim}-D")
        if not (0 <= self.ragged_dim < self.values.ndim):
            raise ValueError(
                f"ragged_dim={self.ragged_dim} out of range for {self.values.ndim}-D values"
            )
        if self.offsets.ndim != 1:
            raise ValueError(f"offsets must be 1-D, got {self.offsets.ndim}-D")
        if len(self.offsets) < 2:
            raise ValueError("offsets must have length >= 2")
        first = int(self.offsets[0])
        if first != 0:
            raise ValueError(f"offsets[0] must be 0, got {first}")
        ragged_size = self.values.shape[self.ragged_dim]
        last = int(self.offsets[-1])
        if last != ragged_size:
            raise ValueError(
                f"offsets[-1] ({last}) must equal "
                f"values.shape[ragged_dim={self.ragged_dim}] ({ragged_size})"
            )

    @classmethod
    def _trusted(cls, values: Any, offsets: Any, ragged_dim: int = 0) -> "Array":
        """An Array whose invariants the caller already holds -- a kernel
        output that reuses the validated offsets of its input -- built
        without ``__post_init__``'s reads of ``offsets[0]`` and
        ``offsets[-1]``, which are host synchronisations for device offsets."""
        obj = object.__new__(cls)
        object.__setattr__(obj, "values", values)
        object.__setattr__(obj, "offsets", offsets)
        object.__setattr__(obj, "ragged_dim", ragged_dim)
        return obj

    @property
    def batch_size(self) -> int:
        return len(self.offsets) - 1

    @property
    def lengths(self) -> Any:
        """``lengths[i] = offsets[i + 1] - offsets[i]``."""
        return self.offsets[1:] - self.offsets[:-1]

    @property
    def total_length(self) -> int:
        return int(self.offsets[-1])

    @property
    def dtype(self) -> Any:
        return self.values.dtype

    @property
    def feature_shape(self) -> tuple:
        return tuple(s for i, s in enumerate(self.values.shape) if i != self.ragged_dim)

    def __len__(self) -> int:
        return self.batch_size

    def __repr__(self) -> str:
        return (
            f"scree.Array(batch_size={self.batch_size}, "
            f"total_length={self.total_length}, "
            f"feature_shape={self.feature_shape}, "
            f"dtype={self.dtype})"
        )


def pack(arrays: List[Any], ragged_dim: int = 0) -> Array:
    """Concatenate a list of arrays along ``ragged_dim`` and record int32 offsets.

    The first array picks the backend.  For torch the offsets are built on the
    first array's device, as the reference does (``_core.py:108-113``).
    """
    if not arrays:
        raise ValueError("Cannot pack an empty list")
    first = arrays[0]
    lengths = [int(a.shape[ragged_dim]) for a in arrays]
    if _is_torch(first):
        import torch

        offsets = torch.from_numpy(_offsets_from_lengths_np(lengths)).to(first.device)
        values = torch.cat(arrays, dim=ragged_dim)
    else:
        offsets = _offsets_from_lengths_np(lengths)
        values = np.concatenate(arrays, axis=ragged_dim)
    return Array(values=values, offsets=offsets, ragged_dim=ragged_dim)


def unpack(arr: Array) -> List[Any]:
    """Split ``arr.values`` back into per-sequence views along the ragged dim."""
    bounds = [int(o) for o in (arr.offsets.tolist() if hasattr(arr.offsets, "tolist") else arr.offsets)]
    rd = arr.ragged_dim
    ndim = arr.values.ndim
    out: List[Any] = []
    for i in range(arr.batch_size):
        slc = [slice(None)] * ndim
        slc[rd] = slice(bounds[i], bounds[i + 1])
        out.append(arr.values[tuple(slc)])
    return out


def to_padded(arr: Array, side: str = "right", fill_value: float = 0.0) -> Tuple[Any, Any]:
    """``(padded, mask)`` with ``padded.shape == (B, max_len, *features)``.

    Semantics of the reference (``_core.py:161-266``).  ROCm tensors go through
    the device kernel; host arrays use the loop below.
    """
    if arr.ragged_dim != 0:
        raise NotImplementedError("to_padded supports ragged_dim=0 only in v0.1")
    if side not in ("right", "left"):
        raise ValueError(f"side must be 'right' or 'left', got {side!r}")
    if _is_torch(arr.values) and arr.values.is_cuda:
        # ROCm tensors: one device launch (scree_to_padded), no per-row host loop
        from .kernels.hip.padding import to_padded_hip

        return to_padded_hip(arr.values, arr.offsets, side, fill_value)
    bounds = [int(o) for o in arr.offsets.tolist()]
    lengths = [bounds[i + 1] - bounds[i] for i in range(arr.batch_size)]
    max_len = max(lengths) if lengths else 0
    feature_shape = tuple(arr.values.shape[1:])
    batch = arr.batch_size
    if _is_torch(arr.values):
        import torch

        padded = torch.full(
            (batch, max_len, *feature_shape), fill_value, dtype=arr.values.dtype,
            device=arr.values.device,
        )
        mask = torch.zeros((batch, max_len), dtype=torch.bool, device=arr.values.device)
    else:
        padded = np.full((batch, max_len, *feature_shape), fill_value, dtype=arr.values.dtype)
        mask = np.zeros((batch, max_len), dtype=np.bool_)
    for i, length in enumerate(lengths):
        row = arr.values[bounds[i] : bounds[i] + length]
        if side == "right":
            padded[i, :length] = row
            mask[i, :length] = True
        else:
            padded[i, max_len - length :] = row
            mask[i, max_len - length :] = True
    return padded, mask


def from_padded(padded: Any, mask: Any) -> Array:
    """Inverse of right-padded :func:`to_padded` (reference ``_core.py:269-301``).

    ROCm tensors go through the device kernels; host arrays use the loop below.
    """
    batch = padded.shape[0]
    if _is_torch(padded) and padded.is_cuda:
        # ROCm tensors: device count/scan + gather (scree_padded_offsets, scree_from_padded)
        from .kernels.hip.padding import from_padded_hip

        values, offsets = from_padded_hip(padded, mask)
        return Array(values=values, offsets=offsets, ragged_dim=0)
    if _is_torch(padded):
        import torch

        lengths = [int(v) for v in mask.sum(dim=1).tolist()]
        rows = [padded[i, : lengths[i]] for i in range(batch)]
        values = torch.cat(rows, dim=0)
        offsets = torch.from_numpy(_offsets_from_lengths_np(lengths)).to(padded.device)
    else:
        lengths = [int(v) for v in np.asarray(mask).sum(axis=1).tolist()]
        rows = [padded[i, : lengths[i]] for i in range(batch)]
        values = np.concatenate(rows, axis=0)
        offsets = _offsets_from_lengths_np(lengths)
    return Array(values=values, offsets=offsets, ragged_dim=0)


def from_cu_seqlens(values: Any, cu_seqlens: Any) -> Array:
    """Wrap FlashAttention-style ``(values, cu_seqlens)``; zero-copy."""
    return Array(values=values, offsets=cu_seqlens, ragged_dim=0)
