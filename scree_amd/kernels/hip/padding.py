"""Packed <-> padded conversions on the HIP kernels.

Device counterparts of ``scree.to_padded`` / ``scree.from_padded``
(``src/scree/_core.py:161-301``), whose torch branch copies one slice per
sequence in a host loop and reads each mask row's length with ``.item()``.
Here ``to_padded_hip`` is one launch (after a single host read of the
offsets to size the output, skipped when the caller passes ``max_len``) and
``from_padded_hip`` is a count/scan launch, one host read of the total
(skipped when the caller passes ``total``), and one gather launch.  Semantics follow the
reference exactly: ``mask`` True on valid rows; left or right padding;
``from_padded`` takes the first ``mask[i].sum()`` rows of each batch row
(right padding assumed, ``_core.py:269-285``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _ffi


def _row_bytes(t, lead):
    n = 1
    for s in t.shape[lead:]:
        n *= int(s)
    return n * t.element_size()


def _fill_bytes(fill_value, dtype):
    """The fill element's bytes, converted exactly as ``torch.full`` would."""
    b = torch.full((1,), fill_value, dtype=dtype).view(torch.uint8).numpy().tobytes()
    return ctypes.create_string_buffer(b, len(b)), len(b)


def to_padded_hip(values, offsets, side="right", fill_value=0.0, max_len=None):
    """``(padded, mask)`` for packed ``values`` (N, *features) with int32 ``offsets``.

    ``padded`` is ``(B, max_len, *features)`` in ``values.dtype``; ``mask`` is
    bool ``(B, max_len)``, True on valid rows.  ``max_len`` defaults to the
    longest sequence (one host read of the offsets).
    """
    assert values.is_cuda, "to_padded on HIP requires ROCm device tensors"
    if side not in ("right", "left"):
        raise ValueError(f"side must be 'right' or 'left', got {side!r}")
    off = offsets.to(device=values.device, dtype=torch.int32).contiguous()
    batch = off.numel() - 1
    assert batch >= 1, "offsets must have batch + 1 entries"
    if max_len is None:
        host = off.cpu()
        max_len = int((host[1:] - host[:-1]).max()) if batch > 0 else 0
    feat = tuple(values.shape[1:])
    vals = values.contiguous()
    padded = torch.empty((batch, max_len, *feat), dtype=vals.dtype, device=vals.device)
    mask = torch.empty((batch, max_len), dtype=torch.bool, device=vals.device)
    fill, elem = _fill_bytes(fill_value, vals.dtype)
    with _ffi.device_guard(vals.device):
        _ffi.check(_ffi.lib().scree_to_padded(
            _ffi.ptr(vals), _ffi.ptr(off), batch, vals.shape[0], max_len, _row_bytes(vals, 1),
            1 if side == "left" else 0, ctypes.cast(fill, ctypes.c_void_p), elem,
            _ffi.ptr(padded), _ffi.ptr(mask), _ffi.stream_of(vals)))
    return padded, mask


def from_padded_hip(padded, mask, total=None):
    """``(values, offsets)`` from right-padded ``padded`` (B, T, *features) and ``mask`` (B, T).

    The number of rows of ``values`` is ``mask.sum()``, a device value: it
    is read on the host (one synchronisation, as ``torch.masked_select``
    makes) unless the caller passes it as ``total``.  A ``total`` below the
    true count keeps the first ``total`` rows (the gather clamps every
    sequence to the output, so nothing is written past it), and then
    ``offsets[-1]`` disagrees with ``values.shape[0]``, which
    :class:`scree_amd.Array` rejects.
    """
    assert padded.is_cuda, "from_padded on HIP requires ROCm device tensors"
    batch, t = int(padded.shape[0]), int(padded.shape[1])
    if batch < 1:
        raise ValueError("from_padded needs at least one batch row")
    assert tuple(mask.shape) == (batch, t), f"mask must have shape ({batch}, {t})"
    m = mask.to(device=padded.device, dtype=torch.bool).contiguous()
    pad = padded.contiguous()
    offsets = torch.empty(batch + 1, dtype=torch.int32, device=pad.device)
    with _ffi.device_guard(pad.device):
        _ffi.check(_ffi.lib().scree_padded_offsets(
            _ffi.ptr(m), batch, t, _ffi.ptr(offsets), _ffi.stream_of(pad)))
        if total is None:
            total = int(offsets[-1].item())
        total = int(total)
        if total < 0:
            raise ValueError(f"total must be non-negative, got {total}")
        values = torch.empty((total, *pad.shape[2:]), dtype=pad.dtype, device=pad.device)
        _ffi.check(_ffi.lib().scree_from_padded(
            _ffi.ptr(pad), _ffi.ptr(offsets), batch, t, _row_bytes(pad, 2), total,
            _ffi.ptr(values), _ffi.stream_of(pad)))
    return values, offsets
