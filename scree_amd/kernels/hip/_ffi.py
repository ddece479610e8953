"""ctypes binding of ``libscree_hip.so`` (C ABI declared in ``include/scree_hip.h``).

The library is built in-tree by ``scree_amd._build`` into ``scree_amd/_lib``.
Loading it needs no GPU; calling into it needs ROCm device tensors.  When the
library is missing or fails to load, :data:`HIP_AVAILABLE` is False and every
entry point raises :class:`HipUnavailableError` -- there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_LIB_PATH = Path(os.environ.get("SCREE_HIP_LIB", Path(__file__).resolve().parents[2] / "_lib" / "libscree_hip.so"))

SCREE_OK = 0
SCREE_ERR_INVALID = -1
SCREE_ERR_UNSUPPORTED = -2
SCREE_ERR_WORKSPACE = -3
SCREE_ERR_HIP = -4

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

# name -> (restype, argtypes); mirrors include/scree_hip.h
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.c_size_t
_SIGNATURES = {
    "scree_abi_version": (_I, []),
    "scree_last_error": (ctypes.c_char_p, []),
    "scree_attn_needs_schedule": (_I, [_I, _L, _I, _I]),
    "scree_attn_workspace_bytes": (_S, [_I, _L, _I]),
    "scree_attn_bwd_workspace_bytes_gqa": (_S, [_I, _L, _I, _I, _I]),
    "scree_attn_schedule": (_I, [_P, _I, _L, _I, _I, _P, _S, _P]),
    "scree_attn_fwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _P, _F, _I, _I, _P, _S, _P]),
    "scree_attn_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _P, _F, _I, _I,
                            _P, _S, _P]),
    "scree_attn_bwd_dq": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _P, _F, _I, _I, _P,
                               _S, _P]),
    "scree_attn_bwd_dkv": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _P, _F, _I, _I, _P,
                                _S, _P]),
    "scree_attn_fwd_gqa": (_I, [_P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _F, _I, _I, _P, _S, _P]),
    "scree_attn_fwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _F, _I, _I, _P]),
    "scree_attn_bwd_gqa": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _F,
                                _I, _I, _P, _S, _P]),
    "scree_attn_bwd_dq_gqa": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _F, _I,
                                   _I, _P, _S, _P]),
    "scree_attn_bwd_dkv_gqa": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _F, _I,
                                    _I, _P, _S, _P]),
    "scree_norm_bwd_workspace_bytes": (_S, [_L, _L]),
    "scree_rmsnorm_fwd": (_I, [_P, _P, _P, _P, _L, _L, _F, _I, _P]),
    "scree_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _L, _L, _I, _P, _S, _P]),
    "scree_layernorm_fwd": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _F, _I, _P]),
    "scree_layernorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _I, _P, _S, _P]),
    "scree_add_rmsnorm_fwd": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _F, _I, _P]),
    "scree_add_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _L, _L, _I, _P, _S, _P]),
    "scree_varlen_softmax": (_I, [_P, _P, _P, _I, _L, _L, _I, _P]),
    "scree_varlen_softmax_bwd": (_I, [_P, _P, _P, _P, _I, _L, _L, _I, _P]),
    "scree_to_padded": (_I, [_P, _P, _I, _L, _L, _L, _I, _P, _I, _P, _P, _P]),
    "scree_padded_offsets": (_I, [_P, _I, _L, _P, _P]),
    "scree_from_padded": (_I, [_P, _P, _I, _L, _L, _L, _P, _P]),
}
EXPORTED = tuple(_SIGNATURES)


class HipUnavailableError(RuntimeError):
    """The HIP library is not built or could not be loaded."""


class ScreeHipError(RuntimeError):
    """The HIP library rejected a call or a launch failed."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[scree_hip {code}] {message}")
        self.code = code


_lib = None
_load_error = None


def _load():
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    try:
        lib = ctypes.CDLL(str(_LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    except OSError as e:  # missing file or unresolved symbols
        _load_error = f"{_LIB_PATH}: {e}"
    except AttributeError as e:
        _load_error = f"{_LIB_PATH}: missing export ({e})"
    return _lib


HIP_AVAILABLE = _load() is not None


def lib():
    if _lib is None:
        raise HipUnavailableError(
            f"scree HIP library unavailable ({_load_error}); build it with "
            "`python -m scree_amd._build`")
    return _lib


def library_path() -> Path:
    return _LIB_PATH


def check(rc: int) -> None:
    if rc == SCREE_OK:
        return
    msg = lib().scree_last_error().decode(errors="replace")
    if rc == SCREE_ERR_INVALID:
        raise ValueError(f"[scree_hip {rc}] {msg}")
    if rc == SCREE_ERR_UNSUPPORTED:
        raise NotImplementedError(f"[scree_hip {rc}] {msg}")
    raise ScreeHipError(rc, msg)


def dtype_code(dtype) -> int:
    import torch

    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.float16:
        return DTYPE_F16
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise NotImplementedError(f"dtype {dtype} not supported by the HIP kernels")


def stream_of(tensor) -> int:
    """The current stream of ``tensor``'s device, as the raw handle the C ABI takes."""
    return _raw_stream(tensor.device.index)


def _raw_stream_public(index: int) -> int:
    import torch

    return torch.cuda.current_stream(index).cuda_stream


def _pick_raw_stream():
    # torch's own accessor for the raw current stream (what its compiled
    # kernels launch on) costs ~0.3 us against ~2 us for the public path
    import torch

    fn = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    return fn if fn is not None else _raw_stream_public


def _raw_stream(index: int) -> int:
    global _raw_stream
    _raw_stream = _pick_raw_stream()
    return _raw_stream(index)


def ptr(tensor) -> int:
    """Device address of ``tensor`` (0 for None); ``c_void_p`` arguments take ints."""
    return 0 if tensor is None else tensor.data_ptr()


_I64_ARRAYS = {}


def int64_array(values):
    n = len(values)
    cls = _I64_ARRAYS.get(n)
    if cls is None:
        cls = _I64_ARRAYS[n] = ctypes.c_int64 * n
    return cls(*values)


def device_guard(device):
    """``torch.cuda.device(device)`` when another device is current, else a no-op
    context (entering the real one costs ~5 us per call)."""
    import contextlib

    import torch

    if device.index is None or torch.cuda.current_device() == device.index:
        return contextlib.nullcontext()
    return torch.cuda.device(device)
