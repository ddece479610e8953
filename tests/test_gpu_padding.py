"""GPU packed <-> padded conversions: bit-exact against the oracle (byte work)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import scree_amd
from oracle.padding import from_padded as o_from_padded, to_padded as o_to_padded
from parity import cu_of, say

pytestmark = pytest.mark.gpu

LENGTHS = [0, 1, 7, 64, 3, 0, 130, 2]


def _values(n, feat, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.bool:
        return (torch.rand((n,) + feat, generator=g) > 0.5).cuda()
    if dtype in (torch.int64, torch.int32, torch.uint8):
        return torch.randint(0, 100, (n,) + feat, generator=g).to(dtype).cuda()
    return torch.randn((n,) + feat, generator=g).to(dtype).cuda()


def _bytes_equal(a: torch.Tensor, b: np.ndarray) -> bool:
    """Bitwise equality (NaN fill values compare by their bytes)."""
    a = a.detach().cpu().contiguous()
    if a.dtype == torch.bfloat16:
        return np.array_equal(a.view(torch.int16).numpy(), b.view(np.int16))
    return a.numpy().tobytes() == np.ascontiguousarray(b).tobytes()


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return t.view(torch.int16).numpy().view(np.uint16).view(np.int16) if t.dtype == torch.bfloat16 else t.numpy()


# feature shapes chosen to hit the 16-byte, 4-byte and 1-byte copy paths
CASES = [
    (torch.float32, (4,)), (torch.float32, (3,)), (torch.float16, (8,)), (torch.float16, (3,)),
    (torch.bfloat16, (2, 8)), (torch.int64, (5,)), (torch.bool, (3,)), (torch.uint8, (16,)),
    (torch.float32, ()),
]


@pytest.mark.parametrize("dtype,feat", CASES, ids=lambda v: str(v))
@pytest.mark.parametrize("side", ["right", "left"])
def test_to_padded_bit_exact(dtype, feat, side):
    n = sum(LENGTHS)
    say(f"case: to_padded {dtype} feat={feat} side={side} lengths={LENGTHS}")
    vals = _values(n, feat, dtype, seed=len(feat))
    off, cu = cu_of(LENGTHS)
    fill = True if dtype == torch.bool else (7 if dtype in (torch.int64, torch.uint8) else -3.25)
    arr = scree_amd.Array(values=vals, offsets=cu, ragged_dim=0)
    padded, mask = scree_amd.to_padded(arr, side=side, fill_value=fill)
    rp, rm = o_to_padded(_np(vals), off, side=side, fill_value=fill if dtype != torch.bfloat16 else 0)
    assert padded.shape == rp.shape and padded.dtype == vals.dtype
    assert np.array_equal(mask.cpu().numpy(), rm)
    if dtype == torch.bfloat16:  # oracle on the int16 bit patterns: compare the valid rows, then the fill
        got = _np(padded)
        assert np.array_equal(got[rm], rp[rm])
        fill_bits = torch.tensor([fill], dtype=torch.bfloat16).view(torch.int16).item()
        assert np.all(got[~rm] == fill_bits)
    else:
        assert _bytes_equal(padded, rp)


@pytest.mark.parametrize("dtype,feat", CASES, ids=lambda v: str(v))
def test_roundtrip_and_from_padded_bit_exact(dtype, feat):
    n = sum(LENGTHS)
    vals = _values(n, feat, dtype, seed=7 + len(feat))
    off, cu = cu_of(LENGTHS)
    arr = scree_amd.Array(values=vals, offsets=cu, ragged_dim=0)
    padded, mask = scree_amd.to_padded(arr)
    back = scree_amd.from_padded(padded, mask)
    assert torch.equal(back.offsets, arr.offsets)
    assert back.values.shape == vals.shape
    assert _bytes_equal(back.values, _np(vals))


def test_from_padded_mask_with_holes():
    """The first mask.sum() rows of each batch row are taken, as the reference does."""
    padded = torch.arange(3 * 6 * 2, dtype=torch.float32).reshape(3, 6, 2).cuda()
    mask = torch.tensor([[0, 1, 0, 1, 1, 0], [0] * 6, [1] * 6], dtype=torch.bool).cuda()
    out = scree_amd.from_padded(padded, mask)
    rv, ro = o_from_padded(padded.cpu().numpy(), mask.cpu().numpy())
    assert np.array_equal(out.offsets.cpu().numpy(), ro)
    assert np.array_equal(out.values.cpu().numpy(), rv)


def test_fill_values_nan_and_inf():
    off, cu = cu_of([2, 5])
    vals = _values(7, (4,), torch.float32, 3)
    for fill in (float("nan"), float("-inf")):
        padded, mask = scree_amd.to_padded(scree_amd.Array(values=vals, offsets=cu, ragged_dim=0),
                                           fill_value=fill)
        rp, _ = o_to_padded(vals.cpu().numpy(), off, fill_value=fill)
        assert _bytes_equal(padded, rp)


def test_max_len_below_longest_keeps_first_rows():
    from scree_amd.kernels.hip.padding import to_padded_hip

    off, cu = cu_of([5, 2])
    vals = _values(7, (4,), torch.float32, 4)
    padded, mask = to_padded_hip(vals, cu, max_len=3)
    assert padded.shape == (2, 3, 4)
    assert torch.equal(padded[0], vals[0:3]) and torch.equal(padded[1, :2], vals[5:7])
    assert mask.cpu().tolist() == [[True, True, True], [True, True, False]]


def test_all_empty_and_hf_bridge():
    from scree_amd.bridges import from_hf_padded, to_hf_padded

    off, cu = cu_of([0, 0, 0])
    arr = scree_amd.Array(values=torch.empty(0, 4, device="cuda"), offsets=cu, ragged_dim=0)
    padded, mask = scree_amd.to_padded(arr)
    assert padded.shape == (3, 0, 4) and mask.shape == (3, 0)
    back = scree_amd.from_padded(padded, mask)
    assert back.values.shape == (0, 4) and back.offsets.cpu().tolist() == [0, 0, 0, 0]

    off, cu = cu_of([3, 5, 2])
    arr = scree_amd.Array(values=_values(10, (4,), torch.float16, 5), offsets=cu, ragged_dim=0)
    hidden, am = to_hf_padded(arr)
    assert am.dtype == torch.int64 and int(am.sum()) == 10
    arr2 = from_hf_padded(hidden, am)
    assert torch.equal(arr2.values, arr.values) and torch.equal(arr2.offsets, arr.offsets)


def test_config2_full_size_roundtrip():
    from scree_amd import workloads

    cfg = workloads.config2()
    off, cu = cu_of(cfg.lengths)
    vals = _values(cfg.total, (cfg.hidden,), torch.bfloat16, 6)
    arr = scree_amd.Array(values=vals, offsets=cu, ragged_dim=0)
    padded, mask = scree_amd.to_padded(arr)
    assert padded.shape == (64, max(cfg.lengths), cfg.hidden)
    assert int(mask.sum()) == cfg.total
    assert torch.equal(mask.sum(1).cpu().to(torch.int64), torch.tensor(cfg.lengths))
    back = scree_amd.from_padded(padded, mask)
    assert torch.equal(back.values, vals) and torch.equal(back.offsets, cu)
    # padding rows hold the fill value (0)
    assert int((padded[~mask] != 0).sum()) == 0
