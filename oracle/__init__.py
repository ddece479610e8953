"""CPU oracle for the varlen kernel path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's numpy
branch (``src/scree/kernels/reference/*.py``) plus the closed-form backward
passes and the tile schedule the HIP library builds.  It exists to check the
HIP kernels and to time the CPU baseline.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product path (``scree_amd``) never does and fails loudly when
its HIP library is missing.

Pinning status of every function (how a plausible mistake would be caught):

* ``core.offsets_from_lengths`` -- closed form ``[0, cumsum]`` int32, checked
  bit-exact against the reference's test expectations (``tests/test_core.py``)
  and against ``np.cumsum`` on random lengths.
* ``attention.attention_fwd`` -- the reference's known-answer tests
  (per-sequence textbook softmax, causal first row == v0), brute force in
  fp64 with explicit Python loops on tiny inputs, and
  ``torch.nn.functional.scaled_dot_product_attention`` per sequence.
* ``attention.attention_lse`` -- closed form logsumexp, the invariant
  ``sum_k exp(S - LSE) == 1`` and ``torch.logsumexp``.
* ``attention.attention_bwd`` -- torch autograd through SDPA on the same
  inputs and fp64 central finite differences; invariant ``sum_k dS == 0``.
* grouped-query attention in the three functions above (``k`` / ``v`` with
  fewer heads) -- torch SDPA with ``enable_gqa=True`` and its autograd per
  sequence (a library routine that implements the grouping independently),
  and the special case of one K/V head, where every query head must see the
  same keys.
* ``norms.*_fwd`` -- the reference's known-answer tests, ``F.rms_norm`` /
  ``F.layer_norm``, unit-RMS and zero-mean/unit-variance properties.
* ``norms.*_bwd`` -- torch autograd of ``F.rms_norm`` / ``F.layer_norm`` and
  fp64 finite differences.
* ``norms.round_bf16`` / ``norms.add_rounded`` -- torch's own float32 ->
  bfloat16 conversion and half-precision ``x + r`` on the CPU, bit for bit,
  including ties and values near the rounding boundary.
* ``norms.add_rmsnorm_fwd`` / ``norms.add_rmsnorm_bwd`` -- torch autograd of
  ``h = x + r; F.rms_norm(h)`` in fp64 with gradients arriving at both ``h``
  and ``y``; the unfused composition ``rmsnorm_fwd(add_rounded(...))``.
* ``softmax.varlen_softmax`` -- the reference's two known-answer tests
  (``tests/test_varlen_kernels.py:119-139``: per-sequence rows sum to one,
  per-sequence numpy baseline), ``torch.softmax`` per sequence, and the
  golden vectors (torch fp64).
* ``softmax.varlen_softmax_bwd`` -- torch autograd through ``torch.softmax``
  per sequence and fp64 finite differences; invariant ``sum_rows dx == 0``.
* ``padding.to_padded`` / ``padding.from_padded`` -- the reference's own
  tests restated (shapes, mask sum 17, left-padding mask rows, round trip
  identity, HF 1/0 mask rows; ``tests/test_core.py:58-78``,
  ``tests/test_bridges.py:17-37``), and the index identity
  ``padded[b, lo_b + t] == values[off_b + t]`` checked elementwise.
* ``schedule.build_schedule`` -- brute-force enumeration: every (sequence,
  block) appears exactly once, costs are non-increasing, ties broken by the
  stated key.

No function is "parity unpinned".
"""

from . import attention, core, norms, padding, schedule, softmax  # noqa: F401
