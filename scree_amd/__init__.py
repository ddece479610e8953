"""scree_amd -- scree's varlen kernel path, native to AMD Instinct MI355X (gfx950).

The package keeps the reference's value type and constructors
(``src/scree/__init__.py:3-21``): :class:`Array`, :func:`pack`,
:func:`unpack`, :func:`to_padded`, :func:`from_padded`,
:func:`from_cu_seqlens`.  The kernels live in :mod:`scree_amd.kernels`
(Array level) and :mod:`scree_amd.kernels.hip` (tensor level, the
counterpart of ``scree.kernels.triton``).
"""

from ._core import Array, from_cu_seqlens, from_padded, pack, to_padded, unpack

__version__ = "0.1.0"

__all__ = [
    "Array",
    "pack",
    "unpack",
    "to_padded",
    "from_padded",
    "from_cu_seqlens",
    "__version__",
]
