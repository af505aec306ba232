"""torchpairwise for MI355X (gfx950): the pairwise-metric ops of inspiros/torchpairwise,
registered under the same ``torch.ops.torchpairwise`` schemas and served by hand-written HIP
kernels on the GPU.

``import torchpairwise_amd as torchpairwise`` gives the reference's module surface
(``torchpairwise/__init__.py:1-8``, ``ops/metrics/pairwise.py:4-47``): every metric name as
an attribute equal to ``torch.ops.torchpairwise.<name>``, plus ``has_ops``, ``with_cuda``,
``cuda_version`` and ``cuda_arch_list``.  ``torchpairwise_amd.packed`` / ``PackedBool`` add a
persistent bit-packed boolean format for repeated boolean-metric calls.
"""
from .extension import _HAS_OPS, cuda_arch_list, cuda_version, has_ops, with_cuda  # noqa: F401

if not _HAS_OPS:
    raise RuntimeError("Couldn't load custom C++ ops of torchpairwise_amd "
                       "(build them with `python torchpairwise_amd/_build.py`).")

from .ops import *  # noqa: E402,F401,F403
from .ops import __all__ as _ops_all  # noqa: E402
from . import packed  # noqa: E402,F401
from .packed import PackedBool  # noqa: E402,F401

__version__ = "0.3.0+mi355x"
__all__ = ["has_ops", "with_cuda", "cuda_version", "cuda_arch_list", *_ops_all]
