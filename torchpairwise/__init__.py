"""``import torchpairwise`` for this build: the reference package's surface
(torchpairwise/__init__.py:1-8) — ``ops``, ``_ops``, ``extension``, ``__version__``,
``has_ops``, ``with_cuda``, ``cuda_version`` and every op binding of ``torchpairwise.ops`` —
over the native libraries of ``torchpairwise_amd`` (gfx950 HIP kernels + the PyTorch
extension that registers ``torch.ops.torchpairwise``).  Importing fails when they are not
built, as the reference's import fails without its ``_C``."""
from .extension import _HAS_OPS, _assert_has_ops, has_ops, with_cuda, cuda_version  # noqa: F401

_assert_has_ops()

from . import ops  # noqa: E402,F401
from ._ops import _ops  # noqa: E402,F401
from ._version import __version__  # noqa: E402,F401
from .ops import *  # noqa: E402,F401,F403
