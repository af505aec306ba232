"""Loader of the native parts (reference: torchpairwise/extension.py:17-192).

The reference finds ``_C`` next to its package and loads it with ``torch.ops.load_library``.
Here the kernels (``libtorchpairwise_hip.so``) and the schema registrations (``_C.so``) live
in ``torchpairwise_amd/``; ``torchpairwise_amd.extension`` loads both.  The helpers keep the
reference's names and meaning; ``cuda_version`` reports the HIP runtime version the kernels
were built against (the reference: CUDA_VERSION, or -1 without CUDA)."""
from typing import List

from torch._ops import _OpNamespace

from torchpairwise_amd import extension as _native

_HAS_OPS = _native.has_ops()
_ops = _OpNamespace("torchpairwise")


def _has_ops() -> bool:
    return _HAS_OPS


def _assert_has_ops() -> None:
    if not _has_ops():
        raise RuntimeError(
            "Couldn't load custom C++ ops. Build the native libraries with:\n"
            "\tpython torchpairwise_amd/_build.py")


def has_ops() -> bool:
    r"""Check if the C++ extension is loaded."""
    return _HAS_OPS


def cuda_version() -> int:
    r"""The GPU runtime version the extension was built with (-1 if none)."""
    if not _HAS_OPS:
        return -1
    return _ops._cuda_version()


def with_cuda() -> bool:
    r"""Check if the extension was built with GPU kernels."""
    return cuda_version() != -1


def cuda_arch_list() -> List[str]:
    r"""The GPU architectures the kernels were compiled for."""
    if not _HAS_OPS:
        return []
    return _ops._cuda_arch_flags().split()
