"""Loads the native parts (reference: torchpairwise/extension.py:17-192).

The kernel library ``libtorchpairwise_hip.so`` is loaded first (its C ABI is what the
extension calls), then ``_C.so`` through ``torch.ops.load_library``, which runs the static
schema registrations.  A missing or broken build leaves ``_HAS_OPS`` False and the package
import fails loudly (there is no Python or CPU fallback for the GPU path).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
_HIP_LIB = _PKG / "libtorchpairwise_hip.so"
_EXT_LIB = _PKG / "_C.so"
_LOAD_ERROR: Exception | None = None


def _load() -> bool:
    global _LOAD_ERROR
    try:
        # RTLD_GLOBAL so _C.so resolves the tpw_* symbols against this exact file
        ctypes.CDLL(str(_HIP_LIB), mode=ctypes.RTLD_GLOBAL)
        torch.ops.load_library(str(_EXT_LIB))
        return True
    except (OSError, RuntimeError) as e:  # not built, or built for another torch
        _LOAD_ERROR = e
        return False


_HAS_OPS = _load()


def has_ops() -> bool:
    return _HAS_OPS


def _assert_has_ops() -> None:
    if not has_ops():
        raise RuntimeError(f"torchpairwise_amd native ops are not available: {_LOAD_ERROR}")


def cuda_version() -> int:
    """HIP runtime version the kernels were built against (reference: CUDA_VERSION or -1)."""
    if not _HAS_OPS:
        return -1
    return torch.ops.torchpairwise._cuda_version()


def with_cuda() -> bool:
    """True when the GPU kernels are built in (reference: extension.py:179-183)."""
    return cuda_version() != -1


def cuda_arch_list() -> list[str]:
    if not _HAS_OPS:
        return []
    return torch.ops.torchpairwise._cuda_arch_flags().split()
