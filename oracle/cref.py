"""ctypes wrapper of oracle/cref.c (built by oracle/Makefile) — TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
LIB = _DIR / "_build" / "liboracle_cref.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} missing: run `make -C oracle` (or __graft_entry__.build())")
        l = C.CDLL(str(LIB))
        p, i64, i = C.c_void_p, C.c_int64, C.c_int
        l.oracle_directed_hausdorff.argtypes = [p, p, i64, i64, i64, i64, i64, i64, p, p, p, p, p, i]
        l.oracle_directed_hausdorff.restype = None
        l.oracle_bool_reduce.argtypes = [p, p, i64, i64, i64, i64, i, i, p, i]
        l.oracle_bool_reduce.restype = None
        l.oracle_jaccard.argtypes = [p, p, i64, i64, i64, i64, p, p, i]
        l.oracle_jaccard.restype = None
        _lib = l
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def directed_hausdorff(x1, x2, perm1=None, perm2=None, threads: int = 1):
    """Early-break restatement of csrc/ops/cpu/hausdorff_kernel.cpp:12-100."""
    a = np.ascontiguousarray(x1, np.float32)
    b = np.ascontiguousarray(x2, np.float32)
    a4 = a if a.ndim == 4 else a[None]
    b4 = b if b.ndim == 4 else b[None]
    B, b1, p1, d = a4.shape
    b2, p2 = b4.shape[1], b4.shape[2]
    q1 = None if perm1 is None else np.ascontiguousarray(perm1, np.int64)
    q2 = None if perm2 is None else np.ascontiguousarray(perm2, np.int64)
    out = np.zeros((B, b1, b2), np.float32)
    i1 = np.zeros((B, b1, b2), np.int64)
    i2 = np.zeros((B, b1, b2), np.int64)
    lib().oracle_directed_hausdorff(_p(a4), _p(b4), B, b1, p1, b2, p2, d, _p(q1), _p(q2),
                                    _p(out), _p(i1), _p(i2), threads)
    if a.ndim == 3:
        return out[0], i1[0], i2[0]
    return out, i1, i2


_OPS = {"and": 0, "or": 1, "xor": 2, "eq": 3, "ne": 4}


def bool_reduce(x1, x2, op: str, mean: bool, threads: int = 1):
    """csrc/ops/cpu/pairwise_binary_kernels.cpp:28-49 on bool bytes."""
    a = np.ascontiguousarray(x1, np.bool_)
    b = np.ascontiguousarray(x2, np.bool_)
    a3 = a if a.ndim == 3 else a[None]
    b3 = b if b.ndim == 3 else b[None]
    B, n, d = a3.shape
    m = b3.shape[1]
    out = np.empty((B, n, m), np.float32)
    lib().oracle_bool_reduce(_p(a3), _p(b3), B, n, m, d, _OPS[op], int(mean), _p(out), threads)
    return out if a.ndim == 3 else out[0]


def jaccard(x1, x2, threads: int = 1):
    """pwxor_sum, pwor_sum, prf_div zero — csrc/ops/pairwise_metrics.cpp:215-222."""
    a = np.ascontiguousarray(x1, np.bool_)
    b = np.ascontiguousarray(x2, np.bool_)
    a3 = a if a.ndim == 3 else a[None]
    b3 = b if b.ndim == 3 else b[None]
    B, n, d = a3.shape
    m = b3.shape[1]
    out = np.empty((B, n, m), np.float32)
    scratch = np.empty((B, n, m), np.float32)
    lib().oracle_jaccard(_p(a3), _p(b3), B, n, m, d, _p(out), _p(scratch), threads)
    return out if a.ndim == 3 else out[0]
