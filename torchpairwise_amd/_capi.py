"""ctypes binding of the C ABI in ``include/torchpairwise_amd.h``.

This is a second host of the kernel library next to the PyTorch extension: the GPU
parity tests and the benchmark drive the kernels through it with raw device pointers
(``tensor.data_ptr()``) and the current HIP stream, exactly as a non-Python caller
would.  Every call raises ``RuntimeError`` with ``tpw_last_error()`` on failure.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libtorchpairwise_hip.so"
HEADER = _PKG.parent / "include" / "torchpairwise_amd.h"

TPW_F32, TPW_BF16, TPW_F16, TPW_F64, TPW_I8, TPW_U8, TPW_I16, TPW_I32, TPW_I64 = range(9)
BIT_AND, BIT_OR, BIT_XOR, BIT_EQ, BIT_NE = 0, 1, 2, 3, 4
RED_SUM, RED_MEAN = 0, 1
CMP_LT, CMP_GT, CMP_LE, CMP_GE = 5, 6, 7, 8
EPI_DOT, EPI_EUCLIDEAN, EPI_SQEUCLIDEAN, EPI_COSINE_SIM, EPI_COSINE_DIST, EPI_CORRELATION = 0, 1, 2, 3, 4, 5
KER_POLYNOMIAL, KER_SIGMOID, KER_RBF, KER_LAPLACIAN = 0, 1, 2, 3
FAM_PPMINKOWSKI, FAM_WMINKOWSKI, FAM_CANBERRA, FAM_BRAYCURTIS, FAM_CHI2, FAM_JS = 0, 1, 2, 3, 4, 5

_i64, _p, _i, _d, _sz = C.c_int64, C.c_void_p, C.c_int, C.c_double, C.c_size_t

_SIGNATURES = {
    "tpw_last_error": (C.c_char_p, []),
    "tpw_runtime_version": (_i, []),
    "tpw_launch_timer_arm": (_i, [C.c_char_p, _i]),
    "tpw_launch_timer_read": (_i, [_p, _i, _p, _p]),
    "tpw_empty_launches": (_i, [_i, _p]),
    "tpw_packed_words": (_i64, [_i64]),
    "tpw_pack_bool_rows": (_i, [_p, _i64, _i64, _p, _p, _p]),
    "tpw_bool_pairwise_reduce": (_i, [_p, _p, _i64, _i64, _i64, _i64, _i, _i, _p, _p]),
    "tpw_bool_pairwise_reduce_counted": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _i, _p, _p]),
    "tpw_jaccard_bool": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_bool_count_metric": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _p, _p]),
    "tpw_bool_row_counts": (_i, [_p, _i64, _i64, _p, _p]),
    "tpw_bool_bytes_reduce": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _i, _p, _p]),
    "tpw_bool_bytes_count_metric": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _p, _p]),
    "tpw_bool_fp4_row_bytes": (_i64, [_i64]),
    "tpw_pack_bool_fp4": (_i, [_p, _i64, _i64, _p, _p, _p]),
    "tpw_bool_fp4_reduce": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _i, _p, _p]),
    "tpw_bool_fp4_count_metric": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, _p, _p]),
    "tpw_count_division_check": (_i, [_i64, _i64, _i64, _i64, _p, _p]),
    "tpw_compare_reduce": (_i, [_p, _p, _i, _i64, _i64, _i64, _i64, _i, _i, _p, _p]),
    "tpw_row_norms": (_i, [_p, _i, _i64, _i64, _i, _p, _p]),
    "tpw_pairwise_inner": (_i, [_p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _i, _p, _p]),
    "tpw_radius_mask_euclidean": (_i, [_p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, C.c_float, _p, _p]),
    "tpw_pairwise_exp_kernel": (_i, [_p, _p, _i64, _i64, _i64, _i64, _i, C.c_float, _p, _p]),
    "tpw_pairwise_exp_kernel_backward_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "tpw_pairwise_exp_kernel_backward": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i, C.c_float, _p, _p, _p, _p]),
    "tpw_pairwise_kernel": (_i, [_p, _p, _i, _i64, _i64, _i64, _i64, _i, C.c_float, C.c_float, _i, _p, _p]),
    "tpw_pairwise_kernel_backward": (_i, [_p, _p, _p, _p, _i, _i64, _i64, _i64, _i64, _i, C.c_float,
                                          C.c_float, _i, _p, _p, _p, _p]),
    "tpw_lp_distances": (_i, [_p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_lp_distances_bf16": (_i, [_p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_snr_centered": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_lp_backward_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "tpw_lp_distances_backward": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _d, _i, _p, _p, _p]),
    "tpw_lp_distances_backward2": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p, _p, _p]),
    "tpw_inner_backward_workspace_size": (_sz, [_i64, _i64, _i64, _i64]),
    "tpw_euclidean_backward": (_i, [_p, _p, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_sqeuclidean_backward": (_i, [_p, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_cosine_backward": (_i, [_p, _p, _p, _p, _p, _p, _i, _i64, _i64, _i64, _i64, _i, _p, _p, _p, _p]),
    "tpw_linear_backward": (_i, [_p, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_sqmahalanobis_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "tpw_sqmahalanobis": (_i, [_p, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "tpw_prf_div": (_i, [_p, _p, _i, _i64, _i, _p, _p]),
    "tpw_prf_div_backward": (_i, [_p, _p, _p, _i, _i64, _i, _p, _p, _p]),
    "tpw_prf_div_scalar": (_i, [_p, _d, _i, _i64, _i, _i, _p, _p]),
    "tpw_prf_div_scalar_backward": (_i, [_p, _p, _d, _i, _i64, _i, _i, _p, _p]),
    "tpw_hausdorff_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "tpw_directed_hausdorff": (_i, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p]),
    "tpw_hausdorff_counters": (_i, [_i, _p]),
    "tpw_directed_hausdorff_noalloc": (_i, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "tpw_directed_hausdorff_backward": (_i, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "tpw_row_smallest_mask": (_i, [_p, _i, _i64, _i64, _i64, _p, _p]),
    "tpw_ppminkowski": (_i, [_p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_wminkowski": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_canberra": (_i, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_braycurtis": (_i, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_family_backward_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "tpw_ppminkowski_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p, _p, _p]),
    "tpw_wminkowski_backward": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p, _p, _p, _p]),
    "tpw_canberra_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_braycurtis_backward": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_additive_chi2": (_i, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_sqjensenshannon": (_i, [_p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_additive_chi2_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_sqjensenshannon_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p, _p, _p]),
    "tpw_haversine_workspace_size": (_sz, [_i64, _i64, _i64]),
    "tpw_haversine": (_i, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "tpw_haversine_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p]),
    "tpw_knn_mask_euclidean_supported": (_i, [_i, _i64, _i64, _i64, _i64]),
    "tpw_knn_mask_workspace_size": (_sz, [_i64, _i64, _i64]),
    "tpw_knn_mask_euclidean": (_i, [_p, _p, _i, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _p]),
    "tpw_pairwise_binary": (_i, [_p, _p, _i, _i, _i64, _i64, _i64, _i64, _p, _p]),
    "tpw_family_f64": (_i, [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p]),
    "tpw_family_f64_backward_workspace_size": (_sz, [_i, _i64, _i64, _i64, _i64, _d]),
    "tpw_family_f64_backward": (_i, [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _d, _p, _p, _p, _p, _p]),
    "tpw_haversine_f64": (_i, [_p, _p, _i64, _i64, _i64, _p, _p]),
    "tpw_haversine_f64_backward": (_i, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "tpw_directed_hausdorff_exact": (_i, [_i, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p,
                                          _p]),
    "tpw_directed_hausdorff_exact_backward": (_i, [_i, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                                   _i64, _p, _p, _p]),
}

_lib = None


def header_symbols(header: Path = HEADER) -> list[str]:
    """Function names declared in the public header."""
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tpw_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run torchpairwise_amd._build")
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"torchpairwise_amd C ABI error {rc}: {lib().tpw_last_error().decode()}")


def call(name: str, *args) -> int:
    rc = getattr(lib(), name)(*args)
    check(rc)
    return rc


# --------------------------------------------------------------------------------------
# torch-tensor conveniences (device tensors only; nothing here falls back to the CPU)
# --------------------------------------------------------------------------------------
class LaunchTimer:
    """Device durations (ms) of every launch of one kernel family made while armed, from HIP
    events recorded on the launch's own stream (``tpw_launch_timer_arm`` / ``_read``)."""

    def __init__(self, family: str, capacity: int):
        self.family, self.capacity = family, capacity

    def arm(self):
        call("tpw_launch_timer_arm", self.family.encode(), self.capacity)
        return self

    def read(self):
        buf = (C.c_float * self.capacity)()
        count, dropped = C.c_int(0), C.c_int(0)
        call("tpw_launch_timer_read", C.cast(buf, C.c_void_p), self.capacity, C.byref(count), C.byref(dropped))
        return [float(buf[i]) for i in range(min(count.value, self.capacity))], dropped.value


class HausdorffCounters:
    """Work of the directed Hausdorff forward calls made while armed (``tpw_hausdorff_counters``):
    read() returns {"pairs": point pairs whose squared distance was evaluated, "cell_tests":
    cell-box tests, "launches": kernel launches}."""

    def arm(self):
        call("tpw_hausdorff_counters", 1, None)
        return self

    def read(self):
        buf = (C.c_ulonglong * 3)()
        call("tpw_hausdorff_counters", 0, C.cast(buf, C.c_void_p))
        return {"pairs": int(buf[0]), "cell_tests": int(buf[1]), "launches": int(buf[2])}


def empty_launches(count: int):
    """`count` empty kernel launches back to back on torch's current stream."""
    call("tpw_empty_launches", count, _stream())


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    import torch

    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_code(t):
    import torch

    if t.dtype == torch.float32:
        return TPW_F32
    if t.dtype == torch.bfloat16:
        return TPW_BF16
    if t.dtype == torch.float16:
        return TPW_F16
    if t.dtype == torch.float64:
        return TPW_F64
    raise TypeError(f"unsupported dtype {t.dtype}")


def _as3(x):
    return x if x.dim() == 3 else x.unsqueeze(0)


def pack_bool(x):
    """x: bool [..., rows, d] cuda -> (words int32 [rows_total, W], popcounts int32)."""
    import torch

    assert x.is_cuda and x.dtype == torch.bool
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    W = lib().tpw_packed_words(d)
    words = torch.empty((rows, W), dtype=torch.int32, device=x.device)
    pops = torch.empty((rows,), dtype=torch.int32, device=x.device)
    call("tpw_pack_bool_rows", _ptr(x.contiguous()), rows, d, _ptr(words), _ptr(pops), _stream())
    return words, pops


def bool_pairwise_reduce(x1, x2, op, reduction):
    import torch

    a, b = _as3(x1), _as3(x2)
    B, n, d = a.shape
    m = b.shape[1]
    wa, _ = pack_bool(a)
    wb, _ = pack_bool(b)
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_bool_pairwise_reduce", _ptr(wa), _ptr(wb), B, n, m, d, op, reduction, _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def jaccard_bool(x1, x2):
    import torch

    a, b = _as3(x1), _as3(x2)
    B, n, d = a.shape
    m = b.shape[1]
    wa, pa = pack_bool(a)
    wb, pb = pack_bool(b)
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_jaccard_bool", _ptr(wa), _ptr(wb), _ptr(pa), _ptr(pb), B, n, m, d, _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def bool_count_metric(x1, x2, metric):
    """A boolean count metric (TPW_BMET_* code) of bool inputs on the packed popcount path."""
    import torch

    a, b = _as3(x1), _as3(x2)
    B, n, d = a.shape
    m = b.shape[1]
    wa, pa = pack_bool(a)
    wb, pb = pack_bool(b)
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_bool_count_metric", _ptr(wa), _ptr(wb), _ptr(pa), _ptr(pb), B, n, m, d, metric, _ptr(out),
         _stream())
    return out if x1.dim() == 3 else out[0]


def count_division_check(o_lo, o_hi, x_step, x_count, device="cuda"):
    """Quotients of the tile kernels' short divide that differ from the IEEE divide (see
    tpw_count_division_check); 0 when the sequence is exact on this domain."""
    import torch

    bad = torch.zeros(1, dtype=torch.int64, device=device)
    call("tpw_count_division_check", o_lo, o_hi, x_step, x_count, _ptr(bad), _stream())
    return int(bad.item())


def bool_row_counts(x):
    """x: bool [..., rows, d] cuda -> int32 [rows_total] set bytes per row."""
    import torch

    assert x.is_cuda and x.dtype == torch.bool
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    counts = torch.empty((rows,), dtype=torch.int32, device=x.device)
    call("tpw_bool_row_counts", _ptr(x.contiguous()), rows, d, _ptr(counts), _stream())
    return counts


def bool_bytes_reduce(x1, x2, op, reduction):
    """The pw{op}_{reduction} of bool inputs on the int8 matrix cores (no packing)."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    ca, cb = bool_row_counts(a), bool_row_counts(b)  # held until the launch is queued
    call("tpw_bool_bytes_reduce", _ptr(a), _ptr(b), _ptr(ca), _ptr(cb), B, n, m, d, op, reduction,
         _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def bool_bytes_count_metric(x1, x2, metric):
    """A boolean count metric (TPW_BMET_* code) of bool inputs on the int8 matrix cores."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    ca, cb = bool_row_counts(a), bool_row_counts(b)  # held until the launch is queued
    call("tpw_bool_bytes_count_metric", _ptr(a), _ptr(b), _ptr(ca), _ptr(cb), B, n, m, d, metric,
         _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def pack_bool_fp4(x):
    """bool [B, rows, d] cuda -> (uint8 [B, rows, row_bytes] fp4 rows, int32 [B * rows] counts)."""
    import torch

    a = _as3(x).contiguous()
    B, rows, d = a.shape
    rb = lib().tpw_bool_fp4_row_bytes(d)
    fp4 = torch.empty((B, rows, rb), dtype=torch.uint8, device=x.device)
    counts = torch.empty((B * rows,), dtype=torch.int32, device=x.device)
    call("tpw_pack_bool_fp4", _ptr(a), B * rows, d, _ptr(fp4), _ptr(counts), _stream())
    return fp4, counts


def bool_fp4_reduce(x1, x2, op, reduction):
    """The pw{op}_{reduction} of bool inputs through the fp4 layout on the scaled matrix cores."""
    import torch

    (fa, ca), (fb, cb) = pack_bool_fp4(x1), pack_bool_fp4(x2)
    B, n, d = _as3(x1).shape
    m = _as3(x2).shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_bool_fp4_reduce", _ptr(fa), _ptr(fb), _ptr(ca), _ptr(cb), B, n, m, d, op, reduction,
         _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def bool_fp4_count_metric(x1, x2, metric):
    """A boolean count metric (TPW_BMET_* code) through the fp4 layout."""
    import torch

    (fa, ca), (fb, cb) = pack_bool_fp4(x1), pack_bool_fp4(x2)
    B, n, d = _as3(x1).shape
    m = _as3(x2).shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_bool_fp4_count_metric", _ptr(fa), _ptr(fb), _ptr(ca), _ptr(cb), B, n, m, d, metric,
         _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


_ELEM_CODES = None


def elem_code(dtype):
    import torch

    global _ELEM_CODES
    if _ELEM_CODES is None:
        _ELEM_CODES = {torch.float32: TPW_F32, torch.bfloat16: TPW_BF16, torch.float16: TPW_F16,
                       torch.float64: TPW_F64, torch.int8: TPW_I8, torch.uint8: TPW_U8,
                       torch.int16: TPW_I16, torch.int32: TPW_I32, torch.int64: TPW_I64}
    return _ELEM_CODES[dtype]


def compare_reduce(x1, x2, op, reduction):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_compare_reduce", _ptr(a), _ptr(b), elem_code(a.dtype), B, n, m, d, op, reduction,
         _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def sqeuclidean_backward(grad, x1, x2):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    g = _as3(grad).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((lib().tpw_inner_backward_workspace_size(B, n, m, d),), dtype=torch.uint8,
                     device=a.device)
    call("tpw_sqeuclidean_backward", _ptr(g), _ptr(a), _ptr(b), _dtype_code(a), B, n, m, d,
         _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
    if x1.dim() == 2:
        return gx1[0], gx2[0]
    return gx1, gx2


def row_norms(x, squared):
    import torch

    x = x.contiguous()
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    out = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    call("tpw_row_norms", _ptr(x), _dtype_code(x), rows, d, int(squared), _ptr(out), _stream())
    return out


def pairwise_inner(x1, x2, epilogue, aux1=None, aux2=None):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    if epilogue in (EPI_EUCLIDEAN, EPI_SQEUCLIDEAN):
        aux1 = row_norms(a, True) if aux1 is None else aux1
        aux2 = row_norms(b, True) if aux2 is None else aux2
    elif epilogue in (EPI_COSINE_SIM, EPI_COSINE_DIST):
        aux1 = row_norms(a, False) if aux1 is None else aux1
        aux2 = row_norms(b, False) if aux2 is None else aux2
    out = torch.empty((B, n, m), dtype=x1.dtype, device=x1.device)
    call("tpw_pairwise_inner", _ptr(a), _ptr(b), _dtype_code(a), B, n, m, d, _ptr(aux1), _ptr(aux2),
         epilogue, _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def lp_distances(x1, x2, p):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=x1.device)
    call("tpw_lp_distances", _ptr(a), _ptr(b), B, n, m, d, float(p), _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def lp_distances_bf16(x1, x2, p):
    """Lp distances of fp32 rows with the output rounded to bf16 by the kernel."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.bfloat16, device=x1.device)
    call("tpw_lp_distances_bf16", _ptr(a), _ptr(b), B, n, m, d, float(p), _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def snr_centered(a, b, v1):
    """v1[i] / sum_k (a[i, k] - b[j, k])^2 for centred rows a, b (fp32)."""
    import torch

    a3, b3 = _as3(a).contiguous(), _as3(b).contiguous()
    B, n, d = a3.shape
    m = b3.shape[1]
    v = v1.reshape(B, n).contiguous()
    out = torch.empty((B, n, m), dtype=torch.float32, device=a.device)
    call("tpw_snr_centered", _ptr(a3), _ptr(b3), _ptr(v), B, n, m, d, _ptr(out), _stream())
    return out if a.dim() == 3 else out[0]


def lp_distances_backward(grad, x1, x2, dist, p):
    """(grad_x1, grad_x2) of lp_distances."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    g, dd = _as3(grad).contiguous(), _as3(dist).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    gx1 = torch.empty_like(a)
    gx2 = torch.empty_like(b)
    ws1 = lib().tpw_lp_backward_workspace_size(B, n, m, d)
    ws2 = lib().tpw_lp_backward_workspace_size(B, m, n, d)
    ws = torch.empty((max(ws1, ws2, 1),), dtype=torch.uint8, device=x1.device)
    call("tpw_lp_distances_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(dd), B, n, m, d, float(p), 0,
         _ptr(gx1), _ptr(ws), _stream())
    call("tpw_lp_distances_backward", _ptr(g), _ptr(b), _ptr(a), _ptr(dd), B, m, n, d, float(p), 1,
         _ptr(gx2), _ptr(ws), _stream())
    if x1.dim() == 2:
        return gx1[0], gx2[0]
    return gx1, gx2


def lp_distances_backward2(grad, x1, x2, dist, p):
    """(grad_x1, grad_x2) of lp_distances from the two-direction entry point."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    g, dd = _as3(grad).contiguous(), _as3(dist).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((max(lib().tpw_lp_backward_workspace_size(B, n, m, d), 1),), dtype=torch.uint8,
                     device=x1.device)
    call("tpw_lp_distances_backward2", _ptr(g), _ptr(a), _ptr(b), _ptr(dd), B, n, m, d, float(p),
         _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
    if x1.dim() == 2:
        return gx1[0], gx2[0]
    return gx1, gx2


def euclidean_backward(grad, x1, x2, res):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    g, r = _as3(grad).contiguous(), _as3(res).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((lib().tpw_inner_backward_workspace_size(B, n, m, d),), dtype=torch.uint8,
                     device=a.device)
    call("tpw_euclidean_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(r), _dtype_code(a), B, n, m, d,
         _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
    if x1.dim() == 2:
        return gx1[0], gx2[0]
    return gx1, gx2


def cosine_backward(grad, x1, x2, similarity=False, out=None):
    """(grad_x1, grad_x2) of the cosine family; with `out` (the forward's output) the weights
    come from it instead of a recomputed x1 . x2^T."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    g = _as3(grad).contiguous()
    o = None if out is None else _as3(out).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    n1, n2 = row_norms(a, False), row_norms(b, False)
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((lib().tpw_inner_backward_workspace_size(B, n, m, d),), dtype=torch.uint8,
                     device=a.device)
    call("tpw_cosine_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(n1), _ptr(n2), _ptr(o), _dtype_code(a), B,
         n, m, d, int(similarity), _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
    if x1.dim() == 2:
        return gx1[0], gx2[0]
    return gx1, gx2


def _as4(x):
    return x if x.dim() == 4 else x.unsqueeze(0)


def directed_hausdorff(x1, x2, perm1=None, perm2=None, noalloc=False):
    """x1 [(batch,) b1, p1, d], x2 [(batch,) b2, p2, d] fp32 -> (out, idx1, idx2); with
    noalloc=True through tpw_directed_hausdorff_noalloc (the library's static scratch)."""
    import torch

    a, b = _as4(x1).contiguous(), _as4(x2).contiguous()
    B, b1, p1, d = a.shape
    b2, p2 = b.shape[1], b.shape[2]
    out = torch.empty((B, b1, b2), dtype=torch.float32, device=a.device)
    i1 = torch.empty((B, b1, b2), dtype=torch.int64, device=a.device)
    i2 = torch.empty((B, b1, b2), dtype=torch.int64, device=a.device)
    q1 = _ptr(None if perm1 is None else perm1.contiguous())
    q2 = _ptr(None if perm2 is None else perm2.contiguous())
    if noalloc:
        call("tpw_directed_hausdorff_noalloc", _ptr(a), _ptr(b), B, b1, p1, b2, p2, d, q1, q2,
             _ptr(out), _ptr(i1), _ptr(i2), _stream())
    else:
        ws = torch.empty((lib().tpw_hausdorff_workspace_size(B, b1, p1, b2, p2, d),), dtype=torch.uint8,
                         device=a.device)
        call("tpw_directed_hausdorff", _ptr(a), _ptr(b), B, b1, p1, b2, p2, d, q1, q2,
             _ptr(out), _ptr(i1), _ptr(i2), _ptr(ws), _stream())
    if x1.dim() == 3:
        return out[0], i1[0], i2[0]
    return out, i1, i2


def directed_hausdorff_exact(x1, x2, perm1=None, perm2=None):
    """tpw_directed_hausdorff_exact on float64 / float32 / float16 clouds -> (out, idx1, idx2)."""
    import torch

    a, b = _as4(x1).contiguous(), _as4(x2).contiguous()
    B, b1, p1, d = a.shape
    b2, p2 = b.shape[1], b.shape[2]
    out = torch.empty((B, b1, b2), dtype=a.dtype, device=a.device)
    i1 = torch.empty((B, b1, b2), dtype=torch.int64, device=a.device)
    i2 = torch.empty((B, b1, b2), dtype=torch.int64, device=a.device)
    q1 = _ptr(None if perm1 is None else perm1.contiguous())
    q2 = _ptr(None if perm2 is None else perm2.contiguous())
    call("tpw_directed_hausdorff_exact", _dtype_code(a), _ptr(a), _ptr(b), B, b1, p1, b2, p2, d, q1, q2,
         _ptr(out), _ptr(i1), _ptr(i2), _stream())
    if x1.dim() == 3:
        return out[0], i1[0], i2[0]
    return out, i1, i2


def directed_hausdorff_exact_backward(grad, x1, x2, out, idx1, idx2):
    import torch

    a, b = _as4(x1).contiguous(), _as4(x2).contiguous()
    g = grad.contiguous().reshape(a.shape[0], a.shape[1], b.shape[1])
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    call("tpw_directed_hausdorff_exact_backward", _dtype_code(a), _ptr(g), _ptr(a), _ptr(b),
         _ptr(out.contiguous()), _ptr(idx1.contiguous()), _ptr(idx2.contiguous()), a.shape[0], a.shape[1],
         a.shape[2], b.shape[1], b.shape[2], a.shape[3], _ptr(gx1), _ptr(gx2), _stream())
    if x1.dim() == 3:
        return gx1[0], gx2[0]
    return gx1, gx2


def family_f64(metric, x1, x2, w=None, p=2.0):
    """tpw_family_f64 on float64 [(batch,) n, d] x [(batch,) m, d]."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    wc = None if w is None else (w if w.dim() == 2 else w.unsqueeze(0)).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float64, device=a.device)
    call("tpw_family_f64", metric, _ptr(a), _ptr(b), _ptr(wc), B, n, m, d, float(p), _ptr(out), _stream())
    return out[0] if x1.dim() == 2 else out


def family_f64_backward(metric, grad, x1, x2, w=None, p=2.0):
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    wc = None if w is None else (w if w.dim() == 2 else w.unsqueeze(0)).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    g = grad.contiguous().reshape(B, n, m)
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    gw = None if wc is None else torch.empty_like(wc)
    ws = torch.empty((lib().tpw_family_f64_backward_workspace_size(metric, B, n, m, d, float(p)),),
                     dtype=torch.uint8, device=a.device)
    call("tpw_family_f64_backward", metric, _ptr(g), _ptr(a), _ptr(b), _ptr(wc), B, n, m, d, float(p),
         _ptr(gx1), _ptr(gx2), _ptr(gw), _ptr(ws), _stream())
    r = [gx1, gx2] if x1.dim() == 3 else [gx1[0], gx2[0]]
    if gw is not None:
        r.append(gw if w.dim() == 2 else gw[0])
    return r


def directed_hausdorff_backward(grad, x1, x2, out, idx1, idx2):
    import torch

    a, b = _as4(x1).contiguous(), _as4(x2).contiguous()
    g = grad.contiguous().reshape(a.shape[0], a.shape[1], b.shape[1])
    o = out.contiguous().reshape(g.shape)
    i1, i2 = idx1.contiguous().reshape(g.shape), idx2.contiguous().reshape(g.shape)
    B, b1, p1, d = a.shape
    b2, p2 = b.shape[1], b.shape[2]
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)  # written whole by the library
    call("tpw_directed_hausdorff_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(o), _ptr(i1), _ptr(i2),
         B, b1, p1, b2, p2, d, _ptr(gx1), _ptr(gx2), _stream())
    if x1.dim() == 3:
        return gx1[0], gx2[0]
    return gx1, gx2


def knn_mask_euclidean(x1, x2, count):
    """tpw_knn_mask_euclidean on [n, d] x [m, d] float32 / bfloat16 -> bool mask [n, m]."""
    import torch

    a, b = x1.contiguous(), x2.contiguous()
    n, d = a.shape
    m = b.shape[0]
    n1, n2 = row_norms(a, True), row_norms(b, True)
    mask = torch.empty((n, m), dtype=torch.bool, device=a.device)
    ws = torch.empty((lib().tpw_knn_mask_workspace_size(n, m, count),), dtype=torch.uint8, device=a.device)
    call("tpw_knn_mask_euclidean", _ptr(a), _ptr(b), _dtype_code(a), n, m, d, _ptr(n1), _ptr(n2), count,
         _ptr(mask), _ptr(ws), _stream())
    return mask


def row_smallest_mask(dist, count):
    """dist [rows, cols] (fp32 / bf16 / fp16) -> bool mask of each row's `count` smallest."""
    import torch

    d = dist.contiguous()
    mask = torch.empty(d.shape, dtype=torch.bool, device=d.device)
    call("tpw_row_smallest_mask", _ptr(d), _dtype_code(d), d.shape[0], d.shape[1], int(count),
         _ptr(mask), _stream())
    return mask


def _as3f(x):
    x = x.contiguous()
    return x if x.dim() == 3 else x.unsqueeze(0)


def family_forward(metric, x1, x2, w=None, p=2.0):
    """The reference's VALU kernels on fp32 [(batch,) n, d] x [(batch,) m, d] inputs.

    ``p`` is the exponent for FAM_PPMINKOWSKI / FAM_WMINKOWSKI and the divisor (2, or
    2 ln base) for FAM_JS."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=a.device)
    if metric == FAM_PPMINKOWSKI:
        call("tpw_ppminkowski", _ptr(a), _ptr(b), B, n, m, d, float(p), _ptr(out), _stream())
    elif metric == FAM_WMINKOWSKI:
        ww = w.contiguous().reshape(B, d)
        call("tpw_wminkowski", _ptr(a), _ptr(b), _ptr(ww), B, n, m, d, float(p), _ptr(out), _stream())
    elif metric == FAM_CANBERRA:
        call("tpw_canberra", _ptr(a), _ptr(b), B, n, m, d, _ptr(out), _stream())
    elif metric == FAM_CHI2:
        call("tpw_additive_chi2", _ptr(a), _ptr(b), B, n, m, d, _ptr(out), _stream())
    elif metric == FAM_JS:
        call("tpw_sqjensenshannon", _ptr(a), _ptr(b), B, n, m, d, float(p), _ptr(out), _stream())
    else:
        call("tpw_braycurtis", _ptr(a), _ptr(b), B, n, m, d, _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def family_backward(metric, grad, x1, x2, w=None, p=2.0, out=None):
    """(grad_x1, grad_x2[, grad_w]) of family_forward."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, d = a.shape
    m = b.shape[1]
    g = grad.contiguous().reshape(B, n, m)
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((max(1, lib().tpw_family_backward_workspace_size(metric, B, n, m, d)),),
                     dtype=torch.uint8, device=a.device)
    if metric == FAM_PPMINKOWSKI:
        call("tpw_ppminkowski_backward", _ptr(g), _ptr(a), _ptr(b), B, n, m, d, float(p), _ptr(gx1),
             _ptr(gx2), _ptr(ws), _stream())
        res = [gx1, gx2]
    elif metric == FAM_WMINKOWSKI:
        ww = w.contiguous().reshape(B, d)
        gw = torch.empty_like(ww)
        o = out.contiguous().reshape(B, n, m)
        call("tpw_wminkowski_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(ww), _ptr(o), B, n, m, d,
             float(p), _ptr(gx1), _ptr(gx2), _ptr(gw), _ptr(ws), _stream())
        res = [gx1, gx2, gw]
    elif metric == FAM_CANBERRA:
        call("tpw_canberra_backward", _ptr(g), _ptr(a), _ptr(b), B, n, m, d, _ptr(gx1), _ptr(gx2),
             _ptr(ws), _stream())
        res = [gx1, gx2]
    elif metric == FAM_CHI2:
        call("tpw_additive_chi2_backward", _ptr(g), _ptr(a), _ptr(b), B, n, m, d, _ptr(gx1),
             _ptr(gx2), _ptr(ws), _stream())
        res = [gx1, gx2]
    elif metric == FAM_JS:
        call("tpw_sqjensenshannon_backward", _ptr(g), _ptr(a), _ptr(b), B, n, m, d, float(p),
             _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
        res = [gx1, gx2]
    else:
        o = out.contiguous().reshape(B, n, m)
        call("tpw_braycurtis_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(o), B, n, m, d, _ptr(gx1),
             _ptr(gx2), _ptr(ws), _stream())
        res = [gx1, gx2]
    if x1.dim() == 2:
        res = [res[0][0], res[1][0]] + ([res[2][0]] if len(res) == 3 else [])
    return tuple(res)


def haversine(x1, x2):
    """Haversine distances of fp32 [(batch,) n, 2] x [(batch,) m, 2] (latitude, longitude)."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, _ = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=a.device)
    ws = torch.empty((lib().tpw_haversine_workspace_size(B, n, m),), dtype=torch.uint8, device=a.device)
    call("tpw_haversine", _ptr(a), _ptr(b), B, n, m, _ptr(out), _ptr(ws), _stream())
    return out if x1.dim() == 3 else out[0]


def haversine_backward(grad, x1, x2):
    """(grad_x1, grad_x2) of haversine."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, _ = a.shape
    m = b.shape[1]
    g = grad.contiguous().reshape(B, n, m)
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((lib().tpw_haversine_workspace_size(B, n, m),), dtype=torch.uint8, device=a.device)
    call("tpw_haversine_backward", _ptr(g), _ptr(a), _ptr(b), B, n, m, _ptr(gx1), _ptr(gx2),
         _ptr(ws), _stream())
    return (gx1, gx2) if x1.dim() == 3 else (gx1[0], gx2[0])


def pairwise_kernel(x1, x2, kind, gamma, coef0=1.0, degree=3):
    """(x1 . x2^T * gamma + coef0)^degree or tanh(...) on [(batch,) n, d] fp32 / bf16 rows."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=x1.dtype, device=x1.device)
    call("tpw_pairwise_kernel", _ptr(a), _ptr(b), _dtype_code(a), B, n, m, d, kind, float(gamma),
         float(coef0), int(degree), _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def pairwise_kernel_backward(grad, x1, x2, out, kind, gamma, coef0=1.0, degree=3):
    """(grad_x1, grad_x2) of pairwise_kernel."""
    import torch

    a, b = _as3(x1).contiguous(), _as3(x2).contiguous()
    B, n, d = a.shape
    m = b.shape[1]
    g = grad.contiguous().reshape(B, n, m)
    o = out.contiguous().reshape(B, n, m) if out is not None else None
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((max(1, lib().tpw_inner_backward_workspace_size(B, n, m, d)),), dtype=torch.uint8,
                     device=a.device)
    call("tpw_pairwise_kernel_backward", _ptr(g), _ptr(a), _ptr(b), _ptr(o) if o is not None else None,
         _dtype_code(a), B, n, m, d, kind, float(gamma), float(coef0), int(degree), _ptr(gx1), _ptr(gx2),
         _ptr(ws), _stream())
    return (gx1, gx2) if x1.dim() == 3 else (gx1[0], gx2[0])


def pairwise_exp_kernel(x1, x2, kind, gamma):
    """exp(-gamma * sqeuclidean) (KER_RBF) or exp(-gamma * L1) (KER_LAPLACIAN), fp32 rows."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, d = a.shape
    m = b.shape[1]
    out = torch.empty((B, n, m), dtype=torch.float32, device=a.device)
    call("tpw_pairwise_exp_kernel", _ptr(a), _ptr(b), B, n, m, d, kind, float(gamma), _ptr(out), _stream())
    return out if x1.dim() == 3 else out[0]


def pairwise_exp_kernel_backward(grad, out, x1, x2, kind, gamma):
    """(grad_x1, grad_x2) of pairwise_exp_kernel's out: the pair gradient (grad * out) * -gamma
    formed inside the backward kernel."""
    import torch

    a, b = _as3f(x1), _as3f(x2)
    B, n, d = a.shape
    m = b.shape[1]
    g = grad.contiguous().reshape(B, n, m)
    o = out.contiguous().reshape(B, n, m)
    gx1, gx2 = torch.empty_like(a), torch.empty_like(b)
    ws = torch.empty((max(1, lib().tpw_pairwise_exp_kernel_backward_workspace_size(kind, B, n, m, d)),),
                     dtype=torch.uint8, device=a.device)
    call("tpw_pairwise_exp_kernel_backward", _ptr(g), _ptr(o), _ptr(a), _ptr(b), B, n, m, d, kind, float(gamma),
         _ptr(gx1), _ptr(gx2), _ptr(ws), _stream())
    return (gx1, gx2) if x1.dim() == 3 else (gx1[0], gx2[0])
