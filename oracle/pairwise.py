"""numpy / torch (CPU) restatements of the reference's hot-path arithmetic.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Citations point into
/root/reference (inspiros/torchpairwise v0.3.0) unless prefixed with "torch/".
"""
from __future__ import annotations

import numpy as np
import torch

F32_EXACT = np.int64(1 << 24)  # a float accumulator of ones stops growing here

BIT_OPS = ("and", "or", "xor", "eq", "ne")


def _as3(x: np.ndarray) -> np.ndarray:
    return x if x.ndim == 3 else x[None]


def _pack_u64(x: np.ndarray) -> np.ndarray:
    """bool [..., d] -> uint64 words [..., ceil(d/64)] (zero padding)."""
    d = x.shape[-1]
    nbytes = (d + 7) // 8
    packed = np.packbits(x.astype(np.uint8), axis=-1, bitorder="little")
    pad = (-nbytes) % 8
    if pad:
        packed = np.concatenate([packed, np.zeros(packed.shape[:-1] + (pad,), np.uint8)], -1)
    return np.ascontiguousarray(packed).view(np.uint64)


def bool_counts(x1: np.ndarray, x2: np.ndarray, op: str, row_block: int = 256) -> np.ndarray:
    """Exact integer count over k of op(x1[b,i,k], x2[b,j,k]) for bool inputs.

    Restates the per-output loop of pairwise_binary_reduction_forward_kernel_impl
    (csrc/ops/cpu/pairwise_binary_kernels.cpp:28-49) with the binary ops of
    common/binary_ops.h (and/or/xor/eq/ne on bool), as integer popcounts.
    """
    a, b = _as3(np.asarray(x1, bool)), _as3(np.asarray(x2, bool))
    d = a.shape[-1]
    pa, pb = _pack_u64(a), _pack_u64(b)
    B, n, m = a.shape[0], a.shape[1], b.shape[1]
    out = np.empty((B, n, m), np.int64)
    base = {"and": np.bitwise_and, "or": np.bitwise_or, "xor": np.bitwise_xor,
            "eq": np.bitwise_xor, "ne": np.bitwise_xor}[op]
    for bb in range(B):
        for i0 in range(0, n, row_block):
            w = base(pa[bb, i0:i0 + row_block, None, :], pb[bb, None, :, :])
            c = np.bitwise_count(w).sum(-1, dtype=np.int64)
            out[bb, i0:i0 + row_block] = d - c if op == "eq" else c
    return out if np.ndim(x1) == 3 else out[0]


def float_accumulated(count: np.ndarray) -> np.ndarray:
    """The reference's float32 accumulator of 1.0f per hit: exact below 2^24, then stuck
    at 2^24 (round-to-nearest-even of 2^24 + 1)."""
    return np.minimum(count, F32_EXACT).astype(np.float32)


def pw_reduce_bool(x1, x2, op: str, reduction: str) -> np.ndarray:
    """pw{op}_{sum,mean} on bool inputs (csrc/ops/pairwise_binary.cpp:135-160;
    sum/mean accumulate in float, Mean divides by float(d):
    csrc/ops/cpu/pairwise_binary_kernels.cpp:40-47, output float32 :146-151)."""
    c = float_accumulated(bool_counts(x1, x2, op))
    if reduction == "sum":
        return c
    d = np.asarray(x1).shape[-1]
    return (c / np.float32(d)).astype(np.float32)


def hamming_distances(x1, x2=None) -> np.ndarray:
    """hamming_distances = pwne_mean (csrc/ops/pairwise_metrics.cpp:206-213).  Bool inputs
    use popcounts; other dtypes compare elementwise with != (no bool coercion)."""
    x2 = x1 if x2 is None else x2
    x1, x2 = np.asarray(x1), np.asarray(x2)
    if x1.dtype == bool and x2.dtype == bool:
        return pw_reduce_bool(x1, x2, "ne", "mean")
    a, b = _as3(x1), _as3(x2)
    cnt = np.stack([(a[bb][:, None, :] != b[bb][None, :, :]).sum(-1) for bb in range(a.shape[0])])
    res = (float_accumulated(cnt) / np.float32(a.shape[-1])).astype(np.float32)
    return res if x1.ndim == 3 else res[0]


def jaccard_distances(x1, x2=None) -> np.ndarray:
    """prf_div(pwxor_sum, pwor_sum, "zero") on bool-coerced inputs
    (csrc/ops/pairwise_metrics.cpp:215-222, pairwise_metrics.h:50-55 coercion,
    csrc/ops/cpu/prf_divide.h:10-11 zero mode)."""
    x2 = x1 if x2 is None else x2
    a, b = np.asarray(x1).astype(bool), np.asarray(x2).astype(bool)
    x = float_accumulated(bool_counts(a, b, "xor"))
    o = float_accumulated(bool_counts(a, b, "or"))
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (x / np.where(o == 0, np.float32(1), o)).astype(np.float32)
    return np.where(o == 0, np.float32(0), q).astype(np.float32)


BOOL_COUNT_METRICS = ("hamming", "jaccard", "dice", "kulczynski1", "kulsinski", "rogerstanimoto",
                      "russellrao", "sokalmichener", "sokalsneath", "yule")


def bool_count_metric(x1, x2, metric: str, gpu_scalar_divide: bool = False) -> np.ndarray:
    """The reference's boolean count metrics as float32 composites over the pw*_sum counts
    (csrc/ops/pairwise_metrics.cpp:206-243,339-399), one numpy float32 rounding per operation
    in the composite's order.  Counts are float accumulators of ones (float_accumulated).
    ``gpu_scalar_divide`` evaluates russellrao's ``/ d`` as ATen's GPU route does (a multiply
    by the float reciprocal of the CPU scalar, torch/aten/src/ATen/native/cuda/
    BinaryDivTrueKernel.cu); the CPU route divides."""
    a, b = np.asarray(x1).astype(bool), np.asarray(x2).astype(bool)
    d = a.shape[-1]
    f = np.float32
    AND = float_accumulated(bool_counts(a, b, "and"))
    XOR = float_accumulated(bool_counts(a, b, "xor"))
    df = f(d)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if metric == "hamming":
            return pw_reduce_bool(a, b, "ne", "mean")
        if metric == "jaccard":
            return jaccard_distances(a, b)
        if metric == "dice":
            return (XOR / (f(2) * AND + XOR)).astype(f)
        if metric == "kulczynski1":
            return (AND / XOR).astype(f)
        if metric == "kulsinski":
            return (((XOR - AND) + df) / (XOR + df)).astype(f)
        if metric in ("rogerstanimoto", "sokalmichener"):
            R = f(2) * XOR
            EQ = float_accumulated(bool_counts(a, b, "eq"))
            return (R / (EQ + R)).astype(f)
        if metric == "russellrao":
            num = (df - AND).astype(f)
            return (num * (f(1) / df) if gpu_scalar_divide else num / df).astype(f)
        if metric == "sokalsneath":
            R = f(2) * XOR
            return (R / (AND + R)).astype(f)
        if metric == "yule":
            n10 = float_accumulated(bool_counts(a, ~b, "and"))
            n01 = float_accumulated(bool_counts(~a, b, "and"))
            n00 = float_accumulated(bool_counts(~a, ~b, "and"))
            hR = (n10 * n01).astype(f)
            den = ((AND * n00).astype(f) + hR).astype(f)
            q = (f(2) * hR / np.where(den == 0, f(1), den)).astype(f)
            return np.where(den == 0, f(0), q).astype(f)
    raise ValueError(metric)


def pack_bool_words(x) -> tuple[np.ndarray, np.ndarray]:
    """Rows of bools -> (uint32 words [..., W], int32 popcounts [...]): bit k at word k // 32,
    bit k % 32, W = ceil(d / 32) rounded up to a multiple of 4, zero padding."""
    x = np.asarray(x, bool)
    d = x.shape[-1]
    W = ((d + 31) // 32 + 3) // 4 * 4
    by = np.packbits(x.astype(np.uint8), axis=-1, bitorder="little")
    full = np.zeros(x.shape[:-1] + (4 * W,), np.uint8)
    full[..., :by.shape[-1]] = by
    words = np.ascontiguousarray(full).view("<u4")
    return words, x.sum(-1).astype(np.int32)


# -------------------------------------------------------------------------------------
# ATen-routed metrics: the reference calls at::cdist, so torch.cdist on CPU is its
# arithmetic (csrc/ops/pairwise_metrics.cpp:24-31 euclidean p=2, :42-49 manhattan p=1,
# :160-168 minkowski p, :299-306 chebyshev p=inf).
# -------------------------------------------------------------------------------------
def cdist_reference(x1: torch.Tensor, x2: torch.Tensor | None, p: float) -> torch.Tensor:
    x1c = x1.detach().cpu().requires_grad_(x1.requires_grad) if x1.is_cuda else x1
    x2 = x1 if x2 is None else x2
    return torch.cdist(x1c, x2, p)


class _PrfDivIdentity(torch.autograd.Function):
    """prf_div(x, y, "identity"): y != 0 ? x / y : x (csrc/ops/cpu/prf_divide.h:12-13);
    backward: g/y and (g/y) * -x / y where y != 0, else g and 0
    (csrc/ops/cpu/prf_div_kernel.cpp:258-277)."""

    @staticmethod
    def forward(ctx, x, y):
        ctx.save_for_backward(x, y)
        nz = y != 0
        return torch.where(nz, x / torch.where(nz, y, torch.ones_like(y)), x)

    @staticmethod
    def backward(ctx, g):
        x, y = ctx.saved_tensors
        nz = y != 0
        ysafe = torch.where(nz, y, torch.ones_like(y))
        gs = g / ysafe
        gx = torch.where(nz, gs, g)
        gy = torch.where(nz, gs * -x / ysafe, torch.zeros_like(g))
        return gx, gy


def prf_div_identity(x, y):
    return _PrfDivIdentity.apply(x, y)


# -------------------------------------------------------------------------------------
# the prf_div family (csrc/ops/prf_div.cpp:359-400; CPU kernels csrc/ops/cpu/prf_div_kernel.cpp)
# elementwise in numpy.  Values ride in float64 carriers; R rounds a float64 result to the
# element type the way the reference's scalar_t arithmetic does: float32 directly (a float64
# quotient or product of float32 values rounds to the same float32 as the float32 operation:
# 53 >= 2 * 24 + 2), float16 / bfloat16 through float32 first, as c10::Half / c10::BFloat16
# compute each operation in float and round the result.
# -------------------------------------------------------------------------------------
def bf16_round(v) -> np.ndarray:
    """float32 -> the nearest bfloat16 (ties to even), returned as float32; NaN -> 0x7fc0."""
    f = np.asarray(v, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(f), np.float32(np.nan), r)


def elem_round(dtype: str):
    """R: float64 carrier -> float64 carrier of the nearest value of `dtype`."""
    def f32(v):
        return np.asarray(v, np.float64).astype(np.float32)
    if dtype == "float64":
        return lambda v: np.asarray(v, np.float64)
    if dtype == "float32":
        return lambda v: f32(v).astype(np.float64)
    if dtype == "float16":
        return lambda v: f32(v).astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        return lambda v: bf16_round(f32(v)).astype(np.float64)
    raise ValueError(dtype)


def prf_divide(x, y, identity: bool, R) -> np.ndarray:
    """y != 0 ? x / y : (identity ? x : 0) (csrc/ops/cpu/prf_divide.h:8-16)."""
    x, y = np.broadcast_arrays(np.asarray(x, np.float64), np.asarray(y, np.float64))
    with np.errstate(all="ignore"):
        q = R(x / np.where(y != 0, y, 1.0))
    return np.where(y != 0, q, x if identity else 0.0)


def prf_div_forward(x, y, identity: bool, R, left: bool = False) -> np.ndarray:
    """prf_div(x, y) / prf_ldiv(x, y) = prf_divide(y, x); either operand may be a scalar
    already rounded to the element type (the Scalar and rScalar forms,
    cpu/prf_div_kernel.cpp:14-54,57-151)."""
    return prf_divide(y, x, identity, R) if left else prf_divide(x, y, identity, R)


def prf_div_backward(g, x, y, identity: bool, R):
    """Gradients of z = x / y, both operands tensors (cpu/prf_div_kernel.cpp:258-277):
    y != 0: gx = g / y, gy = (gx * -x) / y; y == 0: gx = identity ? g : 0, gy = 0."""
    g, x, y = np.broadcast_arrays(*(np.asarray(v, np.float64) for v in (g, x, y)))
    nz = y != 0
    ys = np.where(nz, y, 1.0)
    with np.errstate(all="ignore"):
        gs = R(g / ys)
        gy = R(R(gs * -x) / ys)
    return np.where(nz, gs, g if identity else 0.0), np.where(nz, gy, 0.0)


def prf_div_scalar_divisor_backward(g, c: float, identity: bool, R) -> np.ndarray:
    """gx of z = x / c (cpu/prf_div_kernel.cpp:279-297): c != 0 ? g / c : identity ? g : 0."""
    g = np.asarray(g, np.float64)
    if c != 0:
        with np.errstate(all="ignore"):
            return R(g / c)
    return g.copy() if identity else np.zeros_like(g)


def prf_div_scalar_dividend_backward(g, x, c: float, R) -> np.ndarray:
    """gx of z = c / x (cpu/prf_div_kernel.cpp:298-311): x != 0 ? (g * -c) / (x * x) : 0."""
    g, x = np.broadcast_arrays(np.asarray(g, np.float64), np.asarray(x, np.float64))
    nz = x != 0
    with np.errstate(all="ignore"):
        v = R(R(g * -c) / R(x * x))
    return np.where(nz, v, 0.0)


def cosine_similarity(x1: torch.Tensor, x2: torch.Tensor | None = None) -> torch.Tensor:
    """csrc/ops/pairwise_metrics.cpp:112-122: prf_div(x1 @ x2^T, |x1| |x2|^T, identity);
    with x2=None the second operand and norm alias the first."""
    x2_ = x1 if x2 is None else x2
    n1 = x1.norm(2, -1, keepdim=True)
    n2 = n1 if x2 is None else x2_.norm(2, -1, keepdim=True)
    denom = n1.mul(n2.transpose(-1, -2))
    return prf_div_identity(x1.matmul(x2_.transpose(-1, -2)), denom)


def cosine_distances(x1: torch.Tensor, x2: torch.Tensor | None = None) -> torch.Tensor:
    """csrc/ops/pairwise_metrics.cpp:51-56: cosine_similarity.neg_().add_(1).clip_(0, 2)."""
    return (1 - cosine_similarity(x1, x2)).clip(0, 2)


# -------------------------------------------------------------------------------------
# directed Hausdorff
# -------------------------------------------------------------------------------------
def _as4(x):
    return x if x.ndim == 4 else x[None]


def hausdorff_sqdist_matrix(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """d[m, n] = sum_k (a[m,k] - b[n,k])^2 accumulated k = 0..d-1 in float32 with one
    rounding per operation (no fused multiply-add), as the reference's loop computes it
    (csrc/ops/cpu/hausdorff_kernel.cpp:29-33)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    d = np.zeros((a.shape[0], b.shape[0]), np.float32)
    for k in range(a.shape[1]):
        diff = (a[:, None, k] - b[None, :, k]).astype(np.float32)
        d = (d + (diff * diff).astype(np.float32)).astype(np.float32)
    return d


def directed_hausdorff(x1: np.ndarray, x2: np.ndarray, perm1=None, perm2=None):
    """Brute-force restatement of _directed_hausdorff_forward_kernel_impl
    (csrc/ops/cpu/hausdorff_kernel.cpp:12-53; shuffled :55-100): value sqrt(max_m min_n d),
    x1 index = last m in iteration order whose min equals the max, x2 index = first n in
    iteration order reaching that min; with perms, iteration order m_ -> perm[b][m_] and
    the reported indices are the permuted values.  Inputs [(B,) b1, p1, d] / [(B,) b2, p2, d]
    float32; perms [B, p] int64 or None."""
    a4, b4 = _as4(np.asarray(x1, np.float32)), _as4(np.asarray(x2, np.float32))
    B, b1, p1, _ = a4.shape
    b2, p2 = b4.shape[1], b4.shape[2]
    out = np.zeros((B, b1, b2), np.float32)
    i1 = np.zeros((B, b1, b2), np.int64)
    i2 = np.zeros((B, b1, b2), np.int64)
    for bb in range(B):
        o1 = np.arange(p1) if perm1 is None else np.asarray(perm1)[bb]
        o2 = np.arange(p2) if perm2 is None else np.asarray(perm2)[bb]
        for i in range(b1):
            for j in range(b2):
                if p1 == 0 or p2 == 0:
                    continue
                dmat = hausdorff_sqdist_matrix(a4[bb, i][o1], b4[bb, j][o2])
                mins = dmat.min(1)
                h = mins.max()
                mpos = int(np.nonzero(mins == h)[0][-1])
                npos = int(np.nonzero(dmat[mpos] == mins[mpos])[0][0])
                out[bb, i, j] = np.sqrt(h, dtype=np.float32)
                i1[bb, i, j] = o1[mpos]
                i2[bb, i, j] = o2[npos]
    if np.ndim(x1) == 3:
        return out[0], i1[0], i2[0]
    return out, i1, i2


def directed_hausdorff_backward(grad, x1, x2, out, idx1, idx2):
    """Scatter of _directed_hausdorff_backward_x1/x2_kernel_impl
    (csrc/ops/cpu/hausdorff_kernel.cpp:187-235): grad_x1[b,i,m*,k] += g * diff / out
    summed over j in order (and grad_x2 over i in order), float32 throughout."""
    a4, b4 = _as4(np.asarray(x1, np.float32)), _as4(np.asarray(x2, np.float32))
    B, b1, p1, d = a4.shape
    b2 = b4.shape[1]
    g = np.asarray(grad, np.float32).reshape(B, b1, b2)
    o = np.asarray(out, np.float32).reshape(B, b1, b2)
    m_ = np.asarray(idx1).reshape(B, b1, b2)
    n_ = np.asarray(idx2).reshape(B, b1, b2)
    gx1 = np.zeros_like(a4)
    gx2 = np.zeros_like(b4)
    for bb in range(B):
        for i in range(b1):
            for j in range(b2):
                m, n = m_[bb, i, j], n_[bb, i, j]
                diff = (a4[bb, i, m] - b4[bb, j, n]).astype(np.float32)
                v = ((g[bb, i, j] * diff).astype(np.float32) / o[bb, i, j]).astype(np.float32)
                gx1[bb, i, m] = (gx1[bb, i, m] + v).astype(np.float32)
        for j in range(b2):
            for i in range(b1):
                m, n = m_[bb, i, j], n_[bb, i, j]
                diff = (b4[bb, j, n] - a4[bb, i, m]).astype(np.float32)
                v = ((g[bb, i, j] * diff).astype(np.float32) / o[bb, i, j]).astype(np.float32)
                gx2[bb, j, n] = (gx2[bb, j, n] + v).astype(np.float32)
    if np.ndim(x1) == 3:
        return gx1[0], gx2[0]
    return gx1, gx2


def hausdorff_permutations(batch: int, p1: int, p2: int, generator: torch.Generator):
    """Permutations drawn as the reference draws them: per batch, x1's then x2's, with
    at::randperm_outf(P, generator) (csrc/ops/cpu/hausdorff_kernel.cpp:149-158)."""
    perm1 = torch.empty((batch, p1), dtype=torch.int64)
    perm2 = torch.empty((batch, p2), dtype=torch.int64)
    for b in range(batch):
        perm1[b] = torch.randperm(p1, generator=generator)
        perm2[b] = torch.randperm(p2, generator=generator)
    return perm1, perm2


def k_smallest_mask(dist, count: int) -> np.ndarray:
    """Bool mask of each row's `count` smallest entries of dist [rows, cols].

    The selection of k_neighbors_mask with count = k + 1 (csrc/ops/neighbors.cpp:29-34:
    argsort(1), keep the first k + 1 columns, index_put_ true).  Ordered by a stable
    ascending sort (numpy's comparison order: NaN last, -0 == +0), so ties at the selection
    boundary go to the lower column; the reference's argsort is unstable there and its
    choice is implementation-defined, everywhere else the two sets are the same.
    """
    d = np.asarray(dist)
    if d.dtype not in (np.float32, np.float64):
        d = d.astype(np.float32)
    rows, cols = d.shape
    mask = np.zeros((rows, cols), bool)
    c = min(int(count), cols)
    if c:
        idx = np.argsort(d, axis=1, kind="stable")[:, :c]
        np.put_along_axis(mask, idx, True, axis=1)
    return mask


def radius_mask(dist, epsilon: float) -> np.ndarray:
    """dist <= epsilon (csrc/ops/neighbors.cpp:56-57)."""
    return np.asarray(dist) <= epsilon


# ---------------------------------------------------------------------- VALU family
def _pair_diff(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    return x1.unsqueeze(-2) - x2.unsqueeze(-3)  # [..., n, m, d]


def ppminkowski(x1: torch.Tensor, x2: torch.Tensor, p: float) -> torch.Tensor:
    """sum_k |x1 - x2|^p with no root; p = 0 gives d (the reference fills it), +-inf the
    max / min of |diff| (cpu/ppminkowski_kernel.cpp:13-52,88-114).  Differentiable torch."""
    d = _pair_diff(x1, x2).abs()
    if p == 0:
        return torch.full(d.shape[:-1], float(x1.shape[-1]), dtype=x1.dtype)
    if p == float("inf"):
        return d.amax(-1)
    if p == -float("inf"):
        return d.amin(-1)
    return d.pow(p).sum(-1)


def wminkowski(x1: torch.Tensor, x2: torch.Tensor, w: torch.Tensor, p: float) -> torch.Tensor:
    """(sum_k w_k |x1 - x2|^p)^(1/p); w [d] or [batch, d] (cpu/wminkowski_kernel.cpp:13-60)."""
    d = _pair_diff(x1, x2).abs()
    ww = w if w.dim() == 1 else w[:, None, None, :]
    if p == 0:
        return torch.full(d.shape[:-1], float(x1.shape[-1]), dtype=x1.dtype)
    if p == float("inf"):
        return (d * ww).amax(-1)
    return (d.pow(p) * ww).sum(-1).pow(1.0 / p)


def canberra(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    """sum_k |x1 - x2| / (|x1| + |x2|), 0 / 0 terms skipped (cpu/canberra_kernel.cpp:13-30)."""
    diff = _pair_diff(x1, x2).abs()
    den = x1.abs().unsqueeze(-2) + x2.abs().unsqueeze(-3)
    safe = torch.where(den != 0, den, torch.ones_like(den))
    return torch.where(den != 0, diff / safe, torch.zeros_like(diff)).sum(-1)


def braycurtis(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    """sum_k |x1 - x2| / sum_k |x1 + x2| (cpu/braycurtis_kernel.cpp:13-29)."""
    s = x1.unsqueeze(-2) + x2.unsqueeze(-3)
    return _pair_diff(x1, x2).abs().sum(-1) / s.abs().sum(-1)


# ---------------------------------------------------------------------- remaining custom ops
def additive_chi2(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    """-sum_k (x1 - x2)^2 / (x1 + x2), 0 / 0 terms skipped (cpu/additive_chi2_kernel.cpp:13-30)."""
    nom = x1.unsqueeze(-2) + x2.unsqueeze(-3)
    d = _pair_diff(x1, x2)
    safe = torch.where(nom != 0, nom, torch.ones_like(nom))
    return -torch.where(nom != 0, d * d / safe, torch.zeros_like(d)).sum(-1)


def _rel_entr(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """cpu/rel_entr.h: x log(x / y) for x, y > 0; 0 for x == 0, y >= 0; +inf otherwise."""
    pos = (x > 0) & (y > 0)
    val = torch.where(pos, x * torch.log(torch.where(pos, x, torch.ones_like(x)) /
                                         torch.where(pos, y, torch.ones_like(y))), torch.zeros_like(x))
    return torch.where(pos | ((x == 0) & (y >= 0)), val, torch.full_like(x, float("inf")))


def sqjensenshannon(x1: torch.Tensor, x2: torch.Tensor, base: float | None = None) -> torch.Tensor:
    """sum_k rel_entr(a, m) + rel_entr(b, m), m = (a + b) / 2, over 2 (or 2 ln base)
    (cpu/sqjensenshannon_kernel.cpp:13-31,74)."""
    a, b = x1.unsqueeze(-2), x2.unsqueeze(-3)
    m = (a + b) / 2
    val = (_rel_entr(a.expand_as(m), m) + _rel_entr(b.expand_as(m), m)).sum(-1)
    return val / (2 * np.log(base) if base is not None else 2.0)


def haversine(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    """2 asin(sqrt(sin^2(dlat/2) + cos lat1 cos lat2 sin^2(dlon/2))) (cpu/haversine_kernel.cpp:22-24)."""
    lat1, lon1 = x1[..., 0].unsqueeze(-1), x1[..., 1].unsqueeze(-1)
    lat2, lon2 = x2[..., 0].unsqueeze(-2), x2[..., 1].unsqueeze(-2)
    v = torch.sin((lat1 - lat2) / 2) ** 2 + torch.cos(lat1) * torch.cos(lat2) * torch.sin((lon1 - lon2) / 2) ** 2
    return 2 * torch.asin(torch.sqrt(v))


def snr(x1: torch.Tensor, x2: torch.Tensor) -> torch.Tensor:
    """V1[i] / DV[i, j]: V1 = sum_k (x1 - mean)^2, DV the same of d = x2[j] - x1[i]
    (cpu/snr_kernel.cpp:13-33,96)."""
    d = -_pair_diff(x1, x2)
    dv = ((d - d.mean(-1, keepdim=True)) ** 2).sum(-1)
    v1 = ((x1 - x1.mean(-1, keepdim=True)) ** 2).sum(-1, keepdim=True)
    return v1 / dv


def sqmahalanobis(x1: torch.Tensor, x2: torch.Tensor, VI: torch.Tensor) -> torch.Tensor:
    """sum_kl d_k VI_kl d_l per pair, directly (cpu/sqmahalanobis_kernel.cpp:13-33)."""
    d = _pair_diff(x1, x2)  # [..., n, m, d]; a batched VI [b, d, d] broadcasts over n
    return ((d @ (VI.unsqueeze(-3) if VI.dim() == 3 else VI)) * d).sum(-1)
