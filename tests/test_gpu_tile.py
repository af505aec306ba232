"""The matrix-core tile kernels (16-byte aligned operands and outputs, output rows of whole
16-byte units, full K chunks) against the kernels the same C entry points take otherwise (here:
operands offset by one element for the inner product, an output offset by one element for the
fp4 metrics and the bit-packed rows): identical inputs, bit-identical outputs, edge tiles and
long K.
The inner-product paths form each dot product from the same MFMA sequence (the tile kernel
with the operands swapped); the boolean counts are exact integers on every path; all of them
finish with the same epilogue functions."""
import ctypes as C

import pytest
import torch

from tests._util import rand, randn
from torchpairwise_amd import _capi as capi

pytestmark = pytest.mark.gpu
DEV = "cuda"

EPIS = [capi.EPI_DOT, capi.EPI_EUCLIDEAN, capi.EPI_SQEUCLIDEAN, capi.EPI_COSINE_SIM,
        capi.EPI_COSINE_DIST, capi.EPI_CORRELATION]


def _inner(x1, x2, epi, misaligned):
    """tpw_pairwise_inner on 16-byte aligned inputs (the tile kernel), or on copies of them
    offset by one element (not 16-byte aligned: the register-staged kernel with element loads);
    the output is aligned either way."""
    B, n, d = x1.shape
    m = x2.shape[1]
    if misaligned:
        s1 = torch.empty(B * n * d + 16, dtype=x1.dtype, device=DEV)
        s2 = torch.empty(B * m * d + 16, dtype=x2.dtype, device=DEV)
        a, b = s1[1:1 + B * n * d].view(B, n, d), s2[1:1 + B * m * d].view(B, m, d)
        a.copy_(x1)
        b.copy_(x2)
    else:
        a, b = x1, x2
    squared = epi in (capi.EPI_EUCLIDEAN, capi.EPI_SQEUCLIDEAN)
    n1 = capi.row_norms(x1, squared) if epi != capi.EPI_DOT else None
    n2 = capi.row_norms(x2, squared) if epi != capi.EPI_DOT else None
    out = torch.empty((B, n, m), dtype=x1.dtype, device=DEV)
    capi.call("tpw_pairwise_inner", C.c_void_p(a.data_ptr()), C.c_void_p(b.data_ptr()), capi._dtype_code(x1),
              B, n, m, d, capi._ptr(n1), capi._ptr(n2), epi, C.c_void_p(out.data_ptr()), capi._stream())
    return out


def _same_bits(a, b):
    ia = a.view(torch.int32) if a.dtype == torch.float32 else a.view(torch.int16)
    ib = b.view(torch.int32) if b.dtype == torch.float32 else b.view(torch.int16)
    return torch.equal(ia, ib)


@pytest.mark.parametrize("dtype,B,n,m,d", [
    (torch.float32, 1, 300, 260, 32),
    (torch.float32, 2, 129, 136, 96),
    (torch.float32, 1, 128, 256, 256),
    (torch.float32, 1, 130, 260, 512),     # 16 chunks: the double-buffered long-K variant
    (torch.bfloat16, 1, 300, 264, 64),
    (torch.bfloat16, 3, 257, 520, 192),
    (torch.bfloat16, 1, 128, 128, 256),
    (torch.bfloat16, 1, 200, 136, 1024),   # long K
    # bf16 ragged rows (m % 8 = 1 .. 7): whole units funnel-shifted, head / tail values
    (torch.bfloat16, 1, 300, 259, 64),
    (torch.bfloat16, 2, 129, 133, 192),
    (torch.bfloat16, 1, 130, 262, 1024),
    (torch.bfloat16, 1, 70, 7, 128),
    (torch.bfloat16, 1, 257, 140, 256),
])
@pytest.mark.parametrize("epi", EPIS)
def test_inner_tile_kernel_equals_staged_kernel(dtype, B, n, m, d, epi):
    x1 = randn(B, n, d, seed=1).to(DEV, dtype)
    x2 = randn(B, m, d, seed=2).to(DEV, dtype)
    x2[:, 3] = 0  # a zero row: the guarded cosine divide
    if m > 7:
        x2[:, 7] = x1[:, 0]  # an identical pair: the clamped euclidean floor
    tile = _inner(x1, x2, epi, False)
    staged = _inner(x1, x2, epi, True)
    assert _same_bits(tile, staged)


def _fp4_metric(x1, x2, metric, misaligned):
    (fa, ca), (fb, cb) = capi.pack_bool_fp4(x1), capi.pack_bool_fp4(x2)
    B, n, d = x1.shape
    m = x2.shape[1]
    store = torch.empty(B * n * m + 16, dtype=torch.float32, device=DEV)
    out = store[1:1 + B * n * m] if misaligned else store[:B * n * m]
    capi.call("tpw_bool_fp4_count_metric", capi._ptr(fa), capi._ptr(fb), capi._ptr(ca), capi._ptr(cb), B, n, m, d,
              metric, C.c_void_p(out.data_ptr()), capi._stream())
    return out.view(B, n, m)


@pytest.mark.parametrize("B,n,m,d", [(1, 300, 260, 100), (2, 129, 136, 1000), (1, 128, 256, 256), (1, 70, 132, 3000),
                                     (1, 130, 131, 1000), (2, 70, 134, 300)])
@pytest.mark.parametrize("metric", range(10))
def test_fp4_tile_kernel_equals_staged_kernel(B, n, m, d, metric):
    x1 = (rand(B, n, d, seed=3) < 0.3).to(DEV)
    x2 = (rand(B, m, d, seed=4) < 0.3).to(DEV)
    x2[:, 0] = False  # an all-zero row: the guarded 0 / 0 cases
    tile = _fp4_metric(x1, x2, metric, False)
    staged = _fp4_metric(x1, x2, metric, True)
    assert torch.equal(torch.nan_to_num(tile, nan=-7.0).view(torch.int32),
                       torch.nan_to_num(staged, nan=-7.0).view(torch.int32))


# --------------------------------------------------------------------------------------
# Bit-packed rows on the fp4 matrix cores (bool_bits_tile_kernel: the count metrics at any d,
# the reductions over more than 256 features) against the popcount kernel the same entry points
# take for an output offset by one element: every count metric, jaccard, and every op x
# reduction of the counted entry; partial last chunks (d = 1 .. 256: one chunk of one or two
# pieces; 257: 3 of 8 pieces; 1500: 2 chunks, the second half full; 2081: 3 chunks, the last
# one piece), edge tiles, ragged output rows (m % 4 != 0).  Bit-identical.
# --------------------------------------------------------------------------------------
def _bits_call(x1, x2, kind, code, misaligned):
    wa, pa = capi.pack_bool(x1)
    wb, pb = capi.pack_bool(x2)
    B, n, d = x1.shape
    m = x2.shape[1]
    store = torch.empty(B * n * m + 16, dtype=torch.float32, device=DEV)
    out = store[1:1 + B * n * m] if misaligned else store[:B * n * m]
    o = C.c_void_p(out.data_ptr())
    if kind == "metric":
        capi.call("tpw_bool_count_metric", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb), B, n, m, d,
                  code, o, capi._stream())
    elif kind == "jaccard":
        capi.call("tpw_jaccard_bool", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb), B, n, m, d, o,
                  capi._stream())
    else:
        op, red = code
        capi.call("tpw_bool_pairwise_reduce_counted", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb),
                  B, n, m, d, op, red, o, capi._stream())
    return out.view(B, n, m)


BITS_CASES = ([("metric", k) for k in range(10)] + [("jaccard", 0)] +
              [("reduce", (op, red)) for op in range(5) for red in range(2)])


@pytest.mark.parametrize("B,n,m,d", [(1, 130, 132, 1), (1, 70, 136, 33), (2, 129, 136, 128), (1, 130, 132, 256),
                                     (1, 300, 260, 257), (2, 129, 136, 1024), (1, 130, 132, 1500),
                                     (1, 70, 132, 2081),
                                     # ragged rows (m % 4 != 0): dword row stores
                                     (1, 130, 131, 1024), (2, 70, 133, 300), (1, 129, 130, 100),
                                     (1, 257, 259, 33), (1, 40, 1, 512)])
@pytest.mark.parametrize("kind,code", BITS_CASES)
def test_bits_tile_kernel_equals_popcount_kernel(B, n, m, d, kind, code):
    x1 = (rand(B, n, d, seed=5) < 0.3).to(DEV)
    x2 = (rand(B, m, d, seed=6) < 0.3).to(DEV)
    x2[:, 0] = False  # an all-zero row: the guarded 0 / 0 cases
    x1[:, 1] = True   # an all-one row
    tile = _bits_call(x1, x2, kind, code, False)
    ref = _bits_call(x1, x2, kind, code, True)
    assert torch.equal(torch.nan_to_num(tile, nan=-7.0).view(torch.int32),
                       torch.nan_to_num(ref, nan=-7.0).view(torch.int32))


# --------------------------------------------------------------------------------------
# fp32 backward on the matrix-core tile kernels: the weights formed inside the grad_x1 product
# (euclidean, sqeuclidean, polynomial, sigmoid; 128 x 256 tiles, two column tiles at d = 300),
# x2 (for grad_x1) and W, x1 (for grad_x2) read k-major in place; inputs offset by one element
# take the weight pass and the split-K GEMM instead.
# Bar: float64 autograd of the reference's composite on the CPU, rtol 1e-4 (+ 1e-4 * max);
# the two device paths agree to 1e-5 * max (different summation orders).
# --------------------------------------------------------------------------------------
BWD_OPS = [("euclidean_distances", {}), ("sqeuclidean_distances", {}), ("cosine_distances", {}),
           ("cosine_similarity", {}), ("correlation_distances", {}),
           ("polynomial_kernel", dict(degree=3, gamma=0.05)), ("sigmoid_kernel", dict(gamma=0.02)),
           ("linear_kernel", {})]


def _leaf(x, misaligned):
    if not misaligned:
        return x.to(DEV).requires_grad_()
    buf = torch.empty(x.numel() + 16, dtype=x.dtype, device=DEV)
    v = buf[1:1 + x.numel()].view(x.shape)
    v.copy_(x)
    return v.requires_grad_()


@pytest.mark.parametrize("B,n,m,d", [(1, 96, 160, 36), (2, 256, 128, 64), (1, 544, 512, 132), (1, 128, 96, 300)])
@pytest.mark.parametrize("name,kw", BWD_OPS)
def test_backward_products_tile_fp32(name, kw, B, n, m, d):
    import torchpairwise_amd as tp
    from tests._util import assert_close

    print(f"{name} {kw} B={B} n={n} m={m} d={d}", flush=True)
    fn = getattr(tp, name)
    x1, x2, g = randn(B, n, d, seed=0), randn(B, m, d, seed=1), randn(B, n, m, seed=2)
    grads = {}
    for misaligned in (False, True):
        a, b = _leaf(x1, misaligned), _leaf(x2, misaligned)
        assert (a.data_ptr() % 16 != 0) == misaligned
        fn(a, b, **kw).backward(g.to(DEV))
        grads[misaligned] = (a.grad.cpu(), b.grad.cpu())
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    fn(ra, rb, **kw).backward(g.double())
    for k, want in enumerate((ra.grad, rb.grad)):
        tile, split = grads[False][k], grads[True][k]
        scale = float(want.abs().max())
        assert_close(tile, want, rtol=1e-4, atol=1e-4 * scale, what=f"{name} grad_x{k + 1} (tile)")
        assert_close(split, want, rtol=1e-4, atol=1e-4 * scale, what=f"{name} grad_x{k + 1} (split-K)")
        assert_close(tile, split.double(), rtol=0, atol=1e-5 * scale, what=f"{name} grad_x{k + 1} tile vs split-K")


# bf16: x2 (for grad_x1) and W, x1 (for grad_x2) read k-major through transposing LDS reads,
# and (euclidean, sigmoid; n % 128 == 0) the weights formed inside the grad_x1 product, against
# the path that inputs offset by one element take (W^T and transposed copies of x1, x2
# written first, and the register-staged kernel for their misaligned X); bar: the bf16 tolerance
# against float64 autograd, 1e-2 (+ 1e-2 * max), and the two device paths within one bf16 ulp of
# each other (2^-7 relative, the ulp of values in [1, 2), + 1e-3 * max).  (1, 128, 65536, 256):
# grad_x2's product (M = 65536, N = 256, K = 128) has 512 tiles of 128 x 256, enough to fill the
# GPU, and takes the 128 x 256 bf16 product kernel
@pytest.mark.parametrize("B,n,m,d", [(2, 128, 192, 64), (1, 1088, 1024, 72), (1, 256, 128, 264), (1, 128, 65536, 256)])
@pytest.mark.parametrize("name", ["euclidean_distances", "cosine_distances", "polynomial_kernel", "sigmoid_kernel"])
def test_backward_products_kmajor_bf16(name, B, n, m, d):
    import torchpairwise_amd as tp
    from tests._util import assert_close

    print(f"{name} bf16 B={B} n={n} m={m} d={d}", flush=True)
    fn = getattr(tp, name)
    kw = {"polynomial_kernel": dict(degree=2, gamma=0.05), "sigmoid_kernel": dict(gamma=0.02)}.get(name, {})
    x1 = randn(B, n, d, seed=0, dtype=torch.bfloat16)
    x2 = randn(B, m, d, seed=1, dtype=torch.bfloat16)
    g = randn(B, n, m, seed=2, dtype=torch.bfloat16)
    grads = {}
    for misaligned in (False, True):
        a, b = _leaf(x1, misaligned), _leaf(x2, misaligned)
        fn(a, b, **kw).backward(g.to(DEV))
        grads[misaligned] = (a.grad.float().cpu(), b.grad.float().cpu())
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    fn(ra, rb, **kw).backward(g.double())
    for k, want in enumerate((ra.grad, rb.grad)):
        kmaj, other = grads[False][k], grads[True][k]
        scale = float(want.abs().max())
        assert_close(kmaj, want, rtol=1e-2, atol=1e-2 * scale, what=f"{name} grad_x{k + 1} (k-major)")
        assert_close(kmaj, other.double(), rtol=2.0 ** -7, atol=1e-3 * scale,
                     what=f"{name} grad_x{k + 1} k-major vs transposed")


# --------------------------------------------------------------------------------------
# Rows that are not whole 128-byte chunks: for outputs of 2^20 entries or more the public
# inner-product ops copy the operands zero-padded to whole chunks and take the tile kernel;
# below that, the staged kernel, which zero-fills its last chunk.  Bit-identical either way.
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,n,m,d", [
    (torch.float32, 1100, 1000, 127), (torch.float32, 1024, 1040, 130), (torch.float32, 1030, 1024, 1),
    (torch.bfloat16, 1030, 1024, 255), (torch.bfloat16, 1024, 1032, 200),
])
@pytest.mark.parametrize("op,epi", [("euclidean_distances", capi.EPI_EUCLIDEAN),
                                    ("cosine_similarity", capi.EPI_COSINE_SIM),
                                    ("linear_kernel", capi.EPI_DOT)])
def test_padded_rows_equal_staged_kernel(dtype, n, m, d, op, epi):
    print(f"padded {op} {dtype} {n}x{m}x{d}", flush=True)
    x1 = randn(1, n, d, seed=11).to(DEV, dtype)
    x2 = randn(1, m, d, seed=12).to(DEV, dtype)
    x2[:, 5] = x1[:, 0]
    got = getattr(torch.ops.torchpairwise, op)(x1[0], x2[0])
    assert _same_bits(got, _inner(x1, x2, epi, True)[0])

