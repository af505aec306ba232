"""GPU parity of every C-ABI entry point against the CPU oracle (same seeded inputs).

Bars: bit-exact for the boolean metrics and for the Hausdorff value, indices and
gradients; floating-point values and gradients within the tolerance stated per test
(fp32: rtol 1e-5 plus an absolute floor scaled to the data; bf16: rtol 1e-2 normwise).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import pairwise as P
from tests._util import assert_close, assert_equal, rand, randn
from torchpairwise_amd import _capi as capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


# --------------------------------------------------------------------------------------
# boolean family: bit-exact
# --------------------------------------------------------------------------------------
BOOL_SHAPES = [
    (1, 1, 1, 1),
    (1, 5, 7, 33),
    (1, 130, 257, 128),
    (3, 64, 200, 1000),
    (2, 129, 127, 31),
    (1, 300, 301, 4096 + 17),
    (2, 70, 1030, 200),   # 32 x 512 tiles: ragged rows and columns, scalar stores (m % 4 != 0)
    (1, 33, 1024, 256),   # 32 x 512 tiles at the 8-word limit, full column tiles
]


@pytest.mark.parametrize("B,n,m,d", BOOL_SHAPES)
@pytest.mark.parametrize("op", ["and", "or", "xor", "eq", "ne"])
def test_bool_reduce_bit_exact(B, n, m, d, op):
    x1 = rand(B, n, d, seed=0) < 0.5
    x2 = rand(B, m, d, seed=1) < 0.3
    code = {"and": capi.BIT_AND, "or": capi.BIT_OR, "xor": capi.BIT_XOR, "eq": capi.BIT_EQ,
            "ne": capi.BIT_NE}[op]
    for red, name in ((capi.RED_SUM, "sum"), (capi.RED_MEAN, "mean")):
        got = capi.bool_pairwise_reduce(x1.to(DEV), x2.to(DEV), code, red)
        want = P.pw_reduce_bool(x1.numpy(), x2.numpy(), op, name)
        assert_equal(got, torch.from_numpy(want), f"pw{op}_{name} {B}x{n}x{m}x{d}")


@pytest.mark.parametrize("B,n,m,d", BOOL_SHAPES)
def test_hamming_matches_c_restatement(B, n, m, d):
    x1 = rand(B, n, d, seed=3) < 0.5
    x2 = rand(B, m, d, seed=4) < 0.5
    got = capi.bool_pairwise_reduce(x1.to(DEV), x2.to(DEV), capi.BIT_NE, capi.RED_MEAN)
    want = cref.bool_reduce(x1.numpy(), x2.numpy(), "ne", True, threads=8)
    assert_equal(got, torch.from_numpy(want), "hamming vs C loop")


@pytest.mark.parametrize("B,n,m,d", BOOL_SHAPES)
def test_jaccard_bit_exact(B, n, m, d):
    x1 = rand(B, n, d, seed=5) < 0.1
    x2 = rand(B, m, d, seed=6) < 0.1
    x1[..., : max(1, n // 7), :] = False  # all-zero rows: or == 0 gives 0
    x2[..., : max(1, m // 5), :] = False
    got = capi.jaccard_bool(x1.to(DEV), x2.to(DEV))
    want = P.jaccard_distances(x1.numpy(), x2.numpy())
    assert_equal(got, torch.from_numpy(want), f"jaccard {B}x{n}x{m}x{d}")
    want_c = cref.jaccard(x1.numpy(), x2.numpy(), threads=8)
    assert_equal(got, torch.from_numpy(want_c), "jaccard vs C passes")


def test_bool_empty_sizes():
    x1 = torch.zeros((0, 16), dtype=torch.bool, device=DEV)
    x2 = torch.zeros((5, 16), dtype=torch.bool, device=DEV)
    out = capi.bool_pairwise_reduce(x1, x2, capi.BIT_NE, capi.RED_MEAN)
    assert out.shape == (0, 5)


# --------------------------------------------------------------------------------------
# inner-product family (MFMA)
# --------------------------------------------------------------------------------------
INNER_SHAPES = [(1, 40, 33, 64), (1, 300, 257, 128), (2, 129, 190, 256), (1, 64, 64, 3),
                (1, 50, 70, 1000)]


@pytest.mark.parametrize("B,n,m,d", INNER_SHAPES)
def test_dot_fp32(B, n, m, d):
    x1, x2 = randn(B, n, d, seed=0), randn(B, m, d, seed=1)
    got = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_DOT)
    want = torch.matmul(x1.double(), x2.double().transpose(-1, -2))
    assert_close(got, want, rtol=1e-5, atol=1e-5 * float(want.abs().max()), what="dot fp32")


@pytest.mark.parametrize("B,n,m,d", INNER_SHAPES)
def test_euclidean_fp32(B, n, m, d):
    x1, x2 = randn(B, n, d, seed=0), randn(B, m, d, seed=1)
    got = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_EUCLIDEAN)
    want = torch.cdist(x1, x2, 2)  # the reference's at::cdist on CPU
    assert_close(got, want, rtol=1e-5, atol=1e-5 * float(want.abs().max()), what="euclidean fp32")


def test_euclidean_self_distance_fp32():
    x = randn(1, 200, 128, seed=7)
    got = capi.pairwise_inner(x.to(DEV), x.to(DEV), capi.EPI_EUCLIDEAN)
    want = torch.cdist(x.double(), x.double(), 2)
    # the |a|^2 + |b|^2 - 2ab expansion (used by at::cdist too) cancels on the diagonal:
    # absolute error ~ sqrt(eps * 2|x|^2) there
    floor = 4 * float(np.sqrt(np.finfo(np.float32).eps * 2 * float((x * x).sum(-1).max())))
    assert_close(got, want, rtol=1e-5, atol=floor, what="euclidean self")


@pytest.mark.parametrize("B,n,m,d", INNER_SHAPES)
def test_cosine_fp32(B, n, m, d):
    x1, x2 = randn(B, n, d, seed=0), randn(B, m, d, seed=1)
    x1[0, 0].zero_()  # zero norm: prf_div identity branch
    got = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_COSINE_DIST)
    want = P.cosine_distances(x1.double(), x2.double())
    assert_close(got, want, rtol=1e-5, atol=2e-6, what="cosine fp32")
    got_s = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_COSINE_SIM)
    want_s = P.cosine_similarity(x1.double(), x2.double())
    assert_close(got_s, want_s, rtol=1e-5, atol=2e-6, what="cosine similarity fp32")


@pytest.mark.parametrize("B,n,m,d", [(1, 300, 257, 128), (2, 129, 190, 256), (1, 33, 65, 100)])
def test_inner_bf16(B, n, m, d):
    x1 = randn(B, n, d, seed=0, dtype=torch.bfloat16)
    x2 = randn(B, m, d, seed=1, dtype=torch.bfloat16)
    for epi, ref in ((capi.EPI_EUCLIDEAN, lambda a, b: torch.cdist(a, b, 2)),
                     (capi.EPI_COSINE_DIST, P.cosine_distances)):
        got = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), epi)
        assert got.dtype == torch.bfloat16
        want = ref(x1.double(), x2.double())
        # bf16 output: one bf16 rounding (2^-9 relative) of an fp32-accumulated result
        assert_close(got.float(), want, rtol=1e-2, atol=1e-2 * float(want.abs().max()),
                     what=f"bf16 epilogue {epi}")


# --------------------------------------------------------------------------------------
# VALU Lp family
# --------------------------------------------------------------------------------------
LP_PS = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.5, float("inf")]


@pytest.mark.parametrize("p", LP_PS)
@pytest.mark.parametrize("B,n,m,d", [(1, 130, 257, 128), (2, 33, 64, 7), (1, 5, 300, 65)])
def test_lp_forward(p, B, n, m, d):
    x1 = rand(B, n, d, seed=0) * 2 - 1
    x2 = rand(B, m, d, seed=1) * 2 - 1
    if p == 0.0:
        x2[:, :, : d // 2] = x1[:, : 1, : d // 2]  # some exact zeros
    got = capi.lp_distances(x1.to(DEV), x2.to(DEV), p)
    want = torch.cdist(x1.double(), x2.double(), p)
    if p == 0.0:
        want = torch.cdist(x1, x2, p)  # counts: exact
        assert_equal(got, want, "p=0 counts")
        return
    assert_close(got, want, rtol=1e-5, atol=1e-6 * float(want.abs().max()), what=f"lp p={p}")


@pytest.mark.parametrize("p", [1.0, 1.5, 2.0, 3.0, 4.5, float("inf")])
@pytest.mark.parametrize("B,n,m,d", [(1, 130, 200, 64), (2, 40, 33, 5), (1, 700, 1100, 70), (1, 7, 9, 5),
                                     (1, 300, 257, 128), (2, 65, 130, 200)])
@pytest.mark.parametrize("entry", ["single", "both"])
def test_lp_backward(p, B, n, m, d, entry):
    print(f"lp backward p={p} {B}x{n}x{m}x{d} {entry}", flush=True)
    x1 = (rand(B, n, d, seed=0) * 2 - 1).double().requires_grad_()
    x2 = (rand(B, m, d, seed=1) * 2 - 1).double().requires_grad_()
    g = randn(B, n, m, seed=2).double()
    dist = torch.cdist(x1, x2, p)
    gx1_ref, gx2_ref = torch.autograd.grad(dist, (x1, x2), g)
    dist32 = capi.lp_distances(x1.detach().float().to(DEV), x2.detach().float().to(DEV), p)
    fn = capi.lp_distances_backward if entry == "single" else capi.lp_distances_backward2
    gx1, gx2 = fn(g.float().to(DEV), x1.detach().float().to(DEV), x2.detach().float().to(DEV), dist32, p)
    for got, want, nm in ((gx1, gx1_ref, "grad_x1"), (gx2, gx2_ref, "grad_x2")):
        # sums over up to 200 signed terms: normwise floor 1e-5 * max|grad|
        assert_close(got, want, rtol=1e-4, atol=1e-5 * float(want.abs().max()) + 1e-6,
                     what=f"lp p={p} {nm}")


def _sign_counts(a, b):
    """sum_j sign(a[i, k] - b[j, k]) with sign(NaN) = 0: the p = 1 gradient for grad = 1."""
    diff = a[:, None, :].astype(np.float64) - b[None, :, :].astype(np.float64)
    return np.nan_to_num(np.sign(diff), nan=0.0).sum(axis=1)


@pytest.mark.parametrize("entry", ["single", "both"])
def test_lp_backward_p1_sign_exact(entry):
    """p = 1 with grad = 1: every gradient is an integer count, exact in fp32, so the
    result must equal sign counts bit for bit.  Ties, neighbours one ulp apart and the
    scalable range's ends (2^-52, 2^52) run on the pre-scaled sign path; tiles and stages
    holding 2^-60, a denormal, 2^60, inf or NaN run on the signf path."""
    n, m, d = 300, 1100, 70
    rng = np.random.default_rng(11)
    a = (rng.integers(-8, 9, size=(n, d)) * 0.125).astype(np.float32)
    b = (rng.integers(-8, 9, size=(m, d)) * 0.125).astype(np.float32)
    one_up = np.nextafter(np.float32(1.0), np.float32(2.0))
    a[140, 0], b[50, 0], b[51, 0], b[52, 0] = 1.0, one_up, 1.0, np.nextafter(np.float32(1), np.float32(0))
    lo, hi = np.float32(2.0 ** -52), np.float32(2.0 ** 52)
    a[150, 1], a[151, 1], b[60, 1], b[61, 1] = lo, -lo, np.nextafter(lo, np.float32(1)), hi
    a[152, 2], b[62, 2], b[63, 2] = hi, np.nextafter(hi, np.float32(0)), -hi
    a[5, 3] = np.float32(2.0 ** -60)              # tile (rows 0-127, features 0-63) off the fast path
    a[200, 66] = np.float32(2.0 ** 60)            # tile (rows 128-255, features 64-69)
    b[330, 10] = np.nan                           # stages holding these values
    b[610, 40] = np.inf
    b[611, 41] = -np.inf
    a[260, 40] = np.inf                           # inf - inf = NaN: sign 0
    b[900, 65] = np.float32(2.0 ** 60)
    b[1000, 2] = np.float32(1e-40)
    b[1001, 2] = np.float32(-1e-40)
    x1, x2 = torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV)
    g = torch.ones(n, m, device=DEV)
    dist = capi.lp_distances(x1, x2, 1.0)
    fn = capi.lp_distances_backward if entry == "single" else capi.lp_distances_backward2
    gx1, gx2 = fn(g, x1, x2, dist, 1.0)
    assert_equal(gx1.cpu(), torch.from_numpy(_sign_counts(a, b).astype(np.float32)), "p=1 grad_x1")
    assert_equal(gx2.cpu(), torch.from_numpy(_sign_counts(b, a).astype(np.float32)), "p=1 grad_x2")


@pytest.mark.parametrize("outside", [False, True])
@pytest.mark.parametrize("entry", ["single", "both"])
def test_lp_backward_p1_wide_gated(entry, outside):
    """p = 1 above 64 features with n, m, d multiples of 4 (here 128): a range scan of x1 and x2
    picks the wide kernel's pre-scaled sign path (every value in the scalable range: ties,
    neighbours one ulp apart and the range's ends 2^-52, 2^52) or, with one value outside
    (`outside`: 2^-60, a denormal, 2^60, inf or NaN), the narrow kernel with its per-tile test;
    both are launched with the same split count.  grad = 1 makes every gradient an integer
    count: sign counts bit for bit either way."""
    n, m, d = 300, 1100, 128
    rng = np.random.default_rng(12)
    a = (rng.integers(-8, 9, size=(n, d)) * 0.125).astype(np.float32)
    b = (rng.integers(-8, 9, size=(m, d)) * 0.125).astype(np.float32)
    one_up = np.nextafter(np.float32(1.0), np.float32(2.0))
    a[140, 0], b[50, 0], b[51, 0], b[52, 0] = 1.0, one_up, 1.0, np.nextafter(np.float32(1), np.float32(0))
    lo, hi = np.float32(2.0 ** -52), np.float32(2.0 ** 52)
    a[150, 1], a[151, 1], b[60, 1], b[61, 1] = lo, -lo, np.nextafter(lo, np.float32(1)), hi
    a[152, 127], b[62, 127], b[63, 127] = hi, np.nextafter(hi, np.float32(0)), -hi
    if outside:
        a[5, 3] = np.float32(2.0 ** -60)
        b[330, 100] = np.nan
        b[610, 40], b[611, 41] = np.inf, -np.inf
        b[1000, 2] = np.float32(1e-40)
    x1, x2 = torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV)
    g = torch.ones(n, m, device=DEV)
    dist = capi.lp_distances(x1, x2, 1.0)
    fn = capi.lp_distances_backward if entry == "single" else capi.lp_distances_backward2
    gx1, gx2 = fn(g, x1, x2, dist, 1.0)
    assert_equal(gx1.cpu(), torch.from_numpy(_sign_counts(a, b).astype(np.float32)), "p=1 grad_x1")
    assert_equal(gx2.cpu(), torch.from_numpy(_sign_counts(b, a).astype(np.float32)), "p=1 grad_x2")


# --------------------------------------------------------------------------------------
# inner-product backward
# --------------------------------------------------------------------------------------
# (2, 96, 160, 36) and (1, 544, 512, 132): fp32 products on the tile kernel with k-major
# operands (n, m multiples of 32), edge tiles, K of 16 chunks and more; (2, 128, 192, 64) and
# (1, 1088, 1024, 72): the same for bf16 (n, m multiples of 64, d of 8)
@pytest.mark.parametrize("B,n,m,d", [(1, 130, 200, 64), (2, 64, 33, 256), (1, 300, 290, 128), (2, 96, 160, 36),
                                     (1, 544, 512, 132), (2, 128, 192, 64), (1, 1088, 1024, 72)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_euclidean_backward(B, n, m, d, dtype):
    x1 = randn(B, n, d, seed=0, dtype=dtype)
    x2 = randn(B, m, d, seed=1, dtype=dtype)
    g = randn(B, n, m, seed=2, dtype=dtype)
    a = x1.double().requires_grad_()
    b = x2.double().requires_grad_()
    res = torch.cdist(a, b, 2)
    gx1_ref, gx2_ref = torch.autograd.grad(res, (a, b), g.double())
    res_dev = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_EUCLIDEAN)
    gx1, gx2 = capi.euclidean_backward(g.to(DEV), x1.to(DEV), x2.to(DEV), res_dev)
    if dtype == torch.float32:  # the derived per-element bound, per batch
        from tests import _gradbound as GB
        for bb in range(B):
            GB.check(gx1[bb].cpu(), gx1_ref[bb], GB.euclidean_grad_bound(x1[bb], x2[bb], g[bb]), "euclidean grad_x1")
            GB.check(gx2[bb].cpu(), gx2_ref[bb], GB.euclidean_grad_bound(x2[bb], x1[bb], g[bb].T),
                     "euclidean grad_x2")
        return
    for got, want, nm in ((gx1, gx1_ref, "grad_x1"), (gx2, gx2_ref, "grad_x2")):
        assert_close(got.float(), want, rtol=1e-2, atol=1e-2 * float(want.abs().max()),
                     what=f"euclidean {dtype} {nm}")


@pytest.mark.parametrize("B,n,m,d", [(1, 130, 200, 64), (2, 64, 33, 256), (2, 96, 160, 36), (1, 544, 512, 132),
                                     (2, 128, 192, 64), (1, 1088, 1024, 72)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("similarity", [False, True])
@pytest.mark.parametrize("from_output", [False, True])
def test_cosine_backward(B, n, m, d, dtype, similarity, from_output):
    """Both routes of the cosine backward: x1 . x2^T recomputed, or the weights formed from the
    forward's output (as autograd passes it)."""
    x1 = randn(B, n, d, seed=0, dtype=dtype)
    x2 = randn(B, m, d, seed=1, dtype=dtype)
    g = randn(B, n, m, seed=2, dtype=dtype)
    a = x1.double().requires_grad_()
    b = x2.double().requires_grad_()
    f = P.cosine_similarity if similarity else P.cosine_distances
    gx1_ref, gx2_ref = torch.autograd.grad(f(a, b), (a, b), g.double())
    out = None
    if from_output:
        out = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_COSINE_SIM if similarity else capi.EPI_COSINE_DIST)
    gx1, gx2 = capi.cosine_backward(g.to(DEV), x1.to(DEV), x2.to(DEV), similarity=similarity, out=out)
    if dtype == torch.float32:  # the derived per-element bound, per batch
        from tests import _gradbound as GB
        for bb in range(B):
            GB.check(gx1[bb].cpu(), gx1_ref[bb], GB.cosine_grad_bound(x1[bb], x2[bb], g[bb], similarity),
                     f"cosine sim={similarity} grad_x1")
            GB.check(gx2[bb].cpu(), gx2_ref[bb], GB.cosine_grad_bound(x2[bb], x1[bb], g[bb].T, similarity),
                     f"cosine sim={similarity} grad_x2")
        return
    rtol = 1e-2
    for got, want, nm in ((gx1, gx1_ref, "grad_x1"), (gx2, gx2_ref, "grad_x2")):
        assert_close(got.float(), want, rtol=rtol, atol=rtol * float(want.abs().max()),
                     what=f"cosine sim={similarity} {dtype} {nm}")


# --------------------------------------------------------------------------------------
# directed Hausdorff: bit-exact value, indices and gradients
# --------------------------------------------------------------------------------------
HD_SHAPES = [(None, 2, 300, 3, 400, 3), (2, 2, 257, 3, 129, 3), (None, 3, 100, 2, 700, 2),
             (None, 2, 150, 3, 90, 5), (None, 1, 1, 1, 1, 3), (None, 2, 2100, 2, 3000, 3),
             (None, 2, 5000, 2, 4100, 1), (None, 1, 4500, 2, 70, 2)]


def _hd_inputs(batch, b1, p1, b2, p2, d, seed=0):
    s1 = (b1, p1, d) if batch is None else (batch, b1, p1, d)
    s2 = (b2, p2, d) if batch is None else (batch, b2, p2, d)
    return rand(*s1, seed=seed), rand(*s2, seed=seed + 1) + 0.05


@pytest.mark.parametrize("shape", HD_SHAPES)
def test_hausdorff_forward_bit_exact(shape):
    x1, x2 = _hd_inputs(*shape)
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    w_out, w_i1, w_i2 = cref.directed_hausdorff(x1.numpy(), x2.numpy(), threads=8)
    assert_equal(out, torch.from_numpy(w_out), "hausdorff value")
    assert_equal(i1, torch.from_numpy(w_i1), "hausdorff x1 index")
    assert_equal(i2, torch.from_numpy(w_i2), "hausdorff x2 index")


def test_hausdorff_shuffled_bit_exact():
    x1, x2 = _hd_inputs(2, 2, 300, 3, 400, 3)
    perm1, perm2 = P.hausdorff_permutations(2, 300, 400, torch.Generator().manual_seed(5))
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV), perm1.to(DEV), perm2.to(DEV))
    w = cref.directed_hausdorff(x1.numpy(), x2.numpy(), perm1.numpy(), perm2.numpy(), threads=8)
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(want), f"shuffled {nm}")


@pytest.mark.parametrize("d", [1, 2, 3])
def test_hausdorff_clustered_bit_exact(d):
    """x2 packed into a few grid cells: the 64-point windows of the cell-sorted scan see only
    that cluster and most m go on to the full scan; x1 spread wide, with a far outlier."""
    g = torch.Generator().manual_seed(30 + d)
    x1 = torch.rand(2, 6000, d, generator=g) * 4.0 - 2.0
    x1[1, 17] = 40.0
    x2 = 0.5 + 1e-3 * torch.rand(3, 9000, d, generator=g)
    x2[0, :10] = torch.rand(10, d, generator=g) * 4.0 - 2.0
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    w_out, w_i1, w_i2 = cref.directed_hausdorff(x1.numpy(), x2.numpy(), threads=8)
    assert_equal(out.cpu(), torch.from_numpy(w_out), f"clustered value d={d}")
    assert_equal(i1.cpu(), torch.from_numpy(w_i1), f"clustered idx1 d={d}")
    assert_equal(i2.cpu(), torch.from_numpy(w_i2), f"clustered idx2 d={d}")


@pytest.mark.parametrize("d", [1, 2, 3])
def test_hausdorff_self_distance_bit_exact(d):
    """x2 = x1: every min is 0 and T stays 0, so no m can be dropped: every m goes through the
    second pass and its full scan, and the tie rules pick the indices."""
    g = torch.Generator().manual_seed(40 + d)
    x = torch.rand(2, 3000, d, generator=g)
    x[:, 100:110] = x[:, 200:210]  # duplicated points
    out, i1, i2 = capi.directed_hausdorff(x.to(DEV), x.to(DEV))
    w_out, w_i1, w_i2 = cref.directed_hausdorff(x.numpy(), x.numpy(), threads=8)
    assert_equal(out.cpu(), torch.from_numpy(w_out), f"self value d={d}")
    assert_equal(i1.cpu(), torch.from_numpy(w_i1), f"self idx1 d={d}")
    assert_equal(i2.cpu(), torch.from_numpy(w_i2), f"self idx2 d={d}")


@pytest.mark.parametrize("shape", [
    (None, 2, 700, 2, 900, 4),      # d = 4: parallel seeds and final rescan, plain scan
    (1100, 1, 40, 1, 50, 2),        # 2200 clouds to sort: one block per cloud
    (None, 64, 65537, 64, 4, 2),    # pairs x p1 > 2^28: x1 unsorted, leftovers in the wave
    (None, 1, 9000, 1, 70000, 3),   # seeds over 3 x1 chunks, rescan over 18 x2 chunks
    (None, 3, 20000, 3, 20000, 3),  # the bench's layout: m with min >= T go to the survivor list
])
def test_hausdorff_plan_variants_bit_exact(shape):
    """The launch plan changes with the sizes: each of these shapes takes another branch."""
    x1, x2 = _hd_inputs(*shape, seed=21)
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    w_out, w_i1, w_i2 = cref.directed_hausdorff(x1.numpy(), x2.numpy(), threads=8)
    assert_equal(out.cpu(), torch.from_numpy(w_out), f"value {shape}")
    assert_equal(i1.cpu(), torch.from_numpy(w_i1), f"idx1 {shape}")
    assert_equal(i2.cpu(), torch.from_numpy(w_i2), f"idx2 {shape}")


@pytest.mark.parametrize("case", ["offset", "flat", "tiny_x2", "one_x2", "shuffled_many_clouds"])
def test_hausdorff_cell_scan_edges_bit_exact(case):
    """Cases aimed at the sorted mode's whole-cell test (an x1 cell's exact box against x2
    points) and its window pass: coordinates far from the origin (rounding of every difference),
    an axis with zero span (one cell along it), x2 clouds of fewer points than the cell test
    takes, and a shuffle through the one-block-per-cloud sort."""
    g = torch.Generator().manual_seed(77)
    perm1 = perm2 = None
    if case == "offset":
        x1 = 1.0e4 + torch.rand(2, 3000, 3, generator=g)
        x2 = 1.0e4 + torch.rand(3, 2500, 3, generator=g) + 0.05
    elif case == "flat":
        x1 = torch.rand(2, 3000, 3, generator=g)
        x2 = torch.rand(2, 2000, 3, generator=g) + 0.05
        x1[..., 2] = 0.25
        x2[..., 2] = 0.25
    elif case == "tiny_x2":
        x1 = torch.rand(2, 2000, 3, generator=g)
        x2 = torch.rand(3, 3, 3, generator=g)
    elif case == "one_x2":
        x1 = torch.rand(2, 1500, 2, generator=g)
        x2 = torch.rand(2, 1, 2, generator=g)
    else:
        x1 = torch.rand(1100, 1, 40, 3, generator=g)
        x2 = torch.rand(1100, 1, 50, 3, generator=g) + 0.05
        perm1, perm2 = P.hausdorff_permutations(1100, 40, 50, torch.Generator().manual_seed(8))
    print(case, tuple(x1.shape), tuple(x2.shape), flush=True)
    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV), dev(perm1), dev(perm2))
    w = cref.directed_hausdorff(x1.numpy(), x2.numpy(), None if perm1 is None else perm1.numpy(),
                                None if perm2 is None else perm2.numpy(), threads=8)
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got.cpu(), torch.from_numpy(want), f"{case} {nm}")


def _hd_nonfinite(case):
    """Inputs holding NaN, +-inf, or coordinates whose squared differences overflow, for each
    launch plan: the sorted mode (d <= 3, few pairs), d = 4 (seeds and scan without the grid),
    d = 5 (the generic scan) and the unsorted cell scan (pairs x p1 > 2^28)."""
    g = torch.Generator().manual_seed(91)
    perm1 = perm2 = None
    x1 = torch.rand(3, 500, 3, generator=g)
    x2 = torch.rand(2, 400, 3, generator=g) + 0.05
    if case == "nan_x1":
        x1[0, 10, 1] = float("nan")
    elif case == "nan_x2":
        x2[1, 7, 0] = float("nan")
    elif case == "nan_x2_last":  # the loop's last s of every row is NaN: no row is folded
        x2[0, -1, 2] = float("nan")
    elif case == "inf_x1":
        x1[1, 33, 0] = float("inf")
    elif case == "ninf_x2":
        x2[0, 5, 1] = float("-inf")
    elif case == "nan_cloud":
        x1[2] = float("nan")
    elif case == "overflow":  # finite inputs, every squared difference +inf
        x1 = x1 * 1e20
        x2 = x2 * -1e20
    elif case == "overflow_rows":  # a few rows whose every squared difference is +inf
        x1[0, 40:43] = 3e38
    elif case in ("mixed_d1", "mixed_d2"):
        d = int(case[-1])
        x1 = torch.rand(2, 300, d, generator=g)
        x2 = torch.rand(2, 200, d, generator=g)
        x1[0, 3, 0] = float("nan")
        x2[1, 9, 0] = float("inf")
    elif case == "batched":  # only batch 1 holds a NaN: batches 0 and 2 keep the pruned path
        x1 = torch.rand(3, 2, 300, 3, generator=g)
        x2 = torch.rand(3, 2, 200, 3, generator=g) + 0.05
        x1[1, 0, 17, 2] = float("nan")
    elif case == "shuffled":
        x1 = torch.rand(2, 2, 300, 3, generator=g)
        x2 = torch.rand(2, 3, 400, 3, generator=g) + 0.05
        x2[0, 1, 50, 0] = float("nan")
        x1[1, 1, 60, 1] = float("-inf")
        perm1, perm2 = P.hausdorff_permutations(2, 300, 400, torch.Generator().manual_seed(6))
    elif case == "d4":
        x1 = torch.rand(2, 700, 4, generator=g)
        x2 = torch.rand(3, 900, 4, generator=g)
        x2[2, 100, 3] = float("inf")
    elif case == "d5":
        x1 = torch.rand(2, 150, 5, generator=g)
        x2 = torch.rand(3, 90, 5, generator=g)
        x1[1, 20, 4] = float("nan")
    elif case == "unsorted_cells":  # batch 1 holds a NaN, batch 0 keeps the pruned path
        x1 = torch.rand(2, 64, 65537, 2, generator=g)
        x2 = torch.rand(2, 64, 4, 2, generator=g)
        x1[1, 5, 1000, 0] = float("nan")
    return x1, x2, perm1, perm2


@pytest.mark.parametrize("case", ["nan_x1", "nan_x2", "nan_x2_last", "inf_x1", "ninf_x2", "nan_cloud", "overflow",
                                  "overflow_rows", "mixed_d1", "mixed_d2", "batched", "shuffled", "d4", "d5",
                                  "unsorted_cells"])
def test_hausdorff_nonfinite_bit_exact(case):
    """NaN and infinities follow the reference's loop: its early exits compare with NaN, a row
    whose last s is NaN is not folded, and a row that never improves on +inf carries the
    previous row's indices.  The pruned kernels cannot reproduce that from the mins alone, so
    a batch with a value that is not finite (or a pair whose winning min is +inf) takes the
    loop itself; the values match bit for bit (NaN at the same positions) and so do the
    indices."""
    x1, x2, perm1, perm2 = _hd_nonfinite(case)
    print(case, tuple(x1.shape), tuple(x2.shape), flush=True)
    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV), dev(perm1), dev(perm2))
    w = cref.directed_hausdorff(x1.numpy(), x2.numpy(), None if perm1 is None else perm1.numpy(),
                                None if perm2 is None else perm2.numpy(), threads=8)
    assert_equal(out.cpu(), torch.from_numpy(w[0]), f"{case} value", nan_payload=False)
    assert_equal(i1.cpu(), torch.from_numpy(w[1]), f"{case} idx1")
    assert_equal(i2.cpu(), torch.from_numpy(w[2]), f"{case} idx2")


def test_hausdorff_counters():
    """The work counters: the kernels evaluate far fewer pairs than brute force, the sorted
    mode's cell scan runs its box tests, the forward of a few clouds is ten launches, and
    counting changes no result."""
    x1, x2 = _hd_inputs(None, 3, 20000, 3, 20000, 3, seed=5)
    a, b = x1.to(DEV), x2.to(DEV)
    plain = capi.directed_hausdorff(a, b)
    c = capi.HausdorffCounters().arm()
    counted = capi.directed_hausdorff(a, b)
    n = c.read()
    print(n, flush=True)
    for got, want, nm in zip(counted, plain, ("value", "idx1", "idx2")):
        assert_equal(got, want, f"counted {nm}")
    pairs = 9
    assert 0 < n["pairs"] < pairs * 20000 * 20000 // 100
    assert 0 < n["cell_tests"] <= pairs * 4096  # one box test per (pair, cell)
    assert n["launches"] == 10
    c2 = capi.HausdorffCounters().arm()
    capi.directed_hausdorff(a, b)
    capi.directed_hausdorff(a, b)
    n2 = c2.read()
    # box tests do not depend on T; the pairs do (T rises as waves fold their mins, in no fixed
    # order), so two calls count about twice as many
    assert n2["launches"] == 20 and n2["cell_tests"] == 2 * n["cell_tests"]
    assert 1.5 * n["pairs"] < n2["pairs"] < 2.5 * n["pairs"]


def test_hausdorff_ties_bit_exact():
    # integer grid points: many equal distances, so the tie rules decide the indices
    g = torch.Generator().manual_seed(11)
    x1 = torch.randint(0, 4, (3, 200, 3), generator=g).float()
    x2 = torch.randint(0, 4, (2, 150, 3), generator=g).float()
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    w = cref.directed_hausdorff(x1.numpy(), x2.numpy(), threads=8)
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(want), f"ties {nm}")
    # identical clouds: value 0, last m, first n
    out, i1, i2 = capi.directed_hausdorff(x1[:1].to(DEV), x1[:1].to(DEV))
    w = cref.directed_hausdorff(x1[:1].numpy(), x1[:1].numpy(), threads=1)
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(want), f"self {nm}")


@pytest.mark.parametrize("shape", [(2, 3, 500, 4, 400, 3), (1, 210, 8192, 210, 8192, 3)])
def test_hausdorff_backward_paths_bit_exact(shape):
    """Both scatter routes of tpw_directed_hausdorff_backward on given outputs and indices (many
    pairs sharing an index, so terms of several pairs meet in one element): a wave per cloud (at
    most 64 clouds per side) and a thread per (cloud, feature) (210 x 210 clouds), each after the
    library's zero fill, into buffers holding garbage, against the reference's scatter loop."""
    B, b1, p1, b2, p2, d = shape
    gen = torch.Generator().manual_seed(17)
    x1 = torch.randn(B, b1, p1, d, generator=gen)
    x2 = torch.randn(B, b2, p2, d, generator=gen)
    out = torch.rand(B, b1, b2, generator=gen) + 0.5
    g = torch.randn(B, b1, b2, generator=gen)
    i1 = torch.randint(0, 3, (B, b1, b2), generator=gen)  # few distinct positions: shared targets
    i2 = torch.randint(0, p2, (B, b1, b2), generator=gen)
    i2[..., 0] = 1
    # device copies held in names: a temporary freed before the launch could be reused
    a, b, gd, od, i1d, i2d = (t.to(DEV) for t in (x1, x2, g, out, i1, i2))
    gx1 = torch.full_like(a, float("nan"))
    gx2 = torch.full_like(b, 7.0)
    capi.call("tpw_directed_hausdorff_backward", capi._ptr(gd), capi._ptr(a), capi._ptr(b), capi._ptr(od),
              capi._ptr(i1d), capi._ptr(i2d), B, b1, p1, b2, p2, d, capi._ptr(gx1), capi._ptr(gx2), capi._stream())
    w1, w2 = P.directed_hausdorff_backward(g.numpy(), x1.numpy(), x2.numpy(), out.numpy(), i1.numpy(), i2.numpy())
    assert_equal(gx1.cpu(), torch.from_numpy(w1).reshape(gx1.shape), f"grad_x1 {shape}")
    assert_equal(gx2.cpu(), torch.from_numpy(w2).reshape(gx2.shape), f"grad_x2 {shape}")


@pytest.mark.parametrize("shape", HD_SHAPES[:4])
def test_hausdorff_backward_bit_exact(shape):
    x1, x2 = _hd_inputs(*shape)
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    g = randn(*out.shape, seed=9)
    gx1, gx2 = capi.directed_hausdorff_backward(g.to(DEV), x1.to(DEV), x2.to(DEV), out, i1, i2)
    w1, w2 = P.directed_hausdorff_backward(g.numpy(), x1.numpy(), x2.numpy(), out.cpu().numpy(),
                                           i1.cpu().numpy(), i2.cpu().numpy())
    assert_equal(gx1, torch.from_numpy(w1), "hausdorff grad_x1")
    assert_equal(gx2, torch.from_numpy(w2), "hausdorff grad_x2")


# --------------------------------------------------------------------------------------
# against the reference's own compiled CPU kernels (oracle/_ref, run in a child process)
# --------------------------------------------------------------------------------------
from oracle import ref_runner  # noqa: E402

needs_ref = pytest.mark.skipif(not ref_runner.available(), reason="oracle/_ref not built")


@needs_ref
def test_hausdorff_gpu_equals_reference_kernels(tmp_path):
    x1, x2 = _hd_inputs(2, 3, 700, 2, 900, 3, seed=21)
    ref = ref_runner.run("hausdorff", {"x1": x1.numpy(), "x2": x2.numpy()}, tmp_path)
    out, i1, i2 = capi.directed_hausdorff(x1.to(DEV), x2.to(DEV))
    for got, key in zip((out, i1, i2), ("out", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(ref[key]), f"vs reference {key}")
    g = randn(*out.shape, seed=22)
    ref = ref_runner.run("hausdorff_backward", {"x1": x1.numpy(), "x2": x2.numpy(), "grad": g.numpy()}, tmp_path)
    gx1, gx2 = capi.directed_hausdorff_backward(g.to(DEV), x1.to(DEV), x2.to(DEV), out, i1, i2)
    assert_equal(gx1, torch.from_numpy(ref["grad_x1"]), "grad_x1 vs reference")
    assert_equal(gx2, torch.from_numpy(ref["grad_x2"]), "grad_x2 vs reference")


@needs_ref
def test_boolean_gpu_equals_reference_kernels(tmp_path):
    x1 = rand(2, 150, 300, seed=23) < 0.5
    x2 = rand(2, 140, 300, seed=24) < 0.1
    ref = ref_runner.run("pw_pwne_mean", {"x1": x1.numpy(), "x2": x2.numpy()}, tmp_path)
    got = capi.bool_pairwise_reduce(x1.to(DEV), x2.to(DEV), capi.BIT_NE, capi.RED_MEAN)
    assert_equal(got, torch.from_numpy(ref["out"]), "hamming vs reference")
    ref = ref_runner.run("jaccard", {"x1": x1.numpy(), "x2": x2.numpy()}, tmp_path)
    assert_equal(capi.jaccard_bool(x1.to(DEV), x2.to(DEV)), torch.from_numpy(ref["out"]), "jaccard vs reference")


# --------------------------------------------------------------------------------------
# k-smallest (neighbour) mask: bit-exact selection
# --------------------------------------------------------------------------------------
MASK_SHAPES = [(1, 1), (3, 7), (37, 300), (64, 4096), (5, 16384), (4, 16385), (3, 40000)]


@pytest.mark.parametrize("rows,cols", MASK_SHAPES)
@pytest.mark.parametrize("count", [1, 2, 3, 5, 9, 16, 17, 40, 300])
def test_row_smallest_mask_random(rows, cols, count):
    print(f"row_smallest_mask {rows}x{cols} count={count}", flush=True)
    d = rand(rows, cols, seed=11)
    got = capi.row_smallest_mask(d.to(DEV), count)
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(d.numpy(), count)), f"{rows}x{cols} c={count}")


@pytest.mark.parametrize("rows,cols", [(16, 1000), (6, 20000)])
@pytest.mark.parametrize("count", [1, 4, 16, 17, 100, 999])
def test_row_smallest_mask_ties_nan_signed_zero(rows, cols, count):
    print(f"row_smallest_mask ties {rows}x{cols} count={count}", flush=True)
    g = torch.Generator().manual_seed(12)
    d = torch.randint(0, 7, (rows, cols), generator=g).float() - 3.0  # heavy ties, negatives
    d[0, ::3] = float("nan")
    d[1, ::2] = -0.0
    d[1, 1::4] = 0.0
    d[2, :] = 5.0  # one value everywhere
    d[3, ::7] = float("inf")
    d[3, 1::7] = -float("inf")
    got = capi.row_smallest_mask(d.to(DEV), count)
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(d.numpy(), count)), f"ties c={count}")


def test_row_smallest_mask_golden_rows_and_edges():
    g = dict(np.load(Path(__file__).resolve().parent / "golden" / "neighbors.npz"))
    for i in range(int(g["n_rows"])):
        got = capi.row_smallest_mask(torch.from_numpy(g[f"row{i}_dist"]).to(DEV), int(g[f"row{i}_count"]))
        assert np.array_equal(got.cpu().numpy(), g[f"row{i}_mask"]), i
    d = rand(9, 50, seed=13)
    for count, want in ((0, False), (50, True), (51, True)):
        got = capi.row_smallest_mask(d.to(DEV), count)
        assert bool((got == want).all()), count
    assert capi.row_smallest_mask(torch.empty(0, 5, device=DEV), 2).shape == (0, 5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("count", [2, 33])
def test_row_smallest_mask_half_types(dtype, count):
    d = rand(20, 3000, seed=14).to(dtype)  # rounding to 16 bits creates ties
    got = capi.row_smallest_mask(d.to(DEV), count)
    want = P.k_smallest_mask(d.float().numpy(), count)  # exact widening keeps the order
    assert_equal(got, torch.from_numpy(want), f"{dtype} c={count}")


@pytest.mark.parametrize("cols", [8192, 8191, 20480, 20481])  # vector / scalar access; rows
@pytest.mark.parametrize("count", [17, 40, 200])                  # held in registers / streamed
def test_row_smallest_mask_list_runs_dry(cols, count):
    # the smallest entries all belong to workgroup thread 0 (columns 4c..4c+3 with
    # c = 0, 256, 512, ... for the vector path; columns 0, 256, 512, ... for the scalar
    # one): on rows longer than 16384 its 16-entry list runs dry and the row falls back to
    # the radix select; shorter rows take all of them as candidates
    d = rand(4, cols, seed=15) + 1.0
    own = torch.arange(0, cols, 1024).repeat_interleave(4) + torch.arange(4).repeat(len(range(0, cols, 1024)))
    own = own[own < cols] if cols % 4 == 0 else torch.arange(0, cols, 256)
    d[:, own] = -torch.arange(own.numel(), dtype=torch.float32)  # all distinct, all smallest
    d[2, own[::2]] = 0.5  # ties among them too
    got = capi.row_smallest_mask(d.to(DEV), count)
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(d.numpy(), count)), f"dry {cols} c={count}")


# --------------------------------------------------------------------------------------
# the reference's VALU family (_ppminkowski, _wminkowski, _canberra, _braycurtis)
# fp32 bar: values rtol 1e-5 (+ atol 1e-5 * max); gradients rtol 1e-4 (+ atol 1e-4 * max)
# --------------------------------------------------------------------------------------
FAM_SHAPES = [(1, 1, 1, 1), (1, 130, 70, 64), (2, 129, 131, 33), (1, 300, 257, 7)]


def _fam_ref(metric, a, b, w, p):
    if metric == capi.FAM_PPMINKOWSKI:
        return P.ppminkowski(a, b, p)
    if metric == capi.FAM_WMINKOWSKI:
        return P.wminkowski(a, b, w, p)
    if metric == capi.FAM_CANBERRA:
        return P.canberra(a, b)
    return P.braycurtis(a, b)


def _fam_inputs(B, n, m, d):
    x1 = randn(B, n, d, seed=20)
    x2 = randn(B, m, d, seed=21)
    w = rand(B, d, seed=22) + 0.2
    return x1, x2, w


@pytest.mark.parametrize("B,n,m,d", FAM_SHAPES)
@pytest.mark.parametrize("metric,p", [(0, 2.0), (0, 1.0), (0, 3.0), (0, 1.5), (0, float("inf")),
                                      (0, -float("inf")), (0, 0.0), (1, 2.0), (1, 1.0), (1, 3.0),
                                      (1, 0.7), (1, float("inf")), (2, 1.0), (3, 1.0)])
def test_family_forward(B, n, m, d, metric, p):
    print(f"family fwd metric={metric} p={p} {B}x{n}x{m}x{d}", flush=True)
    x1, x2, w = _fam_inputs(B, n, m, d)
    if metric == capi.FAM_CANBERRA:
        x1[..., ::3, 0] = 0.0  # 0 / 0 terms (skipped)
        x2[..., ::2, 0] = 0.0
    got = capi.family_forward(metric, x1.to(DEV), x2.to(DEV), w.to(DEV), p)
    ref = torch.stack([_fam_ref(metric, x1[i].double(), x2[i].double(), w[i].double(), p) for i in range(B)])
    assert_close(got, ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()), what=f"metric {metric} p={p}")


@pytest.mark.parametrize("B,n,m,d", FAM_SHAPES[1:] + [(1, 600, 900, 40)])
@pytest.mark.parametrize("metric,p", [(0, 2.0), (0, 1.0), (0, 3.0), (0, 1.5), (1, 2.0), (1, 1.0),
                                      (1, 3.0), (1, 2.5), (2, 1.0), (3, 1.0)])
def test_family_backward(B, n, m, d, metric, p):
    print(f"family bwd metric={metric} p={p} {B}x{n}x{m}x{d}", flush=True)
    x1, x2, w = _fam_inputs(B, n, m, d)
    g = randn(B, n, m, seed=23)
    out = capi.family_forward(metric, x1.to(DEV), x2.to(DEV), w.to(DEV), p)
    got = capi.family_backward(metric, g.to(DEV), x1.to(DEV), x2.to(DEV), w.to(DEV), p, out)
    refs = []
    for i in range(B):
        ins = [x1[i].double().requires_grad_(), x2[i].double().requires_grad_()]
        if metric == capi.FAM_WMINKOWSKI:
            ins.append(w[i].double().requires_grad_())
        val = _fam_ref(metric, ins[0], ins[1], ins[2] if len(ins) == 3 else None, p)
        val.backward(g[i].double())
        refs.append([t.grad for t in ins])
    for k, name in enumerate(["grad_x1", "grad_x2", "grad_w"][:len(got)]):
        ref = torch.stack([r[k] for r in refs])
        assert_close(got[k], ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()), what=f"{name} m{metric} p={p}")


def test_family_backward_edge_cases():
    x1, x2, w = _fam_inputs(1, 40, 30, 9)
    g = randn(1, 40, 30, seed=24)
    for metric in (capi.FAM_PPMINKOWSKI, capi.FAM_WMINKOWSKI):  # p = 0: zero gradients
        out = capi.family_forward(metric, x1.to(DEV), x2.to(DEV), w.to(DEV), 0.0)
        assert bool((out == 9.0).all())
        for t in capi.family_backward(metric, g.to(DEV), x1.to(DEV), x2.to(DEV), w.to(DEV), 0.0, out):
            assert bool((t == 0).all())
    # p = +-inf: the first arg-extremum's sign per pair, grad_x1 summed over j and grad_x2 over i
    # in order (ppminkowski_kernel.cpp:171-208): exact against the CPU loop with ties
    xi, yi = torch.randint(-3, 4, (1, 40, 9), generator=torch.Generator().manual_seed(5)).float(), \
        torch.randint(-3, 4, (1, 30, 9), generator=torch.Generator().manual_seed(6)).float()
    for p in (float("inf"), -float("inf")):
        got = capi.family_backward(capi.FAM_PPMINKOWSKI, g.to(DEV), xi.to(DEV), yi.to(DEV), None, p)
        a, b = xi[0].clone().requires_grad_(), yi[0].clone().requires_grad_()
        torch.ops.torchpairwise._ppminkowski(a, b, p).backward(g[0])
        assert_equal(got[0][0], a.grad, f"grad_x1 p={p}")
        assert_equal(got[1][0], b.grad, f"grad_x2 p={p}")


# --------------------------------------------------------------------------------------
# _additive_chi2_kernel, _sqjensenshannon, _haversine through the C ABI
# fp32 bar: values rtol 1e-5 (+ atol 1e-5 * max); gradients rtol 1e-4 (+ atol 1e-4 * max)
# --------------------------------------------------------------------------------------
def _prob_inputs(B, n, m, d, zeros):
    x1 = rand(B, n, d, seed=40) + (0.0 if zeros else 0.05)
    x2 = rand(B, m, d, seed=41) + (0.0 if zeros else 0.05)
    if zeros:  # chi2's skipped 0 / 0 terms, JS's rel_entr(0, .) = 0
        x1[..., ::3, 0] = 0.0
        x2[..., ::2, 0] = 0.0
        x1[..., ::5, 1:3] = 0.0
    return x1, x2


def _special_ref(metric, a, b, p):
    if metric == capi.FAM_CHI2:
        return P.additive_chi2(a, b)
    return P.sqjensenshannon(a, b, None if p == 2.0 else float(np.exp(p / 2)))


@pytest.mark.parametrize("B,n,m,d", FAM_SHAPES + [(1, 600, 900, 40)])
@pytest.mark.parametrize("metric,p", [(4, 1.0), (5, 2.0), (5, 2 * float(np.log(3.0)))])
def test_chi2_js_forward(B, n, m, d, metric, p):
    print(f"chi2/js fwd metric={metric} p={p} {B}x{n}x{m}x{d}", flush=True)
    x1, x2 = _prob_inputs(B, n, m, d, zeros=True)
    got = capi.family_forward(metric, x1.to(DEV), x2.to(DEV), None, p)
    ref = torch.stack([_special_ref(metric, x1[i].double(), x2[i].double(), p) for i in range(B)])
    assert_close(got, ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()), what=f"metric {metric} p={p}")


@pytest.mark.parametrize("B,n,m,d", FAM_SHAPES[1:] + [(1, 600, 900, 40)])
@pytest.mark.parametrize("metric,p", [(4, 1.0), (5, 2.0), (5, 2 * float(np.log(3.0)))])
def test_chi2_js_backward(B, n, m, d, metric, p):
    print(f"chi2/js bwd metric={metric} p={p} {B}x{n}x{m}x{d}", flush=True)
    x1, x2 = _prob_inputs(B, n, m, d, zeros=False)
    g = randn(B, n, m, seed=42)
    got = capi.family_backward(metric, g.to(DEV), x1.to(DEV), x2.to(DEV), None, p)
    refs = []
    for i in range(B):
        a, b = x1[i].double().requires_grad_(), x2[i].double().requires_grad_()
        _special_ref(metric, a, b, p).backward(g[i].double())
        refs.append((a.grad, b.grad))
    for k, name in enumerate(["grad_x1", "grad_x2"]):
        ref = torch.stack([r[k] for r in refs])
        assert_close(got[k], ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()), what=f"{name} m{metric}")


def test_chi2_js_zero_terms_match_the_reference_loops():
    # gradients with 0 coordinates: the reference's own CPU loops (run in float64) are the bar
    x1, x2 = _prob_inputs(1, 70, 50, 9, zeros=True)
    g = randn(1, 70, 50, seed=43)
    ops = torch.ops.torchpairwise
    for metric, p in ((capi.FAM_CHI2, 1.0), (capi.FAM_JS, 2.0)):
        got = capi.family_backward(metric, g.to(DEV), x1.to(DEV), x2.to(DEV), None, p)
        if metric == capi.FAM_CHI2:
            ref = ops.__additive_chi2_kernel_backward(g.double(), x1.double(), x2.double())
        else:
            ref = ops.__sqjensenshannon_backward(g.double(), x1.double(), x2.double(), None)
        for t, r in zip(got, ref):
            fin = torch.isfinite(r)
            assert bool((torch.isfinite(t.cpu()) == fin).all()), f"non-finite pattern m{metric}"
            assert_close(t.cpu()[fin], r[fin], rtol=1e-4, atol=1e-4 * float(r[fin].abs().max()),
                         what=f"zero terms m{metric}")


HAV_SHAPES = [(1, 1, 1), (1, 300, 257), (3, 129, 65), (1, 2000, 1500)]


def _geo(B, n, seed, octant=False):
    """Points (latitude, longitude) over the whole sphere, or over one octant (every pair
    then lies within pi / 2: no ill-conditioned pairs)."""
    u = rand(B, n, 2, seed=seed)
    if octant:
        return u * (np.pi / 2)
    return torch.stack([u[..., 0] * np.pi - np.pi / 2, u[..., 1] * 2 * np.pi - np.pi], -1)


# Haversine's conditioning: with v = sin^2(d / 2) rounded in fp32 (error ~ a few ulp, absolute
# near v = 1), d = 2 asin(sqrt v) moves by 8 eps / cos(d / 2) and the pair weight
# 1 / (sqrt(v) sqrt(1 - v)) = 2 / |sin d| by a relative 4 eps / cos^2(d / 2) beyond ordinary
# rounding.  Any fp32 evaluation of the reference's formula (its own kernel included) has
# these errors, so nearly antipodal pairs (cos(d / 2) < 0.05, i.e. 1 - v < 2.5e-3) get that
# first-order allowance on top of the fp32 bar; every other pair is held to the plain bar.
EPS32 = 2.0 ** -24


def _hav_allowance(ref, g):
    d = ref.detach().double()
    half_cos = torch.cos(d / 2).abs().clamp_min(1e-30)
    ill = half_cos < 0.05
    fwd = torch.where(ill, 16 * EPS32 / half_cos, torch.zeros_like(d))
    pair = 24 * EPS32 * g.double().abs() / torch.sin(d).abs().clamp_min(1e-30) / half_cos ** 2
    pair = torch.where(ill, pair, torch.zeros_like(pair))
    return fwd, pair.sum(-1, keepdim=True), pair.sum(-2).unsqueeze(-1)


@pytest.mark.parametrize("B,n,m", HAV_SHAPES)
@pytest.mark.parametrize("octant", [True, False])
def test_haversine_forward_backward(B, n, m, octant):
    print(f"haversine {B}x{n}x{m} octant={octant}", flush=True)
    x1, x2 = _geo(B, n, 44, octant), _geo(B, m, 45, octant)
    g = randn(B, n, m, seed=46)
    got = capi.haversine(x1.to(DEV), x2.to(DEV))
    a, b = x1.double().requires_grad_(), x2.double().requires_grad_()
    ref = P.haversine(a, b)
    fwd, row, col = _hav_allowance(ref, g)
    if octant:
        assert not bool(fwd.any()) and not bool(row.any())  # the plain fp32 bar only
    assert_close(got, ref.detach(), rtol=1e-5, atol=1e-5 * float(ref.abs().max()) + fwd, what="haversine")
    ref.backward(g.double())
    gx1, gx2 = capi.haversine_backward(g.to(DEV), x1.to(DEV), x2.to(DEV))
    assert_close(gx1, a.grad, rtol=1e-4, atol=1e-4 * float(a.grad.abs().max()) + row, what="grad_x1")
    assert_close(gx2, b.grad, rtol=1e-4, atol=1e-4 * float(b.grad.abs().max()) + col, what="grad_x2")


def test_haversine_empty_and_unbatched():
    x1, x2 = _geo(1, 20, 47)[0], _geo(1, 0, 48)[0]
    assert capi.haversine(x1.to(DEV), x2.to(DEV)).shape == (20, 0)
    gx1, gx2 = capi.haversine_backward(torch.empty(20, 0, device=DEV), x1.to(DEV), x2.to(DEV))
    assert gx1.shape == (20, 2) and bool((gx1 == 0).all()) and gx2.shape == (0, 2)


@pytest.mark.parametrize("empty", ["x1", "x2"])
def test_backward_entries_with_one_empty_side(empty):
    # no pairs: the non-empty side's gradient is zero (its buffer is written, not left as is);
    # the empty side's buffer is a null pointer
    n, m, d = (0, 37, 5) if empty == "x1" else (41, 0, 5)
    x1, x2 = (rand(1, n, d, seed=50) + 0.1).to(DEV), (rand(1, m, d, seed=51) + 0.1).to(DEV)
    g = torch.empty(1, n, m, device=DEV)
    other = lambda res: res[1] if empty == "x1" else res[0]
    for metric in (capi.FAM_PPMINKOWSKI, capi.FAM_CANBERRA, capi.FAM_CHI2, capi.FAM_JS):
        res = capi.family_backward(metric, g, x1, x2, None, 2.0)
        assert bool((other(res) == 0).all()), f"family {metric}"
    assert bool((other(capi.lp_distances_backward2(g, x1, x2, g, 3.0)) == 0).all()), "lp"
    for dt in (torch.float32, torch.bfloat16):
        a, b, gg = x1.to(dt), x2.to(dt), g.to(dt)
        assert bool((other(capi.euclidean_backward(gg, a, b, gg)) == 0).all()), f"euclidean {dt}"
        assert bool((other(capi.sqeuclidean_backward(gg, a, b)) == 0).all()), f"sqeuclidean {dt}"
    geo1, geo2 = x1[..., :2].contiguous(), x2[..., :2].contiguous()
    assert bool((other(capi.haversine_backward(g, geo1, geo2)) == 0).all()), "haversine"


@pytest.mark.parametrize("n,m", [(128, 128), (100, 70)])  # staged full tiles / partial tiles
def test_bf16_outputs_round_to_nearest_even(n, m):
    # x1[i] . x2[j] = a_i + b_i * s_j with s_j a power of two: exact in the fp32 accumulator, so
    # the bf16 output is the RNE rounding of a known fp32 value (ties, carries into the exponent,
    # large magnitudes, signs), compared bit for bit with torch's CPU conversion
    # a, b = +-(1 + k / 128) (bf16-exact, exponent 0) and s in [2^-9, 4]: every sum needs at
    # most 19 significant bits, so it is exact in fp32 whatever the MFMA's summation order
    g = torch.Generator().manual_seed(70)
    sign = lambda: torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    a = sign() * (1 + torch.randint(0, 128, (n,), generator=g).float() / 128)
    b = sign() * (1 + torch.randint(0, 128, (n,), generator=g).float() / 128)
    a[:4] = torch.tensor([1.0, 1.0078125, -1.0, 2.0e38])  # 1 + 2^-7; a large magnitude
    b[:4] = torch.tensor([1.0, 1.0, 1.0, 1.0e37])
    a, b = a.to(torch.bfloat16).float(), b.to(torch.bfloat16).float()
    s = 2.0 ** torch.randint(-9, 3, (m,), generator=g).float()
    s[:3] = torch.tensor([2.0 ** -8, 2.0 ** -8, 2.0 ** -9])  # exact ties for rows 0-2
    x1 = torch.stack([a, b], 1).to(torch.bfloat16)
    x2 = torch.stack([torch.ones(m), s], 1).to(torch.bfloat16)
    want = (a[:, None] + b[:, None] * s[None, :]).to(torch.bfloat16)
    got = capi.pairwise_inner(x1.to(DEV), x2.to(DEV), capi.EPI_DOT)
    assert_equal(got, want, f"bf16 rounding {n}x{m}")


@pytest.mark.parametrize("cols", [16384, 16383, 1000])
@pytest.mark.parametrize("count", [150, 256])
def test_row_smallest_mask_candidate_overflow(cols, count):
    # rows held in registers: the count-th smallest per-thread minimum bounds the selection;
    # here most threads' entries all lie below it (ties at 0 and a ramp), so more than 2048
    # candidates qualify and the row takes the exact radix fallback
    d = rand(3, cols, seed=16) + 1.0
    d[0, : cols * 3 // 4] = 0.0  # three quarters of the row tied at the minimum
    d[1, : cols * 3 // 4] = torch.linspace(-1.0, 0.0, cols * 3 // 4)
    got = capi.row_smallest_mask(d.to(DEV), count)
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(d.numpy(), count)), f"overflow {cols} c={count}")


@pytest.mark.parametrize("kind,degree", [(capi.KER_POLYNOMIAL, 3), (capi.KER_POLYNOMIAL, 5),
                                         (capi.KER_SIGMOID, 0)])
@pytest.mark.parametrize("B,n,m,d", [(1, 130, 200, 64), (2, 257, 129, 96)])
def test_pairwise_kernel_capi(kind, degree, B, n, m, d):
    # tpw_pairwise_kernel / _backward against the composite in float64 (fp32 bar as above)
    x1, x2 = randn(B, n, d, seed=80) / 4, randn(B, m, d, seed=81) / 4
    g = randn(B, n, m, seed=82)
    gamma, coef0 = 0.7, 0.4
    out = capi.pairwise_kernel(x1.to(DEV), x2.to(DEV), kind, gamma, coef0, degree)
    a, b = x1.double().requires_grad_(), x2.double().requires_grad_()
    base = (a @ b.transpose(1, 2)) * gamma + coef0
    ref = base ** degree if kind == capi.KER_POLYNOMIAL else torch.tanh(base)
    assert_close(out, ref.detach(), rtol=1e-4, atol=1e-5 * float(ref.abs().max()), what="forward")
    ref.backward(g.double())
    gx1, gx2 = capi.pairwise_kernel_backward(g.to(DEV), x1.to(DEV), x2.to(DEV), out, kind, gamma, coef0, degree)
    assert_close(gx1, a.grad, rtol=1e-4, atol=1e-4 * float(a.grad.abs().max()), what="grad_x1")
    assert_close(gx2, b.grad, rtol=1e-4, atol=1e-4 * float(b.grad.abs().max()), what="grad_x2")
