"""GPU parity at the benchmark configurations' full sizes (the metric shape M = 16384^2 x 128
and C2..C5), with the inputs the benchmark draws.  The full outputs are too large for the
CPU oracle, so each test checks a seeded sample of output rows (and, for gradients, of
columns) against the oracle on the same inputs, plus size-independent properties of the
whole output: exact count grids for boolean metrics, symmetry for x2 = None, and, for
directed Hausdorff, that every returned index pair realises the value and is the first
nearest x2 point of the returned x1 point."""
import os

import numpy as np
import pytest
import torch

import torchpairwise_amd as tp
from oracle import cref
from oracle import pairwise as P
from tests._util import assert_close, assert_equal, rand, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sample(n: int, k: int, seed: int) -> list[int]:
    """The first and last four indices plus k seeded random ones, sorted and distinct."""
    g = torch.Generator().manual_seed(seed)
    picks = torch.randperm(n, generator=g)[:k].tolist()
    return sorted(set(picks) | set(range(4)) | set(range(n - 4, n)))


def _rows_close(out, ref, rtol, what):
    assert_close(out, ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what=what)


# ------------------------------------------------- C1: manhattan + euclidean [2048,64] x [1024,64]
def test_c1_manhattan_euclidean():
    """BASELINE configs[0] on the GPU: the drop-in ops against the reference's arithmetic
    (at::cdist, pairwise_metrics.cpp:24-31,42-49) in float64, every element."""
    x1, x2 = randn(2048, 64, seed=0), randn(1024, 64, seed=1)
    for name, fn, p in (("euclidean", tp.euclidean_distances, 2.0),
                        ("manhattan", tp.manhattan_distances, 1.0)):
        out = fn(x1.to(DEV), x2.to(DEV))
        assert out.shape == (2048, 1024) and out.dtype == torch.float32, name
        _rows_close(out.cpu(), torch.cdist(x1.double(), x2.double(), p), 1e-5, f"C1 {name}")


# ------------------------------------------------------------------------ M: 16384^2 x 128
def test_metric_shape_euclidean_manhattan():
    x1, x2 = randn(16384, 128, seed=0), randn(16384, 128, seed=1)
    a, b = x1.to(DEV), x2.to(DEV)
    rows = _sample(16384, 40, seed=3)
    for name, fn, p in (("euclidean", tp.euclidean_distances, 2.0),
                        ("manhattan", tp.manhattan_distances, 1.0)):
        out = fn(a, b)
        assert out.shape == (16384, 16384) and out.dtype == torch.float32
        assert bool(torch.isfinite(out).all()) and bool((out >= 0).all()), name
        ref = torch.cdist(x1[rows].double(), x2.double(), p)
        _rows_close(out[rows].cpu(), ref, 1e-5, f"{name} sampled rows")
        del out
    # x2 = None: the matrix of a cloud against itself is symmetric with a near-zero diagonal
    d = tp.euclidean_distances(a)
    scale = float(d.max())
    assert float((d - d.T).abs().max()) <= 1e-5 * scale
    # |a|^2 + |a|^2 - 2 a.a in fp32 leaves at most a few ulp of 2|a|^2 under the root
    floor = 4 * torch.sqrt(torch.finfo(torch.float32).eps * 2 * (x1.double() ** 2).sum(1))
    assert bool((d.diagonal().cpu().double() <= floor).all())


def test_metric_shape_hamming():
    x1 = rand(16384, 128, seed=0) < 0.5
    x2 = rand(16384, 128, seed=1) < 0.5
    out = tp.hamming_distances(x1.to(DEV), x2.to(DEV))
    assert out.shape == (16384, 16384) and out.dtype == torch.float32
    # every output is count / 128 exactly: an integer grid over the whole matrix
    t = out * 128
    assert bool((t == t.round()).all()) and bool((t >= 0).all()) and bool((t <= 128).all())
    rows = _sample(16384, 40, seed=4)
    want = P.hamming_distances(x1[rows].numpy(), x2.numpy())
    assert_equal(out[rows].cpu(), torch.from_numpy(want), "hamming sampled rows")


# ------------------------------------------------------------------ C2: [8, 8192, 256]^2 fwd+bwd
@pytest.fixture(scope="module")
def c2_inputs():
    x1, x2 = randn(8, 8192, 256, seed=0), randn(8, 8192, 256, seed=1)
    g = randn(8, 8192, 8192, seed=2)
    return x1, x2, g


def _c2_ref(metric, r1, r2, gsl):
    """Reference value and gradient of one row block (or column block) in float64 on the CPU:
    the reference's arithmetic (at::cdist for euclidean, the prf_div composite for cosine)."""
    out = torch.cdist(r1, r2, 2) if metric == "euclidean" else P.cosine_distances(r1, r2)
    out.backward(gsl)
    return out.detach()


def _c2_grad_bound(metric, own, other, gsl):
    """The derived fp32 bound (tests/_gradbound.py) of the gradient of `own`'s rows, a sum over
    `other`'s rows, gsl the upstream gradient in that orientation (grad^T for x2's rows)."""
    from tests import _gradbound as GB

    if metric == "euclidean":
        return GB.euclidean_grad_bound(own, other, gsl)
    return GB.cosine_grad_bound(own, other, gsl)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("metric", ["euclidean", "cosine"])
def test_c2_forward_backward(c2_inputs, metric, dtype):
    x1, x2, g = c2_inputs
    x1, x2, g = x1.to(dtype), x2.to(dtype), g.to(dtype)
    a = x1.to(DEV).requires_grad_()
    b = x2.to(DEV).requires_grad_()
    fn = tp.euclidean_distances if metric == "euclidean" else tp.cosine_distances
    out = fn(a, b)
    assert out.shape == (8, 8192, 8192) and out.dtype == dtype
    out.backward(g.to(DEV))
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    grtol = 1e-2  # bf16
    f1, f2 = x1.double(), x2.double()
    from tests import _gradbound as GB
    for bb in (0, 5):
        rows = _sample(8192, 6, seed=10 + bb)
        r1 = f1[bb, rows].clone().requires_grad_()
        ref = _c2_ref(metric, r1, f2[bb], g[bb, rows].double())
        _rows_close(out[bb, rows].detach().float().cpu(), ref, rtol, f"{metric} rows b={bb}")
        got1 = a.grad[bb, rows].float().cpu()
        if dtype == torch.float32:  # the derived per-element bound
            worst = GB.check(got1, r1.grad, _c2_grad_bound(metric, f1[bb, rows], f2[bb], g[bb, rows]),
                             f"{metric} grad_x1 b={bb}")
            print(f"{metric} fp32 grad_x1 b={bb}: largest |err| / derived bound {worst:.4f}", flush=True)
        else:
            _rows_close(got1, r1.grad, grtol, f"{metric} grad_x1 b={bb}")
        cols = _sample(8192, 6, seed=20 + bb)
        r2 = f2[bb, cols].clone().requires_grad_()
        _c2_ref(metric, f1[bb], r2, g[bb][:, cols].double())
        got2 = b.grad[bb, cols].float().cpu()
        if dtype == torch.float32:
            worst = GB.check(got2, r2.grad, _c2_grad_bound(metric, f2[bb, cols], f1[bb], g[bb][:, cols].T),
                             f"{metric} grad_x2 b={bb}")
            print(f"{metric} fp32 grad_x2 b={bb}: largest |err| / derived bound {worst:.4f}", flush=True)
        else:
            _rows_close(got2, r2.grad, grtol, f"{metric} grad_x2 b={bb}")


@pytest.mark.parametrize("metric,extreme", [("cosine", False), ("cosine", True), ("cosine_similarity", False),
                                           ("cosine_similarity", True), ("euclidean", False)])
def test_inner_backward_fused_grid_ragged(metric, extreme):
    """The fp32 backward where the fused weight + grad_x1 kernel runs, at a shape that takes its
    edge cases: n % 128 = 96 (the last row block's fourth wave lies past the end: it stores no W
    rows and writes zero column partials), d = 260 (two column blocks, of which only the first
    writes column partials, and a partial last one).  With `extreme`, one row's norm lies above
    2^60, which sends a cosine call to the kernel instance that divides by every norm product.
    Sampled rows (the partial block's and the scaled one included) and columns against float64
    autograd of the reference's composite (at::cdist for euclidean), within the derived bound."""
    from tests import _gradbound as GB

    B, n, m, d = 2, 16352, 11008, 260
    x1, x2 = randn(B, n, d, seed=40), randn(B, m, d, seed=41)
    if extreme:
        x1[1, 16300] *= 2.0 ** 58
    gen = torch.Generator(device=DEV).manual_seed(42)
    g = torch.randn(B, n, m, device=DEV, generator=gen)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    similarity = metric == "cosine_similarity"
    fn = {"cosine": tp.cosine_distances, "cosine_similarity": tp.cosine_similarity,
          "euclidean": tp.euclidean_distances}[metric]
    ref_fn = {"cosine": P.cosine_distances, "cosine_similarity": P.cosine_similarity,
              "euclidean": lambda u, v: torch.cdist(u, v, 2)}[metric]

    def bound(own, other, gsl):
        if metric == "euclidean":
            return GB.euclidean_grad_bound(own, other, gsl)
        return GB.cosine_grad_bound(own, other, gsl, similarity)

    fn(a, b).backward(g)
    f1, f2 = x1.double(), x2.double()
    for bb in range(B):
        rows = sorted(set(_sample(n, 6, seed=50 + bb)) | {16256, 16300, 16351})
        cols = _sample(m, 6, seed=60 + bb)
        r1 = f1[bb, rows].clone().requires_grad_()
        gr = g[bb, rows].double().cpu()
        ref_fn(r1, f2[bb]).backward(gr)
        worst = GB.check(a.grad[bb, rows].cpu(), r1.grad, bound(f1[bb, rows], f2[bb], gr),
                         f"{metric} grad_x1 b={bb}")
        print(f"{metric} grad_x1 b={bb}: largest |err| / derived bound {worst:.4f}", flush=True)
        r2 = f2[bb, cols].clone().requires_grad_()
        gc = g[bb][:, cols].double().cpu()
        ref_fn(f1[bb], r2).backward(gc)
        worst = GB.check(b.grad[bb, cols].cpu(), r2.grad, bound(f2[bb, cols], f1[bb], gc.T.contiguous()),
                         f"{metric} grad_x2 b={bb}")
        print(f"{metric} grad_x2 b={bb}: largest |err| / derived bound {worst:.4f}", flush=True)


@pytest.mark.parametrize("extreme", [False, True])
@pytest.mark.parametrize("similarity", [False, True])
def test_cosine_backward_fused_grid_bf16(similarity, extreme):
    """The bf16 cosine backward where the fused weight + grad_x1 kernel runs (n % 128 == 0 and a
    grid of two blocks per CU: 4 x 16384 x 8192 x 256), its grad_x2 coefficient from the
    projection -(x2 . P) / |x2|^2 of the product P = W^T x1.  With `extreme`, one row's norm lies
    above 2^60 (the dividing kernel instance).  Sampled rows (the scaled one included) and
    columns against float64 autograd of the reference's composite, bf16 bar 1e-2 (+ 1e-2 max)."""
    B, n, m, d = 4, 16384, 8192, 256
    x1 = randn(B, n, d, seed=70).to(torch.bfloat16)
    x2 = randn(B, m, d, seed=71).to(torch.bfloat16)
    if extreme:
        x1[2, 5000] *= 2.0 ** 58
    gen = torch.Generator(device=DEV).manual_seed(72)
    g = torch.randn(B, n, m, device=DEV, generator=gen).to(torch.bfloat16)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    fn = tp.cosine_similarity if similarity else tp.cosine_distances
    ref_fn = P.cosine_similarity if similarity else P.cosine_distances
    fn(a, b).backward(g)
    f1, f2 = x1.double(), x2.double()
    for bb in (0, 2):
        rows = sorted(set(_sample(n, 6, seed=80 + bb)) | {5000})
        cols = _sample(m, 6, seed=90 + bb)
        r1 = f1[bb, rows].clone().requires_grad_()
        ref_fn(r1, f2[bb]).backward(g[bb, rows].double().cpu())
        _rows_close(a.grad[bb, rows].float().cpu(), r1.grad, 1e-2, f"bf16 cosine sim={similarity} grad_x1 b={bb}")
        r2 = f2[bb, cols].clone().requires_grad_()
        ref_fn(f1[bb], r2).backward(g[bb][:, cols].double().cpu())
        _rows_close(b.grad[bb, cols].float().cpu(), r2.grad, 1e-2, f"bf16 cosine sim={similarity} grad_x2 b={bb}")


# ------------------------------------------------- C3: minkowski p=3 fwd+bwd, chebyshev, [16384,128]^2
def test_c3_minkowski_chebyshev():
    x1 = rand(16384, 128, seed=0) * 2 - 1
    x2 = rand(16384, 128, seed=1) * 2 - 1
    a = x1.to(DEV).requires_grad_()
    b = x2.to(DEV).requires_grad_()
    out = tp.minkowski_distances(a, b, p=3.0)
    out.backward(torch.ones_like(out))
    f1, f2 = x1.double(), x2.double()
    rows = _sample(16384, 12, seed=5)
    r1 = f1[rows].clone().requires_grad_()
    ref = torch.cdist(r1, f2, 3.0)
    ref.backward(torch.ones_like(ref))
    _rows_close(out[rows].detach().cpu(), ref.detach(), 1e-5, "minkowski p=3 rows")
    # the derived per-element bound (tests/_gradbound.py) of sum_j w d |d|, w = 1 / dist^2
    # (upstream gradient of ones): d, d |d|, the weight from the fp32 forward (cube root, square,
    # divide) and the fma, 10 u per term
    from tests import _gradbound as GB

    def p3_bound(own, other, dist):
        dd = own[:, None, :] - other[None, :, :]
        return GB.sum_bound((1.0 / dist ** 2)[:, :, None] * dd * dd.abs(), 1, 10.0)

    worst = GB.check(a.grad[rows].cpu(), r1.grad, p3_bound(f1[rows], f2, ref.detach()), "minkowski grad_x1")
    print(f"minkowski p=3 grad_x1: largest |err| / derived bound {worst:.4f}", flush=True)
    cols = _sample(16384, 12, seed=6)
    r2 = f2[cols].clone().requires_grad_()
    refc = torch.cdist(f1, r2, 3.0)
    refc.backward(torch.ones_like(refc))
    worst = GB.check(b.grad[cols].cpu(), r2.grad, p3_bound(f2[cols], f1, refc.detach().T), "minkowski grad_x2")
    print(f"minkowski p=3 grad_x2: largest |err| / derived bound {worst:.4f}", flush=True)
    del out
    # chebyshev: max |fl(a - b)| is exact in float32, so the sampled rows are bit-exact
    cheb = tp.chebyshev_distances(a.detach(), b.detach())
    rows = _sample(16384, 40, seed=7)
    assert_equal(cheb[rows].cpu(), torch.cdist(x1[rows], x2, float("inf")), "chebyshev rows")


# ----------------------------------------------------------- C4: bool [32768, 1024]^2
@pytest.mark.parametrize("metric,density", [("hamming", 0.5), ("jaccard", 0.1)])
def test_c4_boolean(metric, density):
    x1 = rand(32768, 1024, seed=0) < density
    x2 = rand(32768, 1024, seed=1) < density
    fn = tp.hamming_distances if metric == "hamming" else tp.jaccard_distances
    out = fn(x1.to(DEV), x2.to(DEV))
    assert out.shape == (32768, 32768) and out.dtype == torch.float32
    assert bool((out >= 0).all()) and bool((out <= 1).all())
    if metric == "hamming":
        t = out * 1024  # count / 1024 exactly: an integer grid over the whole matrix
        assert bool((t == t.round()).all())
    rows = _sample(32768, 28, seed=8)
    ref = (P.hamming_distances if metric == "hamming" else P.jaccard_distances)(
        x1[rows].numpy(), x2.numpy())
    assert_equal(out[rows].cpu(), torch.from_numpy(ref), f"{metric} sampled rows")


# ---------------------------------------------- C5: directed Hausdorff [16, 65536, 3]^2
def _first_nearest(cloud2: np.ndarray, point: np.ndarray):
    """min over n of the reference's float32 squared distance (sequential k, no FMA) from
    `point` to every point of `cloud2`, and the first n reaching it."""
    d = np.zeros(cloud2.shape[0], np.float32)
    for k in range(cloud2.shape[1]):
        diff = (np.float32(point[k]) - cloud2[:, k]).astype(np.float32)
        d = (d + (diff * diff).astype(np.float32)).astype(np.float32)
    n = int(np.argmin(d))  # argmin returns the first position of the minimum
    return d[n], n


def test_c5_directed_hausdorff():
    x1 = rand(16, 65536, 3, seed=0)
    x2 = rand(16, 65536, 3, seed=1) + 0.05
    a = x1.to(DEV).requires_grad_()
    b = x2.to(DEV).requires_grad_()
    out, i1, i2 = tp.directed_hausdorff_distances(a, b)
    out.backward(torch.ones_like(out))
    o, m_, n_ = out.detach().cpu().numpy(), i1.cpu().numpy(), i2.cpu().numpy()
    c1, c2 = x1.numpy(), x2.numpy()
    # all 256 cloud pairs against the early-break restatement of the reference loop
    # (csrc/ops/cpu/hausdorff_kernel.cpp:12-53): value, x1 index and x2 index bit for bit
    w = cref.directed_hausdorff(c1, c2, threads=min(16, os.cpu_count() or 1))
    assert_equal(out.detach().cpu(), torch.from_numpy(w[0]), "value, all cloud pairs")
    assert np.array_equal(m_, w[1]), f"x1 indices differ at {np.argwhere(m_ != w[1])[:5].tolist()}"
    assert np.array_equal(n_, w[2]), f"x2 indices differ at {np.argwhere(n_ != w[2])[:5].tolist()}"
    # independently of the loop: the returned x1 point's first nearest x2 point is the returned
    # one and its distance is the output, bit for bit
    for i in range(16):
        for j in range(16):
            h, n = _first_nearest(c2[j], c1[i, m_[i, j]])
            assert n == n_[i, j] and np.sqrt(h, dtype=np.float32) == o[i, j], (i, j)
    # backward: the reference's scatter over those indices, both gradients
    gx1, gx2 = P.directed_hausdorff_backward(np.ones((16, 16), np.float32), c1, c2, o, m_, n_)
    assert_equal(a.grad.cpu(), torch.from_numpy(gx1), "grad_x1")
    assert_equal(b.grad.cpu(), torch.from_numpy(gx2), "grad_x2")


@pytest.mark.parametrize("name,kw,dtype", [("polynomial_kernel", {"degree": 3, "gamma": 0.01, "coef0": 0.5}, torch.float32),
                                           ("sigmoid_kernel", {"gamma": 0.01, "coef0": 0.1}, torch.float32),
                                           ("sigmoid_kernel", {"gamma": 0.01, "coef0": 0.1}, torch.bfloat16)])
def test_kernel_function_backward_fused_grid(name, kw, dtype):
    """The kernel functions' backward where the fused weight + grad_x1 kernel runs (its grid
    and the grad_x2 product's fill the GPU: n 16384, m 8192, d 1024): gradients of 48 sampled
    rows of x1 and columns of x2 against the reference's formulas in float64 (the weights from
    S = x1 x2^T, gamma and coef0; polynomial: degree gamma base^(degree-1), sigmoid:
    gamma (1 - tanh(base)^2)).  fp32 rtol 1e-4, bf16 1e-2 (each + rtol * max)."""
    n, m, d = 16384, 8192, 1024
    g0 = torch.Generator().manual_seed(31)
    x1, x2 = torch.randn(n, d, generator=g0).to(dtype), torch.randn(m, d, generator=g0).to(dtype)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = getattr(tp, name)(a, b, **kw)
    g = torch.randn(n, m, generator=g0).to(DEV, dtype)
    out.backward(g)
    rows, cols = torch.randperm(n, generator=g0)[:48], torch.randperm(m, generator=g0)[:48]
    A, B = x1.double(), x2.double()
    gamma, coef0 = kw["gamma"], kw["coef0"]

    def weight(gs, s):
        base = s * gamma + coef0
        if name == "polynomial_kernel":
            return gs * kw["degree"] * gamma * base ** (kw["degree"] - 1)
        return gs * gamma * (1 - torch.tanh(base) ** 2)

    gr = g[rows.to(DEV)].double().cpu()
    gc = g[:, cols.to(DEV)].double().cpu()
    want1 = weight(gr, A[rows] @ B.T) @ B
    want2 = weight(gc, A @ B[cols].T).T @ A
    rtol = 1e-4 if dtype == torch.float32 else 1e-2
    got1, got2 = a.grad[rows.to(DEV)].double().cpu(), b.grad[cols.to(DEV)].double().cpu()
    assert_close(got1, want1, rtol=rtol, atol=rtol * float(want1.abs().max()), what=f"{name} grad x1 rows")
    assert_close(got2, want2, rtol=rtol, atol=rtol * float(want2.abs().max()), what=f"{name} grad x2 cols")
