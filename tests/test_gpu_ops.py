"""GPU parity of the drop-in ops (torch.ops.torchpairwise on cuda tensors) against the oracle:
forward values, gradients through autograd, and that the HIP library is what runs."""
import numpy as np
import pytest
import torch

import torchpairwise_amd as tp
from oracle import cref
from oracle import pairwise as P
from tests._util import assert_close, assert_equal, rand, randn
from torchpairwise_amd import _capi as capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_native_library_is_loaded():
    maps = open("/proc/self/maps").read()
    assert "libtorchpairwise_hip.so" in maps and "torchpairwise_amd/_C.so" in maps


@pytest.mark.parametrize("shape", [((300, 64), (200, 64)), ((2, 130, 128), (2, 90, 128)),
                                   ((10, 16), (20, 16)), ((1, 40, 8), (3, 30, 8))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_euclidean_forward_backward(shape, dtype):
    x1 = randn(*shape[0], seed=0, dtype=dtype)
    x2 = randn(*shape[1], seed=1, dtype=dtype)
    a = x1.to(DEV).requires_grad_()
    b = x2.to(DEV).requires_grad_()
    out = tp.euclidean_distances(a, b)
    g = randn(*out.shape, seed=2, dtype=dtype)
    out.backward(g.to(DEV))
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    ref = torch.cdist(ra, rb, 2)
    ref.backward(g.double())
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    grtol = 1e-4 if dtype == torch.float32 else 1e-2
    assert out.dtype == dtype
    assert_close(out.float(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what="euclidean")
    assert_close(a.grad.float(), ra.grad, rtol=grtol, atol=grtol * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad.float(), rb.grad, rtol=grtol, atol=grtol * float(rb.grad.abs().max()), what="grad x2")


def test_euclidean_self_pair_grad():
    x = randn(200, 32, seed=0)
    a = x.to(DEV).requires_grad_()
    out = tp.euclidean_distances(a)
    g = randn(200, 200, seed=2)
    out.backward(g.to(DEV))
    ra = x.double().requires_grad_()
    ref = torch.cdist(ra, ra, 2)
    ref.backward(g.double())
    # diagonal: the reference's ratio uses res == 0 masking; away from it both agree
    assert_close(a.grad, ra.grad, rtol=1e-3, atol=1e-3 * float(ra.grad.abs().max()), what="self grad")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fn", ["cosine_distances", "cosine_similarity", "correlation_distances"])
def test_cosine_family(dtype, fn):
    x1 = randn(2, 150, 256, seed=0, dtype=dtype)
    x2 = randn(2, 100, 256, seed=1, dtype=dtype)
    a = x1.to(DEV).requires_grad_()
    b = x2.to(DEV).requires_grad_()
    out = getattr(tp, fn)(a, b)
    g = randn(*out.shape, seed=2, dtype=dtype)
    out.backward(g.to(DEV))
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    if fn == "correlation_distances":
        ca, cb = ra - ra.mean(-1, keepdim=True), rb - rb.mean(-1, keepdim=True)
        ref = 1 - P.cosine_similarity(ca, cb)
    else:
        ref = getattr(P, fn)(ra, rb)
    ref.backward(g.double())
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    grtol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_close(out.float(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()) + 1e-6, what=fn)
    assert_close(a.grad.float(), ra.grad, rtol=grtol, atol=grtol * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad.float(), rb.grad, rtol=grtol, atol=grtol * float(rb.grad.abs().max()), what="grad x2")


def test_sqeuclidean_forward_backward():
    x1, x2 = randn(130, 64, seed=0), randn(70, 64, seed=1)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = tp.sqeuclidean_distances(a, b)
    g = randn(130, 70, seed=2)
    out.backward(g.to(DEV))
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    ref = ((ra[:, None, :] - rb[None, :, :]) ** 2).sum(-1)
    ref.backward(g.double())
    assert_close(out, ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()), what="sqeuclidean")
    assert_close(a.grad, ra.grad, rtol=1e-4, atol=1e-4 * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad, rb.grad, rtol=1e-4, atol=1e-4 * float(rb.grad.abs().max()), what="grad x2")


@pytest.mark.parametrize("n,m,d", [(260, 132, 128), (256, 200, 200), (130, 70, 96), (258, 131, 128)])
def test_sqeuclidean_and_rbf_backward_wide(n, m, d):
    """The p = 2 power-sum backward above 64 features: the wide kernel (n, m, d multiples of 4;
    it sums d g and doubles the sum) or, for the ragged shapes, the narrow kernel (2 d g per
    term).  Gradients against the float64 sum with the derived per-element bound of
    tests/_gradbound.py: each term 2 (a - b) g carries the subtraction's rounding (c_t = 2 to
    spare), the accumulation its six-sigma part.  rbf_kernel's backward reaches the same kernel
    with g' = -gamma exp(-gamma s) g."""
    from tests import _gradbound as GB
    print(f"sqeuclidean / rbf backward n={n} m={m} d={d}", flush=True)
    x1, x2 = randn(n, d, seed=10), randn(m, d, seed=11)
    g = randn(n, m, seed=12)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    gd = g.to(DEV)
    tp.sqeuclidean_distances(a, b).backward(gd)
    x1d, x2d, gdd = x1.double(), x2.double(), g.double()
    # grad_x1[i, k] = sum_j 2 (x1[i, k] - x2[j, k]) g[i, j]; grad_x2 by symmetry with g^T
    for own, other, gsl, got, nm in ((x1d, x2d, gdd, a.grad, "grad x1"), (x2d, x1d, gdd.T, b.grad, "grad x2")):
        terms = 2.0 * (own[:, None, :] - other[None, :, :]) * gsl[:, :, None]
        GB.check(got.cpu(), terms.sum(1), GB.sum_bound(terms, 1, 2.0), f"sqeuclidean {nm}")
    # rbf: out = exp(-gamma s); the same kernel, its g scaled per pair first
    a.grad = None
    b.grad = None
    out = tp.rbf_kernel(a, b, gamma=0.01)
    out.backward(gd)
    ra, rb = x1d.clone().requires_grad_(), x2d.clone().requires_grad_()
    ref = torch.exp(-0.01 * ((ra[:, None, :] - rb[None, :, :]) ** 2).sum(-1))
    ref.backward(gdd)
    assert_close(a.grad, ra.grad, rtol=1e-4, atol=1e-4 * float(ra.grad.abs().max()), what="rbf grad x1")
    assert_close(b.grad, rb.grad, rtol=1e-4, atol=1e-4 * float(rb.grad.abs().max()), what="rbf grad x2")


@pytest.mark.parametrize("kind", [capi.KER_RBF, capi.KER_LAPLACIAN])
@pytest.mark.parametrize("B,n,m,d,outside", [(1, 260, 132, 128, False), (2, 130, 70, 96, False),
                                             (1, 258, 131, 40, False), (1, 260, 132, 128, True)])
def test_exp_kernel_backward_fused_matches_composite(kind, B, n, m, d, outside):
    """tpw_pairwise_exp_kernel_backward forms each pair's gradient (grad * out) * -gamma inside
    the backward kernels (rbf; laplacian on the wide kernel's shapes) or in one elementwise pass
    (laplacian elsewhere); the composite multiplies in two ATen passes and calls the distance's
    backward entry point (tpw_ppminkowski_backward p = 2, tpw_lp_distances_backward2 p = 1).
    Same weights, same kernels, same order of sums: bit-identical.  Shapes: the wide kernels
    (n, m, d multiples of 4), batched, and ragged rows with d <= 64 (narrow kernels); with
    `outside`, one x2 value of 2^60 sends laplacian's p = 1 backward to its narrow instance."""
    print(f"exp kernel backward kind={kind} B={B} n={n} m={m} d={d} outside={outside}", flush=True)
    gamma = 0.02 if kind == capi.KER_RBF else 0.05
    x1 = randn(B, n, d, seed=20).to(DEV)
    x2 = randn(B, m, d, seed=21)
    if outside:
        x2[0, 7, 5] = 2.0 ** 60
    x2 = x2.to(DEV)
    g = randn(B, n, m, seed=22).to(DEV)
    out = capi.pairwise_exp_kernel(x1, x2, kind, gamma)
    gx1, gx2 = capi.pairwise_exp_kernel_backward(g, out, x1, x2, kind, gamma)
    gf = g.mul(out).mul(-gamma)
    if kind == capi.KER_RBF:
        rx1, rx2 = capi.family_backward(capi.FAM_PPMINKOWSKI, gf, x1, x2, p=2.0)
    else:
        rx1, rx2 = capi.lp_distances_backward2(gf, x1, x2, capi.lp_distances(x1, x2, 1.0), 1.0)
    assert_equal(gx1, rx1, what="grad x1")
    assert_equal(gx2, rx2, what="grad x2")
    # through the public op and autograd (fp32 on the GPU takes the fused route)
    fn = tp.rbf_kernel if kind == capi.KER_RBF else tp.laplacian_kernel
    a, b = x1.clone().requires_grad_(), x2.clone().requires_grad_()
    fn(a, b, gamma=gamma).backward(g)
    assert_equal(a.grad, rx1, what="autograd grad x1")
    assert_equal(b.grad, rx2, what="autograd grad x2")


@pytest.mark.parametrize("fn,p", [("manhattan_distances", 1.0), ("chebyshev_distances", float("inf")),
                                  ("minkowski_distances", 3.0), ("minkowski_distances", 1.5),
                                  ("linf_distances", float("inf")), ("l1_distances", 1.0)])
def test_minkowski_family(fn, p):
    x1 = rand(2, 130, 128, seed=0) * 2 - 1
    x2 = rand(2, 77, 128, seed=1) * 2 - 1
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = getattr(tp, fn)(a, b, p) if fn == "minkowski_distances" else getattr(tp, fn)(a, b)
    g = torch.ones(out.shape)
    out.backward(g.to(DEV))
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    ref = torch.cdist(ra, rb, p)
    ref.backward(g.double())
    assert_close(out, ref, rtol=1e-5, atol=1e-6 * float(ref.abs().max()), what=fn)
    assert_close(a.grad, ra.grad, rtol=1e-4, atol=1e-5 * float(ra.grad.abs().max()) + 1e-6, what="grad x1")
    assert_close(b.grad, rb.grad, rtol=1e-4, atol=1e-5 * float(rb.grad.abs().max()) + 1e-6, what="grad x2")


def test_small_euclidean_uses_direct_sum():
    # <= 25 rows on both sides: at::cdist's direct path (exact zeros on the diagonal)
    x = randn(20, 16, seed=0)
    out = tp.euclidean_distances(x.to(DEV))
    assert torch.all(out.diagonal() == 0)
    assert_close(out, torch.cdist(x.double(), x.double()), rtol=1e-5, atol=1e-6, what="small euclidean")


@pytest.mark.parametrize("shape", [((2, 300, 1024), (2, 200, 1024)), ((130, 77), (257, 77))])
def test_boolean_metrics_bit_exact(shape):
    b1 = rand(*shape[0], seed=0) < 0.5
    b2 = rand(*shape[1], seed=1) < 0.1
    assert_equal(tp.hamming_distances(b1.to(DEV), b2.to(DEV)),
                 torch.from_numpy(P.hamming_distances(b1.numpy(), b2.numpy())), "hamming")
    assert_equal(tp.jaccard_distances(b1.to(DEV), b2.to(DEV)),
                 torch.from_numpy(P.jaccard_distances(b1.numpy(), b2.numpy())), "jaccard")
    for name in ("pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean", "pwne_mean"):
        got = getattr(tp, name)(b1.to(DEV), b2.to(DEV))
        assert_equal(got, getattr(tp, name)(b1, b2), name)


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32, torch.float32, torch.float16, torch.uint8])
def test_hamming_non_bool(dtype):
    g = torch.Generator().manual_seed(0)
    x1 = torch.randint(0, 3, (70, 33), generator=g).to(dtype)
    x2 = torch.randint(0, 3, (50, 33), generator=g).to(dtype)
    got = tp.hamming_distances(x1.to(DEV), x2.to(DEV))
    assert_equal(got, torch.from_numpy(P.hamming_distances(x1.numpy(), x2.numpy())), f"hamming {dtype}")


@pytest.mark.parametrize("name", ["dice", "rogerstanimoto", "russellrao", "sokalmichener",
                                  "sokalsneath", "yule", "kulczynski1"])
def test_boolean_family_gpu_equals_cpu(name):
    b1 = rand(60, 100, seed=0) < 0.5
    b2 = rand(50, 100, seed=1) < 0.5
    fn = getattr(tp, f"{name}_distances")
    if name == "russellrao":
        # (D - and_count) / D: ATen divides a GPU tensor by a scalar as a multiply by the
        # reciprocal, its CPU kernel divides; the counts themselves are exact (1 ulp apart)
        assert_close(fn(b1.to(DEV), b2.to(DEV)), fn(b1, b2), rtol=1.2e-7, atol=0, what=name)
        return
    assert_equal(fn(b1.to(DEV), b2.to(DEV)), fn(b1, b2), name)


def test_prf_div_family_gpu(tmp_path):
    """The 20 prf_div-family schemas on GPU tensors (forward, autograd backward, in-place, the
    backward ops called directly; four float dtypes, zeros of both signs, NaN, +-inf,
    integer promotion, errors) bit for bit against the oracle's numpy restatement and, where
    oracle/_ref is built, against the reference's own compiled CPU kernels run in a child
    process (csrc/ops/cpu/prf_div_kernel.cpp, autograd/prf_div_kernel.cpp)."""
    from oracle import ref_runner
    from tests._prf_cases import assert_same_result, cases, oracle_result

    cs = cases()
    ref = ref_runner.run_prf_reference(cs, tmp_path) if ref_runner.available() else [None] * len(cs)
    ops = torch.ops.torchpairwise
    checked_oracle = 0
    for (case, a, b, g), r in zip(cs, ref):
        ours = ref_runner.run_prf_case(ops, case, a, b, g, DEV)
        want = oracle_result(case, a, b, g)
        if want is not None:
            assert "err" not in ours, f"{case}: {ours.get('err')}"
            assert_same_result({k: v for k, v in ours.items() if k in want}, want, f"oracle {case}")
            checked_oracle += 1
        if r is not None:
            assert_same_result(ours, r, f"reference {case}")
    assert checked_oracle >= 240


def test_hausdorff_ops_bit_exact_and_grad():
    c1, c2 = rand(2, 400, 3, seed=0), rand(3, 300, 3, seed=1) + 0.05
    a = c1.to(DEV).requires_grad_()
    b = c2.to(DEV).requires_grad_()
    out, i1, i2 = tp.directed_hausdorff_distances(a, b)
    w = cref.directed_hausdorff(c1.numpy(), c2.numpy())
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(want), nm)
    g = randn(2, 3, seed=5)
    out.backward(g.to(DEV))
    ca, cb = c1.clone().requires_grad_(), c2.clone().requires_grad_()
    tp.directed_hausdorff_distances(ca, cb)[0].backward(g)
    assert_equal(a.grad, ca.grad, "grad x1 (GPU vs CPU op)")
    assert_equal(b.grad, cb.grad, "grad x2 (GPU vs CPU op)")


def test_hausdorff_shuffle_generator_replay():
    c1, c2 = rand(2, 2, 200, 3, seed=0), rand(2, 2, 250, 3, seed=1)
    gen = torch.Generator(device=DEV).manual_seed(3)
    out, i1, i2 = tp.directed_hausdorff_distances(c1.to(DEV), c2.to(DEV), shuffle=True, generator=gen)
    gen2 = torch.Generator(device=DEV).manual_seed(3)
    perm1 = torch.empty((2, 200), dtype=torch.int64, device=DEV)
    perm2 = torch.empty((2, 250), dtype=torch.int64, device=DEV)
    for bb in range(2):
        torch.randperm(200, generator=gen2, out=perm1[bb])
        torch.randperm(250, generator=gen2, out=perm2[bb])
    w = cref.directed_hausdorff(c1.numpy(), c2.numpy(), perm1.cpu().numpy(), perm2.cpu().numpy())
    for got, want, nm in zip((out, i1, i2), w, ("value", "idx1", "idx2")):
        assert_equal(got, torch.from_numpy(want), f"shuffled {nm}")


@pytest.mark.parametrize("shuffle,with_gen", [(False, False), (True, True), (True, False)])
def test_hausdorff_autograd_equals_recomputing_backward(shuffle, with_gen):
    """The autograd backward reuses the forward's output and indices where the reference's
    re-run of the forward would reproduce them (no shuffle, or a replayed generator); the
    gradients must equal those of __directed_hausdorff_backward, which re-runs it, bit for bit.
    A shuffle from the default generator keeps the re-run (checked to run, not compared: its
    permutation is a new draw)."""
    c1, c2 = rand(2, 2, 300, 3, seed=10), rand(2, 3, 260, 3, seed=11) + 0.05
    g = randn(2, 2, 3, seed=12).to(DEV)
    a, b = c1.to(DEV).requires_grad_(), c2.to(DEV).requires_grad_()
    gen = torch.Generator(device=DEV).manual_seed(7) if with_gen else None
    out = tp.directed_hausdorff_distances(a, b, shuffle=shuffle, generator=gen)[0]
    out.backward(g)
    if shuffle and not with_gen:
        assert torch.isfinite(a.grad).all() and torch.isfinite(b.grad).all()
        return
    gen2 = torch.Generator(device=DEV).manual_seed(7) if with_gen else None  # the forward's state
    gx1, gx2 = torch.ops.torchpairwise.__directed_hausdorff_backward(
        g, c1.to(DEV), c2.to(DEV), shuffle=shuffle, generator=gen2)
    assert_equal(a.grad, gx1, "grad x1 (saved indices vs re-run)")
    assert_equal(b.grad, gx2, "grad x2 (saved indices vs re-run)")


def test_empty_inputs():
    e = torch.zeros((0, 8), device=DEV)
    x = torch.randn(5, 8, device=DEV)
    assert tp.euclidean_distances(e, x).shape == (0, 5)
    assert tp.manhattan_distances(x, e).shape == (5, 0)
    assert tp.hamming_distances(e > 0, x > 0).shape == (0, 5)


# --------------------------------------------------------------------------------------
# cdist(metric=...) and the neighbour masks
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("metric,fn", [("euclidean", "euclidean_distances"), ("cosine", "cosine_distances"),
                                       ("cityblock", "manhattan_distances"), ("linf", "chebyshev_distances"),
                                       ("hamming", "hamming_distances")])
def test_cdist_dispatch_gpu(metric, fn):
    a, b = randn(70, 24, seed=0).to(DEV), randn(50, 24, seed=1).to(DEV)
    if metric == "hamming":
        a, b = a > 0, b > 0
    assert_equal(tp.cdist(a, b, metric), getattr(tp, fn)(a, b), metric)


@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "cosine", "minkowski"])
@pytest.mark.parametrize("k", [0, 1, 5, 20])
def test_k_neighbors_mask_gpu(metric, k):
    print(f"k_neighbors_mask {metric} k={k}", flush=True)
    x1, x2 = randn(300, 32, seed=0), randn(500, 32, seed=1)
    kw = {"p": 3.0} if metric == "minkowski" else {}
    got = tp.k_neighbors_mask(x1.to(DEV), x2.to(DEV), k, metric, **kw)
    assert got.dtype == torch.bool and got.shape == (300, 500)
    # selection: bit-exact against the oracle on the same (GPU-computed) distances
    dist = tp.cdist(x1.to(DEV), x2.to(DEV), metric, **kw).cpu()
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(dist.numpy(), k + 1)), "vs oracle")
    # and the reference's own CPU route, except where the boundary is a near-tie that
    # float rounding of the distances may flip
    ref = tp.k_neighbors_mask(x1, x2, k, metric, **kw)
    diff = (got.cpu() != ref).any(1)
    srt = dist.double().sort(1).values
    gap = (srt[:, k + 1] - srt[:, k]) / srt[:, k + 1].abs().clamp_min(1e-30)
    assert bool((gap[diff] < 1e-5).all()), f"{int(diff.sum())} rows differ beyond near-ties"


def test_k_neighbors_mask_gpu_ties_and_self():
    x = torch.randint(0, 3, (400, 8), generator=torch.Generator().manual_seed(3)).float()
    got = tp.k_neighbors_mask(x.to(DEV), None, 2, "manhattan")  # integer distances: many ties
    dist = tp.manhattan_distances(x.to(DEV)).cpu()
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(dist.numpy(), 3)), "ties")
    xb = x > 0
    got = tp.k_neighbors_mask(xb.to(DEV), None, 4, "hamming")
    assert_equal(got, torch.from_numpy(P.k_smallest_mask(tp.hamming_distances(xb).numpy(), 5)), "hamming")
    a = randn(64, 16, seed=4).to(DEV)
    assert torch.equal(tp.k_neighbors_mask(a, None, 0).cpu(), torch.eye(64, dtype=torch.bool))
    with pytest.raises(IndexError):  # k + 1 > M raises, as the reference's index_put_ does
        tp.k_neighbors_mask(a, a[:3], 3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shapes", [((300, 64), (256, 64)), ((2, 256, 128), None), ((300, 64), (200, 64)),
                                    ((2, 130, 48), (2, 96, 48)), ((40, 8), (20, 8)), ((2, 160, 64), (1, 136, 64)),
                                    ((300, 64), None), ((20, 16), (12, 16))])
def test_radius_mask_fused_equals_distances_le(dtype, shapes):
    """The euclidean radius mask straight from the MFMA epilogue (the tile kernel for output
    widths of whole 16-byte units, the register-staged kernel's byte stores otherwise, the
    unfused route at 25 rows or fewer) against the distances the op itself returns, compared
    with Tensor.le on the same device: bit for bit, eps = a middle distance and 0 (with
    x2 = None: exactly the zero distances)."""
    x1 = randn(*shapes[0], seed=0, dtype=dtype).to(DEV)
    x2 = None if shapes[1] is None else randn(*shapes[1], seed=1, dtype=dtype).to(DEV)
    dist = tp.euclidean_distances(x1, x2)
    for eps in (float(dist.float().median()), 0.0):
        got = tp.radius_neighbors_mask(x1, x2, eps)
        want = dist.le(eps)
        assert got.dtype == torch.bool and got.shape == want.shape
        assert torch.equal(got, want), f"eps={eps}: {int((got != want).sum())} differences"


def test_radius_neighbors_mask_gpu():
    x1, x2 = randn(200, 16, seed=0), randn(300, 16, seed=1)
    got = tp.radius_neighbors_mask(x1.to(DEV), x2.to(DEV), 5.0)
    dist = tp.euclidean_distances(x1.to(DEV), x2.to(DEV)).cpu()
    assert_equal(got, torch.from_numpy(P.radius_mask(dist.numpy(), 5.0)), "radius")


# --------------------------------------------------------------------------------------
# the reference's VALU family through the drop-in ops
# --------------------------------------------------------------------------------------
# ops whose reference kernels dispatch floating types and half only (no bfloat16), by the
# kernel name of their refusal (cuda/<op>_kernel.cu)
NO_BF16 = {"canberra_distances": "_canberra", "braycurtis_distances": "_braycurtis",
           "additive_chi2_kernel": "_additive_chi2_kernel", "chi2_kernel": "_additive_chi2_kernel",
           "jensenshannon_distances": "_sqjensenshannon", "snr_distances": "_snr"}


def _refused_bf16(name, dtype, args):
    """bfloat16 where the reference's kernel refuses it: the same NotImplementedError."""
    if dtype != torch.bfloat16 or name not in NO_BF16:
        return False
    with pytest.raises(NotImplementedError, match=f'"{NO_BF16[name]}_forward_cuda" not implemented for'):
        getattr(tp, name)(*args)
    return True


@pytest.mark.parametrize("name", ["sqeuclidean_distances", "canberra_distances", "braycurtis_distances",
                                  "wminkowski_distances", "seuclidean_distances"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_family_ops_gpu(name, dtype):
    print(f"{name} {dtype}", flush=True)
    x1, x2 = randn(150, 24, seed=0, dtype=dtype), randn(90, 24, seed=1, dtype=dtype)
    if _refused_bf16(name, dtype, (x1.to(DEV), x2.to(DEV))):
        return
    w = (rand(24, seed=2) + 0.2).to(dtype)
    extra = {"wminkowski_distances": (3.0, w), "seuclidean_distances": (w,)}.get(name, ())
    fn = getattr(tp, name)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = fn(a, b, *[e.to(DEV) if torch.is_tensor(e) else e for e in extra])
    assert out.dtype == dtype
    g = randn(150, 90, seed=3)
    out.backward(g.to(DEV, dtype))
    ra, rb = x1.double().requires_grad_(), x2.double().requires_grad_()
    ref = fn(ra, rb, *[e.double() if torch.is_tensor(e) else e for e in extra])  # CPU = reference loops
    ref.backward(g.double())
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    grtol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_close(out.float(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what=name)
    assert_close(a.grad.float(), ra.grad, rtol=grtol, atol=grtol * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad.float(), rb.grad, rtol=grtol, atol=grtol * float(rb.grad.abs().max()), what="grad x2")


def test_family_ops_gpu_equal_reference(tmp_path):
    """The reference's internal metric ops on GPU float32 tensors (forward and autograd
    backward) against its own compiled CPU kernels on the same float32 inputs (oracle/_ref):
    values rtol 1e-5, gradients 1e-4 (each + rtol * max); the p = +-inf gradients of x1 and x2
    (first arg-extremum, summed in the reference's order) bit for bit."""
    from oracle import ref_runner
    from tests._family_cases import family_cases
    from tests.test_reference_pin import _assert_results_close

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = family_cases(torch.float32)
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    for (case, tensors), r in zip(cs, ref):
        what = f"{case['op']} {case['kind']} {[tuple(t.shape) for t in tensors.values()]}"
        print(what, flush=True)
        ours = ref_runner.run_op_case(ops, case, tensors, DEV)
        inf = case["kind"] in ("p=inf", "p=-inf")
        exact = ("grad_a", "grad_b") if inf else ()
        _assert_results_close({k: v for k, v in ours.items() if k.startswith("out")},
                              {k: v for k, v in r.items() if k.startswith("out")}, 1e-5, what)
        _assert_results_close({k: v for k, v in ours.items() if k.startswith("grad")},
                              {k: v for k, v in r.items() if k.startswith("grad")}, 1e-4, what, exact)


def test_lp_inf_backward_long_rows_equal_reference(tmp_path):
    """The p = +-inf backward past the LDS accumulator's size (4096 features, 2048 weighted):
    _ppminkowski and _wminkowski at d = 5000 with random and tie-heavy integer inputs against
    the reference's compiled CPU kernels (oracle/_ref); grad_x1 and grad_x2 bit for bit, the
    weight gradient rtol 1e-4, the forward rtol 1e-5."""
    from oracle import ref_runner
    from tests._family_cases import _g, _inputs
    from tests.test_reference_pin import _assert_results_close

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    d = 5000
    cs = []
    for kind in ("normal", "ties"):
        a, b, g = _inputs((21, d), (13, d), torch.float32, 7, kind)
        w = torch.rand((d,), generator=_g(8), dtype=torch.float64).float() + 0.25
        for p in (float("inf"), float("-inf")):
            cs.append(({"op": "_ppminkowski", "args": [{"t": "a"}, {"t": "b"}, {"v": p}], "req": ["a", "b"],
                        "grad": "g", "kind": f"p={p} {kind}"}, {"a": a, "b": b, "g": g}))
            cs.append(({"op": "_wminkowski", "args": [{"t": "a"}, {"t": "b"}, {"t": "w"}, {"v": p}],
                        "req": ["a", "b", "w"], "grad": "g", "kind": f"p={p} {kind}"},
                       {"a": a, "b": b, "w": w, "g": g}))
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    for (case, tensors), r in zip(cs, ref):
        what = f"{case['op']} {case['kind']} d={d}"
        print(what, flush=True)
        ours = ref_runner.run_op_case(ops, case, tensors, DEV)
        _assert_results_close({k: v for k, v in ours.items() if k.startswith("out")},
                              {k: v for k, v in r.items() if k.startswith("out")}, 1e-5, what)
        _assert_results_close({k: v for k, v in ours.items() if k.startswith("grad")},
                              {k: v for k, v in r.items() if k.startswith("grad")}, 1e-4, what,
                              ("grad_a", "grad_b"))


def test_other_gpu_dtypes_served():
    """The cdist metrics, cosine, linear and Mahalanobis run float64 on the GPU (the VALU family,
    haversine and directed Hausdorff: test_gpu_float64.py)."""
    x1, x2 = torch.randn(9, 5, dtype=torch.float64), torch.randn(7, 5, dtype=torch.float64)
    VI = torch.eye(5, dtype=torch.float64) * 2
    for name, args in (("euclidean_distances", ()), ("manhattan_distances", ()), ("chebyshev_distances", ()),
                       ("cosine_distances", ()), ("linear_kernel", ()), ("mahalanobis_distances", (VI,))):
        got = getattr(tp, name)(x1.to(DEV), x2.to(DEV), *[a.to(DEV) for a in args])
        want = getattr(tp, name)(x1, x2, *args)  # CPU: the reference's route
        assert got.dtype == torch.float64
        assert_close(got, want, rtol=1e-12, atol=1e-12 * float(want.abs().max()), what=name)


def test_public_ops_gpu_equal_reference(tmp_path):
    """Every public op on GPU tensors (the 39 metrics, cdist, the neighbour masks, pdist's error)
    against the reference's compiled CPU library on the same inputs: float values rtol 1e-5,
    gradients 1e-4 (each + rtol * max), boolean metrics, directed Hausdorff (value, indices,
    gradients) and the masks bit for bit, and the same error messages."""
    from oracle import ref_runner
    from tests.test_reference_pin import _check_public_cases

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    _check_public_cases(torch.ops.torchpairwise, DEV, tmp_path, rtol=1e-5, grad_rtol=1e-4)


@pytest.mark.parametrize("fn,p", [("manhattan_distances", 1.0), ("chebyshev_distances", float("inf")),
                                  ("minkowski_distances", 3.0)])
def test_bf16_lp_output_written_by_the_kernel(fn, p):
    """bf16 cdist metrics without a gradient to form: the kernel rounds its fp32 result to bf16
    and writes it once; bit for bit what the fp32 kernel plus a bf16 conversion gives (the route
    taken when a gradient is needed), including a ragged row length and NaN rows."""
    x1 = randn(300, 70, seed=0).bfloat16()
    x2 = randn(257, 70, seed=1).bfloat16()
    x1[5, 3] = float("nan")
    a, b = x1.to(DEV), x2.to(DEV)
    args = (p,) if fn == "minkowski_distances" else ()
    with torch.no_grad():
        got = getattr(tp, fn)(a, b, *args)
    want = capi.lp_distances(a.float(), b.float(), p).to(torch.bfloat16)
    assert got.dtype == torch.bfloat16
    assert_equal(got, want, f"{fn} bf16")
    # with a gradient to form the autograd route runs; same values
    ag = a.clone().requires_grad_()
    out = getattr(tp, fn)(ag, b, *args)
    assert_equal(out.detach(), want, f"{fn} bf16 autograd route")


def test_snr_fused_equals_composition():
    """_snr on float32 GPU tensors: the squared distances of the centred rows and the divide in
    one pass (tpw_snr_centered), bit for bit the composition it replaces (variance numerator over
    _ppminkowski p = 2, an IEEE divide), batched and not."""
    ops = torch.ops.torchpairwise
    for s1, s2 in (((130, 33), (257, 33)), ((2, 40, 17), (2, 50, 17))):
        x1, x2 = randn(*s1, seed=3).to(DEV), randn(*s2, seed=4).to(DEV)
        got = ops._snr(x1, x2)
        a, b = x1 - x1.mean(-1, True), x2 - x2.mean(-1, True)
        want = (a * a).sum(-1, True) / ops._ppminkowski(a, b, 2.0)
        assert_equal(got, want, f"snr {s1}")


def test_sqeuclidean_identical_points_are_zero():
    x = randn(200, 64, seed=5).to(DEV)
    d = tp.sqeuclidean_distances(x)
    assert bool((torch.diagonal(d) == 0).all())  # direct sum: no |a|^2 + |b|^2 - 2ab residue
    assert bool((torch.diagonal(tp.sqeuclidean_distances(x.double())) == 0).all())


# --------------------------------------------------------------------------------------
# chi2, jensenshannon, haversine, snr, mahalanobis through the drop-in ops; the CPU op in
# float64 (the reference's loops) is the bar, forward and backward
# --------------------------------------------------------------------------------------
def _special_case(name, dtype):
    gen = torch.Generator().manual_seed(7)
    if name in ("additive_chi2_kernel", "chi2_kernel", "jensenshannon_distances"):
        x1, x2 = torch.rand(150, 24, generator=gen) + 0.05, torch.rand(90, 24, generator=gen) + 0.05
    elif name == "haversine_distances":
        u1, u2 = torch.rand(150, 2, generator=gen), torch.rand(90, 2, generator=gen)
        scale, shift = torch.tensor([np.pi, 2 * np.pi]), torch.tensor([np.pi / 2, np.pi])
        x1, x2 = u1 * scale - shift, u2 * scale - shift
    else:
        x1, x2 = torch.randn(150, 24, generator=gen), torch.randn(90, 24, generator=gen)
    extra = ()
    if name == "chi2_kernel":
        extra = (0.3,)
    elif name == "jensenshannon_distances":
        extra = (2.0,)  # base
    elif name == "mahalanobis_distances":
        a = torch.randn(24, 24, generator=gen)
        extra = (a @ a.T / 24 + torch.eye(24),)
    return x1.to(dtype), x2.to(dtype), extra


@pytest.mark.parametrize("name", ["additive_chi2_kernel", "chi2_kernel", "jensenshannon_distances",
                                  "haversine_distances", "snr_distances", "mahalanobis_distances"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_special_ops_gpu(name, dtype):
    print(f"{name} {dtype}", flush=True)
    x1, x2, extra = _special_case(name, dtype)
    if _refused_bf16(name, dtype, (x1.to(DEV), x2.to(DEV), *[e.to(DEV, dtype) if torch.is_tensor(e) else e
                                                               for e in extra])):
        return
    fn = getattr(tp, name)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    dev_extra = [e.to(DEV, dtype) if torch.is_tensor(e) else e for e in extra]
    out = fn(a, b, *dev_extra)
    assert out.dtype == dtype
    g = randn(150, 90, seed=3)
    out.backward(g.to(DEV, dtype))
    ra, rb = x1.detach().double().requires_grad_(), x2.detach().double().requires_grad_()
    ref = fn(ra, rb, *[e.to(dtype).double() if torch.is_tensor(e) else e for e in extra])
    ref.backward(g.double())
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    grtol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_close(out.float(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what=name)
    assert_close(a.grad.float(), ra.grad, rtol=grtol, atol=grtol * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad.float(), rb.grad, rtol=grtol, atol=grtol * float(rb.grad.abs().max()), what="grad x2")


def test_special_ops_gpu_batched_and_cdist():
    gen = torch.Generator().manual_seed(8)
    x1, x2 = torch.randn(2, 40, 6, generator=gen), torch.randn(2, 30, 6, generator=gen)
    a = torch.randn(2, 6, 6, generator=gen)
    VI = a @ a.transpose(1, 2) + torch.eye(6)
    ops = torch.ops.torchpairwise
    for got, ref in ((ops._snr(x1.to(DEV), x2.to(DEV)), ops._snr(x1.double(), x2.double())),
                     (ops._sqmahalanobis(x1.to(DEV), x2.to(DEV), VI.to(DEV)),
                      ops._sqmahalanobis(x1.double(), x2.double(), VI.double())),
                     (ops._haversine(x1[..., :2].to(DEV), x2[..., :2].to(DEV)),
                      ops._haversine(x1[..., :2].double(), x2[..., :2].double())),
                     (tp.cdist(x1[0].to(DEV), x2[0].to(DEV), "mahalanobis", VI=VI[0].to(DEV)),
                      tp.cdist(x1[0].double(), x2[0].double(), "mahalanobis", VI=VI[0].double()))):
        assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()), what="batched")
    # mahalanobis gradient of VI on the GPU (composite) against the CPU loop
    x, y, v = x1[0].to(DEV), x2[0].to(DEV), VI[0].to(DEV).requires_grad_()
    ops._sqmahalanobis(x, y, v).sum().backward()
    vr = VI[0].double().requires_grad_()
    ops._sqmahalanobis(x1[0].double(), x2[0].double(), vr).sum().backward()
    assert_close(v.grad.cpu(), vr.grad, rtol=1e-4, atol=1e-4 * float(vr.grad.abs().max()), what="grad VI")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_mahalanobis_self_and_near_duplicates(dtype):
    """mahalanobis_distances(x) with the default VI (inverse covariance): the diagonal is exactly
    0 and nothing is NaN; rows within 1e-3 of each other match the reference's per-pair loop
    (the CPU op, cpu/sqmahalanobis_kernel.cpp:13-33, evaluated in float64)."""
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(2000, 24, generator=gen).to(dtype)
    VI = torch.cov(x.double().T).inverse().T.contiguous()
    # bf16: at::cov(...).inverse() of the default VI raises for 16-bit types (as in the
    # reference's functor), so VI is passed
    kw = {"VI": VI.to(dtype).to(DEV)} if dtype == torch.bfloat16 else {}
    d = tp.mahalanobis_distances(x.to(DEV), **kw)
    assert d.dtype == dtype and not bool(torch.isnan(d).any())
    assert bool((torch.diagonal(d) == 0).all())
    near = (x.double() + 1e-3 * torch.randn(2000, 24, generator=gen, dtype=torch.float64)).to(dtype)
    a, b, v = x[:300], near[:200], VI.to(dtype)
    got = torch.ops.torchpairwise._sqmahalanobis(a.to(DEV), b.to(DEV), v.to(DEV))
    ref = torch.ops.torchpairwise._sqmahalanobis(a.double(), b.double(), v.double())
    assert bool((got >= 0).all())  # VI is positive definite
    rtol = {torch.float32: 1e-5, torch.float64: 1e-12, torch.bfloat16: 1e-2}[dtype]
    assert_close(got.double(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what="near rows")
    # the near pairs themselves (|d| ~ 1e-3 |x|): relative accuracy, not just absolute
    idx = torch.arange(200)
    pair = got.double().cpu()[idx, idx]
    want = ref[idx, idx]
    assert_close(pair, want, rtol=64 * rtol if dtype != torch.bfloat16 else 1e-2, atol=0, what="near pairs")


def test_sqmahalanobis_capi_shapes():
    """tpw_sqmahalanobis through the C ABI: edge tiles, d not a multiple of 16, d = 0, x2 the
    same buffer as x1, batched VI, float64."""
    from torchpairwise_amd import _capi as capi

    gen = torch.Generator().manual_seed(12)
    for B, n, m, d, dt in ((1, 65, 130, 17, torch.float32), (3, 7, 5, 1, torch.float32), (2, 40, 33, 0, torch.float32),
                           (2, 64, 64, 16, torch.float64), (1, 129, 1, 48, torch.float64)):
        x1 = torch.randn(B, n, d, generator=gen, dtype=dt)
        x2 = torch.randn(B, m, d, generator=gen, dtype=dt)
        VI = torch.randn(B, d, d, generator=gen, dtype=dt)
        code = capi.TPW_F32 if dt == torch.float32 else capi.TPW_F64
        for same in (False, True):
            a = x1.to(DEV)
            b = a if same else x2.to(DEV)
            mm = n if same else m
            out = torch.full((B, n, mm), float("nan"), dtype=dt, device=DEV)
            ws = torch.empty(max(1, capi.lib().tpw_sqmahalanobis_workspace_size(code, B, n, mm, d)),
                             dtype=torch.uint8, device=DEV)
            capi.call("tpw_sqmahalanobis", a.data_ptr(), b.data_ptr(), VI.to(DEV).data_ptr(), code, B, n, mm, d,
                      out.data_ptr(), ws.data_ptr(), capi._stream())
            want = P.sqmahalanobis(x1.double(), (x1 if same else x2).double(), VI.double())
            tol = 1e-5 if dt == torch.float32 else 1e-12
            assert_close(out.cpu().double(), want, rtol=tol, atol=tol * float(want.abs().max()) + 1e-30,
                         what=f"B={B} n={n} m={mm} d={d} same={same}")
            if same:
                assert bool((torch.diagonal(out, dim1=1, dim2=2) == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [((150, 24), (90, 24)), ((2, 130, 64), (2, 70, 64)), ((300, 128), None)])
def test_linear_kernel_gpu(dtype, shape):
    """linear_kernel on the MFMA kernel (DOT epilogue) and its backward on the matrix cores,
    against the reference's x1 @ x2^T and autograd in float64 (pairwise_metrics.cpp:58-65)."""
    x1 = randn(*shape[0], seed=0, dtype=dtype)
    x2 = None if shape[1] is None else randn(*shape[1], seed=1, dtype=dtype)
    a = x1.to(DEV).requires_grad_()
    b = None if x2 is None else x2.to(DEV).requires_grad_()
    out = tp.linear_kernel(a, b)
    assert out.dtype == dtype
    g = randn(*out.shape, seed=3)
    out.backward(g.to(DEV, dtype))
    ra = x1.double().requires_grad_()
    rb = None if x2 is None else x2.double().requires_grad_()
    ref = tp.linear_kernel(ra, rb)  # CPU: the reference's matmul
    ref.backward(g.double())
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert_close(out.float(), ref, rtol=tol, atol=tol * float(ref.abs().max()), what="linear_kernel")
    gt = 1e-4 if dtype == torch.float32 else 1e-2
    assert_close(a.grad.float(), ra.grad, rtol=gt, atol=gt * float(ra.grad.abs().max()), what="grad x1")
    if b is not None:
        assert_close(b.grad.float(), rb.grad, rtol=gt, atol=gt * float(rb.grad.abs().max()), what="grad x2")


# --------------------------------------------------------------------------------------
# polynomial_kernel / sigmoid_kernel: the function fused into the MFMA epilogue; the
# reference's composite (matmul, mul_, add_, pow_ / tanh_) in float64 on the CPU is the bar
# fp32: values rtol 1e-4 (+ atol 1e-5 * max); grads rtol 1e-4 (+ atol 1e-4 * max)
# bf16: 1e-2 (+ 1e-2 * max) for values and grads
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,kw", [("polynomial_kernel", dict(degree=3)),
                                     ("polynomial_kernel", dict(degree=2, gamma=0.3, coef0=0.5)),
                                     ("polynomial_kernel", dict(degree=4, coef0=-0.25)),
                                     ("polynomial_kernel", dict(degree=1)),
                                     ("polynomial_kernel", dict(degree=0)),
                                     ("sigmoid_kernel", dict()),
                                     ("sigmoid_kernel", dict(gamma=0.05, coef0=-0.3))])
def test_kernel_functions_gpu(dtype, name, kw):
    print(f"{name} {kw} {dtype}", flush=True)
    x1, x2 = randn(150, 24, seed=0, dtype=dtype), randn(90, 24, seed=1, dtype=dtype)
    fn = getattr(tp, name)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = fn(a, b, **kw)
    assert out.dtype == dtype
    g = randn(150, 90, seed=3)
    out.backward(g.to(DEV, dtype))
    ra, rb = x1.detach().double().requires_grad_(), x2.detach().double().requires_grad_()
    ref = fn(ra, rb, **kw)  # CPU float64: the reference's composite
    ref.backward(g.double())
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    atol_v = (1e-5 if dtype == torch.float32 else 1e-2) * float(ref.abs().max())
    assert_close(out.float(), ref, rtol=tol, atol=atol_v, what=name)
    for got, want, nm in ((a.grad, ra.grad, "grad x1"), (b.grad, rb.grad, "grad x2")):
        assert_close(got.float(), want, rtol=tol, atol=tol * float(want.abs().max()) + 1e-30, what=nm)


def test_kernel_functions_gpu_batched_and_self():
    x1 = randn(2, 130, 40, seed=4).to(DEV)
    x2 = randn(2, 70, 40, seed=5).to(DEV)
    for name, kw in (("polynomial_kernel", dict(degree=3)), ("sigmoid_kernel", dict())):
        fn = getattr(tp, name)
        ref = fn(x1.cpu().double(), x2.cpu().double(), **kw)
        assert_close(fn(x1, x2, **kw).cpu(), ref, rtol=1e-4, atol=1e-5 * float(ref.abs().max()), what=name)
        ref = fn(x1[0].cpu().double(), None, **kw)
        assert_close(fn(x1[0], None, **kw).cpu(), ref, rtol=1e-4, atol=1e-5 * float(ref.abs().max()),
                     what=f"{name} x2=None")


# --------------------------------------------------------------------------------------
# rbf_kernel / laplacian_kernel: exp(-gamma * distance) fused into the VALU kernel; the
# reference's composite in float64 on the CPU is the bar (fp32 rtol 1e-5 values, 1e-4 grads;
# bf16 1e-2 for both)
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,gamma", [("rbf_kernel", None), ("rbf_kernel", 0.2), ("rbf_kernel", 0.0),
                                        ("laplacian_kernel", None), ("laplacian_kernel", 0.05)])
def test_exp_kernels_gpu(dtype, name, gamma):
    print(f"{name} gamma={gamma} {dtype}", flush=True)
    x1, x2 = randn(150, 24, seed=0, dtype=dtype), randn(90, 24, seed=1, dtype=dtype)
    fn = getattr(tp, name)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = fn(a, b, gamma)
    assert out.dtype == dtype
    g = randn(150, 90, seed=3)
    out.backward(g.to(DEV, dtype))
    ra, rb = x1.detach().double().requires_grad_(), x2.detach().double().requires_grad_()
    ref = fn(ra, rb, gamma)
    ref.backward(g.double())
    rtol, grtol = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    assert_close(out.float(), ref, rtol=rtol, atol=rtol * float(ref.abs().max()), what=name)
    for got, want, nm in ((a.grad, ra.grad, "grad x1"), (b.grad, rb.grad, "grad x2")):
        assert_close(got.float(), want, rtol=grtol, atol=grtol * float(want.abs().max()) + 1e-30, what=nm)


def test_exp_kernels_gpu_batched_and_capi():
    from torchpairwise_amd import _capi as capi
    x1, x2 = randn(2, 130, 40, seed=4), randn(2, 70, 40, seed=5)
    for name, kind in (("rbf_kernel", capi.KER_RBF), ("laplacian_kernel", capi.KER_LAPLACIAN)):
        fn = getattr(tp, name)
        ref = fn(x1.double(), x2.double(), 0.03)
        assert_close(fn(x1.to(DEV), x2.to(DEV), 0.03).cpu(), ref, rtol=1e-5, atol=1e-6, what=name)
        got = capi.pairwise_exp_kernel(x1.to(DEV), x2.to(DEV), kind, 0.03)
        assert_close(got.cpu(), ref, rtol=1e-5, atol=1e-6, what=f"{name} C ABI")


# --------------------------------------------------------------------------------------
# unreduced pairwise binary ops (pwand ... pwge) on the HIP kernel
# --------------------------------------------------------------------------------------
def test_pw_binary_gpu_equal_cpu():
    """Every case of tests/_pw_binary_cases.py on the GPU against this build's CPU op (which
    test_pw_binary.py pins to the reference's compiled kernels): outputs and shapes bit for
    bit, the same errors (with the device in the dispatch name)."""
    from oracle import ref_runner
    from tests._pw_binary_cases import pw_binary_cases

    ops = torch.ops.torchpairwise
    for case, t in pw_binary_cases():
        ours = ref_runner.run_op_case(ops, case, t, DEV)
        want = ref_runner.run_op_case(ops, case, t, "cpu")
        what = f"{case['op']} {t['a'].dtype}/{t['b'].dtype} {tuple(t['a'].shape)} {tuple(t['b'].shape)}"
        if "err" in want or "err" in ours:
            assert ours.get("err", "").replace("_cuda", "_cpu") == want.get("err"), what
            continue
        assert ours["out0"].shape == want["out0"].shape and torch.equal(ours["out0"], want["out0"]), what


@pytest.mark.parametrize("dtype", [torch.float32, torch.int64, torch.float16, torch.bool])
def test_pw_binary_gpu_large_and_tail(dtype):
    """A size whose byte count is not a multiple of 16 (a partial last store), batched with
    trailing feature dims, for each op the dtype allows."""
    g = torch.Generator().manual_seed(4)
    if dtype == torch.bool:
        a, b = torch.rand(3, 301, 7, 2, generator=g) < 0.5, torch.rand(3, 257, 7, 2, generator=g) < 0.5
        names = ["pwand", "pwor", "pwxor", "pweq", "pwne"]
    else:
        a = torch.randint(-3, 4, (3, 301, 7, 2), generator=g).to(dtype)
        b = torch.randint(-3, 4, (3, 257, 7, 2), generator=g).to(dtype)
        names = ["pweq", "pwne", "pwlt", "pwgt", "pwle", "pwge"]
    for name in names:
        got = getattr(torch.ops.torchpairwise, name)(a.to(DEV), b.to(DEV))
        want = getattr(torch.ops.torchpairwise, name)(a, b)
        assert got.shape == (3, 301, 257, 7, 2)
        assert torch.equal(got.cpu(), want), name


def test_pw_reductions_gpu_equal_cpu():
    """pw*_sum / pw*_mean on the GPU for every case of pw_reduction_cases (every element type,
    the refused ones, bad shapes) against this build's CPU op, which test_pw_binary.py pins to
    the reference's compiled kernels: float32 counts bit for bit, the same errors."""
    from oracle import ref_runner
    from tests._pw_binary_cases import pw_reduction_cases

    ops = torch.ops.torchpairwise
    for case, t in pw_reduction_cases():
        ours = ref_runner.run_op_case(ops, case, t, DEV)
        want = ref_runner.run_op_case(ops, case, t, "cpu")
        what = f"{case['op']} {t['a'].dtype}/{t['b'].dtype} {tuple(t['a'].shape)} {tuple(t['b'].shape)}"
        if "err" in want or "err" in ours:
            assert ours.get("err", "").replace("_cuda", "_cpu") == want.get("err"), what
            continue
        assert ours["out0"].shape == want["out0"].shape, what
        assert_equal(ours["out0"], want["out0"], what)


def test_public_ops_dtypes_gpu_equal_reference(tmp_path):
    """Every public op's forward on GPU tensors of float64, float16, bfloat16, int64, uint8 and
    bool against the reference's compiled CPU library.  Refusals of this build's own ops (the
    reference's kernel dispatch names) must match, device name aside.  Where ATen decides (the
    reference calls at::cdist / matmul, whose CUDA dtype support differs from their CPU support,
    and the reference on a GPU makes the same calls): an ATen CUDA refusal is accepted where the
    CPU computes, a CPU-side ATen refusal is not compared, except that this build serves
    bfloat16 for the cdist metrics where at::cdist refuses it.  Results that both produce agree
    within the dtype's bar (the x2 = None euclidean within the matrix form's self-distance
    floor, which the reference's own GPU route shares)."""
    from oracle import ref_runner
    from tests._public_cases import public_dtype_cases
    from tests.test_reference_pin import _dtype_sweep_compare

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = public_dtype_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    own = ('_forward_cpu"', '_backward_cpu"', '"pairwise_binary')
    failures = []
    for (case, t), r in zip(cs, ref):
        dt = next(iter(t.values())).dtype
        what = f"{case['op']} {dt} {[tuple(v.shape) for v in t.values()]} {case['args'][1:]}"
        ours = ref_runner.run_op_case(ops, case, t, DEV)
        try:
            if "err" in r:
                if any(s in r["err"] for s in own):
                    assert ours.get("err", "").replace('_cuda"', '_cpu"') == r["err"], \
                        f"{what}: {ours.get('err')!r} != {r['err']!r}"
                elif "err" not in ours:
                    assert dt == torch.bfloat16 and '"cdist" not implemented' in r["err"], \
                        f"{what}: computes where the reference raises {r['err']!r}"
                continue
            if "err" in ours:
                assert '_cuda" not implemented for' in ours["err"], f"{what}: raises {ours['err']!r}"
                continue
            floor = 0.0
            if case["op"] == "euclidean_distances" and len(case["args"]) == 1 and dt.is_floating_point:
                a = t["a"].double()
                floor = 4 * float((torch.finfo(dt).eps * 2 * (a * a).sum(-1).max()) ** 0.5)
            _dtype_sweep_compare(ours, r, what, floor, op=case["op"])
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures[:30])


def test_cdist_names_gpu_equal_reference(tmp_path):
    """cdist(metric=...) on GPU tensors for every metric name of the reference's dispatcher
    (with its extra arguments, defaults and a refused argument) against the reference's compiled
    CPU library: values rtol 1e-5 (+ 1e-5 * max), boolean metrics and Hausdorff bit for bit,
    the same TypeError texts."""
    from oracle import ref_runner
    from tests._public_cases import cdist_name_cases
    from tests.test_reference_pin import _assert_results_close

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = cdist_name_cases()
    ref = ref_runner.run_op_reference([(c, t) for c, t, _ in cs], tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t, exact), r in zip(cs, ref):
        what = f"cdist {case['args'][2]['v']} {sorted(case['kwargs'])}"
        ours = ref_runner.run_op_case(ops, case, t, DEV)
        keys = tuple(k for k in r if k != "err") if exact else ()
        if case["args"][2]["v"] == "russellrao":
            keys = ()  # (D - and) / D: the GPU route's division is 1 ulp from the CPU's
        try:
            _assert_results_close(ours, r, 1e-5, what, keys)
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures)


def test_neighbour_masks_gpu_equal_reference(tmp_path):
    """k_neighbors_mask / radius_neighbors_mask on GPU tensors over metrics, extra arguments,
    k up to past the column count, x2 = None and the error paths, against the reference's
    compiled CPU library bit for bit (the cases keep the selection boundaries and radii away
    from near-equal distances, so device rounding cannot move them)."""
    from oracle import ref_runner
    from tests._public_cases import neighbour_cases
    from tests.test_reference_pin import _assert_results_close

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = neighbour_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t), r in zip(cs, ref):
        what = f"{case['op']} {case['args'][2:]} {sorted(case['kwargs'])}"
        try:
            _assert_results_close(ref_runner.run_op_case(ops, case, t, DEV), r, 0.0, what,
                                  tuple(k for k in r if k != "err"))
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,m,d,kind", [(300, 256, 64, "randn"), (257, 272, 128, "ints"), (40, 48, 64, "randn"),
                                        (600, 1008, 256, "randn"), (304, None, 64, "ints"), (130, 144, 64, "ties")])
def test_knn_mask_fused_equals_distances_then_selection(dtype, n, m, d, kind):
    """tpw_knn_mask_euclidean (per-tile candidates + select) against the euclidean distances
    followed by tpw_row_smallest_mask, bit for bit, for every candidate width (count 1 .. 16),
    edge tiles, integer inputs with many equal distances (ties go to the lower column), x2 = x1
    (zero diagonal) and bf16 (distances rounded as stored)."""
    from torchpairwise_amd import _capi as capi

    g = torch.Generator().manual_seed(n + d)
    if kind == "randn":
        x1 = torch.randn(n, d, generator=g)
    elif kind == "ints":
        x1 = torch.randint(-2, 3, (n, d), generator=g).float()
    else:  # a few distinct points repeated: whole rows of equal distances
        x1 = torch.randint(-1, 2, (4, d), generator=g).float()[torch.randint(0, 4, (n,), generator=g)]
    x2 = x1 if m is None else (torch.randn(m, d, generator=g) if kind == "randn"
                               else torch.randint(-2, 3, (m, d), generator=g).float())
    a = x1.to(DEV, dtype)
    b = a if m is None else x2.to(DEV, dtype)
    dist = capi.pairwise_inner(a, b, capi.EPI_EUCLIDEAN)
    for count in (1, 2, 3, 4, 5, 8, 9, 16):
        print(f"{dtype} {n} {m} {d} {kind} count={count}", flush=True)
        got = capi.knn_mask_euclidean(a, b, count)
        want = capi.row_smallest_mask(dist, count)
        assert got.sum(1).eq(count).all(), "count per row"
        assert torch.equal(got, want), f"count={count}: {(got != want).sum().item()} entries differ"


def test_knn_mask_op_routes_fused():
    """k_neighbors_mask on a GPU euclidean case the fused route takes gives the mask of the
    distances-then-selection route, and k + 1 past the fused limit still works."""
    g = torch.Generator().manual_seed(5)
    x1, x2 = torch.randn(300, 64, generator=g).to(DEV), torch.randn(256, 64, generator=g).to(DEV)
    dist = tp.euclidean_distances(x1, x2)
    for k in (0, 1, 3, 15, 16, 40):
        got = tp.k_neighbors_mask(x1, x2, k)
        assert torch.equal(got, torch.ops.torchpairwise._row_smallest_mask(dist, k + 1)), f"k={k}"
