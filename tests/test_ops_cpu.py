"""The drop-in op layer without a GPU: schemas, CPU paths (the reference's routes), errors,
TorchScript, autograd on CPU."""
import warnings
from pathlib import Path

import numpy as np
import pytest
import torch
from scipy.spatial.distance import cdist as scipy_cdist

import torchpairwise_amd as tp
from oracle import cref
from oracle import pairwise as P
from tests._util import assert_close, assert_equal, rand, randn

GOLDEN = Path(__file__).resolve().parent / "golden"

PUBLIC = [
    "euclidean_distances", "haversine_distances", "manhattan_distances", "cosine_distances",
    "linear_kernel", "polynomial_kernel", "sigmoid_kernel", "rbf_kernel", "laplacian_kernel",
    "cosine_similarity", "additive_chi2_kernel", "chi2_kernel", "directed_hausdorff_distances",
    "minkowski_distances", "wminkowski_distances", "sqeuclidean_distances",
    "correlation_distances", "hamming_distances", "jaccard_distances", "kulsinski_distances",
    "kulczynski1_distances", "seuclidean_distances", "cityblock_distances",
    "mahalanobis_distances", "chebyshev_distances", "braycurtis_distances",
    "canberra_distances", "jensenshannon_distances", "yule_distances", "dice_distances",
    "rogerstanimoto_distances", "russellrao_distances", "sokalmichener_distances",
    "sokalsneath_distances", "snr_distances", "l1_distances", "l2_distances", "lp_distances",
    "linf_distances",
]


def test_public_schemas_registered():
    for name in PUBLIC:
        op = getattr(torch.ops.torchpairwise, name)
        assert op is getattr(tp, name)
    s = str(torch.ops.torchpairwise.directed_hausdorff_distances.default._schema)
    assert s == ("torchpairwise::directed_hausdorff_distances(Tensor x1, Tensor? x2=None, *, "
                 "bool shuffle=False, Generator? generator=None) -> (Tensor output, "
                 "Tensor x1_indices, Tensor x2_indices)")
    s = str(torch.ops.torchpairwise.polynomial_kernel.default._schema)
    assert s == ("torchpairwise::polynomial_kernel(Tensor x1, Tensor? x2=None, int degree=3, "
                 "float? gamma=None, float coef0=1.) -> Tensor")


def test_meta_ops():
    assert tp.has_ops()
    assert tp.cuda_version() > 0 and tp.with_cuda()
    assert tp.cuda_arch_list() == ["gfx950"]


def test_c1_manhattan_euclidean_cpu():
    """BASELINE configs[0] (manhattan + euclidean, fp32, [2048, 64] x [1024, 64], N(0, 1),
    seeds 0 / 1) on the reference's CPU route: at::cdist in float32, against float64 cdist and
    scipy for every element."""
    x1, x2 = randn(2048, 64, seed=0), randn(1024, 64, seed=1)
    for name, fn, p, sp in (("euclidean", tp.euclidean_distances, 2.0, "euclidean"),
                            ("manhattan", tp.manhattan_distances, 1.0, "cityblock")):
        out = fn(x1, x2)
        assert out.shape == (2048, 1024) and out.dtype == torch.float32
        assert_equal(out, torch.cdist(x1, x2, p), f"C1 {name} is at::cdist")
        ref = torch.from_numpy(scipy_cdist(x1.double().numpy(), x2.double().numpy(), sp))
        assert_close(out, ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()), what=f"C1 {name} vs scipy")


@pytest.mark.parametrize("p", [0.0, 1.0, 1.5, 2.0, 3.0, float("inf")])
def test_cdist_family_cpu_is_aten(p):
    x1, x2 = randn(40, 9, seed=0, dtype=torch.float64), randn(30, 9, seed=1, dtype=torch.float64)
    got = tp.minkowski_distances(x1, x2, p)
    assert_equal(got, torch.cdist(x1, x2, p), f"minkowski p={p}")
    want = scipy_cdist(x1.numpy(), x2.numpy(), "minkowski", p=p) if p not in (0.0, float("inf")) else None
    if want is not None:
        assert_close(got, torch.from_numpy(want), rtol=1e-12, atol=1e-12, what="vs scipy")


def test_cosine_cpu_matches_sklearn():
    from sklearn.metrics.pairwise import cosine_distances

    x1, x2 = randn(40, 9, seed=0, dtype=torch.float64), randn(30, 9, seed=1, dtype=torch.float64)
    assert_close(tp.cosine_distances(x1, x2), torch.from_numpy(cosine_distances(x1.numpy(), x2.numpy())),
                 rtol=1e-12, atol=1e-12, what="cosine")


def test_boolean_cpu_bit_exact():
    b1, b2 = rand(2, 30, 77, seed=0) < 0.5, rand(2, 20, 77, seed=1) < 0.5
    assert_equal(tp.hamming_distances(b1, b2), torch.from_numpy(P.hamming_distances(b1.numpy(), b2.numpy())))
    assert_equal(tp.jaccard_distances(b1, b2), torch.from_numpy(P.jaccard_distances(b1.numpy(), b2.numpy())))
    i1 = torch.randint(0, 3, (30, 11), generator=torch.Generator().manual_seed(3))
    i2 = torch.randint(0, 3, (20, 11), generator=torch.Generator().manual_seed(4))
    assert_equal(tp.hamming_distances(i1, i2), torch.from_numpy(P.hamming_distances(i1.numpy(), i2.numpy())))


@pytest.mark.parametrize("name", ["dice", "rogerstanimoto", "russellrao", "sokalmichener", "yule"])
def test_boolean_family_cpu_vs_scipy(name):
    b1, b2 = rand(30, 64, seed=0) < 0.5, rand(20, 64, seed=1) < 0.5
    got = getattr(tp, f"{name}_distances")(b1, b2)
    want = scipy_cdist(b1.numpy(), b2.numpy(), name)
    assert_close(got, torch.from_numpy(want), rtol=1e-6, atol=1e-7, what=name)


def test_boolean_coercion_warns(capfd):
    # TORCH_WARN from a dispatcher op reaches the c10 log (stderr), as in the reference
    x = torch.randint(0, 2, (5, 8))
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        tp.jaccard_distances(x, x)
    text = capfd.readouterr().err + " ".join(str(r.message) for r in rec)
    assert "converted to Bool" in text


def test_hausdorff_cpu_bit_exact_and_gradcheck():
    c1, c2 = rand(2, 60, 3, seed=0), rand(3, 50, 3, seed=1) + 0.05
    got = tp.directed_hausdorff_distances(c1, c2)
    want = cref.directed_hausdorff(c1.numpy(), c2.numpy())
    for g, w in zip(got, want):
        assert_equal(g, torch.from_numpy(w))
    a = c1.double().requires_grad_()
    b = c2.double().requires_grad_()
    assert torch.autograd.gradcheck(lambda u, v: tp.directed_hausdorff_distances(u, v)[0], (a, b))
    gen = torch.Generator().manual_seed(7)
    assert torch.autograd.gradcheck(
        lambda u: tp.directed_hausdorff_distances(u, b, shuffle=True, generator=gen)[0], (a,))


def test_prf_div_cpu():
    x = torch.tensor([1.0, 2.0, 3.0, 4.0])
    y = torch.tensor([2.0, 0.0, 4.0, 0.0])
    assert_equal(tp.prf_div(x, y), torch.tensor([0.5, 0.0, 0.75, 0.0]))
    assert_equal(tp.prf_div(x, y, "identity"), torch.tensor([0.5, 2.0, 0.75, 4.0]))
    with pytest.raises(RuntimeError, match="mode must be either zero or identity"):
        tp.prf_div(x, y, "bad")
    xd, yd = x.double().requires_grad_(), (y.double() + 0.5).requires_grad_()
    assert torch.autograd.gradcheck(lambda a, b: tp.prf_div(a, b, "identity"), (xd, yd))


def test_input_errors():
    with pytest.raises(RuntimeError, match="x1 must be 2D tensor"):
        tp.euclidean_distances(torch.randn(3))
    with pytest.raises(RuntimeError, match="same number of features"):
        tp.euclidean_distances(torch.randn(3, 4), torch.randn(3, 5))
    with pytest.raises(RuntimeError, match="feature dimension of x1 and x2 must be 2"):
        tp.haversine_distances(torch.randn(3, 3))


def _scripted(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return torch.ops.torchpairwise.euclidean_distances(a, b) + torch.ops.torchpairwise.hamming_distances(a > 0, b > 0)


def test_torchscript_binds_schemas():
    f = torch.jit.script(_scripted)
    a, b = randn(10, 4, seed=0), randn(8, 4, seed=1)
    assert_close(f(a, b), _scripted(a, b), rtol=0, atol=0, what="scripted")


# ---------------------------------------------------------------------- cdist / neighbours
CDIST_METRICS = {
    "euclidean": lambda a, b: tp.euclidean_distances(a, b),
    "manhattan": lambda a, b: tp.manhattan_distances(a, b),
    "cityblock": lambda a, b: tp.manhattan_distances(a, b),
    "l1": lambda a, b: tp.l1_distances(a, b),
    "l2": lambda a, b: tp.l2_distances(a, b),
    "linf": lambda a, b: tp.chebyshev_distances(a, b),
    "chebyshev": lambda a, b: tp.chebyshev_distances(a, b),
    "cosine": lambda a, b: tp.cosine_distances(a, b),
    "sqeuclidean": lambda a, b: tp.sqeuclidean_distances(a, b),
    "correlation": lambda a, b: tp.correlation_distances(a, b),
    "minkowski": lambda a, b: tp.minkowski_distances(a, b, 2.0),
    "lp": lambda a, b: tp.lp_distances(a, b, 2.0),
    "braycurtis": lambda a, b: tp.braycurtis_distances(a, b),
    "canberra": lambda a, b: tp.canberra_distances(a, b),
    "snr": lambda a, b: tp.snr_distances(a, b),
    "jensenshannon": lambda a, b: tp.jensenshannon_distances(a.abs(), b.abs()),
}


@pytest.mark.parametrize("metric", sorted(CDIST_METRICS))
def test_cdist_dispatches_to_the_metric(metric):
    a, b = randn(9, 6, seed=0), randn(11, 6, seed=1)
    if metric == "jensenshannon":
        a, b = a.abs(), b.abs()
    assert_equal(tp.cdist(a, b, metric), CDIST_METRICS[metric](a, b), metric)


def test_cdist_extra_arguments():
    a, b = randn(9, 6, seed=0), randn(11, 6, seed=1)
    assert_equal(tp.cdist(a, b), tp.minkowski_distances(a, b))  # default metric, p=2
    assert_equal(tp.cdist(a, b, "minkowski", p=3.0), tp.minkowski_distances(a, b, 3.0))
    assert_equal(tp.cdist(a, b, "lp", p=1.0), tp.manhattan_distances(a, b))
    bb, cc = a > 0, b > 0
    assert_equal(tp.cdist(bb, cc, "hamming"), tp.hamming_distances(bb, cc))
    assert_equal(tp.cdist(bb, cc, "jaccard"), tp.jaccard_distances(bb, cc))
    c1, c2 = rand(2, 20, 3, seed=2), rand(3, 25, 3, seed=3)
    g1, g2 = torch.Generator().manual_seed(5), torch.Generator().manual_seed(5)
    assert_equal(tp.cdist(c1, c2, "directed_hausdorff", shuffle=True, generator=g1),
                 tp.directed_hausdorff_distances(c1, c2, shuffle=True, generator=g2)[0])


def test_cdist_errors_match_the_reference():
    a, b = randn(4, 3, seed=0), randn(5, 3, seed=1)
    with pytest.raises(TypeError) as e:
        tp.cdist(a, b, "euclidean", p=3.0, w=a)
    assert str(e.value).startswith(
        "torchpairwise::euclidean_distances was called with incompatible arguments w, p.\n"
        "The following signature is supported:\n"
        "    euclidean_distances(Tensor x1, Tensor? x2=None) -> Tensor\n")
    with pytest.raises(TypeError, match="incompatible arguments generator"):
        tp.cdist(a, b, "minkowski", generator=torch.Generator())
    with pytest.raises(RuntimeError, match=r"Got unkown distance metric: foo\. Supported metrics "
                                           r"are \[braycurtis, canberra, .*, wminkowski, yule\]"):
        tp.cdist(a, b, "foo")
    with pytest.raises(NotImplementedError, match="pdist is yet to be implemented"):
        tp.pdist(a)
    with pytest.raises(RuntimeError, match="feature dimension of x1 and x2 must be 2"):
        tp.cdist(a, b, "haversine")  # dispatched to haversine_distances
    sch = str(torch.ops.torchpairwise.k_neighbors_mask.default._schema)
    assert sch == ("torchpairwise::k_neighbors_mask(Tensor x1, Tensor? x2=None, int k=1, "
                   "str metric=\"euclidean\", *, Tensor? w=None, Tensor? V=None, Tensor? VI=None, "
                   "float? p=None, float? base=None, bool? shuffle=None, Generator? generator=None) "
                   "-> Tensor")


def test_neighbors_cpu_match_sklearn_golden():
    g = dict(np.load(GOLDEN / "neighbors.npz"))
    x1, x2 = torch.from_numpy(g["x1"]), torch.from_numpy(g["x2"])
    for k in (0, 1, 4):
        assert np.array_equal(tp.k_neighbors_mask(x1, x2, k).numpy(), g[f"knn_k{k}"]), k
    assert np.array_equal(tp.radius_neighbors_mask(x1, x2, float(g["radius_eps"])).numpy(),
                          g["radius"])
    # x2 = None: every point is its own nearest neighbour
    m = tp.k_neighbors_mask(x1, None, 0)
    assert torch.equal(m, torch.eye(12, dtype=torch.bool))


def test_neighbors_cpu_edge_cases():
    a, b = randn(6, 3, seed=0), randn(4, 3, seed=1)
    with pytest.raises(RuntimeError, match="k must be non-negative"):
        tp.k_neighbors_mask(a, b, -1)
    with pytest.raises(RuntimeError, match="epsilon must be non-negative"):
        tp.radius_neighbors_mask(a, b, -0.5)
    # k + 1 > M: the reference's index_put_ indices do not broadcast, and it raises
    with pytest.raises(IndexError, match="shape mismatch"):
        tp.k_neighbors_mask(a, b, 4)
    m = tp.k_neighbors_mask(a, b, 3, "manhattan")
    assert torch.equal(m, torch.ones(6, 4, dtype=torch.bool))


def test_row_smallest_mask_cpu_hand_built_rows():
    g = dict(np.load(GOLDEN / "neighbors.npz"))
    for i in range(int(g["n_rows"])):
        got = torch.ops.torchpairwise._row_smallest_mask(torch.from_numpy(g[f"row{i}_dist"]),
                                                         int(g[f"row{i}_count"]))
        assert np.array_equal(got.numpy(), g[f"row{i}_mask"]), i


# ---------------------------------------------------------------------- VALU family (CPU)
def test_family_cpu_match_scipy_golden():
    g = dict(np.load(GOLDEN / "family.npz"))
    x1, x2 = torch.from_numpy(g["x1"]), torch.from_numpy(g["x2"])
    w, V = torch.from_numpy(g["w"]), torch.from_numpy(g["V"])
    tol = dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tp.sqeuclidean_distances(x1, x2).numpy(), g["sqeuclidean"], **tol)
    np.testing.assert_allclose(tp.canberra_distances(x1, x2).numpy(), g["canberra"], **tol)
    np.testing.assert_allclose(tp.braycurtis_distances(x1, x2).numpy(), g["braycurtis"], **tol)
    for p in (1, 2, 3):
        np.testing.assert_allclose(tp.wminkowski_distances(x1, x2, float(p), w).numpy(),
                                   g[f"wminkowski_p{p}"], **tol)
    np.testing.assert_allclose(tp.seuclidean_distances(x1, x2, V).numpy(), g["seuclidean"], **tol)
    np.testing.assert_allclose(tp.seuclidean_distances(x1).numpy(), g["seuclidean_self"], **tol)
    with pytest.raises(RuntimeError, match="V is required for seuclidean"):
        tp.seuclidean_distances(x1, x2)


@pytest.mark.parametrize("p", [0.0, 1.0, 1.5, 2.0, 3.0, float("inf"), -float("inf")])
def test_family_cpu_internal_ops_and_grads(p):
    # batched _wminkowski: the reference checks x1.size(1) (rows) against w.size(1)
    # (cpu/wminkowski_kernel.cpp:84-86), so rows == features here
    x1 = torch.randn(2, 5, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    x2 = torch.randn(2, 6, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    w = torch.rand(2, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(2)) + 0.2
    ops = torch.ops.torchpairwise
    assert_close(ops._ppminkowski(x1, x2, p), P.ppminkowski(x1, x2, p), rtol=1e-12, atol=1e-12, what="pp")
    if p != -float("inf"):
        assert_close(ops._wminkowski(x1, x2, w, p), P.wminkowski(x1, x2, w, p), rtol=1e-12, atol=1e-12,
                     what="w")
    if p in (0.0,):  # p = 0: zero gradients, as the reference's backward returns
        g = torch.ones(2, 5, 6, dtype=torch.float64)
        assert all((t == 0).all() for t in ops.__ppminkowski_backward(g, x1, x2, p))
        return
    a, b, c = (t.clone().requires_grad_() for t in (x1, x2, w))
    assert torch.autograd.gradcheck(lambda u, v: ops._ppminkowski(u, v, p), (a, b))
    if p != -float("inf"):
        assert torch.autograd.gradcheck(lambda u, v, q: ops._wminkowski(u, v, q, p), (a, b, c))


def test_canberra_braycurtis_cpu_grads_and_dtypes():
    gen = torch.Generator().manual_seed(11)
    x1 = torch.randn(6, 4, dtype=torch.float64, generator=gen).requires_grad_()
    x2 = torch.randn(5, 4, dtype=torch.float64, generator=gen).requires_grad_()
    assert torch.autograd.gradcheck(tp.canberra_distances, (x1, x2))
    assert torch.autograd.gradcheck(tp.braycurtis_distances, (x1, x2))
    for fn in (tp.canberra_distances, tp.braycurtis_distances, tp.sqeuclidean_distances):
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            if dt == torch.bfloat16 and fn is not tp.sqeuclidean_distances:
                # the reference's canberra / braycurtis kernels dispatch floating types and half
                with pytest.raises(NotImplementedError, match="_forward_cpu\" not implemented for 'BFloat16'"):
                    fn(x1.detach().to(dt), x2.detach().to(dt))
                continue
            got = fn(x1.detach().to(dt), x2.detach().to(dt))
            assert got.dtype == dt
            ref = fn(x1.detach().to(dt).double(), x2.detach().to(dt).double())
            assert_close(got.double(), ref, rtol=1e-5 if dt == torch.float32 else 1e-2, atol=1e-6,
                         what=f"{fn} {dt}")
    with pytest.raises(RuntimeError, match="batch_size of x1 and x2 do not match"):
        torch.ops.torchpairwise._canberra(torch.randn(2, 3, 4), torch.randn(3, 3, 4))
    with pytest.raises(RuntimeError, match="feature dimension of x1, x2, and w do not match"):
        torch.ops.torchpairwise._wminkowski(torch.randn(2, 3, 4), torch.randn(2, 5, 4), torch.rand(2, 4), 2.0)


# ---------------------------------------------------------------------- chi2, JS, haversine, snr, mahalanobis
def test_special_cpu_match_sklearn_scipy_golden():
    g = dict(np.load(GOLDEN / "special.npz"))
    t = {k: torch.from_numpy(v) for k, v in g.items()}
    tol = dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tp.additive_chi2_kernel(t["p1"], t["p2"]).numpy(), g["additive_chi2"], **tol)
    np.testing.assert_allclose(tp.chi2_kernel(t["p1"], t["p2"], 0.7).numpy(), g["chi2_g07"], **tol)
    np.testing.assert_allclose(tp.jensenshannon_distances(t["p1"], t["p2"]).numpy(), g["js"], **tol)
    np.testing.assert_allclose(tp.jensenshannon_distances(t["p1"], t["p2"], base=2.0).numpy(),
                               g["js_base2"], **tol)
    np.testing.assert_allclose(tp.haversine_distances(t["g1"], t["g2"]).numpy(), g["haversine"], **tol)
    np.testing.assert_allclose(tp.mahalanobis_distances(t["x1"], t["x2"], t["VI"]).numpy(),
                               g["mahalanobis"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(tp.cdist(t["x1"], t["x2"], "mahalanobis", VI=t["VI"]).numpy(),
                               g["mahalanobis"], rtol=1e-10, atol=1e-10)
    with pytest.raises(RuntimeError, match="All elements of x1 and x2 must be positive"):
        tp.additive_chi2_kernel(-t["p1"], t["p2"])
    with pytest.raises(RuntimeError, match="VI is required for manhalanobis when x2 is passed"):
        tp.cdist(t["x1"], t["x2"], "mahalanobis")  # the reference's text, typo included


def test_special_cpu_internal_ops_vs_oracle_and_grads():
    ops = torch.ops.torchpairwise
    gen = torch.Generator().manual_seed(3)
    p1 = torch.rand(2, 5, 4, dtype=torch.float64, generator=gen) + 0.05
    p2 = torch.rand(2, 6, 4, dtype=torch.float64, generator=gen) + 0.05
    x1 = torch.randn(2, 5, 4, dtype=torch.float64, generator=gen)
    x2 = torch.randn(2, 6, 4, dtype=torch.float64, generator=gen)
    a = torch.randn(2, 4, 4, dtype=torch.float64, generator=gen)
    VI = a @ a.transpose(1, 2) + torch.eye(4, dtype=torch.float64)
    tol = dict(rtol=1e-12, atol=1e-12)
    assert_close(ops._additive_chi2_kernel(p1, p2), P.additive_chi2(p1, p2), what="chi2", **tol)
    for base in (None, 2.0, 3.0):
        assert_close(ops._sqjensenshannon(p1, p2, base), P.sqjensenshannon(p1, p2, base), what="js", **tol)
    assert_close(ops._haversine(x1[..., :2], x2[..., :2]), P.haversine(x1[..., :2], x2[..., :2]),
                 what="haversine", **tol)
    assert_close(ops._snr(x1, x2), P.snr(x1, x2), what="snr", **tol)
    assert_close(ops._sqmahalanobis(x1, x2, VI), P.sqmahalanobis(x1, x2, VI), what="maha", **tol)
    req = lambda *ts: tuple(u.clone().requires_grad_() for u in ts)
    assert torch.autograd.gradcheck(ops._additive_chi2_kernel, req(p1, p2))
    for base in (None, 3.0):
        assert torch.autograd.gradcheck(lambda u, v: ops._sqjensenshannon(u, v, base), req(p1, p2))
    assert torch.autograd.gradcheck(ops._haversine, req(x1[..., :2], x2[..., :2]))
    assert torch.autograd.gradcheck(ops._snr, req(x1, x2))
    assert torch.autograd.gradcheck(ops._sqmahalanobis, req(x1, x2, VI))
    assert torch.autograd.gradcheck(tp.jensenshannon_distances, req(p1[0], p2[0]))


def test_special_cpu_edge_cases():
    # chi2: a coordinate with x1 + x2 == 0 adds nothing (cpu/additive_chi2_kernel.cpp:22-27)
    a = torch.tensor([[0.0, 1.0]], dtype=torch.float64)
    b = torch.tensor([[0.0, 3.0]], dtype=torch.float64)
    assert float(torch.ops.torchpairwise._additive_chi2_kernel(a, b)) == -1.0
    # JS of identical distributions is 0; of disjoint supports, (ln 2 + ln 2) / 2 (squared, base e)
    u = torch.tensor([[0.5, 0.5, 0.0, 0.0]], dtype=torch.float64)
    v = torch.tensor([[0.0, 0.0, 0.5, 0.5]], dtype=torch.float64)
    assert float(torch.ops.torchpairwise._sqjensenshannon(u, u, None)) == 0.0
    assert abs(float(torch.ops.torchpairwise._sqjensenshannon(u, v, None)) - np.log(2)) < 1e-15
    # haversine: antipodes are pi apart, a point is 0 from itself
    pts = torch.tensor([[0.3, -1.0], [-0.3, -1.0 + np.pi]], dtype=torch.float64)
    d = tp.haversine_distances(pts)
    assert abs(float(d[0, 1]) - np.pi) < 1e-7 and float(d[0, 0]) == 0.0
    # mahalanobis with VI = I is euclidean
    x = torch.randn(5, 3, dtype=torch.float64)
    assert_close(tp.mahalanobis_distances(x, x, torch.eye(3, dtype=torch.float64)),
                 torch.cdist(x, x), rtol=1e-12, atol=1e-7, what="maha I")
    # snr is V1 / DV, so it is scale-free in x2 - x1 per row
    y = torch.randn(4, 3, dtype=torch.float64)
    assert_close(tp.snr_distances(x, y), torch.ops.torchpairwise._snr(x, y).reciprocal(),
                 rtol=0, atol=0, what="snr")
    with pytest.raises(RuntimeError, match="feature dimension"):
        torch.ops.torchpairwise._sqmahalanobis(x, x, torch.eye(4, dtype=torch.float64))
