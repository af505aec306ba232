"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against the committed golden fixtures (tests/golden, made by
scipy / sklearn / hand-derived cases, see make_golden.py), against independent libraries,
against closed forms and brute force, and the C early-break restatement against the numpy
brute force.  The mutation tests at the end plant plausible mistakes in the oracle (on the
CPU) and check that these pins catch them.
"""
from pathlib import Path

import numpy as np
import pytest
import torch
from scipy.spatial.distance import cdist, directed_hausdorff

from oracle import cref
from oracle import pairwise as P

GOLDEN = Path(__file__).resolve().parent / "golden"


def npz(name):
    return dict(np.load(GOLDEN / name, allow_pickle=False))


# ---------------------------------------------------------------------- boolean family
def test_bool_counts_match_golden_loop_counts():
    g = npz("boolean.npz")
    for op in ("and", "or", "xor", "eq", "ne"):
        assert np.array_equal(P.bool_counts(g["x1"], g["x2"], op), g[f"count_{op}"]), op


def test_hamming_jaccard_match_golden_bitwise():
    g = npz("boolean.npz")
    h = P.hamming_distances(g["x1"], g["x2"])
    j = P.jaccard_distances(g["x1"], g["x2"])
    assert h.dtype == np.float32 and j.dtype == np.float32
    assert np.array_equal(h.view(np.int32), g["hamming_f32"].view(np.int32))
    assert np.array_equal(j.view(np.int32), g["jaccard_f32"].view(np.int32))
    assert j[0, 0] == 0.0  # both rows all-zero: or == 0 -> 0
    # d = 64: the quotients are exact dyadics k/64
    h64 = P.hamming_distances(g["y1"], g["y2"])
    assert np.array_equal(h64, g["hamming_d64"])
    assert np.array_equal(h64 * 64, np.round(h64 * 64))


def test_pw_mean_is_sum_over_d():
    g = npz("boolean.npz")
    s = P.pw_reduce_bool(g["x1"], g["x2"], "eq", "sum")
    m = P.pw_reduce_bool(g["x1"], g["x2"], "eq", "mean")
    assert np.array_equal(m, (s / np.float32(45)).astype(np.float32))
    assert np.array_equal(s, g["count_eq"].astype(np.float32))


def test_float_accumulator_saturates_like_the_reference():
    # a float32 accumulator of 1.0f stops at 2^24 (2^24 + 1 rounds back to 2^24)
    acc = np.float32(2 ** 24)
    assert np.float32(acc + np.float32(1)) == acc
    assert P.float_accumulated(np.array([2 ** 24 + 5]))[0] == np.float32(2 ** 24)


def test_boolean_oracle_vs_c_restatement_random():
    rng = np.random.default_rng(3)
    for d in (1, 31, 64, 100):
        a = rng.random((2, 17, d)) < 0.4
        b = rng.random((2, 13, d)) < 0.6
        for op in ("and", "or", "xor", "eq", "ne"):
            for mean in (False, True):
                want = cref.bool_reduce(a, b, op, mean)
                got = P.pw_reduce_bool(a, b, op, "mean" if mean else "sum")
                assert np.array_equal(got.view(np.int32), want.view(np.int32)), (d, op, mean)
        assert np.array_equal(P.jaccard_distances(a, b).view(np.int32), cref.jaccard(a, b).view(np.int32))


def test_hamming_non_bool_matches_scipy():
    rng = np.random.default_rng(4)
    a = rng.integers(0, 3, (6, 19))
    b = rng.integers(0, 3, (5, 19))
    assert np.array_equal(P.hamming_distances(a, b), cdist(a, b, "hamming").astype(np.float32))


# ---------------------------------------------------------------------- cdist / cosine
@pytest.mark.parametrize("p", [1, 2, 3, "inf"])
def test_cdist_reference_matches_scipy_golden(p):
    g = npz("minkowski_cosine.npz")
    x1, x2 = torch.from_numpy(g["x1"]), torch.from_numpy(g["x2"])
    got = P.cdist_reference(x1, x2, float("inf") if p == "inf" else float(p))
    np.testing.assert_allclose(got.numpy(), g[f"p{p}"], rtol=1e-12, atol=1e-12)


def test_cosine_reference_matches_sklearn_golden():
    g = npz("minkowski_cosine.npz")
    got = P.cosine_distances(torch.from_numpy(g["x1"]), torch.from_numpy(g["x2"]))
    np.testing.assert_allclose(got.numpy(), g["cosine"], rtol=1e-12, atol=1e-12)


def test_cosine_and_prf_div_gradients():
    x1 = torch.randn(6, 5, dtype=torch.float64, requires_grad=True)
    x2 = torch.randn(4, 5, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(P.cosine_distances, (x1, x2))
    assert torch.autograd.gradcheck(P.cosine_similarity, (x1, x2))
    # prf_div identity branch where the denominator is 0: d/dx = 1, d/dy = 0
    x = torch.tensor([3.0], dtype=torch.float64, requires_grad=True)
    y = torch.tensor([0.0], dtype=torch.float64, requires_grad=True)
    P.prf_div_identity(x, y).backward()
    assert x.grad.item() == 1.0 and y.grad.item() == 0.0


@pytest.mark.parametrize("p", [1.0, 1.5, 2.0, 3.0, float("inf")])
def test_cdist_gradients_are_torchs(p):
    x1 = torch.rand(5, 4, dtype=torch.float64, requires_grad=True)
    x2 = torch.rand(6, 4, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: P.cdist_reference(a, b, p), (x1, x2))


# ---------------------------------------------------------------------- Hausdorff
def test_hausdorff_value_matches_scipy_golden():
    g = npz("hausdorff.npz")
    out, i1, i2 = P.directed_hausdorff(g["a"], g["b"])
    np.testing.assert_allclose(out, g["value"], rtol=1e-6)
    # the reported indices realise the value
    for i in range(3):
        for j in range(2):
            d = g["a"][i][i1[i, j]] - g["b"][j][i2[i, j]]
            assert abs(np.sqrt((d.astype(np.float64) ** 2).sum()) - g["value"][i, j]) < 1e-6


@pytest.mark.parametrize("case", [1, 2, 3])
def test_hausdorff_hand_built_ties(case):
    g = npz("hausdorff.npz")
    x1, x2 = g[f"t{case}_x1"][None], g[f"t{case}_x2"][None]
    for impl in (P.directed_hausdorff, cref.directed_hausdorff):
        out, i1, i2 = impl(x1, x2)
        assert out[0, 0] == g[f"t{case}_value"], impl
        assert i1[0, 0] == g[f"t{case}_idx1"] and i2[0, 0] == g[f"t{case}_idx2"], impl


def test_hausdorff_brute_force_equals_early_break_c():
    rng = np.random.default_rng(5)
    for shape1, shape2 in (((2, 3, 150, 3), (2, 2, 170, 3)), ((3, 80, 5), (2, 90, 5)),
                           ((2, 60, 3), (4, 40, 3))):
        a = rng.random(shape1).astype(np.float32)
        b = rng.random(shape2).astype(np.float32) + np.float32(0.05)
        w = P.directed_hausdorff(a, b)
        c = cref.directed_hausdorff(a, b, threads=4)
        for x, y in zip(w, c):
            assert np.array_equal(np.asarray(x).view(np.int32) if x.dtype == np.float32 else x,
                                  np.asarray(y).view(np.int32) if y.dtype == np.float32 else y)


def test_hausdorff_shuffled_orders():
    rng = np.random.default_rng(6)
    a = rng.integers(0, 3, (2, 2, 60, 3)).astype(np.float32)  # many ties
    b = rng.integers(0, 3, (2, 3, 50, 3)).astype(np.float32)
    p1, p2 = P.hausdorff_permutations(2, 60, 50, torch.Generator().manual_seed(1))
    w = P.directed_hausdorff(a, b, p1.numpy(), p2.numpy())
    c = cref.directed_hausdorff(a, b, p1.numpy(), p2.numpy())
    for x, y in zip(w, c):
        assert np.array_equal(x, y)
    # permuted iteration changes which tied index is reported but never the value
    plain = P.directed_hausdorff(a, b)
    assert np.array_equal(w[0], plain[0])


def test_hausdorff_backward_closed_form_gradcheck():
    # the scatter formula is the derivative of sqrt(d(m*, n*)) for fixed argmax/argmin
    rng = np.random.default_rng(7)
    a = rng.random((2, 30, 3)).astype(np.float32)
    b = rng.random((2, 20, 3)).astype(np.float32) + np.float32(0.05)
    out, i1, i2 = P.directed_hausdorff(a, b)
    g = rng.standard_normal(out.shape).astype(np.float32)
    gx1, gx2 = P.directed_hausdorff_backward(g, a, b, out, i1, i2)
    ta = torch.from_numpy(a).double().requires_grad_()
    tb = torch.from_numpy(b).double().requires_grad_()
    val = torch.stack([torch.stack([
        (ta[i, i1[i, j]] - tb[j, i2[i, j]]).pow(2).sum().sqrt() for j in range(2)]) for i in range(2)])
    val.backward(torch.from_numpy(g).double())
    np.testing.assert_allclose(gx1, ta.grad.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gx2, tb.grad.numpy(), rtol=1e-5, atol=1e-6)


def test_hausdorff_sqdist_is_not_fused():
    # one rounding per operation: differs from a fused multiply-add accumulation somewhere
    rng = np.random.default_rng(8)
    a = rng.random((200, 3)).astype(np.float32)
    b = rng.random((300, 3)).astype(np.float32)
    d = P.hausdorff_sqdist_matrix(a, b)
    diff = (a[:, None, :].astype(np.float64) - b[None, :, :])
    exact = (diff.astype(np.float32).astype(np.float64) ** 2).sum(-1)
    assert np.abs(d - exact).max() < 1e-6
    manual = np.float32(0)
    for k in range(3):
        t = np.float32(a[7, k] - b[11, k])
        manual = np.float32(manual + np.float32(t * t))
    assert d[7, 11] == manual


# ---------------------------------------------------------------------- mutation tests
def test_pins_catch_first_m_instead_of_last(monkeypatch):
    g = npz("hausdorff.npz")
    real = P.directed_hausdorff

    def wrong(x1, x2, perm1=None, perm2=None):  # picks the first m reaching the maximum
        a, b = np.asarray(x1, np.float32)[0], np.asarray(x2, np.float32)[0]
        dm = P.hausdorff_sqdist_matrix(a, b)
        mins = dm.min(1)
        m = int(np.nonzero(mins == mins.max())[0][0])
        n = int(np.nonzero(dm[m] == mins[m])[0][0])
        return (np.array([[np.sqrt(mins.max(), dtype=np.float32)]]), np.array([[m]]), np.array([[n]]))

    monkeypatch.setattr(P, "directed_hausdorff", wrong)
    with pytest.raises(AssertionError):
        test_hausdorff_hand_built_ties(1)
    monkeypatch.setattr(P, "directed_hausdorff", real)


def test_pins_catch_a_dropped_float_rounding(monkeypatch):
    # computing the hamming quotient in float64 and not rounding to float32 is caught
    g = npz("boolean.npz")
    h = P.bool_counts(g["x1"], g["x2"], "ne") / 45.0
    assert not np.array_equal(h, g["hamming_f32"].astype(np.float64))


def test_pins_catch_xor_for_or(monkeypatch):
    g = npz("boolean.npz")
    wrong = P.bool_counts(g["x1"], g["x2"], "xor")
    assert not np.array_equal(wrong, g["count_or"])


# ---------------------------------------------------------------------- neighbour masks
def test_k_smallest_mask_matches_sklearn_golden():
    g = npz("neighbors.npz")
    dist = cdist(g["x1"], g["x2"])  # float64, tie-free random points
    for k in (0, 1, 4):
        assert np.array_equal(P.k_smallest_mask(dist, k + 1), g[f"knn_k{k}"]), k
    assert np.array_equal(P.radius_mask(dist, g["radius_eps"]), g["radius"])


def test_k_smallest_mask_hand_built_rows():
    g = npz("neighbors.npz")
    for i in range(int(g["n_rows"])):
        got = P.k_smallest_mask(g[f"row{i}_dist"], int(g[f"row{i}_count"]))
        assert np.array_equal(got, g[f"row{i}_mask"]), i


def test_k_smallest_mask_properties_with_ties():
    rng = np.random.default_rng(9)
    d = rng.integers(0, 6, (40, 57)).astype(np.float32)  # heavy ties
    d[3, ::5] = np.nan
    for count in (0, 1, 2, 7, 30, 57, 80):
        m = P.k_smallest_mask(d, count)
        assert (m.sum(1) == min(count, 57)).all()
        for r in range(40):
            sel, rest = d[r][m[r]], d[r][~m[r]]
            key = np.where(np.isnan(d[r]), np.inf, d[r])
            if sel.size and rest.size:
                # every selected entry precedes every unselected one (NaN last) ...
                ks, kr = key[m[r]], key[~m[r]]
                assert ks.max() <= kr.min()
                assert not (np.isnan(sel).any() and not np.isnan(rest).all())
                # ... and on the tied boundary value the lower columns are taken
                b = ks.max()
                tied = np.nonzero(key == b)[0]
                taken = tied[m[r][tied]]
                assert np.array_equal(taken, tied[: taken.size])


def test_pins_catch_highest_column_on_ties():
    g = npz("neighbors.npz")

    def wrong(dist, count):  # stable sort of the reversed row: ties go to the higher column
        d = np.asarray(dist)[:, ::-1]
        return P.k_smallest_mask(d, count)[:, ::-1]

    bad = sum(not np.array_equal(wrong(g[f"row{i}_dist"], int(g[f"row{i}_count"])), g[f"row{i}_mask"])
              for i in range(int(g["n_rows"])))
    assert bad >= 3


# ---------------------------------------------------------------------- VALU family
def test_family_oracle_matches_scipy_golden():
    g = npz("family.npz")
    x1, x2 = torch.from_numpy(g["x1"]), torch.from_numpy(g["x2"])
    w, V = torch.from_numpy(g["w"]), torch.from_numpy(g["V"])
    tol = dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(P.ppminkowski(x1, x2, 2.0).numpy(), g["sqeuclidean"], **tol)
    np.testing.assert_allclose(P.canberra(x1, x2).numpy(), g["canberra"], **tol)
    np.testing.assert_allclose(P.braycurtis(x1, x2).numpy(), g["braycurtis"], **tol)
    for p in (1, 2, 3):
        np.testing.assert_allclose(P.wminkowski(x1, x2, w, float(p)).numpy(), g[f"wminkowski_p{p}"], **tol)
    np.testing.assert_allclose(P.wminkowski(x1, x2, 1.0 / V, 2.0).numpy(), g["seuclidean"], **tol)
    # closed forms: p = 0 fills d; pp with p = 2 is the squared euclidean distance
    assert (P.ppminkowski(x1, x2, 0.0) == 6.0).all()
    np.testing.assert_allclose(P.ppminkowski(x1, x2, 2.0).numpy(), cdist(g["x1"], g["x2"]) ** 2, rtol=1e-12)


def test_family_oracle_gradients():
    x1 = torch.randn(5, 4, dtype=torch.float64, requires_grad=True)
    x2 = torch.randn(6, 4, dtype=torch.float64, requires_grad=True)
    w = (torch.rand(4, dtype=torch.float64) + 0.2).requires_grad_()
    for p in (1.0, 1.5, 2.0, 3.0, float("inf")):
        assert torch.autograd.gradcheck(lambda a, b: P.ppminkowski(a, b, p), (x1, x2))
        assert torch.autograd.gradcheck(lambda a, b, c: P.wminkowski(a, b, c, p), (x1, x2, w))
    assert torch.autograd.gradcheck(P.canberra, (x1, x2))
    assert torch.autograd.gradcheck(P.braycurtis, (x1, x2))


def test_pins_catch_a_missing_root_or_weight():
    g = npz("family.npz")
    x1, x2, w = (torch.from_numpy(g[k]) for k in ("x1", "x2", "w"))
    assert not np.allclose(P.ppminkowski(x1, x2, 3.0).numpy(), g["wminkowski_p3"])  # root dropped
    assert not np.allclose(P.wminkowski(x1, x2, torch.ones_like(w), 3.0).numpy(), g["wminkowski_p3"])


# ---------------------------------------------------------------------- chi2, JS, haversine, snr, mahalanobis
def test_special_oracle_matches_sklearn_scipy_golden():
    g = npz("special.npz")
    t = {k: torch.from_numpy(v) for k, v in g.items()}
    tol = dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(P.additive_chi2(t["p1"], t["p2"]).numpy(), g["additive_chi2"], **tol)
    np.testing.assert_allclose(torch.exp(0.7 * P.additive_chi2(t["p1"], t["p2"])).numpy(), g["chi2_g07"], **tol)
    # scipy normalises each row to a distribution first
    q1 = t["p1"] / t["p1"].sum(-1, keepdim=True)
    q2 = t["p2"] / t["p2"].sum(-1, keepdim=True)
    np.testing.assert_allclose(P.sqjensenshannon(q1, q2).sqrt().numpy(), g["js"], **tol)
    np.testing.assert_allclose(P.sqjensenshannon(q1, q2, 2.0).sqrt().numpy(), g["js_base2"], **tol)
    np.testing.assert_allclose(P.haversine(t["g1"], t["g2"]).numpy(), g["haversine"], **tol)
    np.testing.assert_allclose(P.sqmahalanobis(t["x1"], t["x2"], t["VI"]).sqrt().numpy(), g["mahalanobis"],
                               rtol=1e-10, atol=1e-10)


def test_snr_oracle_is_the_variance_ratio():
    # snr distance = var(x2 - x1) / var(x1) (population variances; the count cancels)
    rng = np.random.default_rng(4)
    a, b = rng.standard_normal((5, 7)), rng.standard_normal((6, 7))
    want = np.array([[np.var(y - x) / np.var(x) for y in b] for x in a])
    np.testing.assert_allclose(P.snr(torch.from_numpy(a), torch.from_numpy(b)).reciprocal().numpy(), want,
                               rtol=1e-12)


def test_special_oracle_closed_forms_and_gradients():
    # VI = I reduces mahalanobis to squared euclidean; antipodes are pi apart on the sphere
    x = torch.randn(5, 3, dtype=torch.float64)
    np.testing.assert_allclose(P.sqmahalanobis(x, x, torch.eye(3, dtype=torch.float64)).numpy(),
                               cdist(x.numpy(), x.numpy(), "sqeuclidean"), rtol=1e-12, atol=1e-12)
    pts = torch.tensor([[0.3, -1.0], [-0.3, -1.0 + np.pi]], dtype=torch.float64)
    assert abs(float(P.haversine(pts, pts)[0, 1]) - np.pi) < 1e-7
    p1 = torch.rand(4, 5, dtype=torch.float64, requires_grad=True)
    p2 = torch.rand(3, 5, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(P.additive_chi2, (p1, p2))
    assert torch.autograd.gradcheck(lambda a, b: P.sqjensenshannon(a + 0.05, b + 0.05), (p1, p2))
    assert torch.autograd.gradcheck(P.haversine, (p1[:, :2], p2[:, :2]))
    assert torch.autograd.gradcheck(P.snr, (p1, p2))


def test_pins_catch_swapped_coordinates_and_a_dropped_half():
    g = npz("special.npz")
    t = {k: torch.from_numpy(v) for k, v in g.items()}
    assert not np.allclose(P.haversine(t["g1"].flip(-1), t["g2"].flip(-1)).numpy(), g["haversine"])
    q1 = t["p1"] / t["p1"].sum(-1, keepdim=True)
    q2 = t["p2"] / t["p2"].sum(-1, keepdim=True)
    assert not np.allclose((2 * P.sqjensenshannon(q1, q2)).sqrt().numpy(), g["js"])  # the / 2 dropped
    assert not np.allclose(P.sqjensenshannon(q1, q2).sqrt().numpy(), g["js_base2"])  # base ignored
    assert not np.allclose(P.sqmahalanobis(t["x1"], t["x2"], torch.linalg.inv(t["VI"])).sqrt().numpy(),
                           g["mahalanobis"])  # V for VI
