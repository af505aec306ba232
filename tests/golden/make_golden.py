#!/usr/bin/env python3
"""Writes the golden fixtures in tests/golden/*.npz.

The reference ships no golden vectors (its tests only print differences), so the expected
values here come from independent implementations and from hand-derived cases, never from
this build's oracle:

* hamming / jaccard / dice ...:  scipy.spatial.distance.cdist in float64, rounded to float32
  (a float64 quotient of integers below 2^24 rounds to the correctly rounded float32 one);
  the pw*_sum counts by an explicit Python loop over elements;
* minkowski p = 1, 2, 3, inf:   scipy.spatial.distance.cdist in float64;
* cosine:                       sklearn.metrics.pairwise.cosine_distances in float64;
* directed Hausdorff:           scipy.spatial.distance.directed_hausdorff (value, float64) on
  random clouds, plus hand-built clouds whose maxima / minima tie, with the expected
  indices derived by hand from the reference's rules (last m reaching the max, first n
  reaching that m's min; csrc/ops/cpu/hausdorff_kernel.cpp:25-51);
* the reference's VALU family (sqeuclidean, weighted minkowski, seuclidean, canberra,
  braycurtis):                  scipy.spatial.distance.cdist in float64 (with a zero
  coordinate pair for canberra's skipped 0/0 term);
* chi2 / jensenshannon / haversine / mahalanobis: sklearn additive_chi2_kernel, chi2_kernel,
  haversine_distances and scipy jensenshannon (base e and 2), cdist 'mahalanobis', in
  float64 (with a zero coordinate pair for chi2's skipped 0 / 0 term);
* neighbour masks:              sklearn.neighbors.NearestNeighbors(algorithm="brute")
  kneighbors_graph / radius_neighbors_graph (connectivity, float64) on tie-free random
  points, plus hand-built distance rows with ties, NaN, +-0 and inf whose masks are
  written out by hand (ascending, NaN last, -0 == +0, ties to the lower column).

Run from the repository root: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
from scipy.spatial.distance import cdist, directed_hausdorff
from sklearn.metrics.pairwise import cosine_distances

OUT = Path(__file__).resolve().parent


def boolean():
    rng = np.random.default_rng(20260101)
    x1 = rng.random((7, 45)) < 0.5
    x2 = rng.random((6, 45)) < 0.3
    x1[0] = False  # all-zero rows: jaccard 0 against an all-zero partner
    x2[0] = False
    ops = {"and": np.logical_and, "or": np.logical_or, "xor": np.logical_xor,
           "eq": np.equal, "ne": np.not_equal}
    counts = {}
    for name, f in ops.items():
        c = np.zeros((7, 6), np.int64)
        for i in range(7):
            for j in range(6):
                c[i, j] = sum(int(f(x1[i, k], x2[j, k])) for k in range(45))
        counts[f"count_{name}"] = c
    out = dict(x1=x1, x2=x2, **counts)
    for metric in ("hamming", "jaccard", "dice", "rogerstanimoto", "russellrao", "sokalsneath", "yule"):
        with np.errstate(divide="ignore", invalid="ignore"):
            out[metric] = cdist(x1, x2, metric)
    out["hamming_f32"] = out["hamming"].astype(np.float32)
    out["jaccard_f32"] = out["jaccard"].astype(np.float32)
    # hamming with d a power of two: exact dyadic values k / 64
    y1 = rng.random((5, 64)) < 0.5
    y2 = rng.random((4, 64)) < 0.5
    out["y1"], out["y2"] = y1, y2
    out["hamming_d64"] = cdist(y1, y2, "hamming").astype(np.float32)
    np.savez_compressed(OUT / "boolean.npz", **out)


def minkowski():
    rng = np.random.default_rng(20260102)
    x1 = rng.standard_normal((9, 13))
    x2 = rng.standard_normal((11, 13))
    out = dict(x1=x1, x2=x2)
    for p in (1, 2, 3):
        out[f"p{p}"] = cdist(x1, x2, "minkowski", p=p)
    out["pinf"] = cdist(x1, x2, "chebyshev")
    out["cosine"] = cosine_distances(x1, x2)
    np.savez_compressed(OUT / "minkowski_cosine.npz", **out)


def hausdorff():
    rng = np.random.default_rng(20260103)
    a = rng.random((3, 40, 3)).astype(np.float32)
    b = (rng.random((2, 50, 3)) + 0.05).astype(np.float32)
    value = np.zeros((3, 2))
    for i in range(3):
        for j in range(2):
            value[i, j] = directed_hausdorff(a[i].astype(np.float64), b[j].astype(np.float64))[0]
    # hand-built ties (1-D points padded to 3-D)
    def pts(xs):
        return np.array([[x, 0.0, 0.0] for x in xs], np.float32)

    # m mins: [0, 0, 1, 1] -> max 1 reached by m = 2 and m = 3 -> last m = 3;
    # for m = 3 (x = 3), n = 2 (x = 2) and n = 3 (x = 4) tie at 1 -> first n = 2
    t1 = (pts([0, 1, 3, 3]), pts([0, 1, 2, 4]), 1.0, 3, 2)
    # single winner in the middle, later points closer: m = 1 (x = 10) min 4 at n = 2 (x = 6)
    t2 = (pts([0, 10, 1]), pts([0, 1, 6, 14]), 4.0, 1, 2)
    # identical clouds: every min is 0 -> last m, and its first n at distance 0
    t3 = (pts([5, 2, 7]), pts([2, 7, 5, 5]), 0.0, 2, 1)
    np.savez_compressed(
        OUT / "hausdorff.npz", a=a, b=b, value=value,
        **{f"t{k}_{f}": v for k, t in enumerate((t1, t2, t3), 1)
           for f, v in zip(("x1", "x2", "value", "idx1", "idx2"), t)})


def family():
    rng = np.random.default_rng(20260105)
    x1 = rng.standard_normal((8, 6))
    x2 = rng.standard_normal((10, 6))
    x1[0, 2] = x2[1, 2] = 0.0  # canberra: a 0 / 0 term, skipped
    w = rng.random(6) + 0.2
    V = rng.random(6) + 0.5
    out = dict(x1=x1, x2=x2, w=w, V=V)
    out["sqeuclidean"] = cdist(x1, x2, "sqeuclidean")
    out["canberra"] = cdist(x1, x2, "canberra")
    out["braycurtis"] = cdist(x1, x2, "braycurtis")
    for p in (1, 2, 3):
        out[f"wminkowski_p{p}"] = cdist(x1, x2, "minkowski", p=p, w=w)
    out["seuclidean"] = cdist(x1, x2, "seuclidean", V=V)
    out["seuclidean_self"] = cdist(x1, x1, "seuclidean", V=x1.var(0, ddof=1))
    np.savez_compressed(OUT / "family.npz", **out)


def special():
    from scipy.spatial.distance import jensenshannon
    from sklearn.metrics.pairwise import additive_chi2_kernel, chi2_kernel, haversine_distances

    rng = np.random.default_rng(20260106)
    p1 = rng.random((6, 5))
    p2 = rng.random((8, 5))
    p1[0, 1] = p2[3, 1] = 0.0  # chi2: a 0 / 0 term, skipped
    out = dict(p1=p1, p2=p2)
    out["additive_chi2"] = additive_chi2_kernel(p1, p2)
    out["chi2_g07"] = chi2_kernel(p1, p2, gamma=0.7)
    out["js"] = np.array([[jensenshannon(a, b) for b in p2] for a in p1])
    out["js_base2"] = np.array([[jensenshannon(a, b, base=2) for b in p2] for a in p1])
    g1 = rng.random((7, 2)) * np.array([np.pi, 2 * np.pi]) - np.array([np.pi / 2, np.pi])
    g2 = rng.random((9, 2)) * np.array([np.pi, 2 * np.pi]) - np.array([np.pi / 2, np.pi])
    out["g1"], out["g2"] = g1, g2
    out["haversine"] = haversine_distances(g1, g2)
    x1 = rng.standard_normal((7, 4))
    x2 = rng.standard_normal((9, 4))
    a = rng.standard_normal((4, 4))
    VI = a @ a.T + np.eye(4)
    out["x1"], out["x2"], out["VI"] = x1, x2, VI
    out["mahalanobis"] = cdist(x1, x2, "mahalanobis", VI=VI)
    np.savez_compressed(OUT / "special.npz", **out)


def neighbors():
    from sklearn.neighbors import NearestNeighbors

    rng = np.random.default_rng(20260104)
    x1 = rng.standard_normal((12, 6))
    x2 = rng.standard_normal((15, 6))
    out = dict(x1=x1, x2=x2)
    nn = NearestNeighbors(algorithm="brute").fit(x2)
    for k in (0, 1, 4):
        out[f"knn_k{k}"] = nn.kneighbors_graph(x1, n_neighbors=k + 1).toarray().astype(bool)
    out["radius_eps"] = np.float64(3.0)
    out["radius"] = nn.radius_neighbors_graph(x1, radius=3.0).toarray().astype(bool)
    # hand-built rows: (distances, count, expected mask)
    nan, inf = np.nan, np.inf
    T, F = True, False
    cases = [
        ([3, 1, 1, 0, nan], 3, [F, T, T, T, F]),
        ([3, 1, 1, 0, nan], 2, [F, T, F, T, F]),            # tie 1/1 -> lower column
        ([-0.0, 0.0, -1, inf, nan, 2], 2, [T, F, T, F, F, F]),  # -0 == +0 -> lower column
        ([-0.0, 0.0, -1, inf, nan, 2], 3, [T, T, T, F, F, F]),
        ([-0.0, 0.0, -1, inf, nan, 2], 5, [T, T, T, T, F, T]),  # inf before NaN
        ([5, 5, 5, 5], 2, [T, T, F, F]),
        ([nan, nan, 1], 2, [T, F, T]),                      # NaN ties -> lower column
        ([2, 7, 1, 8, 2, 8], 4, [T, T, T, F, T, F]),        # 1, 2, 2, 7
    ]
    for i, (row, count, want) in enumerate(cases):
        out[f"row{i}_dist"] = np.array([row], np.float32)
        out[f"row{i}_count"] = np.int64(count)
        out[f"row{i}_mask"] = np.array([want], bool)
    out["n_rows"] = np.int64(len(cases))
    np.savez_compressed(OUT / "neighbors.npz", **out)


if __name__ == "__main__":
    boolean()
    minkowski()
    hausdorff()
    family()
    special()
    neighbors()
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))
