"""Cases of the public ops (the 39 metric schemas of csrc/ops/pairwise_metrics.h, cdist and
the neighbour masks) for oracle/ref_runner.run_op_case: each runs on this build and on the
reference's compiled CPU library with the same inputs.  "exact" cases (boolean metrics,
directed Hausdorff, masks) compare bit for bit; the others within the fp32 bar."""
from __future__ import annotations

import torch

BOOL_METRICS = ["hamming", "jaccard", "kulsinski", "kulczynski1", "yule", "dice", "rogerstanimoto",
                "russellrao", "sokalmichener", "sokalsneath"]


def _g(seed):
    return torch.Generator().manual_seed(seed)


def public_cases():
    """[(case, tensors, exact)]; a case may carry "atol_floor": an absolute allowance for values
    whose form has a known floor (the matrix-product euclidean of a point with itself)."""
    out = []
    a = torch.randn(37, 16, generator=_g(1))
    b = torch.randn(29, 16, generator=_g(2))
    ab = torch.randn(2, 37, 16, generator=_g(3))
    bb = torch.randn(2, 29, 16, generator=_g(4))
    g = torch.randn(37, 29, generator=_g(5))
    gb = torch.randn(2, 37, 29, generator=_g(6))
    pa, pb = torch.rand(37, 16, generator=_g(7)) + 0.05, torch.rand(29, 16, generator=_g(8)) + 0.05
    la = torch.rand(37, 2, generator=_g(9)) * 2 - 1
    lb = torch.rand(29, 2, generator=_g(10)) * 2 - 1
    w = torch.rand(16, generator=_g(11)) + 0.2
    VI = torch.eye(16) + 0.1 * torch.ones(16, 16)

    def add(op, args, tensors, req=(), grad=None, exact=False, kwargs=None):
        case = {"op": op, "args": args, "kwargs": kwargs or {}, "req": list(req)}
        if grad:
            case["grad"] = grad
        out.append((case, tensors, exact))

    T = lambda name: {"t": name}  # noqa: E731
    V = lambda v: {"v": v}  # noqa: E731
    plain = ["euclidean_distances", "manhattan_distances", "cosine_distances", "linear_kernel",
             "cosine_similarity", "sqeuclidean_distances", "correlation_distances", "cityblock_distances",
             "chebyshev_distances", "braycurtis_distances", "canberra_distances", "l1_distances",
             "l2_distances", "linf_distances", "snr_distances"]
    for name in plain:
        add(name, [T("a"), T("b")], {"a": a, "b": b, "g": g}, ("a", "b"), "g")
        add(name, [T("a"), T("b")], {"a": ab, "b": bb, "g": gb}, ("a", "b"), "g")
    for name in ("euclidean_distances", "cosine_distances", "sqeuclidean_distances"):
        add(name, [T("a")], {"a": a, "g": torch.randn(37, 37, generator=_g(12))}, ("a",), "g")
    # x2 = None euclidean: |a|^2 + |a|^2 - 2 a.a in fp32 leaves a few ulp of 2|a|^2 on the diagonal
    # (the reference's own GPU form, at::cdist's matrix product, does the same)
    out[-3][0]["atol_floor"] = 4 * float((torch.finfo(torch.float32).eps * 2 * (a * a).sum(1).max()) ** 0.5)
    for name, extra in (("polynomial_kernel", [V(3), V(None), V(1.0)]), ("polynomial_kernel", [V(2), V(0.3), V(0.5)]),
                        ("sigmoid_kernel", [V(None), V(1.0)]), ("rbf_kernel", [V(None)]), ("rbf_kernel", [V(0.2)]),
                        ("laplacian_kernel", [V(None)]), ("minkowski_distances", [V(3.0)]),
                        ("minkowski_distances", [V(1.5)]), ("lp_distances", [V(2.0)])):
        add(name, [T("a"), T("b"), *extra], {"a": a, "b": b, "g": g}, ("a", "b"), "g")
    add("wminkowski_distances", [T("a"), T("b"), V(3.0), T("w")], {"a": a, "b": b, "w": w, "g": g},
        ("a", "b", "w"), "g")
    add("seuclidean_distances", [T("a"), T("b"), T("w")], {"a": a, "b": b, "w": w, "g": g}, ("a", "b", "w"), "g")
    add("mahalanobis_distances", [T("a"), T("b"), T("VI")], {"a": a, "b": b, "VI": VI, "g": g},
        ("a", "b", "VI"), "g")
    add("additive_chi2_kernel", [T("a"), T("b")], {"a": pa, "b": pb, "g": g}, ("a", "b"), "g")
    add("chi2_kernel", [T("a"), T("b"), V(0.7)], {"a": pa, "b": pb, "g": g}, ("a", "b"), "g")
    add("jensenshannon_distances", [T("a"), T("b"), V(None)], {"a": pa, "b": pb, "g": g}, ("a", "b"), "g")
    add("jensenshannon_distances", [T("a"), T("b"), V(2.0)], {"a": pa, "b": pb, "g": g}, ("a", "b"), "g")
    add("haversine_distances", [T("a"), T("b")], {"a": la, "b": lb, "g": g}, ("a", "b"), "g")
    # boolean metrics: bit-exact counts and the reference's float32 arithmetic
    ba = torch.rand(37, 70, generator=_g(13)) < 0.3
    bbo = torch.rand(29, 70, generator=_g(14)) < 0.3
    ba[:2] = False
    bbo[:3] = False
    for m in BOOL_METRICS:
        add(f"{m}_distances", [T("a"), T("b")], {"a": ba, "b": bbo}, exact=True)
    add("hamming_distances", [T("a"), T("b")], {"a": torch.randint(0, 3, (37, 21), generator=_g(15)),
                                                "b": torch.randint(0, 3, (29, 21), generator=_g(16))}, exact=True)
    # directed Hausdorff: value and indices bit for bit, gradient of the value
    c1 = torch.rand(3, 200, 3, generator=_g(17))
    c2 = torch.rand(2, 150, 3, generator=_g(18)) + 0.05
    add("directed_hausdorff_distances", [T("a"), T("b")], {"a": c1, "b": c2, "g": torch.randn(3, 2, generator=_g(19))},
        ("a", "b"), "g", exact=True)
    # cdist by name and the neighbour masks
    for metric in ("euclidean", "manhattan", "cosine", "chebyshev", "canberra"):
        add("cdist", [T("a"), T("b"), V(metric)], {"a": a, "b": b})
    add("cdist", [T("a"), T("b"), V("minkowski")], {"a": a, "b": b}, kwargs={"p": V(3.0)})
    add("cdist", [T("a"), T("b"), V("jaccard")], {"a": ba, "b": bbo}, exact=True)
    add("cdist", [T("a"), T("b"), V("nope")], {"a": a, "b": b}, exact=True)
    add("cdist", [T("a"), T("b"), V("euclidean")], {"a": a, "b": b}, exact=True, kwargs={"p": V(2.0)})
    add("k_neighbors_mask", [T("a"), T("b"), V(3)], {"a": a, "b": b}, exact=True)
    add("radius_neighbors_mask", [T("a"), T("b"), V(5.0)], {"a": a, "b": b}, exact=True)
    add("pdist", [T("a")], {"a": a}, exact=True)
    return out


DTYPE_SWEEP = [torch.float64, torch.float16, torch.bfloat16, torch.int64, torch.uint8, torch.bool]


def public_dtype_cases():
    """[(case, tensors)]: the forward cases of public_cases() (directed Hausdorff aside) with
    every tensor cast to each of DTYPE_SWEEP (integers: small rounded values; bool: != 0).  The
    reference raises for many of them; its messages are part of the interface."""
    out = []
    for case, t, _ in public_cases():
        if case["op"] == "directed_hausdorff_distances":
            continue
        for dt in DTYPE_SWEEP:
            tt = {}
            for k, v in t.items():
                if k == "g":
                    continue
                if dt == torch.bool:
                    tt[k] = v != 0
                elif v.dtype == torch.bool:
                    tt[k] = v.to(dt)
                elif dt in (torch.int64, torch.uint8):
                    tt[k] = (v * 3).round().clamp(0 if dt == torch.uint8 else -9, 9).to(dt)
                else:
                    tt[k] = v.to(dt)
            c = {k: v for k, v in case.items() if k not in ("grad", "req")}
            c["req"] = []
            out.append((c, tt))
    return out


def dtype_tolerance(dtype, op=None):
    """The bar for a floating output of `op` in `dtype` against the reference's own result in the
    same dtype.  bfloat16 Mahalanobis takes 3e-2: the reference's loop
    (cpu/sqmahalanobis_kernel.cpp:23-29) adds the quadratic form's d^2 terms (256 at d = 16)
    into a bfloat16 variable, rounding to 8 significant bits after every addition, while this
    build accumulates in float32; every other op and dtype pair holds 1e-2."""
    if op == "mahalanobis_distances" and dtype == torch.bfloat16:
        return 3e-2
    return {torch.float64: 1e-10, torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}.get(dtype, 0.0)


CDIST_METRICS = ["braycurtis", "canberra", "chebyshev", "cityblock", "correlation", "cosine", "dice",
                 "directed_hausdorff", "euclidean", "hamming", "haversine", "jaccard", "jensenshannon",
                 "kulczynski1", "kulsinski", "l1", "l2", "lp", "linf", "mahalanobis", "manhattan", "minkowski",
                 "rogerstanimoto", "russellrao", "seuclidean", "snr", "sokalmichener", "sokalsneath",
                 "sqeuclidean", "wminkowski", "yule"]
BOOL_NAMES = {"dice", "hamming", "jaccard", "kulczynski1", "kulsinski", "rogerstanimoto", "russellrao",
              "sokalmichener", "sokalsneath", "yule"}


def cdist_name_cases():
    """[(case, tensors, exact)] of cdist(x1, x2, metric, **extra) for every metric the reference's
    dispatcher knows (cpdist.cpp), with its extra arguments where it takes them (and their
    defaults), plus one argument it does not take (the reference raises TypeError naming it and
    the supported signature)."""
    a = torch.randn(37, 16, generator=_g(31))
    b = torch.randn(29, 16, generator=_g(32))
    pa, pb = torch.rand(37, 16, generator=_g(33)) + 0.05, torch.rand(29, 16, generator=_g(34)) + 0.05
    ba, bb = torch.rand(37, 70, generator=_g(35)) < 0.3, torch.rand(29, 70, generator=_g(36)) < 0.3
    la, lb = torch.rand(37, 2, generator=_g(37)) * 2 - 1, torch.rand(29, 2, generator=_g(38)) * 2 - 1
    ca, cb = torch.rand(3, 60, 3, generator=_g(39)), torch.rand(2, 50, 3, generator=_g(40)) + 0.05
    w = torch.rand(16, generator=_g(41)) + 0.2
    VI = torch.eye(16) + 0.1 * torch.ones(16, 16)
    T = lambda name: {"t": name}  # noqa: E731
    V = lambda v: {"v": v}  # noqa: E731
    out = []
    for metric in CDIST_METRICS:
        if metric in BOOL_NAMES:
            ts, exact = {"a": ba, "b": bb}, True
        elif metric == "haversine":
            ts, exact = {"a": la, "b": lb}, False
        elif metric == "directed_hausdorff":
            ts, exact = {"a": ca, "b": cb}, True
        elif metric == "jensenshannon":
            ts, exact = {"a": pa, "b": pb}, False
        else:
            ts, exact = {"a": a, "b": b}, False
        variants = [{}]
        if metric in ("minkowski", "lp"):
            variants = [{}, {"p": V(3.0)}, {"p": V(1.0)}]
        elif metric == "wminkowski":
            ts = dict(ts, w=w)
            variants = [{"w": T("w")}, {"w": T("w"), "p": V(3.0)}]
        elif metric == "seuclidean":
            ts = dict(ts, V=w)
            variants = [{"V": T("V")}]
        elif metric == "mahalanobis":
            ts = dict(ts, VI=VI)
            variants = [{"VI": T("VI")}]
        elif metric == "jensenshannon":
            variants = [{}, {"base": V(2.0)}]
        elif metric == "directed_hausdorff":
            variants = [{}, {"shuffle": V(False)}]
        for kw in variants:
            out.append(({"op": "cdist", "args": [T("a"), T("b"), V(metric)], "kwargs": kw, "req": []}, ts, exact))
        bad = {"base": V(2.0)} if metric != "jensenshannon" else {"p": V(2.0)}
        out.append(({"op": "cdist", "args": [T("a"), T("b"), V(metric)], "kwargs": dict(variants[0], **bad), "req": []},
                    ts, True))
    return out


def _margin_eps(d, q):
    """A radius between two consecutive sorted distances near quantile q whose gap is wide
    (relative 1e-3), so no device's rounding moves a distance across it."""
    v = torch.sort(d.flatten().double()).values
    i0 = int(q * (v.numel() - 1))
    for off in range(v.numel()):
        for i in (i0 + off, i0 - off):
            if 0 <= i < v.numel() - 1 and v[i + 1] - v[i] > 1e-3 * max(1.0, float(v[i].abs())):
                return float((v[i] + v[i + 1]) / 2)
    return float(v[-1]) + 1.0


def neighbour_cases():
    """[(case, tensors)] of k_neighbors_mask / radius_neighbors_mask over metrics and their
    extra arguments, k from 0 past the column count, x2 = None, and the error paths.  Inputs
    are tie-free random points (the reference's argsort is unstable on ties); radii sit in wide
    gaps between distances."""
    import torchpairwise_amd as tp  # the CPU route (at::cdist and this build's CPU loops)

    a = torch.randn(37, 16, generator=_g(51))
    b = torch.randn(29, 16, generator=_g(52))
    pa, pb = torch.rand(37, 16, generator=_g(53)) + 0.05, torch.rand(29, 16, generator=_g(54)) + 0.05
    la, lb = torch.rand(37, 2, generator=_g(55)) * 2 - 1, torch.rand(29, 2, generator=_g(56)) * 2 - 1
    ba, bb = torch.rand(37, 70, generator=_g(57)) < 0.3, torch.rand(29, 70, generator=_g(58)) < 0.3
    w = torch.rand(16, generator=_g(59)) + 0.2
    VI = torch.eye(16) + 0.1 * torch.ones(16, 16)
    T = lambda name: {"t": name}  # noqa: E731
    V = lambda v: {"v": v}  # noqa: E731
    metrics = [("euclidean", {}, "f"), ("manhattan", {}, "f"), ("cosine", {}, "f"), ("chebyshev", {}, "f"),
               ("minkowski", {"p": V(3.0)}, "f"), ("sqeuclidean", {}, "f"), ("correlation", {}, "f"),
               ("canberra", {}, "f"), ("braycurtis", {}, "f"), ("wminkowski", {"w": T("w"), "p": V(3.0)}, "f"),
               ("seuclidean", {"V": T("w")}, "f"), ("mahalanobis", {"VI": T("VI")}, "f"),
               ("haversine", {}, "l"), ("jensenshannon", {}, "p"), ("jaccard", {}, "b"), ("hamming", {}, "b")]
    out = []
    for metric, kw, kind in metrics:
        x1, x2 = {"f": (a, b), "p": (pa, pb), "l": (la, lb), "b": (ba, bb)}[kind]
        ts = {"a": x1, "b": x2, "w": w, "VI": VI}
        extra = {"w": w, "V": w, "VI": VI, "p": 3.0}
        d = tp.cdist(x1, x2, metric, **{k: extra[k] for k in kw})
        for q in (0.1, 0.6):
            out.append(({"op": "radius_neighbors_mask", "args": [T("a"), T("b"), V(_margin_eps(d, q)), V(metric)],
                         "kwargs": kw, "req": []}, ts))
        if kind == "b":
            continue  # many equal distances: the reference's argsort order is unspecified there
        for k in (0, 1, 4, 40):
            out.append(({"op": "k_neighbors_mask", "args": [T("a"), T("b"), V(k), V(metric)], "kwargs": kw,
                         "req": []}, ts))
    ts = {"a": a, "b": b}
    out.append(({"op": "k_neighbors_mask", "args": [T("a")], "kwargs": {"k": V(2)}, "req": []}, ts))
    out.append(({"op": "radius_neighbors_mask", "args": [T("a")], "kwargs": {"epsilon": V(5.0)}, "req": []}, ts))
    for case in (("k_neighbors_mask", [T("a"), T("b"), V(-1)]), ("radius_neighbors_mask", [T("a"), T("b"), V(-1.0)]),
                 ("k_neighbors_mask", [T("a"), T("b"), V(1), V("nope")]),
                 ("radius_neighbors_mask", [T("a"), T("b"), V(1.0), V("euclidean")])):
        kw = {"p": V(2.0)} if case[1][-1] == V("euclidean") else {}
        out.append(({"op": case[0], "args": case[1], "kwargs": kw, "req": []}, ts))
    return out
