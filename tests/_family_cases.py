"""Cases of the reference's internal metric ops (_ppminkowski, _wminkowski, _canberra,
_braycurtis, _additive_chi2_kernel, _sqjensenshannon, _haversine, _snr, _sqmahalanobis),
forward and autograd backward, for oracle/ref_runner.run_op_case: the same case runs on this
build (CPU or GPU) and on the reference's compiled CPU kernels (oracle/_ref)."""
from __future__ import annotations

import torch

INF = float("inf")


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _inputs(shape1, shape2, dtype, seed, kind="normal"):
    g = _g(seed)
    if kind == "ties":  # integer values: many equal |d| across k (first-extremum rule)
        a = torch.randint(-3, 4, shape1, generator=g).to(dtype)
        b = torch.randint(-3, 4, shape2, generator=g).to(dtype)
    elif kind == "positive":
        a = torch.rand(shape1, generator=g, dtype=torch.float64).to(dtype) + 0.05
        b = torch.rand(shape2, generator=g, dtype=torch.float64).to(dtype) + 0.05
    elif kind == "latlon":
        a = (torch.rand(shape1, generator=g, dtype=torch.float64) * 2 - 1).to(dtype)
        b = (torch.rand(shape2, generator=g, dtype=torch.float64) * 2 - 1).to(dtype)
    else:
        a = torch.randn(shape1, generator=g, dtype=torch.float64).to(dtype)
        b = torch.randn(shape2, generator=g, dtype=torch.float64).to(dtype)
    out_shape = shape1[:-1] + (shape2[-2],)
    return a, b, torch.randn(out_shape, generator=g, dtype=torch.float64).to(dtype)


def family_cases(dtype):
    """[(case, tensors)] for run_op_case."""
    cases = []
    shapes = [((37, 9), (23, 9)), ((2, 19, 7), (2, 29, 7))]

    def add(op, args, tensors, req, kind=None):
        cases.append(({"op": op, "args": args, "req": req, "grad": "g", "kind": kind or "values"}, tensors))

    for si, (s1, s2) in enumerate(shapes):
        for kind in ("normal", "ties"):
            a, b, g = _inputs(s1, s2, dtype, 10 + si, kind)
            w = torch.rand(s1[:-2] + (s1[-1],), generator=_g(20 + si), dtype=torch.float64).to(dtype) + 0.25
            ps = (1.0, 2.0, 3.0, 1.5, INF, -INF, 0.0) if kind == "normal" else (INF, -INF, 1.0)
            for p in ps:
                add("_ppminkowski", [{"t": "a"}, {"t": "b"}, {"v": p}], {"a": a, "b": b, "g": g}, ["a", "b"],
                    f"p={p}")
                if s1[:-2] == () or s1[-2] == s1[-1]:  # batched w must be [B, d]
                    add("_wminkowski", [{"t": "a"}, {"t": "b"}, {"t": "w"}, {"v": p}],
                        {"a": a, "b": b, "w": w, "g": g}, ["a", "b", "w"], f"p={p}")
        a, b, g = _inputs(s1, s2, dtype, 30 + si)
        a[..., ::3, 0] = 0.0  # canberra 0 / 0 terms are skipped
        b[..., ::2, 0] = 0.0
        add("_canberra", [{"t": "a"}, {"t": "b"}], {"a": a, "b": b, "g": g}, ["a", "b"])
        a, b, g = _inputs(s1, s2, dtype, 40 + si)
        add("_braycurtis", [{"t": "a"}, {"t": "b"}], {"a": a, "b": b, "g": g}, ["a", "b"])
        a, b, g = _inputs(s1, s2, dtype, 50 + si, "positive")
        add("_additive_chi2_kernel", [{"t": "a"}, {"t": "b"}], {"a": a, "b": b, "g": g}, ["a", "b"])
        for base in (None, 2.0):
            a, b, g = _inputs(s1, s2, dtype, 60 + si, "positive")
            a, b = a / a.sum(-1, keepdim=True), b / b.sum(-1, keepdim=True)
            add("_sqjensenshannon", [{"t": "a"}, {"t": "b"}, {"v": base}], {"a": a, "b": b, "g": g}, ["a", "b"])
        a, b, g = _inputs(s1[:-1] + (2,), s2[:-1] + (2,), dtype, 70 + si, "latlon")
        add("_haversine", [{"t": "a"}, {"t": "b"}], {"a": a, "b": b, "g": g}, ["a", "b"])
        a, b, g = _inputs(s1, s2, dtype, 80 + si)
        add("_snr", [{"t": "a"}, {"t": "b"}], {"a": a, "b": b, "g": g}, ["a", "b"])
        a, b, g = _inputs(s1, s2, dtype, 90 + si)
        d = s1[-1]
        m = torch.randn(s1[:-2] + (d, d), generator=_g(95 + si), dtype=torch.float64)
        VI = (m @ m.transpose(-1, -2) / d + torch.eye(d, dtype=torch.float64)).to(dtype)
        add("_sqmahalanobis", [{"t": "a"}, {"t": "b"}, {"t": "VI"}], {"a": a, "b": b, "VI": VI, "g": g},
            ["a", "b", "VI"])
    return cases
