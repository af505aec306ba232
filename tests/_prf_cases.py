"""Cases for the prf_div family (the 20 schemas of csrc/ops/prf_div.cpp:359-400): every
forward overload with its autograd backward, the in-place forms, the ten backward ops called
directly, in float32 / float64 / float16 / bfloat16 with zeros of both signs, NaN, +-inf,
underflow and overflow, plus integer promotion, mixed dtypes, empty, batched and
non-contiguous inputs and the error paths.  Used by the CPU pin against the compiled
reference and by the GPU parity test."""
from __future__ import annotations

import numpy as np
import torch

from oracle import pairwise as P

FLOAT_DTYPES = (torch.float32, torch.float64, torch.float16, torch.bfloat16)
MODES = ("zero", "identity")


def _operands(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(5, 13, generator=g, dtype=torch.float64) * 3
    b = torch.randn(5, 13, generator=g, dtype=torch.float64) * 3
    gr = torch.randn(5, 13, generator=g, dtype=torch.float64)
    special = [0.0, -0.0, float("nan"), float("inf"), -float("inf"), 1e-30, 7e4, -2.5, 1.0, 3.0]
    a[0, :10] = torch.tensor(special, dtype=torch.float64)
    b[1, :10] = torch.tensor(special, dtype=torch.float64)
    b[0, :10] = torch.tensor(special[::-1], dtype=torch.float64)
    b[2, ::3] = 0.0  # zero divisors among ordinary dividends
    b[3, 1::4] = -0.0
    a[4, ::2] = 0.0
    b[4, 5] = 1e30
    gr[2, 4] = float("nan")
    return a.to(dtype), b.to(dtype), gr.to(dtype)


def cases():
    """[(case dict, a, b, g)] — tensors on the CPU."""
    out = []
    for di, dtype in enumerate(FLOAT_DTYPES):
        a, b, g = _operands(dtype, 10 + di)
        for mode in MODES:
            for op in ("prf_div", "prf_ldiv"):
                out.append(({"kind": "fwd", "op": op, "ov": "default", "mode": mode, "grad": True}, a, b, g))
                for c in (0.0, 2.5, -0.1):
                    out.append(({"kind": "fwd", "op": op, "ov": "Scalar", "mode": mode, "grad": True,
                                 "scalar": c}, a, None, g))
                    out.append(({"kind": "fwd", "op": op, "ov": "rScalar", "mode": mode, "grad": True,
                                 "scalar": c}, None, b, g))
                out.append(({"kind": "inplace", "op": op + "_", "ov": "default", "mode": mode, "grad": True},
                            a, b, g))
                for c in (0.0, 2.5):
                    out.append(({"kind": "inplace", "op": op + "_", "ov": "Scalar", "mode": mode,
                                 "grad": True, "scalar": c}, a, None, g))
            for name in ("_prf_div_backward", "_prf_ldiv_backward", "_prf_div__backward", "_prf_ldiv__backward"):
                out.append(({"kind": "bwd", "op": name, "ov": "default", "mode": mode}, a, b, g))
                for c in (0.0, 2.5):
                    out.append(({"kind": "bwd", "op": name, "ov": "Scalar", "mode": mode, "scalar": c}, a, None, g))
                if "__" not in name:
                    for c in (0.0, -3.0):
                        out.append(({"kind": "bwd", "op": name, "ov": "rScalar", "mode": mode, "scalar": c},
                                    None, b, g))
    # integer and bool operands divide in float32; mixed float dtypes promote
    gi = torch.Generator().manual_seed(3)
    ia = torch.randint(-3, 4, (4, 6), generator=gi)
    ib = torch.randint(-2, 3, (4, 6), generator=gi)
    fa, fb, fg = _operands(torch.float32, 4)
    fa, fb, fg = fa[:4, :6].contiguous(), fb[:4, :6].contiguous(), fg[:4, :6].contiguous()
    for mode in MODES:
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode}, ia, ib, None))
        out.append(({"kind": "fwd", "op": "prf_ldiv", "ov": "default", "mode": mode}, ia.int(), ib, None))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode}, ia != 0, ib > 0, None))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "Scalar", "mode": mode, "scalar": 2}, ia, None, None))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "rScalar", "mode": mode, "scalar": 3}, None, ib, None))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode, "grad": True},
                    fa, ib.float(), fg))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode}, fa, fb.double(), None))
        out.append(({"kind": "fwd", "op": "prf_ldiv", "ov": "default", "mode": mode}, ia, fb, None))
        # empty, batched, non-contiguous
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode, "grad": True},
                    torch.zeros(0, 3), torch.ones(0, 3), torch.ones(0, 3)))
        ba, bb, bg = (t.reshape(2, 2, 6) for t in (fa, fb, fg))
        out.append(({"kind": "fwd", "op": "prf_ldiv", "ov": "default", "mode": mode, "grad": True}, ba, bb, bg))
        out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": mode, "grad": True},
                    fa.t(), fb.t(), fg.t()))
        out.append(({"kind": "inplace", "op": "prf_div_", "ov": "default", "mode": mode}, fa, fb.double(), None))
        out.append(({"kind": "inplace", "op": "prf_ldiv_", "ov": "default", "mode": mode}, fa.double(), fb, None))
        out.append(({"kind": "inplace", "op": "prf_div_", "ov": "default", "mode": mode, "grad": True},
                    fa.t(), fb.t(), fg.t()))
        out.append(({"kind": "inplace", "op": "prf_div_", "ov": "Scalar", "mode": mode, "scalar": 0.5}, fa.t(),
                    None, None))
    # error paths: shape mismatch, bad mode, in-place into an integer tensor, mixed-dtype backward
    out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": "zero"}, fa, fb[:3], None))
    out.append(({"kind": "inplace", "op": "prf_ldiv_", "ov": "default", "mode": "zero"}, fa, fb[:, :5], None))
    out.append(({"kind": "fwd", "op": "prf_div", "ov": "default", "mode": "ones"}, fa, fb, None))
    out.append(({"kind": "fwd", "op": "prf_ldiv", "ov": "Scalar", "mode": "bad", "scalar": 1.0}, fa, None, None))
    out.append(({"kind": "inplace", "op": "prf_div_", "ov": "default", "mode": "zero"}, ia, ib, None))
    out.append(({"kind": "inplace", "op": "prf_div_", "ov": "Scalar", "mode": "zero", "scalar": 2.0}, ia, None, None))
    out.append(({"kind": "bwd", "op": "_prf_div_backward", "ov": "default", "mode": "zero"}, fa.double(), fb, fg))
    return out


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


def assert_same_result(ours: dict, ref: dict, what: str) -> None:
    """Results equal bit for bit (NaN positions equal; a NaN's payload and sign may differ),
    or the same error message."""
    if "err" in ref or "err" in ours:
        assert ours.get("err") == ref.get("err"), f"{what}: {ours.get('err')!r} != {ref.get('err')!r}"
        return
    assert sorted(ours) == sorted(ref), f"{what}: results {sorted(ours)} != {sorted(ref)}"
    for k in ref:
        o, r = ours[k].cpu(), ref[k].cpu()
        assert o.dtype == r.dtype and o.shape == r.shape, f"{what}[{k}]: {o.dtype}{tuple(o.shape)} != {r.dtype}{tuple(r.shape)}"
        if o.is_floating_point():
            on, rn = torch.isnan(o), torch.isnan(r)
            assert torch.equal(on, rn), f"{what}[{k}]: NaN positions differ"
            ob, rb = _bits(o.masked_fill(on, 0)), _bits(r.masked_fill(rn, 0))
            assert np.array_equal(ob, rb), f"{what}[{k}]: values differ\n{o}\n{r}"
        else:
            assert torch.equal(o, r), f"{what}[{k}]"


def oracle_result(case: dict, a, b, g):
    """The numpy restatement (oracle/pairwise.py) of the kernel-level results of a case, for the
    float-dtype cases whose operands share one dtype; None where the oracle does not apply
    (integer promotion, errors, autograd through the in-place forms)."""
    tensors = [t for t in (a, b, g) if t is not None]
    if not tensors or any(not t.is_floating_point() or t.dtype != tensors[0].dtype for t in tensors):
        return None
    if case["mode"] not in MODES or (a is not None and b is not None and a.shape != b.shape):
        return None
    name = {torch.float32: "float32", torch.float64: "float64", torch.float16: "float16",
            torch.bfloat16: "bfloat16"}[tensors[0].dtype]
    R = P.elem_round(name)
    ident = case["mode"] == "identity"
    f64 = lambda t: None if t is None else t.double().numpy()  # noqa: E731
    A, B, G = f64(a), f64(b), f64(g)
    c = None if case.get("scalar") is None else float(R(case["scalar"]))
    left = "ldiv" in case["op"]
    kind, ov = case["kind"], case["ov"]
    res = {}
    if kind == "fwd":
        x, y = {"default": (A, B), "Scalar": (A, c), "rScalar": (c, B)}[ov]
        res["out"] = P.prf_div_forward(x, y, ident, R, left)
        if case.get("grad"):
            if ov == "default":
                gx, gy = P.prf_div_backward(G, B, A, ident, R) if left else P.prf_div_backward(G, A, B, ident, R)
                res["ga"], res["gb"] = (gy, gx) if left else (gx, gy)
            elif ov == "Scalar":
                res["ga"] = (P.prf_div_scalar_dividend_backward(G, A, c, R) if left
                             else P.prf_div_scalar_divisor_backward(G, c, ident, R))
            else:
                res["gb"] = (P.prf_div_scalar_divisor_backward(G, c, ident, R) if left
                             else P.prf_div_scalar_dividend_backward(G, B, c, R))
    elif kind == "bwd":
        if ov == "default":
            gx, gy = P.prf_div_backward(G, B, A, ident, R) if left else P.prf_div_backward(G, A, B, ident, R)
            res["ga"], res["gb"] = (gy, gx) if left else (gx, gy)
        elif ov == "Scalar":
            res["ga"] = (P.prf_div_scalar_dividend_backward(G, A, c, R) if left
                         else P.prf_div_scalar_divisor_backward(G, c, ident, R))
        else:
            res["gb"] = (P.prf_div_scalar_divisor_backward(G, c, ident, R) if left
                         else P.prf_div_scalar_dividend_backward(G, B, c, R))
    else:
        return None
    shape = (a if a is not None else b).shape
    return {k: torch.from_numpy(np.asarray(v, np.float64).reshape(shape)).to(tensors[0].dtype)
            for k, v in res.items()}
