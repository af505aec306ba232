"""Cases of the unreduced pairwise binary ops (pwand, pwor, pwxor, pweq, pwne, pwlt, pwgt,
pwle, pwge) for oracle/ref_runner.run_op_case: unbatched, batched and batched with several
trailing feature dims; every element type the reference dispatches, mixed input types (the
common type of at::result_type), values with ties, NaN and +-0; and the refused cases (logical
ops on non-bool, ordering comparisons on bool, mismatched shapes), whose messages must match."""
from __future__ import annotations

import torch

OPS = ["pwand", "pwor", "pwxor", "pweq", "pwne", "pwlt", "pwgt", "pwle", "pwge"]
LOGICAL = {"pwand", "pwor", "pwxor"}


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _values(shape, dtype, seed):
    g = _g(seed)
    if dtype == torch.bool:
        return torch.rand(shape, generator=g) < 0.5
    v = torch.randint(-2, 3, shape, generator=g)  # few distinct values: many ties
    if dtype.is_floating_point:
        v = v.to(torch.float64) / 2
        flat = v.view(-1)
        if flat.numel() > 8:
            flat[3], flat[5], flat[7] = float("nan"), -0.0, 0.0
    elif dtype == torch.uint8:
        v = v + 2
    return v.to(dtype)


def pw_binary_cases():
    """[(case, tensors)] for run_op_case (forward only; the outputs are bool)."""
    cases = []
    shapes = [((7, 5), (9, 5)), ((2, 6, 4), (2, 3, 4)), ((2, 5, 3, 2), (2, 4, 3, 2)), ((3, 1), (2, 1))]
    dtypes = [torch.bool, torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64, torch.float32,
              torch.float64, torch.float16, torch.bfloat16]
    for op in OPS:
        for si, (s1, s2) in enumerate(shapes):
            for di, dt in enumerate(dtypes):
                a, b = _values(s1, dt, 10 * si + di), _values(s2, dt, 100 + 10 * si + di)
                cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]}, {"a": a, "b": b}))
        # mixed input types: the common type decides (float32 x int64 -> float32, bool x int -> int)
        cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]},
                      {"a": _values((4, 3), torch.float32, 1), "b": _values((5, 3), torch.int64, 2)}))
        cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]},
                      {"a": _values((4, 3), torch.bool, 3), "b": _values((5, 3), torch.int32, 4)}))
        # shape errors
        for s1, s2 in (((4,), (5, 4)), ((4, 3), (5,)), ((2, 4, 3), (3, 5, 3)), ((2, 4, 3), (2, 5, 2)),
                       ((4, 3), (5, 2)), ((2, 4, 3, 2), (2, 5, 3))):
            cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]},
                          {"a": torch.zeros(s1, dtype=torch.bool), "b": torch.zeros(s2, dtype=torch.bool)}))
    return cases


RED_OPS = ["pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean", "pwne_mean"]


def pw_reduction_cases():
    """[(case, tensors)] of the reduced forms (pw*_sum / pw*_mean -> float32 [b, n, m]): every
    dispatched element type, mixed types, NaN / +-0 / ties, a feature count past the popcount
    tiles (300), and the refused dtypes and shapes (only 2-D or 3-D inputs are taken)."""
    cases = []
    shapes = [((7, 5), (9, 5)), ((2, 6, 40), (2, 3, 40)), ((5, 300), (4, 300)), ((3, 1), (2, 1))]
    dtypes = [torch.bool, torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64, torch.float32,
              torch.float64, torch.float16, torch.bfloat16]
    for op in RED_OPS:
        for si, (s1, s2) in enumerate(shapes):
            for di, dt in enumerate(dtypes):
                a, b = _values(s1, dt, 10 * si + di), _values(s2, dt, 100 + 10 * si + di)
                cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]}, {"a": a, "b": b}))
        cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]},
                      {"a": _values((4, 3), torch.bool, 3), "b": _values((5, 3), torch.int32, 4)}))
        for s1, s2 in (((4,), (5, 4)), ((2, 4, 3, 2), (2, 5, 3, 2)), ((2, 4, 3), (3, 5, 3)), ((4, 3), (5, 2))):
            cases.append(({"op": op, "args": [{"t": "a"}, {"t": "b"}]},
                          {"a": torch.zeros(s1, dtype=torch.bool), "b": torch.zeros(s2, dtype=torch.bool)}))
    return cases
