"""The unreduced pairwise binary ops (pwand ... pwge) on CPU tensors: against the reference's
compiled CPU kernels (oracle/_ref: values, output shapes and error messages, every case of
tests/_pw_binary_cases.py) and against numpy broadcasting of the same comparison."""
import numpy as np
import pytest
import torch

import torchpairwise_amd  # noqa: F401
from oracle import ref_runner
from tests._pw_binary_cases import LOGICAL, pw_binary_cases

NP = {"pwand": np.logical_and, "pwor": np.logical_or, "pwxor": np.logical_xor, "pweq": np.equal,
      "pwne": np.not_equal, "pwlt": np.less, "pwgt": np.greater, "pwle": np.less_equal, "pwge": np.greater_equal}


def _np(t):
    return t.float().numpy() if t.dtype in (torch.float16, torch.bfloat16) else t.numpy()


def _numpy_expected(op, a, b):
    """op(x1[b, i, k...], x2[b, j, k...]) -> [b, n, m, k...] (unbatched: [n, m, k])."""
    if a.dim() == 2:
        return NP[op](_np(a)[:, None, :], _np(b)[None, :, :])
    return NP[op](_np(a)[:, :, None], _np(b)[:, None, :])


def test_pw_binary_cpu_equal_numpy():
    ops = torch.ops.torchpairwise
    n = 0
    for case, t in pw_binary_cases():
        a, b = t["a"], t["b"]
        if a.dim() < 2 or b.dim() < 2 or a.dtype != b.dtype or (a.dim() > 2 and a.shape[2:] != b.shape[2:]) \
                or (a.dim() == 2 and a.shape[1] != b.shape[1]) or (a.dim() > 2 and a.shape[0] != b.shape[0]):
            continue
        op = case["op"]
        if (op in LOGICAL) != (a.dtype == torch.bool) and not (a.dtype == torch.bool and op in ("pweq", "pwne")):
            with pytest.raises(NotImplementedError, match="pairwise_binary_forward_cpu"):
                getattr(ops, op)(a, b)
            continue
        got = getattr(ops, op)(a, b)
        want = _numpy_expected(op, a, b)
        assert got.dtype == torch.bool and tuple(got.shape) == want.shape, (op, a.shape, b.shape)
        assert np.array_equal(got.numpy(), want), (op, a.dtype, a.shape)
        n += 1
        if op == "pwlt" and a.dim() == 2 and a.dtype == torch.float32:
            # the pin catches swapped operands
            assert not np.array_equal(got.numpy(), _numpy_expected("pwlt", b, a).transpose(1, 0, 2))
    assert n > 150


def test_pw_binary_cpu_equal_reference(tmp_path):
    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = pw_binary_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t), r in zip(cs, ref):
        ours = ref_runner.run_op_case(ops, case, t, "cpu")
        what = f"{case['op']} {t['a'].dtype}/{t['b'].dtype} {tuple(t['a'].shape)} {tuple(t['b'].shape)}"
        if "err" in r or "err" in ours:
            if ours.get("err") != r.get("err"):
                failures.append(f"{what}: {ours.get('err')!r} != {r.get('err')!r}")
            continue
        if not (ours["out0"].shape == r["out0"].shape and torch.equal(ours["out0"], r["out0"])):
            failures.append(f"{what}: outputs differ")
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures[:20])


def test_pw_reductions_cpu_equal_reference(tmp_path):
    """pw*_sum / pw*_mean on CPU tensors of every element type and the refused ones against the
    reference's compiled kernels: float32 counts bit for bit, the same errors."""
    from tests._pw_binary_cases import pw_reduction_cases

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    cs = pw_reduction_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t), r in zip(cs, ref):
        ours = ref_runner.run_op_case(ops, case, t, "cpu")
        what = f"{case['op']} {t['a'].dtype}/{t['b'].dtype} {tuple(t['a'].shape)} {tuple(t['b'].shape)}"
        if "err" in r or "err" in ours:
            if ours.get("err") != r.get("err"):
                failures.append(f"{what}: {ours.get('err')!r} != {r.get('err')!r}")
            continue
        o, w = ours["out0"], r["out0"]
        if not (o.dtype == w.dtype and o.shape == w.shape and torch.equal(o, w)):
            failures.append(f"{what}: outputs differ")
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures[:30])
