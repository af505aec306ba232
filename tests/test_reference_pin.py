"""The oracle against the reference's own CPU kernels, compiled from its sources
(oracle/build_ref.py) and run in a child process (oracle/ref_runner.py).  Skipped when that
library is not built."""
import numpy as np
import pytest
import torch

from oracle import cref, ref_runner
from oracle import pairwise as P

pytestmark = pytest.mark.skipif(not ref_runner.available(), reason="oracle/_ref not built")


def test_hausdorff_oracle_equals_reference(tmp_path):
    rng = np.random.default_rng(11)
    x1 = rng.random((2, 3, 300, 3)).astype(np.float32)
    x2 = (rng.random((2, 2, 250, 3)) + 0.05).astype(np.float32)
    ref = ref_runner.run("hausdorff", {"x1": x1, "x2": x2}, tmp_path)
    for got, key in zip(cref.directed_hausdorff(x1, x2, threads=4), ("out", "idx1", "idx2")):
        assert np.array_equal(got, ref[key]), key
    for got, key in zip(P.directed_hausdorff(x1, x2), ("out", "idx1", "idx2")):
        assert np.array_equal(got, ref[key]), key


def test_hausdorff_ties_and_shuffle_equal_reference(tmp_path):
    rng = np.random.default_rng(12)
    x1 = rng.integers(0, 3, (2, 2, 80, 3)).astype(np.float32)
    x2 = rng.integers(0, 3, (2, 3, 70, 3)).astype(np.float32)
    ref = ref_runner.run("hausdorff", {"x1": x1, "x2": x2}, tmp_path)
    for got, key in zip(cref.directed_hausdorff(x1, x2), ("out", "idx1", "idx2")):
        assert np.array_equal(got, ref[key]), key
    ref = ref_runner.run("hausdorff", {"x1": x1, "x2": x2, "seed": np.int64(9)}, tmp_path)
    p1, p2 = P.hausdorff_permutations(2, 80, 70, torch.Generator().manual_seed(9))
    for got, key in zip(cref.directed_hausdorff(x1, x2, p1.numpy(), p2.numpy()), ("out", "idx1", "idx2")):
        assert np.array_equal(got, ref[key]), f"shuffled {key}"


def test_hausdorff_backward_equals_reference(tmp_path):
    rng = np.random.default_rng(13)
    x1 = rng.random((3, 120, 3)).astype(np.float32)
    x2 = (rng.random((2, 90, 3)) + 0.05).astype(np.float32)
    g = rng.standard_normal((3, 2)).astype(np.float32)
    ref = ref_runner.run("hausdorff_backward", {"x1": x1, "x2": x2, "grad": g}, tmp_path)
    out, i1, i2 = P.directed_hausdorff(x1, x2)
    gx1, gx2 = P.directed_hausdorff_backward(g, x1, x2, out, i1, i2)
    assert np.array_equal(gx1, ref["grad_x1"]) and np.array_equal(gx2, ref["grad_x2"])


@pytest.mark.parametrize("name", ["pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum",
                                  "pweq_mean", "pwne_mean"])
def test_pw_reductions_equal_reference(tmp_path, name):
    rng = np.random.default_rng(14)
    x1 = rng.random((2, 37, 70)) < 0.5
    x2 = rng.random((2, 29, 70)) < 0.3
    ref = ref_runner.run(f"pw_{name}", {"x1": x1, "x2": x2}, tmp_path)
    op = name.split("_")[0][2:]
    got = P.pw_reduce_bool(x1, x2, op, name.split("_")[1])
    assert np.array_equal(got.view(np.int32), ref["out"].view(np.int32))


def test_jaccard_and_non_bool_hamming_equal_reference(tmp_path):
    rng = np.random.default_rng(15)
    x1 = rng.random((40, 65)) < 0.1
    x2 = rng.random((30, 65)) < 0.1
    x1[:3] = False
    x2[:2] = False
    ref = ref_runner.run("jaccard", {"x1": x1, "x2": x2}, tmp_path)
    assert np.array_equal(P.jaccard_distances(x1, x2).view(np.int32), ref["out"].view(np.int32))
    i1 = rng.integers(0, 4, (20, 33)).astype(np.int64)
    i2 = rng.integers(0, 4, (25, 33)).astype(np.int64)
    ref = ref_runner.run("pw_pwne_mean", {"x1": i1, "x2": i2}, tmp_path)
    assert np.array_equal(P.hamming_distances(i1, i2), ref["out"])


def test_prf_div_family_equals_reference(tmp_path):
    """All 20 prf_div-family schemas on CPU tensors against the reference's own compiled CPU
    kernels and autograd (csrc/ops/prf_div.cpp, cpu/prf_div_kernel.cpp,
    autograd/prf_div_kernel.cpp): values, gradients, in-place results and error messages."""
    from tests._prf_cases import assert_same_result, cases

    import torchpairwise_amd  # noqa: F401  (registers this build's ops in this process)

    cs = cases()
    ref = ref_runner.run_prf_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    for (case, a, b, g), r in zip(cs, ref):
        ours = ref_runner.run_prf_case(ops, case, a, b, g, "cpu")
        assert_same_result(ours, r, str(case))


def test_prf_div_oracle_equals_reference(tmp_path):
    """The numpy restatement of the prf_div family (oracle/pairwise.py) against the compiled
    reference on every float case it covers (all four float dtypes, both modes, every
    overload and backward op)."""
    from tests._prf_cases import assert_same_result, cases, oracle_result

    cs = cases()
    ref = ref_runner.run_prf_reference(cs, tmp_path)
    checked = 0
    for (case, a, b, g), r in zip(cs, ref):
        want = oracle_result(case, a, b, g)
        if want is None:
            continue
        assert_same_result(want, {k: v for k, v in r.items() if k in want}, str(case))
        checked += 1
    assert checked >= 240


def _assert_results_close(ours, ref, rtol, what, exact_keys=(), atol_floor=0.0):
    if "err" in ref or "err" in ours:
        assert ours.get("err") == ref.get("err"), f"{what}: {ours.get('err')!r} != {ref.get('err')!r}"
        return
    assert sorted(ours) == sorted(ref), f"{what}: {sorted(ours)} != {sorted(ref)}"
    from tests._util import assert_close, assert_equal
    for k in ref:
        o, r = ours[k].cpu(), ref[k].cpu()
        assert o.dtype == r.dtype and o.shape == r.shape, f"{what}[{k}]"
        if k in exact_keys:
            assert_equal(o, r, f"{what}[{k}]", nan_payload=False)
            continue
        if o.is_floating_point():  # NaN where the reference's formulas give NaN, the rest close
            on, rn = torch.isnan(o), torch.isnan(r)
            assert torch.equal(on, rn), f"{what}[{k}]: NaN positions differ"
            o, r = o.masked_fill(on, 0), r.masked_fill(rn, 0)
        assert_close(o, r, rtol=rtol, atol=max(rtol * float(r.abs().max()), atol_floor) + 1e-300,
                     what=f"{what}[{k}]")


def test_family_ops_cpu_equal_reference(tmp_path):
    """This build's CPU loops of the reference's internal metric ops, forward and backward,
    against the reference's own compiled CPU kernels in float64 (and float32)."""
    from tests._family_cases import family_cases

    import torchpairwise_amd  # noqa: F401

    ops = torch.ops.torchpairwise
    for dtype, rtol in ((torch.float64, 1e-12), (torch.float32, 1e-5)):
        cs = family_cases(dtype)
        ref = ref_runner.run_op_reference(cs, tmp_path)
        for (case, tensors), r in zip(cs, ref):
            ours = ref_runner.run_op_case(ops, case, tensors, "cpu")
            _assert_results_close(ours, r, rtol, f"{case['op']} {case['kind']} {dtype}")


def test_public_ops_cpu_equal_reference(tmp_path):
    """Every public op on CPU tensors (the reference's own routes in this build) against the
    reference's compiled CPU library: values, gradients and error messages."""
    from tests._public_cases import public_cases

    import torchpairwise_amd  # noqa: F401

    _check_public_cases(torch.ops.torchpairwise, "cpu", tmp_path)


# The reference's own backward of these raises (an in-place op on a tensor its autograd saved):
# laplacian_kernel runs at::cdist(...).mul_(-gamma).exp_() (pairwise_metrics.cpp:103-110), and
# cdist's backward needs its output.  This build differentiates them; only the forward compares.
REFERENCE_BACKWARD_RAISES = "modified by an inplace operation"


def _check_public_cases(ops, device, tmp_path, rtol=1e-5, grad_rtol=1e-5):
    from tests._public_cases import public_cases

    cs = public_cases()
    ref = ref_runner.run_op_reference([(c, t) for c, t, _ in cs], tmp_path)
    retry = [(i, dict(c, grad=None, req=[]), t) for i, ((c, t, _), r) in enumerate(zip(cs, ref))
             if REFERENCE_BACKWARD_RAISES in r.get("err", "")]
    if retry:
        for (i, c, t), r in zip(retry, ref_runner.run_op_reference([(c, t) for _, c, t in retry], tmp_path)):
            cs[i] = (c, cs[i][1], cs[i][2])
            ref[i] = r
    failures = []
    for (case, tensors, exact), r in zip(cs, ref):
        ours = ref_runner.run_op_case(ops, case, tensors, device)
        keys = tuple(k for k in r if k != "err") if exact else ()
        if device != "cpu" and case["op"] == "russellrao_distances":
            keys = ()  # (D - and) / D: the GPU route's scalar division is 1 ulp from the CPU's
        what = f"{case['op']} {case['args']} {[tuple(t.shape) for t in tensors.values()]}"
        try:
            _assert_results_close({k: v for k, v in ours.items() if not k.startswith("grad")},
                                  {k: v for k, v in r.items() if not k.startswith("grad")}, rtol, what, keys,
                                  case.get("atol_floor", 0.0) if device != "cpu" else 0.0)
            _assert_results_close({k: v for k, v in ours.items() if k.startswith("grad") or k == "err"},
                                  {k: v for k, v in r.items() if k.startswith("grad") or k == "err"},
                                  grad_rtol, what, keys)
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures)


def _dtype_sweep_compare(ours, ref, what, floor=0.0, op=None):
    """Errors equal; bool / integer outputs equal; floating outputs within the dtype's bar
    (NaN positions equal)."""
    from tests._public_cases import dtype_tolerance

    assert sorted(ours) == sorted(ref), f"{what}: {ours.get('err')!r} != {ref.get('err')!r}"
    for k in ref:
        if k == "err":
            assert ours[k] == ref[k], f"{what}: {ours[k]!r} != {ref[k]!r}"
            continue
        o, r = ours[k].cpu(), ref[k].cpu()
        assert o.dtype == r.dtype and o.shape == r.shape, f"{what}[{k}]: {o.dtype} {tuple(o.shape)} vs {r.dtype} {tuple(r.shape)}"
        if not o.is_floating_point():
            assert torch.equal(o, r), f"{what}[{k}]"
            continue
        on, rn = torch.isnan(o), torch.isnan(r)
        assert torch.equal(on, rn), f"{what}[{k}]: NaN positions differ"
        of, rf = o.double().masked_fill(on, 0), r.double().masked_fill(rn, 0)
        tol = dtype_tolerance(o.dtype, op)
        atol = tol * max(1.0, float(rf.abs().max())) + floor
        assert torch.allclose(of, rf, rtol=tol, atol=atol), f"{what}[{k}]: max diff {float((of - rf).abs().max())}"


def test_public_ops_dtypes_cpu_equal_reference(tmp_path):
    """Every public op's forward on CPU tensors of float64, float16, bfloat16, int64, uint8 and
    bool against the reference's compiled library: the same results, or the same error (the
    reference refuses many of these; its dispatch messages are part of the interface)."""
    from tests._public_cases import public_dtype_cases

    import torchpairwise_amd  # noqa: F401

    cs = public_dtype_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t), r in zip(cs, ref):
        what = f"{case['op']} {[str(v.dtype) for v in t.values()]} {[tuple(v.shape) for v in t.values()]}"
        try:
            _dtype_sweep_compare(ref_runner.run_op_case(ops, case, t, "cpu"), r, what, op=case["op"])
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures[:30])


def test_cdist_names_cpu_equal_reference(tmp_path):
    """cdist(metric=...) for every metric name of the reference's dispatcher, with its extra
    arguments and defaults, and with an argument it does not take: the same values (boolean
    metrics and Hausdorff bit for bit) or the same TypeError."""
    from tests._public_cases import cdist_name_cases

    import torchpairwise_amd  # noqa: F401

    cs = cdist_name_cases()
    ref = ref_runner.run_op_reference([(c, t) for c, t, _ in cs], tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t, exact), r in zip(cs, ref):
        what = f"cdist {case['args'][2]['v']} {sorted(case['kwargs'])}"
        ours = ref_runner.run_op_case(ops, case, t, "cpu")
        try:
            _assert_results_close(ours, r, 1e-5, what, tuple(k for k in r if k != "err") if exact else ())
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures)


def test_neighbour_masks_cpu_equal_reference(tmp_path):
    """k_neighbors_mask / radius_neighbors_mask on CPU tensors over metrics, extra arguments,
    k up to past the column count, x2 = None and the error paths: bit for bit (or the same
    error) against the reference's compiled library."""
    from tests._public_cases import neighbour_cases

    import torchpairwise_amd  # noqa: F401

    cs = neighbour_cases()
    ref = ref_runner.run_op_reference(cs, tmp_path)
    ops = torch.ops.torchpairwise
    failures = []
    for (case, t), r in zip(cs, ref):
        what = f"{case['op']} {case['args'][2:]} {sorted(case['kwargs'])}"
        try:
            _assert_results_close(ref_runner.run_op_case(ops, case, t, "cpu"), r, 0.0, what,
                                  tuple(k for k in r if k != "err"))
        except AssertionError as e:
            failures.append(str(e).splitlines()[0][:300])
    assert not failures, f"{len(failures)} of {len(cs)} cases differ:\n" + "\n".join(failures)
