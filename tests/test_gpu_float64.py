"""float64 (and float16 for directed Hausdorff) on the GPU: the reference's CUDA kernels serve
these dtypes (AT_DISPATCH_FLOATING_TYPES_AND*), so this build runs them on its own kernels
(valu_f64.hip, hausdorff_exact.hip).  The bar: this build's CPU loops in the same dtype (which
test_reference_pin.py pins to the reference's compiled CPU kernels) and, where oracle/_ref is
built, the reference's kernels themselves.  float64 values rtol 1e-12 and gradients 1e-11
(each + rtol * max|ref|: the device's pow / log / sin differ from glibc's in the last bits);
the p = +-inf gradients of x1 and x2 and every directed Hausdorff output (value, indices,
gradients) bit for bit."""
import pytest
import torch

import torchpairwise_amd as tp
from oracle import pairwise as P
from torchpairwise_amd import _capi as capi
from tests._util import assert_close, assert_equal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _close_results(ours, ref, rtol, what, exact=()):
    from tests.test_reference_pin import _assert_results_close

    _assert_results_close(ours, ref, rtol, what, exact)


# --------------------------------------------------------------------------------------
# the reference's internal VALU ops (_ppminkowski, _wminkowski, _canberra, _braycurtis,
# _additive_chi2_kernel, _sqjensenshannon, _haversine, _snr, _sqmahalanobis) in float64
# --------------------------------------------------------------------------------------
def _family_f64_check(ref_fn, tmp_path=None):
    from oracle import ref_runner
    from tests._family_cases import family_cases

    cs = family_cases(torch.float64)
    refs = ref_fn(cs) if ref_fn else [None] * len(cs)
    ops = torch.ops.torchpairwise
    for (case, tensors), r in zip(cs, refs):
        what = f"{case['op']} {case['kind']} {[tuple(t.shape) for t in tensors.values()]}"
        print(what, flush=True)
        ours = ref_runner.run_op_case(ops, case, tensors, DEV)
        want = r if r is not None else ref_runner.run_op_case(ops, case, tensors, "cpu")
        inf = case["kind"] in ("p=inf", "p=-inf")
        rt = 1e-10 if case["op"] == "_snr" else 1e-12  # snr: GPU composite of centred rows
        _close_results({k: v for k, v in ours.items() if not k.startswith("grad")},
                       {k: v for k, v in want.items() if not k.startswith("grad")}, rt, what)
        _close_results({k: v for k, v in ours.items() if k.startswith("grad") or k == "err"},
                       {k: v for k, v in want.items() if k.startswith("grad") or k == "err"}, 10 * rt, what,
                       ("grad_a", "grad_b") if inf else ())


def test_family_f64_gpu_equal_cpu_loops():
    _family_f64_check(None)


def test_family_f64_gpu_equal_reference(tmp_path):
    from oracle import ref_runner

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    _family_f64_check(lambda cs: ref_runner.run_op_reference(cs, tmp_path))


@pytest.mark.parametrize("metric,p", [(capi.FAM_PPMINKOWSKI, 2.0), (capi.FAM_PPMINKOWSKI, 0.7),
                                      (capi.FAM_WMINKOWSKI, 3.0), (capi.FAM_WMINKOWSKI, float("inf")),
                                      (capi.FAM_CANBERRA, 0.0), (capi.FAM_BRAYCURTIS, 0.0),
                                      (capi.FAM_CHI2, 0.0), (capi.FAM_JS, 2.0)])
def test_family_f64_capi_tiles(metric, p):
    """The C ABI on shapes that leave partial 32 x 32 output tiles and a partial 32-feature
    chunk (d = 70), batched, against this build's CPU op in float64.  (n = d: the reference's
    shape check of a batched w compares x1.size(1) with w.size(1).)"""
    B, n, m, d = 2, 70, 77, 70
    g = _g(3)
    pos = metric in (capi.FAM_CHI2, capi.FAM_JS)
    x1 = torch.rand(B, n, d, generator=g, dtype=torch.float64) + (0.05 if pos else -0.5)
    x2 = torch.rand(B, m, d, generator=g, dtype=torch.float64) + (0.05 if pos else -0.5)
    w = torch.rand(B, d, generator=g, dtype=torch.float64) + 0.25
    gr = torch.randn(B, n, m, generator=g, dtype=torch.float64)
    ops = torch.ops.torchpairwise
    if metric == capi.FAM_PPMINKOWSKI:
        want = ops._ppminkowski(x1, x2, p)
        wg = ops.__ppminkowski_backward(gr, x1, x2, p)
    elif metric == capi.FAM_WMINKOWSKI:
        want = ops._wminkowski(x1, x2, w, p)
        wg = ops.__wminkowski_backward(gr, x1, x2, w, p)
    elif metric == capi.FAM_CANBERRA:
        want, wg = ops._canberra(x1, x2), ops.__canberra_backward(gr, x1, x2)
    elif metric == capi.FAM_BRAYCURTIS:
        want, wg = ops._braycurtis(x1, x2), ops.__braycurtis_backward(gr, x1, x2)
    elif metric == capi.FAM_CHI2:
        want, wg = ops._additive_chi2_kernel(x1, x2), ops.__additive_chi2_kernel_backward(gr, x1, x2)
    else:
        want, wg = ops._sqjensenshannon(x1, x2, 2.0), ops.__sqjensenshannon_backward(gr, x1, x2, 2.0)
    divisor = 2.0 * torch.log(torch.tensor(2.0, dtype=torch.float64)).item() if metric == capi.FAM_JS else p
    wd = w.to(DEV) if metric == capi.FAM_WMINKOWSKI else None
    got = capi.family_f64(metric, x1.to(DEV), x2.to(DEV), wd, divisor)
    assert_close(got, want, rtol=1e-12, atol=1e-12 * float(want.abs().max()), what="forward")
    grads = capi.family_f64_backward(metric, gr.to(DEV), x1.to(DEV), x2.to(DEV), wd, divisor)
    for k, (a, b) in enumerate(zip(grads, wg)):
        assert_close(a, b, rtol=1e-11, atol=1e-11 * float(b.abs().max()), what=f"grad {k}")


@pytest.mark.parametrize("name,extra", [
    ("sqeuclidean_distances", ()), ("canberra_distances", ()), ("braycurtis_distances", ()),
    ("wminkowski_distances", (3.0, "w")), ("seuclidean_distances", ("w",)), ("rbf_kernel", ()),
    ("additive_chi2_kernel", ()), ("chi2_kernel", ()), ("jensenshannon_distances", ()),
    ("haversine_distances", ()), ("snr_distances", ()), ("laplacian_kernel", ())])
def test_float64_public_ops_gpu(name, extra):
    """The public ops the reference serves in double on CUDA: GPU float64 forward and autograd
    backward against the same op on CPU float64 tensors (the reference's route)."""
    print(name, flush=True)
    d = 2 if name == "haversine_distances" else 6
    g = _g(5)
    x1 = torch.rand(37, d, generator=g, dtype=torch.float64) + 0.1
    x2 = torch.rand(29, d, generator=g, dtype=torch.float64) + 0.1
    w = torch.rand(d, generator=g, dtype=torch.float64) + 0.2
    gr = torch.randn(37, 29, generator=g, dtype=torch.float64)
    fn = getattr(tp, name)
    a, b = x1.to(DEV).requires_grad_(), x2.to(DEV).requires_grad_()
    out = fn(a, b, *[w.to(DEV) if e == "w" else e for e in extra])
    assert out.dtype == torch.float64 and out.is_cuda
    out.backward(gr.to(DEV))
    ra, rb = x1.clone().requires_grad_(), x2.clone().requires_grad_()
    ref = fn(ra, rb, *[w if e == "w" else e for e in extra])
    ref.backward(gr)
    rt = 1e-10 if name == "snr_distances" else 1e-12
    out, ref = out.detach(), ref.detach()
    assert_close(out, ref, rtol=rt, atol=rt * float(ref.abs().max()), what=name)
    assert_close(a.grad, ra.grad, rtol=10 * rt, atol=10 * rt * float(ra.grad.abs().max()), what="grad x1")
    assert_close(b.grad, rb.grad, rtol=10 * rt, atol=10 * rt * float(rb.grad.abs().max()), what="grad x2")


# --------------------------------------------------------------------------------------
# directed Hausdorff in float64 / float16 (the reference's loop in its own order)
# --------------------------------------------------------------------------------------
def _clouds(kind, dtype, seed):
    g = _g(seed)
    if kind == "ties":  # integer grid points: many equal distances, first / last index rules
        c1 = torch.randint(0, 3, (2, 2, 90, 3), generator=g).to(dtype)
        c2 = torch.randint(0, 3, (2, 3, 70, 3), generator=g).to(dtype)
    elif kind == "overflow":  # float16: squared sums past 65504 become inf (stale indices kept)
        c1 = (torch.rand(1, 2, 60, 3, generator=g, dtype=torch.float64) * 400).to(dtype)
        c2 = (torch.rand(1, 3, 50, 3, generator=g, dtype=torch.float64) * 400 - 200).to(dtype)
    else:
        c1 = torch.rand(2, 3, 300, 3, generator=g, dtype=torch.float64).to(dtype)
        c2 = (torch.rand(2, 2, 250, 3, generator=g, dtype=torch.float64) + 0.05).to(dtype)
    return c1, c2


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16])
@pytest.mark.parametrize("kind", ["random", "ties", "overflow"])
def test_hausdorff_exact_dtypes_equal_cpu_op(dtype, kind):
    """GPU op (forward and autograd backward) against this build's CPU op in the same dtype,
    bit for bit: value, both indices, both gradients."""
    if kind == "overflow" and dtype == torch.float64:
        pytest.skip("no overflow in float64 at these magnitudes")
    print(f"{dtype} {kind}", flush=True)
    c1, c2 = _clouds(kind, dtype, 21)
    gr = torch.randn(c1.shape[0], c1.shape[1], c2.shape[1], generator=_g(22), dtype=torch.float64).to(dtype)
    a, b = c1.to(DEV).requires_grad_(), c2.to(DEV).requires_grad_()
    out = tp.directed_hausdorff_distances(a, b)
    ra, rb = c1.clone().requires_grad_(), c2.clone().requires_grad_()
    ref = tp.directed_hausdorff_distances(ra, rb)
    for got, want, nm in zip(out, ref, ("value", "idx1", "idx2")):
        assert got.dtype == want.dtype
        assert_equal(got, want, f"{nm}")
    if kind == "overflow":
        return  # inf distances: the gradient is 0 * inf terms, as on the CPU (NaN payloads vary)
    out[0].backward(gr.to(DEV))
    ref[0].backward(gr)
    assert_equal(a.grad, ra.grad, "grad x1")
    assert_equal(b.grad, rb.grad, "grad x2")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16])
def test_hausdorff_exact_dtypes_equal_reference(tmp_path, dtype):
    """The same against the reference's compiled CPU kernel (oracle/_ref), forward with and
    without a shuffle (the permutations drawn on the CPU as the reference draws them and handed
    to the C ABI), and the backward."""
    from oracle import ref_runner

    if not ref_runner.available():
        pytest.skip("oracle/_ref not built")
    for kind in ("random", "ties"):
        c1, c2 = _clouds(kind, dtype, 31)
        ref = ref_runner.run("hausdorff", {"x1": c1.numpy(), "x2": c2.numpy()}, tmp_path)
        got = capi.directed_hausdorff_exact(c1.to(DEV), c2.to(DEV))
        for t, key in zip(got, ("out", "idx1", "idx2")):
            assert_equal(t, torch.from_numpy(ref[key]), f"{kind} {key}")
        ref = ref_runner.run("hausdorff", {"x1": c1.numpy(), "x2": c2.numpy(), "seed": 9}, tmp_path)
        p1, p2 = P.hausdorff_permutations(c1.shape[0], c1.shape[2], c2.shape[2], _g(9))
        got = capi.directed_hausdorff_exact(c1.to(DEV), c2.to(DEV), p1.to(DEV), p2.to(DEV))
        for t, key in zip(got, ("out", "idx1", "idx2")):
            assert_equal(t, torch.from_numpy(ref[key]), f"{kind} shuffled {key}")
    c1, c2 = _clouds("random", dtype, 32)
    gr = torch.randn(c1.shape[:2] + (c2.shape[1],), generator=_g(33), dtype=torch.float64).to(dtype)
    ref = ref_runner.run("hausdorff_backward", {"x1": c1.numpy(), "x2": c2.numpy(), "grad": gr.numpy()}, tmp_path)
    a, b = c1.to(DEV).requires_grad_(), c2.to(DEV).requires_grad_()
    tp.directed_hausdorff_distances(a, b)[0].backward(gr.to(DEV))
    assert_equal(a.grad, torch.from_numpy(ref["grad_x1"]), "grad x1")
    assert_equal(b.grad, torch.from_numpy(ref["grad_x2"]), "grad x2")


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.float16])
def test_hausdorff_exact_shuffle_equals_cpu_op(dtype):
    """Shuffled order: the C ABI with the permutations the CPU op draws from the same seeded
    generator, against the CPU op, bit for bit."""
    c1, c2 = _clouds("ties", dtype, 41)
    ref = tp.directed_hausdorff_distances(c1, c2, shuffle=True, generator=_g(5))
    p1, p2 = P.hausdorff_permutations(c1.shape[0], c1.shape[2], c2.shape[2], _g(5))
    got = capi.directed_hausdorff_exact(c1.to(DEV), c2.to(DEV), p1.to(DEV), p2.to(DEV))
    for t, want, nm in zip(got, ref, ("value", "idx1", "idx2")):
        assert_equal(t, want, f"shuffled {nm}")


@pytest.mark.parametrize("shape,kind", [(((2, 3, 2000, 3), (2, 2, 1500, 3)), "random"),
                                        (((1, 2, 700, 2), (1, 3, 650, 2)), "ties"),
                                        (((1, 4, 1000, 5), (1, 3, 1200, 5)), "random")])
def test_hausdorff_exact_f32_equals_pruned_pipeline(shape, kind):
    """Two independent GPU implementations of the same loop: the exact-order wave kernel in
    float32 and the pruned cell-grid pipeline (the float32 op) agree bit for bit."""
    g = _g(51)
    s1, s2 = shape
    if kind == "ties":
        c1 = torch.randint(0, 4, s1, generator=g).float()
        c2 = torch.randint(0, 4, s2, generator=g).float()
    else:
        c1, c2 = torch.rand(s1, generator=g), torch.rand(s2, generator=g) + 0.02
    want = tp.directed_hausdorff_distances(c1.to(DEV), c2.to(DEV))
    got = capi.directed_hausdorff_exact(c1.to(DEV), c2.to(DEV))
    for t, w_, nm in zip(got, want, ("value", "idx1", "idx2")):
        assert_equal(t, w_, nm)
    gr = torch.randn(want[0].shape, generator=g).to(DEV)
    w1, w2 = capi.directed_hausdorff_backward(gr, c1.to(DEV), c2.to(DEV), *want)
    e1, e2 = capi.directed_hausdorff_exact_backward(gr, c1.to(DEV), c2.to(DEV), *got)
    assert_equal(e1, w1, "grad x1")
    assert_equal(e2, w2, "grad x2")


def test_hausdorff_bfloat16_refused_as_reference():
    """The reference's dispatch (floating types and half) has no bfloat16: same refusal."""
    c = torch.rand(1, 20, 3).to(DEV, torch.bfloat16)
    with pytest.raises(NotImplementedError, match="not implemented for 'BFloat16'"):
        tp.directed_hausdorff_distances(c, c)
