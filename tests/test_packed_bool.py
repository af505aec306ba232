"""The persistent packed-bool format and the one-pass boolean count metrics.

CPU: _pack_bool against numpy packbits (the oracle's restatement of the layout), the packed
metrics against the public boolean metrics (the reference's composites) bit-exact, the oracle
restatement of those composites against scipy and against the composites themselves.
GPU: the C ABI and the ops against the reference's composites evaluated on the GPU (the pw*_sum
ops and ATen's elementwise GPU kernels, as the reference runs them) bit-exact.
"""
import warnings

import numpy as np
import pytest
import torch
from scipy.spatial.distance import cdist as scipy_cdist

import torchpairwise_amd as tp
from oracle import pairwise as P
from tests._util import assert_equal, rand
from torchpairwise_amd import _capi as capi

DEV = "cuda"
COUNT = P.BOOL_COUNT_METRICS
PW = ("pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean", "pwne_mean")
DS = (1, 31, 32, 33, 100, 129, 1024)


def _rows(B, n, m, d, seed):
    a = (rand(B, n, d, seed=seed) < 0.5)
    b = (rand(B, m, d, seed=seed + 1) < 0.3)
    a[:, 0] = False  # all-zero rows: 0 / 0 in dice, kulczynski1, sokalsneath, ...
    b[:, 1] = False
    a[:, 2] = True   # all-one row
    if m > 3:
        b[:, 3] = a[:, 3 % n]  # an identical pair
    return a, b


def _public(metric, a, b):
    name = metric if metric.startswith("pw") else f"{metric}_distances"
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        return getattr(tp, name)(a, b)


# ----------------------------------------------------------------------------- CPU
@pytest.mark.parametrize("d", DS)
def test_pack_bool_layout_and_popcounts(d):
    a, _ = _rows(2, 9, 4, d, seed=d)
    words, pops = torch.ops.torchpairwise._pack_bool(a)
    want_w, want_p = P.pack_bool_words(a.numpy())
    assert words.dtype == torch.int32 and words.shape == (2, 9, capi.lib().tpw_packed_words(d))
    assert np.array_equal(words.numpy().view(np.uint32), want_w)
    assert np.array_equal(pops.numpy(), want_p)
    p = tp.PackedBool.pack(a[0])
    assert p.shape == (9, d) and torch.equal(p.unpack(), a[0])


@pytest.mark.parametrize("d", DS)
def test_packed_metrics_cpu_equal_public_ops(d):
    a, b = _rows(2, 9, 11, d, seed=10 + d)
    pa, pb = tp.PackedBool.pack(a), tp.PackedBool.pack(b)
    for metric in COUNT + PW:
        assert_equal(tp.packed.cdist(pa, pb, metric), _public(metric, a, b), f"{metric} d={d}")
    assert_equal(tp.packed.dice_distances(pa), _public("dice", a, a), "x2 = None")
    assert_equal(tp.packed.pwxor_sum(pa, pb), tp.pwxor_sum(a, b), "bound name")


def test_oracle_count_metrics_match_scipy_and_the_composites():
    a, b = _rows(1, 30, 40, 100, seed=3)
    a, b = a[0].numpy(), b[0].numpy()
    a[0], b[1] = True, True  # scipy's dice / kulczynski1 / sokalsneath need nonzero denominators
    names = {"kulczynski1": None, "kulsinski": None}  # no scipy counterpart in this scipy
    for metric in COUNT:
        got = P.bool_count_metric(a, b, metric)
        assert_equal(got, _public(metric, torch.from_numpy(a), torch.from_numpy(b)), metric)
        if metric in names:
            continue
        with warnings.catch_warnings(), np.errstate(divide="ignore", invalid="ignore"):
            warnings.simplefilter("ignore")
            want = scipy_cdist(a, b, metric)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7, err_msg=metric)
    # kulczynski1 (a similarity in the reference: and / xor) and kulsinski from their counts
    n11 = P.bool_counts(a, b, "and")
    x = P.bool_counts(a, b, "xor")
    with np.errstate(divide="ignore", invalid="ignore"):
        np.testing.assert_allclose(P.bool_count_metric(a, b, "kulczynski1"), n11 / x, rtol=1e-6)
    np.testing.assert_allclose(P.bool_count_metric(a, b, "kulsinski"), (x - n11 + 100) / (x + 100),
                               rtol=1e-6)


def test_pins_catch_or_for_xor_and_a_true_divide_on_the_gpu_route():
    a, b = _rows(1, 50, 60, 100, seed=5)
    a, b = a[0].numpy(), b[0].numpy()
    pub = _public("dice", torch.from_numpy(a), torch.from_numpy(b)).numpy()
    OR = P.float_accumulated(P.bool_counts(a, b, "or"))
    AND = P.float_accumulated(P.bool_counts(a, b, "and"))
    with np.errstate(divide="ignore", invalid="ignore"):
        wrong = (OR / (np.float32(2) * AND + OR)).astype(np.float32)
    assert not np.allclose(wrong, pub, equal_nan=True)
    cpu = P.bool_count_metric(a, b, "russellrao")
    gpu = P.bool_count_metric(a, b, "russellrao", gpu_scalar_divide=True)
    assert not np.array_equal(cpu, gpu)  # d = 100: the reciprocal multiply differs somewhere
    np.testing.assert_allclose(gpu, cpu, rtol=1.2e-7, atol=0)


def test_packed_errors():
    a = tp.PackedBool.pack(torch.ones(3, 40, dtype=torch.bool))
    b = tp.PackedBool.pack(torch.ones(3, 41, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="feature dimension"):
        tp.packed.hamming_distances(a, b)
    with pytest.raises(RuntimeError, match="unknown metric"):
        tp.packed.cdist(a, a, "euclidean")
    with pytest.raises(TypeError):
        tp.packed.hamming_distances(torch.ones(3, 40, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="expected a bool tensor"):
        torch.ops.torchpairwise._pack_bool(torch.ones(3, 4))
    with pytest.raises(RuntimeError, match="words per row expected"):
        torch.ops.torchpairwise._packed_bool_metric(a.words, a.popcounts, a.words, a.popcounts, 200, "dice")
    assert tp.PackedBool.pack(torch.ones(3, 5)).unpack().all()  # non-bool rows are coerced


# ----------------------------------------------------------------------------- GPU
def _gpu_composite(metric, a, b):
    """The reference's composite for `metric`, evaluated on the GPU with its own ops
    (pairwise_metrics.cpp:206-243,339-399): the pw*_sum GPU ops and ATen's GPU elementwise
    kernels, as the reference runs it."""
    ops = torch.ops.torchpairwise
    D = a.shape[-1]
    if metric == "hamming":
        return ops.pwne_mean(a, b)
    if metric == "jaccard":
        return ops.prf_div(ops.pwxor_sum(a, b), ops.pwor_sum(a, b), "zero")
    if metric == "kulsinski":
        S = ops.pwxor_sum(a, b)
        return (S - ops.pwand_sum(a, b) + D) / (S + D)
    if metric == "kulczynski1":
        return ops.pwand_sum(a, b) / ops.pwxor_sum(a, b)
    if metric == "yule":
        hR = ops.pwand_sum(a, ~b) * ops.pwand_sum(~a, b)
        return ops.prf_div(2 * hR, ops.pwand_sum(a, b) * ops.pwand_sum(~a, ~b) + hR, "zero")
    if metric == "dice":
        R = ops.pwxor_sum(a, b)
        return R / (2 * ops.pwand_sum(a, b) + R)
    if metric in ("rogerstanimoto", "sokalmichener"):
        R = 2 * ops.pwxor_sum(a, b)
        return R / (ops.pweq_sum(a, b) + R)
    if metric == "russellrao":
        return (D - ops.pwand_sum(a, b)) / D
    R = 2 * ops.pwxor_sum(a, b)  # sokalsneath
    return R / (ops.pwand_sum(a, b) + R)


@pytest.mark.gpu
@pytest.mark.parametrize("d", DS)
@pytest.mark.parametrize("B,n,m", [(1, 130, 257), (2, 64, 33)])
def test_bool_count_metric_capi_equals_gpu_composites(B, n, m, d):
    print(f"bool count metrics {B}x{n}x{m} d={d}", flush=True)
    a, b = _rows(B, n, m, d, seed=20 + d)
    a, b = a.to(DEV), b.to(DEV)
    wa, pa = torch.ops.torchpairwise._pack_bool(a)
    wb, pb = torch.ops.torchpairwise._pack_bool(b)
    for code, metric in enumerate(COUNT):
        out = torch.empty(B, n, m, device=DEV)
        capi.call("tpw_bool_count_metric", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb),
                  B, n, m, d, code, capi._ptr(out), capi._stream())
        assert_equal(out, _gpu_composite(metric, a, b), f"{metric} d={d}", nan_payload=False)


@pytest.mark.gpu
@pytest.mark.parametrize("d", DS)
def test_packed_ops_gpu(d):
    print(f"packed ops d={d}", flush=True)
    a, b = _rows(2, 70, 45, d, seed=40 + d)
    wa, pa = torch.ops.torchpairwise._pack_bool(a.to(DEV))
    wc, pc = torch.ops.torchpairwise._pack_bool(a)
    assert_equal(wa, wc, "words")
    assert_equal(pa, pc, "popcounts")
    ga, gb = tp.PackedBool.pack(a.to(DEV)), tp.PackedBool.pack(b.to(DEV))
    ca, cb = tp.PackedBool.pack(a), tp.PackedBool.pack(b)
    for metric in COUNT + PW:
        got = tp.packed.cdist(ga, gb, metric)
        assert_equal(got, _gpu_composite(metric, a.to(DEV), b.to(DEV)) if metric in COUNT
                     else _public(metric, a.to(DEV), b.to(DEV)), f"{metric} d={d}", nan_payload=False)
        if metric != "russellrao":  # the reference's own CPU and GPU routes differ by 1 ulp there
            assert_equal(got, tp.packed.cdist(ca, cb, metric), f"{metric} gpu = cpu", nan_payload=False)


@pytest.mark.gpu
@pytest.mark.parametrize("metric", COUNT[2:])
def test_public_boolean_metrics_take_the_fused_path(metric):
    a, b = _rows(1, 300, 200, 77, seed=60)
    a, b = a[0].to(DEV), b[0].to(DEV)
    assert_equal(_public(metric, a, b), _gpu_composite(metric, a, b), metric, nan_payload=False)
    assert_equal(_public(metric, a, None), _gpu_composite(metric, a, a), f"{metric} self", nan_payload=False)


# ------------------------------------------------------------- GPU: bool bytes on the int8 MFMA
BYTES_DS = (1, 31, 100, 128, 1024, 4096 + 17)


@pytest.mark.gpu
@pytest.mark.parametrize("d", BYTES_DS)
@pytest.mark.parametrize("B,n,m", [(1, 130, 257), (2, 64, 33), (1, 256, 384)])
def test_bool_bytes_entry_points_equal_packed_and_oracle(B, n, m, d):
    """The int8-MFMA byte path against the packed popcount path (bit for bit) and the
    oracle's float32 composites over exact counts, for every count metric and reduction."""
    print(f"bool bytes {B}x{n}x{m} d={d}", flush=True)
    a, b = _rows(B, n, m, d, seed=80 + d)
    ga, gb = a.to(DEV), b.to(DEV)
    wa, pa = torch.ops.torchpairwise._pack_bool(ga)
    wb, pb = torch.ops.torchpairwise._pack_bool(gb)
    ca, cb = capi.bool_row_counts(ga), capi.bool_row_counts(gb)
    assert_equal(ca.cpu(), a.reshape(-1, d).sum(-1).to(torch.int32), "row counts")
    assert_equal(ca, pa.reshape(-1), "row counts = packed popcounts")
    for code, metric in enumerate(COUNT):
        got = capi.bool_bytes_count_metric(ga, gb, code)
        packed = torch.empty(B, n, m, device=DEV)
        capi.call("tpw_bool_count_metric", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb),
                  B, n, m, d, code, capi._ptr(packed), capi._stream())
        assert_equal(got, packed, f"{metric} bytes = packed d={d}", nan_payload=False)
        want = np.stack([P.bool_count_metric(a[i].numpy(), b[i].numpy(), metric, gpu_scalar_divide=True)
                         for i in range(B)])
        assert_equal(got.cpu(), torch.from_numpy(want), f"{metric} bytes = oracle d={d}", nan_payload=False)
    for op, opname in ((capi.BIT_AND, "and"), (capi.BIT_OR, "or"), (capi.BIT_XOR, "xor"),
                       (capi.BIT_EQ, "eq"), (capi.BIT_NE, "ne")):
        for red, rname in ((capi.RED_SUM, "sum"), (capi.RED_MEAN, "mean")):
            got = capi.bool_bytes_reduce(ga, gb, op, red)
            want = np.stack([P.pw_reduce_bool(a[i].numpy(), b[i].numpy(), opname, rname) for i in range(B)])
            assert_equal(got.cpu(), torch.from_numpy(want), f"pw{opname}_{rname} bytes d={d}")


def _fp4_rows(x, rb):
    """numpy: bool [rows, d] -> fp4 e2m1 nibbles (1.0 = 0x2), feature 2j in the low nibble of byte j."""
    rows, d = x.shape
    f = np.zeros((rows, 2 * rb), np.uint8)
    f[:, :d] = x.astype(np.uint8) * 2
    return (f[:, 0::2] | (f[:, 1::2] << 4)).astype(np.uint8)


@pytest.mark.gpu
@pytest.mark.parametrize("d", BYTES_DS + (255, 256, 257, 512))
@pytest.mark.parametrize("B,n,m", [(1, 130, 257), (2, 64, 33)])
def test_bool_fp4_entry_points_equal_bytes(B, n, m, d):
    """The fp4 layout (pack pass, scaled fp4 MFMA) against the int8 byte path, bit for bit, for
    every count metric and reduction; the packed rows against a numpy restatement."""
    print(f"bool fp4 {B}x{n}x{m} d={d}", flush=True)
    a, b = _rows(B, n, m, d, seed=90 + d)
    ga, gb = a.to(DEV), b.to(DEV)
    rb = capi.lib().tpw_bool_fp4_row_bytes(d)
    assert rb == -(-d // 256) * 128
    fa, ca = capi.pack_bool_fp4(ga)
    assert_equal(fa.cpu().reshape(-1, rb), torch.from_numpy(_fp4_rows(a.reshape(-1, d).numpy(), rb)), "fp4 rows")
    assert_equal(ca.cpu(), a.reshape(-1, d).sum(-1).to(torch.int32), "fp4 row counts")
    for code, metric in enumerate(COUNT):
        assert_equal(capi.bool_fp4_count_metric(ga, gb, code), capi.bool_bytes_count_metric(ga, gb, code),
                     f"{metric} fp4 = bytes d={d}", nan_payload=False)
    for op in (capi.BIT_AND, capi.BIT_OR, capi.BIT_XOR, capi.BIT_EQ, capi.BIT_NE):
        for red in (capi.RED_SUM, capi.RED_MEAN):
            assert_equal(capi.bool_fp4_reduce(ga, gb, op, red), capi.bool_bytes_reduce(ga, gb, op, red),
                         f"op {op} red {red} fp4 = bytes d={d}")


@pytest.mark.gpu
def test_bool_fp4_errors():
    l = capi.lib()
    assert l.tpw_bool_fp4_row_bytes(0) == 0 and l.tpw_bool_fp4_row_bytes(1) == 128
    assert l.tpw_bool_fp4_count_metric(None, None, None, None, 1, 4, 4, 8, 99, None, None) != 0
    assert b"unknown metric" in l.tpw_last_error()
    assert l.tpw_pack_bool_fp4(None, 4, 1 << 24, None, None, None) != 0
    assert b"2^24" in l.tpw_last_error()
    assert l.tpw_bool_fp4_reduce(None, None, None, None, 1, 1 << 22, 4, 1024, 0, 0, None, None) != 0
    assert b"2^31" in l.tpw_last_error()


@pytest.mark.gpu
def test_bool_bytes_empty_and_errors():
    x = torch.zeros((0, 16), dtype=torch.bool, device=DEV)
    y = torch.zeros((5, 16), dtype=torch.bool, device=DEV)
    assert capi.bool_bytes_count_metric(x, y, 0).shape == (0, 5)
    assert capi.bool_row_counts(x).shape == (0,)
    l = capi.lib()
    assert l.tpw_bool_bytes_count_metric(None, None, None, None, 1, 4, 4, 8, 99, None, None) != 0
    assert b"unknown metric" in l.tpw_last_error()
    assert l.tpw_bool_bytes_reduce(None, None, None, None, 1, 4, 4, 0, 0, 0, None, None) != 0


@pytest.mark.gpu
@pytest.mark.parametrize("d", (100, 256, 257, 300, 1024))
def test_public_bool_ops_on_both_routes(d):
    """Public bool ops around the route threshold (packed up to 256 features for the pw
    reductions, int8 matrix cores above; count metrics always on the matrix cores) against the
    oracle bit for bit, with x2 and with x2 = None."""
    print(f"public bool ops d={d}", flush=True)
    a, b = _rows(1, 150, 131, d, seed=90 + d)
    a, b = a[0], b[0]
    ga, gb = a.to(DEV), b.to(DEV)
    for name in PW:
        op, red = name[2:].split("_")
        got = _public(name, ga, gb)
        assert_equal(got.cpu(), torch.from_numpy(P.pw_reduce_bool(a.numpy(), b.numpy(), op, red)),
                     f"{name} d={d}")
    for metric in COUNT:
        want = P.bool_count_metric(a.numpy(), b.numpy(), metric, gpu_scalar_divide=True)
        assert_equal(_public(metric, ga, gb).cpu(), torch.from_numpy(want), f"{metric} d={d}",
                     nan_payload=False)
        want_self = P.bool_count_metric(a.numpy(), a.numpy(), metric, gpu_scalar_divide=True)
        assert_equal(_public(metric, ga, None).cpu(), torch.from_numpy(want_self),
                     f"{metric} self d={d}", nan_payload=False)


# ------------------------------------------------ GPU: the short divide of the tile kernels
@pytest.mark.gpu
@pytest.mark.parametrize("o_lo,o_hi,step,count", [
    (1, 4096, 1, 8193),                    # every x in [0, 8192] over every o up to 4096
    ((1 << 21) - (1 << 16) + 1, 1 << 21, 1, 4096),  # the largest denominators, x < 4096
    (1, 1 << 21, 4093, 1024),              # every o up to 2^21, x strided over [0, 2^22]
])
def test_count_division_equals_ieee_divide(o_lo, o_hi, step, count):
    """The reciprocal + Newton + residual quotient of the bit / fp4 tile kernels (rows of at
    most 2^20 features) against __fdiv_rn bit for bit: the sequence's error bound proves it for
    numerators in [0, 2^22] and denominators in [1, 2^21] given a reciprocal within one ulp;
    this checks that premise and the result on the hardware."""
    print(f"count division o=[{o_lo},{o_hi}] step={step} count={count}", flush=True)
    assert capi.count_division_check(o_lo, o_hi, step, count) == 0


def test_count_division_check_refuses_outside_its_domain():
    l = capi.lib()
    assert l.tpw_count_division_check(0, 4, 1, 1, None, None) != 0
    assert b"[1, 2^21]" in l.tpw_last_error()
    assert l.tpw_count_division_check(1, (1 << 21) + 1, 1, 1, None, None) != 0
    assert l.tpw_count_division_check(1, 4, 1 << 12, 1 << 12, None, None) != 0
    assert b"[0, 2^22]" in l.tpw_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("d", ((1 << 20) - 31, 1 << 20, (1 << 20) + 33))
def test_tile_kernels_across_the_short_divide_limit(d):
    """Rows of up to 2^20 features finish in float with the short divide, longer rows on
    integer counts with the IEEE divide: both sides of the limit, on the bit and fp4 tile
    kernels, against the int8 byte path (integer epilogue) and the oracle, bit for bit, for
    every count metric and reduction."""
    print(f"tile kernels at d={d}", flush=True)
    B, n, m = 1, 40, 36
    a, b = _rows(B, n, m, d, seed=7 + d % 97)
    a[:, 1] = True                     # a full row
    b[:, 2] = a[:, 3]                  # an identical pair
    ga, gb = a.to(DEV), b.to(DEV)
    wa, pa = torch.ops.torchpairwise._pack_bool(ga)
    wb, pb = torch.ops.torchpairwise._pack_bool(gb)
    for code, metric in enumerate(COUNT):
        packed = torch.empty(B, n, m, device=DEV)
        assert capi.call("tpw_bool_count_metric", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb),
                         B, n, m, d, code, capi._ptr(packed), capi._stream()) == 0
        bytes_ = capi.bool_bytes_count_metric(ga, gb, code)
        assert_equal(packed, bytes_, f"{metric} packed = bytes d={d}", nan_payload=False)
        assert_equal(capi.bool_fp4_count_metric(ga, gb, code), bytes_, f"{metric} fp4 = bytes d={d}",
                     nan_payload=False)
        want = P.bool_count_metric(a[0].numpy(), b[0].numpy(), metric, gpu_scalar_divide=True)
        assert_equal(packed[0].cpu(), torch.from_numpy(want), f"{metric} = oracle d={d}", nan_payload=False)
    jac = torch.empty(B, n, m, device=DEV)
    assert capi.call("tpw_jaccard_bool", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa), capi._ptr(pb), B, n, m, d,
                     capi._ptr(jac), capi._stream()) == 0
    assert_equal(jac[0].cpu(), torch.from_numpy(P.jaccard_distances(a[0].numpy(), b[0].numpy())), f"jaccard d={d}")
    for op, opname in ((capi.BIT_AND, "and"), (capi.BIT_OR, "or"), (capi.BIT_XOR, "xor"),
                       (capi.BIT_EQ, "eq"), (capi.BIT_NE, "ne")):
        for red, rname in ((capi.RED_SUM, "sum"), (capi.RED_MEAN, "mean")):
            got = torch.empty(B, n, m, device=DEV)
            assert capi.call("tpw_bool_pairwise_reduce_counted", capi._ptr(wa), capi._ptr(wb), capi._ptr(pa),
                             capi._ptr(pb), B, n, m, d, op, red, capi._ptr(got), capi._stream()) == 0
            want = torch.from_numpy(P.pw_reduce_bool(a[0].numpy(), b[0].numpy(), opname, rname))
            assert_equal(got[0].cpu(), want, f"pw{opname}_{rname} packed d={d}")
            assert_equal(capi.bool_fp4_reduce(ga, gb, op, red)[0].cpu(), want, f"pw{opname}_{rname} fp4 d={d}")
