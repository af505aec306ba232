#!/usr/bin/env python3
"""Benchmark of the torchpairwise hot path on one MI355X.

Workload (BASELINE.json metric): x1, x2 = [16384, 128] fp32 (torch.randn from CPU generators
seeded 0 and 1, moved to HBM before timing).  One step = one call of the drop-in op
(torchpairwise_amd.<metric>, i.e. torch.ops.torchpairwise.<metric>) over that batch; the
headline is euclidean_distances (the MFMA kernel), with manhattan_distances (VALU) and
hamming_distances on bool inputs (rand < 0.5; the op packs the bits inside every call) timed
the same way and reported under "extra".

value = pair-features/s (N*M*D per call / mean call time over the timed steps), inputs
resident in HBM.  Timing: a clock-settle phase (the headline op called for --settle-ms of
wall time, reported as settle_ms; the GPU leaves its idle clocks only after some tens of
milliseconds of load), then W untimed warm-up steps, then K steps between two
torch.cuda.synchronize() calls, one event pair around them; per-kernel durations come from HIP
events stamped by the kernels' own dispatches on the stream they are launched on (torch's
current stream, which the C ABI receives).

roofline (dominant kernel = the MFMA pairwise kernel of euclidean):
  algorithmic flops per launch = 2*N*M*D (one multiply-add per pair-feature), peak = MI355X
  dense FP32 MFMA 157.3 TFLOP/s; the launch duration is the mean device time of the
  tile-kernel launch inside each of the K timed steps themselves: the C ABI's launch timer
  (tpw_launch_timer_arm / _read) hands the launch a start / stop event pair that its own
  dispatch stamps (hipExtLaunchKernelGGL), so kernel_ms <= ms_per_step holds by construction
  and is asserted.  The extras (manhattan,
  hamming) report their dominant kernels the same way.  Defaults W = K = 200.
cpu_baseline: the reference's CPU path for euclidean_distances is at::cdist(p=2) -> on the
  host cores via torch.cdist, timed on a bounded row sample of the same workload; beside it
  manhattan (at::cdist p = 1), and the reference's own compiled CPU kernels (oracle/_ref, in a
  child process: its OpenMP loops with their compiled-in 32 threads) for hamming, jaccard and
  directed Hausdorff on samples of M, C4 and C5, plus the oracle's C restatement of the
  hamming loop on all the cores this process may use.

`python bench.py --gpus N` with N > 1 exits: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_FP32_MFMA = 157.3e12
PEAK_BF16_MFMA = 2.5e15
PEAK_HBM = 8.0e12
# FP32 vector peak 157.3 TFLOP/s = 256 CU x 4 SIMD x 32 lanes x 2 (FMA) x 2.4 GHz.  As an
# issue rate of non-packed VALU instructions that is 7.86e13 lane-ops/s only with dual issue
# (two VALU instructions of a wave pair per clock): the dual-issue rate
PEAK_VALU_LANE_OPS = 256 * 4 * 32 * 2.4e9
# the headline's dominant kernel as rocprofv3 names it (euclidean epilogue, fp32 in and out)
HEADLINE_KERNEL = "inner_tile_kernel<float,float,1,1,false,false,false>"
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "traffic_euclidean_manhattan_hamming_16384x128.txt")


def measured_traffic(kernel_prefix):
    """HBM bytes per launch of a kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (KiB per dispatch), each scaled by what the counter read for a plain 1 GiB copy."""
    try:
        rows = [l.split() for l in open(TRAFFIC_FILE) if l.strip() and not l.startswith("#")]
    except OSError:
        return None
    kv = {r[0]: float(r[1]) for r in rows if len(r) == 2}
    if not {"copy_bytes", "copy_fetch_kib", "copy_write_kib"} <= kv.keys():
        return None
    f_scale = kv["copy_bytes"] / (kv["copy_fetch_kib"] * 1024)
    w_scale = kv["copy_bytes"] / (kv["copy_write_kib"] * 1024)
    for r in rows:
        if len(r) == 5 and r[0].startswith(kernel_prefix) and r[1] == "fetch_kib":
            return (float(r[2]) * f_scale + float(r[4]) * w_scale) * 1024
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 + 200: the GPU leaves its idle clocks only after some tens of milliseconds of load;
    # 5 warm-up steps time the ramp (0.73 ms per headline step instead of 0.63)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--settle-ms", type=float, default=1500.0,
                    help="wall time of headline-op calls before the counted warm-up (clock ramp)")
    ap.add_argument("--n", type=int, default=16384)
    ap.add_argument("--d", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help="comma list of l2,l1,hamming (default all)")
    ap.add_argument("--with-copy", action="store_true",
                    help="also run one plain device copy of 1 GiB (torch copy_) so a rocprofv3 "
                         "--pmc FETCH_SIZE / WRITE_SIZE pass has a known-size reference kernel")
    ap.add_argument("--config", default="M",
                    help="M (default: the metric's workload), C2..C5: time the other "
                         "BASELINE.json configurations, NB: the neighbour masks, KF: the "
                         "polynomial / sigmoid kernels at the metric shape and RAGGED: shapes "
                         "whose rows are not whole 16-byte units beside their aligned twins "
                         "(one JSON line per op, not the headline)")
    return ap.parse_args()


_SETTLE = {"ms": 0.0, "done": False, "spent": 0.0}


def time_op(fn, steps, warmup, family=None):
    """Time per call (ms) of fn over `steps` back-to-back calls after `warmup` untimed ones (one
    event pair around the whole timed loop), and the wall time per call.  With `family`, also
    the mean device duration of that kernel family's launches made by those same timed calls
    (start / stop events stamped by each launch's own dispatch through the C ABI's launch
    timer): (step_ms, wall_ms, kernel_ms, launches_per_step)."""
    import torch

    if not _SETTLE["done"] and _SETTLE["ms"] > 0:  # once per process, before the first timing
        _SETTLE["spent"] = settle(fn, _SETTLE["ms"])
        _SETTLE["done"] = True
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timer = None
    if family is not None:
        from torchpairwise_amd import _capi as capi

        timer = capi.LaunchTimer(family, 64 * steps).arm()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = start.elapsed_time(end) / steps
    if timer is None:
        return ev_ms, wall * 1e3 / steps
    kms, dropped = timer.read()
    assert kms and not dropped, f"launch timer for {family}: {len(kms)} launches, {dropped} dropped"
    per_step = len(kms) / steps
    k_ms = sum(kms) / steps  # the family's device time per step
    # the kernels run inside the steps that contain them: their time cannot exceed the step's
    assert k_ms <= ev_ms, f"{family}: kernel {k_ms:.4f} ms > step {ev_ms:.4f} ms"
    return ev_ms, wall * 1e3 / steps, k_ms / per_step, per_step


def settle(fn, ms):
    """Calls fn for about `ms` of wall time (synchronising every 20 calls); returns the time."""
    import torch

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def _timed(fn, budget_s, max_reps=200):
    fn()  # warm-up
    reps, total = 0, 0.0
    while total < budget_s and reps < max_reps:
        t0 = time.perf_counter()
        fn()
        total += time.perf_counter() - t0
        reps += 1
    return total / reps, reps


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(n, d, budget_s=3.0):
    """The reference's CPU paths on the host cores of this process, on bounded samples of the
    workloads (about 25 s in all), as pair-features/s.  The headline entry is euclidean:
    torch.cdist(p = 2) = the reference's at::cdist (pairwise_metrics.cpp:24-31), with torch's
    intra-op threads."""
    import torch

    threads = torch.get_num_threads()
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    g = lambda s: torch.Generator().manual_seed(s)  # noqa: E731
    x2 = torch.randn(n, d, generator=g(1))
    rows = 1024
    x1 = torch.randn(rows, d, generator=g(0))
    out = {}
    for name, p in (("euclidean", 2.0), ("manhattan", 1.0)):
        t, reps = _timed(lambda: torch.cdist(x1, x2, p), budget_s)
        out[name] = {"value": rows * n * d / t, "unit": "pair-features/s", "cores": threads,
                     "kind": "reference",
                     "sample": f"torch.cdist(x1[{rows},{d}], x2[{n},{d}], p={p:g}) (= at::cdist of "
                               f"{name}_distances), {reps} reps of {t * 1e3:.1f} ms"}
    # the reference's own compiled CPU kernels, in a child process (their schemas would collide
    # with this build's in this one): hamming on M rows, jaccard on C4 rows, one C5 cloud pair
    try:
        import tempfile

        import numpy as np

        from oracle import ref_runner
        if ref_runner.available():
            hr, jr, jd, cp = 256, 16, 1024, 65536
            h1 = (torch.rand(hr, d, generator=g(0)) < 0.5).numpy()
            h2 = (torch.rand(n, d, generator=g(1)) < 0.5).numpy()
            j1 = (torch.rand(jr, jd, generator=g(0)) < 0.1).numpy()
            j2 = (torch.rand(32768, jd, generator=g(1)) < 0.1).numpy()
            c1 = torch.rand(1, cp, 3, generator=g(0)).numpy()
            c2 = (torch.rand(1, cp, 3, generator=g(1)) + 0.05).numpy()
            with tempfile.TemporaryDirectory() as tmp:
                r = ref_runner.run("time", {"h1": h1, "h2": h2, "j1": j1, "j2": j2, "c1": c1, "c2": c2,
                                            "budget": np.float64(budget_s)}, tmp)
            res = json.loads(str(r["results"]))
            for name, work, sample in (
                    ("hamming", hr * n * d, f"pwne_mean(x1[{hr},{d}] bool, x2[{n},{d}] bool)"),
                    ("jaccard", jr * 32768 * jd, f"prf_div(pwxor_sum, pwor_sum) on x1[{jr},{jd}], x2[32768,{jd}] bool"),
                    ("directed_hausdorff", cp * cp * 3, f"_directed_hausdorff of one [{cp},3] cloud pair (C5)")):
                t = res["hausdorff" if name == "directed_hausdorff" else name]["s_per_call"]
                # (one cloud pair: the reference's OpenMP loop runs over cloud pairs, so one thread)
                out[name] = {"value": work / t, "unit": "pair-features/s" if name != "directed_hausdorff"
                             else "nominal pair-features/s", "cores": 1 if name == "directed_hausdorff" else 32,
                             "kind": "reference",
                             "sample": f"{sample}: the reference's compiled CPU kernel (OpenMP, "
                                       f"num_threads(32) as compiled), "
                                       f"{res['hausdorff' if name == 'directed_hausdorff' else name]['reps']} reps of "
                                       f"{t * 1e3:.1f} ms"}
        from oracle import cref
        t, reps = _timed(lambda: cref.bool_reduce(h1, h2, "ne", True, threads=usable), budget_s)
        out["hamming_port_all_cores"] = {
            "value": 256 * n * d / t, "unit": "pair-features/s", "cores": usable, "kind": "port",
            "sample": f"oracle/cref.c restatement of the pwne_mean loop on x1[256,{d}], x2[{n},{d}], "
                      f"{reps} reps of {t * 1e3:.1f} ms"}
    except Exception as e:  # a missing oracle build must not cost the GPU line
        out["error"] = f"{type(e).__name__}: {e}"
    head = dict(out["euclidean"])
    head["cpu_model"] = _cpu_model()
    head["os_cpu_count"] = os.cpu_count()
    head["usable_cores"] = usable
    head["others"] = {k: v for k, v in out.items() if k != "euclidean"}
    return head


def run_config(cfg, steps, warmup):
    """Times the full-size BASELINE.json configurations C2..C5 through the drop-in ops
    (forward, and forward + backward where the configuration asks for it)."""
    import torch

    import torchpairwise_amd as tp

    dev = "cuda"
    lines = []

    def roof(bound, amount, ms, convention):
        """roofline of one line: algorithmic flops / lane-ops / bytes per call over its time"""
        rate = amount / (ms * 1e-3)
        peak, unit, scale = {"mfma": (PEAK_FP32_MFMA, "TFLOP/s", 1e12),
                             "mfma_bf16": (PEAK_BF16_MFMA, "TFLOP/s", 1e12),
                             "valu": (PEAK_VALU_LANE_OPS, "Tlane-op/s", 1e12),
                             "hbm": (PEAK_HBM, "GB/s", 1e9)}[bound]
        return {"roofline": {"bound": bound.split("_")[0], "achieved": rate / scale, "peak": peak / scale,
                             "unit": unit, "frac": rate / peak, "convention": convention}}

    def emit(name, ms, pf, extra=None):
        d = {"config": cfg, "op": name, "ms_per_call": ms, "pair_features_per_s": pf / (ms * 1e-3),
             "steps": steps, "warmup": warmup, "settle_ms": _SETTLE["spent"]}
        d.update(extra or {})
        lines.append(d)
        print(json.dumps(d), flush=True)

    if cfg == "C2":
        B, N, D = 8, 8192, 256
        for dtype in (torch.float32, torch.bfloat16):
            x1 = torch.randn(B, N, D, generator=torch.Generator().manual_seed(0)).to(dtype).to(dev)
            x2 = torch.randn(B, N, D, generator=torch.Generator().manual_seed(1)).to(dtype).to(dev)
            g = torch.randn(B, N, N, generator=torch.Generator().manual_seed(2)).to(dtype).to(dev)
            pf = B * N * N * D
            for fn in ("euclidean_distances", "cosine_distances"):
                f = getattr(tp, fn)
                ms, _ = time_op(lambda: f(x1, x2), steps, warmup)
                if dtype == torch.float32:
                    r = roof("mfma", 2 * pf, ms, "2 flop per pair-feature (one multiply-add)")
                else:
                    r = roof("hbm", 2 * B * N * N, ms, "the bf16 output written once (2 B per pair)")
                emit(f"{fn} fwd {dtype}", ms, pf, {"tflops": 2 * pf / (ms * 1e-3) / 1e12, **r})
                a = x1.detach().requires_grad_()
                b = x2.detach().requires_grad_()

                def fb():
                    a.grad = None
                    b.grad = None
                    f(a, b).backward(g)

                ms, _ = time_op(fb, steps, warmup)
                if dtype == torch.float32:
                    r = roof("mfma", 6 * pf, ms, "forward product + two backward products, 2 flop "
                                                 "per pair-feature each")
                else:
                    r = roof("hbm", 6 * B * N * N, ms, "output written, upstream gradient and output read "
                                                       "once (3 x 2 B per pair)")
                emit(f"{fn} fwd+bwd {dtype}", ms, pf, {"tflops": 6 * pf / (ms * 1e-3) / 1e12, **r})
            del x1, x2, g
            torch.cuda.empty_cache()
    elif cfg == "C3":
        N, D = 16384, 128
        x1 = (torch.rand(N, D, generator=torch.Generator().manual_seed(0)) * 2 - 1).to(dev)
        x2 = (torch.rand(N, D, generator=torch.Generator().manual_seed(1)) * 2 - 1).to(dev)
        pf = N * N * D
        ms, _ = time_op(lambda: tp.minkowski_distances(x1, x2, 3.0), steps, warmup)
        emit("minkowski p=3 fwd", ms, pf, roof("valu", 3 * pf, ms, "3 VALU lane-ops per pair-feature "
                                               "(sub, |d| * d, fma) against the FP32 VALU dual-issue rate"))
        a, b = x1.clone().requires_grad_(), x2.clone().requires_grad_()
        ones = torch.ones(N, N, device=dev)

        def fb():
            a.grad = None
            b.grad = None
            tp.minkowski_distances(a, b, 3.0).backward(ones)

        ms, _ = time_op(fb, steps, warmup)
        emit("minkowski p=3 fwd+bwd", ms, pf, roof("valu", 9 * pf, ms, "3 VALU lane-ops per pair-feature "
                                                   "forward and in each of the two backward directions"))
        ms, _ = time_op(lambda: tp.chebyshev_distances(x1, x2), steps, warmup)
        emit("chebyshev fwd", ms, pf, roof("valu", 1.5 * pf, ms, "1.5 VALU lane-ops per pair-feature "
                                           "(v_sub, and v_max3 over two |d| per instruction)"))
    elif cfg == "C4":
        N, D = 32768, 1024
        h1 = (torch.rand(N, D, generator=torch.Generator().manual_seed(0)) < 0.5).to(dev)
        h2 = (torch.rand(N, D, generator=torch.Generator().manual_seed(1)) < 0.5).to(dev)
        pf = N * N * D
        ms, _ = time_op(lambda: tp.hamming_distances(h1, h2), steps, warmup)
        emit("hamming fwd", ms, pf, {"out_GBps": 4 * N * N / (ms * 1e-3) / 1e9,
                                     **roof("hbm", 4 * N * N, ms, "the fp32 output written once")})
        j1 = (torch.rand(N, D, generator=torch.Generator().manual_seed(0)) < 0.1).to(dev)
        j2 = (torch.rand(N, D, generator=torch.Generator().manual_seed(1)) < 0.1).to(dev)
        ms, _ = time_op(lambda: tp.jaccard_distances(j1, j2), steps, warmup)
        emit("jaccard fwd", ms, pf, {"out_GBps": 4 * N * N / (ms * 1e-3) / 1e9,
                                     **roof("hbm", 4 * N * N, ms, "the fp32 output written once")})
        # the other boolean count metrics: one fused pass (pack + AND-popcount tile with the
        # metric's epilogue), the same on rows packed once (PackedBool), and the reference's
        # composite (2-4 pw*_sum passes + ATen elementwise passes) on the same GPU
        ops = torch.ops.torchpairwise
        p1, p2 = tp.PackedBool.pack(h1), tp.PackedBool.pack(h2)
        for metric in ("dice", "yule"):
            f = getattr(tp, f"{metric}_distances")
            ms, _ = time_op(lambda: f(h1, h2), steps, warmup)
            emit(f"{metric} fwd", ms, pf, {"out_GBps": 4 * N * N / (ms * 1e-3) / 1e9,
                                           **roof("hbm", 4 * N * N, ms, "the fp32 output written once")})
            ms, _ = time_op(lambda: tp.packed.cdist(p1, p2, metric), steps, warmup)
            emit(f"{metric} fwd on PackedBool", ms, pf, {"out_GBps": 4 * N * N / (ms * 1e-3) / 1e9,
                                                         **roof("hbm", 4 * N * N, ms, "the fp32 output written once")})
        def dice_composite():
            R = ops.pwxor_sum(h1, h2)
            return R / (2 * ops.pwand_sum(h1, h2) + R)
        ms, _ = time_op(dice_composite, steps, warmup)
        emit("dice fwd, reference composite route", ms, pf,
             roof("hbm", 4 * N * N, ms, "the fp32 output written once"))
    elif cfg == "RAGGED":
        # shapes whose rows are not whole 16-byte units (output m, or operand d) beside their
        # aligned twins: euclidean fp32 / bf16, manhattan fp32, jaccard bool (forward)
        g = torch.Generator().manual_seed(0)
        for (n, m, d) in ((16384, 16384, 128), (16384, 16383, 128), (16384, 16384, 127), (16384, 16384, 130)):
            x1, x2 = torch.randn(n, d, generator=g).to(dev), torch.randn(m, d, generator=g).to(dev)
            pf = n * m * d
            ms, _ = time_op(lambda: tp.euclidean_distances(x1, x2), steps, warmup)
            emit(f"euclidean fp32 {n}x{m}x{d}", ms, pf, roof("mfma", 2 * pf, ms, "2 flops per pair-feature"))
            ms, _ = time_op(lambda: tp.manhattan_distances(x1, x2), steps, warmup)
            emit(f"manhattan fp32 {n}x{m}x{d}", ms, pf, roof("valu", 2 * pf, ms, "2 VALU lane-ops per pair-feature"))
        for (n, m, d) in ((8192, 8192, 256), (8192, 8191, 256), (8192, 8192, 255)):
            y1 = torch.randn(8, n, d, generator=g).to(dev).bfloat16()
            y2 = torch.randn(8, m, d, generator=g).to(dev).bfloat16()
            ms, _ = time_op(lambda: tp.euclidean_distances(y1, y2), steps, warmup)
            emit(f"euclidean bf16 8x{n}x{m}x{d}", ms, 8 * n * m * d,
                 roof("hbm", 2 * 8 * n * m, ms, "the bf16 output written once"))
        for (n, m, d) in ((16384, 16384, 1024), (16384, 16383, 1024), (16384, 16384, 1023)):
            b1 = (torch.rand(n, d, generator=g) < 0.3).to(dev)
            b2 = (torch.rand(m, d, generator=g) < 0.3).to(dev)
            ms, _ = time_op(lambda: tp.jaccard_distances(b1, b2), steps, warmup)
            emit(f"jaccard bool {n}x{m}x{d}", ms, n * m * d, roof("hbm", 4 * n * m, ms, "the fp32 output written once"))
    elif cfg == "KF":
        # kernel functions at the metric shape: polynomial / sigmoid fused into the MFMA
        # epilogue, rbf / laplacian into the VALU kernel's, each against the reference's
        # composite (distance or matmul, then the elementwise ops) on the same GPU
        N, D = 16384, 128
        x1 = torch.randn(N, D, generator=torch.Generator().manual_seed(0)).to(dev)
        x2 = torch.randn(N, D, generator=torch.Generator().manual_seed(1)).to(dev)
        pf = N * N * D
        ones = torch.ones(N, N, device=dev)
        g = 1.0 / D
        for name, f, ref in (
                ("polynomial_kernel degree=3", lambda a, b: tp.polynomial_kernel(a, b, 3),
                 lambda a, b: a.matmul(b.transpose(-1, -2)).mul_(g).add_(1.0).pow_(3)),
                ("sigmoid_kernel", lambda a, b: tp.sigmoid_kernel(a, b),
                 lambda a, b: a.matmul(b.transpose(-1, -2)).mul_(g).add_(1.0).tanh_()),
                # unfused: this build's distance kernel, then mul_ and exp_ (at::cdist p = 1, the
                # reference's laplacian distance, fails to launch at this size on PyTorch-ROCm:
                # "invalid configuration argument")
                ("rbf_kernel", lambda a, b: tp.rbf_kernel(a, b),
                 lambda a, b: torch.ops.torchpairwise._ppminkowski(a, b, 2.0).mul_(-g).exp_()),
                ("laplacian_kernel", lambda a, b: tp.laplacian_kernel(a, b),
                 lambda a, b: tp.manhattan_distances(a, b).mul_(-g).exp_())):
            mf = name[0] in "ps"  # polynomial / sigmoid: the MFMA kernel; rbf / laplacian: VALU
            conv = ("2 flop per pair-feature (one multiply-add)" if mf else
                    "2 VALU lane-ops per pair-feature (sub, fma or abs-add)")
            ms, _ = time_op(lambda: f(x1, x2), steps, warmup)
            emit(f"{name} fwd", ms, pf, {"tflops": 2 * pf / (ms * 1e-3) / 1e12,
                                         **roof("mfma" if mf else "valu", 2 * pf, ms, conv)})
            ms, _ = time_op(lambda: ref(x1, x2), steps, warmup)
            emit(f"{name} fwd, " + ("reference composite route" if "kernel" in name and name[0] in "ps"
                                    else "unfused route (distance kernel, mul_, exp_)"), ms, pf,
                 roof("mfma" if mf else "valu", 2 * pf, ms, conv))
            a, b = x1.clone().requires_grad_(), x2.clone().requires_grad_()

            def fb():
                a.grad = None
                b.grad = None
                f(a, b).backward(ones)

            ms, _ = time_op(fb, steps, warmup)
            emit(f"{name} fwd+bwd", ms, pf, roof("mfma" if mf else "valu", 6 * pf, ms,
                                                 "forward + two backward directions, 2 per "
                                                 "pair-feature each"))
    elif cfg == "C5":
        from torchpairwise_amd import _capi as capi

        C, P, D = 16, 65536, 3
        x1 = torch.rand(C, P, D, generator=torch.Generator().manual_seed(0)).to(dev)
        x2 = (torch.rand(C, P, D, generator=torch.Generator().manual_seed(1)) + 0.05).to(dev)
        pf = C * C * P * P * D
        # the work the kernels did in one forward, from their own counters
        counters = capi.HausdorffCounters().arm()
        tp.directed_hausdorff_distances(x1, x2)
        work = counters.read()

        def floor_of(ms, launches):
            """The forward is a chain of dependent launches over a pruned search: its floor is
            that many empty launches back to back (timed here, the same way) plus reading both
            inputs once from HBM; frac = floor / measured time."""
            t_empty, _ = time_op(lambda: capi.empty_launches(launches), steps, warmup)
            hbm_ms = 2 * C * P * D * 4 / PEAK_HBM * 1e3
            floor = t_empty + hbm_ms
            evaluated = work["pairs"]
            return {"roofline": {"bound": "launch chain", "achieved": floor, "peak": ms, "unit": "ms",
                                 "frac": floor / ms,
                                 "convention": f"floor = {launches} empty dependent launches "
                                               f"({t_empty * 1e3 / launches:.2f} us each, timed here) + both "
                                               f"inputs read once at 8 TB/s ({hbm_ms * 1e3:.1f} us); frac = "
                                               "floor / ms_per_call"},
                    "launches": launches, "empty_launch_chain_ms": t_empty, "hbm_floor_ms": hbm_ms,
                    "pairs_evaluated": evaluated, "cell_tests": work["cell_tests"],
                    "pairs_nominal": C * C * P * P, "evaluated_fraction": evaluated / (C * C * P * P),
                    "valu_frac_of_evaluated": 8 * evaluated / (ms * 1e-3) / PEAK_VALU_LANE_OPS}

        ms, _ = time_op(lambda: tp.directed_hausdorff_distances(x1, x2), steps, warmup)
        emit("directed_hausdorff fwd", ms, pf, {"note": "nominal B1*B2*P1*P2*D pair-features",
                                                **floor_of(ms, work["launches"])})
        a = x1.clone().requires_grad_()
        g = torch.randn(C, C, generator=torch.Generator().manual_seed(2)).to(dev)

        def fb():
            a.grad = None
            tp.directed_hausdorff_distances(a, x2)[0].backward(g)

        ms, _ = time_op(fb, steps, warmup)
        # the backward adds two launches: the gradients' zero fill and the scatter
        emit("directed_hausdorff fwd+bwd", ms, pf, floor_of(ms, work["launches"] + 2))
    elif cfg == "NB":
        # neighbour masks at the metric shape: the selection kernel alone on a resident
        # distance matrix (HBM-bound: 4 B read + 1 B written per entry), the whole drop-in
        # op, and the reference's own route (argsort + index_put_) on the same GPU
        N, D = 16384, 128
        x1 = torch.randn(N, D, generator=torch.Generator().manual_seed(0)).to(dev)
        x2 = torch.randn(N, D, generator=torch.Generator().manual_seed(1)).to(dev)
        dist = tp.euclidean_distances(x1, x2)
        pf = N * N * D
        for k in (1, 8, 32, 128, 255, 511):
            ms, _ = time_op(lambda: torch.ops.torchpairwise._row_smallest_mask(dist, k + 1), steps, warmup)
            emit(f"row_smallest_mask count={k + 1}", ms, pf,
                 {"hbm_GBps": 5.0 * N * N / (ms * 1e-3) / 1e9,
                  "hbm_frac": 5.0 * N * N / (ms * 1e-3) / PEAK_HBM,
                  **roof("hbm", 5.0 * N * N, ms, "each fp32 distance read once, one mask byte written")})
        conv = "distances written and read once (4 + 4 B per entry) and one mask byte written"
        # k + 1 <= 16: the tile kernel keeps each row's candidates per tile (no distance matrix),
        # bound by the fp32 products like the radius mask; beside it the unfused route
        # (distances, then the selection kernel) at the same k
        for k in (1, 3):
            ms, _ = time_op(lambda: tp.k_neighbors_mask(x1, x2, k), steps, warmup)
            emit(f"k_neighbors_mask k={k} (euclidean, fused candidates + select)", ms, pf,
                 roof("mfma", 2.0 * N * N * D, ms, "2 flop per pair-feature on fp32 MFMA"))
            ms, _ = time_op(lambda: torch.ops.torchpairwise._row_smallest_mask(tp.euclidean_distances(x1, x2), k + 1),
                            steps, warmup)
            emit(f"k_neighbors_mask k={k} unfused (euclidean distances + selection)", ms, pf,
                 roof("hbm", 9.0 * N * N, ms, conv))
        ms, _ = time_op(lambda: tp.k_neighbors_mask(x1, x2, 16), steps, warmup)
        emit("k_neighbors_mask k=16 (euclidean + selection)", ms, pf, roof("hbm", 9.0 * N * N, ms, conv))
        # the radius mask comes straight from the tile kernel's epilogue (no distance matrix,
        # one byte per entry written): bound by the fp32 matrix-core products
        ms, _ = time_op(lambda: tp.radius_neighbors_mask(x1, x2, 14.0), steps, warmup)
        emit("radius_neighbors_mask eps=14 (euclidean + le, one fused launch)", ms, pf,
             roof("mfma", 2.0 * N * N * D, ms, "2 flop per pair-feature on fp32 MFMA"))

        def ref_route():
            inds = dist.argsort(1, False)[:, :2]
            first = torch.arange(N, device=dev).view(-1, 1).repeat(1, 2)
            out = torch.zeros(N, N, dtype=torch.bool, device=dev)
            out.index_put_((first.flatten(), inds.flatten()), torch.tensor(True, device=dev))
            return out

        ms, _ = time_op(ref_route, max(1, steps // 5), 1)
        emit("reference route argsort+index_put_ k=1 (selection only)", ms, pf,
             roof("hbm", 5.0 * N * N, ms, "each fp32 distance read once, one mask byte written"))
    else:
        raise SystemExit(f"unknown config {cfg}")
    return lines


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; run with --gpus 1 "
                                   "(multi-GPU sharding is described in DESIGN.md, not run)"}))
        sys.exit(2)
    _SETTLE["ms"] = args.settle_ms
    if args.config != "M":
        import torch

        assert torch.cuda.is_available(), "bench.py needs a GPU"
        run_config(args.config, args.steps, args.warmup)
        return
    import torch

    import torchpairwise_amd as tp

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = "cuda"
    n, d = args.n, args.d
    g1 = torch.Generator().manual_seed(0)
    g2 = torch.Generator().manual_seed(1)
    x1 = torch.randn(n, d, generator=g1).to(dev)
    x2 = torch.randn(n, d, generator=g2).to(dev)
    b1 = (torch.rand(n, d, generator=torch.Generator().manual_seed(0)) < 0.5).to(dev)
    b2 = (torch.rand(n, d, generator=torch.Generator().manual_seed(1)) < 0.5).to(dev)
    only = set(args.only.split(",")) if args.only else {"l2", "l1", "hamming"}
    pf = n * n * d
    if args.with_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    extra = {}
    res = {}

    if "l2" in only:
        time_op(lambda: tp.euclidean_distances(x1, x2), 1, 0)  # the settle phase (once)
        # the dominant kernel's launches are timed inside the op's own timed steps (events
        # around each tile-kernel launch, on the stream the op launches on)
        ms, wall_ms, k_ms, per_step = time_op(lambda: tp.euclidean_distances(x1, x2), args.steps,
                                              args.warmup, family="inner_tile_kernel")
        assert per_step == 1, f"{per_step} tile-kernel launches per euclidean_distances call"
        flops = 2.0 * n * n * d
        res["l2"] = {"ms": ms, "wall_ms": wall_ms, "value": pf / (ms * 1e-3),
                     "roofline": {"bound": "mfma", "achieved": flops / (k_ms * 1e-3) / 1e12,
                                  "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                                  "frac": flops / (k_ms * 1e-3) / PEAK_FP32_MFMA,
                                  "traffic": measured_traffic(HEADLINE_KERNEL),
                                  "kernel": HEADLINE_KERNEL,
                                  "kernel_ms": k_ms,
                                  "timing": "mean device duration of the tile-kernel launch inside "
                                            "each timed step (start / stop events stamped by "
                                            "the launch's own dispatch on the op's stream); "
                                            "kernel_ms <= ms_per_step is asserted"}}
    if "l1" in only:
        ms, wall_ms, k_ms, _ = time_op(lambda: tp.manhattan_distances(x1, x2), args.steps, args.warmup,
                                       family="lp_forward_kernel")
        ops = 2.0 * pf  # v_sub + abs-modified v_add per pair-feature
        extra["manhattan_fp32"] = {
            "value": pf / (ms * 1e-3), "ms_per_call": ms,
            "roofline": {"bound": "valu", "achieved": ops / (k_ms * 1e-3) / 1e12,
                         "peak": PEAK_VALU_LANE_OPS / 1e12, "unit": "Tlane-op/s",
                         "frac": ops / (k_ms * 1e-3) / PEAK_VALU_LANE_OPS,
                         "kernel": "lp_forward_kernel<0,1,true,0>", "kernel_ms": k_ms,
                         "convention": "2 VALU lane-ops per pair-feature (v_sub_f32, abs-modified "
                                       "v_add_f32) against the FP32 VALU issue rate with dual "
                                       "issue, 256 CU x 4 SIMD x 32 lanes x 2 x 2.4 GHz = 7.86e13 "
                                       "lane-ops/s (157.3 TFLOP/s counts an FMA as 2 flops; "
                                       "neither op here is an FMA, so against that spec, one "
                                       "flop per op, the fraction is half of this)"}}
    if "hamming" in only:
        ms, wall_ms, k_ms, _ = time_op(lambda: tp.hamming_distances(b1, b2), args.steps, args.warmup,
                                       family="bool_reduce_kernel")
        out_bytes = 4.0 * n * n
        extra["hamming_bool"] = {
            "value": pf / (ms * 1e-3), "ms_per_call": ms,
            "roofline": {"bound": "hbm", "achieved": out_bytes / (k_ms * 1e-3) / 1e9,
                         "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                         "frac": out_bytes / (k_ms * 1e-3) / PEAK_HBM,
                         "kernel": "bool_reduce_kernel<2,1,64,2>", "kernel_ms": k_ms,
                         "note": "algorithmic bytes = the fp32 output (inputs are 2 x 2 MiB, "
                                 "packed to 2 x 256 KiB); ms_per_call includes the pack launches"}}

    head = res.get("l2")
    line = {
        "metric": "pair-features/s (N·M·D/s) + % roofline, L2/L1/Hamming at 16k×16k×128, 1 GPU",
        "value": head["value"] if head else None,
        "unit": "pair-features/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": _SETTLE["spent"],
        "ms_per_step": head["ms"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (torch.randn, CPU generators seeded 0/1, moved to HBM before timing)",
        "config": {"workload": f"euclidean_distances x1[{n},{d}] x2[{n},{d}] fp32 "
                               f"(manhattan fp32 and hamming bool at the same shape under extra)",
                   "n": n, "m": n, "d": d},
        "roofline": head["roofline"] if head else None,
        "extra": extra,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(n, d)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
