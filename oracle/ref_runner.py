#!/usr/bin/env python3
"""Runs the reference's own compiled CPU kernels (oracle/_ref) in THIS process on inputs from
an .npz and writes the outputs to another .npz — TEST INFRASTRUCTURE ONLY.  Meant to be
started as a child process (it registers the reference's torch.ops.torchpairwise schemas,
which would collide with torchpairwise_amd's in the same process).

usage: python oracle/ref_runner.py <op> <in.npz> <out.npz>
  op = hausdorff   (x1, x2[, perm seed]) -> out, idx1, idx2
       hausdorff_backward (grad, x1, x2) -> grad_x1, grad_x2
       pw_<name>    (x1, x2) -> out            e.g. pw_pwne_mean, pw_pwxor_sum
       jaccard     (x1, x2) -> out             (prf_div(pwxor_sum, pwor_sum), the reference's composite)
       prf         cases (JSON) + c<i>_a / _b / _g arrays -> c<i>_<result> arrays and c<i>_err
                   messages: the 20 prf_div-family ops through run_prf_case
       ops         cases (JSON) + c<i>_<name> arrays -> results of run_op_case (any op, overload,
                   tensor / scalar arguments, autograd backward of its first output)
       time        h1, h2 (bool), j1, j2 (bool), c1, c2 (clouds), budget -> seconds per call of
                   the reference's pwne_mean (hamming), its jaccard composite and its
                   _directed_hausdorff, each repeated within the budget (the CPU baseline)
"""
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

LIB = Path(__file__).resolve().parent / "_ref" / "libtorchpairwise_ref.so"


def available() -> bool:
    return LIB.exists()


def run(op: str, inputs: dict, tmpdir) -> dict:
    """Parent-side helper: runs `op` in a child process and returns its outputs."""
    tmpdir = Path(tmpdir)
    src, dst = tmpdir / f"{op}_in.npz", tmpdir / f"{op}_out.npz"
    np.savez(src, **inputs)
    subprocess.run([sys.executable, __file__, op, str(src), str(dst)], check=True)
    return dict(np.load(dst, allow_pickle=False))


# --------------------------------------------------------------------------- prf_div cases
# Tensors cross the process boundary as numpy arrays; bfloat16 travels as its int16 bits.
def tensor_to_np(t) -> tuple:
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy(), "bfloat16"
    return t.numpy(), str(t.dtype).replace("torch.", "")


def np_to_tensor(a, tag: str):
    import torch
    t = torch.from_numpy(np.array(a))
    return t.view(torch.bfloat16) if tag == "bfloat16" else t


def run_prf_case(ops, case: dict, a, b, g, device: str) -> dict:
    """Runs one prf_div-family case on `ops` (a torch.ops.torchpairwise namespace, this
    build's or the reference's) and returns its results as tensors, or {"err": message}.

    case: kind "fwd" (op prf_div / prf_ldiv, overload default / Scalar / rScalar, autograd
    backward of grad g when case["grad"]), "inplace" (prf_div_ / prf_ldiv_, default or Scalar,
    applied to a clone of a leaf), or "bwd" (a _prf_*_backward op called directly)."""
    import torch
    kind, name, ov, mode = case["kind"], case["op"], case["ov"], case["mode"]
    c = case.get("scalar")
    grad = bool(case.get("grad"))
    f = getattr(getattr(ops, name), ov)
    dev = lambda t: None if t is None else t.to(device)  # noqa: E731
    a, b, g = dev(a), dev(b), dev(g)
    res = {}
    try:
        if kind == "fwd":
            ta = None if a is None else a.clone().requires_grad_(grad and a.is_floating_point())
            tb = None if b is None else b.clone().requires_grad_(grad and b.is_floating_point())
            args = {"default": (ta, tb), "Scalar": (ta, c), "rScalar": (c, tb)}[ov]
            out = f(*args, mode)
            res["out"] = out
            if grad:
                out.backward(g)
                for key, t in (("ga", ta), ("gb", tb)):
                    if t is not None and t.grad is not None:
                        res[key] = t.grad
        elif kind == "inplace":
            leaf = a.clone().requires_grad_(grad)
            ta = leaf.clone()
            tb = None if b is None else b.clone().requires_grad_(grad and b.is_floating_point())
            ret = f(ta, tb if ov == "default" else c, mode)
            res["out"] = ta
            res["same"] = torch.tensor(ret.data_ptr() == ta.data_ptr())
            if grad:
                ta.backward(g)
                res["ga"] = leaf.grad
                if tb is not None and tb.grad is not None:
                    res["gb"] = tb.grad
        else:
            args = {"default": (g, a, b), "Scalar": (g, a, c), "rScalar": (g, c, b)}[ov]
            r = f(*args, mode)
            if ov == "default":
                res["ga"], res["gb"] = r
            else:
                res["ga" if ov == "Scalar" else "gb"] = r
    except Exception as e:  # the message is part of the interface
        return {"err": f"{type(e).__name__}: {str(e).splitlines()[0]}"}
    return {k: v.detach().cpu() for k, v in res.items()}


def run_op_case(ops, case: dict, tensors: dict, device: str) -> dict:
    """Runs one case of any op on `ops` (this build's or the reference's namespace).

    case: {"op": name, "ov": overload ("default"), "args": [item], "kwargs": {name: item},
    "req": [tensor names that require grad], "grad": tensor name of the upstream gradient of
    the first output (optional)}; item = {"t": tensor name} or {"v": value}.  Returns
    {"out<k>": outputs, "grad_<name>": gradients} or {"err": message}."""
    def item(it, leaves):
        if "t" not in it:
            return it["v"]
        t = tensors[it["t"]].to(device).clone()
        if it["t"] in case.get("req", ()):
            t.requires_grad_(True)
            leaves[it["t"]] = t
        return t
    leaves = {}
    res = {}
    try:
        f = getattr(getattr(ops, case["op"]), case.get("ov", "default"))
        args = [item(a, leaves) for a in case.get("args", [])]
        kwargs = {k: item(v, leaves) for k, v in case.get("kwargs", {}).items()}
        out = f(*args, **kwargs)
        outs = list(out) if isinstance(out, (tuple, list)) else [out]
        for k, o in enumerate(outs):
            res[f"out{k}"] = o
        if case.get("grad"):
            outs[0].backward(tensors[case["grad"]].to(device))
            for name, t in leaves.items():
                if t.grad is not None:
                    res[f"grad_{name}"] = t.grad
    except Exception as e:  # the message is part of the interface
        return {"err": f"{type(e).__name__}: {str(e).splitlines()[0]}"}
    return {k: v.detach().cpu() for k, v in res.items()}


def run_op_reference(cases, tmpdir) -> list:
    """The reference's results for [(case, {name: tensor})], in a child process."""
    arrays, meta = {}, []
    for i, (case, tensors) in enumerate(cases):
        tags = {}
        for name, t in tensors.items():
            arrays[f"c{i}_{name}"], tags[name] = tensor_to_np(t)
        meta.append({"case": case, "tags": tags})
    arrays["cases"] = np.array(json.dumps(meta))
    raw = run("ops", arrays, tmpdir)
    out = []
    for i, m in enumerate(json.loads(str(raw["results"]))):
        out.append({"err": m["err"]} if "err" in m else
                   {k: np_to_tensor(raw[f"c{i}_{k}"], tag) for k, tag in m["tags"].items()})
    return out


def encode_prf_cases(cases) -> dict:
    """[(case, a, b, g)] -> npz members (tensors as arrays + dtype tags in the JSON)."""
    arrays, meta = {}, []
    for i, (case, *ts) in enumerate(cases):
        tags = {}
        for key, t in zip("abg", ts):
            if t is not None:
                arrays[f"c{i}_{key}"], tags[key] = tensor_to_np(t)
        meta.append({"case": case, "tags": tags})
    arrays["cases"] = np.array(json.dumps(meta))
    return arrays


def decode_prf_cases(d: dict):
    meta = json.loads(str(d["cases"]))
    out = []
    for i, m in enumerate(meta):
        ts = [np_to_tensor(d[f"c{i}_{k}"], m["tags"][k]) if k in m["tags"] else None for k in "abg"]
        out.append((m["case"], *ts))
    return out


def run_prf_reference(cases, tmpdir) -> list:
    """The reference's results for [(case, a, b, g)], computed in a child process."""
    raw = run("prf", encode_prf_cases(cases), tmpdir)
    meta = json.loads(str(raw["results"]))
    results = []
    for i, m in enumerate(meta):
        if "err" in m:
            results.append({"err": m["err"]})
        else:
            results.append({k: np_to_tensor(raw[f"c{i}_{k}"], tag) for k, tag in m["tags"].items()})
    return results


def main(op: str, src: str, dst: str) -> None:
    import torch

    torch.ops.load_library(str(LIB))
    ops = torch.ops.torchpairwise
    d = dict(np.load(src, allow_pickle=False))
    t = {k: torch.from_numpy(v) for k, v in d.items() if v.dtype.kind != "U"}
    if op == "hausdorff":
        kw = {}
        if "seed" in d:
            kw = dict(shuffle=True, generator=torch.Generator().manual_seed(int(d["seed"])))
        o, i1, i2 = ops._directed_hausdorff(t["x1"], t["x2"], **kw)
        np.savez(dst, out=o.numpy(), idx1=i1.numpy(), idx2=i2.numpy())
    elif op == "hausdorff_backward":
        x1 = t["x1"].clone().requires_grad_()
        x2 = t["x2"].clone().requires_grad_()
        out = ops._directed_hausdorff(x1, x2)[0]
        out.backward(t["grad"])
        np.savez(dst, grad_x1=x1.grad.numpy(), grad_x2=x2.grad.numpy())
    elif op.startswith("pw_"):
        np.savez(dst, out=getattr(ops, op[3:])(t["x1"], t["x2"]).numpy())
    elif op == "prf":
        arrays, meta = {}, []
        for i, (case, a, b, g) in enumerate(decode_prf_cases(d)):
            r = run_prf_case(ops, case, a, b, g, "cpu")
            if "err" in r:
                meta.append({"err": r["err"]})
                continue
            tags = {}
            for k, v in r.items():
                arrays[f"c{i}_{k}"], tags[k] = tensor_to_np(v)
            meta.append({"tags": tags})
        arrays["results"] = np.array(json.dumps(meta))
        np.savez(dst, **arrays)
    elif op == "ops":
        arrays, meta = {}, []
        for i, m in enumerate(json.loads(str(d["cases"]))):
            tensors = {k: np_to_tensor(d[f"c{i}_{k}"], tag) for k, tag in m["tags"].items()}
            r = run_op_case(ops, m["case"], tensors, "cpu")
            if "err" in r:
                meta.append({"err": r["err"]})
                continue
            tags = {}
            for k, v in r.items():
                arrays[f"c{i}_{k}"], tags[k] = tensor_to_np(v)
            meta.append({"tags": tags})
        arrays["results"] = np.array(json.dumps(meta))
        np.savez(dst, **arrays)
    elif op == "time":
        import time
        budget = float(d["budget"])
        work = {"hamming": lambda: ops.pwne_mean(t["h1"], t["h2"]),
                "jaccard": lambda: ops.prf_div(ops.pwxor_sum(t["j1"], t["j2"]), ops.pwor_sum(t["j1"], t["j2"]), "zero"),
                "hausdorff": lambda: ops._directed_hausdorff(t["c1"], t["c2"])}
        res = {}
        for name, fn in work.items():
            fn()  # warm-up
            reps, total = 0, 0.0
            while total < budget and reps < 100:
                t0 = time.perf_counter()
                fn()
                total += time.perf_counter() - t0
                reps += 1
            res[name] = {"s_per_call": total / reps, "reps": reps}
        np.savez(dst, results=np.array(json.dumps(res)))
    elif op == "jaccard":
        np.savez(dst, out=ops.prf_div(ops.pwxor_sum(t["x1"], t["x2"]), ops.pwor_sum(t["x1"], t["x2"]), "zero").numpy())
    else:
        raise SystemExit(f"unknown op {op}")


if __name__ == "__main__":
    main(*sys.argv[1:4])
