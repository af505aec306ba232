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
"""
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


def main(op: str, src: str, dst: str) -> None:
    import torch

    torch.ops.load_library(str(LIB))
    ops = torch.ops.torchpairwise
    d = dict(np.load(src, allow_pickle=False))
    t = {k: torch.from_numpy(v) for k, v in d.items()}
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
    elif op == "jaccard":
        np.savez(dst, out=ops.prf_div(ops.pwxor_sum(t["x1"], t["x2"]), ops.pwor_sum(t["x1"], t["x2"]), "zero").numpy())
    else:
        raise SystemExit(f"unknown op {op}")


if __name__ == "__main__":
    main(*sys.argv[1:4])
