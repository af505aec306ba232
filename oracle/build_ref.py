#!/usr/bin/env python3
"""Compiles the reference's own CPU kernels for the hot path, from the sources where they
lie under /root/reference, into oracle/_ref/libtorchpairwise_ref.so (git-ignored; it travels
to the GPU box like the other built libraries).  TEST INFRASTRUCTURE ONLY.

Sources (g++ directly, against the installed torch headers, with the reference's own OpenMP
flags; nothing is copied): every CPU source of the reference — csrc/torchpairwise.cpp (built
without CUDA: _cuda_version() returns -1), csrc/ops/*.cpp (the public metrics, cdist /
pdist, the neighbour masks and the internal op stubs), csrc/ops/cpu/*.cpp (the OpenMP kernels)
and csrc/ops/autograd/*.cpp.  Its CUDA half (csrc/ops/cuda/) needs nvcc and is not built.
The library registers the reference's own torch.ops.torchpairwise schemas (all 101), so it is
loaded only in a separate process (oracle/ref_runner.py), never next to torchpairwise_amd.
"""
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

REF = Path(os.environ.get("TPW_REFERENCE", "/root/reference")) / "torchpairwise" / "csrc"
OUT = Path(__file__).resolve().parent / "_ref"
def sources():
    """Every CPU source of the reference, relative to csrc/."""
    found = ["torchpairwise.cpp"]
    for sub in ("ops", "ops/cpu", "ops/autograd"):
        found += sorted(f"{sub}/{p.name}" for p in (REF / sub).glob("*.cpp"))
    return found


def main() -> int:
    if not REF.exists():
        print(f"[build_ref] {REF} not present; skipping the reference build")
        return 0
    import torch
    from torch.utils import cpp_extension

    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    OUT.mkdir(exist_ok=True)
    objs = []

    def compile_one(src):
        obj = OUT / (src.replace("/", "_") + ".o")
        # -DAT_PARALLEL_OPENMP + -fopenmp: the reference's setup.py:26-56,89-91 (its CPU loops
        # then run on OpenMP with num_threads(32), cpu/cpu_helpers.h:6-18)
        subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-fopenmp", "-DAT_PARALLEL_OPENMP",
                        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                        *inc, f"-I{REF}", "-c", str(REF / src), "-o", str(obj)], check=True)
        return obj

    with cf.ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(compile_one, sources()))
    lib = OUT / "libtorchpairwise_ref.so"
    subprocess.run(["g++", "-shared", "-fopenmp", *map(str, objs), "-o", str(lib), f"-L{libdir}",
                    "-lc10", "-ltorch", "-ltorch_cpu", f"-Wl,-rpath,{libdir}"], check=True)
    for o in objs:
        o.unlink()
    print(f"[build_ref] {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
