"""Builds the native parts in-tree (no JIT cache, no hipify).

* ``libtorchpairwise_hip.so`` — the gfx950 kernels behind the C ABI of
  ``include/torchpairwise_amd.h`` (hipcc, one object per ``csrc/hip/*.hip``).
* ``_C.so`` — the PyTorch extension that registers the ``torch.ops.torchpairwise``
  schemas and calls the C ABI (g++ against the installed torch headers).

Run ``python torchpairwise_amd/_build.py [hip|ext|all]`` (by path: importing the package
needs the built libraries) or call :func:`build_all`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
HIP_SRC = PKG / "csrc" / "hip"
OPS_SRC = PKG / "csrc" / "ops"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
HIP_LIB = PKG / "libtorchpairwise_hip.so"
EXT_LIB = PKG / "_C.so"

ARCH = os.environ.get("TPW_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

# Packed-FP32 VALU forms are disabled for every HIP object (the compiler would otherwise
# emit v_pk_* FP32 ops from plain float code).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", f"-I{INCLUDE}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _jobs() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def build_hip_lib(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(HIP_SRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".hip.o") for s in sources]
    with cf.ThreadPoolExecutor(_jobs()) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)])
                for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, HIP_LIB)
    if verbose:
        print(f"[build] {HIP_LIB.relative_to(ROOT)}", flush=True)
    return HIP_LIB


def _torch_paths():
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, libdir, abi


def build_torch_ext(verbose: bool = True) -> Path | None:
    sources = sorted(OPS_SRC.glob("*.cpp"))
    if not sources:
        return None
    BUILD.mkdir(exist_ok=True)
    inc, libdir, abi = _torch_paths()
    py_inc = sysconfig.get_paths()["include"]
    flags = [
        "-O2", "-std=c++17", "-fPIC", "-fopenmp", "-ffp-contract=off", "-Wno-unused-parameter",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C", *[f"-I{p}" for p in inc], f"-I{py_inc}",
        "-I/opt/rocm/include", f"-I{INCLUDE}", f"-I{OPS_SRC}",
    ]
    objs = [BUILD / (s.stem + ".cpp.o") for s in sources]
    with cf.ThreadPoolExecutor(_jobs()) as ex:
        futs = [ex.submit(_run, [CXX, *flags, "-c", str(s), "-o", str(o)])
                for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = EXT_LIB.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-fopenmp", *map(str, objs), "-o", str(tmp),
          f"-L{libdir}", f"-L{PKG}", "-ltorchpairwise_hip", "-lc10", "-ltorch", "-ltorch_cpu",
          "-lc10_hip", "-ltorch_hip", f"-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"])
    os.replace(tmp, EXT_LIB)
    if verbose:
        print(f"[build] {EXT_LIB.relative_to(ROOT)}", flush=True)
    return EXT_LIB


def build_all(verbose: bool = True) -> None:
    build_hip_lib(verbose)
    build_torch_ext(verbose)


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    {"hip": build_hip_lib, "ext": build_torch_ext, "all": build_all}[what]()
