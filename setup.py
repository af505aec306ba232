"""Installs the drop-in package ``torchpairwise`` (the reference's import name and module
layout) together with ``torchpairwise_amd``, whose native libraries are compiled in-tree for
gfx950 by ``torchpairwise_amd/_build.py`` (hipcc for the kernels, g++ against the installed
torch for the extension) and shipped as package data.

    pip install --no-build-isolation --no-deps .

With TPW_USE_BUILT=1 the libraries already built in ``torchpairwise_amd/`` are packaged as
they are instead of being rebuilt.
"""
import importlib.util
import os
from pathlib import Path

from setuptools import Distribution, setup
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent
NATIVE = ("libtorchpairwise_hip.so", "_C.so")


class BuildNative(build_py):
    """Builds the native libraries before the package files are collected."""

    def run(self):
        pkg = ROOT / "torchpairwise_amd"
        reuse = os.environ.get("TPW_USE_BUILT") == "1" and all((pkg / f).exists() for f in NATIVE)
        if not reuse:
            spec = importlib.util.spec_from_file_location("_tpw_build", pkg / "_build.py")
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            mod.build_all(verbose=True)
        super().run()


class BinaryDistribution(Distribution):
    """The packages carry compiled libraries: platform-specific wheels."""

    def has_ext_modules(self):
        return True


setup(
    name="torchpairwise",
    version="0.3.0+mi355x",
    description="Pairwise metrics for PyTorch on MI355X (gfx950): the torchpairwise operator "
                "interface over hand-written HIP kernels",
    python_requires=">=3.8",
    packages=["torchpairwise", "torchpairwise.ops", "torchpairwise.ops.metrics",
              "torchpairwise_amd", "torchpairwise_amd.ops"],
    package_data={"torchpairwise_amd": list(NATIVE),
                  "torchpairwise": ["py.typed", "ops/*.pyi", "ops/metrics/*.pyi"]},
    include_package_data=False,
    zip_safe=False,
    cmdclass={"build_py": BuildNative},
    distclass=BinaryDistribution,
)
