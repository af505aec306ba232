"""`import torchpairwise` gives the reference package's surface (torchpairwise/__init__.py:1-8,
extension.py:163-192, ops/metrics/pairwise.py:4-47, ops/cpdist.py, ops/metrics/neighbors.py)."""
import re
from pathlib import Path

import torch

import torchpairwise

REF_PY = Path("/root/reference/torchpairwise")


def test_top_level_names():
    for name in ("ops", "_ops", "extension", "__version__", "has_ops", "with_cuda", "cuda_version",
                 "_HAS_OPS", "_assert_has_ops"):
        assert hasattr(torchpairwise, name), name
    assert torchpairwise.__version__ == "0.3.0"
    assert torchpairwise.has_ops() and torchpairwise._HAS_OPS
    assert isinstance(torchpairwise.cuda_version(), int) and torchpairwise.with_cuda()
    assert torchpairwise.extension.cuda_arch_list() == ["gfx950"]
    assert torchpairwise._ops.euclidean_distances._qualified_op_name == "torchpairwise::euclidean_distances"


def _bound_names():
    """Names the reference's Python package binds (its binding modules, read as text), or this
    build's list where the reference is absent."""
    files = ["ops/metrics/pairwise.py", "ops/cpdist.py", "ops/metrics/neighbors.py"]
    if not REF_PY.exists():
        from torchpairwise_amd.ops import _CPDIST, _METRICS
        return [n for n in _METRICS if n != "linf_distances"] + list(_CPDIST)
    names = []
    for f in files:
        names += re.findall(r"^(\w+)\s*=\s*torch\.ops\.torchpairwise\.(\w+)", (REF_PY / f).read_text(), re.M)
    assert all(a == b for a, b in names)
    return [a for a, _ in names]


def test_op_bindings_match_the_reference_modules():
    names = _bound_names()
    assert len(names) >= 42
    for n in names:
        op = getattr(torch.ops.torchpairwise, n)
        assert getattr(torchpairwise, n) is op, n
    assert torchpairwise.ops.metrics.pairwise.euclidean_distances is torch.ops.torchpairwise.euclidean_distances
    assert torchpairwise.ops.cpdist.cdist is torch.ops.torchpairwise.cdist
    assert torchpairwise.ops.metrics.neighbors.k_neighbors_mask is torch.ops.torchpairwise.k_neighbors_mask


def test_calls_through_the_package():
    g = torch.Generator().manual_seed(0)
    x1, x2 = torch.randn(7, 5, generator=g), torch.randn(4, 5, generator=g)
    torch.testing.assert_close(torchpairwise.euclidean_distances(x1, x2), torch.cdist(x1, x2))
    assert torchpairwise.cdist(x1, x2, "manhattan").shape == (7, 4)
    out = torchpairwise._ops.prf_ldiv(torch.tensor([2.0, 0.0]), torch.tensor([1.0, 3.0]), "identity")
    assert out.tolist() == [0.5, 3.0]


def _stub_functions():
    import ast

    pkg = Path(torchpairwise.__file__).resolve().parent
    out = {}
    for rel in ("ops/metrics/pairwise.pyi", "ops/cpdist.pyi", "ops/metrics/neighbors.pyi"):
        for node in ast.parse((pkg / rel).read_text()).body:
            if isinstance(node, ast.FunctionDef):
                out[node.name] = node
    return out


def test_stubs_match_the_registered_schemas():
    """Every bound op has a stub whose parameters (names, order, keyword-only split, defaults)
    and return arity are its registered schema's."""
    import ast

    from torchpairwise_amd.ops import _CPDIST, _METRICS

    stubs = _stub_functions()
    names = list(_METRICS) + list(_CPDIST) + ["k_neighbors_mask", "radius_neighbors_mask"]
    assert sorted(stubs) == sorted(set(names))
    for n in names:
        fn, sch = stubs[n], getattr(torch.ops.torchpairwise, n).default._schema
        pos = [a.arg for a in fn.args.args]
        kwo = [a.arg for a in fn.args.kwonlyargs]
        assert pos == [a.name for a in sch.arguments if not a.kwarg_only], n
        assert kwo == [a.name for a in sch.arguments if a.kwarg_only], n
        defaults = [ast.literal_eval(d) for d in fn.args.defaults]
        defaults = [None] * (len(pos) - len(defaults)) + defaults
        defaults += [None if d is None else ast.literal_eval(d) for d in fn.args.kw_defaults]
        for a, d in zip(sch.arguments, defaults):
            want = a.default_value if a.has_default_value() else None
            assert d == want, (n, a.name, d, want)
        ret = ast.unparse(fn.returns)
        assert ret == ("Tensor" if len(sch.returns) == 1 else f"Tuple[{', '.join(['Tensor'] * len(sch.returns))}]"), n


def test_pip_install_into_a_prefix(tmp_path):
    """`pip install` of the repository (the libraries already built in-tree, TPW_USE_BUILT=1)
    into an empty prefix; `import torchpairwise` from outside the repository then loads the
    installed package and its native libraries and computes."""
    import os
    import shutil
    import subprocess
    import sys
    import sysconfig

    root = Path(__file__).resolve().parent.parent
    src = tmp_path / "src"
    src.mkdir()
    for f in ("pyproject.toml", "setup.py"):
        shutil.copy(root / f, src / f)
    ignore = shutil.ignore_patterns("__pycache__", "*.o", "*.so.tmp")
    for d in ("torchpairwise", "torchpairwise_amd", "include"):
        shutil.copytree(root / d, src / d, ignore=ignore)
    prefix = tmp_path / "prefix"
    env = dict(os.environ, TPW_USE_BUILT="1", PIP_NO_INDEX="1")
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps",
                        "--no-index", "--prefix", str(prefix), str(src)],
                       cwd=tmp_path, env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    site = Path(sysconfig.get_path("purelib", vars={"base": str(prefix), "platbase": str(prefix)}))
    plat = Path(sysconfig.get_path("platlib", vars={"base": str(prefix), "platbase": str(prefix)}))
    code = ("import torch, torchpairwise, torchpairwise_amd\n"
            "print(torchpairwise.__file__)\nprint(torchpairwise_amd.__file__)\n"
            "x1, x2 = torch.randn(7, 5, dtype=torch.float64), torch.randn(4, 5, dtype=torch.float64)\n"
            "torch.testing.assert_close(torchpairwise.euclidean_distances(x1, x2), torch.cdist(x1, x2))\n"
            "print(torchpairwise.cdist(x1, x2, 'hamming').shape)\n")
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(str(p) for p in {site, plat}))
    r = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.split()
    assert all(str(prefix) in l for l in lines[:2]), lines
    assert lines[2:] == ["torch.Size([7,", "4])"]
    installed = Path(lines[1]).parent
    assert (installed / "libtorchpairwise_hip.so").exists() and (installed / "_C.so").exists()
    assert (Path(lines[0]).parent / "ops" / "metrics" / "pairwise.pyi").exists()
