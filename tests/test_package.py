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
