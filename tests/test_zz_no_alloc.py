"""tpw_directed_hausdorff_noalloc (the allocation-free entry point, scratch in a static device
array) against tpw_directed_hausdorff (caller workspace): value and both indices bit for bit,
on two calls in a row, the second smaller than the first, so stale scratch from the first call
cannot leak into the second; plus the size limit."""
import numpy as np
import pytest
import torch

from oracle import cref
from torchpairwise_amd import _capi as capi
from tests._util import assert_equal, rand

DEV = "cuda"
LIMIT = 96 << 20


def _both(x1, x2, perm1=None, perm2=None):
    ref = capi.directed_hausdorff(x1, x2, perm1, perm2)
    got = capi.directed_hausdorff(x1, x2, perm1, perm2, noalloc=True)
    torch.cuda.synchronize()
    for r, o, what in zip(ref, got, ("value", "x1 index", "x2 index")):
        assert_equal(o, r, what)
    return got


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point_twice():
    # call 1: the C5 shape (16 x 65536 points per side, d = 3: 67 MiB of scratch)
    x1 = rand(16, 65536, 3, seed=0)
    x2 = rand(16, 65536, 3, seed=1) + 0.05
    print("[noalloc] call 1: [16, 65536, 3] x [16, 65536, 3]", flush=True)
    o, i1, i2 = _both(x1.to(DEV), x2.to(DEV))
    w = cref.directed_hausdorff(x1[:2].numpy(), x2[:3].numpy(), threads=8)
    assert np.array_equal(o[:2, :3].cpu().numpy(), w[0]) and np.array_equal(i1[:2, :3].cpu().numpy(), w[1])
    # call 2, smaller and batched, in a shuffled order: the scratch still holds call 1's data
    y1 = rand(2, 3, 5000, 3, seed=2)
    y2 = rand(2, 2, 7000, 3, seed=3) + 0.02
    g = torch.Generator().manual_seed(4)
    p1 = torch.stack([torch.randperm(5000, generator=g) for _ in range(2)])
    p2 = torch.stack([torch.randperm(7000, generator=g) for _ in range(2)])
    print("[noalloc] call 2: [2, 3, 5000, 3] x [2, 2, 7000, 3], shuffled", flush=True)
    o, i1, i2 = _both(y1.to(DEV), y2.to(DEV), p1.to(DEV), p2.to(DEV))
    w = cref.directed_hausdorff(y1.numpy(), y2.numpy(), p1.numpy(), p2.numpy(), threads=8)
    assert_equal(o, torch.from_numpy(w[0]), "call 2 value vs the C loop")
    assert np.array_equal(i1.cpu().numpy(), w[1]) and np.array_equal(i2.cpu().numpy(), w[2])
    # call 3: d = 5 (the path without the cell grid)
    z1, z2 = rand(3, 900, 5, seed=5), rand(2, 700, 5, seed=6)
    print("[noalloc] call 3: [3, 900, 5] x [2, 700, 5]", flush=True)
    _both(z1.to(DEV), z2.to(DEV))


def test_noalloc_rejects_sizes_beyond_the_buffer():
    l = capi.lib()
    big = (1, 1, 1 << 21, 1, 1 << 21, 3)
    assert l.tpw_hausdorff_workspace_size(*big) > LIMIT
    rc = l.tpw_directed_hausdorff_noalloc(None, None, *big, None, None, None, None, None, None)
    assert rc == 1
    assert b"static buffer" in l.tpw_last_error()
    assert l.tpw_hausdorff_workspace_size(1, 16, 65536, 16, 65536, 3) <= LIMIT
