"""tpw_directed_hausdorff_noalloc (the allocation-free entry point, scratch in a static device
array) against tpw_directed_hausdorff (caller workspace): value and both indices bit for bit,
on two calls in a row, the second smaller than the first, so stale scratch from the first call
cannot leak into the second; overlapping calls on two streams; the scratch loaded only by the
entry point's callers; plus the size limit."""
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
    # call 1: the C5 shape (16 x 65536 points per side, d = 3: 45 MiB of scratch)
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


@pytest.mark.gpu
def test_noalloc_calls_on_two_streams_are_serialised():
    """A large call on one stream and a smaller one on another stream, enqueued back to back
    with no host synchronisation: the second waits for the first (the per-device event), so
    neither overwrites the other's scratch; both equal the workspace entry point's results."""
    x1 = rand(16, 65536, 3, seed=10).to(DEV)
    x2 = (rand(16, 65536, 3, seed=11) + 0.05).to(DEV)
    y1 = rand(4, 3000, 3, seed=12).to(DEV)
    y2 = (rand(5, 2000, 3, seed=13) + 0.01).to(DEV)
    want_x = capi.directed_hausdorff(x1, x2)
    want_y = capi.directed_hausdorff(y1, y2)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    print("[noalloc] two streams: [16, 65536, 3]^2 on s1, [4, 3000, 3] x [5, 2000, 3] on s2", flush=True)
    with torch.cuda.stream(s1):
        got_x = capi.directed_hausdorff(x1, x2, noalloc=True)
    with torch.cuda.stream(s2):
        got_y = capi.directed_hausdorff(y1, y2, noalloc=True)
    torch.cuda.synchronize()
    for got, want, case in ((got_x, want_x, "s1"), (got_y, want_y, "s2")):
        for o, r, what in zip(got, want, ("value", "x1 index", "x2 index")):
            assert_equal(o, r, f"{case} {what}")


@pytest.mark.gpu
def test_noalloc_scratch_is_held_only_by_callers_of_the_entry_point():
    """In a fresh process the other kernels (euclidean, manhattan, the workspace Hausdorff) leave
    the static scratch unloaded; the first no-alloc call loads it (device memory drops by about
    its size), the second loads nothing more."""
    import subprocess
    import sys
    from pathlib import Path

    code = (
        "import sys, torch\n"
        f"sys.path.insert(0, {str(Path(__file__).resolve().parent.parent)!r})\n"
        "import torchpairwise_amd as tp\n"
        "from torchpairwise_amd import _capi as capi\n"
        "free = lambda: torch.cuda.mem_get_info()[0]\n"
        "x = torch.randn(256, 64, device='cuda'); tp.euclidean_distances(x, x); tp.manhattan_distances(x, x)\n"
        "y1 = torch.rand(2, 100, 3, device='cuda'); y2 = torch.rand(2, 120, 3, device='cuda')\n"
        "capi.directed_hausdorff(y1, y2); torch.cuda.synchronize()\n"
        "a = free(); capi.directed_hausdorff(y1, y2, noalloc=True); torch.cuda.synchronize(); b = free()\n"
        "capi.directed_hausdorff(y1, y2, noalloc=True); torch.cuda.synchronize(); c = free()\n"
        "print(a - b, b - c)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    first, second = map(int, r.stdout.split()[-2:])
    assert first >= LIMIT and first < LIMIT + (16 << 20), first
    assert second == 0, second


def test_noalloc_rejects_sizes_beyond_the_buffer():
    l = capi.lib()
    big = (1, 1, 1 << 22, 1, 1 << 22, 3)
    assert l.tpw_hausdorff_workspace_size(*big) > LIMIT
    rc = l.tpw_directed_hausdorff_noalloc(None, None, *big, None, None, None, None, None, None)
    assert rc == 1
    assert b"static buffer" in l.tpw_last_error()
    assert l.tpw_hausdorff_workspace_size(1, 16, 65536, 16, 65536, 3) <= LIMIT
