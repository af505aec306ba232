"""The launch timer the benchmark reads its roofline durations from: one event pair per launch
of the armed kernel family, none for other families, each launch's duration inside the
caller's own events around it."""
import pytest
import torch

from tests._util import randn
from torchpairwise_amd import _capi as capi

pytestmark = pytest.mark.gpu


def test_launch_timer_times_each_launch_of_its_family():
    x1 = randn(1024, 128, seed=0).cuda()
    x2 = randn(2048, 128, seed=1).cuda()
    n1, n2 = capi.row_norms(x1, True), capi.row_norms(x2, True)
    stream = torch.cuda.current_stream()
    outer = []
    timer = capi.LaunchTimer("inner_tile_kernel", 8).arm()
    for _ in range(3):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        capi.pairwise_inner(x1, x2, capi.EPI_EUCLIDEAN, n1, n2)
        capi.row_norms(x1, True)  # another family: not recorded
        e.record(stream)
        outer.append((s, e))
    torch.cuda.synchronize()
    ms, dropped = timer.read()
    assert len(ms) == 3 and dropped == 0
    for k, (s, e) in zip(ms, outer):
        assert 0.0 < k <= s.elapsed_time(e)
    # disarmed after the read: further launches are not recorded
    capi.pairwise_inner(x1, x2, capi.EPI_EUCLIDEAN, n1, n2)
    torch.cuda.synchronize()
    assert capi.LaunchTimer("inner_tile_kernel", 8).read() == ([], 0)


def test_launch_timer_counts_launches_past_its_capacity():
    x1 = randn(256, 64, seed=0).cuda()
    x2 = randn(256, 64, seed=1).cuda()
    timer = capi.LaunchTimer("lp_forward_kernel", 2).arm()
    for _ in range(5):
        capi.lp_distances(x1, x2, 1.0)
    torch.cuda.synchronize()
    ms, dropped = timer.read()
    assert len(ms) == 2 and dropped == 3 and all(v > 0 for v in ms)
