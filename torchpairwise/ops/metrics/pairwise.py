"""Module attributes equal to ``torch.ops.torchpairwise.<name>`` for the metric names the
reference binds (torchpairwise/ops/metrics/pairwise.py:4-47; ``linf_distances`` is registered
but not bound there, and is bound here too)."""
import torch

from torchpairwise_amd.ops import _METRICS

for _name in _METRICS:
    globals()[_name] = getattr(torch.ops.torchpairwise, _name)

__all__ = list(_METRICS)
