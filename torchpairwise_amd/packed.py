"""Persistent bit-packed boolean rows.

``PackedBool.pack(x)`` packs boolean rows ``[(B,) N, D]`` once into 32-bit words (bit k of a
row is bit ``k % 32`` of word ``k // 32``, zero padding, ``torchpairwise_amd._capi`` /
``tpw_packed_words(D)`` words per row, a multiple of 4) and caches each row's popcount.  The
metric functions of this module take packed operands and run one pass per call, with no
pack step, on the GPU kernel that serves the public boolean metrics.  Results are
bit-identical to the public functions on the unpacked rows
(``torchpairwise.<metric>_distances``, ``pairwise_metrics.cpp:206-243,339-399``, and the pw
reductions of ``pairwise_binary.cpp:91-134``).  Non-bool rows are coerced with
``x.to(torch.bool)``, as the public boolean metrics coerce them.
"""
from __future__ import annotations

import torch

__all__ = ["PackedBool", "cdist", "METRICS"]

METRICS = ("hamming", "jaccard", "dice", "kulczynski1", "kulsinski", "rogerstanimoto",
           "russellrao", "sokalmichener", "sokalsneath", "yule",
           "pwand_sum", "pwor_sum", "pwxor_sum", "pweq_sum", "pwne_sum", "pweq_mean", "pwne_mean")


class PackedBool:
    """Bit-packed boolean rows with cached row popcounts (see the module docstring)."""

    __slots__ = ("words", "popcounts", "d")

    def __init__(self, words: torch.Tensor, popcounts: torch.Tensor, d: int):
        self.words, self.popcounts, self.d = words, popcounts, int(d)

    @classmethod
    def pack(cls, x: torch.Tensor) -> "PackedBool":
        if x.dtype != torch.bool:
            x = x.to(torch.bool)
        words, pops = torch.ops.torchpairwise._pack_bool(x)
        return cls(words, pops, x.shape[-1])

    @property
    def shape(self) -> torch.Size:
        """Shape of the unpacked rows, ``[(B,) N, D]``."""
        return torch.Size((*self.words.shape[:-1], self.d))

    @property
    def device(self) -> torch.device:
        return self.words.device

    def to(self, device) -> "PackedBool":
        return PackedBool(self.words.to(device), self.popcounts.to(device), self.d)

    def unpack(self) -> torch.Tensor:
        """The boolean rows again."""
        shifts = torch.arange(32, device=self.words.device, dtype=torch.int32)
        bits = (self.words.unsqueeze(-1) >> shifts) & 1
        return bits.flatten(-2)[..., :self.d].to(torch.bool)


def _metric(metric: str, x1: PackedBool, x2: PackedBool | None) -> torch.Tensor:
    if not isinstance(x1, PackedBool) or not (x2 is None or isinstance(x2, PackedBool)):
        raise TypeError("packed metrics take PackedBool operands (PackedBool.pack(x))")
    x2 = x1 if x2 is None else x2
    if x1.d != x2.d:
        raise RuntimeError(f"feature dimension of x1 and x2 do not match ({x1.d} vs {x2.d}).")
    return torch.ops.torchpairwise._packed_bool_metric(x1.words, x1.popcounts, x2.words,
                                                       x2.popcounts, x1.d, metric)


def cdist(x1: PackedBool, x2: PackedBool | None = None, metric: str = "hamming") -> torch.Tensor:
    """``metric`` (one of ``METRICS``) between packed rows; x2 = None means x1."""
    return _metric(metric, x1, x2)


def _bind(metric: str):
    name = metric if metric.startswith("pw") else f"{metric}_distances"

    def fn(x1: PackedBool, x2: PackedBool | None = None) -> torch.Tensor:
        return _metric(metric, x1, x2)

    fn.__name__ = name
    fn.__doc__ = f"``torchpairwise.{name}`` of packed rows (one pass, no pack step)."
    return name, fn


for _m in METRICS:
    _n, _f = _bind(_m)
    globals()[_n] = _f
    __all__.append(_n)
