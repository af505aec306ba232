"""Shared helpers of the test-suite (tolerance checks, seeded inputs)."""
from __future__ import annotations

import os

import torch


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(*shape, seed: int, dtype=torch.float32):
    return torch.randn(*shape, generator=gen(seed), dtype=torch.float32).to(dtype)


def rand(*shape, seed: int):
    return torch.rand(*shape, generator=gen(seed), dtype=torch.float32)


def assert_close(actual, expected, *, rtol: float, atol: float, what: str = ""):
    """|actual - expected| <= atol + rtol * |expected| elementwise (both moved to CPU
    float64; ``atol`` may be a per-element tensor); the message names the worst element."""
    a = torch.as_tensor(actual).detach().cpu().double()
    e = torch.as_tensor(expected).detach().cpu().double()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    diff = (a - e).abs()
    if torch.is_tensor(atol):
        atol = atol.detach().cpu().double()
    tol = atol + rtol * e.abs()
    bad = ~(diff <= tol)
    if os.environ.get("TPW_TOL_REPORT"):
        # the smallest r with diff <= r * (|want| + max|want|): the rtol this check needs when its
        # atol is rtol * max|want|
        need = float((diff / (e.abs() + e.abs().max() + 1e-300)).max()) if diff.numel() else 0.0
        print(f"[tol] {what}: rtol={rtol} needs {need:.3g}", flush=True)
    if bad.any():
        idx = int(torch.argmax((diff - tol).flatten()))
        at = float(atol.flatten()[idx]) if torch.is_tensor(atol) and atol.numel() > 1 else float(atol)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} elements beyond rtol={rtol} atol={at}; "
            f"worst at flat {idx}: got {a.flatten()[idx].item()!r} want {e.flatten()[idx].item()!r}")


def assert_equal(actual, expected, what: str = "", nan_payload: bool = True):
    """Bit-for-bit equality; with ``nan_payload=False`` NaNs must sit at the same positions but
    may differ in sign and payload (devices produce different NaN bit patterns for 0 / 0)."""
    a = torch.as_tensor(actual).detach().cpu()
    e = torch.as_tensor(expected).detach().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    if a.dtype.is_floating_point:
        iv = {2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
        same = a.view(iv) == e.to(a.dtype).view(iv)
        if not nan_payload:
            same = same | (torch.isnan(a) & torch.isnan(e.to(a.dtype)))
    else:
        same = a == e
    if not bool(same.all()):
        idx = int(torch.nonzero(~same.flatten())[0])
        raise AssertionError(f"{what}: {int((~same).sum())}/{same.numel()} differ; first at flat {idx}: "
                             f"got {a.flatten()[idx].item()!r} want {e.flatten()[idx].item()!r}")
