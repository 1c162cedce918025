"""Shared helpers for the GPU parity tests (imported by tests only)."""

from __future__ import annotations

import sys

import torch


def dev() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run on a host without a ROCm GPU")
    return torch.device("cuda:0")


def say(*a) -> None:
    """Name the case before a GPU step (flushed, so a fault still leaves the name)."""
    print(*a, file=sys.stderr, flush=True)


def rel_err(a: torch.Tensor, b: torch.Tensor, floor: float = 0.0) -> float:
    """max|a-b| / max(max|b|, floor) (max-norm relative error), float64 on the CPU.

    ``floor`` keeps the measure meaningful when the exact result is zero up to
    rounding (e.g. K=1 routing, where the combine weight is identically 1)."""
    a = a.detach().to("cpu", torch.float64)
    b = b.detach().to("cpu", torch.float64)
    den = max(b.abs().max().item() if b.numel() else 0.0, floor)
    if den == 0.0:
        return a.abs().max().item() if a.numel() else 0.0
    return (a - b).abs().max().item() / den


def assert_rel(a: torch.Tensor, b: torch.Tensor, tol: float, what: str = "", floor: float = 0.0) -> None:
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    e = rel_err(a, b, floor)
    assert e <= tol, f"{what}: max-norm relative error {e:.3e} > {tol:.1e}"


# Tolerances stated by the north star: fp32 1e-5 relative, bf16 2e-2 relative.
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
# Index parity is asserted wherever the fp64 top-k probability margin exceeds this.
MARGIN = 1e-6
