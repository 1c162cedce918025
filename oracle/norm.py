"""Float64 CPU restatement of the RMSNorm in front of the router -- TEST INFRASTRUCTURE ONLY.

Reference: ``moe-engine/pkg/models/moe.py`` L:63-86 (``RMSNorm``) and L:125-126 (``ToyMoEBlock.forward``:
``x + moe(norm(x))``).

Pinning (each checked in ``tests/test_oracle_norm.py``):

* ``rmsnorm_fwd`` -- closed forms: a row of constant value c maps to sign(c) * weight / sqrt(1 + eps / c^2);
  rows of unit RMS pass through scaled by ``weight`` up to eps; ``norm(a x) = norm(x)`` for a > 0 up to eps;
  the output has RMS ~1 before ``weight``; and ``torch.rsqrt`` / ``mean`` in float64 (library routines).
* ``rmsnorm_bwd`` -- the closed-form gradient below against torch autograd through the float64 forward, and
  against central finite differences on a tiny case.
* ``rmsnorm_to`` -- the dtype cast of the reference (``.to(x.dtype)``): bf16 rounding of the float64 value.
"""

from __future__ import annotations

from typing import Tuple

import torch

_F64 = torch.float64


def rmsnorm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(x * rsqrt(mean(x^2, -1) + eps)) * weight`` in float64 (moe.py L:83-86, without the final cast).

    Returns ``(y float64 [N, H], rstd float64 [N])``."""
    v = x.to(_F64)
    rstd = torch.rsqrt(v.pow(2).mean(-1) + eps)
    return (v * rstd[:, None]) * weight.to(_F64), rstd


def rmsnorm_to(y: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The reference's ``.to(x.dtype)`` of the float64 result (moe.py L:86)."""
    return y.to(dtype)


def rmsnorm_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, eps: float = 1e-5):
    """Gradients of ``sum(dy * rmsnorm_fwd(x, weight))`` in float64, by the closed form

        xhat = x r,  r = (mean(x^2) + eps)^(-1/2),  g = weight * dy
        dx = r * (g - xhat * mean(g * xhat)),   dweight = sum_t dy * xhat

    Returns ``(dx, dweight)`` in float64."""
    v = x.to(_F64)
    w = weight.to(_F64)
    g_out = dy.to(_F64)
    r = torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    xhat = v * r
    g = w * g_out
    dx = r * (g - xhat * (g * xhat).mean(-1, keepdim=True))
    dweight = (g_out * xhat).sum(0)
    return dx, dweight
