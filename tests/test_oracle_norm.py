"""The float64 RMSNorm oracle (oracle/norm.py) against closed forms, torch autograd and finite differences
(the reference has no test of RMSNorm values: moe-engine/pkg/models/moe.py L:63-86 defines it)."""

from __future__ import annotations

import math

import torch

from oracle import norm as ON


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_constant_rows_closed_form():
    H, eps = 64, 1e-5
    x = torch.tensor([[2.0] * H, [-0.5] * H, [1e-3] * H], dtype=torch.float64)
    w = torch.linspace(0.5, 1.5, H)
    y, rstd = ON.rmsnorm_fwd(x, w, eps)
    for i, c in enumerate([2.0, -0.5, 1e-3]):
        expect = math.copysign(1.0, c) / math.sqrt(1.0 + eps / (c * c))
        assert torch.allclose(y[i], expect * w.double(), rtol=1e-12, atol=0)
        assert abs(rstd[i].item() - 1.0 / math.sqrt(c * c + eps)) < 1e-12 / abs(c)


def test_unit_rms_rows_and_scale_invariance():
    H = 128
    x = torch.randn(16, H, generator=_g(1), dtype=torch.float64)
    x = x / x.pow(2).mean(-1, keepdim=True).sqrt()  # RMS exactly 1
    w = torch.rand(H, generator=_g(2), dtype=torch.float64) + 0.5
    y, _ = ON.rmsnorm_fwd(x, w, eps=0.0)
    assert torch.allclose(y, x * w, rtol=1e-12, atol=1e-12)
    y2, _ = ON.rmsnorm_fwd(7.5 * x, w, eps=0.0)
    assert torch.allclose(y2, y, rtol=1e-12, atol=1e-12)
    # before the weight the output has RMS ~1 (eps small next to the row's mean square)
    z, _ = ON.rmsnorm_fwd(3.0 * torch.randn(8, H, generator=_g(3)), torch.ones(H), eps=1e-5)
    assert torch.allclose(z.pow(2).mean(-1), torch.ones(8, dtype=torch.float64), rtol=1e-5)


def test_backward_matches_autograd():
    N, H, eps = 12, 96, 1e-5
    x = torch.randn(N, H, generator=_g(4), dtype=torch.float64, requires_grad=True)
    w = (torch.rand(H, generator=_g(5), dtype=torch.float64) + 0.5).requires_grad_(True)
    dy = torch.randn(N, H, generator=_g(6), dtype=torch.float64)
    v = x
    y = (v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)) * w
    (y * dy).sum().backward()
    dx, dw = ON.rmsnorm_bwd(x.detach(), w.detach(), dy, eps)
    assert torch.allclose(dx, x.grad, rtol=1e-10, atol=1e-12)
    assert torch.allclose(dw, w.grad, rtol=1e-10, atol=1e-12)


def test_backward_finite_differences():
    N, H, eps, h = 3, 16, 1e-5, 1e-6
    x = torch.randn(N, H, generator=_g(7), dtype=torch.float64)
    w = torch.rand(H, generator=_g(8), dtype=torch.float64) + 0.5
    dy = torch.randn(N, H, generator=_g(9), dtype=torch.float64)
    dx, dw = ON.rmsnorm_bwd(x, w, dy, eps)

    def f(xx, ww):
        return float((ON.rmsnorm_fwd(xx, ww, eps)[0] * dy).sum())

    for (i, j) in [(0, 0), (1, 7), (2, 15)]:
        e = torch.zeros_like(x)
        e[i, j] = h
        assert abs((f(x + e, w) - f(x - e, w)) / (2 * h) - dx[i, j].item()) < 1e-6
    for j in [0, 5, 15]:
        e = torch.zeros_like(w)
        e[j] = h
        assert abs((f(x, w + e) - f(x, w - e)) / (2 * h) - dw[j].item()) < 1e-6


def test_planted_mistake_is_caught():
    """A backward missing the mean-projection term disagrees with autograd."""
    N, H, eps = 4, 32, 1e-5
    x = torch.randn(N, H, generator=_g(10), dtype=torch.float64)
    w = torch.ones(H, dtype=torch.float64)
    dy = torch.randn(N, H, generator=_g(11), dtype=torch.float64)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    wrong = r * (w * dy)  # dropped term
    dx, _ = ON.rmsnorm_bwd(x, w, dy, eps)
    assert (wrong - dx).abs().max() > 1e-3
