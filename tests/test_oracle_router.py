"""Pins the float64 router oracle against the reference's own known answers,
library routines and torch autograd (CPU only)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import router as R

pytestmark = pytest.mark.cpu


@pytest.mark.parametrize("B,S,H,E,K", [(2, 16, 64, 8, 2), (1, 32, 128, 16, 1), (4, 8, 64, 32, 4)])
def test_forward_matches_library_topk(B, S, H, E, K):
    # Shapes of the reference's test_forward_tolerance (tests/test_kernels.py L:32-59).
    torch.manual_seed(0)
    tokens = torch.randn(B * S, H, dtype=torch.float64)
    gate_w = torch.randn(H, E, dtype=torch.float64) * (1.0 / math.sqrt(H))
    out = R.route_fwd(tokens, gate_w, K)
    probs = torch.softmax(tokens @ gate_w, dim=-1)
    vals, idx = torch.topk(probs, k=K, dim=-1, largest=True)
    ok = out["margin"] > 0
    assert torch.equal(out["idx"][ok], idx[ok])
    ref_w = vals / vals.sum(-1, keepdim=True)
    torch.testing.assert_close(out["w"], ref_w, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(out["w"].sum(-1), torch.ones(B * S, dtype=torch.float64))


def test_tie_break_lowest_index():
    probs = torch.tensor([[0.25, 0.25, 0.25, 0.25], [0.1, 0.3, 0.3, 0.3]], dtype=torch.float64)
    _, idx = R.topk_lowest_index(probs, 2)
    assert idx.tolist() == [[0, 1], [1, 2]]


@pytest.mark.parametrize("B,S,H,E,K", [(2, 8, 32, 8, 2), (1, 16, 64, 16, 2), (1, 16, 32, 8, 3)])
def test_backward_matches_autograd(B, S, H, E, K):
    # The reference's test_backward_tolerance (tests/test_kernels.py L:62-108).
    torch.manual_seed(7)
    N = B * S
    tokens = torch.randn(N, H, dtype=torch.float64, requires_grad=True)
    gate_w = (torch.randn(H, E, dtype=torch.float64) / math.sqrt(H)).requires_grad_(True)
    probs = torch.softmax(tokens @ gate_w, -1)
    vals, idx = torch.topk(probs, K, -1)
    w = vals / vals.sum(-1, keepdim=True).clamp_min(1e-30)
    g = torch.randn_like(w)
    (w * g).sum().backward()
    out = R.router_full(tokens, gate_w, K, grad_w=g)
    torch.testing.assert_close(out["dX"], tokens.grad, atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(out["dW"], gate_w.grad, atol=1e-10, rtol=1e-10)


def test_backward_constant_upstream_is_zero():
    # w sums to one per token, so a per-token constant upstream gradient has no effect.
    torch.manual_seed(3)
    x = torch.randn(32, 16, dtype=torch.float64)
    W = torch.randn(16, 8, dtype=torch.float64) * 0.3
    out = R.router_full(x, W, 2, grad_w=torch.ones(32, 2, dtype=torch.float64) * 2.5)
    assert out["grad_logits"].abs().max() < 1e-12


def test_planted_mistake_in_backward_is_caught():
    # Dropping the -<gw,v>/S^2 term must break agreement with autograd.
    torch.manual_seed(11)
    x = torch.randn(16, 32, dtype=torch.float64, requires_grad=True)
    W = (torch.randn(32, 8, dtype=torch.float64) * 0.2).requires_grad_(True)
    p = torch.softmax(x @ W, -1)
    vals, idx = torch.topk(p, 2, -1)
    w = vals / vals.sum(-1, keepdim=True)
    g = torch.randn_like(w)
    (w * g).sum().backward()
    pd = p.detach()
    v = pd.gather(1, idx)
    S = v.sum(-1, keepdim=True)
    grad_p = torch.zeros_like(pd).scatter_add_(1, idx, g / S)  # mutated: term dropped
    G = pd * (grad_p - (grad_p * pd).sum(-1, keepdim=True))
    assert not torch.allclose(G @ W.detach().t(), x.grad, atol=1e-6)


@pytest.mark.parametrize(
    "cnt,expected",
    [([10, 10, 10, 10], 1.0), ([100, 0, 0, 0], 4.0), ([30, 10, 20, 40], 1.6), ([0] * 8, 1.0)],
)
def test_load_imbalance_golden(cnt, expected):
    # tests/test_routing_quality.py L:36-60
    assert abs(R.load_imbalance(torch.tensor(cnt)) - expected) < 1e-12


def test_z_stat_zero_logits():
    # tests/test_routing_quality.py L:75-81
    E = 16
    assert abs(R.z_stat(torch.zeros(32, E)) - math.log(E) ** 2) < 1e-12


def test_z_stat_matches_logsumexp():
    torch.manual_seed(0)
    l = torch.randn(64, 32, dtype=torch.float64) * 3
    lse = torch.logsumexp(l, -1)
    assert abs(R.z_stat(l) - float((lse**2).mean())) < 1e-12


@pytest.mark.parametrize("N,E,K", [(64, 8, 2), (40, 16, 4), (12, 4, 4)])
def test_aux_and_z_grads_match_autograd(N, E, K):
    torch.manual_seed(5)
    alpha, beta = 0.01, 1e-3
    logits = (torch.randn(N, E, dtype=torch.float64) * 2).requires_grad_(True)
    probs = torch.softmax(logits, -1)
    _, idx = torch.topk(probs.detach(), K, -1)
    cnt = torch.bincount(idx.reshape(-1), minlength=E)
    loss = R.aux_loss(probs, cnt, K, alpha) + R.z_loss(logits, beta)
    loss.backward()
    G = R.aux_grad_logits(probs.detach(), cnt, K, alpha) + R.z_grad_logits(logits.detach(), beta)
    torch.testing.assert_close(G, logits.grad, atol=1e-14, rtol=1e-10)
    # closed form values
    f = cnt.double() / (N * K)
    P = probs.detach().mean(0)
    assert abs(float(R.aux_loss(probs.detach(), cnt, K, alpha)) - alpha * E * float((f * P).sum())) < 1e-15


def test_aux_loss_uniform_is_alpha():
    # Perfectly uniform routing (f_e = P_e = 1/E) gives aux = alpha.
    N, E, K = 64, 8, 2
    probs = torch.full((N, E), 1.0 / E, dtype=torch.float64)
    cnt = torch.full((E,), N * K // E)
    assert abs(float(R.aux_loss(probs, cnt, K, 0.01)) - 0.01) < 1e-15


@pytest.mark.parametrize(
    "N,E,K,cf,expected",
    [(64, 8, 2, 1.25, 20), (32, 8, 2, 1.25, 10), (100, 10, 2, 1.0, 20), (100, 10, 2, 1.25, 25), (100, 7, 2, 1.0, 29)],
)
def test_capacity_budget_table(N, E, K, cf, expected):
    # tests/test_router.py L:226-241
    assert R.capacity_budget(N, K, E, cf) == expected
