"""Pins the float64 layer oracle against per-token brute-force loops (CPU only)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as L
from oracle import plan as P

pytestmark = pytest.mark.cpu


def _weights(E, H, Fd, seed):
    g = torch.Generator().manual_seed(seed)
    wg = torch.randn(E, Fd, H, generator=g, dtype=torch.float64) / math.sqrt(H)
    wu = torch.randn(E, Fd, H, generator=g, dtype=torch.float64) / math.sqrt(H)
    wd = torch.randn(E, H, Fd, generator=g, dtype=torch.float64) / math.sqrt(Fd)
    return wg, wu, wd


def _expert(x, wg, wu, wd):
    h = x @ wg.t()
    return (h * torch.sigmoid(h) * (x @ wu.t())) @ wd.t()


@pytest.mark.parametrize("N,H,Fd,E,K,cf,drop", [(12, 8, 16, 4, 2, 1.25, False), (9, 8, 6, 4, 3, 0.5, True), (5, 4, 4, 8, 2, 1.0, False)])
def test_reference_layout_brute_force(N, H, Fd, E, K, cf, drop):
    torch.manual_seed(N)
    x = torch.randn(N, H, dtype=torch.float64)
    gw = torch.randn(H, E, dtype=torch.float64)
    wg, wu, wd = _weights(E, H, Fd, 1)
    res = L.layer_fwd_bwd(x, gw, wg, wu, wd, K, capacity_factor=cf, capacity_dropping=drop)
    idx = res["idx"].numpy()
    p = torch.softmax(x @ gw, -1)
    w = p.gather(1, res["idx"])
    w = w / w.sum(-1, keepdim=True)
    if drop:
        cap = math.ceil(cf * N * K / E)
        w = w.masked_fill(torch.from_numpy(P.drop_mask(idx, cap)), 0.0)
    # the reference's positional semantics written out token by token
    order = sorted(range(N), key=lambda t: (idx[t, 0], t))
    chunk = max(1, N * K // E)
    out = torch.zeros(N, H, dtype=torch.float64)
    for j, t in enumerate(order):
        for k in range(K):
            r = j * K + k
            e = r // chunk
            if e < E:
                out[t] += w[t, k] * _expert(x[t], wg[e], wu[e], wd[e])
    torch.testing.assert_close(res["out"], out, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("drop", [False, True])
def test_routed_layout_brute_force(drop):
    torch.manual_seed(3)
    N, H, Fd, E, K = 20, 8, 12, 5, 2
    x = torch.randn(N, H, dtype=torch.float64)
    gw = torch.randn(H, E, dtype=torch.float64)
    wg, wu, wd = _weights(E, H, Fd, 2)
    res = L.layer_fwd_bwd(x, gw, wg, wu, wd, K, capacity_factor=0.6, capacity_dropping=drop, layout=P.LAYOUT_ROUTED)
    idx = res["idx"]
    p = torch.softmax(x @ gw, -1)
    w = p.gather(1, idx)
    w = w / w.sum(-1, keepdim=True)
    dm = torch.zeros(N, K, dtype=torch.bool)
    if drop:
        dm = torch.from_numpy(P.drop_mask(idx.numpy(), math.ceil(0.6 * N * K / E)))
    out = torch.zeros(N, H, dtype=torch.float64)
    for t in range(N):
        for k in range(K):
            if not dm[t, k]:
                e = int(idx[t, k])
                out[t] += w[t, k] * _expert(x[t], wg[e], wu[e], wd[e])
    torch.testing.assert_close(res["out"], out, atol=1e-12, rtol=1e-12)


def test_layer_backward_finite_difference():
    torch.manual_seed(4)
    N, H, Fd, E, K = 6, 4, 5, 3, 2
    x = torch.randn(N, H, dtype=torch.float64)
    gw = torch.randn(H, E, dtype=torch.float64)
    wg, wu, wd = _weights(E, H, Fd, 3)
    g = torch.randn(N, H, dtype=torch.float64)
    res = L.layer_fwd_bwd(x, gw, wg, wu, wd, K, grad_out=g, layout=P.LAYOUT_ROUTED, alpha=0.01, beta=1e-3)
    idx = res["idx"]
    eps = 1e-6

    def loss(xx):
        r = L.layer_fwd_bwd(xx, gw, wg, wu, wd, K, layout=P.LAYOUT_ROUTED, alpha=0.01, beta=1e-3, idx_override=idx)
        return float((r["out"] * g).sum() + r["aux"] + r["z"])

    fd = torch.zeros_like(x)
    for i in range(N):
        for j in range(H):
            xp = x.clone(); xp[i, j] += eps
            xm = x.clone(); xm[i, j] -= eps
            fd[i, j] = (loss(xp) - loss(xm)) / (2 * eps)
    torch.testing.assert_close(res["dx"], fd, atol=1e-6, rtol=1e-6)
