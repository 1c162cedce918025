"""RMSNorm in front of the router on the GPU: the norm kernels, the norm fused into the router's read of the
hidden state, and ToyMoEBlock (moe-engine/pkg/models/moe.py L:63-126), against the float64 oracle.

Bars (north star): fp32 1e-5 and bf16 2e-2 max-norm relative error; top-k indices and dispatch counts
bit-exact wherever the float64 top-k probability margin exceeds 1e-6.  The routing of the fused kernel is
checked against the oracle router applied to the kernel's own normalised rows (the norm is checked
separately), so a rounding-boundary difference in one bf16 element of the norm cannot mask or fake a router
error."""

from __future__ import annotations

import math

import pytest
import torch

from gpu_util import MARGIN, TOL, assert_rel, dev, say
from oracle import norm as ON
from oracle import router as OR

from moe_mi355 import ops
from moe_mi355.norm import NormRouterCore, RMSNormFn
from moe_mi355.router import RouterCore

pytestmark = pytest.mark.gpu


def _x(N, H, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, H, generator=g) * scale).to(dtype)


def _w(H, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (0.5 + torch.rand(H, generator=g)).to(dtype)


NORM_SHAPES = [
    (4096, 512, torch.float32, torch.float32),
    (1000, 4096, torch.bfloat16, torch.float32),
    (257, 2048, torch.bfloat16, torch.bfloat16),
    (64, 8192, torch.float32, torch.bfloat16),
    (3, 8, torch.bfloat16, torch.float32),
]


def _nid(s):
    N, H, xd, wd = s
    return f"N{N}-H{H}-{str(xd)[6:]}-{str(wd)[6:]}"


@pytest.mark.parametrize("shape", NORM_SHAPES, ids=_nid)
def test_rmsnorm_forward_parity(shape):
    N, H, xd, wd = shape
    say(f"[rmsnorm fwd] {_nid(shape)}")
    x, w = _x(N, H, xd, N + H, scale=3.0), _w(H, wd, H)
    xn, rstd = ops.rmsnorm_forward(x.to(dev()), w.to(dev()), 1e-5)
    y, r = ON.rmsnorm_fwd(x, w, 1e-5)
    assert xn.dtype == xd and xn.shape == (N, H)
    assert_rel(rstd, r, 1e-5, "rstd")
    assert_rel(xn, ON.rmsnorm_to(y, xd), TOL[xd], "xn")
    if xd == torch.float32:
        assert_rel(xn, y, 1e-5, "xn vs float64")


@pytest.mark.parametrize("shape", NORM_SHAPES, ids=_nid)
@pytest.mark.parametrize("second", [False, True], ids=["one_grad", "two_grads"])
def test_rmsnorm_backward_parity(shape, second):
    N, H, xd, wd = shape
    say(f"[rmsnorm bwd] {_nid(shape)} second={second}")
    x, w = _x(N, H, xd, N + H + 1), _w(H, wd, H + 1)
    dy = _x(N, H, xd, N + H + 2)
    dy2 = _x(N, H, xd, N + H + 3) if second else None
    d = dev()
    _, rstd = ops.rmsnorm_forward(x.to(d), w.to(d), 1e-5)
    dx, dw = ops.rmsnorm_backward(x.to(d), w.to(d), rstd, dy.to(d), None if dy2 is None else dy2.to(d))
    # the kernel's contract: the sum of two gradients of xn is rounded to x's dtype (as autograd's sum is)
    g = (dy.float() + dy2.float()).to(xd).double() if second else dy.double()
    rdx, rdw = ON.rmsnorm_bwd(x, w, g, 1e-5)
    assert dx.dtype == xd and dw.dtype == wd
    # each gradient is computed in fp32 and rounded once to its own storage type
    assert_rel(dx, rdx, TOL[xd], "dx")
    assert_rel(dw, rdw, TOL[wd], "dweight")


def test_rmsnorm_function_autograd_and_empty():
    d = dev()
    x = _x(33, 256, torch.float32, 7).to(d).requires_grad_(True)
    w = _w(256, torch.float32, 8).to(d).requires_grad_(True)
    y = RMSNormFn.apply(x, w, 1e-5)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    rdx, rdw = ON.rmsnorm_bwd(x.detach().cpu(), w.detach().cpu(), gy.cpu(), 1e-5)
    assert_rel(x.grad, rdx, 1e-5, "dx")
    assert_rel(w.grad, rdw, 1e-5, "dweight")
    xn, rstd = ops.rmsnorm_forward(torch.zeros(0, 64, device=d), torch.ones(64, device=d), 1e-5)
    assert xn.shape == (0, 64) and rstd.shape == (0,)


def test_rmsnorm_rejects_bad_shapes():
    d = dev()
    with pytest.raises(ValueError):
        ops.rmsnorm_forward(torch.zeros(4, 12, device=d), torch.ones(12, device=d), 1e-5)  # H % 8
    with pytest.raises(ValueError):
        ops.rmsnorm_forward(torch.zeros(4, 16384, device=d), torch.ones(16384, device=d), 1e-5)  # H > 8192


# (N, H, E, K, dtype): the first five take the fused forward kernel, the rest the norm kernel + router kernels
ROUTE_SHAPES = [
    (16384, 4096, 8, 2, torch.bfloat16),   # C2 shape
    (1000, 2048, 16, 4, torch.bfloat16),   # E = 16
    (129, 512, 5, 2, torch.bfloat16),      # E < 8, ragged block
    (40, 256, 12, 12, torch.bfloat16),     # K == E
    (200, 520, 8, 2, torch.bfloat16),      # H % 256 != 0: fused forward, backward through the router kernels
    (300, 2048, 64, 6, torch.bfloat16),    # E = 64: wide router kernel over xn
    (200, 512, 8, 2, torch.float32),       # fp32: generic router over xn
]


def _rid(s):
    N, H, E, K, xd = s
    return f"N{N}-H{H}-E{E}-K{K}-{str(xd)[6:]}"


def _gate(H, E, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(H, E, generator=g) * 0.02 * math.sqrt(4096.0 / H)).to(dtype)


@pytest.mark.parametrize("shape", ROUTE_SHAPES, ids=_rid)
def test_norm_router_forward_parity(shape):
    N, H, E, K, xd = shape
    say(f"[norm router fwd] {_rid(shape)}")
    x, nw, gw = _x(N, H, xd, N + E, scale=2.0), _w(H, torch.float32, H + E), _gate(H, E, xd, E + K)
    d = dev()
    for rep in range(2):  # the second call reuses the zeroed workspace and its completion counter
        xn, rstd, idx, w, logits, lse, cnt, stats, aux, z = ops.rmsnorm_router_forward(
            x.to(d), nw.to(d), 1e-5, gw.to(d), K, aux_coef=0.01, z_coef=1e-3)
        torch.cuda.synchronize()
        y, r = ON.rmsnorm_fwd(x, nw, 1e-5)
        assert_rel(rstd, r, 1e-5, "rstd")
        assert_rel(xn, ON.rmsnorm_to(y, xd), TOL[xd], "xn")
        # the router part: the oracle routes the kernel's own xn
        ref = OR.route_fwd(xn.cpu(), gw, K)
        ok = ref["margin"] > MARGIN
        assert ok.float().mean() > 0.95
        assert torch.equal(idx.cpu()[ok], ref["idx"][ok])
        assert_rel(logits, ref["logits"], 1e-5, "logits")
        v = ref["probs"].gather(1, idx.cpu())
        assert_rel(w.float(), v / v.sum(-1, keepdim=True).clamp_min(1e-30), TOL[xd], "weights")
        assert torch.equal(cnt.cpu(), torch.bincount(idx.cpu().reshape(-1), minlength=E))
        assert_rel(lse, torch.logsumexp(ref["logits"], -1), 1e-5, "lse")
        st = stats.cpu().double()
        assert st[5].item() == N * K and st[6].item() == 0.0
        zs = OR.z_stat(ref["logits"])
        assert abs(st[0].item() - zs) <= 1e-5 * max(1.0, zs)
        P = ref["probs"].mean(0)
        assert_rel(st[8:8 + E], P, 1e-5, "mean probabilities")
        auxr = float(E * ((cnt.cpu().double() / (N * K)) * P).sum())
        assert abs(aux.item() - 0.01 * auxr) <= 1e-5 * 0.01 * auxr
        assert abs(z.item() - 1e-3 * zs) <= 1e-5 * 1e-3 * zs
        # the fused xn is bit-identical to the standalone norm kernel's
        xn2, _ = ops.rmsnorm_forward(x.to(d), nw.to(d), 1e-5)
        assert torch.equal(xn.cpu(), xn2.cpu())


@pytest.mark.parametrize("expert_grad", [True, False], ids=["with_dxn", "router_only"])
@pytest.mark.parametrize("shape", ROUTE_SHAPES[:6], ids=_rid)
def test_norm_router_backward_parity(shape, expert_grad):
    """NormRouterCore's gradients against the chain rule over the oracle: the router backward on xn (oracle
    router_full with the kernel's routing), its dxn plus an expert-path gradient of xn (or none), then the
    norm's backward."""
    N, H, E, K, xd = shape
    N = min(N, 2048)
    say(f"[norm router bwd] {_rid(shape)} expert_grad={expert_grad}")
    x, nw, gw = _x(N, H, xd, N + 1), _w(H, torch.float32, H + 2), _gate(H, E, xd, E + 3)
    g = torch.Generator().manual_seed(N + 4)
    gwt = torch.randn(N, K, generator=g).to(xd)
    gxn = (torch.randn(N, H, generator=g) * 0.01).to(xd)
    d = dev()
    xd_, nwd, gwd = x.to(d).requires_grad_(True), nw.to(d).requires_grad_(True), gw.to(d).requires_grad_(True)
    xn, idx, w, aux, z, logits, cnt, stats = NormRouterCore.apply(xd_, nwd, 1e-5, gwd, K, 0.01, 1e-3, None)
    if not expert_grad:
        gxn = torch.zeros_like(gxn)
    loss = (w.float() * gwt.to(d).float()).sum() + aux + z
    if expert_grad:
        loss = loss + (xn.float() * gxn.to(d).float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    xn_c = xn.detach().cpu()
    ref = OR.router_full(xn_c, gw, K, grad_w=gwt, alpha=0.01, beta=1e-3, idx_override=idx.cpu())
    rdx, rdnw = ON.rmsnorm_bwd(x, nw, ref["dX"] + gxn.double(), 1e-5)
    tol = TOL[xd]
    assert_rel(gwd.grad, ref["dW"], tol, "d gate", floor=1e-4)
    assert_rel(xd_.grad, rdx, tol, "dx", floor=1e-4)
    assert_rel(nwd.grad, rdnw, tol, "d norm weight", floor=1e-4)


def test_norm_router_matches_the_unfused_composition():
    """RMSNormFn then RouterCore, and NormRouterCore, on the same inputs and upstream gradients."""
    N, H, E, K = 4096, 4096, 8, 2
    say("[norm router vs composition]")
    d = dev()
    x, nw, gw = _x(N, H, torch.bfloat16, 31), _w(H, torch.float32, 32), _gate(H, E, torch.bfloat16, 33)
    gwt = torch.randn(N, K, generator=torch.Generator().manual_seed(34)).to(torch.bfloat16).to(d)
    outs = []
    for fused in (True, False):
        xd_, nwd, gwd = x.to(d).requires_grad_(True), nw.to(d).requires_grad_(True), gw.to(d).requires_grad_(True)
        if fused:
            xn, idx, w, aux, z, *_ = NormRouterCore.apply(xd_, nwd, 1e-5, gwd, K, 0.01, 1e-3, None)
        else:
            xn = RMSNormFn.apply(xd_, nwd, 1e-5)
            idx, w, aux, z, *_ = RouterCore.apply(xn, gwd, K, 0.01, 1e-3, None)
        ((w.float() * gwt.float()).sum() + aux + z).backward()
        outs.append((xn.detach(), idx, w.detach(), xd_.grad, nwd.grad, gwd.grad))
    (xa, ia, wa, dxa, dna, dga), (xb, ib, wb, dxb, dnb, dgb) = outs
    assert torch.equal(xa, xb)
    ref = OR.route_fwd(xa.cpu(), gw, K)
    ok = ref["margin"] > MARGIN
    assert torch.equal(ia.cpu()[ok], ib.cpu()[ok])
    for a, b, what in ((wa, wb, "w"), (dxa, dxb, "dx"), (dna, dnb, "d norm weight"), (dga, dgb, "d gate")):
        assert_rel(a, b, 2e-2, what)


def test_toy_moe_block_fused_matches_composition():
    """ToyMoEBlock.forward (norm fused into the router) against x + moe(norm(x)) with the same parameters."""
    from pkg.distributed import build_topology
    from pkg.models import RMSNorm, ToyMoEBlock

    say("[toy moe block]")
    d = dev()
    torch.manual_seed(5)
    blk = ToyMoEBlock(256, 512, 8, 2, build_topology(), dtype=torch.bfloat16).to(d)
    assert isinstance(blk.norm, RMSNorm) and blk.norm.eps == 1e-5
    assert "dim=256, eps=1e-05" in repr(blk.norm)
    x = (torch.randn(4, 32, 256, generator=torch.Generator().manual_seed(6)) * 1.5).to(torch.bfloat16).to(d)
    gout = torch.randn(4, 32, 256, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(d)
    res = []
    for fused in (True, False):
        xi = x.clone().requires_grad_(True)
        blk.zero_grad()
        out = blk(xi) if fused else xi + blk.moe(blk.norm(xi))
        out.backward(gout)
        res.append((out.detach(), xi.grad, blk.norm.weight.grad.clone(), blk.moe.router.gate_w.grad.clone(),
                    blk.moe.w_gate.grad.clone()))
    for a, b, what in zip(res[0], res[1], ("out", "dx", "d norm weight", "d gate", "d w_gate")):
        assert a.shape == b.shape
        assert_rel(a, b, 2e-2, what, floor=1e-3)
