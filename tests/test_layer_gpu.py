"""Full MoE layer (router -> planner -> permute -> SwiGLU grouped GEMM ->
combine, forward and backward) against the float64 layer oracle, evaluated at
the device's own routing so near-tie tokens compare like with like.
Tolerance: bf16 2e-2, fp32 1e-5 (max-norm relative)."""

from __future__ import annotations

import math

import pytest
import torch

from gpu_util import TOL, assert_rel, dev, say
from oracle import layer as OL
from oracle import plan as OP

from moe_mi355 import configs
from pkg.distributed import build_topology
from pkg.distributed.moe_layer import DistributedMoELayer

pytestmark = pytest.mark.gpu


def _layer(H, Fd, E, K, dt, cf=1.25, drop=False, layout="reference", aux=0.0, z=0.0, seed=0):
    torch.manual_seed(seed)
    layer = DistributedMoELayer(H, Fd, E, K, build_topology(), capacity_factor=cf, capacity_dropping=drop, dtype=dt,
                                layout=layout, aux_loss_coef=aux, z_loss_coef=z)
    return layer.to(dev())


CASES = [
    # H, F, E, K, dtype, cf, drop, layout, aux/z
    # K=3 with chunk = 609 // 8 = 76 rows: chunk boundaries split a token's rows across experts
    (128, 256, 8, 3, torch.bfloat16, 1.25, False, "reference", False),
    (128, 256, 8, 2, torch.bfloat16, 0.6, True, "reference", True),
    (256, 128, 16, 4, torch.bfloat16, 1.25, False, "routed", False),
    (256, 128, 16, 4, torch.bfloat16, 0.7, True, "routed", True),
    (64, 96, 4, 1, torch.bfloat16, 1.0, True, "routed", False),
    (64, 64, 5, 3, torch.float32, 1.25, False, "reference", False),
    (64, 64, 5, 3, torch.float32, 0.8, True, "routed", True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"H{c[0]}-F{c[1]}-E{c[2]}-K{c[3]}-{str(c[4])[6:]}-"
                                                   f"cf{c[5]}-{'drop' if c[6] else 'nodrop'}-{c[7]}-{'aux' if c[8] else 'plain'}")
def test_layer_matches_oracle(case):
    H, Fd, E, K, dt, cf, drop, layout, losses = case
    say(f"[layer] {case}")
    N = 203
    aux, z = (0.01, 1e-3) if losses else (0.0, 0.0)
    layer = _layer(H, Fd, E, K, dt, cf, drop, layout, aux, z, seed=H + E)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(N, H, generator=g).to(dt)
    gout = torch.randn(N, H, generator=g).to(dt)
    xd = x.to(dev()).requires_grad_(True)
    out = layer(xd)
    loss = (out.float() * gout.to(dev()).float()).sum()
    if losses:
        loss = loss + layer.router.last_aux_loss + layer.router.last_z_loss
    loss.backward()
    torch.cuda.synchronize()
    idx = layer.last_plan  # device routing is re-derived below
    ref = OL.layer_fwd_bwd(
        x, layer.router.gate_w.detach(), layer.w_gate.detach(), layer.w_up.detach(), layer.w_down.detach(), K,
        grad_out=gout, capacity_factor=cf, capacity_dropping=drop,
        layout=OP.LAYOUT_REFERENCE if layout == "reference" else OP.LAYOUT_ROUTED,
        alpha=aux, beta=z, idx_override=_device_idx(layer, xd),
    )
    tol = TOL[dt]
    assert_rel(out, ref["out"], tol, "out")
    # The floors matter only where the exact gradient vanishes (K=1 routing: the combine weight is
    # identically 1); typical gate gradients here are 1e-2..1.
    assert_rel(xd.grad, ref["dx"], tol, "dx", floor=1e-4)
    assert_rel(layer.router.gate_w.grad, ref["dgate_w"], tol, "dgate_w", floor=1e-3)
    assert_rel(layer.w_gate.grad, ref["dw_gate"], tol, "dw_gate")
    assert_rel(layer.w_up.grad, ref["dw_up"], tol, "dw_up")
    assert_rel(layer.w_down.grad, ref["dw_down"], tol, "dw_down")
    if drop:
        assert abs(layer.last_dropped_token_fraction - float(ref["dropped_fraction"])) < 1e-12
    del idx


def _device_idx(layer, xd):
    with torch.no_grad():
        from moe_mi355 import ops

        idx, *_ = ops.router_forward(xd.detach(), layer.router.gate_w.detach(), layer.top_k)
    return idx.cpu()


def test_layer_custom_experts_path():
    """Replacing ``experts`` (the reference's extension point) runs those modules per expert."""
    say("[layer custom experts]")
    H, Fd, E, K = 64, 128, 4, 2
    layer = _layer(H, Fd, E, K, torch.bfloat16, layout="routed")
    fused_ref = layer(torch.zeros(1, H, dtype=torch.bfloat16, device=dev()))  # warm
    del fused_ref

    class Scale(torch.nn.Module):
        def __init__(self, s):
            super().__init__()
            self.s = s

        def forward(self, x):
            return x * self.s

    layer.experts = torch.nn.ModuleList([Scale(float(i + 1)) for i in range(E)])
    x = torch.randn(50, H, device=dev()).to(torch.bfloat16)
    out = layer(x)
    idx = _device_idx(layer, x)
    from moe_mi355 import ops

    w = ops.router_forward(x, layer.router.gate_w.detach(), K)[1].float().cpu()
    ref = torch.zeros(50, H, dtype=torch.float64)
    for t in range(50):
        for k in range(K):
            ref[t] += float(w[t, k]) * (int(idx[t, k]) + 1) * x[t].double().cpu()
    assert_rel(out, ref, 2e-2, "custom experts out")


def test_layer_c4_shape_vs_torch_fp32():
    """C4 weights at full shape (H=4096, F=14336, E=8, K=2) on 512 tokens, routed
    layout: fused HIP layer vs a float32 torch computation on the GPU."""
    say("[layer C4 shape]")
    cfg = configs.C4
    d = dev()
    torch.manual_seed(3)
    layer = DistributedMoELayer(cfg.H, cfg.F, cfg.E, cfg.K, build_topology(), dtype=torch.bfloat16,
                                layout="routed", check_numerics=True).to(d)
    with torch.no_grad():
        for p_ in (layer.w_gate, layer.w_up, layer.w_down):
            p_.normal_(0.0, 0.02)
    N = 512
    x = torch.randn(N, cfg.H, device=d).to(torch.bfloat16).requires_grad_(True)
    out = layer(x)
    gout = torch.randn(N, cfg.H, device=d).to(torch.bfloat16)
    out.backward(gout)
    from moe_mi355 import ops

    idx, w, *_ = ops.router_forward(x.detach(), layer.router.gate_w.detach(), cfg.K)
    xf = x.detach().float().requires_grad_(True)
    wgf = layer.w_gate.detach().float().requires_grad_(True)
    wuf = layer.w_up.detach().float().requires_grad_(True)
    wdf = layer.w_down.detach().float().requires_grad_(True)
    ref = torch.zeros(N, cfg.H, device=d)
    for e in range(cfg.E):
        for k in range(cfg.K):
            sel = (idx[:, k] == e).nonzero().flatten()
            if sel.numel() == 0:
                continue
            xe = xf[sel]
            ye = (torch.nn.functional.silu(xe @ wgf[e].t()) * (xe @ wuf[e].t())) @ wdf[e].t()
            ref = ref.index_add(0, sel, w[sel, k].float()[:, None] * ye)
    (ref * gout.float()).sum().backward()
    assert_rel(out, ref.detach(), 2e-2, "C4 out")
    assert_rel(layer.w_gate.grad, wgf.grad, 2e-2, "C4 dw_gate")
    assert_rel(layer.w_up.grad, wuf.grad, 2e-2, "C4 dw_up")
    assert_rel(layer.w_down.grad, wdf.grad, 2e-2, "C4 dw_down")


def test_layer_checks_run_at_the_end_of_the_forward():
    """With check_numerics the router's checks are deferred to the forward's final synchronisation: after
    the forward nothing is pending, the profile is resolved and the layer's outputs match a forward with
    the checks off; a non-finite gate still raises the router's assertion (before the output NaN check)
    from the layer's forward, and the router alone still checks at once."""
    say("[layer deferred checks]")
    H, Fd, E, K, N = 256, 512, 8, 2, 300
    layer = _layer(H, Fd, E, K, torch.bfloat16, layout="routed")
    assert layer.check_numerics and layer.router.sync_profile
    x = torch.randn(N, H, device=dev()).to(torch.bfloat16)
    out = layer(x)
    assert layer.router._pending is None and not layer.router._defer_check
    prof = layer.router.last_profile
    assert prof is not None and prof.kernel_ms > 0.0
    from moe_mi355.router import STAT_CNT_TOTAL
    assert int(round(float(layer.router.last_stats_host[STAT_CNT_TOTAL]))) == N * K
    layer.check_numerics = False
    out2 = layer(x)
    assert torch.equal(out, out2)
    layer.check_numerics = True
    with torch.no_grad():
        layer.router.gate_w[0, 3] = float("nan")
    with pytest.raises(AssertionError, match="NaN in expert indices"):
        layer(x)
    assert not layer.router._defer_check
    with pytest.raises(AssertionError, match="NaN in expert indices"):
        layer.router(x)


@pytest.mark.parametrize("case", [(256, 128, 8, 2, "reference", False), (512, 256, 64, 6, "routed", True),
                                  (256, 128, 16, 4, "routed", False)],
                         ids=lambda c: f"H{c[0]}-F{c[1]}-E{c[2]}-K{c[3]}-{c[4]}-{'aux' if c[5] else 'plain'}")
def test_layer_linked_tokens_gradient(case, monkeypatch):
    """The layer hands the expert path's gradient of the tokens to the router's backward, which adds it inside
    its dx kernel: x.grad (and every other gradient) bit-identical to the same layer with the two gradients
    summed by autograd (the router's tokens link switched off)."""
    H, Fd, E, K, layout, losses = case
    say(f"[layer linked tokens] {case}")
    aux, z = (0.01, 1e-3) if losses else (0.0, 0.0)
    g = torch.Generator().manual_seed(5)
    N = 777
    x = torch.randn(N, H, generator=g).to(torch.bfloat16).to(dev())
    gout = torch.randn(N, H, generator=g).to(torch.bfloat16).to(dev())
    grads = []
    for linked in (True, False):
        layer = _layer(H, Fd, E, K, torch.bfloat16, layout=layout, aux=aux, z=z, seed=3)
        if not linked:
            monkeypatch.setattr(type(layer.router), "take_linked_tokens", lambda self: None)
        xd = x.clone().requires_grad_(True)
        out = layer(xd)
        loss = (out.float() * gout.float()).sum()
        if losses:
            loss = loss + layer.router.last_aux_loss + layer.router.last_z_loss
        loss.backward()
        torch.cuda.synchronize()
        grads.append([xd.grad, layer.router.gate_w.grad, layer.w_gate.grad, layer.w_up.grad, layer.w_down.grad])
        monkeypatch.undo()
    for what, a, b in zip(("dx", "dgate_w", "dw_gate", "dw_up", "dw_down"), *grads):
        assert torch.equal(a, b), f"{what} differs between the linked and the autograd-summed token gradients"
