"""The MoE layer at the benchmark's own full sizes: C4 (T=8192, d=4096, E=8, F=14336, K=2, reference layout:
the headline workload) and C5 (T=32768, d=2048, E=128, F=768, K=8, routed layout, Zipf(1.1) logit bias,
capacity factor 1.0 with drops, aux and z losses); and C4's fp8 inference forward.

Inputs have the configs' shapes and scales, drawn on the device from fixed seeds (the CPU draw the benchmark
uses takes minutes for C4's 2.8 GB of weights).  Checks:
* top-k indices bit-exact against the float64 oracle wherever the top-k margin exceeds 1e-6;
* the dispatch plan (capacity drop mask, row <-> slot maps, expert offsets) bit-exact against the integer
  oracle applied to the device's indices;
* output, input gradient, gate gradient, expert weight gradients, aux and z losses and the dropped fraction
  against a float32 torch computation of the same layer on the GPU (autograd through plain matmuls at the
  device's routing and plan): 2e-2 max-norm relative (bf16).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_util import MARGIN, assert_rel, dev, say
from oracle import plan as OP
from oracle import router as OR

from moe_mi355 import configs
from pkg.distributed.parallel_mesh import DistributedMoELayer, build_topology

pytestmark = pytest.mark.gpu


def _inputs(cfg, seed):
    d = dev()
    g = torch.Generator(device=d).manual_seed(seed)
    r = lambda *s, std=1.0: (torch.randn(*s, generator=g, device=d) * std).to(cfg.dtype)  # noqa: E731
    inp = {"x": r(cfg.T, cfg.H), "gate_w": r(cfg.H, cfg.E, std=0.02), "w_gate": r(cfg.E, cfg.F, cfg.H, std=0.02),
           "w_up": r(cfg.E, cfg.F, cfg.H, std=0.02), "w_down": r(cfg.E, cfg.H, cfg.F, std=0.02),
           "grad_out": r(cfg.T, cfg.H)}
    if cfg.zipf_bias:
        inp["bias"] = configs.zipf_bias(cfg.E, torch.Generator().manual_seed(seed)).to(d)
    return inp


def _torch_layer_fp32(inp, cfg, idx, pl, drop):
    """The layer in float32 torch with autograd, at the given routing and plan: softmax over x @ gate_w
    (+ bias), top-k gather at ``idx``, renormalise, zero dropped slots, rows x[row_slot // K] through the
    SwiGLU of their segment's expert, weighted sum per token.  Returns the tensors and their gradients."""
    d = dev()
    K, E = cfg.K, cfg.E
    x = inp["x"].float().requires_grad_(True)
    gw = inp["gate_w"].float().requires_grad_(True)
    Wg = inp["w_gate"].float().requires_grad_(True)
    Wu = inp["w_up"].float().requires_grad_(True)
    Wd = inp["w_down"].float().requires_grad_(True)
    logits = x @ gw
    if "bias" in inp:
        logits = logits + inp["bias"].float()
    p = torch.softmax(logits, dim=-1)
    idx_d = idx.to(d)
    v = p.gather(1, idx_d)
    w = v / v.sum(-1, keepdim=True).clamp_min(1e-30)
    if drop is not None:
        w = w.masked_fill(torch.from_numpy(drop).to(d), 0.0)
    row_slot = torch.from_numpy(pl["row_slot"]).to(d)
    slot_row = torch.from_numpy(pl["slot_row"]).to(d)
    offs = [int(o) for o in pl["offsets"]]
    xp = x[row_slot // K]
    ys = []
    for e in range(E):
        lo, hi = offs[e], offs[e + 1]
        if lo < hi:
            xe = xp[lo:hi]
            ys.append((F.silu(xe @ Wg[e].t()) * (xe @ Wu[e].t())) @ Wd[e].t())
    R = xp.shape[0]
    if R > offs[E]:
        ys.append(xp.new_zeros((R - offs[E], cfg.H)))
    Y = torch.cat(ys, 0)
    sr = slot_row.view(-1, K)
    out = torch.zeros_like(x)
    for k in range(K):
        valid = (sr[:, k] >= 0) & (sr[:, k] < offs[E])
        contrib = w[:, k:k + 1] * Y[sr[:, k].clamp_min(0)]
        out = out + torch.where(valid[:, None], contrib, torch.zeros_like(contrib))
    cnt = torch.bincount(idx_d.reshape(-1), minlength=E).float()
    aux = cfg.aux_coef * E * ((cnt / (cfg.T * K)) * p.mean(0)).sum()
    z = cfg.z_coef * torch.logsumexp(logits, dim=-1).square().mean()
    loss = (out * inp["grad_out"].float()).sum() + aux + z
    loss.backward()
    return {"out": out.detach(), "aux": aux.detach(), "z": z.detach(), "dx": x.grad, "dgate_w": gw.grad,
            "dw_gate": Wg.grad, "dw_up": Wu.grad, "dw_down": Wd.grad}


def _run(cfg, layout, seed):
    inp = _inputs(cfg, seed)
    layer = DistributedMoELayer(cfg.H, cfg.F, cfg.E, cfg.K, build_topology(), capacity_factor=cfg.capacity_factor,
                                capacity_dropping=cfg.capacity_dropping, dtype=cfg.dtype, layout=layout,
                                aux_loss_coef=cfg.aux_coef, z_loss_coef=cfg.z_coef).to(dev())
    with torch.no_grad():
        for name in ("w_gate", "w_up", "w_down"):
            getattr(layer, name).copy_(inp[name])
        layer.router.gate_w.copy_(inp["gate_w"])
    if "bias" in inp:
        layer.router.logit_bias = inp["bias"]
    seen = {}
    layer.router.register_forward_hook(lambda _m, _i, o: seen.update(idx=o[0].detach()))
    x = inp["x"].clone().requires_grad_(True)
    out = layer(x)
    loss = (out.float() * inp["grad_out"].float()).sum()
    if cfg.aux_coef or cfg.z_coef:
        loss = loss + layer.router.last_aux_loss + layer.router.last_z_loss
    loss.backward()
    torch.cuda.synchronize()
    return inp, layer, x, out, seen["idx"].cpu()


def _check(cfg, layout, seed):
    say(f"[fullsize] {cfg.name} layout={layout}")
    inp, layer, x, out, idx = _run(cfg, layout, seed)
    K, E = cfg.K, cfg.E
    # routing: bit-exact against the float64 oracle wherever the margin is clear
    fx = OR.route_fwd(inp["x"].cpu(), inp["gate_w"].cpu(), K, bias=inp["bias"].cpu() if "bias" in inp else None)
    ok = fx["margin"] > MARGIN
    assert ok.float().mean() > 0.99
    assert torch.equal(idx[ok], fx["idx"][ok]), "top-k indices differ from the oracle"
    # plan: bit-exact against the integer oracle on the device's indices
    p = layer.last_plan
    drop = None
    if cfg.capacity_dropping:
        drop = OP.drop_mask(idx.numpy(), configs.capacity(cfg))
        assert np.array_equal(p.drop.cpu().numpy(), drop), "capacity drop mask"
        assert int(p.ndrop.item()) == int(drop.sum())
        assert abs(layer.last_dropped_token_fraction - drop.mean()) < 1e-12
    pl = OP.plan_reference(idx.numpy(), E) if layout == "reference" else OP.plan_routed(idx.numpy(), E, drop)
    R = int(pl["n_rows"])
    assert np.array_equal(p.offsets.cpu().numpy(), pl["offsets"]), "expert offsets"
    assert np.array_equal(p.row_slot.cpu().numpy()[:R], pl["row_slot"]), "row -> slot map"
    assert np.array_equal(p.slot_row.cpu().numpy(), pl["slot_row"]), "slot -> row map"
    say(f"[fullsize] {cfg.name}: rows={R} drops={0 if drop is None else int(drop.sum())}; float32 torch reference")
    ref = _torch_layer_fp32(inp, cfg, idx, pl, drop)
    tol = 2e-2
    assert_rel(out, ref["out"], tol, "out")
    assert_rel(x.grad, ref["dx"], tol, "dx")
    if layout == "reference" and (R // E) % K == 0:
        # Positional layout with a chunk that is a multiple of K: a token's K rows are adjacent and fall in
        # one expert's chunk, so out[t] = (sum_k w[t,k]) Expert(x[t]) = Expert(x[t]) whatever the gate: the
        # exact gate gradient is zero (moe_layer.py L:317-353), and both computations hold rounding noise.
        # Bound: far below |x| N |grad_w|, the size a gradient that did not cancel would have.
        bound = 1e-6 * float(inp["x"].abs().max()) * cfg.T * float(inp["grad_out"].float().abs().max()) * cfg.H ** 0.5
        assert float(layer.router.gate_w.grad.abs().max()) <= bound, "the gate gradient does not cancel"
        assert float(ref["dgate_w"].abs().max()) <= bound
    else:
        assert_rel(layer.router.gate_w.grad, ref["dgate_w"], tol, "dgate_w")
    for name in ("w_gate", "w_up", "w_down"):
        assert_rel(getattr(layer, name).grad, ref["d" + name], tol, "d" + name)
    if cfg.aux_coef:
        assert abs(float(layer.router.last_aux_loss.detach()) - float(ref["aux"])) <= 1e-4 * abs(float(ref["aux"]))
    if cfg.z_coef:
        assert abs(float(layer.router.last_z_loss.detach()) - float(ref["z"])) <= 1e-4 * abs(float(ref["z"]))
    return layer, idx, pl


def test_c4_reference_layout_full_size():
    _check(configs.C4, "reference", seed=3)


def test_c5_skewed_routed_full_size():
    cfg = configs.C5
    layer, idx, pl = _check(cfg, "routed", seed=4)
    # the Zipf bias makes the load heavily imbalanced: a few experts keep most of their queue
    cnt = np.diff(pl["offsets"])
    assert cnt.max() > 8 * max(1, int(np.median(cnt)))
    assert layer.router.last_profile.expert_load_imbalance > 4.0


def test_c4_fp8_forward_full_size():
    """The C4 layer's fp8 inference forward at full size: within the e4m3 rounding of the bf16 forward, and the
    last expert's last rows (the grid's last tiles) through the float64 oracle chain from the kernels' own
    quantized operands, with the block-quantized act bit-exact."""
    from moe_mi355 import ops
    from oracle import fp8 as O8

    cfg = configs.C4
    say(f"[fullsize] {cfg.name} fp8 forward")
    inp = _inputs(cfg, seed=3)
    layer = DistributedMoELayer(cfg.H, cfg.F, cfg.E, cfg.K, build_topology(), dtype=cfg.dtype,
                                layout="reference").to(dev())
    with torch.no_grad():
        for name in ("w_gate", "w_up", "w_down"):
            getattr(layer, name).copy_(inp[name])
        layer.router.gate_w.copy_(inp["gate_w"])
        ref = layer(inp["x"])
    out = layer.forward_fp8(inp["x"])
    torch.cuda.synchronize()
    err = ((out.float() - ref.float()).abs().max() / ref.float().abs().max()).item()
    assert err < 0.1, err
    p = layer.last_plan
    wq, ws = layer.quantize_fp8()
    xq, sx = ops.permute_fp8(inp["x"], p)
    act, _hgu, y, (aq, asc) = ops.swiglu_forward_fp8(xq, sx, wq, ws, p.offsets, return_mx=True)
    torch.cuda.synchronize()
    offs = p.offsets.cpu().tolist()
    e = cfg.E - 1
    hi = int(offs[e + 1])
    lo = hi - 48
    assert lo >= int(offs[e])
    mq, ms = O8.quant_mx(act[lo:hi].cpu().float())
    assert torch.equal(aq[lo:hi].cpu(), mq) and torch.equal(asc[lo:hi].cpu(), ms)
    one = lambda t: t[e:e + 1].cpu()  # noqa: E731
    _rh, _ra, ry = O8.swiglu_fwd_fp8(xq[lo:hi].cpu(), sx[lo:hi].cpu(), [one(w) for w in wq], [one(s) for s in ws],
                                     [0, hi - lo], act_in=act[lo:hi].cpu().float())
    assert_rel(y[lo:hi], ry, 2e-2, "y (last rows)")
