"""The HIP layer and router against the golden fixtures written from the reference itself
(tests/golden/*.npz; made by tests/golden/make_layer_fixtures.py from moe-engine's DistributedMoELayer and
MoERouter on the CPU -- nothing of the reference runs here).

Layer fixtures use the reference ("positional") layout.  Indices, counts and drop masks are compared
bit-exactly (the fixtures' inputs keep every top-k margin above 1e-4); values within 1e-5 (fp32) and 2e-2
(bf16) max-norm relative.  Under exact ties (an all-zero gate) the kernels take the lowest expert indices
while torch.topk, which the reference calls, returns an implementation-defined order: there the weights,
the layer output and the expert gradients still match (the positional layout does not depend on the
choice), and the gate gradient is compared with the oracle at the kernels' own routing."""

from __future__ import annotations

import glob
import json
import os

import numpy as np
import pytest
import torch

from gpu_util import assert_rel, dev, say
from oracle import layer as OL
from oracle import plan as OP

from pkg.distributed.parallel_mesh import DistributedMoELayer, build_topology
from pkg.kernels.moe_router import MoERouter

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"float32": 1e-5, "bfloat16": 2e-2}


def load(name):
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    return json.loads(str(d["config"])), {k: d[k] for k in d.files if k != "config"}


def names(kind):
    out = []
    for f in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        n = os.path.basename(f)[:-4]
        if load(n)[0]["kind"] == kind:
            out.append(n)
    return out


def on_dev(a, dt):
    return torch.from_numpy(np.asarray(a)).to(getattr(torch, dt)).to(dev())


def _gate_grad_vanishes(cfg, a):
    """K = 1 (the renormalised weight is identically 1), or the positional layout with a chunk that is a
    multiple of K and no dropped slot (a token's K rows are adjacent in one expert's chunk, so its output is
    sum_k w[t,k] Expert(x[t]) = Expert(x[t])): the layer's output does not depend on the gate."""
    chunk = max(1, cfg["N"] * cfg["K"] // cfg["E"])
    return cfg["K"] == 1 or (chunk % cfg["K"] == 0 and not bool(a["drop"].any()))


@pytest.mark.parametrize("name", names("layer"))
def test_layer_matches_reference_fixture(name):
    cfg, a = load(name)
    say(f"[golden layer] {name} {cfg}")
    dt = cfg["dtype"]
    tol = TOL[dt]
    layer = DistributedMoELayer(cfg["H"], cfg["F"], cfg["E"], cfg["K"], build_topology(),
                                capacity_factor=cfg["capacity_factor"], capacity_dropping=cfg["capacity_dropping"],
                                dtype=getattr(torch, dt)).to(dev())
    with torch.no_grad():
        layer.router.gate_w.copy_(on_dev(a["gate_w"], dt))
        layer.w_gate.copy_(on_dev(a["w_gate"], dt))
        layer.w_up.copy_(on_dev(a["w_up"], dt))
        layer.w_down.copy_(on_dev(a["w_down"], dt))
    seen = {}
    layer.router.register_forward_hook(lambda _m, _i, o: seen.update(idx=o[0].detach(), w=o[1].detach(),
                                                                     cnt=o[2].detach()))
    x = on_dev(a["x"], dt).requires_grad_(True)
    out = layer(x)
    out.backward(on_dev(a["grad_out"], dt))
    torch.cuda.synchronize()
    idx = seen["idx"].cpu()
    ties = cfg["gate"] == "zero"
    if ties:
        assert idx.tolist() == [list(range(cfg["K"]))] * cfg["N"]
    else:
        assert np.array_equal(idx.numpy(), a["idx"]), "top-k indices differ from the reference"
        assert np.array_equal(seen["cnt"].cpu().numpy(), a["cnt"])
    assert_rel(seen["w"], torch.from_numpy(a["w"]), tol, "router weights")
    p = layer.last_plan
    if cfg["capacity_dropping"]:
        assert np.array_equal(p.drop.cpu().numpy(), a["drop"]), "capacity drop mask differs from the reference"
        assert abs(layer.last_dropped_token_fraction - float(a["dropped_fraction"])) < 1e-7
    assert_rel(out, torch.from_numpy(a["out"]), tol, "out")
    assert_rel(x.grad, torch.from_numpy(a["dx"]), tol, "dx")
    assert_rel(layer.w_gate.grad, torch.from_numpy(a["dw_gate"]), tol, "dw_gate")
    assert_rel(layer.w_up.grad, torch.from_numpy(a["dw_up"]), tol, "dw_up")
    assert_rel(layer.w_down.grad, torch.from_numpy(a["dw_down"]), tol, "dw_down")
    if _gate_grad_vanishes(cfg, a):
        # every token's output is independent of its routing weights: the exact gate gradient is zero and
        # both sides hold rounding noise, far below |x| N |grad_out| sqrt(H) (a gradient that did not cancel)
        bound = 1e-6 * float(np.abs(a["x"]).max()) * cfg["N"] * float(np.abs(a["grad_out"]).max()) * cfg["H"] ** 0.5
        assert float(layer.router.gate_w.grad.abs().max()) <= bound
        assert float(np.abs(a["dgate_w"]).max()) <= bound
    elif ties:
        ref = OL.layer_fwd_bwd(torch.from_numpy(a["x"]), torch.from_numpy(a["gate_w"]),
                               torch.from_numpy(a["w_gate"]), torch.from_numpy(a["w_up"]),
                               torch.from_numpy(a["w_down"]), cfg["K"], grad_out=torch.from_numpy(a["grad_out"]),
                               layout=OP.LAYOUT_REFERENCE, idx_override=idx)
        assert_rel(layer.router.gate_w.grad, ref["dgate_w"], tol, "dgate_w at the kernels' routing", floor=1e-6)
    else:
        assert_rel(layer.router.gate_w.grad, torch.from_numpy(a["dgate_w"]), tol, "dgate_w", floor=1e-6)


@pytest.mark.parametrize("name", [n for n in names("router") if load(n)[0]["bias"]])
def test_bias_router_matches_reference_fixture(name):
    """bias=True: routing on logits + bias, weights without a gradient, and _last_logits / the reported z
    statistic without the bias (moe_router.py L:671-687, L:727-733)."""
    cfg, a = load(name)
    say(f"[golden bias router] {name}")
    dt = cfg["dtype"]
    r = MoERouter(cfg["H"], cfg["E"], cfg["K"], bias=True, dtype=getattr(torch, dt)).to(dev())
    with torch.no_grad():
        r.gate_w.copy_(on_dev(a["gate_w"], dt))
        r.bias.copy_(on_dev(a["bias"], dt))
    x = on_dev(a["x"], dt).requires_grad_(True)
    idx, w, cnt = r(x)
    assert np.array_equal(idx.cpu().numpy(), a["idx"])
    assert np.array_equal(cnt.cpu().numpy(), a["cnt"])
    assert_rel(w, torch.from_numpy(a["w"]), TOL[dt], "w")
    assert not w.requires_grad
    assert_rel(r._last_logits, torch.from_numpy(a["last_logits"]), 1e-5, "_last_logits")
    prof = r.last_profile
    assert abs(prof.router_z_loss - float(a["router_z_loss"])) <= 1e-5 * abs(float(a["router_z_loss"]))
    assert abs(prof.expert_load_imbalance - float(a["expert_load_imbalance"])) < 1e-5
    assert abs(prof.tokens_per_expert_std - float(a["tokens_per_expert_std"])) < 1e-4


def test_ties_router_fixture():
    """All-zero gate: lowest expert indices here, torch.topk's order in the reference; weights 1/K and the
    z statistic ln(E)^2 in both."""
    cfg, a = load("router_ties_f32")
    say("[golden ties router]")
    r = MoERouter(cfg["H"], cfg["E"], cfg["K"]).to(dev())
    with torch.no_grad():
        r.gate_w.zero_()
    idx, w, cnt = r(on_dev(a["x"], "float32"))
    assert idx.cpu().tolist() == [list(range(cfg["K"]))] * cfg["N"]
    assert_rel(w, torch.from_numpy(a["w"]), 1e-6, "w")
    assert int(cnt.sum()) == int(a["cnt"].sum())
    assert abs(r.last_profile.router_z_loss - float(a["router_z_loss"])) <= 1e-5 * float(a["router_z_loss"])


def test_router_profile_fixture():
    """RouterProfile statistics and _last_logits against the reference's own (L:690-745)."""
    cfg, a = load("router_profile_f32")
    say("[golden router profile]")
    r = MoERouter(cfg["H"], cfg["E"], cfg["K"]).to(dev())
    with torch.no_grad():
        r.gate_w.copy_(on_dev(a["gate_w"], "float32"))
    idx, w, cnt = r(on_dev(a["x"], "float32"))
    assert np.array_equal(idx.cpu().numpy(), a["idx"])
    assert np.array_equal(cnt.cpu().numpy(), a["cnt"])
    assert_rel(w, torch.from_numpy(a["w"]), 1e-5, "w")
    assert_rel(r._last_logits, torch.from_numpy(a["last_logits"]), 1e-5, "_last_logits")
    p = r.last_profile
    assert abs(p.tokens_per_expert_mean - float(a["tokens_per_expert_mean"])) < 1e-5
    assert abs(p.tokens_per_expert_std - float(a["tokens_per_expert_std"])) < 1e-4
    assert abs(p.expert_load_imbalance - float(a["expert_load_imbalance"])) < 1e-5
    assert abs(p.router_z_loss - float(a["router_z_loss"])) <= 1e-5 * float(a["router_z_loss"])
