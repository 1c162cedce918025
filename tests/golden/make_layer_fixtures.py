#!/usr/bin/env python3
"""Write the golden fixtures of the MoE layer and router from the reference itself.

Run in the build container only (the reference tree is not present on the GPU box):

    python tests/golden/make_layer_fixtures.py [/root/reference/moe-engine]

It imports the reference's ``DistributedMoELayer`` (``pkg/distributed/moe_layer.py`` L:206-360, through the
``pkg.distributed.parallel_mesh`` shim its own tests use) and ``MoERouter`` (``pkg/kernels/moe_router.py``
L:618-746) on the CPU, runs them on small seeded inputs and stores inputs and outputs as ``.npz`` files next
to this script.  These pin what no closed form or restatement pins independently:

* the positional row layout of the layer -- tokens stable-sorted by first choice, repeated K times, cut into
  E equal chunks, remainder rows left zero (L:317-337) -- and its combine ``combined_sorted[k::K]``
  (L:349-353), with N*K % E != 0, K = 1..3, capacity drops on and off.  Most cases use a chunk that is not a
  multiple of K: with one that is (and no drops), or with K = 1, every token's output is independent of its
  routing weights and the exact gate gradient is zero;
* the bf16 per-k accumulation of the combine (bf16 products added one k at a time);
* the ``bias=True`` router, which recomputes the routing in fp32 under no_grad (L:671-687);
* ``torch.topk``'s order under exact ties (an all-zero gate), and the layer output under them.

Every array is stored as float32 / int64 / bool (bf16 values are exact in float32); ``config`` is a JSON
string.  Nothing here is product code; nothing at run time reads the reference.
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/moe-engine"


def _import_reference():
    # The reference's top-level package is also called ``pkg``: put its tree first and make sure no other
    # ``pkg`` was imported in this process.
    if "pkg" in sys.modules:
        raise RuntimeError("another 'pkg' package is already imported; run this script on its own")
    sys.path.insert(0, REF)
    import torch  # noqa: F401

    from pkg.distributed.parallel_mesh import DistributedMoELayer, build_topology  # type: ignore
    from pkg.distributed.moe_layer import compute_capacity_drop_mask  # type: ignore
    from pkg.kernels.moe_router import MoERouter  # type: ignore

    return DistributedMoELayer, build_topology, compute_capacity_drop_mask, MoERouter


def _np(t):
    import torch

    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy().copy()


LAYER_CASES = [
    # name, dtype, N, H, F, E, K, capacity_factor, capacity_dropping, gate ("randn" | "zero"), seed
    ("layer_f32_rem", "float32", 13, 32, 64, 5, 2, 1.25, False, "randn", 11),
    ("layer_f32_k1_drop", "float32", 10, 32, 32, 4, 1, 1.0, True, "randn", 12),
    ("layer_f32_k3_drop", "float32", 11, 48, 64, 4, 3, 0.5, True, "randn", 13),
    ("layer_bf16_k2", "bfloat16", 12, 64, 64, 8, 2, 1.25, False, "randn", 14),
    ("layer_bf16_k3_drop", "bfloat16", 15, 64, 96, 6, 3, 0.5, True, "randn", 15),
    ("layer_bf16_kE", "bfloat16", 11, 32, 64, 3, 3, 1.25, False, "randn", 16),
    ("layer_f32_ties", "float32", 12, 32, 32, 8, 3, 1.25, False, "zero", 17),
]

ROUTER_CASES = [
    # name, dtype, N, H, E, K, bias, gate, seed
    ("router_bias_f32", "float32", 32, 64, 8, 2, True, "randn", 21),
    ("router_bias_bf16", "bfloat16", 32, 64, 16, 4, True, "randn", 22),
    ("router_ties_f32", "float32", 4, 16, 8, 3, False, "zero", 23),
    ("router_profile_f32", "float32", 64, 32, 16, 2, False, "randn", 24),
]


def _top_margin(x, gate_w, K):
    """Smallest gap between consecutive sorted float64 probabilities among each token's first K+1."""
    import torch

    p = torch.softmax(x.double() @ gate_w.double(), dim=-1)
    s = torch.sort(p, dim=-1, descending=True).values[:, : min(K + 1, p.shape[1])]
    return float((s[:, :-1] - s[:, 1:]).min()) if s.shape[1] > 1 else float("inf")


def make_layer(case, DistributedMoELayer, build_topology, compute_capacity_drop_mask):
    """The case at the first seed from its own (step 1000) whose routing has no near tie and which drops
    slots when the case asks for drops."""
    name, seed0 = case[0], case[-1]
    for seed in range(seed0, seed0 + 100000, 1000):
        res = _layer_at(case[:-1] + (seed,), DistributedMoELayer, build_topology, compute_capacity_drop_mask)
        if res is not None:
            return res
    raise RuntimeError(f"{name}: no usable seed")


def _layer_at(case, DistributedMoELayer, build_topology, compute_capacity_drop_mask):
    import torch

    name, dts, N, H, F, E, K, cf, drop_on, gate, seed = case
    dt = getattr(torch, dts)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, H, generator=g)
    gate_w = torch.randn(H, E, generator=g) * 0.5 if gate == "randn" else torch.zeros(H, E)
    w_gate = torch.randn(E, F, H, generator=g) / math.sqrt(H)
    w_up = torch.randn(E, F, H, generator=g) / math.sqrt(H)
    w_down = torch.randn(E, H, F, generator=g) / math.sqrt(F)
    grad_out = torch.randn(N, H, generator=g)
    # round every input to the case's dtype once; the stored float32 copies are then exact
    x, gate_w, w_gate, w_up, w_down, grad_out = (t.to(dt) for t in (x, gate_w, w_gate, w_up, w_down, grad_out))
    if gate == "randn" and _top_margin(x, gate_w, K) <= 1e-4:
        return None

    torch.manual_seed(seed)
    topo = build_topology(dp_size=1, ep_size=1, device_type="cpu")
    layer = DistributedMoELayer(H, F, E, K, topo, capacity_factor=cf, capacity_dropping=drop_on, dtype=dt)
    with torch.no_grad():
        layer.router.gate_w.copy_(gate_w)
        for i, ex in enumerate(layer.experts):
            ex.w_gate.weight.copy_(w_gate[i])
            ex.w_up.weight.copy_(w_up[i])
            ex.w_down.weight.copy_(w_down[i])
    seen = {}

    def hook(_mod, _inp, out):
        seen["idx"], seen["w"], seen["cnt"] = (o.detach().clone() for o in out)

    layer.router.register_forward_hook(hook)
    xin = x.clone().requires_grad_(True)
    out = layer(xin)
    out.backward(grad_out)
    idx = seen["idx"]
    if drop_on:
        cap = math.ceil(cf * N * K / E)
        drop = compute_capacity_drop_mask(idx, E, cap)
    else:
        drop = torch.zeros(N, K, dtype=torch.bool)
    if drop_on and not bool(drop.any()):
        return None
    arrays = {
        "x": _np(x), "gate_w": _np(gate_w), "w_gate": _np(w_gate), "w_up": _np(w_up), "w_down": _np(w_down),
        "grad_out": _np(grad_out),
        "idx": _np(idx).astype(np.int64), "w": _np(seen["w"]), "cnt": _np(seen["cnt"]).astype(np.int64),
        "drop": _np(drop).astype(bool), "out": _np(out),
        "dx": _np(xin.grad), "dgate_w": _np(layer.router.gate_w.grad),
        "dw_gate": np.stack([_np(ex.w_gate.weight.grad) for ex in layer.experts]),
        "dw_up": np.stack([_np(ex.w_up.weight.grad) for ex in layer.experts]),
        "dw_down": np.stack([_np(ex.w_down.weight.grad) for ex in layer.experts]),
        "dropped_fraction": np.float64(layer.last_dropped_token_fraction),
    }
    cfg = {"kind": "layer", "dtype": dts, "N": N, "H": H, "F": F, "E": E, "K": K, "capacity_factor": cf,
           "capacity_dropping": drop_on, "gate": gate, "seed": seed}
    return name, cfg, arrays


def make_router(case, MoERouter):
    import torch

    name, dts, N, H, E, K, bias, gate, seed = case
    dt = getattr(torch, dts)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, H, generator=g).to(dt)
    gate_w = (torch.randn(H, E, generator=g) * 0.3 if gate == "randn" else torch.zeros(H, E)).to(dt)
    b = torch.randn(E, generator=g).to(dt) if bias else None
    torch.manual_seed(seed)
    r = MoERouter(H, E, K, bias=bias, dtype=dt)
    with torch.no_grad():
        r.gate_w.copy_(gate_w)
        if bias:
            r.bias.copy_(b)
    xin = x.clone().requires_grad_(True)
    idx, w, cnt = r(xin)
    prof = r.last_profile
    arrays = {
        "x": _np(x), "gate_w": _np(gate_w), "idx": _np(idx).astype(np.int64), "w": _np(w),
        "cnt": _np(cnt).astype(np.int64), "last_logits": _np(r._last_logits),
        "w_requires_grad": np.bool_(w.requires_grad),
        "tokens_per_expert_mean": np.float64(prof.tokens_per_expert_mean),
        "tokens_per_expert_std": np.float64(prof.tokens_per_expert_std),
        "expert_load_imbalance": np.float64(prof.expert_load_imbalance),
        "router_z_loss": np.float64(prof.router_z_loss),
    }
    if bias:
        arrays["bias"] = _np(b)
    cfg = {"kind": "router", "dtype": dts, "N": N, "H": H, "E": E, "K": K, "bias": bias, "gate": gate,
           "seed": seed}
    return name, cfg, arrays


def main():
    DistributedMoELayer, build_topology, compute_capacity_drop_mask, MoERouter = _import_reference()
    import torch

    torch.set_num_threads(1)
    written = []
    for case in LAYER_CASES:
        written.append(make_layer(case, DistributedMoELayer, build_topology, compute_capacity_drop_mask))
    for case in ROUTER_CASES:
        written.append(make_router(case, MoERouter))
    for name, cfg, arrays in written:
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, config=np.array(json.dumps(cfg, sort_keys=True)), **arrays)
        print(f"wrote {os.path.relpath(path)}")


if __name__ == "__main__":
    main()
