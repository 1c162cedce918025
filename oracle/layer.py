"""Float64 CPU restatement of the MoE layer (router -> dispatch -> SwiGLU experts -> combine).

TEST INFRASTRUCTURE ONLY.

Reference: ``moe-engine/pkg/distributed/moe_layer.py`` L:166-198 (SwiGLU
expert), L:264-360 (layer forward at ep=1, tp=1) and
``pkg/distributed/tensor_parallel.py`` L:117-121, 195-199 (``F.linear`` with
[out, in] weights at tp=1).  The backward is torch autograd over this float64
forward (the reference's layer backward is autograd too).

Pinning: the reference layout's index arithmetic is pinned through
``oracle.plan`` (brute force) and, when present, golden vectors written from
the reference itself (``tests/golden/``); ``swiglu`` is ``F.linear``/``silu``;
the routed layout is checked against a per-expert brute-force loop in
``tests/test_oracle_layer.py``.
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F

from oracle import plan as _plan
from oracle import router as _router

_F64 = torch.float64


def swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor) -> torch.Tensor:
    """w_down(silu(w_gate(x)) * w_up(x)) with [out, in] weights (moe_layer.py L:197-198)."""
    return F.linear(F.silu(F.linear(x, w_gate)) * F.linear(x, w_up), w_down)


def layer_fwd_bwd(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    w_gate: torch.Tensor,
    w_up: torch.Tensor,
    w_down: torch.Tensor,
    top_k: int,
    grad_out: Optional[torch.Tensor] = None,
    capacity_factor: float = 1.25,
    capacity_dropping: bool = False,
    layout: int = _plan.LAYOUT_REFERENCE,
    alpha: float = 0.0,
    beta: float = 0.0,
    bias: Optional[torch.Tensor] = None,
    idx_override: Optional[torch.Tensor] = None,
) -> Dict[str, object]:
    """Layer forward (and backward when ``grad_out`` is given) in float64.

    ``w_gate``/``w_up``: [E, F, H]; ``w_down``: [E, H, F].  Loss for the
    backward is ``sum(out * grad_out) + aux + z``.  ``idx_override`` pins the
    routing (e.g. to the device's routing) so a near-tie token cannot make
    the comparison diverge.
    """
    need_grad = grad_out is not None
    xs = x.detach().to("cpu", _F64).reshape(-1, x.shape[-1]).requires_grad_(need_grad)
    gw = gate_w.detach().to("cpu", _F64).requires_grad_(need_grad)
    Wg = w_gate.detach().to("cpu", _F64).requires_grad_(need_grad)
    Wu = w_up.detach().to("cpu", _F64).requires_grad_(need_grad)
    Wd = w_down.detach().to("cpu", _F64).requires_grad_(need_grad)
    N, H = xs.shape
    E = gw.shape[1]
    K = top_k

    # ---- router (moe_router.py L:257-271, autograd stands in for L:274-291)
    logits = xs @ gw
    if bias is not None:
        logits = logits + bias.detach().to("cpu", _F64)
    probs = torch.softmax(logits, dim=-1)
    if idx_override is None:
        _, idx = _router.topk_lowest_index(probs.detach(), K)
    else:
        idx = idx_override.detach().to("cpu").long()
    v = probs.gather(1, idx)
    w = v / v.sum(-1, keepdim=True).clamp_min(1e-30)
    cnt = _router.dispatch_counts(idx, E)

    # ---- capacity drop (moe_layer.py L:300-306)
    drop = np.zeros((N, K), dtype=bool)
    if capacity_dropping:
        cap = math.ceil(capacity_factor * N * K / E)
        drop = _plan.drop_mask(idx.numpy(), cap)
        if drop.any():
            w = w.masked_fill(torch.from_numpy(drop), 0.0)
    dropped_fraction = float(drop.mean()) if drop.size else 0.0

    # ---- dispatch plan
    if layout == _plan.LAYOUT_REFERENCE:
        pl = _plan.plan_reference(idx.numpy(), E)
    else:
        pl = _plan.plan_routed(idx.numpy(), E, drop)
    row_slot = torch.from_numpy(pl["row_slot"])
    slot_row = torch.from_numpy(pl["slot_row"])
    offsets = pl["offsets"]
    R = int(pl["n_rows"])

    # ---- permute + experts (moe_layer.py L:318-336)
    xp = xs[row_slot // K] if R else xs.new_zeros((0, H))
    ys = []
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo < hi:
            ys.append(swiglu(xp[lo:hi], Wg[e], Wu[e], Wd[e]))
    tail = R - int(offsets[E])
    if tail > 0:
        ys.append(xs.new_zeros((tail, H)))
    Y = torch.cat(ys, 0) if ys else xs.new_zeros((0, H))

    # ---- weighted combine (moe_layer.py L:349-353)
    sr = slot_row.view(N, K)
    out = xs.new_zeros((N, H))
    for k in range(K):
        valid = sr[:, k] >= 0
        rows = sr[:, k].clamp_min(0)
        contrib = w[:, k : k + 1] * Y[rows] if R else xs.new_zeros((N, H))
        out = out + torch.where(valid[:, None], contrib, torch.zeros_like(contrib))

    aux = _router.aux_loss(probs, cnt, K, alpha) if alpha else torch.zeros((), dtype=_F64)
    z = _router.z_loss(logits, beta) if beta else torch.zeros((), dtype=_F64)

    res: Dict[str, object] = {
        "out": out.detach().reshape(x.shape),
        "idx": idx,
        "w": w.detach(),
        "drop": drop,
        "cnt": cnt,
        "plan": pl,
        "aux": aux.detach(),
        "z": z.detach(),
        "dropped_fraction": dropped_fraction,
        "Y": Y.detach(),
    }
    if need_grad:
        g = grad_out.detach().to("cpu", _F64).reshape(N, H)
        loss = (out * g).sum()
        if alpha:
            loss = loss + aux
        if beta:
            loss = loss + z
        loss.backward()
        res.update(
            dx=xs.grad.reshape(x.shape),
            dgate_w=gw.grad,
            dw_gate=Wg.grad,
            dw_up=Wu.grad,
            dw_down=Wd.grad,
        )
    return res
