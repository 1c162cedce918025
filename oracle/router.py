"""Float64 CPU restatement of the reference top-k router -- TEST INFRASTRUCTURE ONLY.

Reference: ``moe-engine/pkg/kernels/moe_router.py``.

Pinning (each checked in ``tests/test_oracle_router.py``):

* ``route_fwd``          -- torch.softmax / torch.topk in float64 (library
  routines) and the reference's forward-tolerance cases
  (``tests/test_kernels.py`` L:32-59): indices equal, weights within 1e-5.
* ``route_bwd``          -- torch autograd through the float64 forward math,
  exactly the reference's ``test_backward_tolerance``
  (``tests/test_kernels.py`` L:62-108), plus the closed-form invariant that
  ``grad_w = const`` gives zero gradient (weights sum to one).
* ``load_imbalance``     -- golden values 1.0 / 4.0 / 1.6 / zeros->1.0
  (``tests/test_routing_quality.py`` L:36-60).
* ``z_stat``             -- zero logits give ln(E)^2
  (``tests/test_routing_quality.py`` L:75-81) and torch.logsumexp.
* ``aux_loss`` / ``z_loss`` and their logit gradients -- closed forms (not in
  the reference), checked against torch autograd in float64.
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch

_F64 = torch.float64


def topk_lowest_index(probs: torch.Tensor, k: int):
    """Top-k along the last dim, values descending, exact ties -> lowest index first.

    The reference calls ``torch.topk(probs, k, largest=True)`` (moe_router.py
    L:268), whose tie order is unspecified; this restatement fixes the
    tie-break the HIP kernel uses (lowest expert index wins) via a stable
    descending sort.
    """
    order = torch.sort(-probs, dim=-1, stable=True).indices
    idx = order[..., :k]
    return probs.gather(-1, idx), idx


def route_fwd(
    tokens: torch.Tensor,
    gate_w: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
) -> Dict[str, torch.Tensor]:
    """Router forward in float64.

    Restates ``_reference_route_fp64`` (moe_router.py L:257-271):
    logits = X @ W (+ bias, as in the bias branch L:677-687), p = softmax,
    top-k of p (descending), w = v / max(sum v, 1e-30).

    Returns float64 ``logits``, ``probs``, ``w``, long ``idx`` and the per-token
    top-k ``margin``: the smallest gap between consecutive sorted
    probabilities among the first k+1 (first k when k == E).  Index parity is
    only asserted where this margin exceeds the tolerance.
    """
    x64 = tokens.detach().to("cpu", _F64)
    w64 = gate_w.detach().to("cpu", _F64)
    logits = x64 @ w64
    if bias is not None:
        logits = logits + bias.detach().to("cpu", _F64)
    probs = torch.softmax(logits, dim=-1)
    vals, idx = topk_lowest_index(probs, k)
    denom = vals.sum(-1, keepdim=True).clamp_min(1e-30)
    w = vals / denom
    E = probs.shape[-1]
    srt = torch.sort(probs, dim=-1, descending=True).values
    m = min(k + 1, E)
    if m >= 2:
        gaps = srt[:, : m - 1] - srt[:, 1:m]
        margin = gaps.min(dim=-1).values
    else:
        margin = torch.full((probs.shape[0],), float("inf"), dtype=_F64)
    return {"logits": logits, "probs": probs, "idx": idx.long(), "w": w, "margin": margin}


def route_bwd(logits: torch.Tensor, idx: torch.Tensor, grad_w: torch.Tensor) -> torch.Tensor:
    """d(loss)/d(logits) through softmax -> top-k -> renormalise, float64.

    Restates ``_reference_backward_fp64`` (moe_router.py L:274-291):
    S = max(sum v, 1e-30); grad_v = gw/S - <gw, v>/S^2; grad_p = scatter(grad_v);
    grad_l = p * (grad_p - <grad_p, p>).
    """
    l64 = logits.detach().to("cpu", _F64)
    p = torch.softmax(l64, dim=-1)
    idx = idx.detach().to("cpu").long()
    v = p.gather(1, idx)
    S = v.sum(-1, keepdim=True).clamp_min(1e-30)
    gw = grad_w.detach().to("cpu", _F64)
    gwv = (gw * v).sum(-1, keepdim=True)
    grad_v = gw / S - gwv / (S * S)
    grad_p = torch.zeros_like(p)
    grad_p.scatter_add_(1, idx, grad_v)
    inner = (grad_p * p).sum(-1, keepdim=True)
    return p * (grad_p - inner)


def dispatch_counts(idx: torch.Tensor, num_experts: int) -> torch.Tensor:
    """Per-expert slot counts, before any capacity drop (moe_router.py L:690)."""
    return torch.bincount(idx.detach().to("cpu").reshape(-1), minlength=num_experts).long()


def load_imbalance(cnt: torch.Tensor) -> float:
    """max(cnt) / mean(cnt), 1.0 when the mean is ~0 (moe_router.py L:594-600)."""
    c = cnt.detach().to("cpu", _F64)
    mean = float(c.mean())
    if mean < 1e-9:
        return 1.0
    return float(c.max()) / mean


def z_stat(logits: torch.Tensor) -> float:
    """mean_t(logsumexp(l_t)^2) -- the reference's telemetry z-loss (moe_router.py L:603-612)."""
    lse = torch.logsumexp(logits.detach().to("cpu", _F64), dim=-1)
    return float((lse * lse).mean())


# --------------------------------------------------------------------------
# Load-balance aux loss and differentiable z-loss.  The reference has neither
# (its z-loss is a Python float, moe_router.py L:603-612, added without a
# gradient in train.py L:305-318); these are the Switch/GShard closed forms:
#   f_e = cnt_e / (N K)           (pre-drop counts, = dispatch_cnt / (N K))
#   P_e = (1/N) sum_t p[t, e]
#   aux = alpha * E * sum_e f_e P_e
#   z   = beta * (1/N) sum_t lse_t^2
#   d aux / d l[t, j] = (alpha E / N) p[t, j] (f_j - sum_e p[t, e] f_e)
#   d z   / d l[t, j] = (2 beta / N) lse_t p[t, j]
# --------------------------------------------------------------------------


def aux_loss(probs: torch.Tensor, cnt: torch.Tensor, k: int, alpha: float) -> torch.Tensor:
    N, E = probs.shape
    f = cnt.to(_F64) / float(N * k)
    P = probs.to(_F64).mean(0)
    return alpha * E * (f * P).sum()


def aux_grad_logits(probs: torch.Tensor, cnt: torch.Tensor, k: int, alpha: float) -> torch.Tensor:
    N, E = probs.shape
    p = probs.to(_F64)
    f = cnt.to(_F64) / float(N * k)
    pf = (p * f).sum(-1, keepdim=True)
    return (alpha * E / N) * p * (f[None, :] - pf)


def z_loss(logits: torch.Tensor, beta: float) -> torch.Tensor:
    lse = torch.logsumexp(logits.to(_F64), dim=-1)
    return beta * (lse * lse).mean()


def z_grad_logits(logits: torch.Tensor, beta: float) -> torch.Tensor:
    l64 = logits.to(_F64)
    N = l64.shape[0]
    lse = torch.logsumexp(l64, dim=-1, keepdim=True)
    p = torch.softmax(l64, dim=-1)
    return (2.0 * beta / N) * lse * p


def router_full(
    tokens: torch.Tensor,
    gate_w: torch.Tensor,
    k: int,
    grad_w: Optional[torch.Tensor] = None,
    alpha: float = 0.0,
    beta: float = 0.0,
    grad_aux: float = 1.0,
    grad_z: float = 1.0,
    bias: Optional[torch.Tensor] = None,
    idx_override: Optional[torch.Tensor] = None,
) -> Dict[str, torch.Tensor]:
    """Forward + backward of the router with aux and z losses, float64.

    Loss = sum(w * grad_w) + grad_aux * aux + grad_z * z.  dX = G @ W^T and
    dW = X^T @ G with G = d loss / d logits, as in MoERouterFunction.backward
    (moe_router.py L:545-546).  ``idx_override`` evaluates the backward at a
    given routing (used to compare gradients at the device's own routing
    when a token sits on an exact tie).
    """
    fwd = route_fwd(tokens, gate_w, k, bias=bias)
    idx = fwd["idx"] if idx_override is None else idx_override.detach().to("cpu").long()
    probs = fwd["probs"]
    v = probs.gather(1, idx)
    w = v / v.sum(-1, keepdim=True).clamp_min(1e-30)
    E = probs.shape[1]
    cnt = dispatch_counts(idx, E)
    out = dict(fwd)
    out["idx"] = idx
    out["w"] = w
    out["cnt"] = cnt
    out["aux"] = aux_loss(probs, cnt, k, alpha)
    out["z"] = z_loss(fwd["logits"], beta)
    out["z_stat"] = torch.tensor(z_stat(fwd["logits"]), dtype=_F64)
    out["imbalance"] = torch.tensor(load_imbalance(cnt), dtype=_F64)
    G = torch.zeros_like(probs)
    if grad_w is not None:
        G = G + route_bwd(fwd["logits"], idx, grad_w)
    if alpha != 0.0:
        G = G + grad_aux * aux_grad_logits(probs, cnt, k, alpha)
    if beta != 0.0:
        G = G + grad_z * z_grad_logits(fwd["logits"], beta)
    x64 = tokens.detach().to("cpu", _F64)
    w64 = gate_w.detach().to("cpu", _F64)
    out["grad_logits"] = G
    out["dX"] = G @ w64.t()
    out["dW"] = x64.t() @ G
    return out


def capacity_budget(num_tokens: int, top_k: int, num_experts: int, capacity_factor: float) -> int:
    """ceil(cf * N * K / E) (router.py L:234-242; moe_layer.py L:302)."""
    return math.ceil(capacity_factor * num_tokens * top_k / num_experts)
