"""Router interface with the reference's API (moe-engine/pkg/distributed/router.py).

``MoERouterInterface(hidden_dim, num_experts, top_k, capacity_factor=1.25,
dtype)`` -> ``forward(tokens [N,H]) -> RouterStats`` and
``capacity_budget(n)``; same validation and error messages as the reference
(L:136-149, L:190-212).  The statistics come from the router's single
device-to-host copy instead of separate ``.item()`` calls.
"""

from __future__ import annotations

import math
import warnings
from dataclasses import dataclass

import torch
import torch.nn as nn

__all__ = ["MoERouterInterface", "RouterStats"]


@dataclass
class RouterStats:
    expert_indices: torch.Tensor
    combine_weights: torch.Tensor
    dispatch_counts: torch.Tensor
    load_imbalance: float
    router_z_loss: float
    used_triton: bool
    kernel_ms: float
    tokens_per_expert_mean: float
    tokens_per_expert_std: float


class MoERouterInterface(nn.Module):
    def __init__(
        self,
        hidden_dim: int,
        num_experts: int,
        top_k: int,
        capacity_factor: float = 1.25,
        dtype: torch.dtype = torch.float32,
    ) -> None:
        super().__init__()
        if top_k > num_experts:
            raise ValueError(
                f"MoERouterInterface: top_k ({top_k}) must be ≤ num_experts ({num_experts}). "
                "Each token can only be routed to at most num_experts experts."
            )
        if capacity_factor < 1.0:
            warnings.warn(
                f"capacity_factor={capacity_factor} < 1.0 will silently drop tokens "
                "when routing is imbalanced. Consider using ≥ 1.0.",
                UserWarning,
                stacklevel=2,
            )
        self.hidden_dim = hidden_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.capacity_factor = capacity_factor
        from pkg.kernels.moe_router import MoERouter

        self._kernel_router = MoERouter(hidden_dim=hidden_dim, num_experts=num_experts, top_k=top_k, dtype=dtype)

    def extra_repr(self) -> str:
        return (
            f"hidden_dim={self.hidden_dim}, num_experts={self.num_experts}, "
            f"top_k={self.top_k}, capacity_factor={self.capacity_factor}"
        )

    def forward(self, tokens: torch.Tensor) -> RouterStats:
        if tokens.dim() != 2:
            raise ValueError(
                f"MoERouterInterface.forward expects 2D input [N, H], "
                f"got shape {list(tokens.shape)}. "
                "Flatten [B, S, H] → [B*S, H] before calling."
            )
        N, H = tokens.shape
        if H != self.hidden_dim:
            raise ValueError(f"Token hidden dim {H} ≠ router hidden_dim {self.hidden_dim}.")
        idx, weights, dispatch_counts = self._kernel_router(tokens)
        kr = self._kernel_router
        prof = kr.last_profile  # resolves the forward's statistics (one device-to-host copy)
        head = kr.last_stats_host
        total = int(round(float(head[5])))
        expected = N * self.top_k
        if total != expected:
            raise RuntimeError(
                f"Token conservation violation: dispatched {total} "
                f"tokens but expected {expected} (N={N}, K={self.top_k}). "
                "This indicates a bug in the routing kernel."
            )
        return RouterStats(
            expert_indices=idx,
            combine_weights=weights,
            dispatch_counts=dispatch_counts,
            load_imbalance=prof.expert_load_imbalance,
            router_z_loss=prof.router_z_loss,
            used_triton=prof.used_triton,
            kernel_ms=prof.kernel_ms,
            tokens_per_expert_mean=prof.tokens_per_expert_mean,
            tokens_per_expert_std=prof.tokens_per_expert_std,
        )

    def capacity_budget(self, num_tokens: int) -> int:
        """``ceil(capacity_factor * num_tokens * top_k / num_experts)`` (L:234-242)."""
        return math.ceil(self.capacity_factor * num_tokens * self.top_k / self.num_experts)
