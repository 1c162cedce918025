"""``RMSNorm`` and ``ToyMoEBlock`` (moe-engine/pkg/models/moe.py L:63-126) on the fused kernels.

``ToyMoEBlock.forward`` is ``x + moe(norm(x))`` (L:125-126).  Here the norm and the router run as one
operation (:class:`moe_mi355.norm.NormRouterCore`): the hidden state is read once for both, the router
routes the bf16-rounded normalised rows exactly as it would route ``norm(x)``, and the expert path takes
those same rows.  Modules whose experts are not the built-in SwiGLU, or shapes the norm kernels do not
take, use the plain composition ``moe(norm(x))``.
"""

from __future__ import annotations

import torch
from torch import nn

from moe_mi355.norm import RMSNormFn
from pkg.distributed.moe_layer import DistributedMoELayer

_NORM_MAX_H = 8192


class RMSNorm(nn.Module):
    """Root-mean-square layer normalisation (L:63-86): ``weight`` [dim] (ones), ``eps`` (1e-5).

    ``forward(x)`` returns ``((x * rsqrt(mean(x^2, -1) + eps)) * weight).to(x.dtype)`` with fp32 arithmetic,
    one HIP kernel (the reference's torch composition makes several fp32 passes)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def extra_repr(self) -> str:
        return f"dim={self.weight.shape[0]}, eps={self.eps}"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        H = x.shape[-1]
        return RMSNormFn.apply(x.reshape(-1, H), self.weight, self.eps).reshape(x.shape)


class ToyMoEBlock(nn.Module):
    """Single MoE transformer block: RMSNorm + DistributedMoELayer + residual (L:89-126)."""

    def __init__(
        self,
        hidden_dim: int,
        ffn_dim: int,
        num_experts: int,
        top_k: int,
        topology,
        capacity_factor: float = 1.25,
        dtype: torch.dtype = torch.float32,
        **layer_kwargs,
    ):
        super().__init__()
        self.norm = RMSNorm(hidden_dim)
        self.moe = DistributedMoELayer(
            hidden_dim=hidden_dim,
            ffn_dim=ffn_dim,
            num_experts=num_experts,
            top_k=top_k,
            topology=topology,
            capacity_factor=capacity_factor,
            dtype=dtype,
            **layer_kwargs,
        )

    def _fused(self, x: torch.Tensor) -> bool:
        return (
            x.is_cuda
            and x.shape[-1] <= _NORM_MAX_H
            and x.shape[-1] % 8 == 0
            and x.dtype in (torch.float32, torch.bfloat16)
            and self.norm.weight.dtype in (torch.float32, torch.bfloat16)
            and self.moe.router.gate_w.dtype == x.dtype
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._fused(x):
            out = self.moe.forward_normed(x, self.norm.weight, self.norm.eps)
        else:
            out = self.moe(self.norm(x))
        return x + out
