"""Fused top-k MoE router (gfx950 HIP kernels); names as in the reference's
``pkg/kernels/__init__.py`` L:3-17."""

from pkg.kernels.moe_router import (
    TRITON_AVAILABLE,
    MoERouter,
    MoERouterAutograd,
    MoERouterFunction,
    RouterProfile,
    moe_topk_route,
)

__all__ = [
    "MoERouter",
    "moe_topk_route",
    "MoERouterFunction",
    "MoERouterAutograd",
    "RouterProfile",
    "TRITON_AVAILABLE",
]
