"""Single-GPU MoE layer and router interface with the reference's import paths
(``pkg.distributed.{moe_layer,router,mesh}``)."""

from pkg.distributed.mesh import ParallelTopology, build_topology
from pkg.distributed.moe_layer import DistributedMoELayer, compute_capacity_drop_mask
from pkg.distributed.router import MoERouterInterface, RouterStats

__all__ = [
    "ParallelTopology",
    "build_topology",
    "DistributedMoELayer",
    "compute_capacity_drop_mask",
    "MoERouterInterface",
    "RouterStats",
]
