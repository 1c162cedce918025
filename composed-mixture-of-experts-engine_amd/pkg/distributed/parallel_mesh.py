"""``pkg.distributed.parallel_mesh``: the import path the reference keeps for backward compatibility
(moe-engine/pkg/distributed/parallel_mesh.py L:27-60) and that its layer tests import
(tests/test_distributed.py L:23-26).  Re-exports the single-GPU hot-path names; the multi-rank primitives
it also re-exports in the reference (TP linears, pipeline stages, FSDP, EP collectives) are outside this
build."""

from pkg.distributed.mesh import ParallelTopology, build_topology  # noqa: F401
from pkg.distributed.moe_layer import (  # noqa: F401
    DistributedMoELayer,
    _SwiGLUExpert,
    compute_capacity_drop_mask,
)

__all__ = ["ParallelTopology", "build_topology", "DistributedMoELayer", "compute_capacity_drop_mask"]
