"""Degenerate single-GPU topology (reference: moe-engine/pkg/distributed/mesh.py
L:60-162, build_topology L:241-326).

The hot path runs on one GPU: expert, tensor, pipeline and data parallelism
are outside this build, so only the one-rank topology exists.  Asking for a
larger extent raises ``NotImplementedError`` instead of silently running a
different layout.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch


@dataclass(frozen=True)
class ParallelTopology:
    world_size: int = 1
    rank: int = 0
    dp_size: int = 1
    ep_size: int = 1
    tp_size: int = 1
    pp_size: int = 1
    mesh: Optional[object] = field(default=None, compare=False, repr=False)
    device: torch.device = field(default_factory=lambda: torch.device("cuda" if torch.cuda.is_available() else "cpu"))

    def __post_init__(self):
        if max(self.world_size, self.dp_size, self.ep_size, self.tp_size, self.pp_size) != 1:
            raise NotImplementedError(
                "this build runs the MoE hot path on one GPU; multi-rank topologies (the expert-parallel "
                "all-to-all, TP/PP/DP) are outside it"
            )

    @property
    def dp_rank(self) -> int:
        return 0

    @property
    def tp_rank(self) -> int:
        return 0

    @property
    def pp_rank(self) -> int:
        return 0

    @property
    def ep_rank(self) -> int:
        return 0

    def experts_on_this_rank(self, total_experts: int) -> List[int]:
        return list(range(total_experts))

    def is_first_pp_stage(self) -> bool:
        return True

    def is_last_pp_stage(self) -> bool:
        return True

    def validate_world_size(self) -> None:
        return None


def build_topology(dp_size: int = 1, ep_size: int = 1, tp_size: int = 1, pp_size: int = 1,
                   device_type: str = "cuda") -> ParallelTopology:
    """One-rank topology on the current GPU (reference L:274-288)."""
    if max(dp_size, ep_size, tp_size, pp_size) != 1:
        raise NotImplementedError("only the single-GPU topology (all sizes 1) is supported by this build")
    dev = torch.device(device_type if (device_type == "cuda" and torch.cuda.is_available()) else "cpu")
    return ParallelTopology(device=dev)
