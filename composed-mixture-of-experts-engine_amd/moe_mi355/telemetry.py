"""Per-step routing telemetry kept on the device.

The reference's train step builds its routing telemetry on the host every step: it reads the router's
``RouterProfile`` (eight ``.item()`` reads, moe-engine/pkg/kernels/moe_router.py L:690-745) and the dispatch
counts (``(dc == 0).sum().item()`` ..., moe-engine/train.py L:360-399).  ``RoutingTelemetry`` keeps the same
fields as fixed-layout records in a ring buffer in device memory: ``record`` appends one with one kernel launch
(``moe_telemetry_record``) on the current stream, with no host synchronisation, and ``flush`` copies the ring
to the host at once and returns the records appended since the last flush as dicts keyed like the
reference's ``StepRecord.routing`` block (train.py L:382-392).  The ring's write cursor is a device counter
that the kernel advances, so a ``record`` captured in a HIP graph appends a new record on every replay.

With ``MoERouter(..., sync_profile=False)`` a training step then has no routing-related synchronisation at
all; ``MoERouter(..., z_loss_coef=w)`` makes the z-loss a differentiable term (``router.last_z_loss``), which is
what the reference's ``z_loss_weight`` wiring (train.py L:305-318, a detached float) stands in for.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from . import _lib as L

# Record layout (floats), as written by k_telemetry_record.
FIELDS = (
    "step",
    "expert_load_imbalance",
    "router_z_loss",
    "tokens_per_expert_mean",
    "tokens_per_expert_std",
    "dead_expert_count",
    "active_experts",
    "routing_efficiency",
    "dropped_token_fraction",
    "aux_statistic",
    "nonfinite_logits",
    "dispatched_slots",
)
_INT_FIELDS = ("step", "dead_expert_count", "active_experts", "nonfinite_logits", "dispatched_slots")


def records_from_rows(rows: torch.Tensor) -> List[Dict[str, float]]:
    """Host float32 rows [n, >= len(FIELDS)] of the ring -> one dict per record (counts as ints; the step is
    stored as int32 bits)."""
    rows = rows.contiguous()
    steps = rows.view(torch.int32)[:, 0].tolist()
    out = []
    for r, st in zip(rows.tolist(), steps):
        d = {}
        for i, name in enumerate(FIELDS):
            d[name] = int(round(r[i])) if name in _INT_FIELDS else float(r[i])
        d["step"] = int(st)
        out.append(d)
    return out


class RoutingTelemetry:
    """Ring buffer of ``capacity`` per-step routing records in device memory."""

    def __init__(self, capacity: int = 1024, device: Optional[torch.device] = None):
        if capacity < 1:
            raise ValueError("capacity must be >= 1")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        L.require_device(torch.empty(0, device=dev))
        self.capacity = int(capacity)
        self.fields = int(L.load().moe_telemetry_fields())
        # capacity records, then one row whose first word (int32) is the device write cursor
        self._buf = torch.zeros((self.capacity + 1, self.fields), dtype=torch.float32, device=dev)
        self.ring = self._buf[: self.capacity]
        self.flushed = 0  # records appended before the last flush

    def record(self, router, step: Optional[int] = None, layer=None, capacity_factor: Optional[float] = None) -> None:
        """Append the routing record of ``router``'s last forward (a ``MoERouter``).  ``layer`` (a
        ``DistributedMoELayer``) supplies the capacity factor and, when it drops tokens, the drop count;
        otherwise ``capacity_factor`` (default 1.0) is used and nothing is counted as dropped."""
        stats = getattr(router, "last_stats", None)
        if stats is None:
            raise RuntimeError("RoutingTelemetry.record: the router has not run a forward yet")
        N = int(getattr(router, "last_num_tokens", 0))
        ndrop = None
        cf = 1.0 if capacity_factor is None else float(capacity_factor)
        if layer is not None:
            cf = float(layer.capacity_factor) if capacity_factor is None else cf
            plan = getattr(layer, "last_plan", None)
            if getattr(layer, "capacity_dropping", False) and plan is not None:
                ndrop = plan.ndrop
        dev = L.require_device(stats, self._buf, ndrop)
        rc = L.load().moe_telemetry_record(
            stats.data_ptr(), int(router.num_experts), N, int(router.top_k), cf, L.ptr(ndrop),
            -1 if step is None else int(step), self._buf.data_ptr(), self.capacity, L.stream_of(dev),
        )
        L.check(rc, "moe_telemetry_record")

    def flush(self) -> List[Dict[str, float]]:
        """Records appended since the last flush (the newest ``capacity`` of them), oldest first: one
        device-to-host copy of the ring and its cursor."""
        host = self._buf.to("cpu")
        written = int(host.view(torch.int32)[self.capacity, 0])
        n = min(written - self.flushed, self.capacity)
        self.flushed = written
        if n <= 0:
            return []
        first = (written - n) % self.capacity
        idx = [(first + i) % self.capacity for i in range(n)]
        return records_from_rows(host[idx])
