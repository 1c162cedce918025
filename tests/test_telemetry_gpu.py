"""Device routing telemetry (moe-engine/train.py L:360-399 fields) against the same fields computed on the
host from the router's own outputs; ring order and wrap-around; the record runs inside HIP graph capture
(so it has no host synchronisation)."""

from __future__ import annotations

import math

import pytest
import torch

from gpu_util import dev, say

from moe_mi355.telemetry import RoutingTelemetry
from pkg.distributed import build_topology
from pkg.distributed.moe_layer import DistributedMoELayer
from pkg.kernels.moe_router import MoERouter

pytestmark = pytest.mark.gpu


def _expected(cnt, logits, N, K, cf, dropped=0.0):
    c = cnt.double().cpu()
    E = c.numel()
    mean = c.mean().item()
    return {
        "expert_load_imbalance": 1.0 if mean < 1e-9 else c.max().item() / mean,
        "router_z_loss": torch.logsumexp(logits.double().cpu(), -1).pow(2).mean().item(),
        "tokens_per_expert_mean": mean,
        "tokens_per_expert_std": c.std().item(),
        "dead_expert_count": int((c == 0).sum().item()),
        "active_experts": int((c > 0).sum().item()),
        "routing_efficiency": c.sum().item() / max(cf * N * K, 1.0),
        "dropped_token_fraction": dropped,
        "dispatched_slots": int(c.sum().item()),
    }


def _check(rec, exp):
    for k, v in exp.items():
        if isinstance(v, int):
            assert rec[k] == v, (k, rec[k], v)
        else:
            assert rec[k] == pytest.approx(v, rel=1e-5, abs=1e-6), (k, rec[k], v)


@pytest.mark.parametrize("sync_profile", [True, False])
def test_router_record_matches_host_computation(sync_profile):
    say(f"[telemetry router] sync_profile={sync_profile}")
    N, H, E, K = 512, 256, 8, 2
    torch.manual_seed(0)
    router = MoERouter(H, E, top_k=K, dtype=torch.bfloat16, sync_profile=sync_profile).to(dev())
    bias = torch.zeros(E)
    bias[5:] = -1e4  # experts 5, 6, 7 never win a slot: three dead experts
    router.logit_bias = bias.to(dev())
    tel = RoutingTelemetry(capacity=8)
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev())
    idx, w, cnt = router(x)
    tel.record(router, step=7, capacity_factor=1.25)
    (rec,) = tel.flush()
    assert rec["step"] == 7
    exp = _expected(cnt, router._last_logits, N, K, 1.25)
    assert exp["dead_expert_count"] == 3
    _check(rec, exp)
    assert tel.flush() == []


def test_layer_record_counts_capacity_drops():
    say("[telemetry layer drops]")
    torch.manual_seed(2)
    N, H, F, E, K = 256, 128, 256, 8, 2
    layer = DistributedMoELayer(H, F, E, K, build_topology(), dtype=torch.bfloat16, capacity_factor=0.5,
                                capacity_dropping=True).to(dev())
    tel = RoutingTelemetry(capacity=4)
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev())
    layer(x)
    tel.record(layer.router, layer=layer)
    (rec,) = tel.flush()
    frac = layer.last_dropped_token_fraction
    assert frac > 0.0
    assert rec["dropped_token_fraction"] == pytest.approx(frac, rel=1e-6)
    assert rec["routing_efficiency"] == pytest.approx(N * K / (0.5 * N * K), rel=1e-6)


def test_ring_keeps_the_newest_records_in_order():
    say("[telemetry ring]")
    N, H, E, K = 64, 64, 4, 1
    router = MoERouter(H, E, top_k=K, sync_profile=False).to(dev())
    tel = RoutingTelemetry(capacity=3)
    for s in range(5):
        x = torch.randn(N, H, generator=torch.Generator().manual_seed(10 + s)).to(dev())
        router(x)
        tel.record(router, step=100 + s)
    recs = tel.flush()
    assert [r["step"] for r in recs] == [102, 103, 104]
    tel.record(router, step=105)
    assert [r["step"] for r in tel.flush()] == [105]


def test_record_is_capturable_in_a_graph():
    """Capture fails on any host synchronisation: the router forward (sync_profile=False) and the record
    replay as one graph, and each replay appends a new record (the ring's cursor is on the device)."""
    say("[telemetry graph capture]")
    N, H, E, K = 128, 64, 8, 2
    router = MoERouter(H, E, top_k=K, sync_profile=False).to(dev())
    tel = RoutingTelemetry(capacity=4)
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(20)).to(dev())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        router(x)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _idx, _w, cnt = router(x)
        tel.record(router, capacity_factor=1.0)  # step = the record's ordinal
    dead = -1
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        if i == 0:
            dead = int((cnt.cpu() == 0).sum().item())
    recs = tel.flush()
    assert [r["step"] for r in recs] == [0, 1, 2]
    for r in recs:
        assert r["dispatched_slots"] == N * K and r["dead_expert_count"] == dead
        assert not math.isnan(r["expert_load_imbalance"])
    for _ in range(3):  # records 3..5 land in slots 3, 0, 1: across the wrap-around, oldest first
        g.replay()
    torch.cuda.synchronize()
    assert [r["step"] for r in tel.flush()] == [3, 4, 5]
