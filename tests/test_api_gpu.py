"""The reference's router API on the GPU: the invariants and contracts its own
tests check (moe-engine/tests/test_kernels.py L:117-153, tests/test_router.py
L:98-318, tests/test_routing_quality.py L:99-131), run through the drop-in
modules (pkg.kernels.moe_router, pkg.distributed.router) on the HIP kernels."""

from __future__ import annotations

import pytest
import torch

from gpu_util import dev, say

from pkg.distributed.router import MoERouterInterface, RouterStats
from pkg.kernels.moe_router import MoERouter, MoERouterFunction, RouterProfile, moe_topk_route

pytestmark = pytest.mark.gpu


def _tokens(N, H, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(N, H, generator=g).to(dtype).to(dev())


@pytest.mark.parametrize("B,S,H,E,K", [(2, 32, 64, 8, 2), (3, 16, 64, 32, 4), (4, 512, 4096, 8, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_token_conservation(B, S, H, E, K, dtype):
    say(f"[api conservation] {B}x{S} H={H} E={E} K={K} {dtype}")
    N = B * S
    torch.manual_seed(1)
    router = MoERouter(hidden_dim=H, num_experts=E, top_k=K, dtype=dtype).to(dev())
    idx, w, cnt = router(_tokens(N, H, seed=B + S, dtype=dtype))
    assert idx.shape == (N, K) and idx.dtype == torch.int64
    assert w.shape == (N, K) and w.dtype == dtype
    assert cnt.shape == (E,)
    assert int(cnt.sum()) == N * K
    assert bool(((idx >= 0) & (idx < E)).all())
    assert not bool(torch.isnan(w).any())
    if K > 1:
        s, _ = torch.sort(idx, dim=-1)
        assert bool((s[:, 1:] > s[:, :-1]).all()), "a token got the same expert twice"
    assert torch.equal(cnt.cpu(), torch.bincount(idx.reshape(-1).cpu(), minlength=E))


def test_combine_weights_sum_to_one():
    torch.manual_seed(2)
    router = MoERouter(hidden_dim=32, num_experts=16, top_k=2).to(dev())
    _, w, _ = router(_tokens(64, 32, seed=2))
    assert torch.allclose(w.sum(-1), torch.ones(64, device=dev()), atol=1e-5)


def test_router_profile_fields_and_consistency():
    H, E, K, N = 64, 16, 2, 96
    torch.manual_seed(3)
    router = MoERouter(hidden_dim=H, num_experts=E, top_k=K).to(dev())
    assert router.last_profile is None
    router(_tokens(N, H, seed=3))
    p = router.last_profile
    assert isinstance(p, RouterProfile)
    assert p.sram_bytes_per_block > 0
    assert isinstance(p.used_triton, bool) and p.used_triton
    assert p.kernel_ms >= 0.0 and p.achieved_bandwidth_gbps >= 0.0
    assert abs(p.tokens_per_expert_mean - N * K / E) < 1e-4
    assert p.tokens_per_expert_std >= 0.0
    assert p.expert_load_imbalance >= 1.0
    assert p.router_z_loss >= 0.0
    assert router._last_logits is not None and tuple(router._last_logits.shape) == (N, E)


def test_profile_reports_the_streaming_kernels_lds():
    """The C2 shape runs the LDS-ring streaming forward: its workgroup holds four 40 KB slots."""
    router = MoERouter(hidden_dim=4096, num_experts=8, top_k=2, dtype=torch.bfloat16).to(dev())
    router(_tokens(16384, 4096, seed=4, dtype=torch.bfloat16))
    assert router.last_profile.sram_bytes_per_block >= 4 * 40 * 1024


def test_function_report_and_five_gradients():
    N, H, E, K = 40, 64, 8, 2
    x = _tokens(N, H, seed=5).requires_grad_(True)
    gw = (torch.randn(H, E, generator=torch.Generator().manual_seed(6)) * 0.1).to(dev()).requires_grad_(True)
    report = {}
    idx, w = MoERouterFunction.apply(x, gw, K, False, report)
    assert set(report) >= {"used_triton", "kernel_ms", "sram_bytes", "achieved_bw"}
    assert report["used_triton"] is True and report["sram_bytes"] > 0
    # autograd checks that backward returns one gradient per forward input (tokens, gate_w, k,
    # force_reference, report): a wrong count raises here
    (w * torch.randn_like(w)).sum().backward()
    assert x.grad is not None and gw.grad is not None
    assert torch.isfinite(x.grad).all() and torch.isfinite(gw.grad).all()


def test_profile_times_the_router_kernels():
    """kernel_ms comes from timing events around the router's launches and achieved_bandwidth_gbps is the
    forward's byte count over that time (the reference's L:313-343, L:371-379), with and without the
    forward's own synchronisation (sync_profile=False resolves the profile when it is read)."""
    from pkg.kernels.moe_router import router_fwd_bytes

    N, H, E, K = 4096, 1024, 16, 2
    x = _tokens(N, H, seed=9, dtype=torch.bfloat16)
    for sync in (True, False):
        say(f"[profile timing] sync_profile={sync}")
        router = MoERouter(hidden_dim=H, num_experts=E, top_k=K, dtype=torch.bfloat16, sync_profile=sync).to(dev())
        router(x)
        _, w, _ = router(x)
        p = router.last_profile
        assert 0.0 < p.kernel_ms < 1000.0
        nbytes = router_fwd_bytes(x, router.gate_w, K, w.dtype)
        assert abs(p.achieved_bandwidth_gbps - nbytes / (p.kernel_ms * 1e-3) / 1e9) <= 1e-6 * p.achieved_bandwidth_gbps
        assert router.last_profile is p  # resolved once
    report = {}
    gw = router.gate_w.detach()
    MoERouterFunction.apply(x, gw, K, False, report)
    assert report["kernel_ms"] > 0.0
    assert abs(report["achieved_bw"] - router_fwd_bytes(x, gw, K, x.dtype) / (report["kernel_ms"] * 1e-3) / 1e9) \
        <= 1e-6 * report["achieved_bw"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["fused", "per_expert"])
def test_layer_times_the_expert_compute(dtype):
    """last_expert_compute_ms: device events around the expert FFN compute (moe_layer.py L:326-337 times the
    same span): positive, below the whole forward's time, and resolved once."""
    from pkg.distributed.parallel_mesh import DistributedMoELayer, build_topology

    say(f"[expert timing] {dtype}")
    layer = DistributedMoELayer(256, 512, 8, 2, build_topology(), dtype=dtype).to(dev())
    x = _tokens(1024, 256, seed=11, dtype=dtype)
    layer(x)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    layer(x)
    b.record()
    ms = layer.last_expert_compute_ms
    torch.cuda.synchronize()
    assert 0.0 < ms <= a.elapsed_time(b) * 1.01 + 1e-3
    assert layer.last_expert_compute_ms == ms
    layer.last_expert_compute_ms = 0.0
    assert layer.last_expert_compute_ms == 0.0


def test_force_reference_is_not_shipped():
    x = _tokens(8, 16, seed=7)
    gw = torch.zeros(16, 4, device=dev())
    with pytest.raises(NotImplementedError):
        MoERouterFunction.apply(x, gw, 2, True)


def test_moe_topk_route_ranks():
    H, E, K = 32, 8, 2
    gw = (torch.randn(H, E, generator=torch.Generator().manual_seed(8)) * 0.1).to(dev())
    x3 = _tokens(2 * 5, H, seed=8).reshape(2, 5, H)
    idx, w = moe_topk_route(x3, gw, K)
    assert idx.shape == (10, K) and w.shape == (10, K)
    idx2, w2 = moe_topk_route(x3.reshape(10, H), gw, K)
    assert torch.equal(idx, idx2) and torch.equal(w, w2)
    with pytest.raises(ValueError):
        moe_topk_route(x3.reshape(-1), gw, K)


@pytest.mark.parametrize("N,H,E,K", [(1, 8, 2, 1), (16, 64, 8, 2), (128, 256, 32, 4)])
def test_interface_output_shapes(N, H, E, K):
    r = MoERouterInterface(hidden_dim=H, num_experts=E, top_k=K).to(dev())
    stats = r(_tokens(N, H, seed=N + E))
    assert isinstance(stats, RouterStats)
    assert stats.expert_indices.shape == (N, K)
    assert stats.combine_weights.shape == (N, K) and stats.combine_weights.is_floating_point()
    assert stats.dispatch_counts.shape == (E,) and stats.dispatch_counts.dtype == torch.int64


def test_interface_invariants_and_fields():
    N, H, E, K = 32, 64, 8, 2
    r = MoERouterInterface(hidden_dim=H, num_experts=E, top_k=K).to(dev())
    stats = r(_tokens(N, H, seed=9))
    assert int(stats.dispatch_counts.sum()) == N * K
    assert torch.allclose(stats.combine_weights.sum(-1), torch.ones(N, device=dev()), atol=1e-4)
    assert bool(((stats.expert_indices >= 0) & (stats.expert_indices < E)).all())
    assert stats.load_imbalance >= 1.0
    assert abs(stats.tokens_per_expert_mean - N * K / E) < 1e-4
    assert stats.tokens_per_expert_std >= 0.0
    assert stats.router_z_loss >= 0.0
    assert isinstance(stats.used_triton, bool) and stats.kernel_ms >= 0.0
    for f in ("expert_indices", "combine_weights", "dispatch_counts", "load_imbalance", "router_z_loss",
              "used_triton", "kernel_ms", "tokens_per_expert_mean", "tokens_per_expert_std"):
        assert hasattr(stats, f)


def test_interface_input_checks():
    r = MoERouterInterface(hidden_dim=64, num_experts=8, top_k=2).to(dev())
    with pytest.raises(ValueError, match="2D input"):
        r(_tokens(8, 64, seed=10).reshape(2, 4, 64))
    with pytest.raises(ValueError, match="hidden dim"):
        r(_tokens(8, 32, seed=10))


def test_interface_gradients_flow_over_repeated_steps():
    H = 64
    r = MoERouterInterface(hidden_dim=H, num_experts=8, top_k=2).to(dev())
    for step in range(3):
        x = _tokens(16, H, seed=20 + step).requires_grad_(True)
        stats = r(x)
        stats.combine_weights.sum().backward()
        gate = r._kernel_router.gate_w
        assert x.grad is not None and torch.isfinite(x.grad).all()
        assert gate.grad is not None and torch.isfinite(gate.grad).all()
        r.zero_grad()
