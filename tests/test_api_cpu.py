"""The reference's router API surface on the host side: construction checks, the
capacity budget, the telemetry helpers and the names its tests import.  The
expected values are the reference's own test vectors
(moe-engine/tests/test_router.py L:55-95, L:226-241; tests/test_routing_quality.py
L:36-94); nothing here launches a kernel."""

from __future__ import annotations

import math
import warnings

import pytest
import torch

from pkg.distributed.router import MoERouterInterface
from pkg.kernels.moe_router import (
    MoERouter,
    _compute_load_imbalance,
    _compute_router_z_loss,
    _reference_route_fp64,
)


def test_interface_construction_defaults():
    r = MoERouterInterface(hidden_dim=128, num_experts=16, top_k=4)
    assert (r.hidden_dim, r.num_experts, r.top_k, r.capacity_factor) == (128, 16, 4, 1.25)
    assert MoERouterInterface(hidden_dim=64, num_experts=4, top_k=4).top_k == 4  # dense routing is valid


def test_interface_top_k_above_experts_raises():
    with pytest.raises(ValueError, match="top_k.*must be.*num_experts"):
        MoERouterInterface(hidden_dim=64, num_experts=4, top_k=5)


def test_interface_capacity_factor_warning():
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        MoERouterInterface(hidden_dim=64, num_experts=4, top_k=2, capacity_factor=0.9)
    assert len(w) == 1 and "silently drop tokens" in str(w[0].message).lower()
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        MoERouterInterface(hidden_dim=64, num_experts=4, top_k=2, capacity_factor=1.0)
    assert len(w) == 0


def test_interface_repr():
    s = repr(MoERouterInterface(hidden_dim=256, num_experts=32, top_k=2, capacity_factor=1.5))
    assert "256" in s and "32" in s and "1.5" in s


@pytest.mark.parametrize(
    "N,E,K,cf,expected",
    [(64, 8, 2, 1.25, 20), (32, 8, 2, 1.25, 10), (100, 10, 2, 1.0, 20), (100, 10, 2, 1.25, 25), (100, 7, 2, 1.0, 29)],
)
def test_interface_capacity_budget_table(N, E, K, cf, expected):
    r = MoERouterInterface(hidden_dim=16, num_experts=E, top_k=K, capacity_factor=cf)
    assert r.capacity_budget(N) == expected


def test_router_module_validates_top_k():
    with pytest.raises(ValueError):
        MoERouter(hidden_dim=16, num_experts=4, top_k=5)
    with pytest.raises(ValueError):
        MoERouter(hidden_dim=16, num_experts=4, top_k=0)
    r = MoERouter(hidden_dim=16, num_experts=4, top_k=2)
    assert tuple(r.gate_w.shape) == (16, 4) and r.last_profile is None


@pytest.mark.parametrize("cnt,expected", [([10, 10, 10, 10], 1.0), ([100, 0, 0, 0], 4.0), ([30, 10, 20, 40], 1.6)])
def test_load_imbalance_golden(cnt, expected):
    assert abs(_compute_load_imbalance(torch.tensor(cnt, dtype=torch.long)) - expected) < 1e-6


def test_load_imbalance_zero_counts():
    assert _compute_load_imbalance(torch.zeros(8, dtype=torch.long)) == 1.0


def test_z_loss_zero_logits_is_log_e_squared():
    assert abs(_compute_router_z_loss(torch.zeros(32, 16)) - math.log(16) ** 2) < 1e-4


def test_z_loss_nonnegative_and_grows_with_scale():
    g = torch.Generator().manual_seed(1)
    small = torch.randn(64, 16, generator=g) * 0.01
    large = torch.randn(64, 16, generator=g) * 10.0
    assert _compute_router_z_loss(small) >= 0.0
    assert _compute_router_z_loss(large) > _compute_router_z_loss(small)


def test_reference_fp64_helper_is_importable_but_not_shipped():
    with pytest.raises(NotImplementedError):
        _reference_route_fp64(torch.zeros(4, 8), torch.zeros(8, 4), 2)
