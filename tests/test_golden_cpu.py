"""The CPU oracle against the golden fixtures written from the reference itself (tests/golden/*.npz, made by
tests/golden/make_layer_fixtures.py from moe-engine's own DistributedMoELayer and MoERouter).

What the fixtures pin that no closed form does: the reference layer's positional row layout and combine
(moe_layer.py L:317-353, with N*K % E != 0 and capacity drops), its bf16 arithmetic (within the bf16
tolerance), the bias=True router (moe_router.py L:671-687) and torch.topk's order under exact ties.
Tolerances: fp32 1e-5, bf16 2e-2 (max-norm relative)."""

from __future__ import annotations

import glob
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import layer as OL
from oracle import plan as OP
from oracle import router as OR

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"float32": 1e-5, "bfloat16": 2e-2}


def load(name):
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    cfg = json.loads(str(d["config"]))
    return cfg, {k: d[k] for k in d.files if k != "config"}


def names(kind):
    out = []
    for f in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        n = os.path.basename(f)[:-4]
        if load(n)[0]["kind"] == kind:
            out.append(n)
    return out


def t(a, dt="float32"):
    return torch.from_numpy(np.asarray(a)).to(getattr(torch, dt))


def rel(a, b, floor=0.0):
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    den = max(float(b.abs().max()) if b.numel() else 0.0, floor)
    return float((a - b).abs().max()) / den if den else float(a.abs().max())


def test_fixtures_present():
    assert len(names("layer")) >= 7 and len(names("router")) >= 4


def _oracle_layer(cfg, a, idx_override=None):
    dt = cfg["dtype"]
    return OL.layer_fwd_bwd(
        t(a["x"], dt), t(a["gate_w"], dt), t(a["w_gate"], dt), t(a["w_up"], dt), t(a["w_down"], dt), cfg["K"],
        grad_out=t(a["grad_out"], dt), capacity_factor=cfg["capacity_factor"],
        capacity_dropping=cfg["capacity_dropping"], layout=OP.LAYOUT_REFERENCE, idx_override=idx_override,
    )


@pytest.mark.parametrize("name", names("layer"))
def test_oracle_layer_matches_reference(name):
    cfg, a = load(name)
    tol = TOL[cfg["dtype"]]
    ties = cfg["gate"] == "zero"
    ref = _oracle_layer(cfg, a)
    fx = OR.route_fwd(t(a["x"], cfg["dtype"]), t(a["gate_w"], cfg["dtype"]), cfg["K"])
    ok = fx["margin"].numpy() > 1e-6
    if ties:
        # Exact ties: the reference keeps torch.topk's unspecified CPU order, the oracle (and the kernels) the
        # lowest expert index; every weight is 1/K either way.
        assert not ok.any()
        assert not np.array_equal(ref["idx"].numpy(), a["idx"])
    else:
        assert ok.all(), "fixture inputs are chosen away from top-k ties"
        assert np.array_equal(ref["idx"].numpy(), a["idx"])
        assert np.array_equal(ref["cnt"].numpy(), a["cnt"])
    assert rel(ref["w"], np.where(a["drop"], 0.0, a["w"])) <= tol
    assert np.array_equal(ref["drop"], a["drop"])
    assert abs(ref["dropped_fraction"] - float(a["dropped_fraction"])) < 1e-7  # the reference averages in fp32
    # The positional layout ignores which experts a token chose (only the first choice orders the tokens,
    # and under ties every token has the same one), so out, dx and the expert gradients match even at ties.
    assert rel(ref["out"], a["out"]) <= tol
    assert rel(ref["dx"], a["dx"]) <= tol
    for k in ("dw_gate", "dw_up", "dw_down"):
        assert rel(ref[k], a[k]) <= tol, k
    if ties:
        ref = _oracle_layer(cfg, a, idx_override=t(a["idx"]).long())  # the gate gradient depends on the choice
    assert rel(ref["dgate_w"], a["dgate_w"], floor=1e-6) <= tol


def test_fixture_catches_a_misread_combine():
    """A plausible misreading of ``combined_sorted[k::top_k]`` (moe_layer.py L:351) as the k-th block of N rows
    moves rows between tokens; planted in the oracle's plan, the fixture rejects it."""
    cfg, a = load("layer_f32_rem")
    orig = OP.plan_reference

    def misread(idx, num_experts):
        p = orig(idx, num_experts)
        N, K = np.asarray(idx).shape
        r = np.arange(N * K)
        j, k = r % N, r // N  # row r read as (token sort_order[r % N], slot r // N)
        p["row_slot"] = p["sort_order"][j] * K + k
        p["slot_row"] = np.empty(N * K, dtype=np.int64)
        p["slot_row"][p["row_slot"]] = r
        return p

    OP.plan_reference = misread
    try:
        bad = _oracle_layer(cfg, a)
    finally:
        OP.plan_reference = orig
    assert rel(bad["out"], a["out"]) > 1e-2


def test_fixture_catches_a_dropped_remainder():
    """Giving the remainder rows (N*K % E of them) to the last expert instead of leaving them zero
    (moe_layer.py L:328-336) changes the output of the tokens that own them."""
    cfg, a = load("layer_f32_rem")
    assert (cfg["N"] * cfg["K"]) % cfg["E"] != 0
    orig = OP.plan_reference

    def greedy(idx, num_experts):
        p = orig(idx, num_experts)
        p["offsets"] = p["offsets"].copy()
        p["offsets"][-1] = p["n_rows"]
        return p

    OP.plan_reference = greedy
    try:
        bad = _oracle_layer(cfg, a)
    finally:
        OP.plan_reference = orig
    assert rel(bad["out"], a["out"]) > 1e-3


@pytest.mark.parametrize("name", [n for n in names("router") if load(n)[0]["bias"]])
def test_oracle_bias_router_matches_reference(name):
    """bias=True: the reference routes on fp32 logits + bias under no_grad (moe_router.py L:677-687), returns w
    in the token dtype without a gradient, and keeps _last_logits / the z statistic WITHOUT the bias
    (L:727-733)."""
    cfg, a = load(name)
    dt = cfg["dtype"]
    x, gw, b = t(a["x"], dt), t(a["gate_w"], dt), t(a["bias"], dt)
    fx = OR.route_fwd(x, gw, cfg["K"], bias=b)
    ok = fx["margin"].numpy() > 1e-6
    assert ok.all()
    assert np.array_equal(fx["idx"].numpy(), a["idx"])
    assert rel(fx["w"], a["w"]) <= TOL[dt]
    assert not bool(a["w_requires_grad"])
    plain = x.double() @ gw.double()
    assert rel(plain, a["last_logits"]) <= 1e-5
    assert abs(OR.z_stat(plain) - float(a["router_z_loss"])) <= 1e-5 * abs(float(a["router_z_loss"]))
    with_bias = OR.z_stat(plain + b.double())
    assert abs(with_bias - float(a["router_z_loss"])) > 1e-3 * abs(float(a["router_z_loss"]))


def test_oracle_ties_router():
    """All-zero gate: every probability is 1/E.  torch.topk (the reference) returns an implementation-defined
    order; the oracle takes the lowest indices.  The weights (1/K) and the counts' total agree."""
    cfg, a = load("router_ties_f32")
    fx = OR.route_fwd(t(a["x"]), t(a["gate_w"]), cfg["K"])
    assert fx["idx"].tolist() == [list(range(cfg["K"]))] * cfg["N"]
    assert sorted(set(a["idx"].reshape(-1).tolist())) != list(range(cfg["K"]))
    assert rel(fx["w"], a["w"]) <= 1e-7
    assert int(a["cnt"].sum()) == cfg["N"] * cfg["K"]
    assert abs(OR.z_stat(torch.zeros(1, cfg["E"])) - math.log(cfg["E"]) ** 2) < 1e-12
    assert abs(float(a["router_z_loss"]) - math.log(cfg["E"]) ** 2) < 1e-5


def test_oracle_router_profile():
    """The RouterProfile statistics the reference reports (L:594-612, L:736-745) from the oracle's pieces."""
    cfg, a = load("router_profile_f32")
    x, gw = t(a["x"]), t(a["gate_w"])
    full = OR.router_full(x, gw, cfg["K"])
    assert np.array_equal(full["idx"].numpy(), a["idx"])
    cnt = full["cnt"].double()
    assert np.array_equal(full["cnt"].numpy(), a["cnt"])
    assert abs(float(cnt.mean()) - float(a["tokens_per_expert_mean"])) < 1e-6
    assert abs(float(cnt.std()) - float(a["tokens_per_expert_std"])) < 1e-5
    assert abs(OR.load_imbalance(full["cnt"]) - float(a["expert_load_imbalance"])) < 1e-6
    assert abs(float(full["z_stat"]) - float(a["router_z_loss"])) <= 1e-5 * float(a["router_z_loss"])
    assert rel(full["logits"], a["last_logits"]) <= 1e-5
