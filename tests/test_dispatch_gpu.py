"""Planner / permute / combine kernels against the integer numpy oracle
(bit-exact) and float64 sums (within the dtype tolerance)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, assert_rel, dev, say
from oracle import plan as OP

from moe_mi355 import configs, ops

pytestmark = pytest.mark.gpu


def _idx(N, K, E, seed, skew=0.0):
    """Random top-k index sets (distinct experts per token), optionally skewed."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(N, E, generator=g)
    if skew:
        logits = logits + skew * torch.linspace(3, 0, E)
    return torch.topk(logits, K, dim=-1).indices


CASES = [
    # N, K, E, capacity_factor (None = no dropping), skew
    (1000, 2, 8, None, 0.0),
    (1000, 2, 8, 1.0, 2.0),
    (4097, 6, 64, 1.25, 0.0),
    (513, 8, 128, 1.0, 3.0),
    (37, 3, 4, 0.5, 0.0),
    (16, 1, 1, None, 0.0),
    (8, 8, 8, 1.0, 0.0),
    (65536, 6, 64, 1.25, 0.0),  # C3 shape
    (2048, 8, 64, 1.0, 1.0),  # 16384 slots: the largest single-block plan
    (16385, 1, 4, 1.0, 0.0),  # one slot more: the multi-block planner
    (16384, 1, 1024, None, 0.0),  # single block, 1024 keys
    (1500, 8, 1024, 1.0, 2.0),  # 8192 capacity keys: too many for one block's waves at 12000 slots
    (3000, 8, 1024, 1.25, 0.0),  # the same keys over several blocks
    # no capacity, E <= 16: one block per key
    (8192, 2, 8, None, 0.0),  # C4 shape
    (5000, 3, 16, None, 2.0),
    (16384, 1, 16, None, 1.0),  # the largest per-key plan
    (7, 2, 2, None, 0.0),
    (16385, 1, 8, None, 0.0),  # one slot more: the multi-block planner without drops
    # capacity drops + routed layout beyond one block: count / scan2 / rank2
    (70000, 8, 64, 0.5, 1.0),  # 274 planner blocks: scan2 carries its bases across block chunks of 256
    (9000, 12, 32, 1.0, 2.0),  # K > 8: scan2 loads the keys of an expert in two rounds
    (20000, 1, 128, 0.5, 3.0),  # K = 1, heavy drops, a ragged last block
    (33000, 8, 128, 1.0, 3.0),  # C5-like keys (K*E = 1024), skewed
    (5000, 8, 256, 1.0, 2.0),  # K*E = 2048: the capacity grouping on 8 waves, the routed one on 16
]


def _cap(N, K, E, cf):
    return -1 if cf is None else math.ceil(cf * N * K / E)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"N{c[0]}-K{c[1]}-E{c[2]}-cf{c[3]}")
@pytest.mark.parametrize("layout", [ops.LAYOUT_REFERENCE, ops.LAYOUT_ROUTED], ids=["ref", "routed"])
def test_plan_matches_oracle(case, layout):
    N, K, E, cf, skew = case
    say(f"[plan] {case} layout={layout}")
    idx = _idx(N, K, E, seed=N + K + E, skew=skew)
    cap = _cap(N, K, E, cf)
    p = ops.plan(idx.to(dev()), E, capacity=cap, layout=layout)
    torch.cuda.synchronize()
    a = idx.numpy()
    drop = np.zeros((N, K), dtype=bool)
    if cap >= 0:
        drop = OP.drop_mask(a, cap)
        assert np.array_equal(p.drop.cpu().numpy(), drop)
        assert int(p.ndrop.item()) == int(drop.sum())
    ref = OP.plan_reference(a, E) if layout == ops.LAYOUT_REFERENCE else OP.plan_routed(a, E, drop)
    kept = int(ref["n_rows"])
    assert np.array_equal(p.offsets.cpu().numpy().astype(np.int64), ref["offsets"])
    assert np.array_equal(p.row_slot.cpu().numpy()[:kept].astype(np.int64), ref["row_slot"][:kept])
    assert np.array_equal(p.slot_row.cpu().numpy().astype(np.int64), ref["slot_row"])
    if layout == ops.LAYOUT_ROUTED:
        assert (p.row_slot.cpu().numpy()[kept:] == -1).all()


def test_cumcount_and_drop_mask_golden_vectors():
    # tests/test_capacity_dropping.py L:42-152 of the reference
    from pkg.distributed.moe_layer import _cumcount, compute_capacity_drop_mask

    d = dev()
    for g, want in [([2, 0, 2, 1, 0, 2], [0, 0, 1, 0, 1, 2]), ([5, 5, 5, 5], [0, 1, 2, 3]),
                    ([3, 1, 3, 1, 3, 0], [0, 0, 1, 1, 2, 0]), ([7], [0])]:
        assert _cumcount(torch.tensor(g, device=d)).cpu().tolist() == want
    assert _cumcount(torch.tensor([], dtype=torch.long, device=d)).numel() == 0
    m = compute_capacity_drop_mask(torch.tensor([[0], [0], [0], [1], [1]], device=d), 2, 2)
    assert m.cpu().tolist() == [[False], [False], [True], [False], [False]]
    m = compute_capacity_drop_mask(torch.tensor([[0, 1], [0, 1]], device=d), 2, 1)
    assert m.cpu().tolist() == [[False, False], [True, True]]
    assert compute_capacity_drop_mask(torch.tensor([[0], [1], [0], [1]], device=d), 2, 0).all()


WIDE_IDS = [
    ("span_1e6", 200000, lambda g, n: torch.randint(0, 1_000_001, (n,), generator=g)),
    ("few_ids_wide_span", 50000, lambda g, n: torch.tensor([-7, 10**6, 3, 2**40])[torch.randint(0, 4, (n,), generator=g)]),
    ("negative", 30000, lambda g, n: torch.randint(-(2**50), 2**50, (n,), generator=g)),
    ("all_distinct", 4097, lambda g, n: torch.randperm(n, generator=g) * 1000 - 5),
    ("one_element", 1, lambda g, n: torch.tensor([123456789])),
]


@pytest.mark.parametrize("case", WIDE_IDS, ids=lambda c: c[0])
def test_cumcount_any_integer_ids(case):
    """_cumcount on id ranges wider than the planner's keys (moe_cumcount: stable radix sort + ranks) against
    the integer oracle (oracle/plan.py cumcount), bit-exact; and the per-column drop mask on such ids."""
    from pkg.distributed.moe_layer import _cumcount, compute_capacity_drop_mask

    name, n, make = case
    say(f"[cumcount wide ids] {name} n={n}")
    g = torch.Generator().manual_seed(n)
    ids = make(g, n).long()
    got = _cumcount(ids.to(dev())).cpu().numpy()
    assert np.array_equal(got, OP.cumcount(ids.numpy()))
    if n >= 2:
        cols = torch.stack([ids, ids.flip(0)], dim=1)
        cap = max(1, int(np.bincount(OP.cumcount(ids.numpy())).size // 2))
        m = compute_capacity_drop_mask(cols.to(dev()), 8, cap).cpu().numpy()
        assert np.array_equal(m, OP.drop_mask(cols.numpy(), cap))


def _rows_and_y(N, K, E, H, dt, seed, cap, layout):
    idx = _idx(N, K, E, seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(N, H, generator=g).to(dt)
    w = torch.rand(N, K, generator=g).to(dt)
    d = dev()
    p = ops.plan(idx.to(d), E, capacity=cap, layout=layout)
    return idx, x, w, p


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("layout", [ops.LAYOUT_REFERENCE, ops.LAYOUT_ROUTED], ids=["ref", "routed"])
def test_permute_combine_and_backward(dt, layout):
    N, K, E, H = 777, 3, 10, 264
    say(f"[permute/combine] dt={dt} layout={layout}")
    cap = _cap(N, K, E, 0.9)
    idx, x, w, p = _rows_and_y(N, K, E, H, dt, 3, cap, layout)
    d = dev()
    xd, wd = x.to(d), w.to(d)
    xp = ops.permute(xd, p)
    torch.cuda.synchronize()
    offs = p.offsets.cpu().tolist()
    live = offs[E]
    rs = p.row_slot.cpu().long()
    sr = p.slot_row.cpu().long()
    drop = p.drop.cpu() if p.drop is not None else torch.zeros(N, K, dtype=torch.bool)
    # permute: bit-exact row copies
    assert torch.equal(xp[:live].cpu(), x[rs[:live] // K])
    # combine with y = a per-row transform of xp (scaled), float64 reference
    y = (xp.float() * 0.5 + 0.25).to(dt)
    y[live:] = float("nan")  # rows that are never computed must not be read
    out = ops.combine(y, wd, p)
    torch.cuda.synchronize()
    y64 = y.cpu().double()
    ref = torch.zeros(N, H, dtype=torch.float64)
    for t in range(N):
        for k in range(K):
            r = int(sr[t * K + k])
            if 0 <= r < live and not drop[t, k]:
                ref[t] += float(w[t, k]) * y64[r]
    assert_rel(out, ref, TOL[dt], "combine")
    # combine backward
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(N, H, generator=g).to(dt)
    dy, dw = ops.combine_backward(dout.to(d), y, wd, p)
    torch.cuda.synchronize()
    dref = torch.zeros(live, H, dtype=torch.float64)
    dwref = torch.zeros(N, K, dtype=torch.float64)
    d64 = dout.double()
    for t in range(N):
        for k in range(K):
            r = int(sr[t * K + k])
            if 0 <= r < live:
                wk = 0.0 if drop[t, k] else float(w[t, k])
                dref[r] = wk * d64[t]
                dwref[t, k] = 0.0 if drop[t, k] else float((d64[t] * y64[r]).sum())
    assert_rel(dy[:live], dref, TOL[dt], "combine dy")
    assert_rel(dw.float(), dwref, TOL[dt], "combine dw")
    # permute backward (gather-sum) with an addend
    dxp = torch.randn(N * K, H, generator=g).to(dt)
    add = torch.randn(N, H, generator=g).to(dt)
    dx = ops.unpermute_sum(dxp.to(d), p, addend=add.to(d))
    torch.cuda.synchronize()
    dxref = add.double().clone()
    for t in range(N):
        for k in range(K):
            r = int(sr[t * K + k])
            if 0 <= r < live:
                dxref[t] += dxp[r].double()
    assert_rel(dx, dxref, TOL[dt], "unpermute_sum")


def test_dispatch_c3_full_size_roundtrip():
    """C3 (T=65536, d=2048, E=64, K=6, cf=1.25 with drops): permute then an
    identity combine with unit weights reproduces K' * x for each token, where
    K' counts its kept slots -- a size-independent property of the gather."""
    cfg = configs.C3
    say("[dispatch C3 full]")
    d = dev()
    inp = configs.router_inputs(cfg)
    x = inp["x"].to(d)
    from moe_mi355.router import RouterCore

    idx, w, *_ = RouterCore.apply(x, inp["gate_w"].to(d), cfg.K, 0.0, 0.0, None)
    cap = configs.capacity(cfg)
    for layout in (ops.LAYOUT_REFERENCE, ops.LAYOUT_ROUTED):
        p = ops.plan(idx, cfg.E, capacity=cap, layout=layout)
        xp = ops.permute(x, p)
        ones = torch.ones(cfg.T, cfg.K, dtype=torch.float32, device=d)
        out = ops.combine(xp, ones, p)
        kept = (~p.drop).sum(1, keepdim=True).float()
        if layout == ops.LAYOUT_REFERENCE:
            # positional layout: row r carries token row_slot[r] // K; every row < offsets[E] is live
            rs = p.row_slot.long()
            live = int(p.offsets[-1].item())
            assert torch.equal(xp[:live], x[rs[:live] // cfg.K])
        else:
            torch.testing.assert_close(out.float(), (x.float() * kept).to(torch.bfloat16).float(), rtol=2e-2, atol=0)
        a = idx.cpu().numpy()
        assert np.array_equal(p.drop.cpu().numpy(), OP.drop_mask(a, cap))


def test_plan_deterministic():
    d = dev()
    idx = _idx(20000, 4, 32, 5).to(d)
    a = ops.plan(idx, 32, capacity=2000, layout=ops.LAYOUT_ROUTED)
    b = ops.plan(idx, 32, capacity=2000, layout=ops.LAYOUT_ROUTED)
    for u, v in ((a.row_slot, b.row_slot), (a.slot_row, b.slot_row), (a.offsets, b.offsets), (a.drop, b.drop)):
        assert torch.equal(u, v)
