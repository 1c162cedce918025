"""Integer (numpy) CPU restatement of the dispatch planner -- TEST INFRASTRUCTURE ONLY.

Reference: ``moe-engine/pkg/distributed/moe_layer.py``.

Pinning (checked in ``tests/test_oracle_plan.py``):

* ``cumcount``   -- the reference's golden vectors
  (``tests/test_capacity_dropping.py`` L:42-107) and an O(n^2) brute-force
  count on random small inputs.
* ``drop_mask``  -- golden vectors (``tests/test_capacity_dropping.py``
  L:116-152) incl. per-column independence and capacity 0, plus brute force.
* ``plan_reference`` -- brute-force restatement of the reference layer's
  index arithmetic on small inputs (stable sort of column 0, K-fold repeat,
  E equal chunks, zeroed remainder rows).
* ``plan_routed``    -- brute-force per-expert slot lists.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np

LAYOUT_REFERENCE = 0
LAYOUT_ROUTED = 1


def cumcount(groups) -> np.ndarray:
    """0-based rank of each element among earlier elements of its group.

    Same result as ``_cumcount`` (moe_layer.py L:64-115).  Computed here with a
    stable argsort and the first-occurrence index of each group in sorted
    order (``searchsorted``) instead of the reference's cummax trick.
    """
    g = np.asarray(groups, dtype=np.int64).reshape(-1)
    n = g.shape[0]
    if n == 0:
        return np.zeros(0, dtype=np.int64)
    order = np.argsort(g, kind="stable")
    sg = g[order]
    first = np.searchsorted(sg, sg, side="left")
    out = np.empty(n, dtype=np.int64)
    out[order] = np.arange(n, dtype=np.int64) - first
    return out


def drop_mask(idx, capacity: int) -> np.ndarray:
    """Per-top-k-column capacity drop (moe_layer.py L:118-155).

    drop[t, k] = cumcount(idx[:, k])[t] >= capacity, each column on its own
    queue (so the budget is per column, not per expert total).
    """
    a = np.asarray(idx, dtype=np.int64)
    N, K = a.shape
    out = np.zeros((N, K), dtype=bool)
    for k in range(K):
        out[:, k] = cumcount(a[:, k]) >= capacity
    return out


def plan_reference(idx, num_experts: int) -> Dict[str, np.ndarray]:
    """Positional ("reference") layout of ``DistributedMoELayer.forward`` at ep=1.

    moe_layer.py L:317-337 and L:348-353:
      sort_order = stable argsort of idx[:, 0]            (L:318)
      permuted row r holds token sort_order[r // K]        (L:319 repeat_interleave)
      chunk = max(1, R // E); expert i owns rows [i*chunk, min((i+1)*chunk, R))
      rows >= E*chunk are never computed (stay zero)       (L:328-336)
      combine: out[sort_order[j]] += w[sort_order[j], k] * Y[j*K + k]  (L:349-353)

    Returns ``row_slot`` (slot t*K+k held by each row), ``slot_row`` (inverse),
    ``offsets`` ([E+1] row offsets; rows past offsets[E] are uncomputed) and
    ``sort_order``.
    """
    a = np.asarray(idx, dtype=np.int64)
    N, K = a.shape
    R = N * K
    sort_order = np.argsort(a[:, 0], kind="stable") if N else np.zeros(0, dtype=np.int64)
    r = np.arange(R, dtype=np.int64)
    row_slot = sort_order[r // K] * K + (r % K) if R else np.zeros(0, dtype=np.int64)
    slot_row = np.empty(R, dtype=np.int64)
    slot_row[row_slot] = r
    chunk = max(1, R // max(num_experts, 1))
    offsets = np.minimum(np.arange(num_experts + 1, dtype=np.int64) * chunk, R)
    return {
        "row_slot": row_slot,
        "slot_row": slot_row,
        "offsets": offsets,
        "sort_order": sort_order,
        "n_rows": np.int64(R),
    }


def plan_routed(idx, num_experts: int, drop: Optional[np.ndarray] = None) -> Dict[str, np.ndarray]:
    """Routed layout: slot (t, k) goes to expert idx[t, k]; dropped slots get no row.

    Rows are grouped by expert; within an expert, slots keep flattened
    (t*K + k) order.  ``slot_row`` is -1 for dropped slots.
    """
    a = np.asarray(idx, dtype=np.int64)
    N, K = a.shape
    flat = a.reshape(-1)
    keep = np.ones(N * K, dtype=bool) if drop is None else ~np.asarray(drop, dtype=bool).reshape(-1)
    kept_slots = np.nonzero(keep)[0]
    order = np.argsort(flat[kept_slots], kind="stable")
    row_slot = kept_slots[order]
    counts = np.bincount(flat[kept_slots], minlength=num_experts)
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    slot_row = np.full(N * K, -1, dtype=np.int64)
    slot_row[row_slot] = np.arange(row_slot.shape[0], dtype=np.int64)
    return {
        "row_slot": row_slot,
        "slot_row": slot_row,
        "offsets": offsets,
        "n_rows": np.int64(row_slot.shape[0]),
    }


def row_expert(offsets: np.ndarray, n_rows_alloc: int) -> np.ndarray:
    """Expert owning each row (-1 for rows outside every segment)."""
    out = np.full(n_rows_alloc, -1, dtype=np.int64)
    for e in range(offsets.shape[0] - 1):
        out[offsets[e] : offsets[e + 1]] = e
    return out
