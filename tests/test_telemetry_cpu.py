"""Host side of the device routing telemetry: record decoding and the C entry point's argument checks
(no kernel launch here)."""

from __future__ import annotations

import pytest
import torch

from moe_mi355 import _lib
from moe_mi355.telemetry import FIELDS, records_from_rows

pytestmark = pytest.mark.cpu


def test_record_layout_matches_the_library():
    assert _lib.load().moe_telemetry_fields() == 16
    assert len(FIELDS) == 12


def test_records_from_rows_decodes_counts_as_ints():
    row = torch.zeros(2, 16)
    row[0, :12] = torch.tensor([0, 1.5, 2.25, 4.0, 1.0, 2, 6, 0.8, 0.125, 1.01, 0, 32])
    row.view(torch.int32)[0, 0] = 3  # the step is stored as int32 bits
    row.view(torch.int32)[1, 0] = 4
    recs = records_from_rows(row)
    assert recs[0]["step"] == 3 and isinstance(recs[0]["step"], int)
    assert recs[0]["expert_load_imbalance"] == 1.5 and recs[0]["router_z_loss"] == 2.25
    assert recs[0]["dead_expert_count"] == 2 and recs[0]["active_experts"] == 6
    assert recs[0]["routing_efficiency"] == pytest.approx(0.8) and recs[0]["dropped_token_fraction"] == 0.125
    assert recs[0]["dispatched_slots"] == 32 and recs[1]["step"] == 4
    # the reference's StepRecord.routing keys (train.py L:382-392) are all present
    for k in ("expert_load_imbalance", "router_z_loss", "dead_expert_count", "routing_efficiency", "active_experts",
              "dropped_token_fraction"):
        assert k in recs[0]


def test_record_rejects_bad_arguments_without_gpu():
    lib = _lib.load()
    assert lib.moe_telemetry_record(None, 0, 16, 2, 1.0, None, 0, None, 4, None) == -1
    assert "bad arguments" in _lib.last_error()
    assert lib.moe_telemetry_record(None, 8, 16, 2, 1.0, None, 0, None, 0, None) == -1
    assert "bad arguments" in _lib.last_error()
    assert lib.moe_telemetry_record(None, 8, 16, 2, 1.0, None, 0, None, 4, None) == -1
    assert "null" in _lib.last_error()
