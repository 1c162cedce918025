"""moe_plan_noalloc (the planner with its block tables in the library's fixed device array, for callers that
cannot allocate) against moe_plan with a workspace, through the C ABI: every output bit-exact, on two calls in
a row whose second is smaller (the array keeps the first call's tables), for both layouts with and without
capacity drops; and the size limit rejected on the host."""

from __future__ import annotations

import pytest
import torch

from gpu_util import dev, say

from moe_mi355 import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20  # MOE_PLAN_SCRATCH_BYTES


def _idx(N, K, E, seed):
    g = torch.Generator().manual_seed(seed)
    # skewed choices (distinct per token) so capacity drops happen
    w = torch.rand(N, E, generator=g) * torch.linspace(1.0, 4.0, E)
    return w.topk(K, dim=-1).indices.to(torch.int64).to(dev())


def _outputs(N, K, E):
    d = dev()
    M = max(N * K, 1)
    return {
        "drop": torch.full((N, K), 7, dtype=torch.uint8, device=d),
        "row_slot": torch.full((M,), -9, dtype=torch.int32, device=d),
        "slot_row": torch.full((M,), -9, dtype=torch.int32, device=d),
        "offsets": torch.full((E + 1,), -9, dtype=torch.int32, device=d),
        "ndrop": torch.full((1,), -9, dtype=torch.int32, device=d),
    }


def _call(noalloc, idx, E, capacity, layout):
    lib = _lib.load()
    N, K = idx.shape
    o = _outputs(N, K, E)
    stream = torch.cuda.current_stream().cuda_stream
    args = [idx.data_ptr(), N, K, E, capacity, layout, o["drop"].data_ptr(), o["row_slot"].data_ptr(),
            o["slot_row"].data_ptr(), o["offsets"].data_ptr(), o["ndrop"].data_ptr()]
    if noalloc:
        rc = lib.moe_plan_noalloc(*args, stream)
    else:
        nbytes = lib.moe_plan_workspace(N, K, E)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev())
        rc = lib.moe_plan(*args, ws.data_ptr(), nbytes, stream)
    _lib.check(rc, "moe_plan_noalloc" if noalloc else "moe_plan")
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in o.items()}


@pytest.mark.parametrize("layout,drops", [(0, False), (0, True), (1, False), (1, True)])
def test_noalloc_plan_matches_workspace_plan(layout, drops):
    # the second call is smaller and still a multi-block plan (N*K > 16384 slots) with another key count
    # (K*E = 48 against 256), so it runs the same table-using kernels over the first call's leftover tables
    shapes = [(20000, 4, 64, 11), (12000, 3, 16, 12)]
    for N, K, E, seed in shapes:
        say(f"[noalloc plan] layout={layout} drops={drops} N={N} K={K} E={E}")
        lib = _lib.load()
        assert lib.moe_plan_workspace(N, K, E) <= SCRATCH_BYTES
        idx = _idx(N, K, E, seed)
        cap = (N * K) // (2 * E) if drops else -1
        want = _call(False, idx, E, cap, layout)
        got = _call(True, idx, E, cap, layout)
        keys = ["row_slot", "slot_row", "offsets", "ndrop"] + (["drop"] if drops else [])
        for k in keys:
            assert torch.equal(got[k], want[k]), f"{k} differs (N={N}, K={K}, E={E})"
        if drops:
            assert int(want["ndrop"]) > 0


def test_noalloc_plan_rejects_tables_past_the_array():
    """N*K = 2^23 slots at K*E = 1024 keys need 32 MiB of block tables: rejected on the host (MOE_EINVAL),
    nothing launched, with a message naming the limit."""
    lib = _lib.load()
    N, K, E = 1 << 20, 8, 128
    assert lib.moe_plan_workspace(N, K, E) > SCRATCH_BYTES
    d = dev()
    tiny = torch.zeros(16, dtype=torch.int64, device=d)  # never read: the call is rejected before any launch
    p = tiny.data_ptr()
    rc = lib.moe_plan_noalloc(p, N, K, E, -1, 1, p, p, p, p, p, torch.cuda.current_stream().cuda_stream)
    assert rc == -1
    msg = _lib.last_error()
    assert "scratch" in msg and str(SCRATCH_BYTES) in msg


def test_noalloc_plan_empty_input():
    say("[noalloc plan] empty")
    idx = torch.zeros((0, 2), dtype=torch.int64, device=dev())
    got = _call(True, idx, 8, -1, 1)
    assert got["offsets"].tolist() == [0] * 9 and int(got["ndrop"]) == 0
