"""The bench-only MFMA ceiling probe: a memory-free MFMA loop on every CU returns a dense rate below the
published peak and a shader clock within the part's range."""

from __future__ import annotations

import pytest

from gpu_util import say

from moe_mi355 import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("random", [False, True], ids=["const", "random"])
@pytest.mark.parametrize("fp8,peak", [(False, 2500.0), (True, 5000.0)])
def test_mfma_ceiling(fp8, peak, random):
    say(f"[prof] mfma ceiling fp8={fp8} random={random}")
    tf, mhz = _lib.prof_mfma_ceiling(20000, fp8=fp8, random=random)
    assert 0.2 * peak < tf < 1.02 * peak, tf
    assert 500.0 < mhz < 2600.0, mhz


def test_mfma_ceiling_rejects_bad_iters():
    with pytest.raises(ValueError):
        _lib.prof_mfma_ceiling(0)
    with pytest.raises(ValueError):
        _lib.check(_lib.load().moe_prof_mfma_ceiling(100, 4, None, None), "moe_prof_mfma_ceiling")
