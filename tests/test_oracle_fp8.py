"""The fp8 oracle (oracle/fp8.py) against closed forms, known e4m3 encodings and brute-force loops (the
reference has no fp8 path, so nothing of the reference's pins it)."""

from __future__ import annotations

import pytest
import torch

from oracle import fp8 as O8

pytestmark = pytest.mark.cpu


def test_known_encodings():
    q, s = O8.quant_rows(torch.tensor([[1.0, 448.0, -448.0, 0.0]]))
    assert s.item() == 1.0
    assert q[0].tolist() == [0x38, 0x7E, 0xFE, 0x00]


def test_absmax_maps_to_448_and_zero_rows():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 96, generator=g) * torch.logspace(-3, 3, 64).unsqueeze(1)
    x[5] = 0.0
    q, s = O8.quant_rows(x)
    d = O8.dequant(q, s)
    amax_pos = x.abs().argmax(-1)
    for r in range(64):
        if r == 5:
            assert s[r].item() == 1.0 and int(q[r].sum()) == 0
            continue
        v = q[r, amax_pos[r]].view(torch.float8_e4m3fn).float().item()
        assert abs(v) == 448.0
        assert s[r].item() == pytest.approx(x[r].abs().max().item() / 448.0, rel=1e-7)
    # e4m3: 3 mantissa bits -> relative rounding error <= 2^-4 in the normal range, absolute <= scale * 2^-10
    # below it (subnormal spacing 2^-9)
    bound = torch.maximum(x.double().abs() * 2.0 ** -4, s.double().unsqueeze(1) * 2.0 ** -10)
    assert bool(((d - x.double()).abs() <= bound + 1e-30).all())


def test_multiplier_is_the_correctly_rounded_quotient():
    """x * inv with inv = fl32(448 / absmax) exactly (as the kernel's fp32 division is): re-derive each
    element's e4m3 value from a float64 quotient rounded once to fp32."""
    g = torch.Generator().manual_seed(2)
    # bf16 inputs (8 significant bits) land on e4m3 rounding ties often enough to expose a 1-ulp multiplier
    x = (torch.randn(300, 4096, generator=g) * torch.logspace(-4, 4, 300).unsqueeze(1)).to(torch.bfloat16).float()
    q, _ = O8.quant_rows(x)
    inv = (448.0 / x.double().abs().amax(-1)).float()  # float64 division, rounded once
    want = (x * inv.unsqueeze(1)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(q, want)
    # torch's scalar / tensor (reciprocal times the scalar) differs in the last bit for many rows
    loose = (x * (448.0 / x.abs().amax(-1)).unsqueeze(1)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert not torch.equal(q, loose)


def test_planted_mistake_is_caught():
    """An e4m3 'fnuz'-style maximum of 240 instead of 448 leaves the absmax element at +-240."""
    x = torch.tensor([[3.0, -7.0, 1.0]])
    v = x / (x.abs().amax(-1, keepdim=True) / 240.0)
    assert v.abs().max().item() != 448.0
    q, _ = O8.quant_rows(x)
    assert q[0, 1].item() == 0xFE


def test_swiglu_fwd_fp8_matches_loops():
    g = torch.Generator().manual_seed(1)
    R, H, F, E = 7, 16, 32, 3
    x = torch.randn(R, H, generator=g)
    wg, wu = torch.randn(E, F, H, generator=g) * 0.3, torch.randn(E, F, H, generator=g) * 0.3
    wd = torch.randn(E, H, F, generator=g) * 0.3
    xq, sx = O8.quant_rows(x)
    wq = [O8.quant_rows(w) for w in (wg, wu, wd)]
    offsets = [0, 3, 3, 6]  # expert 1 empty, row 6 past offsets[E]
    hgu, act, y = O8.swiglu_fwd_fp8(xq, sx, [q for q, _ in wq], [s for _, s in wq], offsets)
    yl = O8.swiglu_fwd_fp8_loops(xq, sx, [q for q, _ in wq], [s for _, s in wq], offsets)
    assert torch.allclose(y, yl, rtol=0, atol=0) or (y - yl).abs().max().item() <= 2 ** -8 * yl.abs().max().item()
    assert y[6].abs().max().item() == 0.0 and hgu[6].abs().max().item() == 0.0


def test_tiny_rows_quantize_to_zeros_not_nan():
    """A row whose absmax is below 2^-118 (448 / absmax would overflow fp32 below ~1.3e-36, and 0 * inf is NaN)
    is a zero row: scale 1, bytes +-0.  At 2^-118 itself the row keeps its own scale (448 * 2^118 is finite).
    The rule it replaces -- any nonzero absmax gets its own scale -- turns such a row into NaN bytes."""
    x = torch.zeros(4, 32)
    x[0, :] = 1e-37
    x[0, 3] = 0.0
    x[1, :] = -2e-37
    x[2, 5] = 2.0 ** -118
    x[3, 7] = 2.0 ** -118 * 0.75
    q, s = O8.quant_rows(x)
    assert not bool(torch.isnan(O8.dequant(q, s)).any())
    assert s[0].item() == 1.0 and s[1].item() == 1.0 and s[3].item() == 1.0
    assert set(q[0].tolist()) == {0x00} and set(q[1].tolist()) == {0x80}
    assert s[2].item() == pytest.approx(2.0 ** -118 / 448.0, rel=1e-6) and q[2, 5].item() == 0x7E
    # planted mistake: a scale for every nonzero row
    v = x[0:1]
    inv = torch.full((1,), 448.0) / v.abs().amax(-1)
    assert bool(torch.isinf(inv).all())
    bad = (v * inv.unsqueeze(-1)).to(torch.float8_e4m3fn).float()
    assert bool(torch.isnan(bad).any())


def test_mx_exponent_is_the_smallest_that_fits():
    """mx_exponent(amax) = min{e integer : amax <= 448 * 2^e} by brute force over e, for random magnitudes,
    exact powers of two and the 448 * 2^k boundaries (and just past them)."""
    g = torch.Generator().manual_seed(5)
    a = torch.cat([torch.rand(2000, generator=g) * torch.logspace(-30, 30, 2000),
                   torch.pow(2.0, torch.arange(-40.0, 40.0)),
                   448.0 * torch.pow(2.0, torch.arange(-20.0, 20.0)),
                   torch.nextafter(448.0 * torch.pow(2.0, torch.arange(-20.0, 20.0)), torch.tensor(1e30))])
    e = O8.mx_exponent(a)
    for v, ev in zip(a.double().tolist(), e.tolist()):
        want = next(k for k in range(-127, 128) if v <= 448.0 * 2.0 ** k)
        assert ev == want, (v, ev, want)


def test_quant_mx_closed_forms():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(40, 256, generator=g) * torch.logspace(-6, 6, 40).unsqueeze(1)
    x[3, 32:64] = 0.0            # a zero block
    x[4, :32] = 1.0              # a block of ones: e = -8 (448 * 2^-9 < 1 <= 448 * 2^-8), bytes 2^8 -> 0x78
    x[4, 32:64] = 448.0          # e = 0, bytes 0x7e, scale byte 127
    q, sb = O8.quant_mx(x)
    assert q.shape == x.shape and sb.shape == (40, 8)
    assert int(sb[3, 1]) == 0 and int(q[3, 32:64].sum()) == 0
    assert int(sb[4, 0]) == 127 - 8 and set(q[4, :32].tolist()) == {0x78}
    assert int(sb[4, 1]) == 127 and set(q[4, 32:64].tolist()) == {0x7E}
    d = O8.dequant_mx(q, sb)
    blocks = x.double().reshape(40, 8, 32)
    db = d.reshape(40, 8, 32)
    for r in range(40):
        for b in range(8):
            amax = blocks[r, b].abs().max().item()
            if amax == 0.0:
                continue
            # the scaled block maximum lies in (224, 448]: 448 * 2^e covers it and 448 * 2^(e-1) does not
            scaled = amax * 2.0 ** -(int(sb[r, b]) - 127)
            assert 224.0 < scaled <= 448.0, (r, b, scaled)
            i = int(blocks[r, b].abs().argmax())
            v = abs(float(q[r, 32 * b + i].view(torch.float8_e4m3fn).float()))
            assert 224.0 <= v <= 448.0
    # per element: within the e4m3 rounding bound (relative 2^-4, absolute 2^(e-9) in the subnormal range)
    scale = torch.pow(2.0, sb.double() - 127.0).repeat_interleave(32, dim=1)
    bound = torch.maximum(x.double().abs() * 2.0 ** -4, scale * 2.0 ** -9)
    assert bool(((d - x.double()).abs() <= bound + 1e-300).all())


def test_quant_mx_planted_mistake_is_caught():
    """A plausible off-by-one (e = p - 8 for every block, as a floor(log2) - 8 rule gives) leaves blocks whose
    scaled maximum is <= 224, which the (224, 448] pin rejects; the oracle's exponent passes it."""
    x = torch.randn(8, 64, generator=torch.Generator().manual_seed(7))
    amax = x.reshape(8, 2, 32).abs().amax(-1).double()
    _m, p = torch.frexp(amax)
    wrong = (p - 8).double()
    right = O8.quant_mx(x)[1].double() - 127.0
    ok = lambda e: bool((((amax * torch.pow(2.0, -e)) > 224.0) & ((amax * torch.pow(2.0, -e)) <= 448.0)).all())
    assert ok(right) and not ok(wrong)
