"""CPU restatement of the fp8 (e4m3) forward of the expert FFN -- TEST INFRASTRUCTURE ONLY.

The reference has no fp8 path (moe-engine's experts run in the model dtype: pkg/distributed/moe_layer.py
L:166-198, L:326-337); the fp8 variant is this build's own, and its contract is stated here:

* ``quant_rows`` -- one fp32 scale per row, ``absmax / 448`` (448 = the largest finite e4m3 value),
  elements ``x * (448 / absmax)`` (fp32; one division per row) rounded to nearest even into OCP e4m3
  (``torch.float8_e4m3fn``).  A row with absmax below 2^-118 (a zero row, or one so small that 448 / absmax
  would overflow fp32 and turn its zeros into NaN) is a zero row: scale 1, elements ``x`` rounded (to +-0).
* ``swiglu_fwd_fp8`` -- the grouped SwiGLU forward on the dequantized operands in float64: per expert segment
  ``hgu = (xq sx) (Wq sw)^T``, ``g`` and ``u`` rounded to bf16, ``act = silu(g) u`` rounded to bf16, ``act``
  quantized per row, ``y = (actq sa) (Wdq sd)^T`` rounded to bf16.

Pinning (``tests/test_oracle_fp8.py``): ``quant_rows`` by closed forms -- a row's absmax element maps to
exactly +-448, a zero row to zeros with scale 1, every element dequantizes within the e4m3 rounding bound, the
byte encoding of known values (1.0 -> 0x38, 448 -> 0x7e, -448 -> 0xfe), the per-row multiplier equal to the
correctly rounded fp32 quotient 448 / absmax (float64 division rounded once) -- and by torch's own float8
conversion (a library routine); ``swiglu_fwd_fp8`` by per-row brute-force loops over the segments on tiny shapes.
"""

from __future__ import annotations

from typing import Sequence, Tuple

import torch

E4M3_MAX = 448.0
QUANT_TINY = 2.0 ** -118  # smallest absmax quantized with its own scale (448 / 2^-118 < FLT_MAX)


def quant_rows(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [..., cols] -> (e4m3 bytes uint8 [..., cols], fp32 scale [...])."""
    v = x.float()
    amax = v.abs().amax(-1)
    pos = amax >= QUANT_TINY
    scale = torch.where(pos, amax / E4M3_MAX, torch.ones_like(amax))
    # a true tensor division (correctly rounded); torch's ``scalar / tensor`` is reciprocal-times-scalar
    inv = torch.where(pos, torch.full_like(amax, E4M3_MAX) / torch.where(pos, amax, torch.ones_like(amax)),
                      torch.ones_like(amax))
    q = (v * inv.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), scale


def dequant(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """e4m3 bytes and row scales -> float64 values."""
    return q.view(torch.float8_e4m3fn).double() * scale.double().unsqueeze(-1)


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).double()


def swiglu_fwd_fp8(xq: torch.Tensor, sx: torch.Tensor, wq: Sequence[torch.Tensor], ws: Sequence[torch.Tensor],
                   offsets: Sequence[int], act_in: torch.Tensor = None):
    """(hgu [R,2F], act [R,F], y [R,H]) float64 values of the bf16 outputs.  Rows past offsets[E] are zero.
    ``act_in`` (optional): quantize this act for the down projection instead of the oracle's own (lets a
    test follow the kernel's act exactly)."""
    wg, wu, wd = wq
    sg, su, sd = ws
    R, H = xq.shape
    E, F, _ = wg.shape
    hgu = torch.zeros(R, 2 * F, dtype=torch.float64)
    act = torch.zeros(R, F, dtype=torch.float64)
    y = torch.zeros(R, H, dtype=torch.float64)
    xd = dequant(xq, sx)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo >= hi:
            continue
        g = _bf16(xd[lo:hi] @ dequant(wg[e], sg[e]).T)
        u = _bf16(xd[lo:hi] @ dequant(wu[e], su[e]).T)
        hgu[lo:hi, :F], hgu[lo:hi, F:] = g, u
        act[lo:hi] = _bf16(torch.nn.functional.silu(g) * u)
    a_src = act if act_in is None else act_in.double()
    aq, sa = quant_rows(a_src.float())
    ad = dequant(aq, sa)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo < hi:
            y[lo:hi] = _bf16(ad[lo:hi] @ dequant(wd[e], sd[e]).T)
    return hgu, act, y


def swiglu_fwd_fp8_loops(xq, sx, wq, ws, offsets):
    """The same forward as explicit per-row, per-output loops (tiny shapes only)."""
    wg, wu, wd = wq
    sg, su, sd = ws
    R, H = xq.shape
    E, F, _ = wg.shape
    xv = xq.view(torch.float8_e4m3fn).double()
    y = torch.zeros(R, H, dtype=torch.float64)
    for e in range(E):
        Wg = wg[e].view(torch.float8_e4m3fn).double()
        Wu = wu[e].view(torch.float8_e4m3fn).double()
        Wd = wd[e].view(torch.float8_e4m3fn).double()
        for r in range(int(offsets[e]), int(offsets[e + 1])):
            a = torch.zeros(F, dtype=torch.float64)
            for f in range(F):
                g = sum(xv[r, k] * Wg[f, k] for k in range(H)) * float(sx[r]) * float(sg[e, f])
                u = sum(xv[r, k] * Wu[f, k] for k in range(H)) * float(sx[r]) * float(su[e, f])
                g, u = float(_bf16(torch.tensor(g))), float(_bf16(torch.tensor(u)))
                a[f] = float(_bf16(torch.tensor(g / (1.0 + torch.exp(torch.tensor(-g)).item()) * u)))
            aq, sa = quant_rows(a.float().unsqueeze(0))
            av = aq.view(torch.float8_e4m3fn).double()[0]
            for h in range(H):
                y[r, h] = float(_bf16(torch.tensor(sum(av[f] * Wd[h, f] for f in range(F)) * float(sa[0])
                                                  * float(sd[e, h]))))
    return y
