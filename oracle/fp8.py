"""CPU restatement of the fp8 (e4m3) forward of the expert FFN -- TEST INFRASTRUCTURE ONLY.

The reference has no fp8 path (moe-engine's experts run in the model dtype: pkg/distributed/moe_layer.py
L:166-198, L:326-337); the fp8 variant is this build's own, and its contract is stated here:

* ``quant_rows`` -- one fp32 scale per row, ``absmax / 448`` (448 = the largest finite e4m3 value),
  elements ``x * (448 / absmax)`` (fp32; one division per row) rounded to nearest even into OCP e4m3
  (``torch.float8_e4m3fn``).  A row with absmax below 2^-118 (a zero row, or one so small that 448 / absmax
  would overflow fp32 and turn its zeros into NaN) is a zero row: scale 1, elements ``x`` rounded (to +-0).
* ``quant_mx`` -- block quantization of the activations between the two projections (the scaled fp8 MFMA's
  operand format, OCP MX): each run of 32 consecutive elements of a row shares one power-of-two scale 2^e,
  stored as its E8M0 byte e + 127; e is the smallest integer with absmax <= 448 * 2^e (so no element
  saturates), clamped to [-127, 127]; elements ``x * 2^-e`` (exact in fp32) rounded to nearest even into e4m3.
  An all-zero block gets e = -127 and zero bytes.
* ``swiglu_fwd_fp8`` -- the grouped SwiGLU forward on the dequantized operands in float64: per expert segment
  ``hgu = (xq sx) (Wq sw)^T``, ``g`` and ``u`` rounded to bf16, ``act = silu(g) u`` rounded to bf16, ``act``
  block-quantized (``quant_mx``), ``y = (actq 2^e) (Wdq sd)^T`` rounded to bf16.

Pinning (``tests/test_oracle_fp8.py``): ``quant_mx`` by closed forms -- every nonzero block's absmax element
dequantizes into (224, 448] (e is minimal: one smaller would put it above 448), a brute-force search for the
smallest integer e, powers of two mapping to 0x38 / 0x40, zero blocks, the e4m3 rounding bound per element, and
torch's float8 conversion of ``x * 2^-e``; ``quant_rows`` by closed forms -- a row's absmax element maps to
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


MX_BLOCK = 32


def mx_exponent(amax: torch.Tensor) -> torch.Tensor:
    """Smallest integer e with amax <= 448 * 2^e, clamped to [-127, 127] (-127 for a zero block), int32.
    With amax = m 2^p (0.5 <= m < 1, torch.frexp): e = p - 9 when m <= 0.875 (448 = 0.875 * 2^9), else p - 8."""
    m, p = torch.frexp(amax.double())
    e = torch.where(m <= 0.875, p - 9, p - 8)
    e = torch.where(amax > 0, e, torch.full_like(e, -127))
    return e.clamp(-127, 127).to(torch.int32)


def quant_mx(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [rows, cols] (cols % 32 == 0) -> (e4m3 bytes uint8 [rows, cols], E8M0 scale bytes uint8
    [rows, cols / 32]): block b of row r holds elements x[r, 32 b : 32 b + 32] * 2^-e rounded to e4m3."""
    v = x.float()
    R, C = v.shape
    blk = v.reshape(R, C // MX_BLOCK, MX_BLOCK)
    e = mx_exponent(blk.abs().amax(-1))
    q = (blk * torch.pow(2.0, -e.double()).float().unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(R, C), (e + 127).to(torch.uint8)


def dequant_mx(q: torch.Tensor, sbytes: torch.Tensor) -> torch.Tensor:
    """e4m3 bytes and E8M0 block scales -> float64 values."""
    R, C = q.shape
    v = q.view(torch.float8_e4m3fn).double().reshape(R, C // MX_BLOCK, MX_BLOCK)
    return (v * torch.pow(2.0, sbytes.double() - 127.0).unsqueeze(-1)).reshape(R, C)


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
    aq, sa = quant_mx(a_src.float())
    ad = dequant_mx(aq, sa)
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
            aq, sa = quant_mx(a.float().unsqueeze(0))
            av = aq.view(torch.float8_e4m3fn).double()[0]
            for h in range(H):
                acc = sum(av[f] * 2.0 ** (int(sa[0, f // 32]) - 127) * Wd[h, f] for f in range(F))
                y[r, h] = float(_bf16(torch.tensor(acc * float(sd[e, h]))))
    return y
