"""fp8 (e4m3) forward of the expert FFN on the GPU against oracle/fp8.py: row quantization and the quantized
dispatch payload bit-exact, the fp8 grouped GEMMs within the bf16 output tolerance of the float64 product of
the same quantized operands, and the layer's fp8 forward against both the oracle chain and the bf16 layer."""

from __future__ import annotations

import pytest
import torch

from gpu_util import TOL, assert_rel, dev, say

from moe_mi355 import ops
from oracle import fp8 as O8
from pkg.distributed import build_topology
from pkg.distributed.moe_layer import DistributedMoELayer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,dtype", [(64, 16, torch.bfloat16), (300, 4096, torch.bfloat16),
                                             (33, 14336, torch.bfloat16), (100, 512, torch.float32),
                                             (9, 20480, torch.bfloat16),   # past the register path: two passes
                                             (7, 16400, torch.float32)])
def test_quant_rows_bit_exact(rows, cols, dtype):
    say(f"[fp8 quant] {rows}x{cols} {dtype}")
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * torch.logspace(-4, 4, rows).unsqueeze(1)).to(dtype)
    x[rows // 2] = 0.0
    q, s = ops.quant_rows_fp8(x.to(dev()))
    rq, rs = O8.quant_rows(x)
    assert torch.equal(s.cpu(), rs), "row scales"
    assert torch.equal(q.cpu(), rq), "e4m3 bytes"


@pytest.mark.parametrize("cols,dtype", [(4096, torch.bfloat16), (20480, torch.bfloat16), (512, torch.float32)])
def test_quant_tiny_rows_are_zero_rows(cols, dtype):
    """Rows with absmax below 2^-118 (down to bf16 / fp32 subnormals) quantize as zero rows -- scale 1, bytes
    +-0, never NaN -- bit-exactly as the oracle; a row at exactly 2^-118 keeps its own scale."""
    say(f"[fp8 quant tiny rows] cols={cols} {dtype}")
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(6, cols, generator=g)
    x[0] *= 1e-37
    x[1] *= 1e-39                      # subnormal in fp32 and bf16
    x[2] = 0.0
    x[2, 3] = 2.0 ** -118
    x[3] *= 2.0 ** -120
    x[4] = -3e-37
    x = x.to(dtype)
    q, s = ops.quant_rows_fp8(x.to(dev()))
    rq, rs = O8.quant_rows(x)
    assert torch.equal(s.cpu(), rs), "row scales"
    assert torch.equal(q.cpu(), rq), "e4m3 bytes"
    assert not bool(torch.isnan(O8.dequant(q.cpu(), s.cpu())).any())
    assert float(s[2]) != 1.0 and float(s[0]) == 1.0


@pytest.mark.parametrize("layout,cap,dtype", [("reference", -1, torch.bfloat16), ("routed", -1, torch.bfloat16),
                                              ("routed", 40, torch.bfloat16), ("reference", -1, torch.float32)])
def test_permute_fp8_bit_exact(layout, cap, dtype):
    say(f"[fp8 permute] {layout} cap={cap} {dtype}")
    N, H, E, K = 257, 512, 8, 2
    g = torch.Generator().manual_seed(7)
    x = torch.randn(N, H, generator=g).to(dtype)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(N)])
    p = ops.plan(idx.to(dev()), E, capacity=cap, layout=ops.LAYOUT_ROUTED if layout == "routed" else ops.LAYOUT_REFERENCE)
    xq, sx = ops.permute_fp8(x.to(dev()), p)
    rows = int(p.offsets[-1].item())
    src = p.row_slot[:rows].cpu().long() // K
    rq, rs = O8.quant_rows(x[src])
    assert torch.equal(xq[:rows].cpu(), rq) and torch.equal(sx[:rows].cpu(), rs)


def _weights(E, F, H, seed):
    g = torch.Generator().manual_seed(seed)
    wg = (torch.randn(E, F, H, generator=g) * H ** -0.5).to(torch.bfloat16)
    wu = (torch.randn(E, F, H, generator=g) * H ** -0.5).to(torch.bfloat16)
    wd = (torch.randn(E, H, F, generator=g) * F ** -0.5).to(torch.bfloat16)
    return wg, wu, wd


@pytest.mark.parametrize("R,H,F,E,counts", [
    (600, 256, 512, 4, [250, 0, 300, 50]),        # an empty expert, ragged segments, rows past offsets[E]
    (512, 4096, 14336, 2, [300, 212]),            # the C4 expert shape
    (96, 128, 64, 3, [1, 90, 5]),                 # segments shorter than a tile, F < a 256-column tile
    (200, 384, 416, 2, [120, 80]),                # 3 k slices in the gate/up product; 4 in the down
                                                  # projection, the last partial (32 of 128)
])
def test_swiglu_forward_fp8_parity(R, H, F, E, counts):
    say(f"[fp8 swiglu] R={R} H={H} F={F} E={E}")
    g = torch.Generator().manual_seed(R + F)
    xp = torch.randn(R, H, generator=g).to(torch.bfloat16)
    wts = _weights(E, F, H, R + 1)
    offsets = torch.tensor([0] + list(torch.tensor(counts).cumsum(0)), dtype=torch.int32)
    d = dev()
    xq, sx = ops.quant_rows_fp8(xp.to(d))
    wq = [ops.quant_rows_fp8(w.to(d)) for w in wts]
    act, hgu, y, (aq, asc) = ops.swiglu_forward_fp8(xq, sx, [q for q, _ in wq], [s for _, s in wq], offsets.to(d),
                                                    return_mx=True)
    torch.cuda.synchronize()
    used = int(offsets[-1])
    oq = [O8.quant_rows(w) for w in wts]
    for (q, s), (rq, rs) in zip(wq, oq):
        assert torch.equal(q.cpu(), rq) and torch.equal(s.cpu(), rs)
    # act block-quantized in the gate/up epilogue: bytes and E8M0 scales bit-exact with the oracle's quant_mx of
    # the kernel's own act
    mq, ms = O8.quant_mx(act[:used].cpu().float())
    assert torch.equal(asc[:used].cpu(), ms), "E8M0 block scales"
    assert torch.equal(aq[:used].cpu(), mq), "e4m3 bytes of act"
    rh, ra, ry = O8.swiglu_fwd_fp8(xq.cpu(), sx.cpu(), [q for q, _ in oq], [s for _, s in oq], offsets.tolist(),
                                   act_in=act.cpu().float())
    tol = TOL[torch.bfloat16]
    assert_rel(hgu[:used], rh[:used], tol, "hgu")
    # act from the kernel's own g, u (its hardware sigmoid), then y from the kernel's act quantized
    g_, u_ = hgu[:used, :F].double().cpu(), hgu[:used, F:].double().cpu()
    assert_rel(act[:used], torch.nn.functional.silu(g_) * u_, tol, "act")
    assert_rel(y[:used], ry[:used], tol, "y")


def test_layer_forward_fp8():
    say("[fp8 layer]")
    torch.manual_seed(3)
    N, H, F, E, K = 384, 512, 1024, 8, 2
    layer = DistributedMoELayer(H, F, E, K, build_topology(), dtype=torch.bfloat16).to(dev())
    x = torch.randn(N, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(dev())
    with torch.no_grad():
        ref = layer(x)
    out = layer.forward_fp8(x)
    assert out.shape == ref.shape and out.dtype == ref.dtype
    # the fp8 forward follows the bf16 one up to the e4m3 rounding of x, the weights and act
    err = ((out.float() - ref.float()).abs().max() / ref.float().abs().max()).item()
    assert err < 0.1, err
    # and it is the oracle chain exactly (within the bf16 output tolerance) on the same plan
    p = layer.last_plan
    wq, ws = layer.quantize_fp8()
    xq, sx = ops.permute_fp8(x, p)
    act, _hgu, y = ops.swiglu_forward_fp8(xq, sx, wq, ws, p.offsets)
    out2 = ops.combine(y, layer.router(x)[1], p)
    assert torch.equal(out2, out)
    # weights changed in place -> the cached e4m3 copy is rebuilt
    before = layer.quantize_fp8()[0][0].clone()
    with torch.no_grad():
        layer.w_gate.mul_(2.0)
    after = layer.quantize_fp8()[0][0]
    assert torch.equal(before, after)  # doubling every row leaves the e4m3 bytes as they were ...
    assert torch.allclose(layer.quantize_fp8()[1][0], 2.0 * ops.quant_rows_fp8(layer.w_gate.detach() / 2.0)[1])


@pytest.mark.parametrize("fp8,R,H,F", [(False, 600, 256, 512), (True, 600, 256, 512), (True, 700, 4096, 2048)])
def test_forward_without_preactivations(fp8, R, H, F):
    """keep_preact=False (inference) stores no hgu and leaves act and y bit-identical."""
    say(f"[swiglu no-preact] fp8={fp8} R={R} H={H} F={F}")
    E = 4
    g = torch.Generator().manual_seed(11)
    xp = torch.randn(R, H, generator=g).to(torch.bfloat16)
    wts = _weights(E, F, H, 12)
    offsets = torch.tensor([0, 250, 250, 550, R], dtype=torch.int32).to(dev())
    if fp8:
        xq, sx = ops.quant_rows_fp8(xp.to(dev()))
        wq = [ops.quant_rows_fp8(w.to(dev())) for w in wts]
        def run(keep):
            a, h, y, (aq, asc) = ops.swiglu_forward_fp8(xq, sx, [q for q, _ in wq], [s for _, s in wq], offsets,
                                                        keep_preact=keep, return_mx=True)
            run.mx = (aq.clone(), asc.clone())  # views of the workspace, which the next call reuses
            return a, h, y
    else:
        xd, wd = xp.to(dev()), [w.to(dev()) for w in wts]
        run = lambda keep: ops.swiglu_forward(xd, *wd, offsets, keep_preact=keep)
    a1, h1, y1 = run(True)
    mx1 = getattr(run, "mx", None)
    a2, h2, y2 = run(False)
    assert h1 is not None and h2 is None
    assert torch.equal(y1, y2)
    if fp8:
        assert a2 is None  # inference: the down projection reads act block-quantized, no bf16 copy
        # the inference epilogue (SwiGLU on the accumulators) writes the same e4m3 bytes and E8M0 scales
        used = int(offsets[-1])
        assert torch.equal(mx1[0][:used], run.mx[0][:used]) and torch.equal(mx1[1][:used], run.mx[1][:used])
    else:
        assert torch.equal(a1, a2)


def test_layer_no_grad_matches_training_forward():
    say("[layer no_grad forward]")
    torch.manual_seed(5)
    layer = DistributedMoELayer(256, 512, 8, 2, build_topology(), dtype=torch.bfloat16).to(dev())
    x = torch.randn(300, 256, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev())
    out = layer(x)
    assert out.requires_grad
    with torch.no_grad():
        ref = layer(x)
    assert torch.equal(out.detach(), ref)
