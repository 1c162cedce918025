"""SwiGLU grouped GEMM (forward and backward) against a plain PyTorch float32
reference of the same op, on imbalanced expert segments (including empty
experts and segments that are not a multiple of the 128-row tile).
Tolerance: bf16 2e-2 max-norm relative."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gpu_util import assert_rel, dev, say

from moe_mi355 import ops

pytestmark = pytest.mark.gpu


def _ref(xp, wg, wu, wd, offs, dy, dtype=torch.float32):
    """torch reference (CPU autograd, float32 or float64) of act, hgu, y and all gradients."""
    xp = xp.to(dtype).cpu().requires_grad_(True)
    wg = wg.to(dtype).cpu().requires_grad_(True)
    wu = wu.to(dtype).cpu().requires_grad_(True)
    wd = wd.to(dtype).cpu().requires_grad_(True)
    acts, gs, us, ys = [], [], [], []
    for e in range(len(offs) - 1):
        lo, hi = offs[e], offs[e + 1]
        x = xp[lo:hi]
        g = x @ wg[e].t()
        u = x @ wu[e].t()
        a = F.silu(g) * u
        acts.append(a), gs.append(g), us.append(u), ys.append(a @ wd[e].t())
    act, g, u, y = (torch.cat(t, 0) for t in (acts, gs, us, ys))
    (y * dy.to(dtype).cpu()[: y.shape[0]]).sum().backward()
    return act.detach(), g.detach(), u.detach(), y.detach(), xp.grad, wg.grad, wu.grad, wd.grad


SEGS = [
    ("balanced", 256, 512, [128, 128, 128, 128]),
    ("ragged", 264, 192, [0, 130, 127, 300, 1, 0, 45]),
    ("one_expert", 128, 128, [333]),
    ("many_small", 136, 96, [5, 0, 17, 64, 3, 129, 0, 8, 1, 2]),
]


@pytest.mark.parametrize("case", SEGS, ids=lambda c: c[0])
def test_swiglu_grouped_gemm(case):
    name, H, Fd, counts = case
    say(f"[swiglu] {name} H={H} F={Fd} counts={counts}")
    E = len(counts)
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    R = offs[-1]
    g = torch.Generator().manual_seed(len(name))
    xp = torch.randn(R, H, generator=g).to(torch.bfloat16)
    wg = (torch.randn(E, Fd, H, generator=g) / H**0.5).to(torch.bfloat16)
    wu = (torch.randn(E, Fd, H, generator=g) / H**0.5).to(torch.bfloat16)
    wd = (torch.randn(E, H, Fd, generator=g) / Fd**0.5).to(torch.bfloat16)
    dy = torch.randn(R, H, generator=g).to(torch.bfloat16)
    d = dev()
    off_d = torch.tensor(offs, dtype=torch.int32, device=d)
    X, WG, WU, WD, DY = (t.to(d) for t in (xp, wg, wu, wd, dy))
    act, hgu, y = ops.swiglu_forward(X, WG, WU, WD, off_d)
    dxp, dwg, dwu, dwd = ops.swiglu_backward(DY, X, act, hgu, WG, WU, WD, off_d)
    torch.cuda.synchronize()
    r_act, r_g, r_u, r_y, r_dx, r_dwg, r_dwu, r_dwd = _ref(xp, wg, wu, wd, offs, dy)
    tol = 2e-2
    assert_rel(hgu[:, :Fd], r_g, tol, "gate pre-activation")
    assert_rel(hgu[:, Fd:], r_u, tol, "up pre-activation")
    assert_rel(act, r_act, tol, "act")
    assert_rel(y, r_y, tol, "y")
    assert_rel(dxp, r_dx, tol, "dxp")
    for e in range(E):
        if counts[e] == 0:
            assert dwg[e].abs().max().item() == 0 and dwd[e].abs().max().item() == 0
    assert_rel(dwg, r_dwg, tol, "dw_gate")
    assert_rel(dwu, r_dwu, tol, "dw_up")
    assert_rel(dwd, r_dwd, tol, "dw_down")


def test_swiglu_deterministic():
    d = dev()
    E, H, Fd = 4, 256, 256
    offs = torch.tensor([0, 200, 200, 333, 512], dtype=torch.int32, device=d)
    g = torch.Generator().manual_seed(1)
    xp = torch.randn(512, H, generator=g).to(torch.bfloat16).to(d)
    wg = (torch.randn(E, Fd, H, generator=g) * 0.05).to(torch.bfloat16).to(d)
    wu = (torch.randn(E, Fd, H, generator=g) * 0.05).to(torch.bfloat16).to(d)
    wd = (torch.randn(E, H, Fd, generator=g) * 0.05).to(torch.bfloat16).to(d)
    dy = torch.randn(512, H, generator=g).to(torch.bfloat16).to(d)
    outs = []
    for _ in range(2):
        act, hgu, y = ops.swiglu_forward(xp, wg, wu, wd, offs)
        outs.append([y, *ops.swiglu_backward(dy, xp, act, hgu, wg, wu, wd, offs)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


F32_SEGS = SEGS + [("f32_partial_k", 1000, 160, [0, 300, 129, 1, 700, 33]),
                   ("f32_one_slice", 12, 32, [3, 17, 0, 40])]


@pytest.mark.parametrize("case", F32_SEGS, ids=lambda c: c[0])
def test_swiglu_grouped_gemm_f32(case):
    """The float32 grouped GEMM (v_mfma_f32_32x32x2_f32) against a float64 torch reference of the same op:
    forward, pre-activations and every gradient within the fp32 tolerance 1e-5 (max-norm relative)."""
    name, H, Fd, counts = case
    say(f"[swiglu f32] {name} H={H} F={Fd} counts={counts}")
    E = len(counts)
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    R = offs[-1]
    g = torch.Generator().manual_seed(100 + len(name))
    xp = torch.randn(R, H, generator=g)
    wg = torch.randn(E, Fd, H, generator=g) / H**0.5
    wu = torch.randn(E, Fd, H, generator=g) / H**0.5
    wd = torch.randn(E, H, Fd, generator=g) / Fd**0.5
    dy = torch.randn(R, H, generator=g)
    d = dev()
    off_d = torch.tensor(offs, dtype=torch.int32, device=d)
    X, WG, WU, WD, DY = (t.to(d) for t in (xp, wg, wu, wd, dy))
    act, hgu, y = ops.swiglu_forward(X, WG, WU, WD, off_d)
    dxp, dwg, dwu, dwd = ops.swiglu_backward(DY, X, act, hgu, WG, WU, WD, off_d)
    torch.cuda.synchronize()
    r = _ref(xp.double(), wg.double(), wu.double(), wd.double(), offs, dy.double(), dtype=torch.float64)
    r_act, r_g, r_u, r_y, r_dx, r_dwg, r_dwu, r_dwd = r
    tol = 1e-5
    assert_rel(hgu[:, :Fd], r_g, tol, "gate pre-activation")
    assert_rel(hgu[:, Fd:], r_u, tol, "up pre-activation")
    assert_rel(act, r_act, tol, "act")
    assert_rel(y, r_y, tol, "y")
    assert_rel(dxp, r_dx, tol, "dxp")
    for e in range(E):
        if counts[e] == 0:
            assert dwg[e].abs().max().item() == 0 and dwd[e].abs().max().item() == 0
    assert_rel(dwg, r_dwg, tol, "dw_gate")
    assert_rel(dwu, r_dwu, tol, "dw_up")
    assert_rel(dwd, r_dwd, tol, "dw_down")
