"""Parity of the fused HIP router (forward + backward) against the float64 CPU
oracle on the same seeded inputs.

Bars (written here, per the north star): top-k indices and dispatch counts
bit-exact wherever the float64 top-k probability margin exceeds 1e-6; logits,
weights, statistics and gradients within 1e-5 max-norm relative error for
float32 and 2e-2 for bfloat16.
"""

from __future__ import annotations

import math

import pytest
import torch

from gpu_util import MARGIN, TOL, assert_rel, dev, say
from oracle import router as OR

from moe_mi355 import configs, ops
from moe_mi355.router import RouterCore

pytestmark = pytest.mark.gpu

# (N, H, E, K, x dtype, gate dtype)
SHAPES = [
    (4096, 512, 8, 2, torch.float32, torch.float32),      # C1 (fp32 MFMA forward, fp32 dx / dwg kernel)
    (1000, 300, 16, 4, torch.float32, torch.float32),     # fp32: H % 16 != 0 (partial last chunk), E = 16
    (20000, 256, 64, 6, torch.float32, torch.float32),    # fp32: 4 expert tiles, 4 groups per block
    (40000, 128, 8, 2, torch.float32, torch.float32),     # fp32: 8 groups per block
    (257, 64, 3, 2, torch.float32, torch.float32),        # fp32: E < 16, more waves than chunks
    (130, 70, 8, 2, torch.float32, torch.float32),        # fp32 with H % 4 != 0 -> generic kernels
    (16384, 4096, 8, 2, torch.bfloat16, torch.bfloat16),  # C2 at full size (MFMA kernels)
    (1000, 256, 16, 4, torch.bfloat16, torch.bfloat16),   # ragged token count
    (64, 64, 8, 8, torch.bfloat16, torch.bfloat16),       # K == E
    (37, 128, 32, 1, torch.bfloat16, torch.bfloat16),     # K == 1, N < one block
    (300, 2048, 64, 6, torch.bfloat16, torch.bfloat16),   # C3 expert count (wide streaming kernel)
    (4096, 2048, 64, 6, torch.bfloat16, torch.bfloat16),  # C3 shape, 32 blocks folded by the last one
    (260, 512, 128, 8, torch.bfloat16, torch.bfloat16),   # C5 expert count (wide streaming kernels)
    (8192, 2048, 128, 8, torch.bfloat16, torch.bfloat16), # C5 width: 32 backward chunks of 256 tokens
    (200, 256, 50, 4, torch.bfloat16, torch.bfloat16),    # E % 8 != 0 on the wide kernels
    (200, 128, 256, 8, torch.bfloat16, torch.bfloat16),   # E = 256: 16 expert tiles
    (150, 192, 160, 4, torch.bfloat16, torch.bfloat16),   # 128 < E < 256: padded tiles
    (129, 320, 48, 5, torch.bfloat16, torch.bfloat16),    # 32 < E < 64: padded tiles, ragged block
    (96, 96, 64, 4, torch.bfloat16, torch.bfloat16),      # H % 64 != 0 -> packed-gate kernel
    (100, 96, 10, 3, torch.bfloat16, torch.bfloat16),     # E not a multiple of 16
    (128, 256, 40, 18, torch.bfloat16, torch.bfloat16),   # K > 16 on the MFMA path
    (300, 256, 64, 32, torch.bfloat16, torch.bfloat16),   # K = 32 (the largest) on the wide kernel, E = 64
    (170, 256, 128, 12, torch.bfloat16, torch.bfloat16),  # K = 12 on the wide kernel, E = 128 (K = 32 there: the ties test)
    (50, 72, 8, 2, torch.bfloat16, torch.bfloat16),       # H % 32 != 0 -> generic path
    (333, 256, 24, 20, torch.float32, torch.float32),     # K > 16; fp32 forward, generic backward (E > 16)
    (200, 64, 8, 2, torch.bfloat16, torch.float32),       # mixed dtypes -> generic path
    (513, 1024, 8, 5, torch.bfloat16, torch.bfloat16),    # E = 8, K > 4: 16-wave backward, ids read where G is formed
    (700, 1024, 6, 3, torch.bfloat16, torch.bfloat16),    # E < 8, K = 3: 16-wave backward, per-element gate rows
    (2048, 2048, 4, 1, torch.bfloat16, torch.bfloat16),   # K = 1, E = 4 on the 16-wave backward
    (300, 512, 8, 2, torch.bfloat16, torch.bfloat16),     # H % 1024 != 0: 4-wave backward with 8 G slots
]


def _ids(s):
    N, H, E, K, xd, wd = s
    return f"N{N}-H{H}-E{E}-K{K}-{str(xd)[6:]}-{str(wd)[6:]}"


def _inputs(N, H, E, K, xd, wd, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, H, generator=g).to(xd)
    w = (torch.randn(H, E, generator=g) * 0.02 * math.sqrt(4096.0 / H)).to(wd)
    gw = torch.randn(N, K, generator=g).to(xd)
    return x, w, gw


def _check_forward(x, w, K, bias=None):
    d = dev()
    xd, wd = x.to(d), w.to(d)
    bd = bias.to(d) if bias is not None else None
    idx, wt, logits, lse, cnt, stats = ops.router_forward(xd, wd, K, bd)
    torch.cuda.synchronize()
    ref = OR.route_fwd(x, w, K, bias=bias)
    tol = TOL[x.dtype]
    ok = ref["margin"] > MARGIN
    idx_c = idx.cpu()
    assert ok.float().mean() > 0.95, "test inputs have too many near-ties"
    assert torch.equal(idx_c[ok], ref["idx"][ok]), "top-k indices differ where the margin exceeds 1e-6"
    assert_rel(logits, ref["logits"], 1e-5, "logits")
    # weights: compare at the device's routing so a near-tie token compares like with like
    v = ref["probs"].gather(1, idx_c)
    w_at = v / v.sum(-1, keepdim=True).clamp_min(1e-30)
    assert_rel(wt.float(), w_at, tol, "weights")
    cnt_c = cnt.cpu()
    assert torch.equal(cnt_c, torch.bincount(idx_c.reshape(-1), minlength=w.shape[1]))
    if bool(ok.all()):
        assert torch.equal(cnt_c, OR.dispatch_counts(ref["idx"], w.shape[1]))
    lse_ref = torch.logsumexp(ref["logits"], -1)
    assert_rel(lse, lse_ref, 1e-5, "lse")
    st = stats.cpu().double()
    N, E = ref["probs"].shape
    cntd = cnt_c.double()
    assert st[5].item() == N * K
    assert st[6].item() == 0.0
    assert abs(st[0].item() - OR.z_stat(ref["logits"])) <= 1e-5 * max(1.0, OR.z_stat(ref["logits"]))
    P = ref["probs"].mean(0)
    assert_rel(st[8 : 8 + E], P, 1e-5, "mean probabilities")
    aux_ref = float(E * ((cntd / (N * K)) * P).sum())
    assert abs(st[1].item() - aux_ref) <= 1e-5 * aux_ref
    assert abs(st[2].item() - OR.load_imbalance(cnt_c)) <= 1e-6 * OR.load_imbalance(cnt_c)
    assert abs(st[3].item() - float(cntd.mean())) <= 1e-6 * float(cntd.mean())
    if E > 1:
        assert abs(st[4].item() - float(cntd.std())) <= 1e-5 * max(1.0, float(cntd.std()))
    return idx, wt, logits, cnt


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_router_forward_parity(shape):
    N, H, E, K, xd, wd = shape
    say(f"[router fwd] {_ids(shape)}")
    x, w, _ = _inputs(N, H, E, K, xd, wd, seed=N + H + E + K)
    _check_forward(x, w, K)


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
@pytest.mark.parametrize("losses", [False, True], ids=["plain", "aux_z"])
def test_router_backward_parity(shape, losses):
    N, H, E, K, xd, wd = shape
    say(f"[router bwd] {_ids(shape)} losses={losses}")
    x, w, gw = _inputs(N, H, E, K, xd, wd, seed=7 * N + H + E + K)
    d = dev()
    alpha, beta = (0.01, 1e-3) if losses else (0.0, 0.0)
    xd_, wd_ = x.to(d).requires_grad_(True), w.to(d).requires_grad_(True)
    idx, wt, aux, z, logits, cnt, stats = RouterCore.apply(xd_, wd_, K, alpha, beta, None)
    loss = (wt.float() * gw.to(d).float()).sum()
    if losses:
        loss = loss + aux + z
    loss.backward()
    torch.cuda.synchronize()
    ref = OR.router_full(x, w, K, grad_w=gw, alpha=alpha, beta=beta, idx_override=idx.cpu())
    tol = TOL[x.dtype]
    # gradients of order 1e-2 here; the floor only matters where the exact gradient vanishes (K=1)
    assert_rel(xd_.grad, ref["dX"], tol, "dX", floor=1e-4)
    assert_rel(wd_.grad, ref["dW"], tol, "dW", floor=1e-4)
    if losses:
        assert abs(aux.item() - float(ref["aux"])) <= 1e-5 * float(ref["aux"])
        assert abs(z.item() - float(ref["z"])) <= 1e-5 * float(ref["z"])


def test_router_c2_full_size_backward():
    """C2 exactly as the benchmark draws it (seed 1), forward and backward."""
    cfg = configs.C2
    say("[router C2 full]")
    inp = configs.router_inputs(cfg)
    x, w, gw = inp["x"], inp["gate_w"], inp["grad_w"]
    idx, _, _, _ = _check_forward(x, w, cfg.K)
    d = dev()
    xd_, wd_ = x.to(d).requires_grad_(True), w.to(d).requires_grad_(True)
    out = RouterCore.apply(xd_, wd_, cfg.K, 0.0, 0.0, None)
    (out[1].float() * gw.to(d).float()).sum().backward()
    ref = OR.router_full(x, w, cfg.K, grad_w=gw, idx_override=out[0].cpu())
    assert_rel(xd_.grad, ref["dX"], 2e-2, "dX")
    assert_rel(wd_.grad, ref["dW"], 2e-2, "dW")


def test_router_deterministic():
    say("[router determinism]")
    x, w, gw = _inputs(4096, 1024, 64, 6, torch.bfloat16, torch.bfloat16, seed=5)
    d = dev()
    outs = []
    for _ in range(2):
        xd_, wd_ = x.to(d).requires_grad_(True), w.to(d).requires_grad_(True)
        idx, wt, aux, z, logits, cnt, stats = RouterCore.apply(xd_, wd_, 6, 0.01, 1e-3, None)
        ((wt.float() * gw.to(d).float()).sum() + aux + z).backward()
        outs.append([t.detach().cpu() for t in (idx, wt, logits, cnt, stats, xd_.grad, wd_.grad)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("N,H,E,K", [(100, 64, 8, 3), (300, 256, 64, 6), (200, 512, 128, 8), (150, 256, 64, 32),
                                     (120, 256, 128, 32)])
def test_router_exact_ties_take_lowest_index(N, H, E, K):
    """All logits equal: the first K experts in order.  Gate columns equal in pairs (2j, 2j + 1): the device
    logits of a pair are bit-identical, so the picks come in pairs, the lower id first.  E > 32 runs the wide
    streaming forward."""
    say(f"[router ties] N={N} H={H} E={E} K={K}")
    d = dev()
    x = torch.randn(N, H).to(torch.bfloat16).to(d)
    w = torch.zeros(H, E, dtype=torch.bfloat16, device=d)
    idx, wt, *_ = ops.router_forward(x, w, K)
    assert torch.equal(idx.cpu(), torch.arange(K).expand(N, K))
    assert torch.allclose(wt.float().cpu(), torch.full((N, K), 1.0 / K), atol=1e-3)
    if K % 2:
        return
    g = torch.Generator().manual_seed(E + K)
    w = (torch.randn(H, E // 2, generator=g) * 0.05).to(torch.bfloat16).repeat_interleave(2, dim=1).to(d)
    idx, wt, logits, *_ = ops.router_forward(x, w, K)
    idx, wt, logits = idx.cpu(), wt.float().cpu(), logits.float().cpu()
    assert torch.equal(logits[:, 0::2], logits[:, 1::2])
    assert torch.equal(idx[:, 0::2] % 2, torch.zeros(N, K // 2, dtype=idx.dtype))
    assert torch.equal(idx[:, 1::2], idx[:, 0::2] + 1)
    assert torch.equal(wt[:, 0::2], wt[:, 1::2])
    # the picked pairs are the K / 2 largest pair logits, in descending order
    top = logits[:, 0::2].topk(K // 2, dim=-1).values
    assert torch.equal(logits.gather(1, idx[:, 0::2]), top)


def test_router_with_bias_matches_oracle():
    say("[router bias]")
    x, w, _ = _inputs(512, 256, 32, 4, torch.bfloat16, torch.bfloat16, seed=11)
    bias = configs.zipf_bias(32, torch.Generator().manual_seed(4))
    _check_forward(x, w, 4, bias=bias)


def test_router_empty_batch():
    d = dev()
    x = torch.zeros(0, 64, dtype=torch.bfloat16, device=d)
    w = torch.randn(64, 8, device=d).to(torch.bfloat16)
    idx, wt, logits, lse, cnt, stats = ops.router_forward(x, w, 2)
    assert idx.shape == (0, 2) and int(cnt.sum()) == 0


def test_router_forward_workspace_reuse_across_paths():
    """The streaming forwards fold their finalize into the last block through a completion counter kept in the
    reused (per stream) workspace.  Alternate shapes that take the two streaming paths, the packed-gate path and
    the generic path on one stream, twice, and check every call's counts and statistics: a counter that a call
    leaves non-zero, or that another path overwrites, shows up as missing or stale statistics."""
    say("[router workspace reuse]")
    seq = [
        (16384, 4096, 8, 2, torch.bfloat16, torch.bfloat16),  # streaming, 256 blocks
        (300, 2048, 64, 6, torch.bfloat16, torch.bfloat16),   # wide streaming, 3 blocks
        (96, 96, 64, 4, torch.bfloat16, torch.bfloat16),      # packed-gate kernel + finalize launch
        (1000, 256, 16, 4, torch.bfloat16, torch.bfloat16),   # streaming, other block count
        (4096, 512, 8, 2, torch.float32, torch.float32),      # fp32 MFMA form, its own fold
        (130, 70, 8, 2, torch.float32, torch.float32),        # generic path
        (37, 512, 32, 1, torch.bfloat16, torch.bfloat16),     # streaming, a single block
    ]
    for rep in range(2):
        for i, shape in enumerate(seq):
            N, H, E, K, xd, wd = shape
            x, w, _ = _inputs(N, H, E, K, xd, wd, seed=100 + 7 * i + rep)
            _check_forward(x, w, K)


@pytest.mark.parametrize("losses", [False, True], ids=["plain", "aux_z"])
def test_router_fp32_unaligned_x_takes_the_generic_kernels(losses):
    """fp32 x whose data starts 4 bytes past a 16-byte boundary (a contiguous view one element into its storage):
    the fp32 MFMA forward and the fp32 dx / dwg kernel read x with 16-byte loads, so the call takes the generic
    kernels under the same workspace plan; forward and backward still match the oracle."""
    N, H, E, K = 1000, 512, 8, 2
    say(f"[router fp32 unaligned] losses={losses}")
    x, w, gw = _inputs(N, H, E, K, torch.float32, torch.float32, seed=77)
    d = dev()
    base = torch.empty(N * H + 1, device=d)
    xv = base[1:].view(N, H)
    with torch.no_grad():
        xv.copy_(x.to(d))
    assert xv.data_ptr() % 16 != 0 and xv.is_contiguous()
    xv.requires_grad_(True)
    wd_ = w.to(d).requires_grad_(True)
    alpha, beta = (0.01, 1e-3) if losses else (0.0, 0.0)
    idx, wt, aux, z, logits, cnt, stats = RouterCore.apply(xv, wd_, K, alpha, beta, None)
    loss = (wt * gw.to(d)).sum() + (aux + z if losses else 0.0)
    loss.backward()
    torch.cuda.synchronize()
    fwd = OR.route_fwd(x, w, K)
    ok = fwd["margin"] > MARGIN
    assert torch.equal(idx.cpu()[ok], fwd["idx"][ok])
    assert_rel(logits, fwd["logits"], 1e-5, "logits")
    ref = OR.router_full(x, w, K, grad_w=gw, alpha=alpha, beta=beta, idx_override=idx.cpu())
    assert_rel(xv.grad, ref["dX"], 1e-5, "dX", floor=1e-4)
    assert_rel(wd_.grad, ref["dW"], 1e-5, "dW", floor=1e-4)


@pytest.mark.parametrize("N,H,E,K,dt", [
    (300, 256, 8, 2, torch.bfloat16),     # E <= 16 streaming forward (one lane per token)
    (300, 256, 64, 6, torch.bfloat16),    # wide forward, four lanes per token
    (260, 512, 128, 8, torch.bfloat16),   # wide forward, four lanes per token, 8 expert tiles
    (200, 128, 256, 8, torch.bfloat16),   # wide forward, 16 lanes per token
    (300, 256, 16, 4, torch.float32),     # fp32 MFMA forward
], ids=lambda v: str(v)[6:] if isinstance(v, torch.dtype) else str(v))
def test_router_nan_gate_column_is_never_picked(N, H, E, K, dt):
    """A NaN in one gate column makes that expert's logit NaN for every token.  Every forward path maps it to
    -inf for the softmax and the top-k: the expert is never picked and gets probability 0, the weights stay
    finite, the stored logits keep the NaN and the non-finite count is N.  The indices and weights are those
    of the float64 oracle with that expert's logit at -inf (a -inf bias)."""
    from moe_mi355.router import STAT_NONFINITE
    say(f"[router nan column] N={N} H={H} E={E} K={K} {dt}")
    d = dev()
    x, w, _ = _inputs(N, H, E, K, dt, dt, seed=E + 1)
    e0 = E // 2 + 1
    w_nan = w.clone()
    w_nan[5, e0] = float("nan")
    idx, wt, logits, lse, cnt, stats = ops.router_forward(x.to(d), w_nan.to(d), K)
    torch.cuda.synchronize()
    idx, wt, logits, stats = idx.cpu(), wt.float().cpu(), logits.cpu(), stats.float().cpu()
    others = [e for e in range(E) if e != e0]
    assert torch.isnan(logits[:, e0]).all()
    assert torch.isfinite(logits[:, others]).all()
    assert not bool((idx == e0).any())
    assert torch.isfinite(wt).all()
    assert float(stats[STAT_NONFINITE]) == N
    bias = torch.zeros(E, dtype=torch.float64)
    bias[e0] = float("-inf")
    ref = OR.route_fwd(x, w, K, bias=bias)
    ok = ref["margin"] > MARGIN
    assert ok.float().mean() > 0.9
    assert torch.equal(idx[ok], ref["idx"][ok])
    assert_rel(wt[ok], ref["w"][ok], TOL[dt], "weights")


# (N, H, E, K, x dtype, gate dtype): the streaming backward (16- and 4-wave), the wide backward, the
# non-streaming MFMA form, the fp32 and the generic forms (the last three add the addend in a separate pass)
ACC_SHAPES = [
    (16384, 4096, 8, 2, torch.bfloat16, torch.bfloat16),
    (300, 512, 8, 2, torch.bfloat16, torch.bfloat16),
    (1000, 256, 16, 4, torch.bfloat16, torch.bfloat16),
    (8192, 2048, 128, 8, torch.bfloat16, torch.bfloat16),
    (129, 320, 48, 5, torch.bfloat16, torch.bfloat16),
    (96, 96, 64, 4, torch.bfloat16, torch.bfloat16),
    (4096, 512, 8, 2, torch.float32, torch.float32),
    (50, 72, 8, 2, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("shape", ACC_SHAPES, ids=_ids)
def test_router_bwd_acc_adds_the_other_gradient(shape):
    """moe_router_bwd_acc: dx = the router's gradient of x + dx_add, formed inside the dx kernel, bit-identical
    to moe_router_bwd's dx followed by the tensor addition autograd would make (bf16: each rounded value
    widened, summed in fp32, rounded once); dwg unchanged."""
    N, H, E, K, xdt, wdt = shape
    say(f"[router bwd acc] N={N} H={H} E={E} K={K} {xdt} {wdt}")
    d = dev()
    g = torch.Generator().manual_seed(N + H + E)
    x = torch.randn(N, H, generator=g).to(xdt).to(d)
    w = (torch.randn(H, E, generator=g) * 0.05).to(wdt).to(d)
    gw = torch.randn(N, K, generator=g).to(d)
    add = torch.randn(N, H, generator=g).to(xdt).to(d)
    idx, _wt, logits, _lse, cnt, _stats = ops.router_forward(x, w, K)
    dx0, dw0 = ops.router_backward(x, w, logits, idx, gw, cnt, aux_coef=0.01, z_coef=1e-3)
    dx1, dw1 = ops.router_backward(x, w, logits, idx, gw, cnt, aux_coef=0.01, z_coef=1e-3, dx_add=add)
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx0 + add), "dx differs from dx + dx_add"
    assert torch.equal(dw1, dw0)
