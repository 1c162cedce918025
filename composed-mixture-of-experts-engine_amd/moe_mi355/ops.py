"""Tensor-level wrappers over the C ABI: allocate outputs with torch's caching
allocator, pass raw pointers and the current stream, check the return code.

No function here synchronises the host or falls back to a CPU path.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib as L


def _c(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


def router_forward(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
    w_dtype: Optional[torch.dtype] = None,
    aux_coef: float = 0.0,
    z_coef: float = 0.0,
    with_losses: bool = False,
) -> Tuple[torch.Tensor, ...]:
    """Fused router forward on the GPU.

    Returns ``(idx int64 [N,K], w [N,K] (w_dtype, default x.dtype), logits f32 [N,E],
    lse f32 [N], cnt int64 [E], stats f32 [8+E])``, followed by the 0-d tensors
    ``aux = aux_coef * stats[1]`` and ``z = z_coef * stats[0]`` when
    ``with_losses``; the stats layout is documented in include/moe_mi355.h.
    """
    dev = L.require_device(x, gate_w, bias)
    x = x.contiguous()
    gate_w = gate_w.contiguous()
    N, H = x.shape
    H2, E = gate_w.shape
    if H != H2:
        raise ValueError(f"router_forward: hidden dims differ ({H} vs {H2})")
    w_dtype = w_dtype or x.dtype
    if bias is not None:
        bias = bias.detach().to(torch.float32).contiguous()
    lib = L.load()
    xdt, wdt, odt = L.dtype_code(x.dtype), L.dtype_code(gate_w.dtype), L.dtype_code(w_dtype)
    idx = torch.empty((N, k), dtype=torch.int64, device=dev)
    w = torch.empty((N, k), dtype=w_dtype, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev)
    lse = torch.empty((N,), dtype=torch.float32, device=dev)
    cnt = torch.empty((E,), dtype=torch.int64, device=dev)
    stats = torch.empty((L.STATS_HEAD + E,), dtype=torch.float32, device=dev)
    aux = torch.empty((), dtype=torch.float32, device=dev) if with_losses else None
    z = torch.empty((), dtype=torch.float32, device=dev) if with_losses else None
    if N == 0:
        cnt.zero_()
        stats.zero_()
        if with_losses:
            aux.zero_()
            z.zero_()
            return idx, w, logits, lse, cnt, stats, aux, z
        return idx, w, logits, lse, cnt, stats
    nbytes = lib.moe_router_fwd_workspace(N, H, E, k, xdt, wdt)
    ws = L.workspace(nbytes, dev, key="router_fwd")  # zeroed once; the kernel leaves its ticket at zero
    rc = lib.moe_router_fwd(
        x.data_ptr(), xdt, gate_w.data_ptr(), wdt, L.ptr(bias), N, H, E, k,
        idx.data_ptr(), w.data_ptr(), odt, logits.data_ptr(), lse.data_ptr(),
        cnt.data_ptr(), stats.data_ptr(), float(aux_coef), float(z_coef), L.ptr(aux), L.ptr(z),
        ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_router_fwd")
    if with_losses:
        return idx, w, logits, lse, cnt, stats, aux, z
    return idx, w, logits, lse, cnt, stats


def router_backward(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    logits: torch.Tensor,
    idx: torch.Tensor,
    grad_w: Optional[torch.Tensor],
    cnt: Optional[torch.Tensor] = None,
    grad_aux: Optional[torch.Tensor] = None,
    grad_z: Optional[torch.Tensor] = None,
    aux_coef: float = 0.0,
    z_coef: float = 0.0,
    dx_add: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused router backward: returns ``(dx [N,H] x.dtype, dgate_w [H,E] gate_w.dtype)``; with ``dx_add``
    ([N, H], x's dtype) dx is the router's gradient of x plus dx_add, summed inside the dx kernel
    (moe_router_bwd_acc)."""
    dev = L.require_device(x, gate_w, logits, idx, grad_w, cnt, dx_add)
    x = x.contiguous()
    gate_w = gate_w.contiguous()
    logits = logits.contiguous()
    idx = idx.contiguous()
    N, H = x.shape
    E = gate_w.shape[1]
    K = idx.shape[1]
    lib = L.load()
    xdt, wdt = L.dtype_code(x.dtype), L.dtype_code(gate_w.dtype)
    gdt = L.MOE_F32
    if grad_w is not None:
        grad_w = grad_w.contiguous()
        if grad_w.dtype not in (torch.float32, torch.bfloat16):
            grad_w = grad_w.float()
        gdt = L.dtype_code(grad_w.dtype)
    if grad_aux is not None:
        grad_aux = grad_aux.detach().to(torch.float32).reshape(1).contiguous()
    if grad_z is not None:
        grad_z = grad_z.detach().to(torch.float32).reshape(1).contiguous()
    dx = torch.empty((N, H), dtype=x.dtype, device=dev)
    if N == 0:
        return dx, torch.zeros((H, E), dtype=gate_w.dtype, device=dev)
    dw = torch.empty((H, E), dtype=gate_w.dtype, device=dev)
    nbytes = lib.moe_router_bwd_workspace(N, H, E, K, xdt, wdt)
    ws = L.workspace(nbytes, dev)
    if dx_add is None:
        rc = lib.moe_router_bwd(
            x.data_ptr(), xdt, gate_w.data_ptr(), wdt, logits.data_ptr(), idx.data_ptr(),
            L.ptr(grad_w), gdt, L.ptr(cnt), L.ptr(grad_aux), L.ptr(grad_z),
            float(aux_coef), float(z_coef), N, H, E, K,
            dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev),
        )
    else:
        if dx_add.shape != (N, H) or dx_add.dtype != x.dtype:
            raise ValueError(f"router_backward: dx_add must be [{N}, {H}] {x.dtype}")
        dx_add = dx_add.contiguous()
        rc = lib.moe_router_bwd_acc(
            x.data_ptr(), xdt, gate_w.data_ptr(), wdt, logits.data_ptr(), idx.data_ptr(),
            L.ptr(grad_w), gdt, L.ptr(cnt), L.ptr(grad_aux), L.ptr(grad_z),
            float(aux_coef), float(z_coef), N, H, E, K,
            dx_add.data_ptr(), dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev),
        )
    L.check(rc, "moe_router_bwd")
    return dx, dw


# ---------------------------------------------------------------------------
# RMSNorm in front of the router
# ---------------------------------------------------------------------------
def rmsnorm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """``xn = ((x * rsqrt(mean(x^2) + eps)) * weight).to(x.dtype)`` over the last dim of ``x [N, H]``.

    Returns ``(xn [N,H] x.dtype, rstd f32 [N])``."""
    dev = L.require_device(x, weight)
    x = x.contiguous()
    weight = weight.contiguous()
    N, H = x.shape
    xn = torch.empty_like(x)
    rstd = torch.empty((N,), dtype=torch.float32, device=dev)
    if N == 0:
        return xn, rstd
    rc = L.load().moe_rmsnorm_fwd(x.data_ptr(), L.dtype_code(x.dtype), weight.data_ptr(),
                                  L.dtype_code(weight.dtype), float(eps), N, H, xn.data_ptr(), rstd.data_ptr(),
                                  L.stream_of(dev))
    L.check(rc, "moe_rmsnorm_fwd")
    return xn, rstd


def rmsnorm_router_forward(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    gate_w: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
    aux_coef: float = 0.0,
    z_coef: float = 0.0,
) -> Tuple[torch.Tensor, ...]:
    """The norm and the router forward over its output in one call (one read of ``x`` from HBM for bf16 x and
    gate with E <= 16).  Returns ``(xn, rstd, idx, w, logits, lse, cnt, stats, aux, z)`` with the outputs of
    :func:`rmsnorm_forward` and :func:`router_forward` (``with_losses=True``)."""
    dev = L.require_device(x, weight, gate_w, bias)
    x = x.contiguous()
    weight = weight.contiguous()
    gate_w = gate_w.contiguous()
    N, H = x.shape
    H2, E = gate_w.shape
    if H != H2:
        raise ValueError(f"rmsnorm_router_forward: hidden dims differ ({H} vs {H2})")
    if bias is not None:
        bias = bias.detach().to(torch.float32).contiguous()
    lib = L.load()
    xdt, gdt, wdt = L.dtype_code(x.dtype), L.dtype_code(weight.dtype), L.dtype_code(gate_w.dtype)
    xn = torch.empty_like(x)
    rstd = torch.empty((N,), dtype=torch.float32, device=dev)
    idx = torch.empty((N, k), dtype=torch.int64, device=dev)
    w = torch.empty((N, k), dtype=x.dtype, device=dev)
    logits = torch.empty((N, E), dtype=torch.float32, device=dev)
    lse = torch.empty((N,), dtype=torch.float32, device=dev)
    cnt = torch.empty((E,), dtype=torch.int64, device=dev)
    stats = torch.empty((L.STATS_HEAD + E,), dtype=torch.float32, device=dev)
    aux = torch.empty((), dtype=torch.float32, device=dev)
    z = torch.empty((), dtype=torch.float32, device=dev)
    if N == 0:
        for t in (cnt, stats, aux, z):
            t.zero_()
        return xn, rstd, idx, w, logits, lse, cnt, stats, aux, z
    nbytes = lib.moe_rmsnorm_router_fwd_workspace(N, H, E, k, xdt, wdt)
    ws = L.workspace(nbytes, dev, key="router_fwd")  # zeroed once; the kernels leave the counter at zero
    rc = lib.moe_rmsnorm_router_fwd(
        x.data_ptr(), xdt, weight.data_ptr(), gdt, float(eps), gate_w.data_ptr(), wdt, L.ptr(bias), N, H, E, k,
        xn.data_ptr(), rstd.data_ptr(), idx.data_ptr(), w.data_ptr(), xdt, logits.data_ptr(), lse.data_ptr(),
        cnt.data_ptr(), stats.data_ptr(), float(aux_coef), float(z_coef), aux.data_ptr(), z.data_ptr(),
        ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_rmsnorm_router_fwd")
    return xn, rstd, idx, w, logits, lse, cnt, stats, aux, z


def rmsnorm_backward(
    x: torch.Tensor,
    weight: torch.Tensor,
    rstd: torch.Tensor,
    dxn: torch.Tensor,
    dxn2: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Backward of :func:`rmsnorm_forward` for the gradient ``dxn (+ dxn2)`` of its output: ``(dx, dweight)``."""
    dev = L.require_device(x, weight, rstd, dxn, dxn2)
    x = x.contiguous()
    weight = weight.contiguous()
    dxn = dxn.contiguous().to(x.dtype)
    if dxn2 is not None:
        dxn2 = dxn2.contiguous().to(x.dtype)
    N, H = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    lib = L.load()
    nbytes = lib.moe_rmsnorm_bwd_workspace(N, H)
    ws = L.workspace(nbytes, dev)
    rc = lib.moe_rmsnorm_bwd(
        x.data_ptr(), L.dtype_code(x.dtype), weight.data_ptr(), L.dtype_code(weight.dtype), rstd.data_ptr(),
        dxn.data_ptr(), L.ptr(dxn2), N, H, dx.data_ptr(), dweight.data_ptr(), ws.data_ptr(), nbytes,
        L.stream_of(dev),
    )
    L.check(rc, "moe_rmsnorm_bwd")
    return dx, dweight


def rmsnorm_router_backward(
    x: torch.Tensor,
    weight: torch.Tensor,
    rstd: torch.Tensor,
    xn: torch.Tensor,
    gate_w: torch.Tensor,
    logits: torch.Tensor,
    idx: torch.Tensor,
    grad_w: Optional[torch.Tensor],
    dxn: Optional[torch.Tensor],
    cnt: Optional[torch.Tensor] = None,
    grad_aux: Optional[torch.Tensor] = None,
    grad_z: Optional[torch.Tensor] = None,
    aux_coef: float = 0.0,
    z_coef: float = 0.0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of :func:`rmsnorm_router_forward` for the router's upstream gradients (as
    :func:`router_backward`) and a gradient ``dxn`` of ``xn`` from the expert path (or None).

    Returns ``(dx [N,H] x.dtype, dweight [H] weight.dtype, dgate_w [H,E] gate_w.dtype)``."""
    dev = L.require_device(x, weight, rstd, xn, gate_w, logits, idx, grad_w, dxn, cnt)
    x = x.contiguous()
    weight = weight.contiguous()
    xn = xn.contiguous()
    gate_w = gate_w.contiguous()
    logits = logits.contiguous()
    idx = idx.contiguous()
    if dxn is not None:
        dxn = dxn.contiguous().to(x.dtype)
    N, H = x.shape
    E = gate_w.shape[1]
    K = idx.shape[1]
    lib = L.load()
    xdt, ndt, wdt = L.dtype_code(x.dtype), L.dtype_code(weight.dtype), L.dtype_code(gate_w.dtype)
    gdt = L.MOE_F32
    if grad_w is not None:
        grad_w = grad_w.contiguous()
        if grad_w.dtype not in (torch.float32, torch.bfloat16):
            grad_w = grad_w.float()
        gdt = L.dtype_code(grad_w.dtype)
    if grad_aux is not None:
        grad_aux = grad_aux.detach().to(torch.float32).reshape(1).contiguous()
    if grad_z is not None:
        grad_z = grad_z.detach().to(torch.float32).reshape(1).contiguous()
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    dgate = torch.empty((H, E), dtype=gate_w.dtype, device=dev)
    nbytes = lib.moe_rmsnorm_router_bwd_workspace(N, H, E, K, xdt, wdt)
    ws = L.workspace(nbytes, dev)
    rc = lib.moe_rmsnorm_router_bwd(
        x.data_ptr(), xdt, weight.data_ptr(), ndt, rstd.data_ptr(), xn.data_ptr(), gate_w.data_ptr(), wdt,
        logits.data_ptr(), idx.data_ptr(), L.ptr(grad_w), gdt, L.ptr(cnt), L.ptr(grad_aux), L.ptr(grad_z),
        float(aux_coef), float(z_coef), L.ptr(dxn), N, H, E, K, dx.data_ptr(), dweight.data_ptr(),
        dgate.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_rmsnorm_router_bwd")
    return dx, dweight, dgate


# ---------------------------------------------------------------------------
# Dispatch planner, permute, combine
# ---------------------------------------------------------------------------
LAYOUT_REFERENCE = 0
LAYOUT_ROUTED = 1


class Plan:
    """Device-side dispatch plan (every field is a tensor on the GPU).

    ``drop`` [N,K] bool or None, ``row_slot`` [N*K] int32, ``slot_row`` [N*K]
    int32, ``offsets`` [E+1] int32, ``ndrop`` [1] int32; ``rows`` = N*K is the
    allocated row count (rows past offsets[E] are not computed).
    """

    __slots__ = ("drop", "row_slot", "slot_row", "offsets", "ndrop", "N", "K", "E", "layout")

    def __init__(self, drop, row_slot, slot_row, offsets, ndrop, N, K, E, layout):
        self.drop, self.row_slot, self.slot_row, self.offsets, self.ndrop = drop, row_slot, slot_row, offsets, ndrop
        self.N, self.K, self.E, self.layout = N, K, E, layout

    @property
    def rows(self) -> int:
        return self.N * self.K

    def drop_u8(self):
        return None if self.drop is None else self.drop.view(torch.uint8)


def cumcount(groups: torch.Tensor) -> torch.Tensor:
    """Each element's 0-based position among the earlier elements of its group, for any int64 group ids
    (moe_cumcount: stable radix sort of the ids, ranks from the sorted positions)."""
    dev = L.require_device(groups)
    g = groups.reshape(-1).contiguous()
    if g.dtype != torch.int64:
        g = g.long()
    n = g.numel()
    out = torch.empty(n, dtype=torch.int64, device=dev)
    if n == 0:
        return out
    lib = L.load()
    nbytes = lib.moe_cumcount_workspace(n)
    ws = L.workspace(nbytes, dev)
    rc = lib.moe_cumcount(g.data_ptr(), n, out.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev))
    L.check(rc, "moe_cumcount")
    return out


def plan(idx: torch.Tensor, num_experts: int, capacity: int = -1, layout: int = LAYOUT_REFERENCE) -> Plan:
    """Build the dispatch plan from the router's top-k indices (no host sync)."""
    dev = L.require_device(idx)
    idx = idx.contiguous()
    if idx.dtype != torch.int64:
        idx = idx.long()
    N, K = idx.shape
    E = int(num_experts)
    lib = L.load()
    drop = torch.empty((N, K), dtype=torch.bool, device=dev) if capacity >= 0 else None
    M = N * K
    row_slot = torch.empty((max(M, 1),), dtype=torch.int32, device=dev)
    slot_row = torch.empty((max(M, 1),), dtype=torch.int32, device=dev)
    offsets = torch.empty((E + 1,), dtype=torch.int32, device=dev)
    ndrop = torch.zeros((1,), dtype=torch.int32, device=dev) if M == 0 else torch.empty((1,), dtype=torch.int32,
                                                                                         device=dev)
    nbytes = lib.moe_plan_workspace(N, K, E)
    ws = L.workspace(nbytes, dev)
    rc = lib.moe_plan(
        idx.data_ptr(), N, K, E, int(capacity), int(layout),
        L.ptr(drop), row_slot.data_ptr(), slot_row.data_ptr(), offsets.data_ptr(), ndrop.data_ptr(),
        ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_plan")
    return Plan(drop, row_slot[:M], slot_row[:M], offsets, ndrop, N, K, E, layout)


def permute(x: torch.Tensor, p: Plan) -> torch.Tensor:
    """xp [N*K, H]: row slot_row[t*K+k] holds x[t] (one read of each token row; rows past offsets[E] are left
    unwritten)."""
    dev = L.require_device(x)
    x = x.contiguous()
    H = x.shape[1]
    xp = torch.empty((p.rows, H), dtype=x.dtype, device=dev)
    if p.rows == 0:
        return xp
    rc = L.load().moe_permute(x.data_ptr(), H * x.element_size(), p.slot_row.data_ptr(), p.offsets.data_ptr(),
                              p.N, p.K, p.E, xp.data_ptr(), L.stream_of(dev))
    L.check(rc, "moe_permute")
    return xp


def combine(y: torch.Tensor, w: torch.Tensor, p: Plan) -> torch.Tensor:
    dev = L.require_device(y, w)
    y = y.contiguous()
    w = w.contiguous()
    H = y.shape[1]
    out = torch.empty((p.N, H), dtype=y.dtype, device=dev)
    rc = L.load().moe_combine(y.data_ptr(), L.dtype_code(y.dtype), w.data_ptr(), L.dtype_code(w.dtype),
                              L.ptr(p.drop_u8()), p.slot_row.data_ptr(), p.offsets.data_ptr(), p.N, p.K, H, p.E,
                              out.data_ptr(), L.stream_of(dev))
    L.check(rc, "moe_combine")
    return out


def combine_backward(dout: torch.Tensor, y: torch.Tensor, w: torch.Tensor, p: Plan, need_dw: bool = True,
                     zero_tail: bool = False):
    """Returns (dy [rows, H], dw [N, K] or None).  Rows past offsets[E] of dy are
    left unwritten unless ``zero_tail`` (then the whole buffer starts at zero)."""
    dev = L.require_device(dout, y, w)
    dout = dout.contiguous()
    H = y.shape[1]
    dy = torch.zeros_like(y) if zero_tail else torch.empty_like(y)
    dw = torch.empty((p.N, p.K), dtype=w.dtype, device=dev) if need_dw else None
    rc = L.load().moe_combine_bwd(dout.data_ptr(), y.data_ptr(), L.dtype_code(y.dtype), w.contiguous().data_ptr(),
                                  L.dtype_code(w.dtype), L.ptr(p.drop_u8()), p.slot_row.data_ptr(),
                                  p.offsets.data_ptr(), p.N, p.K, H, p.E, dy.data_ptr(), L.ptr(dw),
                                  L.stream_of(dev))
    L.check(rc, "moe_combine_bwd")
    return dy, dw


def unpermute_sum(dxp: torch.Tensor, p: Plan, addend: Optional[torch.Tensor] = None) -> torch.Tensor:
    dev = L.require_device(dxp, addend)
    H = dxp.shape[1]
    dx = torch.empty((p.N, H), dtype=dxp.dtype, device=dev)
    if addend is not None:
        addend = addend.contiguous()
    rc = L.load().moe_unpermute_sum(dxp.contiguous().data_ptr(), L.ptr(addend), L.dtype_code(dxp.dtype),
                                    p.slot_row.data_ptr(), p.offsets.data_ptr(), p.N, p.K, H, p.E, dx.data_ptr(),
                                    L.stream_of(dev))
    L.check(rc, "moe_unpermute_sum")
    return dx


# ---------------------------------------------------------------------------
# SwiGLU grouped GEMM (bf16)
# ---------------------------------------------------------------------------
def swiglu_forward(xp: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                   offsets: torch.Tensor, keep_preact: bool = True):
    """xp [R,H]; w_gate/w_up [E,F,H]; w_down [E,H,F] (all bf16 or all fp32, contiguous) -> (act [R,F], hgu [R,2F],
    y [R,H]).  ``keep_preact=False`` (no backward follows) skips storing the pre-activations: hgu is None."""
    dev = L.require_device(xp, w_gate, w_up, w_down, offsets)
    f32 = _gemm_dtype_is_f32("swiglu_forward", xp, w_gate, w_up, w_down)
    R, H = xp.shape
    E, F, _ = w_gate.shape
    act = torch.empty((R, F), dtype=xp.dtype, device=dev)
    hgu = torch.empty((R, 2 * F), dtype=xp.dtype, device=dev) if keep_preact else None
    y = torch.empty((R, H), dtype=xp.dtype, device=dev)
    lib = L.load()
    nbytes = lib.moe_swiglu_f32_workspace(E) if f32 else lib.moe_swiglu_workspace(E)
    ws = L.workspace(nbytes, dev)
    fn = lib.moe_swiglu_fwd_f32 if f32 else lib.moe_swiglu_fwd
    rc = fn(xp.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), w_down.data_ptr(), offsets.data_ptr(), R, H, F, E,
            act.data_ptr(), L.ptr(hgu), y.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev))
    L.check(rc, "moe_swiglu_fwd_f32" if f32 else "moe_swiglu_fwd")
    return act, hgu, y


def _gemm_dtype_is_f32(what, *ts) -> bool:
    """The grouped GEMM runs on all-bf16 (moe_swiglu_*) or all-fp32 (moe_swiglu_*_f32) contiguous tensors."""
    dt = ts[0].dtype
    if dt not in (torch.bfloat16, torch.float32) or any(t.dtype != dt for t in ts):
        raise TypeError(f"{what}: the grouped GEMM runs on all-bfloat16 or all-float32 tensors")
    if not all(t.is_contiguous() for t in ts):
        raise ValueError(f"{what}: tensors must be contiguous")
    return dt == torch.float32


# ---------------------------------------------------------------------------
# fp8 (e4m3) forward of the expert FFN
# ---------------------------------------------------------------------------
def quant_rows_fp8(t: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rows of ``t`` [..., cols] (bf16 / fp32) -> (e4m3 bytes uint8 [..., cols], fp32 scale [...]): scale =
    absmax(row) / 448 (1 for a zero row), element = x * (448 / absmax) rounded to nearest even."""
    dev = L.require_device(t)
    t = t.contiguous()
    cols = t.shape[-1]
    rows = t.numel() // cols if cols else 0
    q = torch.empty(t.shape, dtype=torch.uint8, device=dev)
    sc = torch.empty(t.shape[:-1], dtype=torch.float32, device=dev)
    if rows == 0:
        return q, sc
    rc = L.load().moe_quant_rows_fp8(t.data_ptr(), L.dtype_code(t.dtype), rows, cols, cols, q.data_ptr(),
                                     sc.data_ptr(), L.stream_of(dev))
    L.check(rc, "moe_quant_rows_fp8")
    return q, sc


def permute_fp8(x: torch.Tensor, p: Plan) -> Tuple[torch.Tensor, torch.Tensor]:
    """The quantized dispatch payload: (xq [N*K, H] uint8 e4m3, sx [N*K] f32); row r is x[row_slot[r] // K]
    quantized (rows past offsets[E] are left unwritten)."""
    dev = L.require_device(x)
    x = x.contiguous()
    H = x.shape[1]
    xq = torch.empty((p.rows, H), dtype=torch.uint8, device=dev)
    sx = torch.empty((p.rows,), dtype=torch.float32, device=dev)
    if p.rows == 0:
        return xq, sx
    rc = L.load().moe_permute_fp8(x.data_ptr(), L.dtype_code(x.dtype), p.slot_row.data_ptr(), p.offsets.data_ptr(),
                                  p.N, p.K, p.E, H, xq.data_ptr(), sx.data_ptr(), L.stream_of(dev))
    L.check(rc, "moe_permute_fp8")
    return xq, sx


def swiglu_forward_fp8(xq, sx, wq, wscale, offsets, out_dtype=torch.bfloat16, keep_preact: bool = True,
                       return_mx: bool = False):
    """fp8 forward of the SwiGLU experts: ``xq`` [R,H] uint8 e4m3 with row scales ``sx`` [R]; ``wq`` =
    (gate [E,F,H], up [E,F,H], down [E,H,F]) e4m3 bytes with ``wscale`` = (sg [E,F], su [E,F], sd [E,H])
    -> (act [R,F], hgu [R,2F], y [R,H]) bf16, as :func:`swiglu_forward`; with keep_preact=False (inference)
    act and hgu are None (the down projection reads act block-quantized from the gate/up epilogue).
    ``return_mx``: also return (act e4m3 bytes [R, F], E8M0 block scales [R, F/32]) as the kernels wrote them:
    views of the call's workspace, valid until the next call that takes the same workspace (clone to keep them)."""
    wg, wu, wd = wq
    sg, su, sd = wscale
    dev = L.require_device(xq, sx, wg, wu, wd, sg, su, sd, offsets)
    for t in (xq, wg, wu, wd):
        if t.dtype != torch.uint8 or not t.is_contiguous():
            raise TypeError("swiglu_forward_fp8: quantized operands are contiguous uint8 (e4m3 bytes)")
    if out_dtype != torch.bfloat16:
        raise TypeError("swiglu_forward_fp8: outputs are bfloat16")
    R, H = xq.shape
    E, F, _ = wg.shape
    act = torch.empty((R, F), dtype=out_dtype, device=dev) if keep_preact else None
    hgu = torch.empty((R, 2 * F), dtype=out_dtype, device=dev) if keep_preact else None
    y = torch.empty((R, H), dtype=out_dtype, device=dev)
    lib = L.load()
    nbytes = lib.moe_swiglu_fwd_fp8_workspace(R, F, E)
    ws = L.workspace(nbytes, dev)
    rc = lib.moe_swiglu_fwd_fp8(
        xq.data_ptr(), sx.contiguous().data_ptr(), wg.data_ptr(), sg.contiguous().data_ptr(), wu.data_ptr(),
        su.contiguous().data_ptr(), wd.data_ptr(), sd.contiguous().data_ptr(), offsets.data_ptr(), R, H, F, E,
        L.ptr(act), L.ptr(hgu), y.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_swiglu_fwd_fp8")
    if not return_mx:
        return act, hgu, y
    # the workspace: tile tables (moe_swiglu_workspace(E) bytes), act in e4m3 [R, F] (256-byte aligned), then
    # the block scales [F/128 slices][R rounded up to 4][4 blocks]
    off_a = lib.moe_swiglu_workspace(E)
    off_s = off_a + (R * F + 255) // 256 * 256
    srows = (R + 3) // 4 * 4
    nsl = (F + 127) // 128
    aq = ws[off_a:off_a + R * F].view(R, F)
    sc = ws[off_s:off_s + nsl * srows * 4].view(nsl, srows, 4)[:, :R].permute(1, 0, 2).reshape(R, nsl * 4)
    return act, hgu, y, (aq, sc[:, : F // 32])


def swiglu_backward(dy, xp, act, hgu, w_gate, w_up, w_down, offsets):
    """-> (dxp [R,H], dw_gate [E,F,H], dw_up [E,F,H], dw_down [E,H,F])."""
    dev = L.require_device(dy, xp, act, hgu, w_gate, w_up, w_down, offsets)
    dy = dy.contiguous()
    f32 = _gemm_dtype_is_f32("swiglu_backward", dy, xp, act, hgu, w_gate, w_up, w_down)
    R, H = xp.shape
    E, F, _ = w_gate.shape
    dh = torch.empty((R, 2 * F), dtype=xp.dtype, device=dev)
    dxp = torch.empty((R, H), dtype=xp.dtype, device=dev)
    dwg = torch.empty_like(w_gate)
    dwu = torch.empty_like(w_up)
    dwd = torch.empty_like(w_down)
    lib = L.load()
    nbytes = lib.moe_swiglu_f32_workspace(E) if f32 else lib.moe_swiglu_workspace(E)
    ws = L.workspace(nbytes, dev)
    fn = lib.moe_swiglu_bwd_f32 if f32 else lib.moe_swiglu_bwd
    rc = fn(dy.data_ptr(), xp.data_ptr(), act.data_ptr(), hgu.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(),
            w_down.data_ptr(), offsets.data_ptr(), R, H, F, E, dh.data_ptr(), dxp.data_ptr(), dwg.data_ptr(),
            dwu.data_ptr(), dwd.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev))
    L.check(rc, "moe_swiglu_bwd_f32" if f32 else "moe_swiglu_bwd")
    return dxp, dwg, dwu, dwd
