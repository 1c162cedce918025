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
    ws = L.workspace(nbytes, dev)
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
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused router backward: returns ``(dx [N,H] x.dtype, dgate_w [H,E] gate_w.dtype)``."""
    dev = L.require_device(x, gate_w, logits, idx, grad_w, cnt)
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
    rc = lib.moe_router_bwd(
        x.data_ptr(), xdt, gate_w.data_ptr(), wdt, logits.data_ptr(), idx.data_ptr(),
        L.ptr(grad_w), gdt, L.ptr(cnt), L.ptr(grad_aux), L.ptr(grad_z),
        float(aux_coef), float(z_coef), N, H, E, K,
        dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), nbytes, L.stream_of(dev),
    )
    L.check(rc, "moe_router_bwd")
    return dx, dw
