"""Autograd Functions of the RMSNorm in front of the router.

``RMSNormFn``       xn = ((x * rsqrt(mean(x^2) + eps)) * weight).to(x.dtype) and its backward
                    (moe-engine/pkg/models/moe.py L:83-86, the norm of ToyMoEBlock L:125-126).
``NormRouterCore``  the norm with the router forward fused onto its output: one read of the hidden state
                    for both (bf16 x and gate, E <= 16), returning ``xn`` for the expert path together with
                    everything :class:`moe_mi355.router.RouterCore` returns.  Its backward is one call
                    (ops.rmsnorm_router_backward): the router's weight gradient over ``xn`` and dL/dlogits,
                    then the norm backward, which forms the router's gradient of ``xn`` from dL/dlogits and
                    the gate inside the kernel and adds the expert path's (no [N, H] gradient in between).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops


class RMSNormFn(torch.autograd.Function):
    """(x [N,H], weight [H], eps) -> xn [N,H]."""

    @staticmethod
    def forward(ctx, x, weight, eps: float):
        xn, rstd = ops.rmsnorm_forward(x, weight, eps)
        ctx.save_for_backward(x, weight, rstd)
        return xn

    @staticmethod
    def backward(ctx, dxn):
        x, weight, rstd = ctx.saved_tensors
        dx, dweight = ops.rmsnorm_backward(x, weight, rstd, dxn)
        return (dx if ctx.needs_input_grad[0] else None), (dweight if ctx.needs_input_grad[1] else None), None


class NormRouterCore(torch.autograd.Function):
    """(x [N,H], norm_weight [H], eps, gate_w [H,E], k, aux_coef, z_coef, bias|None) ->
    (xn, idx, w, aux, z, logits, cnt, stats)."""

    @staticmethod
    def forward(ctx, x, norm_weight, eps: float, gate_w, k: int, aux_coef: float, z_coef: float,
                bias: Optional[torch.Tensor] = None):
        xn, rstd, idx, w, logits, _lse, cnt, stats, aux, z = ops.rmsnorm_router_forward(
            x, norm_weight, eps, gate_w, k, bias, aux_coef=aux_coef, z_coef=z_coef
        )
        ctx.save_for_backward(x, norm_weight, rstd, xn, gate_w, logits, idx, cnt)
        ctx.aux_coef = float(aux_coef)
        ctx.z_coef = float(z_coef)
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(idx, logits, cnt, stats)
        return xn, idx, w, aux, z, logits, cnt, stats

    @staticmethod
    def backward(ctx, g_xn, g_idx, g_w, g_aux, g_z, g_logits, g_cnt, g_stats):
        x, norm_weight, rstd, xn, gate_w, logits, idx, cnt = ctx.saved_tensors
        need_x, need_nw, need_gw = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[3]
        dx = dnw = dgate = None
        if g_w is not None or g_aux is not None or g_z is not None:
            # the router backward and the norm backward in one call: the router's gradient of xn is formed
            # inside the norm kernel
            aux_coef = ctx.aux_coef if g_aux is not None else 0.0
            z_coef = ctx.z_coef if g_z is not None else 0.0
            dx, dnw, dgate = ops.rmsnorm_router_backward(x, norm_weight, rstd, xn, gate_w, logits, idx, g_w, g_xn,
                                                         cnt, g_aux, g_z, aux_coef, z_coef)
        elif need_x or need_nw:
            if g_xn is None:
                dx, dnw = torch.zeros_like(x), torch.zeros_like(norm_weight)
            else:
                dx, dnw = ops.rmsnorm_backward(x, norm_weight, rstd, g_xn)
        if need_gw and dgate is None:
            dgate = torch.zeros_like(gate_w)
        return (dx if need_x else None), (dnw if need_nw else None), None, (dgate if need_gw else None), \
            None, None, None, None
