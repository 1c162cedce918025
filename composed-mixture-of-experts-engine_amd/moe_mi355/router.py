"""Autograd Function over the fused HIP router.

``RouterCore`` is the differentiable router used by the modules: it returns
the top-k indices and weights together with the load-balance aux loss and
the z-loss as differentiable 0-d tensors, the fp32 logits the kernel
produced, the dispatch counts and the statistics vector -- all from one
kernel launch sequence, with no host synchronisation.

The aux / z losses have no counterpart in the reference (its z-loss is a
detached Python float, moe-engine/pkg/kernels/moe_router.py L:603-612); their
closed forms are

    aux = aux_coef * E * sum_e f_e P_e,  f_e = cnt_e / (N K),  P_e = mean_t p[t, e]
    z   = z_coef * mean_t lse_t^2

and their gradients are added to dL/dlogits inside the backward kernel.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops

STAT_Z = 0
STAT_AUX = 1
STAT_IMBALANCE = 2
STAT_CNT_MEAN = 3
STAT_CNT_STD = 4
STAT_CNT_TOTAL = 5
STAT_NONFINITE = 6
STAT_DEAD = 7


class RouterCore(torch.autograd.Function):
    """(x [N,H], gate_w [H,E], k, aux_coef, z_coef, bias|None) ->
    (idx, w, aux, z, logits, cnt, stats)."""

    @staticmethod
    def forward(ctx, x, gate_w, k: int, aux_coef: float, z_coef: float, bias: Optional[torch.Tensor] = None):
        idx, w, logits, lse, cnt, stats, aux, z = ops.router_forward(
            x, gate_w, k, bias, aux_coef=aux_coef, z_coef=z_coef, with_losses=True
        )
        ctx.save_for_backward(x, gate_w, logits, idx, cnt)
        ctx.aux_coef = float(aux_coef)
        ctx.z_coef = float(z_coef)
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(idx, logits, cnt, stats)
        return idx, w, aux, z, logits, cnt, stats

    @staticmethod
    def backward(ctx, g_idx, g_w, g_aux, g_z, g_logits, g_cnt, g_stats):
        x, gate_w, logits, idx, cnt = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_x or need_w):
            return None, None, None, None, None, None
        aux_coef = ctx.aux_coef if g_aux is not None else 0.0
        z_coef = ctx.z_coef if g_z is not None else 0.0
        dx, dw = ops.router_backward(x, gate_w, logits, idx, g_w, cnt, g_aux, g_z, aux_coef, z_coef)
        return (dx if need_x else None), (dw if need_w else None), None, None, None, None


def route(x: torch.Tensor, gate_w: torch.Tensor, k: int, aux_coef: float = 0.0, z_coef: float = 0.0,
          bias: Optional[torch.Tensor] = None):
    """Functional form of :class:`RouterCore`."""
    return RouterCore.apply(x, gate_w, k, aux_coef, z_coef, bias)
