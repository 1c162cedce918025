"""Autograd Functions of the MoE layer's expert path.

``ExpertsFn``   permute -> SwiGLU grouped GEMM (gate|up, down) -> weighted
                combine, and the fused backward: combine-bwd (dy, dw) ->
                grouped GEMM backward (dh, dxp, dW) -> permute-bwd (dx).  bf16.
``PermuteFn`` / ``CombineFn``  the dispatch and combine alone, for expert
                modules that are not the built-in SwiGLU (per-expert calls in
                between) and for dtypes the grouped GEMM does not take.
"""

from __future__ import annotations

import torch

from . import ops


class ExpertsFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, w_gate, w_up, w_down, p: ops.Plan, keep_preact: bool = True, timer=None):
        xp = ops.permute(x, p)
        # timer (optional): an object with start() / stop(), bracketing the expert GEMMs on the stream
        if timer is not None:
            timer.start()
        # keep_preact=False (the caller knows no backward follows) skips storing the pre-activations
        act, hgu, y = ops.swiglu_forward(xp, w_gate, w_up, w_down, p.offsets, keep_preact=keep_preact)
        if timer is not None:
            timer.stop()
        out = ops.combine(y, w, p)
        ctx.save_for_backward(w, w_gate, w_up, w_down, xp, act, hgu, y)
        ctx.p = p
        return out

    @staticmethod
    def backward(ctx, dout):
        w, w_gate, w_up, w_down, xp, act, hgu, y = ctx.saved_tensors
        p = ctx.p
        dy, dw = ops.combine_backward(dout, y, w, p, need_dw=ctx.needs_input_grad[1])
        dxp, dwg, dwu, dwd = ops.swiglu_backward(dy, xp, act, hgu, w_gate, w_up, w_down, p.offsets)
        dx = ops.unpermute_sum(dxp, p) if ctx.needs_input_grad[0] else None
        return dx, dw, dwg, dwu, dwd, None, None, None


class PermuteFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, p: ops.Plan):
        ctx.p = p
        return ops.permute(x, p)

    @staticmethod
    def backward(ctx, dxp):
        return ops.unpermute_sum(dxp, ctx.p), None


class CombineFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, w, p: ops.Plan):
        ctx.save_for_backward(y, w)
        ctx.p = p
        return ops.combine(y, w, p)

    @staticmethod
    def backward(ctx, dout):
        y, w = ctx.saved_tensors
        dy, dw = ops.combine_backward(dout, y, w, ctx.p, need_dw=ctx.needs_input_grad[1], zero_tail=True)
        return dy, dw, None
