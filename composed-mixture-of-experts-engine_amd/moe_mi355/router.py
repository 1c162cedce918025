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

from . import _lib as L

STAT_Z = 0
STAT_AUX = 1
STAT_IMBALANCE = 2
STAT_CNT_MEAN = 3
STAT_CNT_STD = 4
STAT_CNT_TOTAL = 5
STAT_NONFINITE = 6
STAT_DEAD = 7


_native = None


def _binding():
    """The native autograd binding (moe_mi355/_moe_torch.so, built with libmoe_mi355.so)."""
    global _native
    if _native is None:
        try:
            from . import _moe_torch
        except ImportError as e:
            raise RuntimeError(
                "moe_mi355/_moe_torch.so is not built or does not load; run __graft_entry__.build() "
                f"(or python moe_mi355/build.py) on a host with ROCm/hipcc ({e})"
            ) from e
        _native = _moe_torch
    return _native


class RouterCore:
    """(x [N,H], gate_w [H,E], k, aux_coef, z_coef, bias|None) ->
    (idx, w, aux, z, logits, cnt, stats).

    ``apply`` runs a torch C++ autograd Function (csrc/torch_router.cpp): the forward launches moe_router_fwd
    and saves (x, gate_w, logits, idx, cnt); the backward, run by the autograd engine without a return to
    Python, launches moe_router_bwd with the upstream gradients of w, aux and z (an aux or z output that gets
    no gradient contributes no term).  idx, logits, cnt and stats are not differentiable; no gradient flows
    to k, the coefficients or the bias.  The checks below raise the errors the ctypes path raises."""

    @staticmethod
    def apply(x, gate_w, k: int, aux_coef: float, z_coef: float, bias: Optional[torch.Tensor] = None,
              link_x: bool = False):
        """``link_x``: also return x itself as an eighth output.  A caller that feeds that output (rather than
        x) to its other consumer of the tokens hands that consumer's gradient of x to this Function's backward,
        which adds it inside the dx kernel (moe_router_bwd_acc) instead of autograd summing the two
        contributions to x's gradient in a separate addition."""
        L.require_device(x, gate_w, bias)
        N, H = x.shape
        H2, E = gate_w.shape
        if H != H2:
            raise ValueError(f"router_forward: hidden dims differ ({H} vs {H2})")
        L.dtype_code(x.dtype)
        L.dtype_code(gate_w.dtype)
        return tuple(_binding().router_core(x, gate_w, int(k), float(aux_coef), float(z_coef), bias, bool(link_x)))


def route(x: torch.Tensor, gate_w: torch.Tensor, k: int, aux_coef: float = 0.0, z_coef: float = 0.0,
          bias: Optional[torch.Tensor] = None):
    """Functional form of :class:`RouterCore`."""
    return RouterCore.apply(x, gate_w, k, aux_coef, z_coef, bias)
