"""Top-k MoE router with the reference's API, running on the gfx950 HIP kernels.

Mirrors ``moe-engine/pkg/kernels/moe_router.py``:

* ``RouterProfile``            -- same 8 fields (L:84-94).
* ``MoERouterFunction``        -- ``apply(tokens[N,H], gate_w[H,E], k,
  force_reference=False, report=None) -> (idx, w)``, backward returns 5
  gradients (L:456-553).  ``MoERouterAutograd`` is an alias (L:556).
* ``moe_topk_route``           -- functional entry point (L:562-588).
* ``MoERouter``                -- ``nn.Module`` (L:618-746): same constructor,
  ``forward(tokens, force_reference=False) -> (idx, w, dispatch_cnt)``,
  ``gate_w`` [H, E] parameter, ``bias``, ``last_profile``, ``_last_logits``.
* ``_compute_load_imbalance`` / ``_compute_router_z_loss`` (L:594-612).

Differences from the reference, all deliberate:

* Every compute step runs on the fused HIP kernels (``moe_mi355``); there is
  no Triton and no fp64 PyTorch path in the product.  CPU tensors raise
  ``RuntimeError``; ``force_reference=True`` raises ``NotImplementedError``
  (the fp64 restatement of the reference path is test infrastructure under
  ``oracle/``).  ``RouterProfile.used_triton`` keeps its name and is True
  when the native kernel ran.
* ``MoERouter.forward`` reads every statistic it reports (conservation check,
  NaN check, z-loss, imbalance, count mean/std) from one device buffer with
  one device-to-host copy, instead of ~8 ``.item()`` calls and a second fp32
  logits GEMM (L:690-745).  ``sync_profile=False`` skips even that copy.
* New, opt-in: ``aux_loss_coef`` / ``z_loss_coef`` constructor arguments; the
  differentiable load-balance loss and z-loss of the last forward are kept in
  ``last_aux_loss`` / ``last_z_loss`` (0-d tensors).  With both coefficients
  at 0 (the default) behaviour matches the reference.
* Exact ties in the gate probabilities go to the lower expert index.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from moe_mi355 import _lib, ops
from moe_mi355.router import STAT_CNT_MEAN, STAT_CNT_STD, STAT_CNT_TOTAL, STAT_IMBALANCE, STAT_NONFINITE, STAT_Z
from moe_mi355.norm import NormRouterCore
from moe_mi355.router import RouterCore

# Kept for import compatibility: True when the native gfx950 library is built
# (the reference sets it when Triton imports, L:70-78).
TRITON_AVAILABLE = __import__("os").path.exists(_lib.LIB_PATH)


def _fwd_lds_bytes(tokens: torch.Tensor, gate_w: torch.Tensor) -> int:
    """LDS bytes per workgroup of the forward kernel this call launches (reported as sram_bytes_per_block,
    the reference's sram_bytes, L:380)."""
    N, H = tokens.shape
    E = gate_w.shape[1]
    return int(_lib.load().moe_router_fwd_lds_bytes(N, H, E, _lib.dtype_code(tokens.dtype),
                                                     _lib.dtype_code(gate_w.dtype)))


@dataclass
class RouterProfile:
    sram_bytes_per_block: int
    achieved_bandwidth_gbps: float
    kernel_ms: float
    used_triton: bool
    tokens_per_expert_mean: float
    tokens_per_expert_std: float
    expert_load_imbalance: float
    router_z_loss: float


def router_fwd_bytes(tokens: torch.Tensor, gate_w: torch.Tensor, k: int, w_dtype: torch.dtype) -> int:
    """Bytes the router forward moves to and from HBM, each tensor once: tokens and gate read; logits and
    logsumexp (fp32), top-k indices (int64) and weights, dispatch counts (int64) and the statistics vector
    written.  The rate the profile reports is this over the launch's duration (the reference's figure counts
    the same tensors at its own widths, L:371-379)."""
    N, H = tokens.shape
    E = gate_w.shape[1]
    wsz = torch.empty((), dtype=w_dtype).element_size()
    return (N * H * tokens.element_size() + H * E * gate_w.element_size() + N * E * 4 + N * 4
            + N * k * (8 + wsz) + E * 8 + (_lib.STATS_HEAD + E) * 4)


def _gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9 if ms > 0.0 else 0.0


class _LaunchTiming:
    """Two timing events recorded on the current stream around a launch sequence; the elapsed time is read
    only when asked for (it then waits for the second event).  Not recorded under graph capture."""

    __slots__ = ("a", "b")

    def __init__(self, a, b):
        self.a, self.b = a, b

    @classmethod
    def start(cls, like: torch.Tensor) -> Optional["_LaunchTiming"]:
        if not like.is_cuda or torch.cuda.is_current_stream_capturing():
            return None
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        return cls(a, b)

    def stop(self) -> None:
        self.b.record()

    def elapsed_ms(self) -> float:
        self.b.synchronize()
        return max(float(self.a.elapsed_time(self.b)), 0.0)


def _reference_route_fp64(tokens: torch.Tensor, gate_w: torch.Tensor, k: int):
    """The reference's float64 PyTorch router (L:257-271).  Not shipped with this build: every routing call
    runs the gfx950 kernels, and the float64 restatement used to check them is test infrastructure (oracle/).
    Kept so that ``from pkg.kernels.moe_router import _reference_route_fp64`` resolves; calling it raises."""
    raise NotImplementedError(
        "_reference_route_fp64: the float64 reference router is not part of this build; compare "
        "MoERouterFunction's output with a float64 computation in the test instead"
    )


def _no_reference_path():
    raise NotImplementedError(
        "force_reference=True selects the reference's fp64 PyTorch router, which this build does not "
        "ship; every call runs the gfx950 kernels (the fp64 restatement is test infrastructure in oracle/)"
    )


class MoERouterFunction(torch.autograd.Function):
    """``apply(tokens, gate_w, k, force_reference=False, report=None) -> (idx, w)``."""

    @staticmethod
    def forward(ctx, tokens, gate_w, k, force_reference=False, report=None):
        assert tokens.dim() == 2
        assert gate_w.dim() == 2
        N, H = tokens.shape
        H2, E = gate_w.shape
        assert H == H2
        assert 1 <= k <= E
        if force_reference:
            _no_reference_path()
        timing = _LaunchTiming.start(tokens) if report is not None else None
        idx, w, logits, _lse, _cnt, _stats = ops.router_forward(tokens, gate_w, k)
        if timing is not None:
            timing.stop()
        ctx.save_for_backward(tokens, gate_w, logits, idx)
        ctx.k = k
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(idx)
        if report is not None:
            # The kernels' duration is read back only for a caller that asks for the report (the reference
            # synchronises on its timing event in every forward, L:342): one event pair on the launch stream.
            report["used_triton"] = True
            report["sram_bytes"] = _fwd_lds_bytes(tokens, gate_w)
            report["kernel_ms"] = timing.elapsed_ms() if timing is not None else 0.0
            report["achieved_bw"] = _gbps(router_fwd_bytes(tokens, gate_w, k, w.dtype), report["kernel_ms"])
        return idx, w

    @staticmethod
    def backward(ctx, grad_idx, grad_w):
        tokens, gate_w, logits, idx = ctx.saved_tensors
        if grad_w is None or not (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]):
            return None, None, None, None, None
        dx, dw = ops.router_backward(tokens, gate_w, logits, idx, grad_w)
        return dx, dw, None, None, None


MoERouterAutograd = MoERouterFunction


def moe_topk_route(
    tokens: torch.Tensor,
    gate_w: torch.Tensor,
    k: int,
    force_reference: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Differentiable top-k routing: ``tokens`` [B,S,H] or [N,H] -> (idx [N,K], w [N,K])."""
    if tokens.dim() == 3:
        B, S, H = tokens.shape
        flat = tokens.reshape(B * S, H)
    elif tokens.dim() == 2:
        flat = tokens
    else:
        raise ValueError(f"tokens must be rank 2 or 3, got {tokens.dim()}")
    return MoERouterFunction.apply(flat, gate_w, k, force_reference)


def _compute_load_imbalance(dispatch_cnt: torch.Tensor) -> float:
    """max_load / mean_load; 1.0 when the mean is ~0 (reference L:594-600)."""
    cnt = dispatch_cnt.float()
    mean = cnt.mean().item()
    if mean < 1e-9:
        return 1.0
    return float(cnt.max().item()) / mean


def _compute_router_z_loss(logits: torch.Tensor) -> float:
    """mean_t(logsumexp(logits_t)^2) (reference L:603-612)."""
    lse = torch.logsumexp(logits.float(), dim=-1)
    return float((lse**2).mean().item())


class MoERouter(torch.nn.Module):
    """Top-k router module; the gate ``gate_w`` [H, E] is a learnable parameter.

    ``last_profile`` is built from the forward's statistics vector and the duration of its kernels (two
    timing events on the launch stream).  With ``sync_profile=True`` (the default) the forward reads both
    back at once -- the one device-to-host copy that also feeds the reference's conservation and NaN checks;
    with ``sync_profile=False`` the forward does not synchronise and ``last_profile`` is resolved when it is
    first read."""

    def __init__(
        self,
        hidden_dim: int,
        num_experts: int,
        top_k: int = 2,
        bias: bool = False,
        dtype: torch.dtype = torch.float32,
        aux_loss_coef: float = 0.0,
        z_loss_coef: float = 0.0,
        sync_profile: bool = True,
    ):
        super().__init__()
        if top_k < 1 or top_k > num_experts:
            raise ValueError("top_k must be in [1, num_experts]")
        self.hidden_dim = hidden_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.gate_w = torch.nn.Parameter(torch.empty(hidden_dim, num_experts, dtype=dtype))
        torch.nn.init.normal_(self.gate_w, mean=0.0, std=1.0 / math.sqrt(hidden_dim))
        self.bias = torch.nn.Parameter(torch.zeros(num_experts, dtype=dtype)) if bias else None
        self.aux_loss_coef = float(aux_loss_coef)
        self.z_loss_coef = float(z_loss_coef)
        self.sync_profile = sync_profile
        self._profile: Optional[RouterProfile] = None
        self._pending = None  # what a not-yet-read profile is built from
        # set by a caller that enqueues more GPU work after the routing and runs the checks itself at its next
        # synchronisation (check_pending): the forward then does not stop the stream mid-way
        self._defer_check = False
        # set by DistributedMoELayer around its call: the forward also returns the tokens as a linked output
        # (take_linked_tokens) whose gradient the router's backward adds into its own gradient of the tokens
        self._link_x = False
        self._x_link: Optional[torch.Tensor] = None
        self._last_logits: Optional[torch.Tensor] = None
        self.last_aux_loss: Optional[torch.Tensor] = None
        self.last_z_loss: Optional[torch.Tensor] = None
        self.last_stats: Optional[torch.Tensor] = None
        self.last_stats_host: Optional[torch.Tensor] = None
        self.last_num_tokens = 0
        # Fixed (non-learnable) additive logit bias [E] f32, e.g. a load-skew
        # harness; unlike ``bias`` it keeps w differentiable.  None = off.
        self.register_buffer("logit_bias", None)

    @property
    def last_profile(self) -> Optional[RouterProfile]:
        if self._pending is not None:
            self._resolve()
        return self._profile

    @last_profile.setter
    def last_profile(self, value: Optional[RouterProfile]) -> None:
        self._pending = None
        self._profile = value

    def forward(self, tokens: torch.Tensor, force_reference: bool = False):
        """Returns ``(topk_idx [N,K] int64, topk_w [N,K] tokens.dtype, dispatch_cnt [E] int64)``."""
        if tokens.dim() == 3:
            B, S, H = tokens.shape
            flat = tokens.reshape(B * S, H)
        else:
            flat = tokens
        N = flat.shape[0]
        H = flat.shape[1]
        assert H == self.hidden_dim
        if force_reference:
            _no_reference_path()

        timing = _LaunchTiming.start(flat)
        outs = RouterCore.apply(
            flat, self.gate_w, self.top_k, self.aux_loss_coef, self.z_loss_coef, self._logit_bias(),
            link_x=self._link_x,
        )
        idx, w, aux, z, logits, cnt, stats = outs[:7]
        # with _link_x (set by DistributedMoELayer around its call) the tokens come back as an eighth output for
        # the expert path, so its gradient of the tokens is summed inside the router's dx kernel
        self._x_link = outs[7] if self._link_x else None
        if timing is not None:
            timing.stop()
        return self._finish(flat, idx, w, aux, z, logits, cnt, stats, timing)

    def take_linked_tokens(self) -> Optional[torch.Tensor]:
        """The tokens of the last forward made with ``_link_x`` set, as the router's linked output (once)."""
        x, self._x_link = self._x_link, None
        return x

    def forward_with_norm(self, tokens: torch.Tensor, norm_weight: torch.Tensor, eps: float):
        """Route ``rmsnorm(tokens)`` with the norm fused into the router's read of ``tokens``
        (moe-engine/pkg/models/moe.py L:83-86, L:125-126).  Returns ``(xn, topk_idx, topk_w, dispatch_cnt)``:
        ``xn`` is the normalised input the routing used, for the expert path."""
        flat = tokens.reshape(-1, tokens.shape[-1])
        assert flat.shape[1] == self.hidden_dim
        timing = _LaunchTiming.start(flat)
        xn, idx, w, aux, z, logits, cnt, stats = NormRouterCore.apply(
            flat, norm_weight, float(eps), self.gate_w, self.top_k, self.aux_loss_coef, self.z_loss_coef,
            self._logit_bias(),
        )
        if timing is not None:
            timing.stop()
        idx, w, cnt = self._finish(flat, idx, w, aux, z, logits, cnt, stats, timing)
        return xn, idx, w, cnt

    def _logit_bias(self):
        bias = self.bias
        if self.logit_bias is not None:
            bias = self.logit_bias if bias is None else bias.detach().float() + self.logit_bias
        return bias

    def _finish(self, flat, idx, w, aux, z, logits, cnt, stats, timing):
        N = flat.shape[0]
        z_plain = None
        if self.bias is not None:
            # Reference semantics (L:677-687): with a bias the combine weights are
            # recomputed under no_grad, so no gradient flows through w; _last_logits
            # and the reported z statistic are computed without the bias (L:727-733).
            w = w.detach()
            # the bias-free logits as the reference forms them (x and gate in fp32, one product), not the
            # kernel's biased logits minus the bias, which would carry ~ulp(|bias|) of cancellation error
            with torch.no_grad():
                logits = flat.detach().float() @ self.gate_w.detach().float()
                if self.logit_bias is not None:
                    logits = logits + self.logit_bias.float()
            z_plain = torch.logsumexp(logits, dim=-1).square().mean().reshape(1) if N else logits.new_zeros(1)
        self._last_logits = logits
        self.last_aux_loss = aux
        self.last_z_loss = z
        self.last_stats = stats
        self.last_num_tokens = N
        self._profile = None
        self._pending = (N, _fwd_lds_bytes(flat, self.gate_w), router_fwd_bytes(flat, self.gate_w, self.top_k,
                                                                                   w.dtype), stats, z_plain, timing)
        if self.sync_profile and not self._defer_check:
            self._resolve(check=True)
        return idx, w, cnt

    def check_pending(self) -> None:
        """Run the checks of a forward made with the checks deferred (the token conservation and non-finite
        logits asserts; one device-to-host copy, which waits for the work enqueued so far)."""
        if self._pending is not None:
            self._resolve(check=True)

    def _resolve(self, check: bool = False) -> None:
        """Build ``last_profile`` from the pending forward: one device-to-host copy of the statistics (after
        which the forward's kernels, and so the second timing event, have completed)."""
        N, lds, nbytes, stats, z_plain, timing = self._pending
        self._pending = None
        head = stats[:8] if z_plain is None else torch.cat([stats[:8], z_plain])
        head = head.to("cpu")
        self.last_stats_host = head[:8]
        if check:
            total = int(round(float(head[STAT_CNT_TOTAL])))
            expected_total = N * self.top_k
            assert total == expected_total, (
                f"Token conservation violation: dispatched={total} "
                f"expected={expected_total} (N={N}, K={self.top_k})"
            )
            assert float(head[STAT_NONFINITE]) == 0.0, "NaN in expert indices (non-finite gate logits)"
        kernel_ms = timing.elapsed_ms() if timing is not None else 0.0
        self._profile = RouterProfile(
            sram_bytes_per_block=lds,
            achieved_bandwidth_gbps=_gbps(nbytes, kernel_ms),
            kernel_ms=kernel_ms,
            used_triton=True,
            tokens_per_expert_mean=float(head[STAT_CNT_MEAN]),
            tokens_per_expert_std=float(head[STAT_CNT_STD]),
            expert_load_imbalance=float(head[STAT_IMBALANCE]),
            router_z_loss=float(head[STAT_Z] if z_plain is None else head[8]),
        )
