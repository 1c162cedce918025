"""MoE layer with the reference's API, on the gfx950 kernels.

Mirrors ``moe-engine/pkg/distributed/moe_layer.py``:

* ``DistributedMoELayer(hidden_dim, ffn_dim, num_experts, top_k, topology,
  capacity_factor=1.25, capacity_dropping=False, dtype=torch.float32)``,
  ``forward([B,S,H] | [N,H]) -> same shape`` (L:206-360);
* ``compute_capacity_drop_mask(idx, num_experts, capacity) -> Bool[N,K]``
  and ``_cumcount(groups) -> Long[n]`` (L:64-155);
* ``_SwiGLUExpert`` (L:166-198) and the attributes ``router``, ``experts``,
  ``local_expert_ids``, ``last_{dispatch,combine,expert_compute}_ms``,
  ``last_overlap_ratio``, ``last_dropped_token_fraction``, ``_expert_to_rank``.

Forward pipeline, all on the GPU with no host synchronisation:
router kernel -> planner kernels (capacity drops, row layout) -> permute ->
SwiGLU grouped GEMM -> weighted combine.  The backward is the fused mirror
(combine-bwd, grouped GEMM backward, permute-bwd) plus the router backward.

Row layout (``layout`` argument, new):
* ``"reference"`` (default) reproduces the reference exactly: tokens are
  stable-sorted by their first choice, repeated K times, and the [N*K, H]
  buffer is cut into E equal chunks, chunk i going to expert i whatever the
  router chose (L:317-337); rows past E*chunk contribute zero.
* ``"routed"``: slot (t, k) goes to expert idx[t, k]; dropped slots get no row.

Expert weights are held stacked -- ``w_gate`` / ``w_up`` [E, F, H] and
``w_down`` [E, H, F] -- so one grouped GEMM reads them; ``experts[i]`` exposes
expert i's slices as ``w_gate.weight`` etc., and ``state_dict`` /
``load_state_dict`` use the reference's per-expert keys
(``experts.{i}.w_gate.weight``).  Assigning a different ModuleList to
``experts`` (the reference's extension point) switches the layer to calling
those modules per expert between the dispatch and combine kernels.  bf16 and
fp32 (the reference's default dtype) use the fused HIP grouped GEMM (bf16 or
fp32 MFMA); other dtypes and shapes call the expert modules per expert.
"""

from __future__ import annotations

import contextlib
import math
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from moe_mi355 import ops
from moe_mi355.layer import CombineFn, ExpertsFn, PermuteFn
from pkg.kernels.moe_router import MoERouter

__all__ = ["DistributedMoELayer", "compute_capacity_drop_mask", "_cumcount"]

_LAYOUTS = {"reference": ops.LAYOUT_REFERENCE, "routed": ops.LAYOUT_ROUTED}


class _ExpertTimer:
    """Two timing events on the current stream around the expert compute; the elapsed time is read only when
    asked for.  None on the CPU and under graph capture."""

    __slots__ = ("a", "b")

    @classmethod
    def new(cls, like: torch.Tensor) -> Optional["_ExpertTimer"]:
        if not like.is_cuda or torch.cuda.is_current_stream_capturing():
            return None
        t = cls()
        t.a = torch.cuda.Event(enable_timing=True)
        t.b = torch.cuda.Event(enable_timing=True)
        return t

    def start(self) -> None:
        self.a.record()

    def stop(self) -> None:
        self.b.record()

    def elapsed_ms(self) -> float:
        self.b.synchronize()
        return max(float(self.a.elapsed_time(self.b)), 0.0)


# The planner's key tables hold one contiguous range of at most this many ids (and K * E <= 8192 keys).
_PLAN_MAX_KEYS = 1024


def _cumcount(groups: torch.Tensor) -> torch.Tensor:
    """Each element's 0-based position among earlier elements of its group (L:64-115), for any integer ids.

    Ids spanning at most 1024 values run the planner's stable-grouping kernel (one column of K=1); wider
    ranges run moe_cumcount (a stable radix sort of the ids).  One host read of the id range."""
    n = groups.shape[0]
    if n == 0:
        return torch.empty(0, dtype=torch.long, device=groups.device)
    g = groups.reshape(n, 1).long()
    lo, hi = (int(v) for v in torch.stack([g.min(), g.max()]).tolist())
    if hi - lo + 1 > _PLAN_MAX_KEYS:
        return ops.cumcount(g.reshape(-1))
    g = g - lo
    E = hi - lo + 1
    # rank of each element within its key = position in the stable sort minus the key's offset
    p = ops.plan(g, max(E, 1), capacity=-1, layout=ops.LAYOUT_ROUTED)
    pos = p.slot_row.long()
    return pos - p.offsets.long()[g.reshape(-1)]


def compute_capacity_drop_mask(idx: torch.Tensor, num_experts: int, capacity: int) -> torch.Tensor:
    """``drop[t, k] = cumcount(idx[:, k])[t] >= capacity`` per column (L:118-155), for any integer ids."""
    N, K = idx.shape
    if N == 0:
        return torch.zeros(N, K, dtype=torch.bool, device=idx.device)
    if capacity < 0:  # every slot is at a position >= capacity
        return torch.ones(N, K, dtype=torch.bool, device=idx.device)
    # any integer group ids are valid here, as in the reference (one host read of the range)
    lo, hi = (int(v) for v in torch.stack([idx.min(), idx.max()]).tolist())
    if lo < 0 or hi >= num_experts:
        idx = idx - lo
        num_experts = hi - lo + 1
    if num_experts > _PLAN_MAX_KEYS or K * num_experts > 8192 or K > num_experts:
        # ids too many for the planner's key tables: the column ranks from the general kernel
        return torch.stack([_cumcount(idx[:, k]) >= capacity for k in range(K)], dim=1)
    p = ops.plan(idx, num_experts, capacity=int(capacity), layout=ops.LAYOUT_REFERENCE)
    return p.drop


class _ExpertWeight(nn.Module):
    """``.weight`` of one expert projection: a view of the layer's stacked tensor."""

    def __init__(self, owner_ref, name: str, index: int):
        super().__init__()
        object.__setattr__(self, "_owner", owner_ref)
        object.__setattr__(self, "_name", name)
        object.__setattr__(self, "_index", index)

    @property
    def weight(self) -> torch.Tensor:
        return getattr(self._owner(), self._name)[self._index]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.weight)


class _SwiGLUExpert(nn.Module):
    """``w_down(silu(w_gate(x)) * w_up(x))`` (L:166-198) over expert ``index``'s slices."""

    def __init__(self, owner_ref, index: int):
        super().__init__()
        self.w_gate = _ExpertWeight(owner_ref, "w_gate", index)
        self.w_up = _ExpertWeight(owner_ref, "w_up", index)
        self.w_down = _ExpertWeight(owner_ref, "w_down", index)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w_down(F.silu(self.w_gate(x)) * self.w_up(x))


class DistributedMoELayer(nn.Module):
    def __init__(
        self,
        hidden_dim: int,
        ffn_dim: int,
        num_experts: int,
        top_k: int,
        topology,
        capacity_factor: float = 1.25,
        capacity_dropping: bool = False,
        dtype: torch.dtype = torch.float32,
        layout: str = "reference",
        aux_loss_coef: float = 0.0,
        z_loss_coef: float = 0.0,
        check_numerics: bool = True,
    ):
        super().__init__()
        if getattr(topology, "ep_size", 1) != 1 or getattr(topology, "tp_size", 1) != 1:
            raise NotImplementedError("this build runs one GPU's experts; ep_size/tp_size > 1 are out of scope")
        if layout not in _LAYOUTS:
            raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}, got {layout!r}")
        self.hidden_dim = hidden_dim
        self.ffn_dim = ffn_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.topology = topology
        self.capacity_factor = capacity_factor
        self.capacity_dropping = capacity_dropping
        self.layout = layout
        self.check_numerics = check_numerics
        self.local_expert_ids: List[int] = topology.experts_on_this_rank(num_experts)
        dev = getattr(topology, "device", None)
        E = len(self.local_expert_ids)
        # nn.Linear-style init N(0, 1/sqrt(in)) per projection (tensor_parallel.py L:109, L:187)
        self.w_gate = nn.Parameter(torch.empty(E, ffn_dim, hidden_dim, device=dev, dtype=dtype))
        self.w_up = nn.Parameter(torch.empty(E, ffn_dim, hidden_dim, device=dev, dtype=dtype))
        self.w_down = nn.Parameter(torch.empty(E, hidden_dim, ffn_dim, device=dev, dtype=dtype))
        nn.init.normal_(self.w_gate, mean=0.0, std=1.0 / math.sqrt(hidden_dim))
        nn.init.normal_(self.w_up, mean=0.0, std=1.0 / math.sqrt(hidden_dim))
        nn.init.normal_(self.w_down, mean=0.0, std=1.0 / math.sqrt(ffn_dim))
        import weakref

        ref = weakref.ref(self)
        self.experts = nn.ModuleList([_SwiGLUExpert(ref, i) for i in range(E)])
        self.router = MoERouter(hidden_dim, num_experts, top_k, dtype=dtype, aux_loss_coef=aux_loss_coef,
                                z_loss_coef=z_loss_coef, sync_profile=check_numerics)
        if dev is not None:
            self.router.to(dev)
        self.last_dispatch_ms: float = 0.0
        self.last_combine_ms: float = 0.0
        self._expert_ms: float = 0.0
        self._expert_timer: Optional[_ExpertTimer] = None
        self.last_overlap_ratio: float = 0.0
        self.last_plan: Optional[ops.Plan] = None
        self._register_state_dict_hook(DistributedMoELayer._to_reference_keys)
        self._register_load_state_dict_pre_hook(DistributedMoELayer._from_reference_keys, with_module=True)

    # ---- state_dict in the reference's per-expert key format ----
    @staticmethod
    def _to_reference_keys(module, state_dict, prefix, local_metadata):
        for name in ("w_gate", "w_up", "w_down"):
            key = prefix + name
            if key in state_dict:
                stacked = state_dict.pop(key)
                for i in range(stacked.shape[0]):
                    state_dict[f"{prefix}experts.{i}.{name}.weight"] = stacked[i]
        return state_dict

    @staticmethod
    def _from_reference_keys(module, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                             error_msgs):
        for name in ("w_gate", "w_up", "w_down"):
            keys = [f"{prefix}experts.{i}.{name}.weight" for i in range(getattr(module, name).shape[0])]
            if all(k in state_dict for k in keys):
                state_dict[prefix + name] = torch.stack([state_dict.pop(k) for k in keys])

    @property
    def last_expert_compute_ms(self) -> float:
        """Time of the last forward's expert FFN compute (the grouped GEMMs, or the per-expert module calls),
        measured with device events on the launch stream (moe_layer.py L:326-337 times the same span with the
        host clock).  Reading it waits for the GPU to finish that span."""
        t = self._expert_timer
        if t is not None:
            self._expert_timer = None
            self._expert_ms = t.elapsed_ms()
        return self._expert_ms

    @last_expert_compute_ms.setter
    def last_expert_compute_ms(self, v: float) -> None:
        self._expert_timer = None
        self._expert_ms = float(v)

    @property
    def last_dropped_token_fraction(self) -> float:
        """Fraction of (token, k) slots dropped by capacity in the last forward (reads the device count)."""
        p = self.last_plan
        if p is None or not self.capacity_dropping or p.rows == 0:
            return 0.0
        return float(p.ndrop.item()) / float(p.rows)

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_dim}, num_experts={self.num_experts}, top_k={self.top_k}, "
            f"local_experts={len(self.local_expert_ids)}, ep_size=1, layout={self.layout}"
        )

    def _fused(self) -> bool:
        return (
            # the grouped GEMM's shapes: bf16 H % 8 == 0, fp32 H % 4 == 0, both F % 32 == 0
            self.w_gate.dtype in (torch.bfloat16, torch.float32)
            and self.w_gate.shape[-1] % (8 if self.w_gate.dtype == torch.bfloat16 else 4) == 0
            and self.w_gate.shape[1] % 32 == 0
            and all(type(m) is _SwiGLUExpert and m.w_gate._owner() is self for m in self.experts)
            and len(self.experts) == self.num_experts
        )

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        original_shape = tokens.shape
        if tokens.dim() not in (2, 3):
            raise ValueError(f"tokens must be rank 2 or 3, got {tokens.dim()}")
        H = tokens.shape[-1]
        flat = tokens.reshape(-1, H)
        with self._deferred_router_check(), self._linked_tokens():
            idx, weights, _cnt = self.router(flat)
        # the router hands the tokens back as a linked output (a view of the same memory): the expert path's
        # gradient of the tokens then reaches the router's backward, which adds it inside its dx kernel, so
        # x's gradient is formed in one pass instead of autograd adding the two paths' gradients afterwards
        # (the reference's autograd sums them, moe_layer.py L:288 and L:317-319)
        linked = self.router.take_linked_tokens()
        return self._experts_forward(flat if linked is None else linked, idx, weights).reshape(original_shape)

    @contextlib.contextmanager
    def _linked_tokens(self):
        r = self.router
        r._link_x = isinstance(r, MoERouter) and r.bias is None
        try:
            yield
        finally:
            r._link_x = False

    @contextlib.contextmanager
    def _deferred_router_check(self):
        """With ``check_numerics`` the router's checks (token conservation, non-finite logits) run at the end
        of the forward, at the synchronisation of the output NaN check, rather than right after the routing:
        the expert path is enqueued first, so the GPU does not wait for the host in the middle of the forward.
        The assertions and their order are the reference's (router first, then the output)."""
        r = self.router
        r._defer_check = self.check_numerics and r.sync_profile
        try:
            yield
        finally:
            r._defer_check = False

    def forward_normed(self, tokens: torch.Tensor, norm_weight: torch.Tensor, eps: float) -> torch.Tensor:
        """``forward(rmsnorm(tokens))`` with the norm fused into the router's read of the hidden state
        (moe-engine/pkg/models/moe.py L:125-126): the normalised rows feed both the router and the experts."""
        original_shape = tokens.shape
        if tokens.dim() not in (2, 3):
            raise ValueError(f"tokens must be rank 2 or 3, got {tokens.dim()}")
        H = tokens.shape[-1]
        flat = tokens.reshape(-1, H)
        with self._deferred_router_check():
            xn, idx, weights, _cnt = self.router.forward_with_norm(flat, norm_weight, eps)
        return self._experts_forward(xn, idx, weights).reshape(original_shape)

    def _experts_forward(self, flat: torch.Tensor, idx: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        N = flat.shape[0]
        capacity = (
            math.ceil(self.capacity_factor * N * self.top_k / self.num_experts) if self.capacity_dropping else -1
        )
        p = ops.plan(idx, self.num_experts, capacity=capacity, layout=_LAYOUTS[self.layout])
        self.last_plan = p
        if self._fused():
            train = torch.is_grad_enabled() and any(
                t.requires_grad for t in (flat, weights, self.w_gate, self.w_up, self.w_down))
            timer = _ExpertTimer.new(flat)
            out = ExpertsFn.apply(flat, weights, self.w_gate, self.w_up, self.w_down, p, train, timer)
        else:
            timer = _ExpertTimer.new(flat)
            out = self._forward_per_expert(flat, weights, p, timer)
        self._expert_timer = timer
        if self.check_numerics:
            has_nan = torch.isnan(out).any()  # enqueued before the router's deferred checks synchronise
            self.router.check_pending()
            assert not has_nan, (
                "NaN detected in DistributedMoELayer output after combine step. "
                "Check expert FFN numerics and router weights."
            )
        return out

    # ------------------------------------------------------------------
    # fp8 (e4m3) forward, new: an inference variant of the fused expert path
    # ------------------------------------------------------------------
    def quantize_fp8(self):
        """e4m3 copies of the expert weights with one fp32 scale per weight row (per output channel), made
        on the GPU; kept until the weights change (their in-place version counters are checked)."""
        key = tuple((t.data_ptr(), t._version) for t in (self.w_gate, self.w_up, self.w_down))
        cache = getattr(self, "_fp8_cache", None)
        if cache is None or cache[0] != key:
            with torch.no_grad():
                q = [ops.quant_rows_fp8(t.detach()) for t in (self.w_gate, self.w_up, self.w_down)]
            self._fp8_cache = (key, tuple(t for t, _ in q), tuple(sc for _, sc in q))
        return self._fp8_cache[1], self._fp8_cache[2]

    @torch.no_grad()
    def forward_fp8(self, tokens: torch.Tensor) -> torch.Tensor:
        """The layer's forward with an e4m3 dispatch payload and e4m3 expert GEMMs (no autograd): router and
        planner as in ``forward``, the permute writes each token row quantized (one fp32 scale per row),
        the gate/up and down projections run on the fp8 MFMA with per-row x per-channel scales, the
        SwiGLU activations are quantized per row between them, and the combine is the bf16 one.  Needs
        the fused bf16 expert layout (``self._fused()``) and hidden_dim % 16 == 0."""
        if not self._fused() or self.w_gate.dtype != torch.bfloat16:
            raise NotImplementedError("forward_fp8 needs the built-in SwiGLU experts in bfloat16")
        shape = tokens.shape
        flat = tokens.reshape(-1, shape[-1])
        idx, weights, _cnt = self.router(flat)
        N = flat.shape[0]
        capacity = (
            math.ceil(self.capacity_factor * N * self.top_k / self.num_experts) if self.capacity_dropping else -1
        )
        p = ops.plan(idx, self.num_experts, capacity=capacity, layout=_LAYOUTS[self.layout])
        self.last_plan = p
        wq, ws = self.quantize_fp8()
        xq, sx = ops.permute_fp8(flat, p)
        _act, _hgu, y = ops.swiglu_forward_fp8(xq, sx, wq, ws, p.offsets, keep_preact=False)
        out = ops.combine(y, weights, p)
        return out.reshape(shape)

    def _forward_per_expert(self, flat: torch.Tensor, weights: torch.Tensor, p: ops.Plan,
                            timer: Optional["_ExpertTimer"] = None) -> torch.Tensor:
        """Dispatch/combine kernels around per-expert module calls (custom experts, non-bf16 dtypes)."""
        xp = PermuteFn.apply(flat, p)
        offs = p.offsets.tolist()  # segment bounds for the per-expert calls
        parts = []
        if timer is not None:
            timer.start()
        for i, expert in enumerate(self.experts):
            lo, hi = offs[i], offs[i + 1]
            if lo < hi:
                parts.append(expert(xp[lo:hi]))
        if timer is not None:
            timer.stop()
        tail = p.rows - offs[len(self.experts)]
        if tail > 0:
            parts.append(xp.new_zeros((tail, xp.shape[1])))
        y = torch.cat(parts, 0) if parts else xp.new_zeros(xp.shape)
        return CombineFn.apply(y.contiguous(), weights, p)

    def _expert_to_rank(self, expert_ids: torch.Tensor) -> torch.Tensor:
        """Every expert lives on this (single) rank (reference L:362-389 at ep_size=1)."""
        return torch.zeros_like(expert_ids, dtype=torch.long)
