"""Synthetic inputs of the benchmark configurations.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(seed)``
in a fixed order, in float32, then cast, so the GPU run and any CPU check see
bit-identical inputs.

C1  router fwd+bwd, fp32:  T=4096  H=512  E=8   K=2   seed 0
C2  router fwd+bwd, bf16:  T=16384 H=4096 E=8   K=2   seed 1
C3  router+dispatch+combine, bf16: T=65536 H=2048 E=64 K=6 cf=1.25 (drops) seed 2
C4  layer fwd+bwd, bf16:   T=8192  H=4096 E=8   F=14336 K=2 seed 3
C5  skewed layer, bf16:    T=32768 H=2048 E=128 F=768 K=8 cf=1.0 (drops), Zipf(1.1) gate bias, seed 4
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class Config:
    name: str
    T: int
    H: int
    E: int
    K: int
    F: int = 0
    seed: int = 0
    dtype: torch.dtype = torch.bfloat16
    capacity_factor: float = 1.25
    capacity_dropping: bool = False
    aux_coef: float = 0.0
    z_coef: float = 0.0
    zipf_bias: bool = False

    def scaled(self, T: int) -> "Config":
        d = dict(self.__dict__)
        d["T"] = T
        return Config(**d)


C1 = Config("C1_router_fp32", T=4096, H=512, E=8, K=2, seed=0, dtype=torch.float32, aux_coef=0.01, z_coef=1e-3)
C2 = Config("C2_router_bf16", T=16384, H=4096, E=8, K=2, seed=1)
C3 = Config("C3_dispatch_bf16", T=65536, H=2048, E=64, K=6, seed=2, capacity_dropping=True)
C4 = Config("C4_layer_bf16", T=8192, H=4096, E=8, K=2, F=14336, seed=3)
# C4 in the reference module's default dtype (float32 tokens, gate and experts), inputs widened from C4's draws
C4_F32 = Config("C4_layer_fp32", T=8192, H=4096, E=8, K=2, F=14336, seed=3, dtype=torch.float32)
C5 = Config("C5_skewed_layer_bf16", T=32768, H=2048, E=128, K=8, F=768, seed=4, capacity_factor=1.0,
            capacity_dropping=True, aux_coef=0.01, z_coef=1e-3, zipf_bias=True)

CONFIGS = {c.name: c for c in (C1, C2, C3, C4, C5)}


def zipf_bias(E: int, g: torch.Generator, s: float = 1.1) -> torch.Tensor:
    """Per-expert logit bias from a Zipf(s) ranking: b_e = -s * ln(rank_e)."""
    r = torch.randperm(E, generator=g).to(torch.float32) + 1.0
    return -s * torch.log(r)


def router_inputs(cfg: Config) -> Dict[str, torch.Tensor]:
    """x [T,H], gate_w [H,E] ~N(0,0.02), grad_w [T,K] ~N(0,1), optional bias [E]; CPU tensors."""
    g = torch.Generator().manual_seed(cfg.seed)
    x = torch.randn(cfg.T, cfg.H, generator=g).to(cfg.dtype)
    gate_w = (torch.randn(cfg.H, cfg.E, generator=g) * 0.02).to(cfg.dtype)
    grad_w = torch.randn(cfg.T, cfg.K, generator=g).to(cfg.dtype)
    out = {"x": x, "gate_w": gate_w, "grad_w": grad_w}
    if cfg.zipf_bias:
        out["bias"] = zipf_bias(cfg.E, g)
    return out


def layer_inputs(cfg: Config, device: Optional[torch.device] = None) -> Dict[str, torch.Tensor]:
    """Router inputs plus expert weights w_gate/w_up [E,F,H], w_down [E,H,F] ~N(0,0.02) and
    grad_out [T,H] ~N(0,1).  Weights are generated per expert in order (gate, up, down)."""
    g = torch.Generator().manual_seed(cfg.seed)
    dev = device or torch.device("cpu")
    x = torch.randn(cfg.T, cfg.H, generator=g).to(cfg.dtype)
    gate_w = (torch.randn(cfg.H, cfg.E, generator=g) * 0.02).to(cfg.dtype)
    wg = torch.empty(cfg.E, cfg.F, cfg.H, dtype=cfg.dtype, device=dev)
    wu = torch.empty(cfg.E, cfg.F, cfg.H, dtype=cfg.dtype, device=dev)
    wd = torch.empty(cfg.E, cfg.H, cfg.F, dtype=cfg.dtype, device=dev)
    for e in range(cfg.E):
        wg[e].copy_((torch.randn(cfg.F, cfg.H, generator=g) * 0.02).to(cfg.dtype))
        wu[e].copy_((torch.randn(cfg.F, cfg.H, generator=g) * 0.02).to(cfg.dtype))
        wd[e].copy_((torch.randn(cfg.H, cfg.F, generator=g) * 0.02).to(cfg.dtype))
    grad_out = torch.randn(cfg.T, cfg.H, generator=g).to(cfg.dtype)
    out = {"x": x, "gate_w": gate_w, "w_gate": wg, "w_up": wu, "w_down": wd, "grad_out": grad_out}
    if cfg.zipf_bias:
        out["bias"] = zipf_bias(cfg.E, g)
    return out


def capacity(cfg: Config, T: Optional[int] = None) -> int:
    return math.ceil(cfg.capacity_factor * (T or cfg.T) * cfg.K / cfg.E)
