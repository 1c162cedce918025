#!/usr/bin/env python3
"""Benchmark of the MI355X MoE hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

Workloads (inputs drawn on the CPU from fixed seeds, resident in HBM before
timing starts; ``moe_mi355/configs.py``):

  layer   (default) C4, the headline line: full MoE layer fwd+bwd, T=8192
          d=4096 E=8 SwiGLU F=14336 K=2, bf16 -- router, planner, permute,
          grouped gate/up/down GEMM, combine, and the whole backward.
          ``value`` = tokens/s.  The same run measures every other config
          under its own key: "router" (C2), "c1", "norm_router", "fp8_fwd",
          "dispatch" (C3) and "skewed" (C5), each with its roofline and,
          where the config has one, its CPU baseline.
  c4      the headline C4 leg alone.
  router  C2: router fwd+bwd, T=16384 d=4096 E=8 K=2.
  c1      C1: router fwd+bwd, T=4096 d=512 E=8 K=2, fp32, aux 0.01 + z 1e-3,
          timed the reference's way (3 warmup + 20 timed, mean +- std), beside
          the float64 oracle of the same step on the CPU.
  norm_router  C2 shape with the block's RMSNorm in front of the router:
          the norm fused into the router's read of the hidden state, fwd+bwd,
          beside the unfused composition and a torch-ops norm.
  dispatch C3: router + planner + permute + combine forward, T=65536 d=2048
          E=64 K=6, cf=1.25 with drops.
  skewed  C5: layer fwd+bwd, T=32768 d=2048 E=128 F=768 K=8, cf=1.0 drops,
          aux+z losses, Zipf(1.1) gate bias, routed layout.
  fp8_fwd C4 layer forward without autograd, bf16 beside the e4m3 dispatch
          payload + fp8 expert GEMMs (the fp8 line's dtype is "fp8-e4m3").

One step = one forward + backward (forward only for dispatch).  W untimed
warmup steps, then exactly K steps bracketed by torch.cuda.synchronize();
prints ONE JSON line on stdout.  Per-kernel durations come from a separate
pass (after the timed one) in which libmoe_mi355.so records hipEvents around
each of its launches on the launch stream.  The router leg is also replayed
as a captured HIP graph (``graph_*`` fields: the rate without host launch
overhead).  The CPU baselines are the float64 oracle timed on a bounded
sample of the same workload (the whole config for C1) on this host's cores.
The headline layer is timed with check_numerics=False; the layer's default
configuration (per-forward NaN assert and checked router statistics, each
with a host synchronisation) is timed too ("check_numerics_ms_per_step").
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "composed-mixture-of-experts-engine_amd")
for _p in (PKG_DIR, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "MoE layer fwd+bwd tokens/s @E=8,d=4096 bf16; router fwd+bwd HBM GB/s vs peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_counters.md")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")


def kernel_src_digest():
    """sha256 over the GPU kernel sources (csrc/*.hip and csrc/*.h, sorted by name): the identity of the
    kernels a counter summary was measured on."""
    import hashlib

    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC_DIR)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(CSRC_DIR, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()


def measured_traffic(kernel, workload):
    """HBM bytes per launch of ``kernel`` on ``workload`` from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the counter reads for a plain
    copy of known size), or None when the summary has no entry for it or was measured on other
    kernel sources than the ones built here (its ``kernel_src_sha256`` differs)."""
    try:
        with open(TRAFFIC_FILE) as f:
            text = f.read()
    except OSError:
        return None
    start = text.find("```json")
    if start < 0:
        return None
    end = text.find("```", start + 7)
    try:
        data = json.loads(text[start + 7:end])
    except ValueError:
        return None
    if data.get("kernel_src_sha256") != kernel_src_digest():
        log(f"[bench] {os.path.relpath(TRAFFIC_FILE, REPO)} was measured on other kernel sources: "
            "roofline.traffic left null")
        return None
    ent = data.get("workloads", {}).get(workload, {}).get(kernel)
    if ent is None:
        return None
    return int(ent["fetch_bytes"] + ent["write_bytes"])


def cpu_thread_count():
    """Threads for the CPU baselines: every core this process may run on (its affinity set), or fewer when
    the host sets OMP_NUM_THREADS (the GPU box grants each GPU a share of its cores and sets it to that)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(n, 1)


def cpu_cores(torch):
    """The core-count fields of a cpu_baseline record: the threads the baseline ran with, and the host's
    os.cpu_count() and affinity set beside it."""
    return {"cores": torch.get_num_threads(), "host_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def copy_probe(torch):
    """One plain 1 GiB device-to-device copy (torch copy kernel): the known-size reference that the
    FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    src = torch.ones(1 << 29, dtype=torch.int16, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def timed(torch, step, steps, warmup, prof_steps=None):
    """Run W warmup steps, then K timed steps bracketed by synchronize (no per-kernel events: ms/step is the
    plain steady-state rate), then a separate pass of ``prof_steps`` steps with the library's per-launch
    hipEvents on for the per-kernel table.  Returns (ms/step, {kernel: (launches, total ms)})."""
    from moe_mi355 import _lib

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    _lib.prof_enable(True)
    for _ in range(prof_steps or steps):
        step()
    torch.cuda.synchronize()
    _lib.prof_enable(False)
    return ms, _lib.prof_summary()


def mean_std_ms(fn, warmup=3, iters=20, sync=None):
    """The reference's timing (run_benchmark.py L:63-79): ``warmup`` untimed calls, then ``iters`` calls each
    timed on the host clock (after a device synchronize when ``sync`` is given); mean and population std."""
    for _ in range(warmup):
        fn()
    if sync:
        sync()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        if sync:
            sync()
        times.append((time.perf_counter() - t0) * 1e3)
    mean = sum(times) / len(times)
    return mean, (sum((t - mean) ** 2 for t in times) / len(times)) ** 0.5


def graph_timed(torch, step, steps, warmup):
    """The same step captured once as a HIP graph (torch.cuda.graph) and replayed K times: the rate without
    host launch overhead.  Returns ms/step."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(warmup, 3)):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    del g
    return t0.elapsed_time(t1) / steps


def kernel_table(prof, work, unit_scale, unit):
    """Per-kernel launches / avg us / rate (GB/s or TFLOP/s) from algorithmic work per launch."""
    out = {}
    for name, (n, tot) in prof.items():
        avg_us = 1e3 * tot / max(n, 1)
        ent = {"launches": n, "avg_us": round(avg_us, 3)}
        if name in work:
            ent["work_per_launch"] = work[name]
            ent[unit] = round(work[name] / (avg_us * 1e-6) / unit_scale, 2)
        out[name] = ent
    return out


# ---------------------------------------------------------------------------
# router (C2)
# ---------------------------------------------------------------------------
def router_bytes(N, H, E, K):
    """Algorithmic HBM bytes per launch of the main router kernels and of one fwd+bwd."""
    fwd = N * H * 2 + H * E * 2 + N * E * 4 + N * 4 + N * K * (8 + 2)
    glog = N * E * 4 + N * K * (8 + 2) + E * 8 + N * E * 4 + N * E * 2
    dxdw = 2 * N * H * 2 + N * E * 2 + H * E * 2
    total = 3 * N * H * 2 + 2 * H * E * 2 + H * E * 4 + 2 * N * E * 4 + N * K * (8 + 2 + 8 + 2) + E * 8
    return {"k_router_fwd_bf16": fwd, "k_router_glogits": glog, "k_router_dxdw_bf16": dxdw, "step": total}


def run_router(args, torch):
    from moe_mi355 import configs
    from moe_mi355.router import RouterCore

    cfg = configs.C2
    dev = torch.device("cuda:0")
    inp = configs.router_inputs(cfg)
    x = inp["x"].to(dev).requires_grad_(True)
    w = inp["gate_w"].to(dev).requires_grad_(True)
    gw = inp["grad_w"].to(dev)
    N, H, E, K = cfg.T, cfg.H, cfg.E, cfg.K

    def step():
        out = RouterCore.apply(x, w, K, 0.0, 0.0, None)
        torch.autograd.grad(out[1], (x, w), grad_outputs=gw)

    ms, prof = timed(torch, step, max(args.steps, 20), args.warmup)
    gms = graph_timed(torch, step, max(args.steps, 20), args.warmup)
    alg = router_bytes(N, H, E, K)
    kernels = kernel_table(prof, alg, 1e9, "GBps")
    dom = max((k for k in kernels if k in alg), key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    achieved = kernels[dom]["GBps"]
    gbs = alg["step"] / (ms * 1e-3) / 1e9
    return {
        "workload": "C2 router fwd+bwd", "tokens": N, "d_model": H, "experts": E, "top_k": K,
        "ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3),
        "fwd_bwd_GBps": round(gbs, 1), "fwd_bwd_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "graph_ms_per_step": gms, "graph_fwd_bwd_GBps": round(alg["step"] / (gms * 1e-3) / 1e9, 1),
        "graph_fwd_bwd_frac_of_hbm_peak": round(alg["step"] / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "alg_bytes_per_step": alg["step"],
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom, cfg.name),
                     "alg_bytes_per_launch": alg[dom], "avg_us": kernels[dom]["avg_us"]},
        "kernels": kernels,
    }


def cpu_baseline_router(torch):
    """The float64 oracle of the whole C2 router step (forward + backward, same seed) on the host's cores, timed
    the reference's way: 3 warmup + 20 timed calls, mean +- std (run_benchmark.py L:63-79)."""
    from oracle import router as OR

    from moe_mi355 import configs

    cfg = configs.C2
    inp = configs.router_inputs(cfg)
    x, w, gw = inp["x"], inp["gate_w"], inp["grad_w"]
    mean, std = mean_std_ms(lambda: OR.router_full(x, w, cfg.K, grad_w=gw))
    return {"value": cfg.T / (mean * 1e-3), "unit": "tokens/s", **cpu_cores(torch), "kind": "port",
            "ms_mean": round(mean, 2), "ms_std": round(std, 2),
            "sample": f"the whole C2 config: float64 oracle router fwd+bwd (oracle/router.py router_full), "
                      f"T={cfg.T} d={cfg.H} E={cfg.E} K={cfg.K}, seed {cfg.seed}, 3 warmup + 20 timed calls"}


# ---------------------------------------------------------------------------
# C1: the reference's CPU-runnable router config (fp32, aux and z losses)
# ---------------------------------------------------------------------------
def run_c1(args, torch, with_cpu=True):
    """Router fwd+bwd at C1 (T=4096, d=512, E=8, K=2, fp32, seed 0, aux 0.01, z 1e-3) on the GPU and, as the
    CPU baseline, the float64 oracle of the same step (oracle/router.py router_full), both timed the
    reference's way: 3 warmup + 20 timed calls, mean +- std (run_benchmark.py L:63-79)."""
    from moe_mi355 import configs
    from moe_mi355.router import RouterCore

    cfg = configs.C1
    inp = configs.router_inputs(cfg)
    dev = torch.device("cuda:0")
    x = inp["x"].to(dev).requires_grad_(True)
    w = inp["gate_w"].to(dev).requires_grad_(True)
    gw = inp["grad_w"].to(dev)
    one = torch.ones((), device=dev)
    N, H, E, K = cfg.T, cfg.H, cfg.E, cfg.K

    def step():
        out = RouterCore.apply(x, w, K, cfg.aux_coef, cfg.z_coef, None)
        torch.autograd.grad([out[1], out[2], out[3]], (x, w), grad_outputs=[gw, one, one])

    mean, std = mean_std_ms(step, sync=torch.cuda.synchronize)
    ms, _ = timed(torch, step, max(args.steps, 20), args.warmup, prof_steps=1)
    nbytes = 3 * N * H * 4 + 2 * H * E * 4 + 2 * N * E * 4 + N * K * (8 + 4 + 4) + E * 8
    res = {"workload": "C1 router fwd+bwd, fp32, aux 0.01 + z 1e-3", "tokens": N, "d_model": H, "experts": E,
           "top_k": K, "ms_mean": round(mean, 4), "ms_std": round(std, 4), "tokens_per_s": N / (mean * 1e-3),
           "pipelined_ms_per_step": ms, "pipelined_tokens_per_s": N / (ms * 1e-3),
           "fwd_bwd_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    if with_cpu:
        from oracle import router as OR

        xc, wc, gc = inp["x"], inp["gate_w"], inp["grad_w"]
        cm, cs = mean_std_ms(lambda: OR.router_full(xc, wc, K, grad_w=gc, alpha=cfg.aux_coef, beta=cfg.z_coef))
        res["cpu_baseline"] = {
            "value": N / (cm * 1e-3), "unit": "tokens/s", **cpu_cores(torch), "kind": "port",
            "ms_mean": round(cm, 3), "ms_std": round(cs, 3),
            "sample": "the whole C1 config: float64 oracle router fwd+bwd with aux and z losses (oracle/router.py "
                      "router_full), T=4096 d=512 E=8 K=2, seed 0, 3 warmup + 20 timed calls"}
        res["gpu_vs_cpu"] = round(cm / mean, 1)
    return res


# ---------------------------------------------------------------------------
# layer (C4, C5)
# ---------------------------------------------------------------------------
GEMM_KERNELS = ("k_gemm_swiglu_fwd1", "k_gemm_swiglu_fwd2", "k_gemm_swiglu_dact", "k_gemm_swiglu_dxp",
                "k_gemm_swiglu_dwd", "k_gemm_swiglu_dw1")


def gemm_flops(R, H, F):
    """FLOPs per launch of each grouped-GEMM kernel for R computed rows."""
    return {"k_gemm_swiglu_fwd1": 2 * R * H * 2 * F, "k_gemm_swiglu_fwd2": 2 * R * F * H,
            "k_gemm_swiglu_dact": 2 * R * H * F, "k_gemm_swiglu_dxp": 2 * R * 2 * F * H,
            "k_gemm_swiglu_dwd": 2 * R * H * F, "k_gemm_swiglu_dw1": 2 * R * 2 * F * H}


def layer_hbm_bytes(N, H, E, K, R, es=2):
    """Algorithmic HBM bytes per launch of the layer's data-movement and router kernels (bf16 rows, R computed
    rows): each token row is read once by the permute and written to its rows; the combine reads the rows and
    writes the tokens; the backward passes mirror them."""
    return {"k_permute": N * H * es + R * H * es + N * K * 4,
            "k_combine": R * H * es + N * H * es + N * K * (2 + 4 + 1),
            "k_combine_bwd": N * H * es + 2 * R * H * es + N * K * (2 + 4 + 1 + 2),
            "k_unpermute_sum": R * H * es + N * H * es + N * K * 4,
            "k_router_fwd_bf16": N * H * es + H * E * es + N * E * 4 + N * 4 + N * K * (8 + es),
            # read x and the expert path's gradient of x (added in the dx stores), write dx
            "k_router_dxdw_bf16": 3 * N * H * es + N * E * 2 + H * E * es}


def build_layer(cfg, torch, inp, layout):
    from pkg.distributed import build_topology
    from pkg.distributed.moe_layer import DistributedMoELayer

    dev = torch.device("cuda:0")
    layer = DistributedMoELayer(cfg.H, cfg.F, cfg.E, cfg.K, build_topology(), capacity_factor=cfg.capacity_factor,
                                capacity_dropping=cfg.capacity_dropping, dtype=cfg.dtype, layout=layout,
                                aux_loss_coef=cfg.aux_coef, z_loss_coef=cfg.z_coef, check_numerics=False).to(dev)
    with torch.no_grad():
        layer.router.gate_w.copy_(inp["gate_w"])
        layer.w_gate.copy_(inp["w_gate"])
        layer.w_up.copy_(inp["w_up"])
        layer.w_down.copy_(inp["w_down"])
    if "bias" in inp:
        layer.router.logit_bias = inp["bias"].to(dev)
    return layer


MFMA_F32_PEAK_TFLOPS = 157.3


def run_layer(args, torch, cfg, layout, inp, default_numerics=False):
    """Layer fwd+bwd at ``cfg`` (its dtype: bf16, or fp32 with the inputs widened from ``inp``)."""
    dev = torch.device("cuda:0")
    layer = build_layer(cfg, torch, inp, layout)
    x = inp["x"].to(dev).to(cfg.dtype).requires_grad_(True)
    gout = inp["grad_out"].to(dev).to(cfg.dtype)
    peak = MFMA_F32_PEAK_TFLOPS if cfg.dtype == torch.float32 else MFMA_BF16_PEAK_TFLOPS
    if cfg.dtype == torch.float32:  # ~17 TFLOP of fp32 MFMA per C4 step: a few steps suffice
        args = argparse.Namespace(**{**vars(args), "steps": min(args.steps, 5), "warmup": min(args.warmup, 1)})
    params = [x, layer.router.gate_w, layer.w_gate, layer.w_up, layer.w_down]
    use_losses = cfg.aux_coef != 0.0 or cfg.z_coef != 0.0
    one = torch.ones((), device=dev)

    def step():
        out = layer(x)
        if use_losses:
            torch.autograd.grad([out, layer.router.last_aux_loss, layer.router.last_z_loss], params,
                                grad_outputs=[gout, one, one])
        else:
            torch.autograd.grad(out, params, grad_outputs=gout)

    log(f"[bench] timing {cfg.name}")
    ms, prof = timed(torch, step, args.steps, args.warmup, prof_steps=min(args.steps, 5))
    R = int(layer.last_plan.offsets[-1].item())  # rows run through the experts
    expert_ms = layer.last_expert_compute_ms
    numerics_ms = None
    if default_numerics:
        # the layer's default configuration: the per-forward NaN assert and the router's checked statistics,
        # each with its host synchronisation (the timed steps above run with check_numerics=False)
        layer.check_numerics = True
        layer.router.sync_profile = True
        numerics_ms, _ = timed(torch, step, args.steps, args.warmup, prof_steps=1)
        layer.check_numerics = False
        layer.router.sync_profile = False
    fl = gemm_flops(R, cfg.H, cfg.F)
    if cfg.dtype == torch.float32:
        fl = {k + "_f32": v for k, v in fl.items()}
    kernels = kernel_table(prof, fl, 1e12, "TFLOPs")
    hbm = layer_hbm_bytes(cfg.T, cfg.H, cfg.E, cfg.K, R, es=4 if cfg.dtype == torch.float32 else 2)
    for name, ent in kernel_table(prof, hbm, 1e9, "GBps").items():
        if name in hbm:
            kernels[name].update(ent)
            kernels[name]["frac_of_hbm_peak"] = round(ent["GBps"] / HBM_PEAK_GBS, 4)
    dom = max((k for k in kernels if k in fl), key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    achieved = kernels[dom]["TFLOPs"]
    step_flops = 18 * R * cfg.H * cfg.F
    gemm_ms = sum(prof[k][1] / prof[k][0] for k in fl if k in prof)
    res = {
        "workload": f"{cfg.name} layer fwd+bwd ({layout} layout)", "tokens": cfg.T, "d_model": cfg.H,
        "experts": cfg.E, "ffn": cfg.F, "top_k": cfg.K, "rows_computed": R,
        "capacity_factor": cfg.capacity_factor if cfg.capacity_dropping else None,
        "ms_per_step": ms, "tokens_per_s": cfg.T / (ms * 1e-3),
        "check_numerics_ms_per_step": numerics_ms,
        "last_expert_compute_ms": round(expert_ms, 4),
        "expert_TFLOP_per_step": step_flops / 1e12,
        "step_TFLOPs": round(step_flops / (ms * 1e-3) / 1e12, 2),
        "step_frac_of_mfma_peak": round(step_flops / (ms * 1e-3) / 1e12 / peak, 4),
        "gemm_ms_per_step": round(gemm_ms, 4),
        "gemm_TFLOPs": round(step_flops / (gemm_ms * 1e-3) / 1e12, 2) if gemm_ms else None,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": peak,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic(dom, f"{cfg.name}:{layout}"),
                     "flops_per_launch": fl[dom], "avg_us": kernels[dom]["avg_us"]},
        "kernels": kernels,
    }
    del layer
    torch.cuda.empty_cache()
    return res


MFMA_FP8_PEAK_TFLOPS = 5000.0


def run_fp8_fwd(args, torch, inp):
    """C4 layer forward (no autograd) in bf16 and with the e4m3 dispatch payload and fp8 expert GEMMs
    (weights quantized once, outside the timed region, as an inference deployment keeps them)."""
    cfg = configs_mod().C4
    layer = build_layer(cfg, torch, inp, "reference")
    x = inp["x"].to(torch.device("cuda:0"))
    layer.quantize_fp8()

    def bf16_step():
        with torch.no_grad():
            layer(x)

    def fp8_step():
        layer.forward_fp8(x)

    log("[bench] timing C4 forward bf16 / fp8")
    ms_bf16, prof_bf16 = timed(torch, bf16_step, args.steps, args.warmup, prof_steps=min(args.steps, 5))
    ms_fp8, prof_fp8 = timed(torch, fp8_step, args.steps, args.warmup, prof_steps=min(args.steps, 5))
    R = int(layer.last_plan.offsets[-1].item())
    fl = gemm_flops(R, cfg.H, cfg.F)
    fl8 = {"k_gemm_swiglu_fwd1_fp8": fl["k_gemm_swiglu_fwd1"], "k_gemm_swiglu_fwd2_fp8": fl["k_gemm_swiglu_fwd2"]}
    k16 = kernel_table(prof_bf16, fl, 1e12, "TFLOPs")
    k8 = kernel_table(prof_fp8, fl8, 1e12, "TFLOPs")
    dom = "k_gemm_swiglu_fwd1_fp8"
    fwd_flops = fl["k_gemm_swiglu_fwd1"] + fl["k_gemm_swiglu_fwd2"]
    res = {
        "workload": "C4 layer forward, bf16 vs e4m3 payload + fp8 expert GEMMs (no autograd)",
        "tokens": cfg.T, "rows_computed": R,
        "bf16_ms_per_step": ms_bf16, "bf16_tokens_per_s": cfg.T / (ms_bf16 * 1e-3),
        "fp8_ms_per_step": ms_fp8, "fp8_tokens_per_s": cfg.T / (ms_fp8 * 1e-3),
        "fp8_speedup": round(ms_bf16 / ms_fp8, 3),
        "expert_TFLOP_per_step": fwd_flops / 1e12,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": k8[dom]["TFLOPs"], "peak": MFMA_FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(k8[dom]["TFLOPs"] / MFMA_FP8_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(dom, f"{cfg.name}:fp8"),
                     "flops_per_launch": fl8[dom], "avg_us": k8[dom]["avg_us"]},
        "kernels_bf16": k16, "kernels_fp8": k8,
    }
    del layer
    torch.cuda.empty_cache()
    return res


def configs_mod():
    from moe_mi355 import configs

    return configs


def cpu_baseline_layer(torch, cfg, layout, inp, sample_T=32, budget_s=12.0, min_reps=3):
    """float64 oracle layer fwd+bwd on the first ``sample_T`` tokens with the full-size weights (converted to
    float64 once, before timing), at least ``min_reps`` reps; mean +- std per rep."""
    from oracle import layer as OL
    from oracle import plan as OP

    f64 = {k: inp[k].double() for k in ("gate_w", "w_gate", "w_up", "w_down")}
    x = inp["x"][:sample_T].double()
    g = inp["grad_out"][:sample_T].double()
    lay = OP.LAYOUT_REFERENCE if layout == "reference" else OP.LAYOUT_ROUTED
    bias = inp.get("bias")

    def rep():
        OL.layer_fwd_bwd(x, f64["gate_w"], f64["w_gate"], f64["w_up"], f64["w_down"], cfg.K, grad_out=g,
                         capacity_factor=cfg.capacity_factor, capacity_dropping=cfg.capacity_dropping, layout=lay,
                         alpha=cfg.aux_coef, beta=cfg.z_coef, bias=bias)

    rep()  # warmup
    times, t0 = [], time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t0 < budget_s and len(times) < 50):
        a = time.perf_counter()
        rep()
        times.append(time.perf_counter() - a)
    mean = sum(times) / len(times)
    std = (sum((t - mean) ** 2 for t in times) / len(times)) ** 0.5
    del f64
    return {"value": sample_T / mean, "unit": "tokens/s", **cpu_cores(torch), "kind": "port",
            "ms_mean": round(mean * 1e3, 1), "ms_std": round(std * 1e3, 1),
            "sample": f"float64 oracle layer fwd+bwd (oracle/layer.py layer_fwd_bwd) on the first {sample_T} "
                      f"tokens of {cfg.name} with the full-size expert weights (converted to float64 before "
                      f"timing), {len(times)} reps after 1 warmup"}


# ---------------------------------------------------------------------------
# RMSNorm fused into the router read (C2 shape)
# ---------------------------------------------------------------------------
def norm_router_bytes(N, H, E, K):
    """Algorithmic HBM bytes of the fused norm+router forward launch and of one fused fwd+bwd step.

    Forward: read x, write xn, the router's per-token outputs (logits, lse, rstd, idx, w).  Backward, counted
    once: read x and the expert path's gradient of xn, write dx (three [N,H] passes), plus the saved logits,
    top-k, upstream weight gradients, rstd, the gate and its gradient, gamma and its gradient.  (The kernels
    re-read xn for the gate gradient: four passes.)"""
    tok = N * E * 4 + N * 4 + N * 4 + N * K * (8 + 2)
    fwd = 2 * N * H * 2 + H * E * 2 + H * 4 + tok
    bwd = 3 * N * H * 2 + 2 * H * E * 2 + N * E * 4 + N * K * (8 + 2) + N * 4 + E * 8 + 2 * H * 4
    return {"k_rmsnorm_route": fwd, "step": fwd + bwd}


def run_norm_router(args, torch):
    from moe_mi355 import configs
    from moe_mi355.norm import NormRouterCore, RMSNormFn
    from moe_mi355.router import RouterCore

    cfg = configs.C2
    dev = torch.device("cuda:0")
    inp = configs.router_inputs(cfg)
    N, H, E, K = cfg.T, cfg.H, cfg.E, cfg.K
    eps = 1e-5
    g = torch.Generator().manual_seed(77)
    x = inp["x"].to(dev).requires_grad_(True)
    gate = inp["gate_w"].to(dev).requires_grad_(True)
    nw = (1.0 + 0.1 * torch.randn(H, generator=g)).to(dev).requires_grad_(True)
    g_w = inp["grad_w"].to(dev)
    g_xn = (torch.randn(N, H, generator=g) * 0.01).to(torch.bfloat16).to(dev)

    def fused():
        xn, _i, w, *_ = NormRouterCore.apply(x, nw, eps, gate, K, 0.0, 0.0, None)
        torch.autograd.grad((xn, w), (x, nw, gate), grad_outputs=(g_xn, g_w))

    def composed():
        xn = RMSNormFn.apply(x, nw, eps)
        out = RouterCore.apply(xn, gate, K, 0.0, 0.0, None)
        torch.autograd.grad((xn, out[1]), (x, nw, gate), grad_outputs=(g_xn, g_w))

    def torch_norm():
        # the reference's RMSNorm as torch ops (moe-engine/pkg/models/moe.py L:83-86) in front of the router
        v = x.float()
        xn = ((v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)) * nw).to(x.dtype)
        out = RouterCore.apply(xn, gate, K, 0.0, 0.0, None)
        torch.autograd.grad((xn, out[1]), (x, nw, gate), grad_outputs=(g_xn, g_w))

    steps = max(args.steps, 20)
    ms, prof = timed(torch, fused, steps, args.warmup)
    gms = graph_timed(torch, fused, steps, args.warmup)
    ms_comp, _ = timed(torch, composed, steps, args.warmup, prof_steps=1)
    ms_torch, _ = timed(torch, torch_norm, steps, args.warmup, prof_steps=1)
    alg = norm_router_bytes(N, H, E, K)
    kernels = kernel_table(prof, alg, 1e9, "GBps")
    dom = "k_rmsnorm_route"
    achieved = kernels[dom]["GBps"]
    return {
        "workload": "C2 RMSNorm + router fwd+bwd (norm fused into the router read)", "tokens": N, "d_model": H,
        "experts": E, "top_k": K, "ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3),
        "fwd_bwd_GBps": round(alg["step"] / (ms * 1e-3) / 1e9, 1),
        "fwd_bwd_frac_of_hbm_peak": round(alg["step"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "graph_ms_per_step": gms,
        "unfused_ms_per_step": ms_comp, "torch_norm_ms_per_step": ms_torch,
        "alg_bytes_per_step": alg["step"],
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom, cfg.name),
                     "alg_bytes_per_launch": alg[dom], "avg_us": kernels[dom]["avg_us"]},
        "kernels": kernels,
    }


# ---------------------------------------------------------------------------
# dispatch (C3)
# ---------------------------------------------------------------------------
def run_dispatch(args, torch, with_cpu=True):
    from moe_mi355 import configs, ops

    cfg = configs.C3
    dev = torch.device("cuda:0")
    inp = configs.router_inputs(cfg)
    x = inp["x"].to(dev)
    w = inp["gate_w"].to(dev)
    cap = configs.capacity(cfg)
    state = {}

    def step():
        idx, wt, *_ = ops.router_forward(x, w, cfg.K)
        p = ops.plan(idx, cfg.E, capacity=cap, layout=ops.LAYOUT_ROUTED)
        xp = ops.permute(x, p)
        state["out"] = ops.combine(xp, wt, p)
        state["p"] = p

    log("[bench] timing C3")
    ms, prof = timed(torch, step, args.steps, args.warmup)
    R = int(state["p"].offsets[-1].item())
    N, H, E, K = cfg.T, cfg.H, cfg.E, cfg.K
    hbm = layer_hbm_bytes(N, H, E, K, R)
    work = {k: hbm[k] for k in ("k_router_fwd_bf16", "k_permute", "k_combine")}
    kernels = kernel_table(prof, work, 1e9, "GBps")
    for k in work:
        if k in kernels:
            kernels[k]["frac_of_hbm_peak"] = round(kernels[k]["GBps"] / HBM_PEAK_GBS, 4)
    dom = max((k for k in kernels if k in work), key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    total = sum(work.values())
    res = {"workload": "C3 router + plan + permute + combine (routed layout, cf=1.25 drops)", "tokens": N,
           "d_model": H, "experts": E, "top_k": K, "rows_kept": R, "ms_per_step": ms,
           "tokens_per_s": N / (ms * 1e-3), "alg_bytes_per_step": total,
           "GBps": round(total / (ms * 1e-3) / 1e9, 1),
           "roofline": {"bound": "hbm", "kernel": dom, "achieved": kernels[dom]["GBps"], "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(kernels[dom]["GBps"] / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic(dom, cfg.name), "alg_bytes_per_launch": work[dom],
                        "avg_us": kernels[dom]["avg_us"]},
           "kernels": kernels}
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline_dispatch(torch, cfg, inp)
    return res


def cpu_baseline_dispatch(torch, cfg, inp, sample_T=8192, budget_s=6.0):
    """The C3 step on the CPU for the first ``sample_T`` tokens: float64 oracle routing (oracle/router.py
    route_fwd), the oracle's capacity drop mask and routed plan (oracle/plan.py), then the permute (gather of
    token rows into expert order) and the weighted combine in float32 torch ops."""
    from oracle import plan as OP
    from oracle import router as OR

    x = inp["x"][:sample_T]
    gw = inp["gate_w"]
    K, E = cfg.K, cfg.E
    cap = OR.capacity_budget(sample_T, K, E, cfg.capacity_factor)

    def rep():
        f = OR.route_fwd(x, gw, K)
        idx = f["idx"]
        v = f["probs"].gather(1, idx)
        wt = (v / v.sum(-1, keepdim=True)).float()
        drop = OP.drop_mask(idx.numpy(), cap)
        pl = OP.plan_routed(idx.numpy(), E, drop)
        R = int(pl["n_rows"])
        rs = torch.from_numpy(pl["row_slot"][:R].astype("int64"))
        xp = x[rs // K].float()  # permute
        sr = torch.from_numpy(pl["slot_row"].astype("int64")).view(-1, K)
        out = torch.zeros(sample_T, x.shape[1])
        for k in range(K):  # combine
            keep = sr[:, k] >= 0
            out[keep] += wt[keep, k:k + 1] * xp[sr[keep, k]]
        return out

    rep()
    times, t0 = [], time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t0 < budget_s and len(times) < 50):
        a = time.perf_counter()
        rep()
        times.append(time.perf_counter() - a)
    mean = sum(times) / len(times)
    std = (sum((t - mean) ** 2 for t in times) / len(times)) ** 0.5
    return {"value": sample_T / mean, "unit": "tokens/s", **cpu_cores(torch), "kind": "port",
            "ms_mean": round(mean * 1e3, 1), "ms_std": round(std * 1e3, 1),
            "sample": f"first {sample_T} tokens of C3: float64 oracle routing + oracle drop mask and routed plan "
                      f"+ float32 torch permute and combine, {len(times)} reps after 1 warmup"}


def add_mfma_ceiling(roof, extra, fp8):
    """The dense MFMA rate this GPU sustains in a memory-free loop of the GEMM's instruction (and the shader
    clock under that load), beside the published peak: ``roof["frac_of_ceiling"]`` is the kernel's share of it."""
    from moe_mi355 import _lib

    peak = MFMA_FP8_PEAK_TFLOPS if fp8 else MFMA_BF16_PEAK_TFLOPS
    tf, mhz = _lib.prof_mfma_ceiling(100000, fp8=fp8)
    tfr, mhzr = _lib.prof_mfma_ceiling(100000, fp8=fp8, random=True)
    roof["ceiling"] = round(tf, 1)
    roof["frac_of_ceiling"] = round(roof["achieved"] / tf, 4)
    roof["ceiling_random_operands"] = round(tfr, 1)
    roof["frac_of_ceiling_random_operands"] = round(roof["achieved"] / tfr, 4)
    extra["mfma_ceiling"] = {"instruction": "v_mfma_scale_f32_32x32x64_f8f6f4" if fp8 else "v_mfma_f32_32x32x16_bf16",
                             "TFLOPs": round(tf, 1), "frac_of_peak": round(tf / peak, 4), "shader_MHz": round(mhz),
                             "random_operands_TFLOPs": round(tfr, 1), "random_operands_frac_of_peak": round(tfr / peak, 4),
                             "random_operands_shader_MHz": round(mhzr)}
    log(f"[bench] MFMA ceiling ({'fp8' if fp8 else 'bf16'}): {tf:.0f} TFLOP/s at {mhz:.0f} MHz; random operands "
        f"{tfr:.0f} TFLOP/s at {mhzr:.0f} MHz")


_HBM_CEILING = {}


def hbm_ceiling(mode, nbytes):
    """GB/s of a plain stream on this GPU (moe_prof_hbm_ceiling): mode 0 read, 1 write, 2 copy of ``nbytes``,
    3 fan-out (``nbytes`` of 4 KB rows each read once and written 6 times).  The working set decides how much the
    256 MB Infinity Cache serves, so each caller sizes the stream like the kernel it is compared with."""
    from moe_mi355 import _lib

    key = (mode, int(nbytes))
    if key not in _HBM_CEILING:
        _HBM_CEILING[key] = round(_lib.prof_hbm_ceiling(int(nbytes), mode), 1)
    return _HBM_CEILING[key]


def add_hbm_ceiling_dispatch(res):
    """The permute reads the token rows once and writes each to its K rows: its practical ceiling is the fan-out
    stream over the same rows (C3: 268 MB in, 1.6 GB out), reported beside the 8 TB/s peak."""
    xb = res["tokens"] * res["d_model"] * 2
    c = {"fanout6": hbm_ceiling(3, xb), "write": hbm_ceiling(1, 6 * xb), "read": hbm_ceiling(0, xb)}
    log(f"[bench] HBM stream ceilings at C3 sizes (GB/s): {c}")
    res["hbm_ceiling_GBps"] = c
    roof = res["roofline"]
    roof["ceiling"] = c["fanout6"]
    roof["ceiling_kind"] = "fan-out stream over the same rows (each read once, written 6 times)"
    roof["frac_of_ceiling"] = round(roof["achieved"] / c["fanout6"], 4)


def add_hbm_ceiling_router(res):
    """The router step reads x (forward) and reads x + writes dx (backward): its stream floor is that read at a plain
    read stream's rate plus that copy at a plain copy stream's rate, over buffers of x's size."""
    xb = res["tokens"] * res["d_model"] * 2
    c = {"read": hbm_ceiling(0, xb), "copy": hbm_ceiling(2, xb)}
    log(f"[bench] HBM stream ceilings at the router's size (GB/s): {c}")
    res["hbm_ceiling_GBps"] = c
    floor_us = xb / (c["read"] * 1e3) + 2 * xb / (c["copy"] * 1e3)
    res["stream_floor_us"] = round(floor_us, 1)
    res["graph_frac_of_stream_floor"] = round(floor_us / (res["graph_ms_per_step"] * 1e3), 4)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="layer", choices=["layer", "c4", "c4_f32", "router", "c1", "norm_router", "dispatch", "skewed", "fp8_fwd", "all"])
    ap.add_argument("--layout", default="reference", choices=["reference", "routed"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run one 1 GiB device copy first (the size reference for HBM counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the expert-parallel "
              "all-to-all is out of scope), so --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    torch.set_num_threads(cpu_thread_count())
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    from moe_mi355 import configs

    log(f"[bench] workload={args.workload} steps={args.steps} warmup={args.warmup}")
    if args.copy_probe:
        copy_probe(torch)
    extra = {}
    with_cpu = not args.no_cpu_baseline
    if args.workload in ("layer", "all"):
        # every config of the benchmark: C4 (the headline line), C2, C1, the fused norm, fp8, C3, C5
        log("[bench] generating C4 inputs")
        inp = configs.layer_inputs(configs.C4)
        main_res = run_layer(args, torch, configs.C4, args.layout, inp, default_numerics=True)
        log(f"[bench] layer: {main_res['ms_per_step']:.3f} ms/step")
        extra["router"] = run_router(args, torch)
        log(f"[bench] router: {extra['router']['ms_per_step']:.4f} ms/step")
        extra["c1"] = run_c1(args, torch, with_cpu=with_cpu)
        log(f"[bench] C1 router: {extra['c1']['ms_mean']:.4f} ms/step")
        extra["norm_router"] = run_norm_router(args, torch)
        log(f"[bench] norm_router: {extra['norm_router']['ms_per_step']:.4f} ms/step")
        extra["c4_f32"] = run_layer(args, torch, configs.C4_F32, args.layout, inp)
        log(f"[bench] C4 layer in fp32: {extra['c4_f32']['ms_per_step']:.2f} ms/step")
        extra["fp8_fwd"] = run_fp8_fwd(args, torch, inp)
        add_mfma_ceiling(extra["fp8_fwd"]["roofline"], extra["fp8_fwd"], fp8=True)
        log(f"[bench] fp8 forward: {extra['fp8_fwd']['fp8_ms_per_step']:.3f} ms/step "
            f"(bf16 forward {extra['fp8_fwd']['bf16_ms_per_step']:.3f})")
        log("[bench] CPU baselines (C4 layer sample, C2 router sample)")
        cpu = cpu_baseline_layer(torch, configs.C4, args.layout, inp) if with_cpu else None
        del inp
        if with_cpu:
            extra["router"]["cpu_baseline"] = cpu_baseline_router(torch)
        extra["dispatch"] = run_dispatch(args, torch, with_cpu=with_cpu)
        log(f"[bench] C3 dispatch: {extra['dispatch']['ms_per_step']:.4f} ms/step")
        add_hbm_ceiling_dispatch(extra["dispatch"])
        add_hbm_ceiling_router(extra["router"])
        log("[bench] generating C5 inputs")
        inp5 = configs.layer_inputs(configs.C5)
        extra["skewed"] = run_layer(args, torch, configs.C5, "routed", inp5)
        log(f"[bench] C5 skewed layer: {extra['skewed']['ms_per_step']:.3f} ms/step")
        if with_cpu:
            extra["skewed"]["cpu_baseline"] = cpu_baseline_layer(torch, configs.C5, "routed", inp5, sample_T=64,
                                                                 budget_s=6.0, min_reps=2)
        del inp5
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        add_mfma_ceiling(roof, extra, fp8=False)
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "ffn", "top_k")}
        config["layout"] = args.layout
    elif args.workload == "c4":
        # the headline leg alone (as in the default run)
        inp = configs.layer_inputs(configs.C4)
        main_res = run_layer(args, torch, configs.C4, args.layout, inp, default_numerics=True)
        cpu = cpu_baseline_layer(torch, configs.C4, args.layout, inp) if with_cpu else None
        del inp
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        add_mfma_ceiling(roof, extra, fp8=False)
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "ffn", "top_k")}
        config["layout"] = args.layout
    elif args.workload == "c4_f32":
        main_res = run_layer(args, torch, configs.C4_F32, args.layout, configs.layer_inputs(configs.C4))
        cpu = None
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "ffn", "top_k")}
    elif args.workload == "router":
        main_res = run_router(args, torch)
        add_hbm_ceiling_router(main_res)
        cpu = None if args.no_cpu_baseline else cpu_baseline_router(torch)
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "top_k")}
    elif args.workload == "norm_router":
        main_res = run_norm_router(args, torch)
        cpu = None
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "top_k")}
    elif args.workload == "fp8_fwd":
        main_res = run_fp8_fwd(args, torch, configs.layer_inputs(configs.C4))
        cpu = None
        value, unit, ms = main_res["fp8_tokens_per_s"], "tokens/s", main_res["fp8_ms_per_step"]
        roof = main_res.pop("roofline")
        add_mfma_ceiling(roof, extra, fp8=True)
        config = {"workload": main_res.pop("workload"), "tokens": main_res.pop("tokens")}
    elif args.workload == "dispatch":
        main_res = run_dispatch(args, torch, with_cpu=with_cpu)
        add_hbm_ceiling_dispatch(main_res)
        cpu = main_res.pop("cpu_baseline", None)
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "top_k")}
    elif args.workload == "c1":
        main_res = run_c1(args, torch, with_cpu=with_cpu)
        cpu = main_res.pop("cpu_baseline", None)
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_mean"]
        roof = None
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "top_k")}
    else:
        inp = configs.layer_inputs(configs.C5)
        main_res = run_layer(args, torch, configs.C5, "routed", inp)
        cpu = cpu_baseline_layer(torch, configs.C5, "routed", inp, sample_T=64) if with_cpu else None
        value, unit, ms = main_res["tokens_per_s"], "tokens/s", main_res["ms_per_step"]
        roof = main_res.pop("roofline")
        config = {k: main_res.pop(k) for k in ("workload", "tokens", "d_model", "experts", "ffn", "top_k")}
    main_res.pop("ms_per_step", None)
    main_res.pop("tokens_per_s", None)
    out = {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"fp8_fwd": "fp8-e4m3", "c1": "f32", "c4_f32": "f32"}.get(args.workload, "bf16"),
        "data": "synthetic (seeded randn of the BASELINE config shapes; random-init weights)", "config": config,
        "roofline": roof, "cpu_baseline": cpu,
    }
    out.update(main_res)
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
