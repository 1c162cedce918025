"""The router step and a layer step captured as HIP graphs (torch.cuda.graph) and replayed: every replay,
with eager work and synchronisations between the replays, reproduces the eager step bit for bit.  The
kernels' reductions run in a fixed order and the router's ticket workspace is zeroed by a captured fill
kernel (no memset node), so a replay has nothing that could differ from the eager call.

Every step, eager or captured, runs on one side stream.  A leaf's gradient accumulator is bound to the stream
it was made on, and the layer keeps it alive from one step to the next (``router.last_aux_loss`` holds the
step's autograd graph): an accumulator made by an eager step on another stream would make the captured
backward synchronise with that stream, which a capture cannot hold."""

from __future__ import annotations

import pytest
import torch

from gpu_util import dev, say

from moe_mi355.router import RouterCore
from pkg.distributed import build_topology
from pkg.distributed.moe_layer import DistributedMoELayer

pytestmark = pytest.mark.gpu


def _replays_match_eager(step, names) -> None:
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = [t.detach().clone() for t in step()]
        for _ in range(2):  # warm-up
            step()
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        outs = step()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for n, a, b in zip(names, outs, eager):
            assert a.shape == b.shape and a.dtype == b.dtype, f"replay {rep} {n}"
            assert torch.equal(a, b), f"replay {rep} {n}: differs from the eager step"
        with torch.cuda.stream(s):  # eager work between the replays
            step()
        torch.cuda.synchronize()
    del graph


@pytest.mark.parametrize("shape", [(2048, 1024, 8, 2), (1500, 512, 16, 4)], ids=lambda s: f"N{s[0]}-H{s[1]}-E{s[2]}-K{s[3]}")
def test_router_step_graph_replays_match_eager(shape):
    N, H, E, K = shape
    say(f"[graph router] {shape}")
    d = dev()
    g_ = torch.Generator(device=d).manual_seed(N + H)
    x = torch.randn(N, H, device=d, generator=g_).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(H, E, device=d, generator=g_) * 0.05).to(torch.bfloat16).requires_grad_(True)
    gw = torch.randn(N, K, device=d, generator=g_).to(torch.bfloat16)
    one = torch.ones((), device=d)

    def step():
        idx, wt, aux, z, logits, cnt, stats = RouterCore.apply(x, w, K, 0.01, 1e-3, None)
        dx, dw = torch.autograd.grad((wt, aux, z), (x, w), grad_outputs=(gw, one, one))
        return idx, wt, aux, z, logits, cnt, dx, dw

    _replays_match_eager(step, ("idx", "w", "aux", "z", "logits", "cnt", "dx", "dw"))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_layer_step_graph_replays_match_eager(dt):
    """The whole layer step (float32 too: the fp32 grouped GEMM, with no host synchronisation anywhere in the
    step, which capture would reject) replayed as a graph, bit-identical to the eager step."""
    H, Fd, E, K, N = 256, 512, 8, 2, 512
    say(f"[graph layer] H{H} F{Fd} E{E} K{K} N{N} {dt}")
    d = dev()
    torch.manual_seed(7)
    layer = DistributedMoELayer(H, Fd, E, K, build_topology(), dtype=dt, layout="reference",
                                aux_loss_coef=0.01, z_loss_coef=1e-3, check_numerics=False).to(d)
    x = torch.randn(N, H, device=d).to(dt).requires_grad_(True)
    gout = torch.randn(N, H, device=d).to(dt)
    one = torch.ones((), device=d)
    params = [x, layer.router.gate_w, layer.w_gate, layer.w_up, layer.w_down]

    def step():
        out = layer(x)
        grads = torch.autograd.grad([out, layer.router.last_aux_loss, layer.router.last_z_loss], params,
                                    grad_outputs=[gout, one, one])
        return (out,) + tuple(grads)

    _replays_match_eager(step, ("out", "dx", "dgate_w", "dw_gate", "dw_up", "dw_down"))
