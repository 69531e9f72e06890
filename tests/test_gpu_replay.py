"""HIP-graph capture of the fused SBDA forward and backward.

Callers that launch the attention from a captured graph (a training step
replayed with hipGraphLaunch instead of re-issuing every launch) need the
entry points to be capturable: every launch on the caller's current stream,
no host synchronisation with host-side offsets, no memset nodes, outputs
and workspace from the caller's allocator.  The graph is replayed several
times with eager work and synchronisations in between, and every replay must
reproduce the eager results bit for bit (the kernels are deterministic).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _offsets(layer: int) -> tuple[int, ...]:
    jump = 1 << (layer - 1)
    return (0, jump) if layer <= 2 else (0, 1, 2, jump)


def test_captured_forward_backward_replays_match_eager(sbda):
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)
    b, t, h, d = 2, 4096, 8, 64
    print(f"graph replay: B={b} T={t} H={h} D={d} bf16, layers 1, 3, 9", flush=True)
    q, k, v, go = (torch.randn(b, t, h, d, generator=gen, device=dev)
                   .to(torch.bfloat16).permute(0, 2, 1, 3) for _ in range(4))
    # Far-free walk, transposed chain (F = 4), row chain (F = 256).
    layers = (1, 3, 9)

    def run():
        res = []
        for layer in layers:
            offs = _offsets(layer)
            out, lse = sbda.sbda_forward(q, k, v, offs)
            res += [out, lse, *sbda.sbda_backward(q, k, v, go, lse, offs)]
        return res

    eager = [x.clone() for x in run()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    torch.cuda.synchronize()

    for rep in range(4):
        # Eager work between replays: wipe the graph's outputs and run
        # another layer outside the graph.
        for x in captured:
            x.fill_(0)
        sbda.sbda_forward(q, k, v, _offsets(5 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), f"replay {rep}, output {i}"


def test_captured_prologue_autograd_replays_match_eager(sbda):
    """The fused norm + RoPE route through autograd: forward and backward
    (including the norm-weight gradients) captured as one graph."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(6)
    b, t, h, d = 2, 4096, 8, 64
    print(f"graph replay, prologue: B={b} T={t} H={h} D={d} bf16, layers 1, 4, 9", flush=True)
    q, k, v, go = (torch.randn(b, t, h, d, generator=gen, device=dev)
                   .to(torch.bfloat16).permute(0, 2, 1, 3) for _ in range(4))
    q, k, v = (x.detach().requires_grad_() for x in (q, k, v))
    wq = (1 + 0.1 * torch.randn(d, generator=gen, device=dev)).requires_grad_()
    wk = (1 + 0.1 * torch.randn(d, generator=gen, device=dev)).requires_grad_()
    # Far-free fused backward, two-pass backward (F = 8), row chain (F = 256).
    layers = (1, 4, 9)

    def run():
        res = []
        for layer in layers:
            out = sbda.fused_sbda_prologue(q, k, v, _offsets(layer), wq, wk, theta=10000.0)
            res += [out, *torch.autograd.grad(out, (q, k, v, wq, wk), go)]
        return res

    eager = [x.detach().clone() for x in run()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = [x.detach() for x in run()]
    torch.cuda.synchronize()

    for rep in range(4):
        for x in captured:
            x.fill_(0)
        sbda.sbda_forward(q.detach(), k.detach(), v.detach(), _offsets(5 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), f"replay {rep}, output {i}"
