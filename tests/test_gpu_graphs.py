"""The front-end's Hessian-vector product captured in a HIP graph.

The kernels allocate nothing, synchronise nothing and record no memset, so a
whole HVP (forward, first backward, double backward and the autograd glue
between them) can be captured with torch.cuda.graph and replayed; at small
shapes that removes the host overhead that dominates the eager HVP. The HVP is
written as two vector-Jacobian products (no reduction kernel in the graph).

Each replay is checked against the eager result on the same inputs, with other
eager work and synchronisations between replays and new values copied into the
static inputs, for several replays.
"""

from __future__ import annotations

import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu


def hvp(x, cot, tan, causal_alignment="top_left"):
    import flash_hog

    x = [t.detach().requires_grad_(True) for t in x]
    out = flash_hog.dot_product_attention(*x, is_causal=True, causal_alignment=causal_alignment)
    g = torch.autograd.grad(out, x, cot, create_graph=True)
    return torch.autograd.grad(g, x, tan)


def _draw(seed, B, Nq, Nk, H, Hk, D, device):
    d = make_inputs(B, Nq, Nk, H, D, torch.bfloat16, seed=seed, kv_heads=Hk, device=device)
    return [d["q"], d["k"], d["v"]], d["do"], [d["ddq"], d["ddk"], d["ddv"]]


@pytest.mark.parametrize("shape,alignment", [((1, 512, 512, 4, 2, 64), "top_left"),
                                             ((2, 200, 320, 4, 4, 64), "bottom_right")],
                         ids=["gqa_512", "ragged_bottom_right"])
def test_hvp_graph_replays_match_eager(shape, alignment, cuda_device):
    print("[case] graph hvp", shape, alignment, flush=True)
    x, cot, tan = _draw(61, *shape, cuda_device)
    static = [t.clone() for t in x + [cot] + tan]
    sx, scot, stan = static[:3], static[3], static[4:]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            hvp(sx, scot, stan, alignment)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = hvp(sx, scot, stan, alignment)
    torch.cuda.synchronize()

    for replay in range(4):
        new_x, new_cot, new_tan = _draw(100 + replay, *shape, cuda_device)
        for dst, src in zip(static, new_x + [new_cot] + new_tan):
            dst.copy_(src)
        eager = hvp(new_x, new_cot, new_tan, alignment)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b, n in zip(static_out, eager, ("q", "k", "v")):
            assert torch.equal(a, b), f"replay {replay}: HVP wrt {n} differs from eager"
