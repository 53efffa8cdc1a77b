"""Every entry point is stream-ordered and allocation- and memset-free, so a
caller can capture it into a HIP graph. A graph holding the quantizer, the
dense GEMM and the whole MoE layer is replayed several times with eager work
and synchronizations between replays; every replay must equal the eager
result for the inputs it was given."""
import numpy as np
import pytest
import torch

import clef_i4

pytestmark = pytest.mark.gpu


def randn(shape, std, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


@pytest.mark.parametrize("t,pm,pn", [(4, 4, 1024), (256, 256, 1024), (512, 2048, 6144)])
def test_graph_replays_match_eager(t, pm, pn):
    """4 tokens and a 4 x 1024 projection take the decode kernels (the MoE
    block as two kernels, the dot-product GEMM); 256 tokens and a 256 x 1024
    projection the few-rows kernels (32-slot expert tiles, the K-split GEMM);
    512 tokens and a 2048 x 6144 projection the 128-slot expert kernels and
    the persistent GEMM."""
    d, inter = 512, 256
    gate = clef_i4.load_quantized_weight(randn((128 * inter, d), 0.02, 1))
    up = clef_i4.load_quantized_weight(randn((128 * inter, d), 0.02, 2))
    down = clef_i4.load_quantized_weight(randn((128 * d, inter), 0.02, 3))
    qw = clef_i4.load_quantized_weight(randn((pn, d), 0.02, 4))
    layer = clef_i4.MoeLayer(gate, up, down)
    inputs = [(randn((t, d), 1.0, 10 + i), randn((t, 128), 1.0, 20 + i), randn((pm, d), 1.0, 30 + i))
              for i in range(4)]

    # static buffers the graph reads and writes
    x = inputs[0][0].clone()
    logits = inputs[0][1].clone()
    px = inputs[0][2].clone()
    moe_out = torch.empty((t, d), dtype=torch.bfloat16, device="cuda")
    a = clef_i4.prepare(px)
    proj_out = torch.empty((pm, pn), dtype=torch.bfloat16, device="cuda")

    def step():
        clef_i4.prepare(px, out=a.storage)
        clef_i4.project_prepared(a, qw, out=proj_out)
        layer(x, logits, out=moe_out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # first calls: workspaces and kernel attributes outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()

    for i, (xi, li, pi) in enumerate(inputs * 2):
        want_moe = layer(xi, li)
        want_proj = clef_i4.project_prepared(clef_i4.prepare(pi), qw)
        torch.cuda.synchronize()
        x.copy_(xi)
        logits.copy_(li)
        px.copy_(pi)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(moe_out.view(torch.int16), want_moe.view(torch.int16)), f"replay {i}: MoE layer"
        assert torch.equal(proj_out.view(torch.int16), want_proj.view(torch.int16)), f"replay {i}: projection"
        _ = (moe_out.float().sum() + 1).item()  # eager work between replays
