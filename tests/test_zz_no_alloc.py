"""clef_moe_layer_static, the MoE block that allocates nothing (its
intermediates live in the library's static per-device scratch), against
clef_moe_layer with a caller workspace, both through the C ABI: two calls in
a row, the second with fewer tokens (so the scratch holds the first call's
contents when the second starts), outputs and routes bit for bit; the same
call captured in a HIP graph and replayed; the device's free memory unchanged
by a call."""
import numpy as np
import pytest
import torch

import clef_i4

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # CLEF_MOE_STATIC_SCRATCH_BYTES


def _weight(gen, rows, cols):
    w = (torch.randn((rows, cols), generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    return clef_i4.load_quantized_weight(w)


def _static(layer, x, logits, out, routes):
    lib = clef_i4.lib()
    return lib.clef_moe_layer_static(
        x.data_ptr(), logits.data_ptr(), 0, x.shape[0], layer.hidden, layer.inter, 128, layer.topk,
        layer.gate.codes.data_ptr(), layer.gate.scales.data_ptr(), layer.up.codes.data_ptr(),
        layer.up.scales.data_ptr(), layer.down.codes.data_ptr(), layer.down.scales.data_ptr(),
        routes.data_ptr(), out.data_ptr(), torch.cuda.current_stream().cuda_stream)


def test_static_scratch_layer_matches_workspace_layer():
    d, inter, topk = 2048, 768, 8
    gen = torch.Generator(device="cuda").manual_seed(1004)
    layer = clef_i4.MoeLayer(_weight(gen, 128 * inter, d), _weight(gen, 128 * inter, d),
                             _weight(gen, 128 * d, inter), topk=topk)
    # 600 tokens: 4800 routed rows on the 128-slot expert tiles; 97 tokens:
    # 776 routed rows on the 32-slot tiles; 5 tokens: the two-kernel layer
    # (each call smaller than the last, the scratch holding its contents).
    for tokens in (600, 97, 5):
        print(f"static MoE layer tokens={tokens}", flush=True)
        need = clef_i4.lib().clef_moe_layer_workspace_bytes(tokens, d, inter, topk)
        assert need <= SCRATCH_BYTES, need
        x = torch.randn((tokens, d), generator=gen, device="cuda").to(torch.bfloat16)
        logits = torch.randn((tokens, 128), generator=gen, device="cuda").to(torch.bfloat16)
        want_routes = torch.empty((tokens, 2 * topk), dtype=torch.float32, device="cuda")
        want = layer(x, logits, routes_out=want_routes)
        out = torch.full((tokens, d), -1, dtype=torch.int16, device="cuda").view(torch.bfloat16)
        routes = torch.full((tokens, 2 * topk), -7.0, dtype=torch.float32, device="cuda")
        rc = _static(layer, x, logits, out, routes)
        assert rc == 0, clef_i4.lib().clef_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(routes.view(torch.int32), want_routes.view(torch.int32)), f"routes tokens={tokens}"
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"output tokens={tokens}"


def test_static_scratch_layer_in_a_graph_allocates_nothing():
    """What the entry point is for: a caller that cannot allocate. One call
    captured in a HIP graph (torch.cuda.graph), replayed over changing inputs
    with eager work and synchronizations between the replays; every replay
    equals the workspace path bit for bit. A call after the first on the
    device leaves the device's free memory unchanged (the library reserves
    nothing per call: its scratch is the static array, resident once the
    library's code is loaded)."""
    d, inter, topk, tokens = 2048, 768, 8, 200
    gen = torch.Generator(device="cuda").manual_seed(1005)
    layer = clef_i4.MoeLayer(_weight(gen, 128 * inter, d), _weight(gen, 128 * inter, d),
                             _weight(gen, 128 * d, inter), topk=topk)
    x = torch.randn((tokens, d), generator=gen, device="cuda").to(torch.bfloat16)
    logits = torch.randn((tokens, 128), generator=gen, device="cuda").to(torch.bfloat16)
    out = torch.empty((tokens, d), dtype=torch.bfloat16, device="cuda")
    routes = torch.empty((tokens, 2 * topk), dtype=torch.float32, device="cuda")

    print("static MoE layer: free memory across a call", flush=True)
    assert _static(layer, x, logits, out, routes) == 0, clef_i4.lib().clef_last_error().decode()
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    assert _static(layer, x, logits, out, routes) == 0, clef_i4.lib().clef_last_error().decode()
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before, (free_before, free_after)

    print("static MoE layer: graph capture and replays", flush=True)
    graph = torch.cuda.CUDAGraph()
    rc = []
    with torch.cuda.graph(graph):
        rc.append(_static(layer, x, logits, out, routes))
    assert rc == [0], clef_i4.lib().clef_last_error().decode()
    for replay in range(4):
        x.copy_(torch.randn((tokens, d), generator=gen, device="cuda").to(torch.bfloat16))
        logits.copy_(torch.randn((tokens, 128), generator=gen, device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_routes = torch.empty_like(routes)
        want = layer(x, logits, routes_out=want_routes)
        torch.cuda.synchronize()
        assert torch.equal(routes.view(torch.int32), want_routes.view(torch.int32)), f"routes replay {replay}"
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"output replay {replay}"
