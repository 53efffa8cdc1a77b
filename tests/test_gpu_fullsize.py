"""Parity at the full benchmark shapes.

Operands are generated on the GPU (seeded), packed by the library, and the
whole shape runs through the C ABI. The oracle then recomputes a sample of
rows from the same packed operands: every stage on this path is row-local
(the quantizer, the GEMM epilogue, each token's routing, experts and
combine), so a sampled row must match bit for bit. Routing and grouping are
cheap on the CPU and are checked for every token.

Shapes: the dense INT4 GEMM M4096 K4096 N12288; the dense INT4 MLP M4096
(gate/up K4096 N12288 each, down K12288 N4096); attention projections
M16384 (4096->4096 and 4096->1024); the Omni MoE layer at 4096 tokens; and a
skewed 65536-token MoE with eight experts never chosen and one expert
holding tens of thousands of rows.
"""
import numpy as np
import pytest
import torch

import clef_i4
import oracle

pytestmark = pytest.mark.gpu


def randn_bf16(shape, std, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std).to(torch.bfloat16)


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_weight(w: clef_i4.QuantizedWeight):
    return w.codes.cpu().numpy().view(np.uint32), w.scales.cpu().numpy()


def sample_rows(m: int, count: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    picks = rng.choice(m, size=count - 4, replace=False)
    return np.unique(np.concatenate([[0, 1, m - 2, m - 1], picks]))


def assert_rows(got: np.ndarray, want: np.ndarray, rows: np.ndarray, what: str):
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)
        r, c = bad[0]
        raise AssertionError(f"{what}: {len(bad)} mismatches, first at sampled row {rows[r]} col {c}: "
                             f"got {got[r, c]:#06x} want {want[r, c]:#06x}")


def check_prepared_rows(a: clef_i4.Prepared, x_rows: np.ndarray, rows: np.ndarray):
    codes, scales, _ = oracle.prepare(x_rows, a.stride, a.bits)
    words = a.width * a.bits // 32
    got = a.codes[torch.from_numpy(rows).cuda()].cpu().numpy().view(np.uint32)[:, :words]
    assert np.array_equal(got, codes[:, :words]), "prepared codes"
    got_s = a.scales[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.array_equal(got_s.view(np.uint32), scales.view(np.uint32)), "prepared scales"


def check_packed_blocks(w_dev: torch.Tensor, qw: clef_i4.QuantizedWeight):
    """First and last 128-row blocks of the GPU-packed weight against the
    oracle's packing of the same bf16 rows (tiles of 128 rows are contiguous
    in the tiled layout, kernels/retile_codes.loom:2-5)."""
    n, k = w_dev.shape
    words = 128 * k // 8
    codes = qw.codes.cpu().numpy().view(np.uint32)
    scales = qw.scales.cpu().numpy()
    for b in (0, n // 128 - 1):
        tiled, sc = oracle.pack_weight(u16(w_dev[128 * b: 128 * (b + 1)]))
        assert np.array_equal(codes[b * words: (b + 1) * words], tiled), f"packed block {b}"
        assert np.array_equal(scales[128 * b: 128 * (b + 1)].view(np.uint32), sc.view(np.uint32))


def test_headline_gemm_full_shape():
    """M4096 K4096 N12288, the bench workload: every sampled output row
    bit-exact (kernels/gemm_integer.loom:394-433)."""
    m, k, n = 4096, 4096, 12288
    x = randn_bf16((m, k), 1.0, 1002 * 16 + 0)
    w = randn_bf16((n, k), 0.02, 1002 * 16 + 1)
    qw = clef_i4.load_quantized_weight(w)
    check_packed_blocks(w, qw)
    a = clef_i4.prepare(x)
    out = clef_i4.project_prepared(a, qw)
    rows = sample_rows(m, 40, 1)
    x_rows = u16(x[torch.from_numpy(rows).cuda()])
    check_prepared_rows(a, x_rows, rows)
    codes, scales, _ = oracle.prepare(x_rows, a.stride)
    want = oracle.gemm(codes, scales, *host_weight(qw), n, k)
    assert_rows(u16(out[torch.from_numpy(rows).cuda()]), want, rows, "gemm 4096x4096x12288")
    # every configuration agrees with the default one at the full shape
    for cfg in range(clef_i4.gemm_configs()):
        other = clef_i4.project_prepared(a, qw, config=cfg)
        assert torch.equal(other.view(torch.int16), out.view(torch.int16)), f"config {cfg}"
    # the bf6 form of the same codes (the benchmark kernel: 48 column tiles,
    # several tiles per workgroup), whole output bit for bit
    f6 = clef_i4.project_f6(clef_i4.prepare_f6(x), clef_i4.f6_weight(qw))
    assert torch.equal(f6.view(torch.int16), out.view(torch.int16)), "bf6 GEMM 4096x4096x12288"


@pytest.mark.parametrize("n", [4096, 1024])
def test_attention_projection_full_shape(n):
    """M16384 K4096 with N 4096 (Q/O) and 1024 (K/V), sampled rows."""
    m, k = 16384, 4096
    x = randn_bf16((m, k), 1.0, 1003 * 16 + 0)
    w = randn_bf16((n, k), 0.02, 1003 * 16 + (1 if n == 4096 else 2))
    qw = clef_i4.load_quantized_weight(w)
    res = randn_bf16((m, n), 1.0, 1003 * 16 + 3)
    a = clef_i4.prepare(x)
    out = clef_i4.project_prepared(a, qw, residual=res)
    rows = sample_rows(m, 24, n)
    idx = torch.from_numpy(rows).cuda()
    codes, scales, _ = oracle.prepare(u16(x[idx]), a.stride)
    want = oracle.gemm(codes, scales, *host_weight(qw), n, k, residual=u16(res[idx]))
    assert_rows(u16(out[idx]), want, rows, f"projection 16384x4096x{n} + residual")
    f6 = clef_i4.project_f6(clef_i4.prepare_f6(x), clef_i4.f6_weight(qw), residual=res)
    assert torch.equal(f6.view(torch.int16), out.view(torch.int16)), f"bf6 projection 16384x4096x{n} + residual"


def test_dense_mlp_full_shape():
    """Dense INT4 MLP at M4096 D4096 F12288: Q1(x) -> G1 gate, G1 up ->
    fused SwiGLU+Q1 (prepare_with_inputs, src/quantized.rs:605-613) -> G1 down."""
    m, d, f = 4096, 4096, 12288
    x = randn_bf16((m, d), 1.0, 1002 * 16 + 0)
    wg = clef_i4.load_quantized_weight(randn_bf16((f, d), 0.02, 1002 * 16 + 2))
    wu = clef_i4.load_quantized_weight(randn_bf16((f, d), 0.02, 1002 * 16 + 3))
    wd = clef_i4.load_quantized_weight(randn_bf16((d, f), 0.02, 1002 * 16 + 4))
    a = clef_i4.prepare(x)
    gate = clef_i4.project_prepared(a, wg)
    up = clef_i4.project_prepared(a, wu)
    h = clef_i4.prepare_swiglu(gate, up)
    y = clef_i4.project_prepared(h, wd)
    rows = sample_rows(m, 16, 7)
    idx = torch.from_numpy(rows).cuda()
    codes, scales, _ = oracle.prepare(u16(x[idx]), a.stride)
    g_want = oracle.gemm(codes, scales, *host_weight(wg), f, d)
    u_want = oracle.gemm(codes, scales, *host_weight(wu), f, d)
    assert_rows(u16(gate[idx]), g_want, rows, "mlp gate")
    assert_rows(u16(up[idx]), u_want, rows, "mlp up")
    h_codes, h_scales, _ = oracle.prepare_swiglu(g_want, u_want, h.stride)
    y_want = oracle.gemm(h_codes, h_scales, *host_weight(wd), d, f)
    assert_rows(u16(y[idx]), y_want, rows, "mlp down")
    # the same block on the bf6 form of the codes (as the benchmark runs it),
    # every stage's whole output bit for bit
    af = clef_i4.prepare_f6(x)
    g6 = clef_i4.project_f6(af, clef_i4.f6_weight(wg))
    u6 = clef_i4.project_f6(af, clef_i4.f6_weight(wu))
    assert torch.equal(g6.view(torch.int16), gate.view(torch.int16)), "bf6 mlp gate"
    assert torch.equal(u6.view(torch.int16), up.view(torch.int16)), "bf6 mlp up"
    y6 = clef_i4.project_f6(clef_i4.prepare_swiglu_f6(g6, u6), clef_i4.f6_weight(wd))
    assert torch.equal(y6.view(torch.int16), y.view(torch.int16)), "bf6 mlp down"
    # the fused gate/up + SwiGLU GEMM (the benchmark's block): h bit for bit
    # the SwiGLU of the separate projections, and the block output unchanged
    hf = clef_i4.project_gate_up_f6(af, clef_i4.f6_weight(wg), clef_i4.f6_weight(wu))
    assert torch.equal(hf.view(torch.int16), clef_i4.swiglu(gate, up).view(torch.int16)), "fused gate/up h"
    yf = clef_i4.project_f6(clef_i4.prepare_f6(hf), clef_i4.f6_weight(wd))
    assert torch.equal(yf.view(torch.int16), y.view(torch.int16)), "fused mlp down"


def skewed_logits(tokens: int, seed: int) -> torch.Tensor:
    """Router logits N(0,1) + bias_e, bias_e = -1.1 * 0.57 * ln(1 + rank(e))
    for a seeded rank permutation (seed 55); the eight lowest-ranked experts
    get -30 and are never chosen."""
    rank = np.random.default_rng(55).permutation(128)
    bias = -1.1 * 0.57 * np.log1p(rank)
    bias[rank >= 120] = -30.0
    g = torch.Generator(device="cuda").manual_seed(seed)
    z = torch.randn((tokens, 128), generator=g, device="cuda", dtype=torch.float32)
    return (z + torch.from_numpy(bias.astype(np.float32)).cuda()).to(torch.bfloat16)


def run_moe(tokens: int, logits: torch.Tensor, seed: int, sample: int):
    d, inter = 2048, 768
    x = randn_bf16((tokens, d), 1.0, seed * 16 + 0)
    gate = clef_i4.load_quantized_weight(randn_bf16((128 * inter, d), 0.02, seed * 16 + 2))
    up = clef_i4.load_quantized_weight(randn_bf16((128 * inter, d), 0.02, seed * 16 + 3))
    down = clef_i4.load_quantized_weight(randn_bf16((128 * d, inter), 0.02, seed * 16 + 4))
    layer = clef_i4.MoeLayer(gate, up, down)
    routes = torch.empty((tokens, 16), dtype=torch.float32, device="cuda")
    out = layer(x, logits, routes_out=routes)
    torch.cuda.synchronize()

    # routing and grouping of every token
    logits_h = u16(logits)
    want_routes = oracle.route(logits_h, 8)
    got_routes = routes.cpu().numpy()
    assert np.array_equal(got_routes.view(np.uint32), want_routes.view(np.uint32)), "routes"
    groups, order = clef_i4.omni_group_routes(routes)
    want_groups, want_order = oracle.group_routes(want_routes)
    g = groups.cpu().numpy()
    assert np.array_equal(g[:, 0], want_groups[:, 0]), "expert counts"
    for e in range(128):
        c = int(want_groups[e, 0])
        assert np.array_equal(g[e, 1:1 + c], want_groups[e, 1:1 + c]), f"expert {e} rows"
    assert np.array_equal(order.cpu().numpy(), want_order), "order"

    # sampled tokens through the whole layer, plus the tokens of the busiest expert
    rows = sample_rows(tokens, sample, tokens)
    busiest = int(np.argmax(want_groups[:, 0]))
    last = int(want_groups[busiest, int(want_groups[busiest, 0])]) // 8
    rows = np.unique(np.concatenate([rows, [last]]))
    idx = torch.from_numpy(rows).cuda()
    want, r = oracle.moe_layer(u16(x[idx]), logits_h[rows], host_weight(gate), host_weight(up),
                               host_weight(down))
    assert np.array_equal(r.view(np.uint32), want_routes[rows].view(np.uint32))
    assert_rows(u16(out[idx]), want, rows, f"moe layer tokens={tokens}")
    return want_groups


def test_moe_layer_full_shape():
    """Omni INT4 MoE at 4096 tokens, 128 experts, top-8 (src/omni.rs:762-857)."""
    logits = randn_bf16((4096, 128), 1.0, 1004 * 16 + 1)
    run_moe(4096, logits, 1004, 24)


def test_moe_layer_skewed_65536_tokens():
    """65536 tokens with skewed routing: eight empty experts and one expert
    with tens of thousands of rows (hundreds of row tiles)."""
    groups = run_moe(65536, skewed_logits(65536, 1005 * 16 + 1), 1005, 12)
    counts = groups[:, 0]
    assert (counts == 0).sum() >= 8
    assert counts.max() > 20000


@pytest.mark.parametrize("tokens,skewed", [(32768, False), (40000, True)])
def test_expert_down_matches_row_halves(tokens, skewed):
    """The routed expert GEMM at the down projection's shape (K 768 -> N 2048,
    top-8) over 262144 and 320000 routed rows. E1 is row-local, so the whole
    output for `tokens` tokens must equal the outputs for the first and the
    second half of the tokens computed separately (their own groupings and
    tile schedules), bit for bit; a sample of tokens is also checked against
    the oracle's E1 (src/omni.rs:289-534, input_routed)."""
    seed = 1006 + int(skewed)
    d, inter, topk = 2048, 768, 8
    logits = skewed_logits(tokens, seed * 16 + 1) if skewed else randn_bf16((tokens, 128), 1.0, seed * 16 + 1)
    routes = clef_i4.omni_route(logits, topk)
    h = randn_bf16((tokens * topk, inter), 1.0, seed * 16 + 2)
    down = clef_i4.load_quantized_weight(randn_bf16((128 * d, inter), 0.02, seed * 16 + 3))
    groups, _ = clef_i4.omni_group_routes(routes)
    full = clef_i4.omni_expert(clef_i4.prepare(h), down, groups, tokens, topk, True)
    half = tokens // 2
    parts = []
    for lo, hi in ((0, half), (half, tokens)):
        g, _ = clef_i4.omni_group_routes(routes[lo:hi].contiguous())
        a = clef_i4.prepare(h[lo * topk: hi * topk].contiguous())
        parts.append(clef_i4.omni_expert(a, down, g, hi - lo, topk, True))
    torch.cuda.synchronize()
    assert torch.equal(full.view(torch.int16), torch.cat(parts).view(torch.int16)), "whole against halves"
    del parts

    rows = sample_rows(tokens, 64, seed)
    slots = (rows[:, None] * topk + np.arange(topk)[None, :]).ravel()
    sub_routes = routes[torch.from_numpy(rows).cuda()].cpu().numpy()
    sub_groups, _ = oracle.group_routes(sub_routes)
    stride = oracle.activation_stride(inter)
    codes, scales, _ = oracle.prepare(u16(h[torch.from_numpy(slots).cuda()]), stride)
    w_codes, w_scales = host_weight(down)
    want = oracle.expert_i4(codes, scales, w_codes, w_scales, sub_groups, len(rows), topk, inter, d, True)
    got = u16(full[torch.from_numpy(slots).cuda()])
    assert_rows(got, want, slots, f"routed expert GEMM tokens={tokens}")
