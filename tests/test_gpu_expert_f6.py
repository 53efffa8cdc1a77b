"""The grouped expert GEMMs on the bf6 form of the INT4 codes against the
oracle's E1 (and E1, E1, S1 for the fused gate/up), bit for bit, and against
the INT4 entry points on the same operands. Activations come from the bf6
quantizer (clef_i4_prepare_f6), weights from clef_i4_f6_weight of the tiled
expert weights: the same codes and scales as the INT4 path.

Cases follow the reference's expert tests (src/omni.rs:946-1051,
src/benchmarking/omni.rs:328-356): skewed routes leaving experts empty,
partial and many tiles long, routed (down) and token (gate/up) inputs.
"""
import numpy as np
import pytest
import torch

import clef_i4
import oracle
from test_gpu_parity import (assert_same_bf16_nan_aware, assert_same_u16, bf16_host, dev_weight,
                             packed_experts, randn_bf16, random_routes, to_dev_bf16, to_dev_f32)

pytestmark = pytest.mark.gpu


def f6_operands(x, w_t, w_s, n_rows, k):
    a = clef_i4.prepare_f6(to_dev_bf16(x))
    w = clef_i4.f6_weight(dev_weight(w_t, w_s, n_rows, k))
    return a, w


@pytest.mark.parametrize("tokens,k,n,routed,skew", [
    (300, 768, 512, True, 2.0),    # the down projection's K (six half-steps)
    (600, 512, 1024, False, 0.0),  # the shortest K the kernel takes (four half-steps)
    (1000, 1024, 512, True, 4.0),  # skewed: some experts span many tiles, others are empty
    (3, 512, 256, False, 0.0),     # 24 routes: one partial tile per expert hit
    (257, 2048, 256, False, 1.0),
])
def test_expert_f6_matches_oracle(tokens, k, n, routed, skew):
    rng = np.random.default_rng(31 * tokens + k + n)
    topk = 8
    routes = random_routes(rng, tokens, skew=skew)
    groups, _ = oracle.group_routes(routes)
    rows = tokens * topk if routed else tokens
    x = randn_bf16(rng, (rows, k))
    sx = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, sx)
    w_t, w_s = packed_experts(rng, n, k)
    want = oracle.expert_i4(codes, scales, w_t, w_s, groups, tokens, topk, k, n, routed)
    a, w = f6_operands(x, w_t, w_s, 128 * n, k)
    g = to_dev_f32(groups)
    got = clef_i4.omni_expert_f6(a, w, g, tokens, topk, routed)
    assert_same_u16(bf16_host(got), want, f"bf6 expert tokens={tokens} k={k} n={n} routed={routed}")
    again = clef_i4.omni_expert_f6(a, w, g, tokens, topk, routed)
    assert torch.equal(again.view(torch.int16), got.view(torch.int16))


@pytest.mark.parametrize("tokens,k,n,skew,wide", [
    (600, 2048, 768, 0.0, False),  # the Omni gate/up shape: K 2048, 768 columns
    (700, 768, 256, 3.0, False),
    (3, 512, 256, 0.0, False),
    (300, 512, 512, 2.0, True),    # gate scales over 82 decades: every SiLU range and overflow
])
def test_expert_gate_up_f6_matches_oracle(tokens, k, n, skew, wide):
    rng = np.random.default_rng(13 * tokens + k + n + int(wide))
    topk = 8
    routes = random_routes(rng, tokens, skew=skew)
    groups, _ = oracle.group_routes(routes)
    x = randn_bf16(rng, (tokens, k))
    sx = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, sx)
    gw, gs = packed_experts(rng, n, k)
    uw, us = packed_experts(rng, n, k)
    if wide:
        gs = (10.0 ** rng.uniform(-44, 38, size=gs.shape)).astype(np.float32)
    g = oracle.expert_i4(codes, scales, gw, gs, groups, tokens, topk, k, n, False)
    u = oracle.expert_i4(codes, scales, uw, us, groups, tokens, topk, k, n, False)
    want = oracle.swiglu(g, u)
    a = clef_i4.prepare_f6(to_dev_bf16(x))
    gw_d = clef_i4.f6_weight(dev_weight(gw, gs, 128 * n, k))
    uw_d = clef_i4.f6_weight(dev_weight(uw, us, 128 * n, k))
    got = clef_i4.omni_gate_up_f6(a, gw_d, uw_d, to_dev_f32(groups), tokens, topk)
    if wide:
        # inf * 0 where overflowing gates meet zero up values: NaN payload
        # signs differ between the host oracle and the GPU
        assert_same_bf16_nan_aware(bf16_host(got), want, "bf6 gate/up, wide scales")
    else:
        assert_same_u16(bf16_host(got), want, f"bf6 gate/up tokens={tokens} k={k} n={n}")
    again = clef_i4.omni_gate_up_f6(a, gw_d, uw_d, to_dev_f32(groups), tokens, topk)
    assert torch.equal(again.view(torch.int16), got.view(torch.int16))


def random_expert_weight(gen, rows, k):
    """Random tiled INT4 codes (every nibble pattern, -8 included) and scales."""
    words = torch.randint(-2**31, 2**31 - 1, (rows * k // 8,), dtype=torch.int32, device="cuda", generator=gen)
    scales = torch.rand(rows, dtype=torch.float32, device="cuda", generator=gen) * 0.01 + 1e-4
    return clef_i4.QuantizedWeight(words, scales, rows, k, oracle.activation_stride(k), 4)


@pytest.mark.parametrize("tokens,skew", [(4096, 1.0), (4100, 0.0)])
def test_expert_f6_equals_int4_at_omni_shape(tokens, skew):
    """The Omni layer's expert GEMMs at 4096 tokens (gate/up K 2048 -> 768
    columns, down K 768 -> 2048 columns) through the bf6 and the INT4 entry
    points on the same codes: equal bit for bit, whole outputs."""
    rng = np.random.default_rng(tokens)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(tokens)
    topk, hidden, inter = 8, 2048, 768
    routes = random_routes(rng, tokens, skew=skew)
    groups, _ = oracle.group_routes(routes)
    g = to_dev_f32(groups)
    x = torch.randn((tokens, hidden), device="cuda", generator=gen).to(torch.bfloat16)
    gq, uq = random_expert_weight(gen, 128 * inter, hidden), random_expert_weight(gen, 128 * inter, hidden)
    h_i4 = clef_i4.omni_gate_up(clef_i4.prepare(x), gq, uq, g, tokens, topk)
    h_f6 = clef_i4.omni_gate_up_f6(clef_i4.prepare_f6(x), clef_i4.f6_weight(gq), clef_i4.f6_weight(uq), g,
                                   tokens, topk)
    assert torch.equal(h_f6.view(torch.int16), h_i4.view(torch.int16))
    dq = random_expert_weight(gen, 128 * hidden, inter)
    y_i4 = clef_i4.omni_expert(clef_i4.prepare(h_i4), dq, g, tokens, topk, True)
    y_f6 = clef_i4.omni_expert_f6(clef_i4.prepare_f6(h_f6), clef_i4.f6_weight(dq), g, tokens, topk, True)
    assert torch.equal(y_f6.view(torch.int16), y_i4.view(torch.int16))


def test_expert_f6_rejects_short_k():
    """K below 512 (four 128-k half-steps) is refused with the INT4 entry's
    shape message, before any launch."""
    rng = np.random.default_rng(5)
    tokens, k, n = 16, 256, 256
    groups, _ = oracle.group_routes(random_routes(rng, tokens))
    x = randn_bf16(rng, (tokens, k))
    w_t, w_s = packed_experts(rng, n, k)
    a, w = f6_operands(x, w_t, w_s, 128 * n, k)
    with pytest.raises(clef_i4.ClefError, match="unsupported Omni expert tile shape"):
        clef_i4.omni_expert_f6(a, w, to_dev_f32(groups), tokens, 8, False)
