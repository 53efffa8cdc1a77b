"""Fused quantizer producers beyond SwiGLU (kernels/prepare_integer_register.loom):
the attention-gate producer and the named-RMSNorm producer, through the C ABI,
bit for bit against the oracle.
"""
import numpy as np
import pytest
import torch

import clef_i4
import oracle
from test_oracle import norm_test_rows, norm_test_weight

pytestmark = pytest.mark.gpu

BF = oracle.f32_to_bf16


def dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def host_u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def assert_prepared(p: clef_i4.Prepared, codes: np.ndarray, scales: np.ndarray, what: str):
    words = p.width * p.bits // 32
    got = p.codes.cpu().numpy().view(np.uint32)[:, :words]
    if not np.array_equal(got, codes[:, :words]):
        bad = np.argwhere(got != codes[:, :words])
        raise AssertionError(f"{what}: {len(bad)} code words differ, first at {tuple(bad[0])}")
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint32), scales.view(np.uint32)), f"{what}: scales"


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,width", [(1, 256), (17, 768), (5, 2048), (33, 5120), (3, 6144), (2, 17408)])
def test_attention_gate_matches_oracle(rows, width, bits):
    """h3_prepare_attention_gate (src/quantized.rs:440-468, 615-635); both the
    multi-row (width <= 4096) and the one-row-per-workgroup kernels."""
    rng = np.random.default_rng(rows * 7 + width + bits)
    x = BF(rng.standard_normal((rows, width)).astype(np.float32))
    q = BF((rng.standard_normal((rows, 2 * width)) * 3.0).astype(np.float32))
    q[0, 256:256 + 16] = BF(np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 100.0, -100.0, 1e-30] * 2,
                                     dtype=np.float32))
    stride = oracle.activation_stride(width, bits)
    codes, scales, _ = oracle.prepare_attention_gate(x, q, stride, bits)
    p = clef_i4.prepare_attention_gate(dev_bf16(x), dev_bf16(q), bits=bits, stride=stride)
    assert_prepared(p, codes, scales, f"attention gate rows={rows} width={width} bits={bits}")


@pytest.mark.parametrize("store", [False, True])
@pytest.mark.parametrize("exceptional", [False, True])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows", [1, 2, 7, 65, 129])
def test_norm_matches_oracle(rows, bits, exceptional, store):
    """h3_prepare_norm[_store] on the inputs of the reference's fused-norm test
    (src/quantized.rs:1567-1610): codes, scales and stored normalized rows."""
    x = norm_test_rows(rows)
    w = norm_test_weight(exceptional=exceptional)
    stride = 5120 + 512 // bits
    codes, scales, _, normalized = oracle.prepare_norm(x, w, stride, bits)
    p, norm = clef_i4.prepare_norm(dev_bf16(x), dev_bf16(w), bits=bits, stride=stride, store=store)
    assert_prepared(p, codes, scales, f"norm rows={rows} bits={bits}")
    if store:
        assert np.array_equal(host_u16(norm), normalized)


def test_attention_gate_projection_matches_oracle():
    """Engine::project_attention_gate: gated packing then the residual G1."""
    rng = np.random.default_rng(5)
    rows, width, n = 40, 2048, 512
    x = BF(rng.standard_normal((rows, width)).astype(np.float32))
    q = BF((rng.standard_normal((rows, 2 * width)) * 2.0).astype(np.float32))
    w = BF((rng.standard_normal((n, width)) * 0.02).astype(np.float32))
    res = BF(rng.standard_normal((rows, n)).astype(np.float32))
    stride = oracle.activation_stride(width)
    codes, scales, _ = oracle.prepare_attention_gate(x, q, stride)
    w_tiled, w_scales = oracle.pack_weight(w)
    want = oracle.gemm(codes, scales, w_tiled, w_scales, n, width, residual=res)
    qw = clef_i4.load_quantized_weight(dev_bf16(w))
    got = clef_i4.project_attention_gate(dev_bf16(x), dev_bf16(q), qw, dev_bf16(res))
    assert np.array_equal(host_u16(got), want)


@pytest.mark.parametrize("tokens,experts", [(1, 128), (31, 128), (33, 64), (4096, 128), (70, 32)])
def test_router_logits_within_f32_summation_bound(tokens, experts):
    """Router gate projection (src/omni.rs:764): each logit within the f32
    summation bound of the exact dot product (float64), plus half a bf16 step
    for the final rounding. The reference's WMMA summation order is not
    reproduced, so bits are compared only through this bound."""
    hidden = 2048
    rng = np.random.default_rng(tokens + experts)
    x = BF(rng.standard_normal((tokens, hidden)).astype(np.float32))
    w = BF((rng.standard_normal((experts, hidden)) * 0.02).astype(np.float32))
    got = oracle.bf16_to_f32(host_u16(clef_i4.router_logits(dev_bf16(x), dev_bf16(w)))).astype(np.float64)
    xf, wf = oracle.bf16_to_f32(x).astype(np.float64), oracle.bf16_to_f32(w).astype(np.float64)
    exact = xf @ wf.T
    bound = hidden * 2.0 ** -23 * (np.abs(xf) @ np.abs(wf).T) + np.abs(exact) * 2.0 ** -8 + 1e-30
    assert (np.abs(got - exact) <= bound).all()


def test_router_logits_one_hot_weights_are_exact():
    """With one-hot gate rows every logit is a single exact product, so the
    output is the selected input column bit for bit: pins the token/expert
    indexing and the tail of a partial 32-token block."""
    tokens, hidden, experts = 45, 256, 128
    rng = np.random.default_rng(9)
    x = BF(rng.standard_normal((tokens, hidden)).astype(np.float32))
    w = np.zeros((experts, hidden), dtype=np.uint16)
    cols = rng.permutation(hidden)[:experts]
    w[np.arange(experts), cols] = 0x3F80  # 1.0
    got = host_u16(clef_i4.router_logits(dev_bf16(x), dev_bf16(w)))
    assert np.array_equal(got, x[:, cols])
