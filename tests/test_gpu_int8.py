"""INT8 x INT8 projections (h3_gemm_i8_256, kernels/gemm_integer.loom:444-485):
bits-8 activations and weights through the C ABI, bit for bit against the
oracle's G1 with bits = 8."""
import numpy as np
import pytest
import torch

import clef_i4
import oracle

pytestmark = pytest.mark.gpu

BF = oracle.f32_to_bf16


def dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def host_u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def run(x, w, residual=None):
    n, k = w.shape
    qw = clef_i4.load_quantized_weight(dev_bf16(w), bits=8)
    a = clef_i4.prepare(dev_bf16(x), bits=8)
    got = clef_i4.project_prepared(a, qw, residual=None if residual is None else dev_bf16(residual))
    stride = oracle.activation_stride(k, 8)
    codes, scales, _ = oracle.prepare(x, stride, 8)
    w_tiled, w_scales = oracle.pack_weight(w, bits=8)
    assert np.array_equal(qw.codes.cpu().numpy().view(np.uint32), w_tiled), "packed int8 weight"
    want = oracle.gemm(codes, scales, w_tiled, w_scales, n, k, bits=8, residual=residual)
    return host_u16(got), want


@pytest.mark.parametrize("m,n,k", [(1, 256, 256), (17, 256, 768), (300, 768, 1024), (1100, 512, 2048),
                                   (64, 1024, 4096)])
def test_i8_gemm_matches_oracle(m, n, k):
    rng = np.random.default_rng(m + n + k)
    x = BF(rng.standard_normal((m, k)).astype(np.float32))
    w = BF((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    got, want = run(x, w)
    assert np.array_equal(got, want), f"{np.sum(got != want)} mismatches"


@pytest.mark.parametrize("m", [1, 255, 1030])
def test_i8_gemm_residual_matches_oracle(m):
    rng = np.random.default_rng(m)
    n, k = 256, 1024
    x = BF(rng.standard_normal((m, k)).astype(np.float32))
    w = BF((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    res = BF(rng.standard_normal((m, n)).astype(np.float32))
    got, want = run(x, w, res)
    assert np.array_equal(got, want)


def test_i8_gemm_extreme_codes_and_nonfinite_rows():
    """Constant rows give codes +-127 everywhere (the largest |acc|); huge
    scales saturate; NaN and Inf rows give zero codes with infinite scales."""
    m, n, k = 8, 256, 512
    x = np.zeros((m, k), dtype=np.float32)
    x[0] = 1.0
    x[1] = -3.0e38
    x[2, 5] = np.nan
    x[3, 7] = np.inf
    x[4] = np.linspace(-1, 1, k)
    x[5] = 3.0e38
    w = np.ones((n, k), dtype=np.float32)
    w[1::2] = -2.0e38
    got, want = run(BF(x), BF(w))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("n,k", [(256, 256), (512, 2304), (1024, 4096), (256, 12288)])
def test_i8_gemm_decode_rows_match_oracle(m, n, k):
    """At most 8 rows: the v_dot4_i32_i8 kernel, k-steps of 128 k (2 to 96 of
    them over its 8 waves), with and without the residual."""
    rng = np.random.default_rng(m * 100 + n + k)
    x = BF(rng.standard_normal((m, k)).astype(np.float32))
    w = BF((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    got, want = run(x, w)
    assert np.array_equal(got, want), f"{np.sum(got != want)} mismatches"
    res = BF(rng.standard_normal((m, n)).astype(np.float32))
    got, want = run(x, w, res)
    assert np.array_equal(got, want), f"residual: {np.sum(got != want)} mismatches"
