"""Parity of the HIP path (through the C ABI) with the CPU oracle on the same
seeded inputs. Integer stages and bf16 outputs are compared bit for bit: the
kernels and the oracle compute the same IEEE sequence (routing probabilities
and SwiGLU use the same explicit exp steps on both sides).

Each test names the reference test whose inputs or edge cases it follows.
"""
import numpy as np
import pytest
import torch

import clef_i4
import oracle

pytestmark = pytest.mark.gpu

BF = oracle.f32_to_bf16
F = oracle.bf16_to_f32
DEV = "cuda"


def to_dev_bf16(a_u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).view(torch.bfloat16).to(DEV)


def bf16_host(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def u32_host(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().numpy().view(np.uint32)


def to_dev_u32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(DEV)


def to_dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def randn_bf16(rng, shape, std=1.0) -> np.ndarray:
    return BF((rng.standard_normal(shape) * std).astype(np.float32))


def assert_same_u16(got: np.ndarray, want: np.ndarray, what: str):
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} mismatches, first at {i}: got {got[i]:#06x} "
                             f"want {want[i]:#06x}")


def assert_same_u32(got: np.ndarray, want: np.ndarray, what: str):
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} mismatches, first at {i}: got {got[i]:#010x} "
                             f"want {want[i]:#010x}")


def exceptional_rows(width: int) -> np.ndarray:
    """Rows of src/quantized.rs:1138-1150 plus zero and e_0 rows."""
    rows = []
    base = F(BF(np.array([((i * 37 % 257) - 128) / 91.0 for i in range(width)], dtype=np.float32)))
    r = base.copy()
    r[259 % width] = np.nan
    rows.append(r)
    r = base.copy()
    r[515 % width] = np.inf
    rows.append(r)
    r = base.copy()
    r[3] = F(np.array([0x7F7F], dtype=np.uint16))[0]  # bf16::MAX
    rows.append(r)
    r = base.copy()
    r[7] = F(np.array([0x0001], dtype=np.uint16))[0]  # bf16 denormal
    rows.append(r)
    rows.append(np.full(width, -0.5, dtype=np.float32))
    rows.append(np.full(width, 19.0, dtype=np.float32))
    rows.append(np.zeros(width, dtype=np.float32))
    e0 = np.zeros(width, dtype=np.float32)
    e0[0] = 1.0
    rows.append(e0)
    rows.append(base)
    return BF(np.stack(rows))


# ---------------------------------------------------------------- Q1 / Q2

@pytest.mark.parametrize("width", [256, 768, 1024, 2048, 4096, 4352, 5120, 12288, 17408, 32768])
@pytest.mark.parametrize("bits", [4, 8])
def test_prepare_matches_oracle(width, bits):
    """rotated_packing_cpu_oracle / register_packing_matches_reference
    (src/quantized.rs:1074-1185): codes and scales exact."""
    rng = np.random.default_rng(width * 10 + bits)
    rows = 37 if width <= 4096 else 11
    x = np.concatenate([randn_bf16(rng, (rows, width)), exceptional_rows(width)])
    stride = oracle.activation_stride(width, bits)
    _, _, want = oracle.prepare(x, stride, bits)
    got = clef_i4.prepare(to_dev_bf16(x), bits=bits, stride=stride)
    assert_same_u32(u32_host(got.storage), want, f"prepare width={width} bits={bits}")


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 16, 17, 1000])
def test_prepare_row_counts(rows):
    rng = np.random.default_rng(rows)
    for width in (768, 2048):
        x = randn_bf16(rng, (rows, width), std=3.0)
        stride = oracle.activation_stride(width)
        _, _, want = oracle.prepare(x, stride)
        got = clef_i4.prepare(to_dev_bf16(x), stride=stride)
        assert_same_u32(u32_host(got.storage), want, f"prepare rows={rows} width={width}")


@pytest.mark.parametrize("width", [768, 2048, 17408])
def test_prepare_swiglu_matches_oracle(width):
    """fused_swiglu_packing_matches_reference (src/quantized.rs:1189-1266)."""
    rng = np.random.default_rng(width)
    rows = 19
    g = randn_bf16(rng, (rows, width), std=2.0)
    u = randn_bf16(rng, (rows, width), std=2.0)
    stride = oracle.activation_stride(width)
    _, _, want = oracle.prepare_swiglu(g, u, stride)
    got = clef_i4.prepare_swiglu(to_dev_bf16(g), to_dev_bf16(u), stride=stride)
    assert_same_u32(u32_host(got.storage), want, f"prepare_swiglu width={width}")


@pytest.mark.parametrize("width,bits,row_counts", __import__("ref_inputs").fused_swiglu_cases())
def test_prepare_swiglu_reference_inputs(width, bits, row_counts):
    """fused_swiglu_packing_matches_reference (src/quantized.rs:1189-1266) on
    its own inputs: gate rows 0, NaN at column 259, +inf at 515, bf16::MAX,
    the bf16 denormal 0x0001, +-80 and the formula (every out-of-table SiLU
    case of the fused kernel), the up formula, the row-offset slices (gate
    from row 1, up from row 2) and stride width + 512 / bits. The fused
    producer equals the oracle, equals clef_swiglu followed by clef_i4_prepare
    on the device, and is the same on a second run, codes and scales bit for
    bit."""
    import ref_inputs

    stride = width + 512 // bits
    words = width // (32 // bits)
    for rows in row_counts:
        print(f"prepare_swiglu width={width} bits={bits} rows={rows}", flush=True)
        gate, up = ref_inputs.swiglu_gate_up(width, rows)
        want_c, want_s, _ = oracle.prepare_swiglu(gate, up, stride, bits)
        g_dev, u_dev = to_dev_bf16(gate), to_dev_bf16(up)
        fused = clef_i4.prepare_swiglu(g_dev, u_dev, bits=bits, stride=stride)
        again = clef_i4.prepare_swiglu(g_dev, u_dev, bits=bits, stride=stride)
        split = clef_i4.prepare(clef_i4.swiglu(g_dev, u_dev), bits=bits, stride=stride)
        for what, got in (("fused", fused), ("fused again", again), ("swiglu then prepare", split)):
            codes = u32_host(got.codes).reshape(rows, -1)[:, :words]
            assert_same_u32(codes, want_c[:, :words], f"{what} codes width={width} bits={bits} rows={rows}")
            assert_same_u32(got.scales.cpu().numpy().view(np.uint32), want_s.view(np.uint32),
                            f"{what} scales width={width} bits={bits} rows={rows}")


@pytest.mark.parametrize("rows,cols", [(128, 256), (256, 2048), (384, 768)])
def test_retile_matches_block_formula(rows, cols):
    """retiled_codes_match_block_formula (src/quantized.rs:1371-1407)."""
    in_words = cols // 8 + 16
    codes = (np.arange(rows * in_words, dtype=np.uint64) * 2654435761 % (1 << 32)).astype(np.uint32)
    codes = codes.reshape(rows, in_words)
    want = oracle.retile(codes, cols)
    got = clef_i4.retile_codes(to_dev_u32(codes), rows, cols)
    assert_same_u32(u32_host(got), want, "retile")


def test_pack_weight_matches_oracle():
    rng = np.random.default_rng(3)
    for rows, cols in [(256, 2048), (512, 768), (256, 4096)]:
        w = randn_bf16(rng, (rows, cols), std=0.02)
        want_codes, want_scales = oracle.pack_weight(w)
        qw = clef_i4.load_quantized_weight(to_dev_bf16(w))
        assert_same_u32(u32_host(qw.codes), want_codes, "pack codes")
        assert np.array_equal(qw.scales.cpu().numpy().view(np.uint32), want_scales.view(np.uint32))


def test_untile_rows_roundtrip():
    rng = np.random.default_rng(4)
    w = rng.integers(0, 1 << 16, size=(512, 192), dtype=np.uint16)
    tiled = oracle.tile_rows(w)
    got = clef_i4.untile_rows(to_dev_bf16(tiled))
    assert_same_u16(bf16_host(got), w, "untile")
    back = clef_i4.tile_rows(to_dev_bf16(w))
    assert_same_u16(bf16_host(back), tiled, "tile")


# ---------------------------------------------------------------- G1

def make_operands(rng, m, n, k, x_std=1.0, w_std=0.02):
    x = randn_bf16(rng, (m, k), std=x_std)
    w = randn_bf16(rng, (n, k), std=w_std)
    stride = oracle.activation_stride(k)
    a_codes, a_scales, _ = oracle.prepare(x, stride)
    w_tiled, w_scales = oracle.pack_weight(w)
    return x, w, stride, a_codes, a_scales, w_tiled, w_scales


def dev_prepared(x_u16, stride):
    return clef_i4.prepare(to_dev_bf16(x_u16), stride=stride)


def dev_weight(w_tiled, w_scales, n, k):
    return clef_i4.QuantizedWeight(to_dev_u32(w_tiled), to_dev_f32(w_scales), n, k,
                                   oracle.activation_stride(k), 4)


@pytest.mark.parametrize("m,n,k", [(1, 128, 256), (17, 256, 768), (128, 128, 2048), (300, 384, 1024),
                                   (257, 512, 4096), (64, 1024, 12288)])
def test_gemm_matches_oracle_all_configs(m, n, k):
    """G1 epilogue bit-exact for every tile configuration; M not a tile
    multiple exercises the row guard (residual_projection_matches_separate_addition
    covers 36 row counts, src/quantized.rs:1411-1552)."""
    rng = np.random.default_rng(m * 7 + n + k)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, config=cfg)
        assert_same_u16(bf16_host(got), want, f"gemm m={m} n={n} k={k} config={cfg}")
    got = clef_i4.project_quantized(to_dev_bf16(x), qw)
    assert_same_u16(bf16_host(got), want, "project_quantized")


@pytest.mark.parametrize("m", [1, 31, 128, 129, 255, 256, 257, 4032])
def test_gemm_residual_matches_oracle(m):
    """residual_projection_matches_separate_addition (src/quantized.rs:1411-1552)."""
    n, k = 256, 1024
    rng = np.random.default_rng(m)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    res = randn_bf16(rng, (m, n), std=4.0)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k, residual=res)
    sep = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    assert np.array_equal(want, BF(F(res) + F(sep)))
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, residual=to_dev_bf16(res), config=cfg)
        assert_same_u16(bf16_host(got), want, f"residual m={m} config={cfg}")


@pytest.mark.parametrize("resid", [False, True])
def test_gemm_several_tiles_per_workgroup(resid):
    """M8292 N4096 K512: 33 x 16 = 528 tiles of 256x256, more than twice the
    workgroups a persistent grid holds on 256 CUs, so persistent workgroups
    run two or three tiles each (a tile then starts on k-steps loaded during
    the previous tile's last k-step), and the last row tile is ragged. Every
    configuration agrees with the first over the whole output; sampled rows
    bit-exact against the oracle (with and without the residual,
    src/quantized.rs:1411-1552)."""
    m, n, k = 8292, 4096, 512
    rng = np.random.default_rng(8292 + resid)
    x, _, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    res = randn_bf16(rng, (m, n), std=4.0) if resid else None
    rows = np.unique(np.concatenate([[0, 255, 256, 4095, 8191, 8192, m - 1], rng.choice(m, 40, replace=False)]))
    want = oracle.gemm(a_codes[rows], a_scales[rows], w_tiled, w_scales, n, k,
                       residual=None if res is None else res[rows])
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    res_dev = to_dev_bf16(res) if resid else None
    idx = torch.from_numpy(rows).to(DEV)
    first = None
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, residual=res_dev, config=cfg)
        assert_same_u16(bf16_host(got[idx]), want, f"several tiles resid={resid} config={cfg}")
        if first is None:
            first = got
        else:
            assert torch.equal(got.view(torch.int16), first.view(torch.int16)), f"config {cfg} vs 0"


def test_gemm_extreme_codes_and_saturation():
    """All codes at +-7 (|acc| = 49 K), huge scales (saturation to bf16 max),
    infinite and NaN activation scales (kernels/gemm_integer.loom:411-418)."""
    m, n, k = 64, 128, 4096
    stride = oracle.activation_stride(k)
    a_words = np.full((m, stride // 8), 0x77777777, dtype=np.uint32)
    a_words[1::2, : k // 8] = 0x99999999  # -7
    w_codes = np.full((n, stride // 8), 0x99999999, dtype=np.uint32)
    w_codes[::3, : k // 8] = 0x77777777
    w_tiled = oracle.retile(w_codes, k)
    a_scales = np.full(m, 1e30, dtype=np.float32)
    a_scales[5] = np.inf
    a_scales[6] = np.nan
    a_scales[7] = 1e-3
    w_scales = np.full(n, 1e10, dtype=np.float32)
    w_scales[::5] = 1e-30
    want = oracle.gemm(a_words, a_scales, w_tiled, w_scales, n, k)
    storage = np.concatenate([a_words.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    qw = dev_weight(w_tiled, w_scales, n, k)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, config=cfg)
        assert_same_u16(bf16_host(got), want, f"extreme config={cfg}")


def test_gemm_zero_and_tiny_scales():
    """Scales that make the "+ 0" of the epilogue matter (kernels/gemm_integer.loom:411-418):
    zero weight scales (a negative accumulator times +0 is -0, which the + 0
    turns into +0) and scale products near and below the f32 normal range
    (results that round to zero or to denormals). Every configuration against
    the oracle, bit for bit; rows past a tile multiple included."""
    m, n, k = 300, 512, 512
    rng = np.random.default_rng(77)
    stride = oracle.activation_stride(k)

    def code_words(rows):
        # codes in -7..7 as the quantizer makes them, 8 nibbles per word
        nib = (rng.integers(-7, 8, size=(rows, stride)) & 15).astype(np.uint32)
        nib[:, k:] = 0
        return sum(nib[:, j::8] << np.uint32(4 * j) for j in range(8)).astype(np.uint32)

    a_words = code_words(m)
    a_scales = (10.0 ** rng.uniform(-12, 0, size=m)).astype(np.float32)
    a_scales[::7] = np.float32(1e-20)
    a_scales[3] = np.float32(1e-37)
    w_tiled = oracle.retile(code_words(n), k)
    w_scales = (10.0 ** rng.uniform(-6, 0, size=n)).astype(np.float32)
    w_scales[::11] = 0.0
    w_scales[5::13] = np.float32(1e-30)
    want = oracle.gemm(a_words, a_scales, w_tiled, w_scales, n, k)
    # the fixture reaches the cases it is for: negative accumulators in
    # zero-scale columns (+0 in the reference, -0 without its + 0), and bf16
    # denormals and underflows from tiny products
    acc = oracle.gemm_acc(a_words, w_tiled, n, k)
    zero_cols = w_scales == 0
    assert (acc[:, zero_cols] < 0).any() and (want[:, zero_cols] == 0).all()
    assert (((want & 0x7F80) == 0) & ((want & 0x7F) != 0)).any()
    storage = np.concatenate([a_words.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    qw = dev_weight(w_tiled, w_scales, n, k)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, config=cfg)
        assert_same_u16(bf16_host(got), want, f"zero/tiny scales config={cfg}")


def assert_same_bf16_nan_aware(got: np.ndarray, want: np.ndarray, what: str):
    """Bit-exact, except that any NaN equals any NaN: a NaN made by 0 * inf
    carries the sign bit of the machine's default NaN (0x7fc00000 on the GPU,
    0xffc00000 on x86), which the reference does not specify."""
    gn = (got & 0x7FFF) > 0x7F80
    wn = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    assert_same_u16(np.where(gn, 0, got), np.where(wn, 0, want), what)


def test_gemm_nan_and_inf_activation_rows():
    """NaN/Inf rows quantize to zero codes with scale +inf
    (kernels/prepare_integer_single.loom:251-271) and stay observable through
    the GEMM (kernels/gemm_integer.loom:411-418)."""
    n, k = 256, 1024
    rng = np.random.default_rng(21)
    x = np.concatenate([randn_bf16(rng, (40, k)), exceptional_rows(k)])
    w = randn_bf16(rng, (n, k), std=0.02)
    stride = oracle.activation_stride(k)
    a_codes, a_scales, _ = oracle.prepare(x, stride)
    w_tiled, w_scales = oracle.pack_weight(w)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    assert ((want[40] & 0x7FFF) > 0x7F80).all(), "NaN row must give NaN outputs"
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, config=cfg)
        assert_same_bf16_nan_aware(bf16_host(got), want, f"nan rows config={cfg}")


def test_identity_weight_reproduces_input():
    """activation_scratch_is_bounded (src/quantized.rs:880-915): a 256x256
    identity weight maps a constant row to itself exactly."""
    k = n = 256
    w = np.zeros((n, k), dtype=np.float32)
    np.fill_diagonal(w, 1.0)
    qw = clef_i4.load_quantized_weight(to_dev_bf16(BF(w)))
    x = BF(np.stack([np.full(k, v, dtype=np.float32) for v in (0.25, 1.0, -3.0, 8.0)]))
    y = clef_i4.project_quantized(to_dev_bf16(x), qw)
    assert_same_u16(bf16_host(y), x, "identity projection")


def test_gemm_is_deterministic():
    m, n, k = 512, 512, 2048
    rng = np.random.default_rng(11)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    first = bf16_host(clef_i4.project_prepared(a, qw))
    for _ in range(3):
        assert np.array_equal(bf16_host(clef_i4.project_prepared(a, qw)), first)


# ---------------------------------------------------------------- MoE routing

def tie_logits(rng, tokens, experts, dtype):
    """Router phases of src/benchmarking/omni.rs:43-55: duplicates, +-0, large values."""
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    logits[::4] = np.round(logits[::4] * 2) / 2          # many exact ties
    logits[1::7] = 0.0
    logits[1::7, ::3] = -0.0
    logits[2::9] *= 1e4
    logits[3::11, :16] = 7.0                             # one tied block
    if dtype == "bf16":
        return BF(logits)
    return logits


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("experts,topk", [(128, 8), (64, 8), (128, 1), (100, 16)])
def test_route_matches_oracle(dtype, experts, topk):
    """OmniRouter paired check (src/benchmarking/omni.rs:42-90): ids exact,
    probabilities bit-exact (same exp steps)."""
    rng = np.random.default_rng(experts + topk)
    logits = tie_logits(rng, 333, experts, dtype)
    want = oracle.route(logits, topk)
    dev = to_dev_bf16(logits) if dtype == "bf16" else to_dev_f32(logits)
    got = clef_i4.omni_route(dev, topk).cpu().numpy()
    assert np.array_equal(got[:, :topk], want[:, :topk]), "route ids"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "route probabilities"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("experts,topk", [(128, 8), (100, 16), (66, 8), (72, 16), (128, 24), (72, 17), (8, 8)])
def test_route_edge_values_match_oracle(dtype, experts, topk):
    """Rows with quiet NaNs (ignored by the maximum), -inf, -FLT_MAX and
    all-equal values (no +inf: exp(inf - inf) makes the probabilities NaN,
    whose bits are not part of the contract); topk up to 16 runs 16 lanes per token, above that one
    wave per token; rows of 100 or 66 experts are read element by element
    (their row starts are not 16-byte aligned). Ids and probability bits
    against the oracle."""
    rng = np.random.default_rng(experts * 7 + topk)
    tokens = 97
    logits = tie_logits(rng, tokens, experts, "f32")
    logits[5::6, ::5] = np.nan
    logits[4::13, ::2] = -np.inf
    logits[7::17] = -np.inf
    logits[7::17, 3] = 1.5
    logits[8::19, :] = 2.0
    logits[9::23, ::3] = -3.402823466e38
    if dtype == "bf16":
        logits = BF(logits)
    want = oracle.route(logits, topk)
    dev = to_dev_bf16(logits) if dtype == "bf16" else to_dev_f32(logits)
    got = clef_i4.omni_route(dev, topk).cpu().numpy()
    assert np.array_equal(got[:, :topk], want[:, :topk]), "route ids"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "route probabilities"


def test_route_ids_are_stable_sort():
    """The selected ids equal a stable descending sort (src/omni.rs:997-1009)."""
    rng = np.random.default_rng(5)
    logits = tie_logits(rng, 200, 128, "f32")
    got = clef_i4.omni_route(to_dev_f32(logits), 8).cpu().numpy()
    want = np.argsort(-logits, axis=1, kind="stable")[:, :8]
    assert np.array_equal(got[:, :8].astype(np.int64), want)


def random_routes(rng, tokens, topk=8, skew=0.0):
    logits = rng.standard_normal((tokens, 128)).astype(np.float32)
    if skew:
        logits -= skew * np.log1p(rng.permutation(128)).astype(np.float32)
    return oracle.route(logits, topk)


@pytest.mark.parametrize("tokens", [1, 2, 17, 255, 256, 257, 511, 512, 513, 1000, 4096, 6000])
def test_group_routes_matches_oracle(tokens):
    """grouped_routes_match_cpu (src/omni.rs:908-942): stable lists, counts, order.
    Up to 512 tokens at top-8 one workgroup groups them, above that three
    kernels do; both sides of the switch are covered."""
    rng = np.random.default_rng(tokens)
    routes = random_routes(rng, tokens, skew=1.0 if tokens > 100 else 0.0)
    want_g, want_o = oracle.group_routes(routes)
    g, o = clef_i4.omni_group_routes(to_dev_f32(routes))
    g = g.cpu().numpy()
    o = o.cpu().numpy()
    for e in range(128):
        c = int(want_g[e, 0])
        assert g[e, 0] == want_g[e, 0], f"count e={e}"
        assert np.array_equal(g[e, 1:1 + c], want_g[e, 1:1 + c]), f"list e={e}"
    assert np.array_equal(o, want_o), "order"
    tasks = clef_i4.omni_expert_tasks(to_dev_f32(want_g)).cpu().numpy()
    want_t = oracle.expert_tasks(want_g)
    total = int(want_t[0])
    assert np.array_equal(tasks[: 1 + 2 * total], want_t[: 1 + 2 * total]), "tasks"


@pytest.mark.parametrize("tokens,topk", [(1, 1), (17, 4), (300, 6), (513, 2), (4100, 4), (2000, 16), (700, 24)])
def test_group_routes_other_topk(tokens, topk):
    """Grouping at topk other than 8 (the generic count and scatter kernels:
    the one-workgroup and register paths take top-8 only): lists, counts and
    the ascending-expert order of each token's topk ranks."""
    rng = np.random.default_rng(tokens * 3 + topk)
    routes = random_routes(rng, tokens, topk=topk, skew=1.0 if tokens > 100 else 0.0)
    want_g, want_o = oracle.group_routes(routes, topk=topk)
    g, o = clef_i4.omni_group_routes(to_dev_f32(routes))
    g = g.cpu().numpy()
    for e in range(128):
        c = int(want_g[e, 0])
        assert g[e, 0] == want_g[e, 0], f"count e={e}"
        assert np.array_equal(g[e, 1:1 + c], want_g[e, 1:1 + c]), f"list e={e}"
    assert np.array_equal(o.cpu().numpy(), want_o), "order"


def test_group_routes_empty_and_full_experts():
    """Empty experts and one expert taking every token (src/omni.rs:920-938)."""
    tokens = 600
    routes = np.zeros((tokens, 16), dtype=np.float32)
    for t in range(tokens):
        ids = [5] + [int(x) for x in np.random.default_rng(t).choice(np.arange(6, 128), 7, replace=False)]
        routes[t, :8] = ids
        routes[t, 8:] = 0.125
    want_g, want_o = oracle.group_routes(routes)
    g, o = clef_i4.omni_group_routes(to_dev_f32(routes))
    g = g.cpu().numpy()
    assert g[5, 0] == tokens and all(g[e, 0] == 0 for e in range(5))
    for e in range(128):
        c = int(want_g[e, 0])
        assert np.array_equal(g[e, :1 + c], want_g[e, :1 + c]), f"e={e}"
    assert np.array_equal(o.cpu().numpy(), want_o)


@pytest.mark.parametrize("tokens", [300, 512, 513, 5000])
def test_group_routes_duplicate_and_invalid_ids(tokens):
    """Route rows that name an expert twice (the last rank is listed), ids
    outside 0..127 (-1, 128, 130: no expert) and fractional ids (7.5 names
    expert 7, 0.25 expert 0), as the oracle truncates them; on both sides of
    the one-workgroup switch at 512 tokens. (An id in (-1, 0) would name
    expert 0 yet sort below it, so two experts of the row would claim the
    same order slot, and which write lands is not specified.)"""
    rng = np.random.default_rng(tokens + 77)
    routes = random_routes(rng, tokens)
    special = [-1.0, 128.0, 130.0, 7.5, 0.25]
    for t in range(0, tokens, 3):
        r1, r2 = rng.choice(8, 2, replace=False)
        routes[t, r2] = routes[t, r1]  # duplicate
        if t % 2 == 0:
            routes[t, rng.integers(8)] = special[(t // 6) % len(special)]
    want_g, want_o = oracle.group_routes(routes)
    g, o = clef_i4.omni_group_routes(to_dev_f32(routes))
    g = g.cpu().numpy()
    for e in range(128):
        c = int(want_g[e, 0])
        assert g[e, 0] == want_g[e, 0], f"count e={e}"
        assert np.array_equal(g[e, 1:1 + c], want_g[e, 1:1 + c]), f"list e={e}"
    assert np.array_equal(o.cpu().numpy(), want_o), "order"


# ---------------------------------------------------------------- E1, S1, C1

def packed_experts(rng, n, k):
    w = randn_bf16(rng, (128 * n, k), std=0.02)
    return oracle.pack_weight(w)


@pytest.mark.parametrize("tokens,hidden", [(1, 512), (3, 512), (20, 768), (64, 512), (300, 512), (7, 256)])
def test_expert_gemm_matches_oracle(tokens, hidden):
    """routed_experts_match_sparse_cpu_oracle (src/omni.rs:946-1051) and the
    OmniExpert paired check (src/benchmarking/omni.rs:328-356), bit-exact.
    Up to 256 routed rows the VALU decode kernel runs on the 32-slot tiles
    (skewed routes give experts several two-slot passes; K = 256 and 768 give
    one and three k-steps), up to 2048 the 32-slot skinny kernel (one wave
    per k-step), above it the 128-slot kernel."""
    rng = np.random.default_rng(tokens)
    inter, topk = 256, 8
    routes = random_routes(rng, tokens, skew=2.0)
    groups, _ = oracle.group_routes(routes)
    x = randn_bf16(rng, (tokens, hidden))
    sx = oracle.activation_stride(hidden)
    ax_codes, ax_scales, _ = oracle.prepare(x, sx)
    gw, gs = packed_experts(rng, inter, hidden)
    want = oracle.expert_i4(ax_codes, ax_scales, gw, gs, groups, tokens, topk, hidden, inter, False)
    got = clef_i4.omni_expert(dev_prepared(x, sx), dev_weight(gw, gs, 128 * inter, hidden),
                              to_dev_f32(groups), tokens, topk, False)
    assert_same_u16(bf16_host(got), want, "expert gate")
    # routed input (down projection): rows are routes
    h = randn_bf16(rng, (tokens * topk, inter))
    sh = oracle.activation_stride(inter)
    ah_codes, ah_scales, _ = oracle.prepare(h, sh)
    dw, ds = packed_experts(rng, hidden, inter)
    want = oracle.expert_i4(ah_codes, ah_scales, dw, ds, groups, tokens, topk, inter, hidden, True)
    got = clef_i4.omni_expert(dev_prepared(h, sh), dev_weight(dw, ds, 128 * hidden, inter),
                              to_dev_f32(groups), tokens, topk, True)
    assert_same_u16(bf16_host(got), want, "expert down")


@pytest.mark.parametrize("tokens", [3, 64, 300, 600])
@pytest.mark.parametrize("input_routed", [False, True])
def test_expert_ungrouped_matches_oracle(tokens, input_routed):
    """Engine::omni_expert (src/omni.rs:280-288), the expert GEMM without a
    groups table, on routes with a duplicate expert, an all-127 token and
    ids naming no expert: every slot bit-exact against the oracle's ungrouped
    E1 (both tile regimes: 24 / 512 routed rows on 32-slot tiles, 2400 on
    128-slot tiles), and equal to the grouped entry point on router output."""
    from test_oracle import duplicate_routes

    rng = np.random.default_rng(tokens * 2 + input_routed)
    k, n, topk = 512, 256, 8
    rows = tokens * topk if input_routed else tokens
    x = randn_bf16(rng, (rows, k))
    sx = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, sx)
    w_t, w_s = packed_experts(rng, n, k)
    a, w = dev_prepared(x, sx), dev_weight(w_t, w_s, 128 * n, k)
    routes = duplicate_routes(rng, tokens, topk)
    want = oracle.expert_i4_ungrouped(codes, scales, w_t, w_s, routes, k, n, input_routed)
    got = clef_i4.omni_expert_ungrouped(a, w, to_dev_f32(routes), input_routed)
    assert_same_u16(bf16_host(got), want, f"ungrouped tokens={tokens} routed={input_routed}")
    clean = random_routes(rng, tokens)
    groups, _ = oracle.group_routes(clean)
    grouped = clef_i4.omni_expert(a, w, to_dev_f32(groups), tokens, topk, input_routed)
    got = clef_i4.omni_expert_ungrouped(a, w, to_dev_f32(clean), input_routed)
    assert torch.equal(got.view(torch.int16), grouped.view(torch.int16))


@pytest.mark.parametrize("tokens,wide", [(1, False), (3, False), (20, False), (20, True), (64, False), (300, False),
                                         (300, True)])
def test_expert_gate_up_swiglu_matches_oracle(tokens, wide):
    """Fused gate/up + SwiGLU (Engine::omni_gate_up, src/omni.rs:300-372) equals
    E1(gate), E1(up) then S1 of the oracle, bit for bit; inter = 512 gives four
    128-column tiles and skewed routes leave experts empty, partial and
    multi-tile."""
    rng = np.random.default_rng(100 + tokens)
    hidden, inter, topk = 512, 512, 8
    routes = random_routes(rng, tokens, skew=2.0)
    groups, _ = oracle.group_routes(routes)
    x = randn_bf16(rng, (tokens, hidden))
    sx = oracle.activation_stride(hidden)
    ax_codes, ax_scales, _ = oracle.prepare(x, sx)
    gw, gs = packed_experts(rng, inter, hidden)
    uw, us = packed_experts(rng, inter, hidden)
    if wide:
        # gate scales over 82 decades: gate values from bf16 denormals to
        # overflow, through every range the SiLU table covers and beyond it
        gs = (10.0 ** rng.uniform(-44, 38, size=gs.shape)).astype(np.float32)
    g = oracle.expert_i4(ax_codes, ax_scales, gw, gs, groups, tokens, topk, hidden, inter, False)
    u = oracle.expert_i4(ax_codes, ax_scales, uw, us, groups, tokens, topk, hidden, inter, False)
    want = oracle.swiglu(g, u)
    got = clef_i4.omni_gate_up(dev_prepared(x, sx), dev_weight(gw, gs, 128 * inter, hidden),
                               dev_weight(uw, us, 128 * inter, hidden), to_dev_f32(groups), tokens, topk)
    if wide:
        # overflowing gates meet zero up values (inf * 0): NaN payload signs
        # differ between the host oracle and the GPU
        assert_same_bf16_nan_aware(bf16_host(got), want, "fused gate/up swiglu, wide scales")
    else:
        assert_same_u16(bf16_host(got), want, "fused gate/up swiglu")


@pytest.mark.parametrize("tokens,k,n,routed,skew", [
    (300, 768, 512, True, 2.0),    # the down projection's regime: K = 768 (six half-steps)
    (600, 512, 1024, False, 0.0),  # the shortest K the persistent kernel takes (four half-steps)
    (1000, 1024, 512, True, 4.0),  # strongly skewed: some experts span many tiles, others are empty
    (257, 2048, 512, False, 0.0),  # 2056 routed rows, just past the 32-slot regime
])
def test_expert_persistent_matches_oracle(tokens, k, n, routed, skew):
    """The persistent grouped expert GEMM (every active expert's items in one
    launch, taken from per-XCD queues) against the oracle's E1, the whole
    output bit for bit; a second call on the same workspace gives the same
    result (the queue counters are reset with each schedule)."""
    rng = np.random.default_rng(tokens + k + n)
    topk = 8
    routes = random_routes(rng, tokens, skew=skew)
    groups, _ = oracle.group_routes(routes)
    rows = tokens * topk if routed else tokens
    x = randn_bf16(rng, (rows, k))
    sx = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, sx)
    w_t, w_s = packed_experts(rng, n, k)
    want = oracle.expert_i4(codes, scales, w_t, w_s, groups, tokens, topk, k, n, routed)
    a, w = dev_prepared(x, sx), dev_weight(w_t, w_s, 128 * n, k)
    g = to_dev_f32(groups)
    got = clef_i4.omni_expert(a, w, g, tokens, topk, routed)
    assert_same_u16(bf16_host(got), want, f"persistent expert tokens={tokens} k={k} n={n}")
    again = clef_i4.omni_expert(a, w, g, tokens, topk, routed)
    assert torch.equal(again.view(torch.int16), got.view(torch.int16))


@pytest.mark.parametrize("tokens,k,n,skew", [(600, 2048, 768, 0.0), (700, 768, 256, 3.0), (300, 1024, 512, 1.0)])
def test_expert_gate_up_persistent_matches_oracle(tokens, k, n, skew):
    """The persistent fused gate/up + SwiGLU kernel (items of 256 gate and
    256 up rows) at the Omni shape (K 2048, 768 columns: three column blocks)
    and others, the whole h against E1, E1, S1 of the oracle, bit for bit."""
    rng = np.random.default_rng(7 * tokens + k + n)
    topk = 8
    routes = random_routes(rng, tokens, skew=skew)
    groups, _ = oracle.group_routes(routes)
    x = randn_bf16(rng, (tokens, k))
    sx = oracle.activation_stride(k)
    codes, scales, _ = oracle.prepare(x, sx)
    gw, gs = packed_experts(rng, n, k)
    uw, us = packed_experts(rng, n, k)
    g = oracle.expert_i4(codes, scales, gw, gs, groups, tokens, topk, k, n, False)
    u = oracle.expert_i4(codes, scales, uw, us, groups, tokens, topk, k, n, False)
    want = oracle.swiglu(g, u)
    a = dev_prepared(x, sx)
    gw_d, uw_d = dev_weight(gw, gs, 128 * n, k), dev_weight(uw, us, 128 * n, k)
    got = clef_i4.omni_gate_up(a, gw_d, uw_d, to_dev_f32(groups), tokens, topk)
    assert_same_u16(bf16_host(got), want, f"persistent gate/up tokens={tokens} k={k} n={n}")
    again = clef_i4.omni_gate_up(a, gw_d, uw_d, to_dev_f32(groups), tokens, topk)
    assert torch.equal(again.view(torch.int16), got.view(torch.int16))


def test_swiglu_every_bf16_gate():
    """swiglu_preserves_materialized_rounding (src/ops.rs:482-520) over all
    65536 gate bit patterns."""
    gate = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(9)
    up = randn_bf16(rng, 65536, std=3.0)
    want = oracle.swiglu(gate, up)
    got = clef_i4.swiglu(to_dev_bf16(gate), to_dev_bf16(up))
    assert_same_u16(bf16_host(got), want, "swiglu")
    odd = clef_i4.swiglu(to_dev_bf16(gate[:1003]), to_dev_bf16(up[:1003]))
    assert_same_u16(bf16_host(odd), want[:1003], "swiglu tail")


@pytest.mark.parametrize("ordered", [True, False])
@pytest.mark.parametrize("topk,width", [(8, 2048), (8, 264), (4, 2048)])
def test_combine_matches_oracle(ordered, topk, width):
    """OmniCombine paired check (src/benchmarking/omni.rs:387-431); top-8 runs
    the kernel that loads every rank first, other topk the rank-by-rank one;
    width 264 leaves a partial last wave of 8-column chunks."""
    rng = np.random.default_rng(int(ordered) + 2 * topk + width)
    tokens = 77
    routes = random_routes(rng, tokens, topk=topk)
    _, order = oracle.group_routes(routes, topk=topk)
    values = randn_bf16(rng, (tokens * topk, width), std=2.0)
    want = oracle.combine(values, routes, order if ordered else None, topk=topk)
    got = clef_i4.omni_combine(to_dev_bf16(values), to_dev_f32(routes),
                               to_dev_f32(order) if ordered else None)
    assert_same_u16(bf16_host(got), want, "combine")


@pytest.mark.parametrize("tokens,hidden,inter", [(1, 2048, 768), (2, 512, 256), (4, 2048, 768), (5, 512, 256),
                                                 (6, 512, 1024), (7, 512, 256), (12, 2048, 768), (13, 2048, 768),
                                                 (3, 512, 2048), (16, 512, 256),
                                                 (17, 512, 256), (32, 512, 256), (33, 512, 256),
                                                 (96, 2048, 768), (300, 1024, 512),
                                                 (256, 512, 256), (257, 512, 256), (1100, 512, 256),
                                                 (4160, 512, 256)])
def test_moe_layer_matches_oracle(tokens, hidden, inter):
    """Whole Omni INT4 MoE block (src/omni.rs:762-857) bit-exact vs the oracle.
    Up to 12 tokens (inter up to 1024) the block is two kernels: the router,
    Q1(x) and gate/up + SwiGLU, then the down projection, its quantizer and
    combine; 13 tokens take the separate router and grouping; with inter 2048
    up to 4 tokens the down projection quantizes its own h rows; 32 and 33 tokens sit on
    either side of the VALU decode expert kernels' limit, 256 and 257 tokens
    (2048 and 2056 routed rows) on either side of the switch from 32-slot to
    128-slot expert tiles; 1100 and 4160 tokens group from the router's
    per-16-token expert counts (partial last blocks of 16 and 64 tokens)."""
    rng = np.random.default_rng(tokens + hidden)
    x = randn_bf16(rng, (tokens, hidden))
    logits = BF(rng.standard_normal((tokens, 128)).astype(np.float32))
    gate = packed_experts(rng, inter, hidden)
    up = packed_experts(rng, inter, hidden)
    down = packed_experts(rng, hidden, inter)
    want, want_routes = oracle.moe_layer(x, logits, gate, up, down)
    layer = clef_i4.MoeLayer(dev_weight(*gate, 128 * inter, hidden), dev_weight(*up, 128 * inter, hidden),
                             dev_weight(*down, 128 * hidden, inter))
    routes = torch.empty((tokens, 16), dtype=torch.float32, device=DEV)
    got = layer(to_dev_bf16(x), to_dev_bf16(logits), routes_out=routes)
    assert np.array_equal(routes.cpu().numpy().view(np.uint32), want_routes.view(np.uint32))
    assert_same_u16(bf16_host(got), want, f"moe layer tokens={tokens}")
    again = layer(to_dev_bf16(x), to_dev_bf16(logits))
    assert_same_u16(bf16_host(again), want, "moe layer replay")


@pytest.mark.parametrize("tokens,hidden,inter,topk", [
    (12, 512, 256, 4), (300, 512, 256, 6), (700, 512, 256, 2), (40, 512, 256, 16), (20, 512, 256, 24),
    (64, 5120, 256, 8), (300, 4352, 256, 8), (9, 6144, 256, 4), (3, 4352, 256, 8), (5, 3072, 512, 8)])
def test_moe_layer_other_topk_and_wide_hidden(tokens, hidden, inter, topk):
    """The MoE block off the Omni shape, bit-exact against the oracle.
    topk other than 8 runs the generic grouping and combine kernels (the
    routing workgroup groups only top-8 routes); topk above 16 takes the
    wave-per-token router. hidden above 4096 (16 groups of 256) runs the
    router, the grouping and the quantizer of x as three launches instead of
    the router beside the quantizer; above hidden 2048, up to 6 tokens run
    the router (with the grouping up to hidden 4096), the gate/up kernel and
    one kernel for the down projection, its quantizer and combine."""
    rng = np.random.default_rng(tokens * 31 + hidden + topk)
    x = randn_bf16(rng, (tokens, hidden))
    logits = BF(rng.standard_normal((tokens, 128)).astype(np.float32))
    gate = packed_experts(rng, inter, hidden)
    up = packed_experts(rng, inter, hidden)
    down = packed_experts(rng, hidden, inter)
    want, want_routes = oracle.moe_layer(x, logits, gate, up, down, topk=topk)
    layer = clef_i4.MoeLayer(dev_weight(*gate, 128 * inter, hidden), dev_weight(*up, 128 * inter, hidden),
                             dev_weight(*down, 128 * hidden, inter), topk=topk)
    routes = torch.empty((tokens, 2 * topk), dtype=torch.float32, device=DEV)
    got = layer(to_dev_bf16(x), to_dev_bf16(logits), routes_out=routes)
    assert np.array_equal(routes.cpu().numpy().view(np.uint32), want_routes.view(np.uint32)), "routes"
    assert_same_u16(bf16_host(got), want, f"moe layer tokens={tokens} hidden={hidden} topk={topk}")


@pytest.mark.parametrize("tokens", [5, 20, 300, 1100])
def test_moe_layer_degenerate_logit_rows(tokens):
    """Logit rows that make a token name an expert twice (three finite
    logits, the rest -inf: once those three are taken the reset -FLT_MAX
    slots win again) or no expert (all NaN) leave combine-order entries
    unwritten. With the workspace filled with 0xFF bytes first (so unwritten
    entries hold NaN), the layer must keep every access in range, route
    every token as the oracle's router does, and give the other tokens'
    outputs bit for bit: every stage is token-local, so the oracle runs on
    the other tokens alone. The degenerate tokens' outputs are unspecified
    (as in the reference) and not compared. 5 tokens take the two-kernel
    layer, 20 the decode kernels, 300 and 1100 the grouped paths."""
    hidden, inter = 512, 256
    rng = np.random.default_rng(tokens + 77)
    x = randn_bf16(rng, (tokens, hidden))
    lg = rng.standard_normal((tokens, 128)).astype(np.float32)
    bad = np.zeros(tokens, dtype=bool)
    bad[1::4] = True
    for i in np.nonzero(bad)[0]:
        if i % 8 == 1:
            lg[i] = np.nan
        else:
            lg[i] = -np.inf
            lg[i, rng.choice(128, 3, replace=False)] = rng.standard_normal(3)
    logits = BF(lg)
    gate = packed_experts(rng, inter, hidden)
    up = packed_experts(rng, inter, hidden)
    down = packed_experts(rng, hidden, inter)
    layer = clef_i4.MoeLayer(dev_weight(*gate, 128 * inter, hidden), dev_weight(*up, 128 * inter, hidden),
                             dev_weight(*down, 128 * hidden, inter))
    layer.workspace(tokens, DEV).fill_(0xFF)
    routes = torch.empty((tokens, 16), dtype=torch.float32, device=DEV)
    got = bf16_host(layer(to_dev_bf16(x), to_dev_bf16(logits), routes_out=routes))
    want_routes = oracle.route(logits, 8)
    got_routes = routes.cpu().numpy()
    assert np.array_equal(got_routes[:, :8], want_routes[:, :8]), "route ids"
    nan_rows = np.isnan(lg).all(axis=1)  # their probabilities are NaN, whose bits are not part of the contract
    assert np.isnan(got_routes[nan_rows, 8:]).all()
    assert np.array_equal(got_routes[~nan_rows].view(np.uint32), want_routes[~nan_rows].view(np.uint32)), "routes"
    ids = want_routes[:, :8]
    assert all(len(set(ids[i].tolist())) < 8 for i in np.nonzero(bad)[0]), "every degenerate row repeats or lacks ids"
    good = ~bad
    want, _ = oracle.moe_layer(x[good], logits[good], gate, up, down)
    assert_same_u16(got[good], want, f"moe layer tokens={tokens}, the well-formed tokens")


def test_moe_layer_closed_form():
    """The MoE block on constant rows (every code +-7, silu(g) = g for the
    gates >= 17 these inputs give) against the closed form of
    test_oracle.moe_closed_form, and against the oracle, bit for bit; the
    device routes are the routes the closed form is evaluated on."""
    from test_oracle import closed_form_case, moe_closed_form

    t, d, inter, topk = 300, 512, 256, 8  # 2400 routed rows: the 128-slot expert tiles
    c, x, logits, (gate, up, down), (wg, wu, wd) = closed_form_case(11, t, d, inter, topk)
    dev = [clef_i4.load_quantized_weight(to_dev_bf16(w)) for w in (gate, up, down)]
    layer = clef_i4.MoeLayer(*dev)
    routes = torch.empty((t, 2 * topk), dtype=torch.float32, device=DEV)
    got = bf16_host(layer(to_dev_bf16(x), to_dev_bf16(logits), routes_out=routes))
    want, gates = moe_closed_form(c, routes.cpu().numpy(), wg, wu, wd, d, inter, topk)
    assert np.all(gates >= 17.0)
    assert np.array_equal(F(got), want)
    small = bf16_host(layer(to_dev_bf16(x[:40]), to_dev_bf16(logits[:40])))  # 320 rows: 32-slot tiles
    assert np.array_equal(small, got[:40])


def test_c1_linear_full_output():
    """The single INT4 linear of the reference's CPU path at its exact shape,
    M512 K2048 N2048 (x ~ N(0, 1), w ~ N(0, 0.02), seed 1001): the whole
    [512][2048] output of the default path (quantize + projection) and of
    every tile configuration equals the oracle, bit for bit."""
    m, k, n = 512, 2048, 2048
    rng = np.random.default_rng(1001)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    qw = clef_i4.load_quantized_weight(to_dev_bf16(w))
    assert_same_u32(u32_host(qw.codes), w_tiled, "c1 packed weight")
    got = clef_i4.project_quantized(to_dev_bf16(x), qw)
    assert_same_u16(bf16_host(got), want, "c1 default path")
    a = dev_prepared(x, stride)
    for cfg in range(clef_i4.gemm_configs()):
        got = clef_i4.project_prepared(a, qw, config=cfg)
        assert_same_u16(bf16_host(got), want, f"c1 config={cfg}")


# ---------------------------------------------------------------- bf6 G1
# The bf6 (e3m2) re-encoding of G1's operands (clef_i4_f6_activation,
# clef_i4_f6_weight, clef_i4_gemm_f6) must give exactly what G1 gives on the
# INT4 operands they came from.

E3M2 = np.array([0x00, 0x0C, 0x10, 0x12, 0x14, 0x15, 0x16, 0x17,
                 0x38, 0x37, 0x36, 0x35, 0x34, 0x32, 0x30, 0x2C], dtype=np.uint64)


def e3m2_value(bits):
    """Value of e3m2 bits (sign, exponent with bias 3, 2 mantissa bits)."""
    bits = np.asarray(bits, dtype=np.int64)
    sign = np.where(bits & 0x20, -1.0, 1.0)
    e, m = (bits >> 2) & 7, bits & 3
    return sign * np.where(e == 0, m / 4.0 * 2.0 ** -2, (1 + m / 4.0) * 2.0 ** (e - 3))


def test_e3m2_table_is_exact_for_every_int4_code():
    codes = np.arange(16)
    signed = np.where(codes < 8, codes, codes - 16)
    assert np.array_equal(e3m2_value(E3M2), signed.astype(np.float64))


def f6_rows_numpy(codes_u32: np.ndarray, k: int) -> np.ndarray:
    """bf6 rows of packed codes ([rows][words], nibble p of word q = column
    8q+p): value j at bits 6j of the row's k*3/4 bytes."""
    rows = codes_u32.shape[0]
    nib = (codes_u32[:, : k // 8, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    v = E3M2[nib.reshape(rows, k)]  # [rows][k] 6-bit values
    v = v.reshape(rows, k // 32, 32)
    words = np.zeros((rows, k // 32, 3), dtype=np.uint64)  # 64-bit words: 32 values = 192 bits
    for j in range(32):
        bit = 6 * j
        words[:, :, bit // 64] |= v[:, :, j] << np.uint64(bit % 64)
        if bit % 64 > 58:
            words[:, :, bit // 64 + 1] |= v[:, :, j] >> np.uint64(64 - bit % 64)
    return words.reshape(rows, -1).view(np.uint8).reshape(rows, k * 3 // 4)


def f6_untile_numpy(buf: np.ndarray, rows: int, k: int) -> np.ndarray:
    """bf6 rows [rows][k*3/4] of the bf6 activation layout: blocks of 128 rows
    x 128 k (96-byte rows, 12 KiB) at ((r // 128) * (k // 128) + k // 128) *
    12288, row r % 128 of a block at (r % 128) * 96; padding rows dropped."""
    rb = (rows + 127) // 128
    assert buf.size >= rb * 128 * k * 3 // 4
    blocks = buf[: rb * 128 * k * 3 // 4].reshape(rb, k // 128, 128, 96)
    return blocks.transpose(0, 2, 1, 3).reshape(rb * 128, k * 3 // 4)[:rows]


def test_f6_untile_numpy_places_blocks():
    """The layout helper on a buffer whose bytes name their own position:
    byte j of row r's 96-byte piece of k-block b sits at ((r // 128) * kb + b)
    * 12288 + (r % 128) * 96 + j."""
    rows, k = 300, 384
    kb = k // 128
    buf = np.arange(3 * 128 * k * 3 // 4, dtype=np.int64)
    got = f6_untile_numpy(buf, rows, k)
    for r in (0, 1, 127, 128, 255, 299):
        for b in range(kb):
            want = ((r // 128) * kb + b) * 12288 + (r % 128) * 96 + np.arange(96)
            assert np.array_equal(got[r, 96 * b: 96 * b + 96], want)


def test_f6_converters_match_numpy_layout():
    """Activation in 128-row x 128-k blocks of plainly packed 96-byte rows;
    tiled weight in the same blocks with chunk c of block row r at
    c ^ ((r >> 3) & 1)."""
    rng = np.random.default_rng(61)
    m, n, k = 37, 256, 768
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    a_codes = a_codes.copy()
    a_codes[0, : k // 8] = 0x89ABCDEF  # every negative code, -8 included
    storage = np.concatenate([a_codes.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    got = clef_i4.f6_activation(a).cpu().numpy()
    assert got.size == clef_i4.f6_codes_bytes(m, k) == 128 * k * 3 // 4
    assert np.array_equal(f6_untile_numpy(got, m, k), f6_rows_numpy(a_codes, k))
    # weight: untile the reference layout to rows, pack, then block + swizzle
    kb4 = k // 256
    rows_u32 = w_tiled.reshape(n // 128, kb4, 128, 32).transpose(0, 2, 1, 3).reshape(n, k // 8)
    flat = f6_rows_numpy(rows_u32, k)  # [n][k*3/4]
    blocks = flat.reshape(n // 128, 128, k // 128, 6, 16)  # panel, row, k-block, chunk, byte
    swz = np.empty_like(blocks)
    for r in range(128):
        s = (r >> 3) & 1
        for c in range(6):
            swz[:, r, :, c ^ s] = blocks[:, r, :, c]
    want_w = swz.transpose(0, 2, 1, 3, 4).reshape(-1)
    qw = dev_weight(w_tiled, w_scales, n, k)
    got_w = clef_i4.f6_weight(qw).codes.cpu().numpy()
    assert np.array_equal(got_w, want_w)


@pytest.mark.parametrize("m,n,k", [(1, 256, 256), (17, 256, 768), (128, 512, 2048), (300, 768, 1024),
                                   (257, 512, 4096), (64, 1024, 12288)])
def test_gemm_f6_matches_oracle(m, n, k):
    rng = np.random.default_rng(m * 11 + n + k)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    a = dev_prepared(x, stride)
    fw = clef_i4.f6_weight(dev_weight(w_tiled, w_scales, n, k))
    got = clef_i4.project_prepared_f6(a, fw)
    assert_same_u16(bf16_host(got), want, f"gemm_f6 m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 129, 256, 257, 4032])
def test_gemm_f6_residual_matches_oracle(m):
    n, k = 256, 1024
    rng = np.random.default_rng(m + 5)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    res = randn_bf16(rng, (m, n), std=4.0)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k, residual=res)
    a = dev_prepared(x, stride)
    fw = clef_i4.f6_weight(dev_weight(w_tiled, w_scales, n, k))
    got = clef_i4.project_prepared_f6(a, fw, residual=to_dev_bf16(res))
    assert_same_u16(bf16_host(got), want, f"gemm_f6 residual m={m}")


@pytest.mark.parametrize("resid", [False, True])
def test_gemm_f6_several_tiles_per_workgroup(resid):
    """M8292 N4096 K512: 33 x 16 tiles, two or three per persistent
    workgroup, ragged last row tile; the whole output equals G1's."""
    m, n, k = 8292, 4096, 512
    rng = np.random.default_rng(77 + resid)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    res = to_dev_bf16(randn_bf16(rng, (m, n), std=2.0)) if resid else None
    want = bf16_host(clef_i4.project_prepared(a, qw, residual=res))
    got = bf16_host(clef_i4.project_prepared_f6(a, clef_i4.f6_weight(qw), residual=res))
    assert_same_u16(got, want, f"gemm_f6 several tiles resid={resid}")
    rows = [0, 1, 255, 256, 4097, 8191, 8291]
    sub = oracle.gemm(a_codes[rows], a_scales[rows], w_tiled, w_scales, n, k,
                      residual=bf16_host(res)[rows] if resid else None)
    assert_same_u16(got[rows], sub, "gemm_f6 sampled rows vs oracle")


def test_gemm_f6_extreme_codes_and_saturation():
    """Codes -8 and +7 (|acc| up to 64 K), huge scales (clamp), infinite and
    NaN activation scales, as test_gemm_extreme_codes_and_saturation."""
    m, n, k = 64, 256, 4096
    stride = oracle.activation_stride(k)
    a_words = np.full((m, stride // 8), 0x77777777, dtype=np.uint32)
    a_words[1::2, : k // 8] = 0x88888888  # -8
    w_codes = np.full((n, stride // 8), 0x88888888, dtype=np.uint32)
    w_codes[::3, : k // 8] = 0x77777777
    w_codes[1::7, : k // 8] = 0x0F1E2D3C
    w_tiled = oracle.retile(w_codes, k)
    a_scales = np.full(m, 1e30, dtype=np.float32)
    a_scales[5] = np.inf
    a_scales[6] = np.nan
    a_scales[7] = 1e-3
    a_scales[8:12] = [1e-38, 2e-45, 0.0, -3.0]
    w_scales = np.full(n, 1e10, dtype=np.float32)
    w_scales[::5] = 1e-30
    want = oracle.gemm(a_words, a_scales, w_tiled, w_scales, n, k)
    storage = np.concatenate([a_words.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    got = clef_i4.project_prepared_f6(a, clef_i4.f6_weight(dev_weight(w_tiled, w_scales, n, k)))
    assert_same_bf16_nan_aware(bf16_host(got), want, "gemm_f6 extreme")


def test_gemm_f6_zero_rows_give_positive_zero():
    """An all-zero activation row against negative weights: the MFMA's f32 sum
    of -0 products is -0, and the epilogue's + 0 must still give +0 as G1's
    integer accumulator does."""
    m, n, k = 3, 256, 512
    stride = oracle.activation_stride(k)
    a_words = np.zeros((m, stride // 8), dtype=np.uint32)
    a_words[1, : k // 8] = 0x11111111
    w_codes = np.full((n, stride // 8), 0x99999999, dtype=np.uint32)
    w_tiled = oracle.retile(w_codes, k)
    a_scales = np.ones(m, dtype=np.float32)
    w_scales = np.ones(n, dtype=np.float32)
    want = oracle.gemm(a_words, a_scales, w_tiled, w_scales, n, k)
    assert (want[0] == 0).all() and (want[2] == 0).all()
    storage = np.concatenate([a_words.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    got = clef_i4.project_prepared_f6(a, clef_i4.f6_weight(dev_weight(w_tiled, w_scales, n, k)))
    assert_same_u16(bf16_host(got), want, "gemm_f6 zero rows")


def assert_prepared_f6(got, codes_u32: np.ndarray, scales: np.ndarray, what: str):
    """A PreparedF6 holds the oracle's INT4 codes as bf6 (untiled from the
    activation layout) and its scales, byte for byte; the buffer is exactly
    clef_i4_f6_prepared_bytes long."""
    rows, width = got.rows, got.width
    buf = got.storage.cpu().numpy()
    assert buf.size == clef_i4.lib().clef_i4_f6_prepared_bytes(rows, width) == \
        clef_i4.f6_codes_bytes(rows, width) + 4 * rows, what
    assert np.array_equal(f6_untile_numpy(buf, rows, width), f6_rows_numpy(codes_u32, width)), what
    start = clef_i4.f6_codes_bytes(rows, width)
    assert np.array_equal(buf[start:start + 4 * rows].view(np.uint32),
                          np.ascontiguousarray(scales, dtype=np.float32).view(np.uint32)), what


@pytest.mark.parametrize("width,rows", [(256, 5), (768, 37), (2048, 1000), (4096, 33), (8192, 3), (17408, 7)])
def test_prepare_f6_matches_oracle(width, rows):
    """The bf6 quantizer writes the oracle's INT4 codes as e3m2 and its
    scales, byte for byte: both the grid-stride kernel (width <= 4096) and the
    one-row kernel (more than 16 groups), random rows and the exceptional
    rows (NaN, inf, bf16::MAX, zero)."""
    rng = np.random.default_rng(width + rows)
    x = np.concatenate([randn_bf16(rng, (rows, width), std=3.0), exceptional_rows(width)])
    stride = oracle.activation_stride(width)
    codes, scales, _ = oracle.prepare(x, stride)
    got = clef_i4.prepare_f6(to_dev_bf16(x))
    assert_prepared_f6(got, codes, scales, f"prepare_f6 width={width} rows={rows}")


@pytest.mark.parametrize("width", [768, 2048, 17408])
def test_prepare_swiglu_f6_matches_oracle(width):
    rng = np.random.default_rng(width + 3)
    rows = 19
    g = randn_bf16(rng, (rows, width), std=2.0)
    u = randn_bf16(rng, (rows, width), std=2.0)
    stride = oracle.activation_stride(width)
    codes, scales, _ = oracle.prepare_swiglu(g, u, stride)
    got = clef_i4.prepare_swiglu_f6(to_dev_bf16(g), to_dev_bf16(u))
    assert_prepared_f6(got, codes, scales, f"prepare_swiglu_f6 width={width}")


def test_prepare_f6_equals_prepare_then_convert():
    """M4096 K4096 (the benchmark activation): one pass gives what
    clef_i4_prepare + clef_i4_f6_activation give, codes and scales."""
    x = torch.randn((4096, 4096), generator=torch.Generator(device=DEV).manual_seed(5), device=DEV,
                    dtype=torch.float32).to(torch.bfloat16)
    a = clef_i4.prepare(x)
    f = clef_i4.prepare_f6(x)
    assert torch.equal(f.codes, clef_i4.f6_activation(a))
    assert torch.equal(f.scales.view(torch.int32), a.scales.view(torch.int32))


@pytest.mark.parametrize("m,n,k,resid", [(1, 256, 256, False), (300, 768, 1024, True), (257, 512, 4096, False)])
def test_project_f6_matches_oracle(m, n, k, resid):
    """bf16 x -> prepare_f6 -> gemm_f6 against the oracle's quantize + G1."""
    rng = np.random.default_rng(m + n + k)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    res = randn_bf16(rng, (m, n), std=4.0) if resid else None
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k, residual=res)
    fw = clef_i4.f6_weight(dev_weight(w_tiled, w_scales, n, k))
    got = clef_i4.project_f6(clef_i4.prepare_f6(to_dev_bf16(x)), fw,
                             residual=to_dev_bf16(res) if resid else None)
    assert_same_u16(bf16_host(got), want, f"project_f6 m={m} n={n} k={k} resid={resid}")


# ---------------------------------------------------------------- fused gate/up (bf6)

def _gate_up_operands(rng, m, n, k, gate_row_scale=None):
    x = randn_bf16(rng, (m, k))
    wg = randn_bf16(rng, (n, k), std=0.02)
    wu = randn_bf16(rng, (n, k), std=0.02)
    if gate_row_scale is not None:  # per-row multipliers of the gate weight
        wg = oracle.f32_to_bf16(oracle.bf16_to_f32(wg) * gate_row_scale[:, None].astype(np.float32))
    return x, wg, wu


@pytest.mark.parametrize("m,n,k", [(1, 128, 256), (300, 384, 512), (257, 256, 2048), (512, 1152, 4096),
                                   (96, 768, 1024)])
def test_gemm_f6_gate_up_matches_oracle(m, n, k):
    """h = S1(G1(gate), G1(up)) in one bf6 GEMM against the oracle's two
    projections and S1, and, where the separate bf6 GEMM takes the width
    (n % 256 == 0), bit-equal to the unfused library path (two bf6 GEMMs, then
    clef_swiglu); ragged m and h widths of 1, 2, 3, 6 and 9 panels."""
    rng = np.random.default_rng(31 * m + n + k)
    x, wg, wu = _gate_up_operands(rng, m, n, k)
    stride = oracle.activation_stride(k)
    a_codes, a_scales, _ = oracle.prepare(x, stride)
    g_tiled, g_scales = oracle.pack_weight(wg)
    u_tiled, u_scales = oracle.pack_weight(wu)
    want = oracle.swiglu(oracle.gemm(a_codes, a_scales, g_tiled, g_scales, n, k),
                         oracle.gemm(a_codes, a_scales, u_tiled, u_scales, n, k))
    fg = clef_i4.f6_weight(dev_weight(g_tiled, g_scales, n, k))
    fu = clef_i4.f6_weight(dev_weight(u_tiled, u_scales, n, k))
    a = clef_i4.prepare_f6(to_dev_bf16(x))
    got = clef_i4.project_gate_up_f6(a, fg, fu)
    assert_same_u16(bf16_host(got), want, f"gate_up m={m} n={n} k={k}")
    if n % 256 == 0:
        unfused = clef_i4.swiglu(clef_i4.project_f6(a, fg), clef_i4.project_f6(a, fu))
        assert_same_u16(bf16_host(got), bf16_host(unfused), f"gate_up vs unfused m={m} n={n} k={k}")


def test_gemm_f6_gate_up_silu_window_edges():
    """Gate rows scaled so that g falls below the SiLU table window (|g| <
    2^-10: the g/2 form), far above it (|g| >= 64: the exact silu), and a NaN
    and an infinite activation row (the slow epilogue and the exact silu on
    non-finite g), all bit-equal to the unfused path and to the oracle."""
    m, n, k = 200, 256, 1024
    rng = np.random.default_rng(7)
    row_scale = np.ones(n, dtype=np.float32)
    row_scale[0:48] = 1e-4      # |g| ~ 1e-4
    row_scale[48:64] = 1e-6     # |g| ~ 1e-6
    row_scale[64:96] = 300.0    # |g| ~ 300
    row_scale[96:100] = 0.0     # g = 0 exactly
    x, wg, wu = _gate_up_operands(rng, m, n, k, gate_row_scale=row_scale)
    x[5, :] = 0x7FC0            # NaN row
    x[9, 3] = 0x7F80            # an infinite value
    x[11, :] = 0x8000           # -0 row
    stride = oracle.activation_stride(k)
    a_codes, a_scales, _ = oracle.prepare(x, stride)
    g_tiled, g_scales = oracle.pack_weight(wg)
    u_tiled, u_scales = oracle.pack_weight(wu)
    gate = oracle.gemm(a_codes, a_scales, g_tiled, g_scales, n, k)
    gf = np.abs(oracle.bf16_to_f32(gate[np.isfinite(oracle.bf16_to_f32(gate))]))
    assert (gf[gf > 0] < 2.0 ** -10).any() and (gf >= 64).any(), "the case must reach both sides of the window"
    want = oracle.swiglu(gate, oracle.gemm(a_codes, a_scales, u_tiled, u_scales, n, k))
    fg = clef_i4.f6_weight(dev_weight(g_tiled, g_scales, n, k))
    fu = clef_i4.f6_weight(dev_weight(u_tiled, u_scales, n, k))
    a = clef_i4.prepare_f6(to_dev_bf16(x))
    got = clef_i4.project_gate_up_f6(a, fg, fu)
    unfused = clef_i4.swiglu(clef_i4.project_f6(a, fg), clef_i4.project_f6(a, fu))
    assert_same_u16(bf16_host(got), bf16_host(unfused), "gate_up window edges vs unfused")
    assert_same_u16(bf16_host(got), want, "gate_up window edges vs oracle")


def test_gemm_f6_gate_up_rejects():
    fw = clef_i4.F6Weight(torch.zeros(192 * 256 * 3 // 4, dtype=torch.uint8, device="cuda"),
                          torch.ones(192, device="cuda"), 192, 256)
    a = clef_i4.prepare_f6(torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(clef_i4.ClefError, match="unsupported integer projection shape"):
        clef_i4.project_gate_up_f6(a, fw, fw)  # 192 columns: not whole 128-column panels


# ---------------------------------------------------------------- decode-sized G1
# Configuration 4: v_dot8_i32_i4 on the packed codes for m <= 8.

@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("n,k", [(128, 256), (256, 768), (384, 2304), (1024, 4096), (128, 12544)])
def test_gemm_decode_matches_oracle(m, n, k):
    """Few rows against the oracle, with and without the residual: one
    k-step (fewer than the kernel's eight waves), k-step counts that leave
    some waves a round short (9, 49), ragged m inside the 4- and 8-row forms."""
    rng = np.random.default_rng(m * 1000 + n + k)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    assert_same_u16(bf16_host(clef_i4.project_prepared(a, qw, config=4)), want, f"decode m={m} n={n} k={k}")
    res = randn_bf16(rng, (m, n), std=3.0)
    want_r = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k, residual=res)
    got_r = clef_i4.project_prepared(a, qw, residual=to_dev_bf16(res), config=4)
    assert_same_u16(bf16_host(got_r), want_r, f"decode residual m={m} n={n} k={k}")
    if m <= 4:  # the automatic choice
        assert_same_u16(bf16_host(clef_i4.project_prepared(a, qw)), want, f"auto m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 4, 8])
def test_gemm_decode_extreme_codes_and_scales(m):
    """Codes -8 and +7 (|acc| up to 8 * 8 * 4096), huge, infinite, NaN, zero,
    negative and tiny scales through the dot-product kernel."""
    n, k = 256, 4096
    stride = oracle.activation_stride(k)
    a_words = np.full((m, stride // 8), 0x88888888, dtype=np.uint32)
    a_words[1::2, : k // 8] = 0x77777777
    w_codes = np.full((n, stride // 8), 0x88888888, dtype=np.uint32)
    w_codes[::3, : k // 8] = 0x77777777
    w_codes[1::7, : k // 8] = 0x0F1E2D3C
    w_tiled = oracle.retile(w_codes, k)
    a_scales = np.array([1e30, 1e-3, np.inf, np.nan, 0.0, -3.0, 1e-38, 2e-45][:m], dtype=np.float32)
    w_scales = np.full(n, 1e10, dtype=np.float32)
    w_scales[::5] = 1e-30
    w_scales[2::11] = 0.0
    want = oracle.gemm(a_words, a_scales, w_tiled, w_scales, n, k)
    storage = np.concatenate([a_words.reshape(-1), a_scales.view(np.uint32)])
    a = clef_i4.Prepared(to_dev_u32(storage), m, k, stride, 4)
    got = clef_i4.project_prepared(a, dev_weight(w_tiled, w_scales, n, k), config=4)
    assert_same_bf16_nan_aware(bf16_host(got), want, f"decode extreme m={m}")


# ---------------------------------------------------------------- split-K tiles
# Configuration 5: 64x64, 32x64 or 32x32 tiles (chosen by shape) whose
# k-steps are shared among the workgroup's eight waves.

@pytest.mark.parametrize("m,n,k", [
    (100, 8192, 768),     # 64x64 tiles, 3 k-steps for 8 waves, ragged last row tile
    (512, 2048, 2048),    # 64x64 tiles: the 512 x 2048 x 2048 linear
    (65, 12288, 256),     # 64x64 tiles, one k-step (seven waves without one)
    (200, 4096, 4864),    # 64x64 tiles, 19 k-steps (waves with 2 and 3 k-steps)
    (64, 12288, 4096),    # 64x64 tiles, exactly one row tile
    (20, 12288, 2304),    # 32x64 tiles (m <= 32), 9 k-steps
    (40, 1024, 12544),    # 32x32 tiles, two stages per wave, 49 k-steps
    (9, 128, 256),        # one k-step, one tile column
    (300, 384, 1024),
])
def test_gemm_ksplit_matches_oracle(m, n, k):
    rng = np.random.default_rng(m * 3 + n + k)
    x, w, stride, a_codes, a_scales, w_tiled, w_scales = make_operands(rng, m, n, k)
    a = dev_prepared(x, stride)
    qw = dev_weight(w_tiled, w_scales, n, k)
    want = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k)
    assert_same_u16(bf16_host(clef_i4.project_prepared(a, qw, config=5)), want, f"ksplit m={m} n={n} k={k}")
    res = randn_bf16(rng, (m, n), std=3.0)
    want_r = oracle.gemm(a_codes, a_scales, w_tiled, w_scales, n, k, residual=res)
    got_r = clef_i4.project_prepared(a, qw, residual=to_dev_bf16(res), config=5)
    assert_same_u16(bf16_host(got_r), want_r, f"ksplit residual m={m} n={n} k={k}")
    assert_same_u16(bf16_host(clef_i4.project_prepared(a, qw)), want, f"auto m={m} n={n} k={k}")


@pytest.mark.parametrize("m,n,k,resid", [(5, 256, 512, True), (1000, 768, 2048, False)])
def test_project_quantized_f6_matches_project_quantized(m, n, k, resid):
    """clef_i4_project_f6 (bf6 quantize + GEMM in one call) against
    clef_i4_project on the same bf16 input and weight, bit for bit."""
    rng = np.random.default_rng(m + k)
    x = to_dev_bf16(randn_bf16(rng, (m, k)))
    qw = clef_i4.load_quantized_weight(to_dev_bf16(randn_bf16(rng, (n, k), std=0.02)))
    res = to_dev_bf16(randn_bf16(rng, (m, n))) if resid else None
    want = bf16_host(clef_i4.project_quantized(x, qw, residual=res))
    got = bf16_host(clef_i4.project_quantized_f6(x, clef_i4.f6_weight(qw), residual=res))
    assert_same_u16(got, want, f"project_quantized_f6 m={m} n={n} k={k}")


@pytest.mark.parametrize("forms", [("int4",), ("bf6",), ("int4", "bf6")])
def test_projection_forms_resident_bytes_and_output(forms):
    """QuantizedProjections.pack keeps exactly the forms asked for, their
    buffers add up to resident_bytes, and a projection through either form
    gives the reference-format GEMM's output bit for bit."""
    name = "model.language_model.layers.0.mlp.gate_proj.weight"
    n, k, m = 512, 1024, 40
    rng = np.random.default_rng(77)
    w = to_dev_bf16(randn_bf16(rng, (n, k), std=0.02))
    x = to_dev_bf16(randn_bf16(rng, (m, k)))
    policy = clef_i4.QuantizedProjections.for_precision("int4_mlp", forms=forms)
    packed = policy.pack(w, name)
    assert set(packed) == set(forms)
    held = sum(t.numel() * t.element_size() for p in packed.values() for t in (p.codes,))
    held += n * 4  # the shared row scales
    assert held == policy.resident_bytes(name, n, k)
    want = clef_i4.project_prepared(clef_i4.prepare(x), clef_i4.load_quantized_weight(w))
    if "int4" in packed:
        got = clef_i4.project_prepared(clef_i4.prepare(x), packed["int4"])
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    if "bf6" in packed:
        got = clef_i4.project_f6(clef_i4.prepare_f6(x), packed["bf6"])
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
