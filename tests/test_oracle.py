"""Pin the C oracle against the reference's own test formulas, closed forms and
brute force. CPU only.

Each test names the reference test or kernel whose behaviour it checks.
"""
import math

import numpy as np
import pytest

import oracle

BF = oracle.f32_to_bf16
F = oracle.bf16_to_f32


def kron_rotation() -> np.ndarray:
    """The radix-4 stage is the 4x4 matrix below on one base-4 digit of the
    index; four stages give its 4-fold Kronecker power
    (kernels/prepare_integer_single.loom:109-116)."""
    m4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = m4
    for _ in range(3):
        h = np.kron(h, m4)
    return h


# ---------------------------------------------------------------- rotation

def test_rotation_is_kronecker_power_and_orthogonal():
    h = kron_rotation()
    assert np.array_equal(h @ h.T, 256.0 * np.eye(256))
    for i in range(256):
        e = np.zeros(256, dtype=np.float32)
        e[i] = 1.0
        assert np.array_equal(oracle.rotate256(e), h[:, i].astype(np.float32)), i


def test_rotation_exact_on_representable_inputs():
    # multiples of 2^-8 bounded by 4: every partial sum fits in 24 bits, so the
    # f32 radix-4 result equals the float64 matrix product exactly.
    rng = np.random.default_rng(7)
    h = kron_rotation()
    for _ in range(20):
        x = (rng.integers(-1024, 1024, size=256) / 256.0).astype(np.float32)
        assert np.array_equal(oracle.rotate256(x).astype(np.float64), h @ x.astype(np.float64))


def test_rotation_preserves_inner_product():
    """src/quantized.rs:858-876."""
    a = F(BF(np.array([((i * 17 % 71) - 35.0) / 64.0 for i in range(512)], dtype=np.float32)))
    b = F(BF(np.array([((i * 31 % 59) - 29.0) / 64.0 for i in range(512)], dtype=np.float32)))
    expected = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    ra = np.concatenate([oracle.rotate256(a[:256]), oracle.rotate256(a[256:])])
    rb = np.concatenate([oracle.rotate256(b[:256]), oracle.rotate256(b[256:])])
    actual = float(np.sum(ra.astype(np.float64) * rb.astype(np.float64) / 256.0))
    assert abs(actual - expected) < 1e-8


# ---------------------------------------------------------------- Q1

def decode_codes(words: np.ndarray, width: int, bits: int = 4) -> np.ndarray:
    per = 32 // bits
    w = words[:, : width // per].astype(np.uint64)
    shifts = (np.arange(per, dtype=np.uint64) * bits)
    vals = ((w[:, :, None] >> shifts) & ((1 << bits) - 1)).astype(np.int64)
    vals = np.where(vals >= (1 << (bits - 1)), vals - (1 << bits), vals)
    return vals.reshape(words.shape[0], width)


def reference_test_quantize(row_f32: np.ndarray, bits: int):
    """The reference test oracle, src/quantized.rs:1094-1113 (f32 numpy)."""
    width = row_f32.shape[0]
    rot = np.concatenate([oracle.rotate256(row_f32[g:g + 256]) for g in range(0, width, 256)])
    max_code = np.float32((1 << (bits - 1)) - 1)
    m = np.float32(np.max(np.abs(rot))) if width else np.float32(0)
    scale = np.float32(max(np.float32(m / np.float32(16.0)), np.float32(1e-30)) / max_code)
    inv = np.float32(np.float32(0.0625) / scale)
    codes = np.clip(np.rint((rot * inv).astype(np.float32)), -max_code, max_code).astype(np.int64)
    return codes, scale


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("width", [256, 768, 1280, 2048, 5120, 6144, 8192, 17408])
def test_prepare_matches_reference_test_oracle(bits, width):
    """rotated_packing_cpu_oracle inputs: zero row, e_0, ((i*37%257)-128)/91
    (src/quantized.rs:1074-1129)."""
    vals = np.zeros((3, width), dtype=np.float32)
    vals[1, 0] = 1.0
    vals[2] = [((i * 37 % 257) - 128.0) / 91.0 for i in range(width)]
    x = BF(vals)
    stride = width + 512 // bits
    codes, scales, _ = oracle.prepare(x, stride, bits)
    for row in range(3):
        want_codes, want_scale = reference_test_quantize(F(x[row]), bits)
        assert scales[row] == want_scale, (row, scales[row], want_scale)
        got = decode_codes(codes[row:row + 1], width, bits)[0]
        assert np.array_equal(got, want_codes), row


def test_prepare_closed_forms():
    h = kron_rotation()
    width = 256
    x = np.zeros((4, width), dtype=np.float32)
    x[0, 0] = 1.0          # e_0: rotated row is column 0 of H, all +-1
    x[1, :] = 2.0          # constant: H.1 = 16.1, so every code is +7
    x[2, 5] = -0.5
    x[3, :] = 0.0          # zero row: scale = 1e-30/7, codes 0
    codes, scales, _ = oracle.prepare(BF(x), 384, 4)
    c = decode_codes(codes, width)
    s7 = np.float32(np.float32(0.0625) / np.float32(7.0))
    assert scales[0] == s7 and np.array_equal(c[0], 7 * h[:, 0].astype(np.int64))
    assert scales[1] == np.float32(np.float32(2.0) / np.float32(7.0)) and np.all(c[1] == 7)
    assert np.array_equal(c[2], -7 * h[:, 5].astype(np.int64))
    assert scales[3] == np.float32(np.float32(1e-30) / np.float32(7.0)) and np.all(c[3] == 0)


def exceptional_rows(width: int) -> np.ndarray:
    """The seven rows of register_packing_matches_reference
    (src/quantized.rs:1138-1150): 0, 1, ((c*37%257)-128)/91, -0.5 with NaN at
    column 259, -0.5 with +inf at column 515, bf16::MAX, bf16 denormal."""
    x = np.full((7, width), BF(np.float32(-0.5)), dtype=np.uint16)
    x[0, :] = 0
    x[1, :] = BF(np.float32(1.0))
    x[2, :] = BF(np.array([((c * 37 % 257) - 128.0) / 91.0 for c in range(width)], np.float32))
    x[3, 259] = 0x7FC0
    x[4, 515] = 0x7F80
    x[5, :] = 0x7F7F
    x[6, :] = 0x0001
    return x


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("width", [768, 5120, 6144, 17408])
def test_prepare_exceptional_rows(bits, width):
    """NaN or Inf anywhere in a row (or an overflowing rotation, as for a row of
    bf16::MAX) -> scale +inf and all-zero codes; the other rows follow the
    reference test oracle."""
    x = exceptional_rows(width)
    codes, scales, _ = oracle.prepare(x, width + 512 // bits, bits)
    c = decode_codes(codes, width, bits)
    for r in (3, 4, 5):
        assert np.isinf(scales[r]) and scales[r] > 0 and np.all(c[r] == 0), r
    for r in (0, 1, 2, 6):
        assert np.isfinite(scales[r]) and scales[r] > 0, r
        want, wscale = reference_test_quantize(F(x[r]), bits)
        assert wscale == scales[r] and np.array_equal(c[r], want), r
    assert np.max(np.abs(c[2])) == (7 if bits == 4 else 127)
    assert np.all(c[6] == 0) and np.all(c[0] == 0)


def test_prepare_padding_words_untouched():
    x = BF(np.ones((2, 1024), dtype=np.float32))
    codes, _, storage = oracle.prepare(x, 1024 + 128, 4)
    assert np.all(codes[:, 128:] == 0)  # storage was zero-filled; padding unwritten


# ---------------------------------------------------------------- Q2

def test_retile_block_formula():
    """retiled_codes_match_block_formula (src/quantized.rs:1371-1407)."""
    rows, cols = 256, 512
    words = cols // 8
    in_words = words + 16
    codes = (np.arange(rows)[:, None] * 100000 + np.arange(in_words)[None, :]).astype(np.uint32)
    tiled = oracle.retile(codes, cols)
    assert tiled.shape == (rows * words,)
    for n in range(rows):
        for q in range(words):
            idx = ((n // 128) * (words // 32) + q // 32) * 4096 + (n % 128) * 32 + q % 32
            assert tiled[idx] == codes[n, q]
    # a permutation of the logical words; padding dropped
    assert np.array_equal(np.sort(tiled), np.sort(codes[:, :words].ravel()))


def test_retile_rejects_bad_shapes():
    with pytest.raises(oracle.OracleError, match="unsupported packed weight shape for tiling"):
        oracle.retile(np.zeros((100, 64), np.uint32), 512)


# ---------------------------------------------------------------- G1

def random_codes(rng, rows, width, stride):
    vals = rng.integers(-7, 8, size=(rows, width))
    words = np.zeros((rows, stride // 8), dtype=np.uint32)
    nib = (vals & 0xF).astype(np.uint32).reshape(rows, width // 8, 8)
    words[:, : width // 8] = np.bitwise_or.reduce(nib << (np.arange(8, dtype=np.uint32) * 4), axis=2)
    return vals, words


def test_gemm_acc_brute_force():
    rng = np.random.default_rng(3)
    m, n, k = 37, 256, 768
    a_vals, a_words = random_codes(rng, m, k, k + 0)
    w_vals, w_words = random_codes(rng, n, k, k)
    tiled = oracle.retile(w_words, k)
    acc = oracle.gemm_acc(a_words, tiled, n, k)
    assert np.array_equal(acc.astype(np.int64), a_vals @ w_vals.T)


def random_codes8(rng, rows, width, stride):
    """INT8 codes in [-127, 127], four per word (byte p of word q = column 4q + p)."""
    vals = rng.integers(-127, 128, size=(rows, width))
    words = np.zeros((rows, stride // 4), dtype=np.uint32)
    byt = (vals & 0xFF).astype(np.uint32).reshape(rows, width // 4, 4)
    words[:, : width // 4] = np.bitwise_or.reduce(byt << (np.arange(4, dtype=np.uint32) * 8), axis=2)
    return vals, words


def untile(tiled: np.ndarray, rows: int, words: int) -> np.ndarray:
    """Inverse of the retile block formula (src/quantized.rs:1394-1397) for
    `words` logical words per row, whatever the codes per word."""
    n = np.arange(rows)[:, None]
    q = np.arange(words)[None, :]
    idx = ((n // 128) * (words // 32) + q // 32) * 4096 + (n % 128) * 32 + q % 32
    return tiled[idx]


def test_retile_block_formula_bits8():
    """The same block formula with four codes per word: K = 512 gives 128
    words per row, four 32-word blocks."""
    rows, cols = 256, 512
    words = cols // 4
    codes = (np.arange(rows)[:, None] * 100000 + np.arange(words + 16)[None, :]).astype(np.uint32)
    tiled = oracle.retile(codes, cols, bits=8)
    assert tiled.shape == (rows * words,)
    assert np.array_equal(untile(tiled, rows, words), codes[:, :words])


@pytest.mark.parametrize("m,n,k", [(37, 256, 768), (5, 128, 256)])
def test_gemm_acc_brute_force_bits8(m, n, k):
    """G1 accumulators at bits 8 (h3_gemm_i8_256, kernels/gemm_integer.loom:454-485):
    exact i32 sums of int8 products, the weight read back through the tiled
    layout. Codes of +-127 in every slot bound |acc| by 127^2 * k."""
    rng = np.random.default_rng(11)
    a_vals, a_words = random_codes8(rng, m, k, k + 64)
    w_vals, w_words = random_codes8(rng, n, k, k)
    a_vals[0, :] = 127
    w_vals[0, :] = -127
    a_words[0, : k // 4] = np.uint32(0x7F7F7F7F)
    w_words[0, : k // 4] = np.uint32(0x81818181)
    tiled = oracle.retile(w_words, k, bits=8)
    acc = oracle.gemm_acc(a_words, tiled, n, k, bits=8)
    assert np.array_equal(acc.astype(np.int64), a_vals @ w_vals.T)
    assert acc[0, 0] == -127 * 127 * k


def test_pack_weight_bits8_is_quantizer_then_block_formula():
    """Q2 at bits 8 (Engine::load_quantized_weight, src/quantized.rs:147-234):
    each row's codes, read back through the block formula, are the reference
    test quantizer's (src/quantized.rs:1092-1113) of that row, and the scales
    are its scales."""
    rows, cols = 256, 1024
    w = BF(np.array([[((i * 37 + 11 * r) % 257 - 128) / 91.0 for i in range(cols)] for r in range(rows)],
                    dtype=np.float32))
    tiled, scales = oracle.pack_weight(w, bits=8)
    words = untile(tiled, rows, cols // 4)
    got = decode_codes(words, cols, 8)
    for r in range(rows):
        want_codes, want_scale = reference_test_quantize(F(w[r]), 8)
        assert np.array_equal(got[r], want_codes), r
        assert np.float32(scales[r]) == np.float32(want_scale), r


def test_gemm_epilogue_power_of_two_scales_bits8():
    """The G1 epilogue on bits-8 accumulators: with power-of-two scales every
    step before the bf16 rounding is exact."""
    rng = np.random.default_rng(12)
    m, n, k = 16, 128, 512
    a_vals, a_words = random_codes8(rng, m, k, k + 64)
    w_vals, w_words = random_codes8(rng, n, k, k)
    tiled = oracle.retile(w_words, k, bits=8)
    a_s = (2.0 ** rng.integers(-12, 0, size=m)).astype(np.float32)
    w_s = (2.0 ** rng.integers(-12, 0, size=n)).astype(np.float32)
    out = oracle.gemm(a_words, a_s, tiled, w_s, n, k, bits=8)
    exact = (a_vals @ w_vals.T).astype(np.float64) * w_s[None, :].astype(np.float64) * a_s[:, None]
    assert np.array_equal(out, BF(exact.astype(np.float32)))


def test_gemm_epilogue_power_of_two_scales():
    rng = np.random.default_rng(4)
    m, n, k = 16, 128, 256
    a_vals, a_words = random_codes(rng, m, k, k + 128)
    w_vals, w_words = random_codes(rng, n, k, k)
    tiled = oracle.retile(w_words, k)
    a_s = (2.0 ** rng.integers(-10, 3, size=m)).astype(np.float32)
    w_s = (2.0 ** rng.integers(-10, 3, size=n)).astype(np.float32)
    out = oracle.gemm(a_words, a_s, tiled, w_s, n, k)
    exact = (a_vals @ w_vals.T).astype(np.float64) * w_s[None, :].astype(np.float64) * a_s[:, None]
    assert np.array_equal(out, BF(exact.astype(np.float32)))  # exact before the bf16 step
    # residual: bf16(f32(res) + f32(out))
    res = BF(rng.standard_normal((m, n)).astype(np.float32))
    out_r = oracle.gemm(a_words, a_s, tiled, w_s, n, k, residual=res)
    assert np.array_equal(out_r, BF(F(res) + F(out)))


def test_gemm_saturation_and_nonfinite_rows():
    k, n = 256, 128
    a = np.zeros((3, 256), np.float32)
    a[0, :] = 1.0
    a[1, :] = 1.0
    a[2, 0] = np.nan
    codes, scales, _ = oracle.prepare(BF(a), k, 4)
    w = np.zeros((n, k), np.float32)
    w[:, :] = 1.0
    w_t, w_s = oracle.pack_weight(BF(w))
    acc = oracle.gemm_acc(codes, w_t, n, k)
    r0 = np.float32(np.float32(acc[1, 0]) * w_s[0])
    big = scales.copy()
    big[1] = np.float32(np.float32(3.4e38) / r0)         # finite y above the bf16 range
    y = np.float32(r0 * big[1])
    assert np.isfinite(y) and y > np.float32(3.3895313892515355e38)
    out = F(oracle.gemm(codes, big, w_t, w_s, n, k))
    assert np.all(out[0] == F(BF(np.float32(256.0))))  # 256 ones . ones
    assert np.all(out[1] == F(np.uint16(0x7F7F)))       # finite overflow clamps to bf16::MAX
    assert np.all(np.isnan(out[2]))                     # 0 * inf scale stays observable
    big[1] = np.float32(3e38)                            # f32 overflow is not clamped
    out = F(oracle.gemm(codes, big, w_t, w_s, n, k))
    assert np.all(np.isposinf(out[1]))


def test_identity_weight_round_trip():
    """activation_scratch_is_bounded (src/quantized.rs:880-915): identity
    weights reproduce rows 1 + r/16 exactly through 32 layers."""
    w = np.eye(256, dtype=np.float32)
    w_t, w_s = oracle.pack_weight(BF(w))
    x0 = BF(np.array([[1.0 + r / 16.0] * 256 for r in range(17)], dtype=np.float32))
    x = x0
    for _ in range(32):
        codes, scales, _ = oracle.prepare(x, 256, 4)
        x = oracle.gemm(codes, scales, w_t, w_s, 256, 256)
    assert np.array_equal(x, x0)


def test_packed_weights_cpu_dot_tolerance():
    """packed_weights_survive_plan_reset oracle (src/quantized.rs:979-1070):
    bf16(dot*as*ws) within one bf16 step of the product, on its inputs."""
    vals = F(BF(np.array([((i * 17 % 251) - 125.0) / 128.0 for i in range(256 * 256)], np.float32)))
    w_t, w_s = oracle.pack_weight(BF(vals.reshape(256, 256)))
    xin = F(BF(np.array([((i * 31 % 257) - 128.0) / 64.0 for i in range(18 * 256)], np.float32)))
    codes, scales, _ = oracle.prepare(BF(xin.reshape(18, 256)), 256, 4)
    out = F(oracle.gemm(codes, scales, w_t, w_s, 256, 256))
    acc = oracle.gemm_acc(codes, w_t, 256, 256)
    expected = F(BF((acc.astype(np.float32) * scales[:, None]) * w_s[None, :]))
    assert np.all(np.isfinite(out))
    assert np.all(np.abs(out - expected) <= np.maximum(np.abs(out), np.abs(expected)) / 128 + 1e-6)


# ---------------------------------------------------------------- R1

def router_phase_values(tokens, experts, phase):
    """OmniRouterBenchmark phases (src/benchmarking/omni.rs:42-55)."""
    i = np.arange(tokens * experts)
    if phase == 0:
        v = ((i * 37 + i // experts * 11) % 257) / 16.0 - 8.0
    elif phase == 1:
        v = ((i * 53 + i // experts * 7) % 5) - 2.0
    elif phase == 2:
        v = np.where(i % 2 == 0, 0.0, -0.0)
    else:
        v = ((i * 79 + i // experts * 17) % 263) * 16.0 - 2048.0
    return v.astype(np.float32).reshape(tokens, experts)


@pytest.mark.parametrize("phase", [0, 1, 2, 3])
@pytest.mark.parametrize("bf16_logits", [False, True])
def test_route_matches_stable_sort(phase, bf16_logits):
    tokens, experts, topk = 65, 128, 8
    v = router_phase_values(tokens, experts, phase)
    logits = BF(v) if bf16_logits else v
    if bf16_logits:
        v = F(logits)
    routes = oracle.route(logits, topk)
    for t in range(tokens):
        order = sorted(range(experts), key=lambda e: -float(v[t, e]))  # stable, ties -> lower id
        assert [int(x) for x in routes[t, :topk]] == order[:topk]
        sel = np.array([v[t, e] for e in order[:topk]], dtype=np.float64)
        p = np.exp(sel - sel[0])
        want = p / p.sum()
        got = routes[t, topk:].astype(np.float64)
        # bf16-rounded probabilities: within one bf16 step of the exact value
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)


def test_route_experts_below_128_and_bad_shape():
    v = router_phase_values(3, 60, 0)
    routes = oracle.route(v, 4)
    for t in range(3):
        order = sorted(range(60), key=lambda e: -float(v[t, e]))
        assert [int(x) for x in routes[t, :4]] == order[:4]
    with pytest.raises(oracle.OracleError, match="invalid expert router shape"):
        oracle.route(np.zeros((2, 129), np.float32), 8)


# ---------------------------------------------------------------- R2 / R3

def grouped_phase_routes(tokens, phase, topk=8):
    """grouped_routes_match_cpu (src/omni.rs:908-942)."""
    routes = np.zeros((tokens, 2 * topk), np.float32)
    for t in range(tokens):
        for r in range(topk):
            routes[t, r] = ((0 if phase == 1 else t * 13) + r * 7 + phase * 19) % 128
    return routes


@pytest.mark.parametrize("tokens", [1, 17, 64, 65, 128, 255, 256, 511, 512, 1023, 1024, 2047, 2048])
def test_group_routes_brute_force(tokens):
    for phase in range(3):
        routes = grouped_phase_routes(tokens, phase)
        groups, order = oracle.group_routes(routes)
        expected = [[] for _ in range(128)]
        for t in range(tokens):
            for r in range(8):
                expected[int(routes[t, r])].append(t * 8 + r)
        for e in range(128):
            assert groups[e, 0] == len(expected[e])
            assert np.array_equal(groups[e, 1:1 + len(expected[e])], np.array(expected[e], np.float32))
        # order: ranks sorted by expert id (total order)
        want = np.argsort(routes[:, :8], axis=1, kind="stable")
        assert np.array_equal(order, want.astype(np.float32))
        tasks = oracle.expert_tasks(groups)
        pairs = [(e, 16 * j) for e in range(128) for j in range((len(expected[e]) + 15) // 16)]
        assert tasks[0] == len(pairs)
        assert np.array_equal(tasks[1:1 + 2 * len(pairs)], np.array(pairs, np.float32).ravel())


# ---------------------------------------------------------------- E1

def test_expert_matches_dense_oracle_on_routed_rows():
    rng = np.random.default_rng(11)
    tokens, topk, k, n = 23, 8, 512, 256
    logits = rng.standard_normal((tokens, 128)).astype(np.float32)
    routes = oracle.route(logits, topk)
    groups, _ = oracle.group_routes(routes)
    x = BF(rng.standard_normal((tokens, k)).astype(np.float32))
    codes, scales, _ = oracle.prepare(x, k, 4)
    w = BF((0.02 * rng.standard_normal((128 * n, k))).astype(np.float32))
    w_t, w_s = oracle.pack_weight(w)
    out = oracle.expert_i4(codes, scales, w_t, w_s, groups, tokens, topk, k, n, False)
    acc = oracle.gemm_acc(codes, w_t, 128 * n, k)  # every token x every expert row
    for t in range(tokens):
        for r in range(topk):
            e = int(routes[t, r])
            cols = slice(e * n, (e + 1) * n)
            s = (scales[t] * w_s[cols]).astype(np.float32)
            want = BF((acc[t, cols].astype(np.float32) * s).astype(np.float32))
            assert np.array_equal(out[t * topk + r], want)


def duplicate_routes(rng, tokens, topk=8):
    """Router output with some slots rewritten: a token naming one expert
    twice, a token naming expert 127 in every slot, and slots naming no
    expert (-1.0 and 128.0), which the ungrouped kernel skips."""
    routes = oracle.route(rng.standard_normal((tokens, 128)).astype(np.float32), topk)
    if tokens >= 3:
        routes[0, 3] = routes[0, 1]
        routes[1, :topk] = 127.0
        routes[2, 5] = -1.0
        routes[2, 6] = 128.0
    return routes


@pytest.mark.parametrize("input_routed", [False, True])
def test_expert_ungrouped_matches_grouped_and_dense(input_routed):
    """Engine::omni_expert without groups (src/omni.rs:280-288,
    kernels/omni_expert.loom:86-150): on router output (no duplicates) it
    equals the grouped E1 bit for bit; on routes with a duplicate expert,
    an all-127 token and out-of-range ids every slot naming an expert is the
    dense oracle's value for that expert and row, and the others stay zero."""
    rng = np.random.default_rng(5 + input_routed)
    tokens, topk, k, n = 19, 8, 512, 256
    rows = tokens * topk if input_routed else tokens
    x = BF(rng.standard_normal((rows, k)).astype(np.float32))
    codes, scales, _ = oracle.prepare(x, k, 4)
    w_t, w_s = oracle.pack_weight(BF((0.02 * rng.standard_normal((128 * n, k))).astype(np.float32)))
    routes = oracle.route(rng.standard_normal((tokens, 128)).astype(np.float32), topk)
    groups, _ = oracle.group_routes(routes)
    grouped = oracle.expert_i4(codes, scales, w_t, w_s, groups, tokens, topk, k, n, input_routed)
    assert np.array_equal(oracle.expert_i4_ungrouped(codes, scales, w_t, w_s, routes, k, n, input_routed), grouped)
    routes = duplicate_routes(rng, tokens, topk)
    out = oracle.expert_i4_ungrouped(codes, scales, w_t, w_s, routes, k, n, input_routed)
    acc = oracle.gemm_acc(codes, w_t, 128 * n, k)  # every row x every expert row
    for t in range(tokens):
        for r in range(topk):
            slot = t * topk + r
            xr = slot if input_routed else t
            e = routes[t, r]
            if not (-1.0 < e < 128.0):
                assert np.all(out[slot] == 0)
                continue
            cols = slice(int(e) * n, (int(e) + 1) * n)
            want = BF((acc[xr, cols].astype(np.float32) * (scales[xr] * w_s[cols]).astype(np.float32))
                      .astype(np.float32))
            assert np.array_equal(out[slot], want), (t, r)


# ---------------------------------------------------------------- S1 / exp

def test_expf_within_two_ulp():
    xs = np.concatenate([np.linspace(-103.0, 88.7, 200001, dtype=np.float32),
                         F(np.arange(0, 65536, dtype=np.uint16))])
    xs = xs[np.isfinite(xs) & (xs > -103.0) & (xs < 88.7)]
    got = np.array([oracle.expf(float(x)) for x in xs[::7]], dtype=np.float32)
    want = np.exp(xs[::7].astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    ulp = np.maximum(ulp, 2.0 ** -149)
    assert np.max(np.abs(got - want) / ulp) <= 2.0
    assert oracle.expf(0.0) == 1.0
    assert math.isinf(oracle.expf(100.0)) and oracle.expf(-200.0) == 0.0


def test_swiglu_every_bf16_gate():
    """S1 over every bf16 gate value (kernels/swiglu.loom:43-51) against a
    float64 SiLU: each of the two bf16 roundings adds at most half a step."""
    g = np.arange(65536, dtype=np.uint16)
    gf = F(g).astype(np.float64)
    # exp(-g) overflows f32 below g = -88.72: the f32 formula then gives
    # g / inf = -0, as the reference kernel does.
    overflow = gf < -88.72283935546875
    for u_val in (1.0, -3.5, 0.0078125):
        u = np.full_like(g, BF(np.float32(u_val)))
        h = F(oracle.swiglu(g, u)).astype(np.float64)
        with np.errstate(over="ignore", invalid="ignore"):
            silu = gf / (1.0 + np.exp(-gf))
        want = silu * u_val
        # above the bf16 range the product rounds to +-inf
        big = np.abs(want) >= 3.3961775292304601e38
        assert np.all(np.isinf(h[big & np.isfinite(want)]))
        fin = np.isfinite(want) & np.isfinite(gf) & ~overflow & ~big
        # bf16(silu) then bf16(. * u): half a step each, the first scaled by |u|
        half = 2.0 ** -8
        tol = (abs(u_val) * (np.abs(silu) * half + 2.0 ** -134)
               + np.abs(want) * (half + 2.0 ** -20) + 2.0 ** -134)
        assert np.all(np.abs(h[fin] - want[fin]) <= tol[fin])
        assert np.all(h[overflow & np.isfinite(gf)] == 0.0)
        assert np.all(np.isnan(h[np.isnan(gf)]))


# ---------------------------------------------------------------- C1 / MoE

def test_sparse_moe_oracle_matches_reference_formula():
    """routed_experts_match_sparse_cpu_oracle (src/omni.rs:946-1051), INT4:
    identity-scaled experts applied twice, combined in ascending expert order,
    within the reference's 0.08 absolute tolerance."""
    experts, topk = 128, 8
    logits = BF(np.array([((i * 37 + i // experts * 11) % experts) / 16.0 for i in range(3 * experts)],
                         np.float32).reshape(3, experts))
    inp = BF(np.array([(i % 17) / 16.0 - 0.5 for i in range(3 * 256)], np.float32).reshape(3, 256))
    rows = np.arange(experts * 256)
    w = np.zeros((experts * 256, 256), np.float32)
    w[rows, rows % 256] = (rows // 256 + 1) / 128.0
    w_t, w_s = oracle.pack_weight(BF(w))
    routes = oracle.route(logits, topk)
    groups, order = oracle.group_routes(routes)
    codes, scales, _ = oracle.prepare(inp, 256, 4)
    values = oracle.expert_i4(codes, scales, w_t, w_s, groups, 3, topk, 256, 256, False)
    codes2, scales2, _ = oracle.prepare(values, 256, 4)
    values2 = oracle.expert_i4(codes2, scales2, w_t, w_s, groups, 3, topk, 256, 256, True)
    out = F(oracle.combine(values2, routes))
    out_ordered = F(oracle.combine(values2, routes, order))
    assert np.array_equal(out, out_ordered)
    lf = F(logits)
    xf = F(inp)
    for t in range(3):
        ranked = sorted(range(experts), key=lambda e: -float(lf[t, e]))
        assert [int(v) for v in routes[t, :topk]] == ranked[:topk]
        mx = lf[t, ranked[0]]
        sel = [(e, np.float32(np.exp(np.float32(lf[t, e] - mx)))) for e in ranked[:topk]]
        s = np.float32(sum(p for _, p in sel))
        sel = sorted([(e, F(BF(np.float32(p / s)))) for e, p in sel])
        for col in range(256):
            acc = np.float32(0.0)
            for e, p in sel:
                y = F(BF(np.float32(xf[t, col] * np.float32((e + 1) / 128.0))))
                y = F(BF(np.float32(y * np.float32((e + 1) / 128.0))))
                y = F(BF(np.float32(y * p)))
                acc = F(BF(np.float32(acc + y)))
            assert abs(out[t, col] - acc) <= 0.08, (t, col, out[t, col], acc)


def test_checkpoint_tiles_round_trip():
    """src/checkpoint.rs:63-106: [rows][cols] <-> [rows/256][cols/64][256][64]."""
    rows, cols = 512, 192
    w = np.arange(rows * cols, dtype=np.uint32).astype(np.uint16).reshape(rows, cols)
    t = oracle.tile_rows(w)
    flat = t.ravel()
    for tile in range(rows // 256):
        for ks in range(cols // 64):
            for r in (0, 1, 255):
                base = tile * 256 * cols + (ks * 256 + r) * 64
                assert np.array_equal(flat[base:base + 64], w[tile * 256 + r, ks * 64:(ks + 1) * 64])
    assert np.array_equal(oracle.untile_rows(t), w)


# ---------------------------------------------------------------- fused producers

def norm_test_rows(rows: int, width: int = 5120) -> np.ndarray:
    """Input rows of the reference's fused-norm packing test
    (src/quantized.rs:1567-1598): eleven row classes cycling (+-0, tiny,
    bf16::MAX, the smallest denormal, 1e15 scale, NaN / +Inf / -Inf at one
    column, +-1, 1e-3 scale, the plain formula)."""
    i = np.arange(rows * width, dtype=np.int64)
    c = i % width
    value = ((i * 37 % 1031).astype(np.float32) - 515.0) / 37.0
    cls = (i // width) % 11
    v = value.copy()
    v[cls == 0] = np.where(c[cls == 0] % 2 == 0, 0.0, -0.0)
    v[cls == 1] = value[cls == 1] * np.float32(1e-5)
    v[cls == 2] = F(np.array([0x7F7F], dtype=np.uint16))[0]
    v[cls == 3] = F(np.array([0x0001], dtype=np.uint16))[0]
    v[cls == 4] = value[cls == 4] * np.float32(1e15)
    v[(cls == 5) & (c == 37)] = np.nan
    v[(cls == 6) & (c == 113)] = np.inf
    v[(cls == 7) & (c == 259)] = -np.inf
    v[cls == 8] = np.where(c[cls == 8] % 2 == 0, 1.0, -1.0)
    v[cls == 9] = value[cls == 9] * np.float32(1e-3)
    return BF(v.astype(np.float32)).reshape(rows, width)


def norm_test_weight(width: int = 5120, exceptional: bool = False) -> np.ndarray:
    """Weight row of the same test (row 2 of its 3-row buffer)."""
    i = np.arange(3 * width)[2 * width:]
    if exceptional:
        m = i % 1009
        w = np.where(m == 0, np.nan, np.where(m == 1, np.inf, np.where(m == 2, -np.inf, np.where(
            m == 3, float(F(np.array([0x7F7F], dtype=np.uint16))[0]), 0.5))))
    else:
        m = i % 19
        w = np.where(m == 0, -1.0, np.where(m == 1, -0.0, np.where(m == 2, 0.0, ((i * 13 % 127) - 63.0) / 128.0)))
    return BF(w.astype(np.float32))


def bf16_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps along the ordered bit line."""
    def ordered(h):
        h = h.astype(np.int64)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + h)
    return np.abs(ordered(a) - ordered(b))


@pytest.mark.parametrize("exceptional", [False, True])
def test_rms_norm_within_one_bf16_step_of_float64(exceptional):
    """The named RMSNorm (weight + 1, eps 1e-6) against float64 arithmetic: at
    most one bf16 step apart wherever the float64 value is finite, the
    reference test's own bound for normalized values (src/quantized.rs:1706-1716)."""
    x = norm_test_rows(33)
    w = norm_test_weight(exceptional=exceptional)
    got = oracle.rms_norm(x, w)
    xf = F(x).astype(np.float64)
    with np.errstate(all="ignore"):
        inv = 1.0 / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6)
        want = BF((xf * inv * (F(w).astype(np.float64) + 1.0)).astype(np.float32))
    wf = F(want)
    # rows whose f32 sum of squares overflows (bf16::MAX rows) have inv = 0 in
    # f32 arithmetic, as in the reference kernels, and normalize to zeros
    overflow = np.isfinite(xf).all(axis=1) & (np.sum(xf * xf, axis=1) > np.finfo(np.float32).max)
    wfin = np.isfinite(F(w))
    assert overflow.any() and (F(got[overflow][:, wfin]) == 0).all()
    fin = np.isfinite(wf) & ~overflow[:, None]
    assert (bf16_ulps(got[fin], want[fin]) <= 1).all()
    # non-finite float64 results stay non-finite (NaN where float64 is NaN)
    assert np.isnan(F(got)[np.isnan(wf) & ~overflow[:, None]]).all()


@pytest.mark.parametrize("bits", [4, 8])
def test_prepare_norm_is_quantizer_of_the_norm(bits):
    """Fused RMSNorm packing equals Q1 of the separately normalized rows, code
    for code and scale for scale, and stores those normalized rows: the
    reference test's check 'storing normalization changed packed codes'
    (src/quantized.rs:1664-1676) and its fused-vs-unfused comparison."""
    x = norm_test_rows(22)
    w = norm_test_weight()
    stride = 5120 + 512 // bits
    codes, scales, _, normalized = oracle.prepare_norm(x, w, stride, bits)
    assert np.array_equal(normalized, oracle.rms_norm(x, w))
    want_codes, want_scales, _ = oracle.prepare(normalized, stride, bits)
    assert np.array_equal(codes[:, : 5120 * bits // 32], want_codes[:, : 5120 * bits // 32])
    assert np.array_equal(scales.view(np.uint32), want_scales.view(np.uint32))
    # rows holding NaN or +-Inf give zero codes and an infinite scale
    bad = ~np.isfinite(F(x)).all(axis=1)
    assert np.isinf(scales[bad]).all() and not codes[bad, : 5120 * bits // 32].any()
    # an all-zero row normalizes to zeros (inv = 1 / sqrt(1e-6))
    assert not normalized[0].any() or (F(normalized[0]) == 0).all()


def test_prepare_norm_rejects_other_widths():
    x = np.zeros((2, 4096), dtype=np.uint16)
    with pytest.raises(oracle.OracleError, match="unsupported normalized packing shape"):
        oracle.prepare_norm(x, np.zeros(4096, dtype=np.uint16), 4224)


@pytest.mark.parametrize("width", [256, 768, 2048])
def test_prepare_attention_gate_closed_forms(width):
    """Attention-gate packing (kernels/prepare_integer_register.loom:137-155):
    the gate of column c sits at (c/256)*512 + 256 + c%256 of the doubled row.
    Gates of +100 give sigmoid 1 (x itself), 0 gives exactly 1/2 (x/2), -100
    gives bf16 0; the query halves hold NaN, so reading a wrong column would
    turn every row invalid."""
    rng = np.random.default_rng(width)
    rows = 5
    x = BF(rng.standard_normal((rows, width)).astype(np.float32))
    stride = oracle.activation_stride(width)
    for gate, expect in ((100.0, x), (0.0, BF(F(x) * np.float32(0.5))),
                         (-100.0, np.zeros_like(x))):
        q = np.full((rows, 2 * width), 0x7FC0, dtype=np.uint16)  # NaN
        for h in range(width // 256):
            q[:, 512 * h + 256: 512 * h + 512] = BF(np.float32(gate))
        got = oracle.prepare_attention_gate(x, q, stride)
        want = oracle.prepare(expect, stride)
        assert np.array_equal(got[0][:, : width // 8], want[0][:, : width // 8]), gate
        assert np.array_equal(got[1].view(np.uint32), want[1].view(np.uint32)), gate


# ---------------------------------------------------------------- fused SwiGLU quantizer

@pytest.mark.parametrize("width,bits,row_counts", __import__("ref_inputs").fused_swiglu_cases())
def test_prepare_swiglu_is_swiglu_then_prepare(width, bits, row_counts):
    """fused_swiglu_packing_matches_reference (src/quantized.rs:1189-1266): on
    the reference test's gate rows (0, NaN at 259, +inf at 515, bf16::MAX, the
    bf16 denormal, +-80, the formula) and up rows, with its row-offset slices
    and stride width + 512 / bits, the fused producer equals S1 materialized as
    bf16 and then Q1, codes and scales bit for bit. orc_swiglu and orc_prepare
    are pinned on their own (every bf16 gate against float64; the reference
    test oracle of Q1)."""
    import ref_inputs

    stride = width + 512 // bits
    words = width // (32 // bits)
    for rows in row_counts:
        gate, up = ref_inputs.swiglu_gate_up(width, rows)
        fc, fs, _ = oracle.prepare_swiglu(gate, up, stride, bits)
        uc, us, _ = oracle.prepare(oracle.swiglu(gate, up), stride, bits)
        assert np.array_equal(fc[:, :words], uc[:, :words]), (width, bits, rows)
        assert np.array_equal(fs.view(np.uint32), us.view(np.uint32)), (width, bits, rows)


def test_swiglu_on_reference_gate_classes():
    """S1 on the special gate rows of the fused test, against what the
    arithmetic fixes: silu(0) = 0, NaN stays NaN, silu(+inf) = +inf,
    silu(bf16::MAX) = bf16::MAX (exp underflows), silu(+-80) = 80 and a
    negative value of magnitude 80 * e^-80, silu(denormal 0x0001) = bf16(g / 2)
    = 0 (ties to even)."""
    import ref_inputs

    gate, up = ref_inputs.swiglu_gate_up(768, 7)
    h = F(oracle.swiglu(gate, up)).astype(np.float64)
    u = F(up).astype(np.float64)
    # slice row r is buffer row r + 1: classes 1, 2, 3, 4, 5, 6 (formula), 0
    assert np.isnan(h[0, 259])
    assert np.isinf(h[1, 515]) and np.sign(h[1, 515]) == np.sign(u[1, 515]) or u[1, 515] == 0
    big = F(np.array([ref_inputs.BF16_MAX], np.uint16)).astype(np.float64)[0]
    want_max = F(BF((big * u[2]).astype(np.float32))).astype(np.float64)  # bf16(MAX * u), may overflow
    fin = np.isfinite(want_max)
    assert np.array_equal(h[2][fin], want_max[fin])
    assert np.all(np.isinf(h[2][~fin]))
    assert np.all(h[3] == 0.0)
    even = np.arange(768) % 2 == 0
    assert np.array_equal(h[4][~even], F(BF((80.0 * u[4][~even]).astype(np.float32))))
    # silu(-80) = -80 e^-80 / (1 + e^-80): two bf16 roundings of half a step
    want_neg = -80.0 * math.exp(-80.0) * u[4][even]
    assert np.all(np.abs(h[4][even] - want_neg) <= np.abs(want_neg) * 2.0 ** -7)
    assert np.all(h[6] == 0.0)


# ---------------------------------------------------------------- MoE block

def _moe_inputs(rng, t, d, inter):
    x = BF(rng.standard_normal((t, d)).astype(np.float32))
    logits = BF(rng.standard_normal((t, 128)).astype(np.float32))
    gate = oracle.pack_weight(BF((rng.standard_normal((128 * inter, d)) * 0.02).astype(np.float32)))
    up = oracle.pack_weight(BF((rng.standard_normal((128 * inter, d)) * 0.02).astype(np.float32)))
    down = oracle.pack_weight(BF((rng.standard_normal((128 * d, inter)) * 0.02).astype(np.float32)))
    return x, logits, gate, up, down


@pytest.mark.parametrize("t,d,inter,topk", [(1, 512, 256, 8), (37, 512, 256, 8), (40, 1024, 256, 8),
                                            (23, 256, 512, 4)])
def test_moe_layer_is_stage_composition(t, d, inter, topk):
    """The MoE block of forward_layers_cached (src/omni.rs:762-857) with the
    fast defaults: R1 -> ordered R2 -> Q1(x) shared by gate and up -> E1 gate,
    E1 up -> S1 -> Q1 of each routed h row -> E1 down on routed input ->
    ordered C1. orc_moe_layer equals this recipe built from the separately
    pinned stage functions, bit for bit."""
    rng = np.random.default_rng(t * 1000 + d + inter + topk)
    x, logits, gate, up, down = _moe_inputs(rng, t, d, inter)
    want, routes_want = oracle.moe_layer(x, logits, gate, up, down, topk)
    routes = oracle.route(logits, topk)
    assert np.array_equal(routes, routes_want)
    groups, order = oracle.group_routes(routes, topk)
    sx, sh = oracle.activation_stride(d), oracle.activation_stride(inter)
    ax, axs, _ = oracle.prepare(x, sx)
    g = oracle.expert_i4(ax, axs, gate[0], gate[1], groups, t, topk, d, inter, False)
    u = oracle.expert_i4(ax, axs, up[0], up[1], groups, t, topk, d, inter, False)
    h = oracle.swiglu(g, u)
    ah, ahs, _ = oracle.prepare(h, sh)
    values = oracle.expert_i4(ah, ahs, down[0], down[1], groups, t, topk, inter, d, True)
    got = oracle.combine(values, routes, order, topk)
    assert np.array_equal(got, want)


def _bf16_rne(v: np.ndarray) -> np.ndarray:
    """float32 -> bf16-rounded float32 (finite values), written out here so
    the closed form below uses none of the oracle's arithmetic."""
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def moe_closed_form(c, routes, wg, wu, wd, d, inter, topk):
    """MoE output when every row of x and every weight row of an expert is
    constant. A constant row v rotates to 16 v in every position (each radix-4
    stage doubles it), so its row maximum is 16|v|, its scale RN(|v| / 7) and
    every code 7 sign(v). Then every E1 dot over K is 49 K sign(a) sign(w),
    gate and up are constant along their rows, and with gate >= 17
    bf16(silu(g)) = g exactly (1 + e^-17 rounds to 1 in f32), so h = bf16(g u)
    is constant too and Q1 of h follows the same rule. Returns float32
    [T][d] (constant along each row) and the gate values (for the >= 17
    check)."""
    f = np.float32
    t_n = len(c)
    out = np.zeros(t_n, np.float32)
    gates = []
    for t in range(t_n):
        a_s = f(abs(c[t])) / f(7.0)
        sel = sorted((int(routes[t, r]), f(routes[t, topk + r])) for r in range(topk))
        acc = f(0.0)
        for e, p in sel:
            def e1(w_const, k, a_scale, a_sign):
                w_s = f(abs(w_const)) / f(7.0)
                dot = f(49 * k * a_sign * np.sign(w_const))
                return _bf16_rne(np.array([dot * (a_scale * w_s)], np.float32))[0]
            g = e1(wg[e], d, a_s, np.sign(c[t]))
            u = e1(wu[e], d, a_s, np.sign(c[t]))
            gates.append(g)
            h = _bf16_rne(np.array([g * u], np.float32))[0]  # bf16(bf16(silu(g)) u) with silu(g) = g
            h_s = f(abs(h)) / f(7.0)
            v = e1(wd[e], inter, h_s, np.sign(h))
            y = _bf16_rne(np.array([v * p], np.float32))[0]
            acc = _bf16_rne(np.array([acc + y], np.float32))[0]
        out[t] = acc
    return np.repeat(out[:, None], d, axis=1), np.array(gates)


def closed_form_case(seed, t, d, inter, topk=8):
    """Inputs of moe_closed_form: x row t = c_t > 0, expert e's gate rows
    (e % 8 + 3) / 32, up rows +-((e % 5) + 1) / 16, down rows
    +-((e % 3) + 1) / 64, logits N(0, 1)."""
    rng = np.random.default_rng(seed)
    c = F(BF((0.5 + 1.5 * rng.random(t)).astype(np.float32)))
    x = BF(np.repeat(c[:, None], d, axis=1).astype(np.float32))
    logits = BF(rng.standard_normal((t, 128)).astype(np.float32))
    e = np.arange(128)
    wg = ((e % 8 + 3) / 32.0).astype(np.float32)
    wu = (np.where(e % 2 == 0, 1.0, -1.0) * ((e % 5) + 1) / 16.0).astype(np.float32)
    wd = (np.where(e % 3 == 0, -1.0, 1.0) * ((e % 3) + 1) / 64.0).astype(np.float32)
    gate = BF(np.repeat(np.repeat(wg, inter)[:, None], d, axis=1))
    up = BF(np.repeat(np.repeat(wu, inter)[:, None], d, axis=1))
    down = BF(np.repeat(np.repeat(wd, d)[:, None], inter, axis=1))
    return c, x, logits, (gate, up, down), (wg, wu, wd)


def test_moe_layer_closed_form():
    """orc_moe_layer against the closed form of moe_closed_form (the routes,
    pinned by the stable-sort test, are its only input from the oracle)."""
    t, d, inter, topk = 24, 512, 256, 8
    c, x, logits, (gate, up, down), (wg, wu, wd) = closed_form_case(7, t, d, inter, topk)
    packed = [oracle.pack_weight(w) for w in (gate, up, down)]
    # every code of every packed row is +-7: 0x77777777 or 0x99999999 words
    for codes, _ in packed:
        assert np.all((codes == 0x77777777) | (codes == 0x99999999))
    got, routes = oracle.moe_layer(x, logits, *packed, topk=topk)
    want, gates = moe_closed_form(c, routes, wg, wu, wd, d, inter, topk)
    assert np.all(gates >= 17.0)
    assert np.array_equal(F(got), want)


def test_silu_is_half_below_the_table_window():
    """For every bf16 g with exponent field 2..116 (2^-125 <= |g| < 2^-10),
    both signs, S1 with u = 1 gives g / 2 exactly (g's exponent field minus
    one), and +-0 gives +-0: the closed form the fused gate/up epilogue uses
    below its SiLU table window. Also pins where it stops holding: exponent
    field 119 has values where it fails, so the window's lower edge (117)
    keeps a margin."""
    e = np.arange(2, 117, dtype=np.uint32)
    mant = np.arange(128, dtype=np.uint32)
    mag = ((e[:, None] << 7) | mant[None, :]).ravel()
    g = np.concatenate([mag, mag | 0x8000, np.array([0, 0x8000], dtype=np.uint32)]).astype(np.uint16)
    ones = np.full(g.shape, 0x3F80, dtype=np.uint16)
    got = oracle.swiglu(g.reshape(1, -1), ones.reshape(1, -1)).ravel()
    want = g.copy()
    nz = (g & 0x7FFF) != 0
    want[nz] = g[nz] - 0x80
    assert np.array_equal(got, want)
    e119 = ((np.uint32(119) << 7) | mant).astype(np.uint16)
    half119 = e119 - np.uint16(0x80)
    assert not np.array_equal(oracle.swiglu(e119.reshape(1, -1), np.full((1, 128), 0x3F80, np.uint16)).ravel(),
                              half119)
