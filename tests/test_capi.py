"""C ABI checks that need no GPU: the library loads, exports every entry point
include/clef_i4.h declares, and rejects bad shapes with the reference's
messages before touching the device."""
import ctypes
import os
import re

import pytest

import clef_i4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "clef_i4.h")
FAKE = 1 << 20  # never dereferenced: every call below fails its checks first


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clef_\w+)\s*\(", text)))


def call(name, *args):
    rc = getattr(clef_i4.lib(), name)(*args)
    return rc, clef_i4.lib().clef_last_error().decode()


def test_header_symbols_exported_and_bound():
    syms = declared_symbols()
    assert len(syms) >= 20
    handle = ctypes.CDLL(clef_i4.LIB_PATH)
    for s in syms:
        assert hasattr(handle, s), s
        assert s in clef_i4.SIGNATURES, f"{s} missing from the Python binding"
    assert set(clef_i4.SIGNATURES) == set(syms)


def test_abi_version_and_stride_rule():
    assert clef_i4.lib().clef_abi_version() == 100
    # src/quantized.rs:161-166
    assert clef_i4.activation_stride(2048, 4) == 2176
    assert clef_i4.activation_stride(768, 4) == 768
    assert clef_i4.activation_stride(4096, 8) == 4160
    assert clef_i4.activation_stride(12288, 4) == 12416
    assert clef_i4.lib().clef_i4_prepared_words(3, 2176, 4) == 3 * 273


@pytest.mark.parametrize("rows,width,stride,bits", [
    (4, 255, 256, 4), (4, 300, 384, 4), (0, 256, 256, 4), (1048577, 256, 256, 4),
    (4, 256, 200, 4), (4, 256, 65664, 4), (4, 256, 320, 4), (4, 256, 256, 5), (4, 32768 + 256, 33024, 4),
])
def test_prepare_rejects(rows, width, stride, bits):
    rc, msg = call("clef_i4_prepare", FAKE, rows, width, stride, bits, FAKE, None)
    assert rc == -1 and msg == "unsupported rotated integer operand"


def test_prepare_rejects_misaligned_pointer():
    rc, msg = call("clef_i4_prepare", FAKE + 2, 4, 256, 256, 4, FAKE, None)
    assert rc == -1 and "aligned" in msg


@pytest.mark.parametrize("rows,in_words,cols", [(100, 32, 256), (128, 16, 256), (128, 32, 200)])
def test_retile_rejects(rows, in_words, cols):
    rc, msg = call("clef_i4_retile", FAKE, rows, in_words, cols, 4, FAKE, None)
    assert rc == -1 and msg == "unsupported packed weight shape for tiling"


def test_pack_weight_rejects():
    rc, msg = call("clef_i4_pack_weight", FAKE, 128, 256, 4, FAKE, FAKE, FAKE, 1 << 20, None)
    assert rc == -1 and msg == "unsupported quantized weight shape"
    need = clef_i4.lib().clef_i4_pack_weight_workspace_bytes(256, 256, 4)
    assert need >= 256 * (256 // 8 + 1) * 4
    rc, msg = call("clef_i4_pack_weight", FAKE, 256, 256, 4, FAKE, FAKE, FAKE, need - 1, None)
    assert rc == -1 and msg == "workspace too small"


@pytest.mark.parametrize("m,n,k,ks", [(0, 128, 256, 256), (4, 100, 256, 256), (4, 128, 300, 320),
                                      (4, 128, 256, 200), (4, 128, 256, 272)])
def test_gemm_rejects(m, n, k, ks):
    rc, msg = call("clef_i4_gemm", FAKE, ks, FAKE, FAKE, FAKE, m, n, k, None, FAKE, None)
    assert rc == -1 and msg == "unsupported integer projection shape"


def test_gemm_rejects_unknown_config():
    rc, msg = call("clef_i4_gemm_config", FAKE, 256, FAKE, FAKE, FAKE, 4, 128, 256, None, FAKE, 99, None)
    assert rc == -1 and "configuration" in msg


@pytest.mark.parametrize("experts,topk", [(129, 8), (8, 9), (8, 0)])
def test_route_rejects(experts, topk):
    rc, msg = call("clef_moe_route", FAKE, 0, 4, experts, topk, FAKE, None)
    assert rc == -1 and msg == "invalid expert router shape"


def test_group_rejects():
    rc, msg = call("clef_moe_group_routes", FAKE, 0, 8, FAKE, None, FAKE, 1 << 20, None)
    assert rc == -1 and msg == "unsupported Omni route grouping shape"
    need = clef_i4.lib().clef_moe_group_workspace_bytes(4096)
    rc, msg = call("clef_moe_group_routes", FAKE, 4096, 8, FAKE, None, FAKE, need - 1, None)
    assert rc == -1 and msg == "workspace too small"


def test_build_identity_matches_sources():
    """The library's embedded build identity is the hash of the sources it was
    built from; the loader refuses a stale library."""
    import build_id

    assert build_id.stale() is None
    assert clef_i4.lib().clef_build_id().decode() == build_id.source_id() == build_id.library_id()


# Route ordinals t * topk + r are f32 in the reference's tables: exact below
# 2^24 only, so every entry point that reads or writes them caps tokens * topk.
@pytest.mark.parametrize("tokens,topk", [(1048576, 32), (1048576, 17), (262144, 65), (524289, 32)])
def test_route_ordinals_capped_below_2_pow_24(tokens, topk):
    msg = "unsupported Omni route grouping shape"
    rc, got = call("clef_moe_group_routes", FAKE, tokens, topk, FAKE, None, FAKE, 1 << 40, None)
    assert rc == -1 and got == msg
    rc, got = call("clef_moe_expert_i4", FAKE, 256, FAKE, FAKE, FAKE, FAKE, tokens, topk, 256, 256, 0, FAKE, FAKE,
                   1 << 40, None)
    assert rc == -1 and got == msg
    rc, got = call("clef_moe_expert_gate_up_i4", FAKE, 256, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, tokens, topk, 256,
                   256, FAKE, FAKE, 1 << 40, None)
    assert rc == -1 and got == msg
    rc, got = call("clef_moe_layer", FAKE, FAKE, 0, tokens, 256, 256, 128, topk, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, 1 << 40, None)
    assert rc == -1 and got == msg


def test_route_ordinal_cap_admits_2_pow_24():
    """tokens * topk == 2^24 passes the grouping checks (fails later, on the
    workspace)."""
    rc, got = call("clef_moe_group_routes", FAKE, 1048576, 16, FAKE, None, FAKE, 16, None)
    assert rc == -1 and got == "workspace too small"


@pytest.mark.parametrize("tokens,topk,stride,routed", [(1048576, 8, 16384, 0), (65536, 16, 16384, 1),
                                                       (1048576, 2, 4096, 0)])
def test_expert_operand_below_2gib(tokens, topk, stride, routed):
    """Gathered activation rows are addressed by 32-bit buffer offsets: the
    packed operand (rows * stride / 2 bytes) must stay below 2 GiB."""
    rows = tokens * topk if routed else tokens
    big = rows * stride // 2 >= 1 << 31
    rc, got = call("clef_moe_expert_i4", FAKE, stride, FAKE, FAKE, FAKE, FAKE, tokens, topk, 256, 256, routed, FAKE,
                   FAKE, 16, None)
    assert rc == -1 and got == ("expert activation operand of 2 GiB or more (split the tokens into chunks, as the "
                                "reference does)" if big else "workspace too small")
    if not routed:
        rc, got = call("clef_moe_expert_gate_up_i4", FAKE, stride, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, tokens, topk,
                       256, 256, FAKE, FAKE, 16, None)
        assert rc == -1 and got.startswith("expert activation operand" if big else "workspace too small")


def test_moe_layer_rejects_operands_of_2gib():
    # x packed: 131072 rows of (32768 + 128) / 2 bytes > 2 GiB
    rc, got = call("clef_moe_layer", FAKE, FAKE, 0, 131072, 32768, 256, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, 1 << 40, None)
    assert rc == -1 and got.startswith("expert activation operand of 2 GiB")
    # h packed: 131072 * 8 routed rows of (8192 + 128) / 2 bytes > 2 GiB
    rc, got = call("clef_moe_layer", FAKE, FAKE, 0, 131072, 256, 8192, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, 1 << 40, None)
    assert rc == -1 and got.startswith("expert activation operand of 2 GiB")


def test_expert_stride_multiple_of_32():
    """include/clef_i4.h: stride % 32 == 0 for the grouped expert GEMM."""
    for stride, ok in [(272, False), (288, True)]:
        rc, got = call("clef_moe_expert_i4", FAKE, stride, FAKE, FAKE, FAKE, FAKE, 4, 8, 256, 256, 0, FAKE, FAKE,
                       16, None)
        assert rc == -1 and got == ("workspace too small" if ok else "unsupported Omni expert tile shape")


@pytest.mark.parametrize("k,n,stride", [(300, 256, 320), (256, 128, 256), (256, 256, 200)])
def test_expert_rejects(k, n, stride):
    rc, msg = call("clef_moe_expert_i4", FAKE, stride, FAKE, FAKE, FAKE, FAKE, 4, 8, k, n, 0, FAKE, FAKE,
                   1 << 20, None)
    assert rc == -1 and msg == "unsupported Omni expert tile shape"


@pytest.mark.parametrize("k,n,stride,tokens,msg", [
    (512, 96, 512, 4, "incompatible fused expert weights"),
    (500, 128, 512, 4, "incompatible fused expert weights"),
    (512, 128, 256, 4, "incompatible fused expert weights"),
    (512, 128, 512, 0, "fused gate/up requires regular grouped routes"),
])
def test_gate_up_rejects(k, n, stride, tokens, msg):
    rc, got = call("clef_moe_expert_gate_up_i4", FAKE, stride, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, tokens, 8, k, n,
                   FAKE, FAKE, 1 << 20, None)
    assert rc == -1 and got == msg


def test_combine_rejects():
    rc, msg = call("clef_moe_combine", FAKE, FAKE, FAKE, 4, 12, 8, FAKE, None)
    assert rc == -1 and msg == "unsupported ordered Omni accumulation"


def test_swiglu_rejects_and_empty_is_noop():
    rc, msg = call("clef_swiglu", FAKE, FAKE, -1, FAKE, None)
    assert rc == -1 and msg == "SwiGLU shape/dtype mismatch"
    rc, _ = call("clef_swiglu", FAKE, FAKE, 0, FAKE, None)
    assert rc == 0


def test_tile_rows_rejects():
    rc, msg = call("clef_untile_rows", FAKE, 128, 64, FAKE, None)
    assert rc == -1 and msg == "tiled layout requires 256-row and 64-column multiples"


def test_moe_layer_rejects():
    rc, msg = call("clef_moe_layer", FAKE, FAKE, 0, 16, 2048, 768, 64, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, 1 << 30, None)
    assert rc == -1 and msg == "Omni MoE requires 128 experts"
    need = clef_i4.lib().clef_moe_layer_workspace_bytes(16, 2048, 768, 8)
    assert need > 16 * 8 * 2048 * 2
    rc, msg = call("clef_moe_layer", FAKE, FAKE, 0, 16, 2048, 768, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, need - 1, None)
    assert rc == -1 and msg == "workspace too small"


def test_resident_storage_keeps_scales_and_original_precision_outside_backbone():
    """resident_storage_keeps_scales_and_original_precision_outside_backbone
    (src/quantized.rs:782-799)."""
    packing = clef_i4.QuantizedProjections.for_precision("int4")
    assert packing.resident_bytes("model.language_model.layers.0.mlp.up_proj.weight", 17408, 5120) == \
        17408 * 5120 // 2 + 17408 * 4
    for name in ("model.visual.blocks.0.mlp.up_proj.weight", "head.scorer.weight"):
        assert packing.resident_bytes(name, 4096, 4096) == 4096 * 4096 * 2


@pytest.mark.parametrize("mode,mlp_bits,qkv_bits", [("bf16", None, None), ("int4_mlp", 4, None),
                                                    ("int4", 4, 4)])
def test_explicit_precision_selects_only_requested_projections(mode, mlp_bits, qkv_bits):
    """explicit_precision_selects_only_requested_projections
    (src/quantized.rs:826-857)."""
    mlp = "model.language_model.layers.0.mlp.up_proj.weight"
    qkv = "model.language_model.layers.0.linear_attn.in_proj_qkv.weight"
    config = clef_i4.QuantizedProjections.for_precision(mode)
    assert config.is_bf16() == (mode == "bf16")
    assert config.is_full_int4() == (mode == "int4")
    assert config.precision(mlp, 17408, 5120) == mlp_bits
    assert config.precision(qkv, 10240, 5120) == qkv_bits
    assert config.precision("model.visual.blocks.0.mlp.up_proj.weight", 17408, 5120) is None
    assert config.precision("joint_head.weight", 5120, 5120) is None
    assert config.precision("model.language_model.layers.3.self_attn.k_proj.weight", 1024, 5120) is None


def test_precision_policy_mlp_projection_subset():
    """Only the listed MLP projections are packed; other .mlp. weights stay bf16
    (src/quantized.rs:108-115)."""
    config = clef_i4.QuantizedProjections(bits=4, projections=("up",))
    assert config.precision("model.language_model.layers.1.mlp.up_proj.weight", 4096, 4096) == 4
    assert config.precision("model.language_model.layers.1.mlp.down_proj.weight", 4096, 4096) is None
    # backbone eligibility needs rows >= 4096, cols >= 1024, both multiples of 256
    backbone = clef_i4.QuantizedProjections.for_precision("int4")
    name = "model.language_model.layers.1.self_attn.q_proj.weight"
    assert backbone.precision(name, 4096, 1024) == 4
    assert backbone.precision(name, 4096, 768) is None
    assert backbone.precision(name, 4352, 1280) == 4
    assert backbone.precision(name, 4100, 1024) is None
    with pytest.raises(ValueError):
        clef_i4.QuantizedProjections.for_precision("int8")


def test_silu_table_matches_oracle():
    """The fused gate/up epilogue's SiLU table, generated on the host at build
    time, equals bf16(silu(g)) of the oracle (kernels/swiglu.loom:43-47) for
    every tabulated bf16 g."""
    import numpy as np

    import oracle
    path = os.path.join(ROOT, "clef-hrx_amd", "_build", "silu_table.inc")
    body = open(path).read().split("\n", 1)[1]
    table = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-f]{4}", body)], dtype=np.uint16)
    idx = np.arange(8192)
    g = (((idx >> 12) << 15) | ((102 + ((idx >> 7) & 31)) << 7) | (idx & 127)).astype(np.uint16)
    assert len(table) == 8192
    assert np.array_equal(table, oracle.swiglu(g, np.full(8192, 0x3F80, dtype=np.uint16)))


@pytest.mark.parametrize("rows,width,stride,bits", [(4, 300, 384, 4), (0, 256, 256, 4), (4, 256, 200, 4),
                                                    (4, 256, 256, 5)])
def test_prepare_attention_gate_rejects(rows, width, stride, bits):
    rc, msg = call("clef_i4_prepare_attention_gate", FAKE, FAKE, rows, width, stride, bits, FAKE, None)
    assert rc == -1 and msg == "unsupported rotated integer operand"


@pytest.mark.parametrize("rows,width,stride,bits", [(4, 4096, 4224, 4), (0, 5120, 5248, 4), (4, 5120, 5000, 4),
                                                    (4, 5120, 5248, 5), (4, 5120, 5136, 4), (4, 5120, 70000, 4)])
def test_prepare_norm_rejects(rows, width, stride, bits):
    """src/quantized.rs:721-731: width 5120 only."""
    rc, msg = call("clef_i4_prepare_norm", FAKE, FAKE, rows, width, stride, bits, 0, FAKE, None)
    assert rc == -1 and msg == "unsupported normalized packing shape"


def test_prepare_norm_storage_layout():
    """Normalized rows start at the packed words rounded up to 128 bytes
    (src/quantized.rs:731-740)."""
    f = clef_i4.lib().clef_i4_prepare_norm_words
    for rows, stride, bits in [(1, 5248, 4), (7, 5248, 4), (129, 5184, 8)]:
        packed = rows * (stride // (32 // bits) + 1)
        assert f(rows, 5120, stride, bits, 0) == packed
        offset = -(-packed * 4 // 128) * 128
        assert f(rows, 5120, stride, bits, 1) == offset // 4 + rows * 2560
    assert f(4, 5120, 5248, 5, 0) == -1


@pytest.mark.parametrize("m,n,k,ks", [(0, 128, 256, 320), (4, 100, 256, 320), (4, 128, 300, 320),
                                      (4, 128, 256, 288), (4, 128, 256, 200)])
def test_i8_gemm_rejects(m, n, k, ks):
    rc, msg = call("clef_i8_gemm", FAKE, ks, FAKE, FAKE, FAKE, m, n, k, None, FAKE, None)
    assert rc == -1 and msg == "unsupported integer projection shape"


@pytest.mark.parametrize("tokens,hidden,experts", [(0, 2048, 128), (4, 100, 128), (4, 2048, 129), (4, 2048, 48),
                                                   (4, 2048, 16)])
def test_router_logits_rejects(tokens, hidden, experts):
    rc, msg = call("clef_moe_router_logits", FAKE, FAKE, tokens, hidden, experts, FAKE, None)
    assert rc == -1 and msg == "linear shape/dtype mismatch"


def test_moe_layer_static_rejects_beyond_scratch():
    """clef_moe_layer_static allocates nothing: shapes whose intermediates
    exceed its 32 MiB static scratch are rejected before any device work."""
    need = clef_i4.lib().clef_moe_layer_workspace_bytes(4096, 2048, 768, 8)
    assert need > 32 << 20
    rc, msg = call("clef_moe_layer_static", FAKE, FAKE, 0, 4096, 2048, 768, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, None)
    assert rc == -1 and msg.startswith(f"MoE layer needs {need} bytes of scratch; the static scratch holds "
                                       f"{32 << 20}")
    rc, msg = call("clef_moe_layer_static", FAKE, FAKE, 0, 16, 2048, 768, 64, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, None)
    assert rc == -1 and msg == "Omni MoE requires 128 experts"


@pytest.mark.parametrize("k,ok", [(32768, True), (33024, False), (65536, False)])
def test_gemm_f6_bounds_k_to_quantizer_width(k, ok):
    """The bf6 GEMM's f32 sums equal the integer dots only while they stay
    exact; k is capped at 32768, the widest row the quantizer packs. A shape
    that passes reaches the alignment check (the fake pointer + 8 is not
    16-byte aligned), one that fails stops at the shape check."""
    rc, msg = call("clef_i4_gemm_f6", FAKE + 8, FAKE, FAKE, FAKE, 256, 256, k, None, FAKE, None)
    assert rc == -1
    assert msg == ("device pointer is NULL or not 16-byte aligned" if ok else "unsupported integer projection shape")


@pytest.mark.parametrize("rows,width", [(1, 256), (127, 768), (128, 4096), (129, 4096), (4096, 12288)])
def test_f6_prepared_bytes_pad_rows_to_whole_blocks(rows, width):
    """A bf6-prepared activation holds its codes in 128-row blocks (the last
    one padded), then one f32 scale per row; the C ABI's size, the Python
    helper and the project workspace agree on it."""
    codes = (rows + 127) // 128 * 128 * width * 3 // 4
    assert clef_i4.f6_codes_bytes(rows, width) == codes
    assert clef_i4.lib().clef_i4_f6_prepared_bytes(rows, width) == codes + 4 * rows
    assert clef_i4.lib().clef_i4_project_f6_workspace_bytes(rows, width) >= codes + 4 * rows


@pytest.mark.parametrize("offset", [2, 4, 8])
def test_router_rejects_logits_not_16_byte_aligned(offset):
    """The router reads each token's logits as 16-byte pieces where the row
    length allows, so the logits must start on a 16-byte boundary, in
    clef_moe_route and in the MoE layer that runs it."""
    align = "device pointer is NULL or not 16-byte aligned"
    rc, msg = call("clef_moe_route", FAKE + offset, 0, 4, 128, 8, FAKE, None)
    assert rc == -1 and msg == align
    rc, msg = call("clef_moe_layer", FAKE, FAKE + offset, 0, 16, 2048, 768, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, FAKE, 1 << 40, None)
    assert rc == -1 and msg == align
    rc, msg = call("clef_moe_layer_static", FAKE, FAKE + offset, 0, 16, 2048, 768, 128, 8, FAKE, FAKE, FAKE, FAKE,
                   FAKE, FAKE, None, FAKE, None)
    assert rc == -1 and msg == align


def test_static_layer_rejects_700_tokens():
    """Just past the static scratch: 700 tokens at the Omni shape need more
    than its 32 MiB, and the entry point says so before touching the device."""
    need = clef_i4.lib().clef_moe_layer_workspace_bytes(700, 2048, 768, 8)
    assert need > 32 << 20
    rc, msg = call("clef_moe_layer_static", FAKE, FAKE, 0, 700, 2048, 768, 128, 8, FAKE, FAKE, FAKE, FAKE, FAKE,
                   FAKE, None, FAKE, None)
    assert rc == -1 and msg.startswith(f"MoE layer needs {need} bytes of scratch")


def test_resident_bytes_count_the_kept_weight_forms():
    """A 4-bit projection kept in the bf6 form costs N*K*3/4 code bytes, both
    forms N*K*5/4; the f32 row scales are shared. bf16 weights are unaffected."""
    name = "model.language_model.layers.0.mlp.up_proj.weight"
    n, k = 17408, 5120
    ref = clef_i4.QuantizedProjections.for_precision("int4_mlp")
    both = clef_i4.QuantizedProjections.for_precision("int4_mlp", forms=("int4", "bf6"))
    f6 = clef_i4.QuantizedProjections.for_precision("int4_mlp", forms=("bf6",))
    assert ref.resident_bytes(name, n, k) == n * k // 2 + 4 * n
    assert both.resident_bytes(name, n, k) == n * k // 2 + n * k * 3 // 4 + 4 * n
    assert f6.resident_bytes(name, n, k) == n * k * 3 // 4 + 4 * n
    assert f6.resident_bytes("model.visual.blocks.0.mlp.up_proj.weight", 4096, 4096) == 4096 * 4096 * 2
    with pytest.raises(ValueError):
        clef_i4.QuantizedProjections(bits=4, forms=("int4", "fp8"))
    with pytest.raises(ValueError):
        clef_i4.QuantizedProjections(bits=4, forms=())
