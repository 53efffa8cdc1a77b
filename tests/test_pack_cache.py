"""The packed-weight cache (src/packed_cache.rs): file format, hashing and
corruption checks through the C ABI. CPU only, except the last test.

SHA-256 and the compact JSON are checked against Python's hashlib and json:
the file name is the hash of the key's JSON, the header carries the hashes of
the source, codes and scales.
"""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import clef_i4


def entry(path):
    raw = open(path, "rb").read()
    assert raw[:8] == b"CLFPACK1"
    (n,) = struct.unpack("<I", raw[8:12])
    return json.loads(raw[12:12 + n].decode()), raw[12:12 + n], raw[12 + n:]


def test_source_and_compiler_changes_miss_and_corruption_is_rejected(tmp_path):
    """source_and_compiler_changes_miss_and_corruption_is_rejected
    (src/packed_cache.rs:195-231)."""
    cache = clef_i4.PackedWeightCache(tmp_path, "compiler-a", "gfx1151")
    key = cache.key("weight", 256, 256, 4, b"source")
    assert cache.read(key) is None and cache.misses == 1
    codes, scales = bytes([0x5A]) * 32768, bytes([0x17]) * 1024
    cache.write(key, codes, scales)
    assert cache.read(key) == (codes, scales) and cache.hits == 1
    assert cache.read(cache.key("weight", 256, 256, 4, b"changed source")) is None
    other = clef_i4.PackedWeightCache(tmp_path, "compiler-b", "gfx1151")
    assert other.read(other.key("weight", 256, 256, 4, b"source")) is None
    path = cache.path(key)
    data = bytearray(open(path, "rb").read())
    data[-1] ^= 1
    open(path, "wb").write(bytes(data))
    with pytest.raises(clef_i4.ClefError, match="checksum"):
        cache.read(key)
    open(path, "wb").write(bytes(data[:-1]))
    with pytest.raises(clef_i4.ClefError, match="length"):
        cache.read(key)


@pytest.mark.parametrize("n", [0, 1, 55, 56, 63, 64, 65, 119, 120, 1000])
def test_header_hashes_and_file_name(tmp_path, n):
    """SHA-256 at every padding boundary and the compact JSON key: the header's
    hashes equal hashlib's, and the file name is the hash of the key JSON as
    serde_json writes it (compact, declared field order)."""
    source = bytes(range(256)) * 4
    source = source[:n]
    cache = clef_i4.PackedWeightCache(tmp_path, "cc", "gfx950")
    key = cache.key("model.layers.0.mlp.up_proj.weight", 256, 512, 8, source)
    rng = np.random.default_rng(n)
    codes = rng.integers(0, 256, 256 * 512, dtype=np.uint8).tobytes()
    scales = rng.integers(0, 256, 1024, dtype=np.uint8).tobytes()
    cache.write(key, codes, scales)
    path = cache.path(key)
    header, header_text, rest = entry(path)
    assert rest == codes + scales
    assert list(header) == ["key", "codes_sha256", "scales_sha256"]
    k = header["key"]
    assert list(k) == ["name", "rows", "cols", "bits", "compiler", "target", "source_sha256", "packing_sha256"]
    assert (k["name"], k["rows"], k["cols"], k["bits"], k["compiler"], k["target"]) == \
        ("model.layers.0.mlp.up_proj.weight", 256, 512, 8, "cc", "gfx950")
    assert k["source_sha256"] == hashlib.sha256(source).hexdigest()
    assert header["codes_sha256"] == hashlib.sha256(codes).hexdigest()
    assert header["scales_sha256"] == hashlib.sha256(scales).hexdigest()
    compact = json.dumps(k, separators=(",", ":"), ensure_ascii=False)
    assert header_text == json.dumps(header, separators=(",", ":"), ensure_ascii=False).encode()
    assert os.path.basename(path) == hashlib.sha256(compact.encode()).hexdigest() + ".pack"


def test_names_are_escaped_as_json(tmp_path):
    cache = clef_i4.PackedWeightCache(tmp_path / "nested" / "dir")
    name = 'w"eird\\name\n\t\x01 ünïcode'
    key = cache.key(name, 256, 256, 4, b"x")
    cache.write(key, bytes(32768), bytes(1024))
    header, _, _ = entry(cache.path(key))
    assert header["key"]["name"] == name
    assert cache.read(key) == (bytes(32768), bytes(1024))


def test_extent_and_size_errors(tmp_path):
    cache = clef_i4.PackedWeightCache(tmp_path)
    with pytest.raises(clef_i4.ClefError, match="invalid packed-cache extent"):
        cache.write(cache.key("w", 200, 256, 4, b""), bytes(25600), bytes(800))
    with pytest.raises(clef_i4.ClefError, match="data size mismatch"):
        cache.write(cache.key("w", 256, 256, 4, b""), bytes(100), bytes(1024))
    key = cache.key("w", 256, 256, 4, b"")
    cache.write(key, bytes(32768), bytes(1024))
    path = cache.path(key)
    data = bytearray(open(path, "rb").read())
    data[0:8] = b"CLFPACK2"
    open(path, "wb").write(bytes(data))
    with pytest.raises(clef_i4.ClefError, match="magic"):
        cache.read(key)


@pytest.mark.gpu
def test_load_quantized_weight_through_the_cache(tmp_path):
    """A miss packs on the GPU and writes the entry; the next load hits and
    yields the same codes and scales (src/quantized.rs:169-190, 212-220)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn((512, 1024), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    cache = clef_i4.PackedWeightCache(tmp_path)
    first = clef_i4.load_quantized_weight(w, cache=cache, name="model.layers.0.mlp.up_proj.weight")
    assert (cache.hits, cache.misses) == (0, 1)
    second = clef_i4.load_quantized_weight(w, cache=cache, name="model.layers.0.mlp.up_proj.weight")
    assert (cache.hits, cache.misses) == (1, 1)
    assert torch.equal(first.codes, second.codes) and torch.equal(first.scales, second.scales)
    plain = clef_i4.load_quantized_weight(w)
    assert torch.equal(plain.codes, second.codes)


@pytest.mark.gpu
def test_expert_concat_keeps_tiled_layout():
    """omni::load_expert_layer (src/omni.rs:40-72): per-expert tiled
    checkpoint tensors concatenated and untiled once pack to the same bytes as
    the dense concatenation."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(4)
    rows, cols = 256, 512
    dense = [(torch.randn((rows, cols), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
             for _ in range(128)]
    tiled = [clef_i4.tile_rows(t) for t in dense]
    got = clef_i4.load_expert_layer(tiled, rows, cols, tiled_checkpoint=True)
    want = clef_i4.load_quantized_weight(torch.cat(dense, dim=0))
    assert torch.equal(got.codes, want.codes) and torch.equal(got.scales, want.scales)
    with pytest.raises(clef_i4.ClefError, match="invalid Omni expert shape"):
        clef_i4.load_expert_layer(dense[:127] + [dense[0][:128]], rows, cols)
