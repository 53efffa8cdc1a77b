"""Python binding of the gfx950 INT4 path (C ABI in include/clef_i4.h).

A thin ctypes layer: torch supplies device memory and the current HIP stream,
the library does all the work. Function names follow the reference's operator
API (src/quantized.rs, src/omni.rs, src/ops.rs) so callers read the same:
outputs are allocated here (as the reference's Engine allocates them) and the
C entry points only write into them.

Import fails loudly when lib/libclef_i4.so is missing: there is no fallback
path.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libclef_i4.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/clef_i4.h.
SIGNATURES = {
    "clef_last_error": (ctypes.c_char_p, []),
    "clef_abi_version": (ctypes.c_int, []),
    "clef_build_id": (ctypes.c_char_p, []),
    "clef_i4_activation_stride": (_I32, [_I32, _I32]),
    "clef_i4_prepared_words": (_I64, [_I64, _I32, _I32]),
    "clef_i4_prepare": (ctypes.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P]),
    "clef_i4_prepare_swiglu": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P, _P]),
    "clef_i4_prepare_attention_gate": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P, _P]),
    "clef_i4_prepare_norm_words": (_I64, [_I64, _I32, _I32, _I32, _I32]),
    "clef_i4_prepare_norm": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P]),
    "clef_i4_retile": (ctypes.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P]),
    "clef_i4_pack_weight_workspace_bytes": (_SZ, [_I64, _I32, _I32]),
    "clef_i4_pack_weight": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _SZ, _P]),
    "clef_untile_rows": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
    "clef_tile_rows": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
    "clef_i4_gemm": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I64, _I32, _I32, _P, _P, _P]),
    "clef_i4_gemm_config": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I64, _I32, _I32, _P, _P, _I32, _P]),
    "clef_i4_gemm_configs": (ctypes.c_int, []),
    "clef_i8_gemm": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I64, _I32, _I32, _P, _P, _P]),
    "clef_i4_f6_activation": (ctypes.c_int, [_P, _I32, _I64, _I32, _P, _P]),
    "clef_i4_f6_weight": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
    "clef_i4_gemm_f6": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, _P, _P, _P]),
    "clef_i4_gemm_f6_gate_up": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P, _P]),
    "clef_i4_f6_prepared_bytes": (ctypes.c_int64, [_I64, _I32]),
    "clef_i4_prepare_f6": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
    "clef_i4_prepare_swiglu_f6": (ctypes.c_int, [_P, _P, _I64, _I32, _P, _P]),
    "clef_i4_project_f6_workspace_bytes": (ctypes.c_size_t, [_I64, _I32]),
    "clef_i4_project_f6": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _I32, _P, _P, _P, ctypes.c_size_t, _P]),
    "clef_i4_project_workspace_bytes": (_SZ, [_I64, _I32]),
    "clef_i4_project": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _I32, _P, _P, _P, _SZ, _P]),
    "clef_moe_router_logits": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _P, _P]),
    "clef_moe_route": (ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _P, _P]),
    "clef_moe_group_workspace_bytes": (_SZ, [_I64]),
    "clef_moe_group_routes": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _P, _SZ, _P]),
    "clef_moe_expert_tasks": (ctypes.c_int, [_P, _I64, _P, _P]),
    "clef_moe_expert_workspace_bytes": (_SZ, [_I64, _I32]),
    "clef_moe_expert_gate_up_i4": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _P,
                                                  _P, _SZ, _P]),
    "clef_moe_expert_i4": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P,
                                          _P, _SZ, _P]),
    "clef_moe_expert_ungrouped_workspace_bytes": (_SZ, [_I64, _I32]),
    "clef_moe_expert_i4_ungrouped": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P,
                                                    _P, _SZ, _P]),
    "clef_swiglu": (ctypes.c_int, [_P, _P, _I64, _P, _P]),
    "clef_moe_combine": (ctypes.c_int, [_P, _P, _P, _I64, _I32, _I32, _P, _P]),
    "clef_pack_cache_path": (ctypes.c_int, [_P, _P, _P, _SZ]),
    "clef_pack_cache_read": (ctypes.c_int, [_P, _P, _P, _SZ, _P, _SZ, _P]),
    "clef_pack_cache_write": (ctypes.c_int, [_P, _P, _P, _SZ, _P, _SZ]),
    "clef_moe_layer_workspace_bytes": (_SZ, [_I64, _I32, _I32, _I32]),
    "clef_moe_layer": (ctypes.c_int, [_P, _P, _I32, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P,
                                      _P, _P, _P, _SZ, _P]),
    "clef_moe_layer_static": (ctypes.c_int, [_P, _P, _I32, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P,
                                             _P, _P, _P]),
}

_lib = None


class ClefError(RuntimeError):
    """A failed entry point: precondition (code -1) or HIP error (code > 0)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library. Raises ImportError when it is missing or, where the
    sources sit beside it, built from other sources than the tree's."""
    global _lib
    if _lib is None:
        import build_id

        problem = build_id.stale()
        if problem:
            raise ImportError(f"{problem}; run `make -C clef-hrx_amd` (or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise ClefError(rc, lib().clef_last_error().decode())


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    assert t.is_cuda and t.is_contiguous(), "device tensors must be contiguous CUDA tensors"
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _empty(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


# ---------------------------------------------------------------- Q1 / Q2

def activation_stride(width: int, bits: int = 4) -> int:
    """src/quantized.rs:161-166."""
    return int(lib().clef_i4_activation_stride(width, bits))


@dataclass
class Prepared:
    """quantized::prepare output: one u32 buffer, codes then f32 scales."""
    storage: torch.Tensor  # int32 [rows * (words + 1)]
    rows: int
    width: int
    stride: int
    bits: int

    @property
    def words(self) -> int:
        return self.stride // (32 // self.bits)

    @property
    def codes(self) -> torch.Tensor:
        return self.storage[: self.rows * self.words].view(self.rows, self.words)

    @property
    def scales(self) -> torch.Tensor:
        start = self.rows * self.words
        return self.storage[start: start + self.rows].view(torch.float32)


def prepare(x: torch.Tensor, bits: int = 4, stride: int | None = None, out: torch.Tensor | None = None
            ) -> Prepared:
    """quantized::prepare (src/quantized.rs:574-686)."""
    rows, width = x.shape
    stride = activation_stride(width, bits) if stride is None else stride
    words = int(lib().clef_i4_prepared_words(rows, stride, bits))
    if out is None:
        out = torch.zeros(max(words, 1), dtype=torch.int32, device=x.device)
    _check(lib().clef_i4_prepare(_ptr(x), rows, width, stride, bits, _ptr(out), _stream()))
    return Prepared(out, rows, width, stride, bits)


def prepare_swiglu(gate: torch.Tensor, up: torch.Tensor, bits: int = 4, stride: int | None = None
                   ) -> Prepared:
    """prepare_with_inputs([gate, up]) (src/quantized.rs:605-613)."""
    rows, width = gate.shape
    stride = activation_stride(width, bits) if stride is None else stride
    words = int(lib().clef_i4_prepared_words(rows, stride, bits))
    out = torch.zeros(max(words, 1), dtype=torch.int32, device=gate.device)
    _check(lib().clef_i4_prepare_swiglu(_ptr(gate), _ptr(up), rows, width, stride, bits, _ptr(out),
                                        _stream()))
    return Prepared(out, rows, width, stride, bits)


def prepare_attention_gate(attention: torch.Tensor, q_gate: torch.Tensor, bits: int = 4,
                           stride: int | None = None) -> Prepared:
    """prepare_attention_gate_with_source (src/quantized.rs:615-635): packs
    bf16(attention * bf16(sigmoid(gate))), q_gate bf16 [rows][2*width]."""
    rows, width = attention.shape
    if tuple(q_gate.shape) != (rows, 2 * width) or q_gate.dtype != attention.dtype:
        raise ClefError(-1, "packing input shape/dtype mismatch")
    stride = activation_stride(width, bits) if stride is None else stride
    words = int(lib().clef_i4_prepared_words(rows, stride, bits))
    out = torch.zeros(max(words, 1), dtype=torch.int32, device=attention.device)
    _check(lib().clef_i4_prepare_attention_gate(_ptr(attention), _ptr(q_gate), rows, width, stride, bits,
                                                _ptr(out), _stream()))
    return Prepared(out, rows, width, stride, bits)


def prepare_norm(x: torch.Tensor, weight: torch.Tensor, bits: int = 4, stride: int | None = None,
                 store: bool = False):
    """prepare_norm[_store]_with_source (src/quantized.rs:687-779): named RMSNorm
    (weight + 1, eps 1e-6) fused into the quantizer. Returns (Prepared,
    normalized bf16 [rows][width] view of the same storage, or None)."""
    rows, width = x.shape
    if weight.numel() != width:
        raise ClefError(-1, "unsupported normalized packing shape")
    stride = activation_stride(width, bits) if stride is None else stride
    total = int(lib().clef_i4_prepare_norm_words(rows, width, stride, bits, int(store)))
    out = torch.zeros(max(total, 1), dtype=torch.int32, device=x.device)
    _check(lib().clef_i4_prepare_norm(_ptr(x), _ptr(weight.contiguous()), rows, width, stride, bits, int(store),
                                      _ptr(out), _stream()))
    normalized = None
    if store:
        first = total - rows * width // 2
        normalized = out[first:].view(torch.bfloat16).view(rows, width)
    return Prepared(out, rows, width, stride, bits), normalized


def retile_codes(codes: torch.Tensor, rows: int, cols: int, bits: int = 4) -> torch.Tensor:
    """quantized::retile_codes (src/quantized.rs:542-572); codes [rows][in_words]."""
    in_words = codes.shape[1]
    tiled = torch.empty(rows * cols // (32 // bits), dtype=torch.int32, device=codes.device)
    _check(lib().clef_i4_retile(_ptr(codes.contiguous()), rows, in_words, cols, bits, _ptr(tiled),
                                _stream()))
    return tiled


@dataclass
class QuantizedWeight:
    """src/quantized.rs:12-20."""
    codes: torch.Tensor   # int32 tiled words
    scales: torch.Tensor  # f32 [rows]
    rows: int
    cols: int
    stride: int
    bits: int


class QuantizedProjections:
    """Which checkpoint weights the INT4 path packs, and their resident size.

    Mirrors QuantizedProjections::{for_precision, precision, resident_bytes,
    is_bf16, is_full_int4} (src/quantized.rs:41-62, 104-127) with Precision
    from src/model.rs:22-29 given as "bf16", "int4_mlp" or "int4".

    `forms` (this library's addition) names the packed forms each 4-bit
    weight keeps resident: "int4" is the reference's tiled codes (N*K/2
    bytes), "bf6" the same codes as e3m2 for the bf6 GEMM (N*K*3/4 bytes,
    clef_i4_f6_weight); both share the N f32 row scales. The default keeps the
    reference's form only; ("int4", "bf6") keeps both (2.5x the reference's
    code bytes), ("bf6",) the bf6 form alone (1.5x), which serves every
    projection through project_f6 with the same output bits.
    """

    PRECISIONS = ("bf16", "int4_mlp", "int4")
    FORMS = ("int4", "bf6")

    def __init__(self, bits: int | None = None, backbone_bits: int | None = None,
                 projections=("up", "gate", "down"), share_packing: bool = False, forms=("int4",)):
        self.bits = bits
        self.backbone_bits = backbone_bits
        self.projections = list(projections)
        self.share_packing = share_packing
        if not forms or any(f not in self.FORMS for f in forms):
            raise ValueError(f"unknown resident weight forms {forms!r}")
        self.forms = tuple(forms)

    @classmethod
    def for_precision(cls, precision: str, forms=("int4",)) -> "QuantizedProjections":
        if precision not in cls.PRECISIONS:
            raise ValueError(f"unknown precision {precision!r}")
        return cls(bits=4 if precision == "int4_mlp" else None,
                   backbone_bits=4 if precision == "int4" else None,
                   share_packing=precision != "bf16", forms=forms)

    def is_bf16(self) -> bool:
        return self.bits is None and self.backbone_bits is None

    def is_full_int4(self) -> bool:
        return self.bits is None and self.backbone_bits == 4 and self.projections == ["up", "gate", "down"]

    def precision(self, name: str, rows: int, cols: int) -> int | None:
        """Bits a weight is packed with, or None if it stays bf16."""
        if not name.startswith("model.language_model.layers.") or not name.endswith(".weight"):
            return None
        if ".mlp." in name:
            if any(name.endswith(f".{p}_proj.weight") for p in self.projections):
                return self.bits if self.bits is not None else self.backbone_bits
            return None
        if rows >= 4096 and cols >= 1024 and rows % 256 == 0 and cols % 256 == 0:
            return self.backbone_bits
        return None

    def resident_bytes(self, name: str, rows: int, cols: int) -> int:
        bits = self.precision(name, rows, cols)
        if bits is None:
            return rows * cols * 2
        # retiled codes carry no stride padding; one f32 scale per row, shared
        # by the forms of a 4-bit weight
        if bits != 4:
            return rows * cols * bits // 8 + rows * 4
        code_bytes = {"int4": rows * cols // 2, "bf6": rows * cols * 3 // 4}
        return sum(code_bytes[f] for f in self.forms) + rows * 4

    def pack(self, w: torch.Tensor, name: str, tiled_checkpoint: bool = False):
        """The resident forms of checkpoint weight `name` (bf16 [rows][cols]):
        a dict with "int4" (QuantizedWeight) and/or "bf6" (F6Weight) as
        `forms` asks, or {"bf16": w} when the weight stays bf16. The bf6 form
        is made from the packed codes, whose buffer is dropped when "int4" is
        not kept; resident_bytes counts exactly what is returned."""
        rows, cols = w.shape
        bits = self.precision(name, rows, cols)
        if bits is None:
            return {"bf16": w}
        qw = load_quantized_weight(w, bits=bits, tiled_checkpoint=tiled_checkpoint)
        if bits != 4:
            return {"int" + str(bits): qw}
        out = {}
        if "bf6" in self.forms:
            out["bf6"] = f6_weight(qw)
        if "int4" in self.forms:
            out["int4"] = qw
        return out


class _PackKey(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("bits", ctypes.c_int32), ("compiler", ctypes.c_char_p), ("target", ctypes.c_char_p),
                ("source", ctypes.c_void_p), ("source_bytes", ctypes.c_size_t)]


class PackedWeightCache:
    """PackedWeightCache (src/packed_cache.rs:68-190): "CLFPACK1" files of the
    exact packed codes and scales, keyed by name, extent, bits, compiler,
    target and the SHA-256 of the source bytes and of the packing definition.
    The file format, hashing and checks are the library's (clef_pack_cache_*)."""

    def __init__(self, directory: str, compiler: str = "clef-hrx_amd", target: str = "gfx950"):
        self.directory = str(directory)
        self.compiler = compiler
        self.target = target
        self.hits = 0
        self.misses = 0

    def key(self, name: str, rows: int, cols: int, bits: int, source: bytes):
        source = bytes(source)
        buf = ctypes.create_string_buffer(source, len(source))
        k = _PackKey(name.encode(), rows, cols, bits, self.compiler.encode(), self.target.encode(),
                     ctypes.cast(buf, ctypes.c_void_p), len(source))
        k._source = buf  # keeps the bytes alive with the key
        return k

    def path(self, key) -> str:
        out = ctypes.create_string_buffer(4096)
        _check(lib().clef_pack_cache_path(self.directory.encode(), ctypes.byref(key), out, 4096))
        return out.value.decode()

    @staticmethod
    def sizes(key) -> tuple[int, int]:
        return key.rows * key.cols * key.bits // 8, key.rows * 4

    def read(self, key):
        """(codes bytes, scales bytes) of a hit, None on a miss."""
        nc, ns = self.sizes(key)
        codes = ctypes.create_string_buffer(max(nc, 1))
        scales = ctypes.create_string_buffer(max(ns, 1))
        hit = ctypes.c_int32(0)
        _check(lib().clef_pack_cache_read(self.directory.encode(), ctypes.byref(key), codes, nc, scales, ns,
                                          ctypes.byref(hit)))
        if not hit.value:
            self.misses += 1
            return None
        self.hits += 1
        return codes.raw[:nc], scales.raw[:ns]

    def write(self, key, codes: bytes, scales: bytes) -> None:
        _check(lib().clef_pack_cache_write(self.directory.encode(), ctypes.byref(key), codes, len(codes), scales,
                                           len(scales)))


def load_quantized_weight(w: torch.Tensor, bits: int = 4, tiled_checkpoint: bool = False,
                          cache: PackedWeightCache | None = None, name: str = "") -> QuantizedWeight:
    """Packing half of Engine::load_quantized_weight (src/quantized.rs:147-234),
    with the optional packed-weight cache of its bench builds (:169-190,
    :212-220): a hit uploads the cached bytes, a miss packs and writes them."""
    rows, cols = w.shape
    key = None
    if cache is not None:
        source = w.contiguous().view(torch.int16).cpu().numpy().tobytes()
        key = cache.key(name, rows, cols, bits, source)
        cached = cache.read(key)
        if cached is not None:
            import numpy as np
            codes = torch.from_numpy(np.frombuffer(cached[0], dtype=np.int32).copy()).to(w.device)
            scales = torch.from_numpy(np.frombuffer(cached[1], dtype=np.float32).copy()).to(w.device)
            return QuantizedWeight(codes, scales, rows, cols, activation_stride(cols, bits), bits)
    packed = _pack(w, bits, tiled_checkpoint)
    if key is not None:
        cache.write(key, packed.codes.cpu().numpy().tobytes(), packed.scales.cpu().numpy().tobytes())
    return packed


def _pack(w: torch.Tensor, bits: int, tiled_checkpoint: bool) -> QuantizedWeight:
    rows, cols = w.shape
    if tiled_checkpoint:
        dense = torch.empty_like(w)
        _check(lib().clef_untile_rows(_ptr(w), rows, cols, _ptr(dense), _stream()))
        w = dense
    codes = torch.empty(rows * cols // (32 // bits), dtype=torch.int32, device=w.device)
    scales = torch.empty(rows, dtype=torch.float32, device=w.device)
    ws_bytes = int(lib().clef_i4_pack_weight_workspace_bytes(rows, cols, bits))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=w.device)
    _check(lib().clef_i4_pack_weight(_ptr(w), rows, cols, bits, _ptr(codes), _ptr(scales), _ptr(ws),
                                     ws_bytes, _stream()))
    return QuantizedWeight(codes, scales, rows, cols, activation_stride(cols, bits), bits)


def load_expert_layer(experts: list[torch.Tensor], rows: int, cols: int, bits: int = 4,
                      tiled_checkpoint: bool = False, cache: PackedWeightCache | None = None,
                      name: str = "") -> QuantizedWeight:
    """omni::load_expert_layer (src/omni.rs:40-72): the 128 experts' [rows][cols]
    weights of one projection concatenated row-wise into [128*rows][cols] and
    packed as one weight. Concatenating whole 256-row tiles keeps a tiled
    checkpoint's layout, so the untile happens once on the concatenation."""
    if len(experts) != 128:
        raise ClefError(-1, "Omni MoE requires 128 experts")
    for t in experts:
        if tuple(t.shape) != (rows, cols):
            raise ClefError(-1, f"invalid Omni expert shape: {name}")
    combined = torch.cat([t.contiguous() for t in experts], dim=0)
    return load_quantized_weight(combined, bits=bits, tiled_checkpoint=tiled_checkpoint, cache=cache, name=name)


def untile_rows(tiled: torch.Tensor) -> torch.Tensor:
    rows, cols = tiled.shape
    out = torch.empty_like(tiled)
    _check(lib().clef_untile_rows(_ptr(tiled), rows, cols, _ptr(out), _stream()))
    return out


def tile_rows(dense: torch.Tensor) -> torch.Tensor:
    rows, cols = dense.shape
    out = torch.empty_like(dense)
    _check(lib().clef_tile_rows(_ptr(dense), rows, cols, _ptr(out), _stream()))
    return out


# ---------------------------------------------------------------- G1

def gemm_configs() -> int:
    return int(lib().clef_i4_gemm_configs())


def project_prepared(a: Prepared, w: QuantizedWeight, residual: torch.Tensor | None = None,
                     config: int = -1, out: torch.Tensor | None = None) -> torch.Tensor:
    """Engine::project_prepared (src/quantized.rs:470-537)."""
    if out is None:
        out = _empty((a.rows, w.rows), torch.bfloat16, a.storage.device)
    if a.bits != w.bits:
        raise ClefError(-1, "unsupported integer projection shape")
    if w.bits == 8:  # h3_gemm_i8_256
        _check(lib().clef_i8_gemm(_ptr(a.storage), a.stride, _ptr(a.scales), _ptr(w.codes), _ptr(w.scales),
                                  a.rows, w.rows, w.cols, _ptr(residual), _ptr(out), _stream()))
        return out
    _check(lib().clef_i4_gemm_config(_ptr(a.storage), a.stride, _ptr(a.scales), _ptr(w.codes),
                                     _ptr(w.scales), a.rows, w.rows, w.cols, _ptr(residual), _ptr(out),
                                     config, _stream()))
    return out


@dataclass
class F6Weight:
    """A 4-bit QuantizedWeight re-encoded for the bf6 GEMM (clef_i4_f6_weight):
    the same codes as 6-bit e3m2 values, rows x cols x 3/4 bytes."""
    codes: torch.Tensor   # uint8 bf6 tiled
    scales: torch.Tensor  # f32 [rows], shared with the source weight
    rows: int
    cols: int


def f6_weight(w: QuantizedWeight) -> F6Weight:
    """bf6 form of a 4-bit tiled weight (no counterpart in the reference)."""
    if w.bits != 4:
        raise ClefError(-1, "unsupported integer projection shape")
    codes = torch.empty(w.rows * w.cols * 3 // 4, dtype=torch.uint8, device=w.codes.device)
    _check(lib().clef_i4_f6_weight(_ptr(w.codes), w.rows, w.cols, _ptr(codes), _stream()))
    return F6Weight(codes, w.scales, w.rows, w.cols)


def f6_codes_bytes(rows: int, width: int) -> int:
    """Bytes of bf6 activation codes (clef_i4_f6_activation's layout): 128-row
    blocks, the last one padded."""
    return (rows + 127) // 128 * 128 * width * 3 // 4


def f6_activation(a: Prepared, out: torch.Tensor | None = None) -> torch.Tensor:
    """The bf6 activation codes (uint8 [f6_codes_bytes(rows, width)], blocks
    of 128 rows x 128 k) of a 4-bit prepared activation."""
    if a.bits != 4:
        raise ClefError(-1, "unsupported integer projection shape")
    nbytes = f6_codes_bytes(a.rows, a.width)
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=a.storage.device)
    elif out.dtype != torch.uint8 or out.numel() < nbytes:
        raise ClefError(-1, "bf6 activation buffer too small")
    _check(lib().clef_i4_f6_activation(_ptr(a.storage), a.stride, a.rows, a.width, _ptr(out), _stream()))
    return out


def gemm_f6(a_f6: torch.Tensor, a_scales: torch.Tensor, w: F6Weight, residual: torch.Tensor | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """G1 on bf6 operands: equal to project_prepared on the operands they came
    from. The rows are those of a_scales (one f32 scale per row)."""
    rows = a_scales.numel()
    if a_f6.numel() < f6_codes_bytes(rows, w.cols):
        raise ClefError(-1, "bf6 activation buffer too small")
    if out is None:
        out = _empty((rows, w.rows), torch.bfloat16, a_f6.device)
    _check(lib().clef_i4_gemm_f6(_ptr(a_f6), _ptr(a_scales), _ptr(w.codes), _ptr(w.scales), rows, w.rows, w.cols,
                                 _ptr(residual), _ptr(out), _stream()))
    return out


@dataclass
class PreparedF6:
    """Q1 output in bf6 form (clef_i4_prepare_f6): one uint8 buffer holding
    the e3m2 codes in the bf6 activation layout (f6_codes_bytes), then rows
    f32 scales."""
    storage: torch.Tensor  # uint8 [f6_codes_bytes(rows, width) + 4 * rows]
    rows: int
    width: int

    @property
    def codes(self) -> torch.Tensor:
        return self.storage[: f6_codes_bytes(self.rows, self.width)]

    @property
    def scales(self) -> torch.Tensor:
        start = f6_codes_bytes(self.rows, self.width)
        return self.storage[start: start + 4 * self.rows].view(torch.float32)


def _prepared_f6_storage(rows: int, width: int, device, out: torch.Tensor | None) -> torch.Tensor:
    nbytes = int(lib().clef_i4_f6_prepared_bytes(rows, width))
    if out is None:
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    if out.dtype != torch.uint8 or out.numel() < nbytes:
        raise ClefError(-1, "bf6 activation buffer too small")
    return out


def prepare_f6(x: torch.Tensor, out: torch.Tensor | None = None) -> PreparedF6:
    """prepare (bits 4) with the codes written as bf6: the same codes and
    scales as prepare followed by f6_activation, in one pass."""
    rows, width = x.shape
    out = _prepared_f6_storage(rows, width, x.device, out)
    _check(lib().clef_i4_prepare_f6(_ptr(x), rows, width, _ptr(out), _stream()))
    return PreparedF6(out, rows, width)


def prepare_swiglu_f6(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> PreparedF6:
    """prepare_swiglu (bits 4) with the codes written as bf6."""
    rows, width = gate.shape
    out = _prepared_f6_storage(rows, width, gate.device, out)
    _check(lib().clef_i4_prepare_swiglu_f6(_ptr(gate), _ptr(up), rows, width, _ptr(out), _stream()))
    return PreparedF6(out, rows, width)


def project_f6(a: PreparedF6, w: F6Weight, residual: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """G1 through the bf6 GEMM on a bf6-prepared activation: equal to
    project_prepared(prepare(x), w) for the weight w came from."""
    if a.width != w.cols:
        raise ClefError(-1, "unsupported integer projection shape")
    return gemm_f6(a.codes, a.scales, w, residual, out)


def project_gate_up_f6(a: PreparedF6, gate: F6Weight, up: F6Weight, out: torch.Tensor | None = None
                       ) -> torch.Tensor:
    """The dense MLP's gate and up projections with SwiGLU in one bf6 GEMM
    (clef_i4_gemm_f6_gate_up): h = swiglu(project_f6(a, gate), project_f6(a,
    up)) bit for bit, for the reference's dense MLP (src/quantized.rs:399-401,
    406-439), without writing gate and up."""
    if a.width != gate.cols or gate.cols != up.cols or gate.rows != up.rows:
        raise ClefError(-1, "unsupported integer projection shape")
    if out is None:
        out = _empty((a.rows, gate.rows), torch.bfloat16, a.storage.device)
    _check(lib().clef_i4_gemm_f6_gate_up(_ptr(a.codes), _ptr(a.scales), _ptr(gate.codes), _ptr(gate.scales),
                                         _ptr(up.codes), _ptr(up.scales), a.rows, gate.rows, gate.cols, _ptr(out),
                                         _stream()))
    return out


def project_quantized_f6(x: torch.Tensor, w: F6Weight, residual: torch.Tensor | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """project_quantized through the bf6 path in one C call
    (clef_i4_project_f6): x quantized into bf6 in a workspace, then the bf6
    GEMM. Same output as project_quantized(x, the 4-bit weight)."""
    m, k = x.shape
    if out is None:
        out = _empty((m, w.rows), torch.bfloat16, x.device)
    nbytes = int(lib().clef_i4_project_f6_workspace_bytes(m, k))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    _check(lib().clef_i4_project_f6(_ptr(x), m, k, _ptr(w.codes), _ptr(w.scales), w.rows, _ptr(residual), _ptr(out),
                                    _ptr(ws), nbytes, _stream()))
    return out


def project_prepared_f6(a: Prepared, w: F6Weight, residual: torch.Tensor | None = None,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """project_prepared through the bf6 GEMM: the activation re-encoded, then G1."""
    if a.width != w.cols:
        raise ClefError(-1, "unsupported integer projection shape")
    return gemm_f6(f6_activation(a), a.scales, w, residual, out)


def project_quantized(x: torch.Tensor, w: QuantizedWeight, residual: torch.Tensor | None = None
                      ) -> torch.Tensor:
    """Engine::project_quantized[_with_residual] (src/quantized.rs:235-303)."""
    m, k = x.shape
    out = _empty((m, w.rows), torch.bfloat16, x.device)
    ws_bytes = int(lib().clef_i4_project_workspace_bytes(m, k))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=x.device)
    _check(lib().clef_i4_project(_ptr(x), m, k, _ptr(w.codes), _ptr(w.scales), w.rows, _ptr(residual),
                                 _ptr(out), _ptr(ws), ws_bytes, _stream()))
    return out


def project_attention_gate(attention: torch.Tensor, q_gate: torch.Tensor, w: QuantizedWeight,
                           residual: torch.Tensor) -> torch.Tensor:
    """Engine::project_attention_gate (src/quantized.rs:440-468): gated
    attention packed in one pass, then the residual projection."""
    if attention.shape[1] != w.cols:
        raise ClefError(-1, "attention projection width mismatch")
    a = prepare_attention_gate(attention, q_gate, w.bits, w.stride)
    return project_prepared(a, w, residual=residual)


# ---------------------------------------------------------------- MoE

def router_logits(x: torch.Tensor, gate_w: torch.Tensor) -> torch.Tensor:
    """The Omni router gate, e.project(norm, "mlp.gate") (src/omni.rs:764):
    bf16 logits [tokens][experts] = x @ gate_w.T with f32 accumulation."""
    tokens, hidden = x.shape
    experts = gate_w.shape[0]
    if gate_w.shape[1] != hidden or x.dtype != torch.bfloat16 or gate_w.dtype != torch.bfloat16:
        raise ClefError(-1, "linear shape/dtype mismatch")
    out = _empty((tokens, experts), torch.bfloat16, x.device)
    _check(lib().clef_moe_router_logits(_ptr(x.contiguous()), _ptr(gate_w.contiguous()), tokens, hidden, experts,
                                        _ptr(out), _stream()))
    return out


def omni_route(logits: torch.Tensor, topk: int = 8) -> torch.Tensor:
    """Engine::omni_route (src/omni.rs:170-190)."""
    tokens, experts = logits.shape
    dtype = 0 if logits.dtype == torch.bfloat16 else 1
    routes = _empty((tokens, 2 * topk), torch.float32, logits.device)
    _check(lib().clef_moe_route(_ptr(logits), dtype, tokens, experts, topk, _ptr(routes), _stream()))
    return routes


def omni_group_routes(routes: torch.Tensor, ordered: bool = True):
    """Engine::omni_group_routes[_ordered] (src/omni.rs:192-245) -> (groups, order|None)."""
    tokens = routes.shape[0]
    topk = routes.shape[1] // 2
    groups = torch.zeros((128, tokens + 1), dtype=torch.float32, device=routes.device)
    order = torch.zeros((tokens, topk), dtype=torch.float32, device=routes.device) if ordered else None
    ws_bytes = int(lib().clef_moe_group_workspace_bytes(tokens))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=routes.device)
    _check(lib().clef_moe_group_routes(_ptr(routes), tokens, topk, _ptr(groups), _ptr(order), _ptr(ws),
                                       ws_bytes, _stream()))
    return groups, order


def omni_expert_tasks(groups: torch.Tensor, topk: int = 8) -> torch.Tensor:
    """omni_expert_tasks dispatch of Engine::omni_compact_routes (src/omni.rs:155-165)."""
    tokens = groups.shape[1] - 1
    tasks = torch.zeros(1 + 2 * ((tokens * topk + 15) // 16 + 127), dtype=torch.float32,
                        device=groups.device)
    _check(lib().clef_moe_expert_tasks(_ptr(groups), tokens, _ptr(tasks), _stream()))
    return tasks


def omni_expert(a: Prepared, w: QuantizedWeight, groups: torch.Tensor, tokens: int, topk: int,
                input_routed: bool) -> torch.Tensor:
    """Engine::omni_expert_impl (src/omni.rs:289-534); w holds 128 experts' rows."""
    n = w.rows // 128
    out = torch.zeros((tokens * topk, n), dtype=torch.bfloat16, device=groups.device)
    ws_bytes = int(lib().clef_moe_expert_workspace_bytes(tokens, topk))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=groups.device)
    _check(lib().clef_moe_expert_i4(_ptr(a.storage), a.stride, _ptr(a.scales), _ptr(w.codes),
                                    _ptr(w.scales), _ptr(groups), tokens, topk, w.cols, n,
                                    int(input_routed), _ptr(out), _ptr(ws), ws_bytes, _stream()))
    return out


def omni_expert_ungrouped(a: Prepared, w: QuantizedWeight, routes: torch.Tensor, input_routed: bool
                          ) -> torch.Tensor:
    """Engine::omni_expert (src/omni.rs:280-288), the expert GEMM without a
    groups table: every route slot computed on its own. Rows of slots naming
    no expert stay zero."""
    tokens = routes.shape[0]
    topk = routes.shape[1] // 2
    n = w.rows // 128
    out = torch.zeros((tokens * topk, n), dtype=torch.bfloat16, device=routes.device)
    ws_bytes = int(lib().clef_moe_expert_ungrouped_workspace_bytes(tokens, topk))
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=routes.device)
    _check(lib().clef_moe_expert_i4_ungrouped(_ptr(a.storage), a.stride, _ptr(a.scales), _ptr(w.codes),
                                              _ptr(w.scales), _ptr(routes), tokens, topk, w.cols, n,
                                              int(input_routed), _ptr(out), _ptr(ws), ws_bytes, _stream()))
    return out


def omni_gate_up(a: Prepared, gate: QuantizedWeight, up: QuantizedWeight, groups: torch.Tensor, tokens: int,
                 topk: int) -> torch.Tensor:
    """Engine::omni_gate_up (src/omni.rs:300-372): fused gate/up expert GEMMs
    and SwiGLU over the routed rows; h bf16 [tokens * topk][n]."""
    n = gate.rows // 128
    h = torch.zeros((tokens * topk, n), dtype=torch.bfloat16, device=groups.device)
    ws_bytes = int(lib().clef_moe_expert_workspace_bytes(tokens, topk))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=groups.device)
    _check(lib().clef_moe_expert_gate_up_i4(_ptr(a.storage), a.stride, _ptr(a.scales), _ptr(gate.codes),
                                            _ptr(gate.scales), _ptr(up.codes), _ptr(up.scales), _ptr(groups),
                                            tokens, topk, gate.cols, n, _ptr(h), _ptr(ws), ws_bytes, _stream()))
    return h


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Engine::swiglu (src/ops.rs:9-29)."""
    if gate.shape != up.shape:
        raise ClefError(-1, "SwiGLU shape/dtype mismatch")
    h = torch.empty_like(gate)
    _check(lib().clef_swiglu(_ptr(gate), _ptr(up), gate.numel(), _ptr(h), _stream()))
    return h


def omni_combine(values: torch.Tensor, routes: torch.Tensor, order: torch.Tensor | None = None
                 ) -> torch.Tensor:
    """Engine::omni_combine[_ordered] (src/omni.rs:246-278, 535-556)."""
    tokens = routes.shape[0]
    topk = routes.shape[1] // 2
    width = values.shape[1]
    out = _empty((tokens, width), torch.bfloat16, values.device)
    _check(lib().clef_moe_combine(_ptr(values), _ptr(routes), _ptr(order), tokens, width, topk, _ptr(out),
                                  _stream()))
    return out


class MoeLayer:
    """Omni INT4 MoE block (src/omni.rs:760-857) over resident packed experts.

    The workspace is allocated once per (tokens) and reused by every call.
    """

    def __init__(self, gate: QuantizedWeight, up: QuantizedWeight, down: QuantizedWeight, topk: int = 8,
                 router: torch.Tensor | None = None):
        self.gate, self.up, self.down, self.topk = gate, up, down, topk
        self.router = router  # bf16 [128][hidden] router gate, used when no logits are given
        self.hidden = gate.cols
        self.inter = gate.rows // 128
        self._ws = None
        self._ws_tokens = -1

    def workspace(self, tokens: int, device) -> torch.Tensor:
        if self._ws_tokens != tokens:
            nbytes = int(lib().clef_moe_layer_workspace_bytes(tokens, self.hidden, self.inter, self.topk))
            self._ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._ws_tokens = tokens
        return self._ws

    def __call__(self, x: torch.Tensor, logits: torch.Tensor | None = None, routes_out: torch.Tensor | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        tokens = x.shape[0]
        if logits is None:
            if self.router is None:
                raise ClefError(-1, "MoE layer needs router logits or a router gate weight")
            logits = router_logits(x, self.router)  # e.project(norm, "mlp.gate"), src/omni.rs:764
        if out is None:
            out = _empty((tokens, self.hidden), torch.bfloat16, x.device)
        ws = self.workspace(tokens, x.device)
        dtype = 0 if logits.dtype == torch.bfloat16 else 1
        _check(lib().clef_moe_layer(_ptr(x), _ptr(logits), dtype, tokens, self.hidden, self.inter, 128,
                                    self.topk, _ptr(self.gate.codes), _ptr(self.gate.scales),
                                    _ptr(self.up.codes), _ptr(self.up.scales), _ptr(self.down.codes),
                                    _ptr(self.down.scales), _ptr(routes_out), _ptr(out), _ptr(ws),
                                    ws.numel(), _stream()))
        return out
