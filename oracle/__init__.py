"""numpy front end of the C oracle (oracle/clef_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product path never does.

Arrays: bf16 tensors travel as uint16 bit patterns, packed codes as uint32,
routing tables as float32, exactly the reference's layouts.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libclef_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


def build() -> None:
    """Compile the oracle library with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_last_error": (ctypes.c_char_p, []),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_expf": (ctypes.c_float, [ctypes.c_float]),
            "orc_rotate256": (None, [_P]),
            "orc_prepare": (ctypes.c_int, [_P, _I64, _I32, _I32, _I32, _P]),
            "orc_prepare_swiglu": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P]),
            "orc_prepare_attention_gate": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P]),
            "orc_prepare_norm": (ctypes.c_int, [_P, _P, _I64, _I32, _I32, _I32, _P, _P]),
            "orc_rms_norm": (ctypes.c_int, [_P, _P, _I64, _I32, _P]),
            "orc_retile": (ctypes.c_int, [_P, _I64, _I32, _I32, _I32, _P]),
            "orc_gemm_acc": (ctypes.c_int, [_P, _I32, _P, _I64, _I32, _I32, _I32, _P]),
            "orc_gemm": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P]),
            "orc_route": (ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _P]),
            "orc_group_routes": (ctypes.c_int, [_P, _I64, _I32, _P, _P]),
            "orc_expert_tasks": (ctypes.c_int, [_P, _I64, _P]),
            "orc_expert_i4": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
            "orc_swiglu": (None, [_P, _P, _I64, _P]),
            "orc_combine": (ctypes.c_int, [_P, _P, _P, _I64, _I32, _I32, _P]),
            "orc_expert_i4_ungrouped": (ctypes.c_int, [_P, _I32, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32,
                                                       _P]),
            "orc_moe_layer": (ctypes.c_int, [_P, _P, _I32, _I64, _I32, _I32, _I32, _I32,
                                             _P, _P, _P, _P, _P, _P, _P, _P]),
            "orc_tile_rows": (ctypes.c_int, [_P, _I64, _I32, _P]),
            "orc_untile_rows": (ctypes.c_int, [_P, _I64, _I32, _P]),
            "orc_threads": (ctypes.c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


class OracleError(RuntimeError):
    pass


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(rc):
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


# ---- scalar helpers -------------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    """float32 array -> bf16 bit patterns (RNE, NaN stays NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def expf(x: float) -> float:
    return lib().orc_expf(float(x))


def rotate256(group) -> np.ndarray:
    g = np.array(group, dtype=np.float32).copy()
    assert g.shape == (256,)
    lib().orc_rotate256(_ptr(g))
    return g


# ---- Q1 / Q2 --------------------------------------------------------------

def activation_stride(width: int, bits: int = 4) -> int:
    """src/quantized.rs:161-166."""
    return width + (512 // bits if width % 1024 == 0 else 0)


def prepare(x: np.ndarray, stride: int, bits: int = 4):
    """Q1 -> (codes u32 [rows][stride/(32/bits)], scales f32 [rows], storage)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    rows, width = x.shape
    words = stride // (32 // bits)
    out = np.zeros(rows * (words + 1), dtype=np.uint32)
    _check(lib().orc_prepare(_ptr(x), rows, width, stride, bits, _ptr(out)))
    codes = out[: rows * words].reshape(rows, words)
    scales = out[rows * words:].view(np.float32)
    return codes, scales, out


def prepare_swiglu(gate: np.ndarray, up: np.ndarray, stride: int, bits: int = 4):
    gate = np.ascontiguousarray(gate, dtype=np.uint16)
    up = np.ascontiguousarray(up, dtype=np.uint16)
    rows, width = gate.shape
    words = stride // (32 // bits)
    out = np.zeros(rows * (words + 1), dtype=np.uint32)
    _check(lib().orc_prepare_swiglu(_ptr(gate), _ptr(up), rows, width, stride, bits, _ptr(out)))
    return out[: rows * words].reshape(rows, words), out[rows * words:].view(np.float32), out


def prepare_attention_gate(x: np.ndarray, q_gate: np.ndarray, stride: int, bits: int = 4):
    """Q1 of bf16(x * bf16(sigmoid(gate))); q_gate is [rows][2*width]
    (kernels/prepare_integer_register.loom:137-155)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    q_gate = np.ascontiguousarray(q_gate, dtype=np.uint16)
    rows, width = x.shape
    assert q_gate.shape == (rows, 2 * width)
    words = stride // (32 // bits)
    out = np.zeros(rows * (words + 1), dtype=np.uint32)
    _check(lib().orc_prepare_attention_gate(_ptr(x), _ptr(q_gate), rows, width, stride, bits, _ptr(out)))
    return out[: rows * words].reshape(rows, words), out[rows * words:].view(np.float32), out


def prepare_norm(x: np.ndarray, weight: np.ndarray, stride: int, bits: int = 4):
    """Q1 of the named RMSNorm (width 5120, weight + 1, eps 1e-6) ->
    (codes, scales, storage, normalized bf16 [rows][5120])."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    rows, width = x.shape
    words = stride // (32 // bits)
    out = np.zeros(rows * (words + 1), dtype=np.uint32)
    normalized = np.zeros((rows, width), dtype=np.uint16)
    _check(lib().orc_prepare_norm(_ptr(x), _ptr(weight), rows, width, stride, bits, _ptr(out),
                                  _ptr(normalized)))
    return out[: rows * words].reshape(rows, words), out[rows * words:].view(np.float32), out, normalized


def rms_norm(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.zeros_like(x)
    _check(lib().orc_rms_norm(_ptr(x), _ptr(weight), x.shape[0], x.shape[1], _ptr(out)))
    return out


def retile(codes: np.ndarray, cols: int, bits: int = 4) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    rows, in_words = codes.shape
    words = cols // (32 // bits)
    tiled = np.zeros(rows * words, dtype=np.uint32)
    _check(lib().orc_retile(_ptr(codes), rows, in_words, cols, bits, _ptr(tiled)))
    return tiled


def pack_weight(w: np.ndarray, bits: int = 4):
    """Q2: bf16 [N][K] row-major -> (tiled codes u32 [N*K/(32/bits)], scales f32 [N])."""
    n, k = w.shape
    stride = activation_stride(k, bits)
    codes, scales, _ = prepare(w, stride, bits)
    return retile(codes, k, bits), scales.copy()


# ---- G1 -------------------------------------------------------------------

def gemm_acc(a_codes: np.ndarray, w_tiled: np.ndarray, n: int, k: int, bits: int = 4) -> np.ndarray:
    a_codes = np.ascontiguousarray(a_codes, dtype=np.uint32)
    m, a_words = a_codes.shape
    acc = np.zeros((m, n), dtype=np.int32)
    _check(lib().orc_gemm_acc(_ptr(a_codes), a_words * (32 // bits), _ptr(w_tiled), m, n, k, bits,
                              _ptr(acc)))
    return acc


def gemm(a_codes, a_scales, w_tiled, w_scales, n: int, k: int, bits: int = 4, residual=None):
    a_codes = np.ascontiguousarray(a_codes, dtype=np.uint32)
    a_scales = np.ascontiguousarray(a_scales, dtype=np.float32)
    w_scales = np.ascontiguousarray(w_scales, dtype=np.float32)
    m, a_words = a_codes.shape
    out = np.zeros((m, n), dtype=np.uint16)
    if residual is not None:
        residual = np.ascontiguousarray(residual, dtype=np.uint16)
    _check(lib().orc_gemm(_ptr(a_codes), a_words * (32 // bits), _ptr(a_scales), _ptr(w_tiled),
                          _ptr(w_scales), m, n, k, bits, _ptr(residual), _ptr(out)))
    return out


# ---- MoE ------------------------------------------------------------------

def route(logits: np.ndarray, topk: int = 8) -> np.ndarray:
    if logits.dtype == np.uint16:
        dtype = 0
    else:
        logits = logits.astype(np.float32)
        dtype = 1
    logits = np.ascontiguousarray(logits)
    t, e = logits.shape
    routes = np.zeros((t, 2 * topk), dtype=np.float32)
    _check(lib().orc_route(_ptr(logits), dtype, t, e, topk, _ptr(routes)))
    return routes


def group_routes(routes: np.ndarray, topk: int = 8):
    routes = np.ascontiguousarray(routes, dtype=np.float32)
    t = routes.shape[0]
    groups = np.zeros((128, t + 1), dtype=np.float32)
    order = np.zeros((t, topk), dtype=np.float32)
    _check(lib().orc_group_routes(_ptr(routes), t, topk, _ptr(groups), _ptr(order)))
    return groups, order


def expert_tasks(groups: np.ndarray) -> np.ndarray:
    groups = np.ascontiguousarray(groups, dtype=np.float32)
    t = groups.shape[1] - 1
    tasks = np.zeros(1 + 2 * ((8 * t + 15) // 16 + 127), dtype=np.float32)
    _check(lib().orc_expert_tasks(_ptr(groups), t, _ptr(tasks)))
    return tasks


def expert_i4(a_codes, a_scales, w_tiled, w_scales, groups, tokens: int, topk: int, k: int, n: int,
              input_routed: bool) -> np.ndarray:
    a_codes = np.ascontiguousarray(a_codes, dtype=np.uint32)
    stride = a_codes.shape[1] * 8
    out = np.zeros((tokens * topk, n), dtype=np.uint16)
    _check(lib().orc_expert_i4(_ptr(a_codes), stride, _ptr(np.ascontiguousarray(a_scales, np.float32)),
                               _ptr(w_tiled), _ptr(np.ascontiguousarray(w_scales, np.float32)),
                               _ptr(np.ascontiguousarray(groups, np.float32)), tokens, topk, k, n,
                               int(input_routed), _ptr(out)))
    return out


def expert_i4_ungrouped(a_codes, a_scales, w_tiled, w_scales, routes, k: int, n: int,
                        input_routed: bool) -> np.ndarray:
    """Every route slot of routes [T][2*topk] on its own; rows of slots naming
    no expert stay zero."""
    a_codes = np.ascontiguousarray(a_codes, dtype=np.uint32)
    routes = np.ascontiguousarray(routes, dtype=np.float32)
    tokens, topk = routes.shape[0], routes.shape[1] // 2
    stride = a_codes.shape[1] * 8
    out = np.zeros((tokens * topk, n), dtype=np.uint16)
    _check(lib().orc_expert_i4_ungrouped(_ptr(a_codes), stride, _ptr(np.ascontiguousarray(a_scales, np.float32)),
                                         _ptr(w_tiled), _ptr(np.ascontiguousarray(w_scales, np.float32)),
                                         _ptr(routes), tokens, topk, k, n, int(input_routed), _ptr(out)))
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.uint16)
    up = np.ascontiguousarray(up, dtype=np.uint16)
    h = np.zeros_like(gate)
    lib().orc_swiglu(_ptr(gate), _ptr(up), gate.size, _ptr(h))
    return h


def combine(values, routes, order=None, topk: int = 8) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.uint16)
    routes = np.ascontiguousarray(routes, dtype=np.float32)
    t = routes.shape[0]
    width = values.shape[1]
    out = np.zeros((t, width), dtype=np.uint16)
    if order is not None:
        order = np.ascontiguousarray(order, dtype=np.float32)
    _check(lib().orc_combine(_ptr(values), _ptr(routes), _ptr(order), t, width, topk, _ptr(out)))
    return out


def moe_layer(x, logits, gate, up, down, topk: int = 8):
    """x bf16 [T][D]; logits bf16/f32 [T][128]; gate/up/down = (tiled, scales)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    t, d = x.shape
    inter = gate[1].shape[0] // 128
    if logits.dtype == np.uint16:
        ldt = 0
    else:
        logits = logits.astype(np.float32)
        ldt = 1
    logits = np.ascontiguousarray(logits)
    routes = np.zeros((t, 2 * topk), dtype=np.float32)
    out = np.zeros((t, d), dtype=np.uint16)
    _check(lib().orc_moe_layer(_ptr(x), _ptr(logits), ldt, t, d, inter, 128, topk,
                               _ptr(gate[0]), _ptr(gate[1]), _ptr(up[0]), _ptr(up[1]),
                               _ptr(down[0]), _ptr(down[1]), _ptr(routes), _ptr(out)))
    return out, routes


def tile_rows(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint16)
    out = np.zeros_like(w)
    _check(lib().orc_tile_rows(_ptr(w), w.shape[0], w.shape[1], _ptr(out)))
    return out


def untile_rows(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint16)
    out = np.zeros_like(w)
    _check(lib().orc_untile_rows(_ptr(w), w.shape[0], w.shape[1], _ptr(out)))
    return out


def threads() -> int:
    return lib().orc_threads()
