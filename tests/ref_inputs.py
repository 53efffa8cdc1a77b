"""Input formulas of the reference's own tests, restated in numpy (bf16 bit
patterns), shared by the CPU pins of the oracle and the GPU parity tests."""
import numpy as np

import oracle

BF16_MAX = 0x7F7F


def swiglu_gate_up(width: int, rows: int):
    """gate and up of fused_swiglu_packing_matches_reference
    (src/quantized.rs:1189-1266): the gate buffer holds rows + 2 rows and the
    test takes rows [1, rows + 1); the up buffer holds rows + 3 rows and the
    test takes rows [2, rows + 2). Gate row classes cycle with the buffer row
    (i / width) % 7: 0 -> 0.0; 1 -> NaN at column 259; 2 -> +inf at column
    515; 3 -> bf16::MAX; 4 -> f32::from_bits(0x00010000) (the bf16 denormal
    0x0001); 5 -> -80 on even and +80 on odd columns; other rows and columns
    ((i * 17 % 1031) - 515) / 16. up: ((i * 29 % 997) - 498) / 32."""
    i = np.arange((rows + 2) * width, dtype=np.int64)
    col = i % width
    cls = (i // width) % 7
    g = ((i * 17 % 1031).astype(np.float32) - np.float32(515.0)) / np.float32(16.0)
    g = np.where(cls == 0, np.float32(0.0), g)
    g = np.where((cls == 1) & (col == 259), np.float32(np.nan), g)
    g = np.where((cls == 2) & (col == 515), np.float32(np.inf), g)
    g = np.where(cls == 5, np.where(col % 2 == 0, np.float32(-80.0), np.float32(80.0)), g)
    gate = oracle.f32_to_bf16(g.astype(np.float32))
    gate[cls == 3] = BF16_MAX
    gate[cls == 4] = 0x0001  # bf16::from_f32(f32::from_bits(0x0001_0000))
    j = np.arange((rows + 3) * width, dtype=np.int64)
    u = ((j * 29 % 997).astype(np.float32) - np.float32(498.0)) / np.float32(32.0)
    up = oracle.f32_to_bf16(u.astype(np.float32))
    gate = gate.reshape(rows + 2, width)[1:rows + 1]
    up = up.reshape(rows + 3, width)[2:rows + 2]
    return np.ascontiguousarray(gate), np.ascontiguousarray(up)


def fused_swiglu_cases():
    """(width, bits, row counts) of the reference test; 768 at bits 8 is added."""
    return [(17408, 4, [1, 128, 158, 620]), (17408, 8, [1, 128, 158, 620]),
            (768, 4, [8, 136, 2048, 8192, 16384]), (768, 8, [8, 136, 2048])]
