// silu_bf16 of every bf16 value with exponent field kSiluLutExp0 ..
// kSiluLutExp0 + kSiluLutBinades - 1, at silu_lut_index (16 KiB). The entries
// are generated at build time on the host by silu_table_gen.cpp from the same
// host-and-device functions, so the table is part of each code object that
// includes this header and needs no set-up launch.
#pragma once

#include "common.hpp"

namespace clef {

__device__ const uint16_t g_silu_lut[kSiluLutSize] __attribute__((unused, aligned(16))) = {
#include "silu_table.inc"
};

// bf16(silu(g)) for N bf16 values g (exact bf16 values in f32): table reads
// for all, then wave-uniform branches for values outside the table (zeros,
// then the rest).
// `table` is g_silu_lut or a copy of it (in LDS).
template <int N>
__device__ __forceinline__ void silu_lut(const float (&g)[N], float (&act)[N], const uint16_t* table = g_silu_lut) {
  bool inside[N];
  bool slow = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t off = silu_lut_offset(as_uint(g[i]), inside[i]);
    slow |= !inside[i];
    act[i] = bf16_to_f32(table[off >> 1]);
  }
  if (__any(slow)) {
    // silu(+-0) = +-0 directly, then the other values outside the table
    bool others = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (!inside[i] && g[i] == 0.0f) act[i] = g[i];
      others = others | (!inside[i] & (g[i] != 0.0f));
    }
    if (__any(others)) {
#pragma unroll
      for (int i = 0; i < N; ++i)
        if (!inside[i] & (g[i] != 0.0f)) act[i] = silu_bf16(g[i]);
    }
  }
}

}  // namespace clef
