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

// An 8 KiB window of the table for epilogues whose LDS budget cannot hold
// all of it: exponent fields kSiluWinExp0 .. kSiluWinExp0 + 15 (2^-10 <= |g| <
// 2^6), both signs, at byte sign * 4096 + (e - kSiluWinExp0) * 256 + mantissa
// * 2; the window's half for sign s is the 4 KiB of g_silu_lut at byte
// s * kSiluLutSize + kSiluWinSrc.
constexpr int kSiluWinExp0 = 117, kSiluWinBinades = 16;
constexpr int kSiluWinBytes = 2 * kSiluWinBinades * 128 * 2;
constexpr int kSiluWinSrc = (kSiluWinExp0 - kSiluLutExp0) * 256;
static_assert(kSiluWinExp0 >= kSiluLutExp0 && kSiluWinExp0 + kSiluWinBinades <= kSiluLutExp0 + kSiluLutBinades,
              "window inside the SiLU table");

// bf16 silu of both halves of `pair` (bf16 bits) from the window:
//  * 2^-10 <= |g| < 2^6: the window entry;
//  * |g| < 2^-10 with exponent field >= 2, and +-0: g / 2 (the exponent field
//    minus one), which equals silu_bf16 for every such bf16 g: there
//    |silu(g) - g / 2| ~ g^2 / 4 stays below half a bf16 ulp of g / 2 (the
//    equality is checked on every such bf16 by the tests);
//  * the rest (|g| >= 2^6, inf, NaN and, with TINY, subnormal g and exponent
//    field 1) is flagged in bit 15 of its half of `outside` for the caller's
//    exact path (silu_bf16).
// Callers that know every nonzero g has exponent field >= 2 pass TINY = false.
template <bool TINY>
__device__ __forceinline__ uint32_t silu_window_pair(uint32_t pair, const char* __restrict__ table,
                                                     uint32_t& outside) {
  const u16x2 h = __builtin_bit_cast(u16x2, pair);
  const u16x2 a = h & (uint16_t)0x7FFF;
  // exponent field >= kSiluWinExp0 + 16 (a <= 0x7FFF: no carry out of bit 15)
  const u16x2 big = (a + (uint16_t)(0x8000 - ((kSiluWinExp0 + kSiluWinBinades) << 7))) & (uint16_t)0x8000;
  uint32_t flag = __builtin_bit_cast(uint32_t, big);
  if constexpr (TINY) {
    // 1 <= a <= 0x100 (a == 0x100 is flagged needlessly): (a - 1) >> 8 is 0
    // exactly there (a == 0 wraps to 0xFFFF), and 0 - 1 sets bit 15
    const u16x2 hi8 = (u16x2)(a - (uint16_t)1) >> (uint16_t)8;
    flag |= __builtin_bit_cast(uint32_t, (u16x2)((u16x2)(hi8 - (uint16_t)1) & (uint16_t)0x8000));
  }
  outside |= flag;
  // 0xFFFF in the halves below the window (a < kSiluWinExp0 << 7), +-0 included
  const s16x2 d = __builtin_bit_cast(s16x2, (u16x2)(a - (uint16_t)(kSiluWinExp0 << 7)));
  const uint32_t small = __builtin_bit_cast(uint32_t, (s16x2)(d >> (int16_t)15));
  // g / 2: the exponent field minus one (saturating: +-0 stays +-0), sign kept
  const uint32_t half =
      __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(a, (u16x2)(uint16_t)0x80)) | (pair & 0x80008000u);
  // window byte offsets (e - e0) << 8 | mantissa << 1 with the sign at bit 12;
  // inside [0, 8 KiB) for every input
  const u16x2 t = h - (uint16_t)(kSiluWinExp0 << 7);
  const uint32_t off = (__builtin_bit_cast(uint32_t, (u16x2)(t << (uint16_t)1)) & 0x0FFF0FFFu) |
                       (__builtin_bit_cast(uint32_t, (u16x2)(h >> (uint16_t)3)) & 0x10001000u);
  const uint32_t lo = *reinterpret_cast<const uint16_t*>(table + (off & 0xFFFFu));
  const uint32_t hi = *reinterpret_cast<const uint16_t*>(table + (off >> 16));
  const uint32_t tbl = lo | (hi << 16);
  return (tbl & ~small) | (half & small);
}

}  // namespace clef
