// Device helpers shared by the gfx950 kernels of the INT4 quantized-matmul and
// Omni INT4 MoE path. Every helper states the IEEE steps it performs so the
// arithmetic can be checked against the reference kernels line by line.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace clef {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

// Host-and-device helpers: the SiLU table is generated on the host at build
// time from the same steps (see silu_table_gen.cpp).
#define CLEF_HD __host__ __device__ __forceinline__

CLEF_HD float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
CLEF_HD uint32_t as_uint(float f) { return __builtin_bit_cast(uint32_t, f); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// f32 -> bf16 round-to-nearest-even; a NaN stays a quiet NaN with its sign and
// top payload bits ((u >> 16) | 0x40). kernels/common.loom:29-35
// (scalar.fptrunc f32 to bf16). gfx950's v_cvt_pk_bf16_f32 computes exactly
// this for every f32 bit pattern (checked exhaustively on the device), so the
// conversion is one instruction per pair.
CLEF_HD uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
// bf16(+0) is 0x0000, so the other half of the pair needs no mask: each of
// these is the one conversion instruction.
CLEF_HD uint32_t f32_to_bf16(float f) { return pack_bf16x2(f, 0.0f); }

CLEF_HD float bf16_to_f32(uint32_t h) { return as_float(h << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return as_float(pair & 0xffff0000u); }
CLEF_HD float bf16_round(float f) { return as_float(pack_bf16x2(0.0f, f)); }

// exp(x) by Cody-Waite reduction with ln 2 split as 0.693359375 - 2.12194440e-4
// and the degree-5 minimax polynomial of the Cephes expf (S. L. Moshier, Cephes
// Math Library). Every step is an explicit IEEE op (fma where written), so the
// host restatement in the oracle produces the same bits. Stands in for the
// reference's approximate expf<afn> (kernels/swiglu.loom:46,
// kernels/omni_route.loom:131).
CLEF_HD float cephes_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_huge_valf();
  if (x < -103.972076416015625f) return 0.0f;
  float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float r2 = r * r;
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  p = __builtin_fmaf(p, r2, r);
  p = p + 1.0f;
  return __builtin_ldexpf(p, (int)n);
}

// The activation half of S1: bf16(g / (1 + exp(-g))). kernels/swiglu.loom:43-47.
CLEF_HD float silu_bf16(float g) {
  float e = cephes_expf(-g);
  float d = 1.0f + e;
  return bf16_round(g / d);
}

// S1: h = bf16(f32(bf16(g / (1 + exp(-g)))) * u). kernels/swiglu.loom:43-51.
__device__ __forceinline__ float swiglu1(float g, float u) { return bf16_round(silu_bf16(g) * u); }

// silu_bf16 tabulated for every bf16 g with 2^-25 <= |g| < 2^7 (exponent field
// 102..133), as bf16 bits at index sign * 4096 + (exponent - 102) * 128 +
// mantissa. Other g (tiny, large, inf, NaN) are computed directly.
constexpr int kSiluLutExp0 = 102, kSiluLutBinades = 32;
constexpr int kSiluLutSize = 2 * kSiluLutBinades * 128;
__device__ __forceinline__ int silu_lut_index(uint32_t gbits) {
  const uint32_t e = ((gbits >> 7) & 0xFFu) - kSiluLutExp0;
  return e < (uint32_t)kSiluLutBinades ? (int)(((gbits >> 15) << 12) | (e << 7) | (gbits & 127u)) : -1;
}

// Byte offset in the table of the bf16 value held in the high half of w (low
// half zero): 2 * silu_lut_index. Bits 28..30 of t = w - (kSiluLutExp0 << 23)
// are zero exactly when the exponent field lies in the table's range, for
// either sign; then t >> 15 holds (exponent - kSiluLutExp0) << 8 | mantissa << 1
// in its low 13 bits and the sign bit moves to bit 13. Outside the range
// `inside` is false and the offset is still within the 16 KiB table.
__device__ __forceinline__ uint32_t silu_lut_offset(uint32_t w, bool& inside) {
  const uint32_t t = w - ((uint32_t)kSiluLutExp0 << 23);
  inside = (t & 0x70000000u) == 0;
  return ((t >> 15) & 0x1FFFu) | ((w >> 18) & ~0x1FFFu);  // w >> 18 < 2^14: bit 13 is the sign
}

// Makes v opaque to the compiler (an empty asm that "changes" it in its
// VGPR): later uses take the register, never a re-read of the memory it came
// from. For values read from LDS that other lanes overwrite afterwards.
__device__ __forceinline__ void pin_vgpr(float& v) { asm volatile("" : "+v"(v)); }

// e3m2 (bf6: sign, 3 exponent bits with bias 3, 2 mantissa bits) of the int4
// code held in nibble n (two's complement); every code -8..7 is exact.
__host__ __device__ constexpr uint32_t e3m2_of_nibble(uint32_t n) {
  // magnitudes 0..7: 0, 1.0*2^0, 1.0*2^1, 1.5*2^1, 1.0*2^2, 1.25*2^2, 1.5*2^2, 1.75*2^2
  constexpr uint64_t kPos = 0x1716151412100C00ull;
  const uint32_t m = n < 8 ? n : 16 - n;  // |code|, 8 for n == 8
  const uint32_t mag = m == 8 ? 0x18u : (uint32_t)(kPos >> (8 * m)) & 0xFFu;
  return n < 8 ? mag : (mag | 0x20u);
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef int16_t s16x2 __attribute__((ext_vector_type(2)));

// 0x8000 in each half of a bf16 pair that holds +-0, 0xFFFF in the others:
// ANDed into a result pair it keeps only the sign where the operand was zero.
__device__ __forceinline__ uint32_t bf16x2_zero_keep(uint32_t pair) {
  // bit 15 of each half of f: that half of pair is nonzero (no carry between
  // halves: each is at most 0x7FFF + 0x7FFF)
  const uint32_t f = (pair & 0x7FFF7FFFu) + 0x7FFF7FFFu;
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, f) >> (int16_t)15) | 0x80008000u;
}

// silu_lut_offset of two bf16 values at once, with packed 16-bit operations:
// `pair` holds the bf16 bits of two values (low and high half); the result
// holds their two byte offsets in the same halves. In 16 bits,
// t = h - (kSiluLutExp0 << 7) has bits 12..14 zero exactly when h's exponent
// field is in the table's range, (t << 1) & 0x1FFF = (exponent - kSiluLutExp0)
// << 8 | mantissa << 1 and h >> 2 puts the sign at bit 13, as in
// silu_lut_offset. Bits 12..14 of either half of t are ORed into `outside`.
// Halves whose bits in `flag_mask` are clear are not flagged.
__device__ __forceinline__ uint32_t silu_lut_offset2(uint32_t pair, uint32_t& outside,
                                                     uint32_t flag_mask = 0xFFFFFFFFu) {
  const u16x2 h = __builtin_bit_cast(u16x2, pair);
  const u16x2 t = h - (u16x2)(uint16_t)(kSiluLutExp0 << 7);
  const uint32_t tb = __builtin_bit_cast(uint32_t, t);
  outside |= tb & flag_mask & 0x70007000u;
  const uint32_t lo = __builtin_bit_cast(uint32_t, (u16x2)(t << (uint16_t)1));
  const uint32_t sg = __builtin_bit_cast(uint32_t, (u16x2)(h >> (uint16_t)2));
  return (lo & 0x1FFF1FFFu) | (sg & 0xE000E000u);
}

// One radix-4 stage of the reference rotation on a quad (a, b, c, d) taken at
// stride s: s01=a+b, s23=c+d, d01=a-b, d23=c-d; a'=s01+d23, b'=s01-d23,
// c'=d01+s23, d'=s23-d01. Separate f32 adds, no contraction.
// kernels/prepare_integer_single.loom:109-116, src/quantized.rs:801-824.
__device__ __forceinline__ void radix4(float& a, float& b, float& c, float& d) {
  float s01 = a + b, s23 = c + d, d01 = a - b, d23 = c - d;
  a = s01 + d23;
  b = s01 - d23;
  c = d01 + s23;
  d = s23 - d01;
}

// Two consecutive stages on 16 values held by one lane: stride 1 over the low
// base-4 digit of the index, then stride 4 over the next digit.
__device__ __forceinline__ void radix4x2(float* v) {
#pragma unroll
  for (int q = 0; q < 4; ++q) radix4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
#pragma unroll
  for (int q = 0; q < 4; ++q) radix4(v[q], v[q + 4], v[q + 8], v[q + 12]);
}

// Between the writes and the reads of a 16x16 transpose that one 16-lane
// group makes in its own LDS rows. The group's lanes are in one wave, and the
// LDS executes one wave's operations in issue order, so its reads see its
// writes (and its later writes follow its reads) without a workgroup barrier;
// this only keeps the compiler from moving memory operations across it.
__device__ __forceinline__ void group_lds_order() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ uint32_t group_max16(uint32_t m) {
  // Reduce over the 16 lanes of a group (lanes differ in the low 4 bits): a
  // DPP row. quad_perm [1,0,3,2] and [2,3,0,1], then row_ror 4 and 8, leave
  // the row's maximum in every lane (every lane of the wave is active here).
  auto step = [](uint32_t v, uint32_t o) { return v > o ? v : o; };
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x124, 0xF, 0xF, false));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x128, 0xF, 0xF, false));
  return m;
}

template <int BITS>
__device__ __forceinline__ uint32_t pack_codes(const float* v, float inv, bool valid) {
  constexpr int per = 32 / BITS;
  constexpr float qmax = BITS == 8 ? 127.0f : 7.0f;
  constexpr uint32_t mask = BITS == 8 ? 0xffu : 0xfu;
  // Round to nearest even by adding 1.5 * 2^23: when valid, |v * inv| <= qmax
  // (times 1 + 2^-22), so the sum lies in [2^23, 2^24), where the f32 spacing is
  // 1 and the addend is even; the add then rounds exactly as rint does, and
  // the integer n sits two's complement in the low mantissa bits (the addend's
  // mantissa is 0x400000). Clamping the biased value to magic +- qmax is the
  // clamp of n.
  constexpr float magic = 12582912.0f;
  uint32_t word = 0;
#pragma unroll
  for (int p = 0; p < per; ++p) {
    float t = v[p] * inv + magic;
    t = __builtin_fminf(__builtin_fmaxf(t, magic - qmax), magic + qmax);
    word |= (as_uint(t) & mask) << (p * BITS);
  }
  return valid ? word : 0u;
}

// Eight int4 codes of one word (nibble p = code for k = 8q + p) -> two words of
// int8 bytes holding 16 * code: `lo` carries the even nibbles, `hi` the odd
// ones. Both GEMM operands use the same map, so their byte products are
// 256 * code_a * code_b and the i32 sum is 256 times the code dot product.
__device__ __forceinline__ void unpack16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  hi = w & 0xf0f0f0f0u;
  lo = (w << 4) & 0xf0f0f0f0u;
}

__device__ __forceinline__ v4i unpack_pair(uint32_t w0, uint32_t w1) {
  uint32_t a, b, c, d;
  unpack16(w0, a, b);
  unpack16(w1, c, d);
  v4i r;
  r.x = (int)a;
  r.y = (int)b;
  r.z = (int)c;
  r.w = (int)d;
  return r;
}

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

}  // namespace clef
