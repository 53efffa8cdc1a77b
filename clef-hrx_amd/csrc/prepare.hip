// Q1: Hadamard-rotated per-row quantizer, and Q2's retile permutation.
//
// Q1 follows kernels/prepare_integer_single.loom:65-286 (and the CPU test
// oracle at src/quantized.rs:801-824, 990-1004): per 256-column group a
// four-stage radix-4 rotation (strides 1, 4, 16, 64, exact op order), the row
// maximum of |v| with NaN counted as +inf, scale = (max(m/16, 1e-30)) / qmax,
// inv = (1/16) / scale, codes = clamp(roundeven(v * inv), -qmax, qmax), all
// codes 0 when the scale is not finite. Storage is the reference's single
// buffer: codes [rows][stride/(32/bits)] followed by rows f32 scales
// (src/quantized.rs:656-664).
//
// gfx950 mapping: 16 lanes own one 256-column group, 16 consecutive values per
// lane (one 32-byte load). Stages 1-2 run in-lane; a transpose through LDS
// gives each lane the 16 values that differ in the two high base-4 digits, and
// stages 3-4 run in-lane again. After the row maximum, a second LDS transpose
// returns natural order so each lane packs two (int4) or four (int8) whole
// words. A 256-thread workgroup holds 16 groups: 16/G rows of G groups when
// the row has G <= 16 groups, else one row over P passes kept in registers.
//
// A third output form (this library's, for the bf6 projection): the INT4
// codes written as e3m2 values, 6 bits each, value c of a row at bits 6c of
// its width * 3/4 bytes, with the same f32 row scales after the rows.
#include "common.hpp"
#include "silu_table.hpp"
#include "kernels.hpp"
#include "group.hpp"
#include "route.hpp"

namespace clef {

namespace {

constexpr int kPitch = 20;            // floats per 16-value LDS row (80 bytes)
constexpr int kGroupLds = 16 * kPitch; // LDS floats per 256-column group

struct PlainSource {
  static constexpr bool kRowNorm = false;
  static constexpr bool kLdsTable = false;
  const uint16_t* x;
  struct Raw {
    u4 a, b;
  };
  __device__ __forceinline__ Raw fetch(int64_t rowoff, int col) const {
    // each input value is read once: non-temporal loads
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* p = reinterpret_cast<const u32x4*>(x + rowoff + col);
    const u32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
    return Raw{u4{a.x, a.y, a.z, a.w}, u4{b.x, b.y, b.z, b.w}};
  }
  __device__ __forceinline__ void convert(const Raw& r, float* v) const {
    uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = bf16_lo(w[i]);
      v[2 * i + 1] = bf16_hi(w[i]);
    }
  }
  __device__ __forceinline__ void load16(int64_t rowoff, int col, float* v) const {
    convert(fetch(rowoff, col), v);
  }
};

// S1 applied on load (kernels/prepare_integer_register.loom:155-172): the
// rotation sees f32(bf16(swiglu)) exactly as if h had been materialized.
struct SwigluSource {
  static constexpr bool kRowNorm = false;
  // prepare_kernel copies the SiLU table into LDS for convert_with.
  static constexpr bool kLdsTable = true;
  const uint16_t* gate;
  const uint16_t* up;
  struct Raw {
    u4 ga, gb, ua, ub;
  };
  __device__ __forceinline__ Raw fetch(int64_t rowoff, int col) const {
    const u4* pg = reinterpret_cast<const u4*>(gate + rowoff + col);
    const u4* pu = reinterpret_cast<const u4*>(up + rowoff + col);
    return Raw{pg[0], pg[1], pu[0], pu[1]};
  }
  __device__ __forceinline__ void convert(const Raw& r, float* v) const { convert_with(r, v, g_silu_lut); }
  __device__ __forceinline__ void convert_with(const Raw& r, float* v, const uint16_t* table) const {
    const uint32_t gw[8] = {r.ga.x, r.ga.y, r.ga.z, r.ga.w, r.gb.x, r.gb.y, r.gb.z, r.gb.w};
    const uint32_t uw[8] = {r.ua.x, r.ua.y, r.ua.z, r.ua.w, r.ub.x, r.ub.y, r.ub.z, r.ub.w};
    float g[16], act[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      g[2 * i] = bf16_lo(gw[i]);
      g[2 * i + 1] = bf16_hi(gw[i]);
    }
    silu_lut<16>(g, act, table);  // = silu_bf16(g), from the table where it covers g
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = bf16_round(act[2 * i] * bf16_lo(uw[i]));
      v[2 * i + 1] = bf16_round(act[2 * i + 1] * bf16_hi(uw[i]));
    }
  }
  __device__ __forceinline__ void load16(int64_t rowoff, int col, float* v) const {
    convert(fetch(rowoff, col), v);
  }
};

// Attention output times its sigmoid gate, applied on load
// (kernels/prepare_integer_register.loom:137-155): the gate of column c is
// column (c/256)*512 + 256 + c%256 of the [rows][2*width] q_gate row, and the
// value is bf16(x * bf16(1 / (1 + exp(-g)))).
struct AttentionGateSource {
  static constexpr bool kRowNorm = false;
  static constexpr bool kLdsTable = false;
  const uint16_t* x;
  const uint16_t* q_gate;
  struct Raw {
    u4 xa, xb, ga, gb;
  };
  __device__ __forceinline__ Raw fetch(int64_t rowoff, int col) const {
    const u4* px = reinterpret_cast<const u4*>(x + rowoff + col);
    const int gcol = (col >> 8) * 512 + 256 + (col & 255);  // 16 values stay inside one 256-column half
    const u4* pg = reinterpret_cast<const u4*>(q_gate + 2 * rowoff + gcol);  // rows of 2 * width
    return Raw{px[0], px[1], pg[0], pg[1]};
  }
  __device__ __forceinline__ static float gated(float x, float g) {
    const float sig = bf16_round(1.0f / (1.0f + cephes_expf(-g)));
    return bf16_round(x * sig);
  }
  __device__ __forceinline__ void convert(const Raw& r, float* v) const {
    uint32_t a[8] = {r.xa.x, r.xa.y, r.xa.z, r.xa.w, r.xb.x, r.xb.y, r.xb.z, r.xb.w};
    uint32_t g[8] = {r.ga.x, r.ga.y, r.ga.z, r.ga.w, r.gb.x, r.gb.y, r.gb.z, r.gb.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = gated(bf16_lo(a[i]), bf16_lo(g[i]));
      v[2 * i + 1] = gated(bf16_hi(a[i]), bf16_hi(g[i]));
    }
  }
  __device__ __forceinline__ void load16(int64_t rowoff, int col, float* v) const {
    convert(fetch(rowoff, col), v);
  }
};

// Named RMSNorm applied to a whole row before the rotation
// (kernels/prepare_integer_register.loom:63-80, 112-134; weight offset 1,
// eps 1e-6): inv = 1 / sqrt(ss / width + 1e-6) with ss summed in a fixed
// order (per thread fma over its own values, group p then value i; a
// butterfly over the wave's lanes at offsets 32..1; the four wave sums in wave
// order), then r = fma(x * inv, w + 1, 0) rounded to bf16; the bf16 rows are
// optionally stored to `normalized`. Used by the one-row-per-workgroup kernel.
struct NormSource {
  static constexpr bool kRowNorm = true;
  static constexpr bool kLdsTable = false;
  const uint16_t* x;
  const uint16_t* weight;
  uint16_t* normalized;  // nullable
  using Raw = PlainSource::Raw;
  __device__ __forceinline__ Raw fetch(int64_t rowoff, int col) const { return PlainSource{x}.fetch(rowoff, col); }
  __device__ __forceinline__ void convert(const Raw& r, float* v) const { PlainSource{x}.convert(r, v); }
  __device__ __forceinline__ void load16(int64_t rowoff, int col, float* v) const {
    convert(fetch(rowoff, col), v);
  }
  template <int P>
  __device__ __forceinline__ void normalize(float (&v)[P][16], int64_t row, int width, int grp0, int L,
                                            bool active, float* red) const {
    const int G = width >> 8;
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (active && grp0 + 16 * p < G)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc = __builtin_fmaf(v[p][i], v[p][i], acc);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float ss = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = 1.0f / __builtin_sqrtf(ss / (float)width + 1e-6f);
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int grp = grp0 + 16 * p;
      if (!(active && grp < G)) continue;
      const int col = grp * 256 + 16 * L;
      const u4* pw = reinterpret_cast<const u4*>(weight + col);
      const u4 wa = pw[0], wb = pw[1];
      const uint32_t ww[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
      uint32_t hb[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float r0 = __builtin_fmaf(v[p][2 * i] * inv, bf16_lo(ww[i]) + 1.0f, 0.0f);
        const float r1 = __builtin_fmaf(v[p][2 * i + 1] * inv, bf16_hi(ww[i]) + 1.0f, 0.0f);
        hb[i] = pack_bf16x2(r0, r1);
        v[p][2 * i] = bf16_lo(hb[i]);
        v[p][2 * i + 1] = bf16_hi(hb[i]);
      }
      if (normalized) {
        u4* dst = reinterpret_cast<u4*>(normalized + row * width + col);
        dst[0] = u4{hb[0], hb[1], hb[2], hb[3]};
        dst[1] = u4{hb[4], hb[5], hb[6], hb[7]};
      }
    }
  }
};

// The 16 codes clamp(rint(v * inv), -7, 7) of one lane as e3m2 (exact for
// these integers), value i at bits 6i of o[0..2]: the bf6 form of the INT4
// codes, for the bf6 projection.
__device__ __forceinline__ void pack_codes_f6(const float* v, float inv, bool valid, uint32_t (&o)[3]) {
  constexpr float magic = 12582912.0f;  // as in pack_codes
  o[0] = o[1] = o[2] = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    // r = the code as an exact f32 (the biased sum minus the bias). For
    // 1 <= |r| <= 7 its bits 21..30 are (exponent << 2) | top two mantissa
    // bits, exponent 127..129, so that field minus (127 - 3) << 2 is the e3m2
    // magnitude (bias 3); the saturating subtraction gives 0 for r = +0, and
    // the f32 sign bit moves to bit 5. Equal to e3m2_of_nibble of the code.
    float t = v[i] * inv + magic;
    t = __builtin_fminf(__builtin_fmaxf(t, magic - 7.0f), magic + 7.0f);
    const uint32_t b = as_uint(t - magic);
    const uint32_t field = (b >> 21) & 0x3ffu;
    const uint32_t e = (field > 496u ? field - 496u : 0u) | ((b >> 26) & 0x20u);
    const int bit = 6 * i, d = bit >> 5, sh = bit & 31;
    o[d] |= e << sh;
    if (sh > 26) o[d + 1] |= e >> (32 - sh);
  }
  if (!valid) o[0] = o[1] = o[2] = 0;
}

// Codes of the 16 values at column col of a row whose output starts at
// row_out: BITS 4 and 8 pack two's complement fields (32 / BITS per word).
template <int BITS>
__device__ __forceinline__ void store_codes(uint32_t* row_out, int col, const float* nat, float inv, bool valid) {
  if constexpr (BITS == 4) {
    *reinterpret_cast<uint2*>(row_out + col / 8) =
        make_uint2(pack_codes<4>(nat, inv, valid), pack_codes<4>(nat + 8, inv, valid));
  } else if constexpr (BITS == 8) {
    *reinterpret_cast<uint4*>(row_out + col / 4) =
        make_uint4(pack_codes<8>(nat, inv, valid), pack_codes<8>(nat + 4, inv, valid),
                   pack_codes<8>(nat + 8, inv, valid), pack_codes<8>(nat + 12, inv, valid));
  } else {
    static_assert(BITS == 8, "codes of 4 or 8 bits (bf6: store_codes_f6)");
  }
}

// bf6 codes of the 16 values at column col of row `row`: 12 bytes in the
// tiled bf6 activation layout (f6_offset).
__device__ __forceinline__ void store_codes_f6(uint32_t* out, int64_t row, int col, int width, const float* nat,
                                               float inv, bool valid) {
  uint32_t o[3];
  pack_codes_f6(nat, inv, valid, o);
  uint32_t* dst = out + f6_offset(row, col, width) / 4;
  dst[0] = o[0];
  dst[1] = o[1];
  dst[2] = o[2];
}

// Codes of one 16-value group, in the output layout of BITS (out_row: the
// row's first word for BITS 4 and 8; out: the whole buffer for bf6).
template <int BITS>
__device__ __forceinline__ void store_group(uint32_t* out, uint32_t* out_row, int64_t row, int col, int width,
                                            const float* nat, float inv, bool valid) {
  if constexpr (BITS == 6)
    store_codes_f6(out, row, col, width, nat, inv, valid);
  else
    store_codes<BITS>(out_row, col, nat, inv, valid);
}

// Where a prepared buffer's f32 row scales start.
template <int BITS>
__device__ __forceinline__ float* scales_of(uint32_t* out, int64_t rows, int width, int out_words) {
  if constexpr (BITS == 6) return reinterpret_cast<float*>(reinterpret_cast<char*>(out) + f6_codes_bytes(rows, width));
  return reinterpret_cast<float*>(out + rows * out_words);
}

template <int P, int BITS, class Src>
__global__ __launch_bounds__(256) void prepare_kernel(Src src, int64_t rows, int width,
                                                      int out_words, uint32_t* __restrict__ out) {
  __shared__ __align__(16) float lds[16 * kGroupLds];
  __shared__ uint32_t gmax[16];
  const int tid = threadIdx.x;
  const int lg = tid >> 4;
  const int L = tid & 15;
  const int G = width >> 8;
  int rows_per_block, row_local, grp0;
  if (P == 1) {
    rows_per_block = 16 / G;
    row_local = lg / G;
    grp0 = lg - row_local * G;
  } else {
    rows_per_block = 1;
    row_local = 0;
    grp0 = lg;
  }
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + row_local;
  const bool active = row_local < rows_per_block && row < rows;
  float* buf = lds + lg * kGroupLds;

  float v[P][16];
  if constexpr (Src::kLdsTable) {
    // The SiLU table (16 KiB) goes into the transpose buffer, which is idle
    // until the values are converted: LDS reads instead of one global gather
    // per value. Its loads go out with the inputs'.
    static_assert(kSiluLutSize * 2 <= 16 * kGroupLds * 4 && kSiluLutSize * 2 == 256 * 4 * 16, "table copy");
    u4 t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = reinterpret_cast<const u4*>(g_silu_lut)[tid + 256 * i];
    typename Src::Raw raw[P];
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (active && grp0 + 16 * p < G) raw[p] = src.fetch(row * width, (grp0 + 16 * p) * 256 + 16 * L);
    uint16_t* table = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<u4*>(table)[tid + 256 * i] = t[i];
    __syncthreads();
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (active && grp0 + 16 * p < G) {
        src.convert_with(raw[p], v[p], table);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[p][i] = 0.0f;
      }
    }
    __syncthreads();  // the table's LDS becomes the transpose buffer
  } else {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int grp = grp0 + 16 * p;
      if (active && grp < G) {
        src.load16(row * width, grp * 256 + 16 * L, v[p]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[p][i] = 0.0f;
      }
    }
  }
  if constexpr (Src::kRowNorm) {
    static_assert(P > 1, "row normalization needs one row per workgroup");
    src.template normalize<P>(v, row, width, grp0, L, active, reinterpret_cast<float*>(gmax));
    __syncthreads();  // gmax is reused for the row maximum below
  }
  uint32_t mbits = 0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int grp = grp0 + 16 * p;
    const bool on = active && grp < G;
    radix4x2(v[p]);  // strides 1 and 4
    float4* wrow = reinterpret_cast<float4*>(buf + L * kPitch);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      wrow[c] = make_float4(v[p][4 * c], v[p][4 * c + 1], v[p][4 * c + 2], v[p][4 * c + 3]);
    group_lds_order();
#pragma unroll
    for (int k = 0; k < 16; ++k) v[p][k] = buf[k * kPitch + L];
    group_lds_order();
    radix4x2(v[p]);  // strides 16 and 64 (value k holds index L + 16k)
    if (on) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        uint32_t a = as_uint(v[p][k]) & 0x7fffffffu;
        mbits = mbits > a ? mbits : a;
      }
    }
  }
  mbits = group_max16(mbits);
  if (L == 0) gmax[lg] = mbits;
  __syncthreads();
  uint32_t m = 0;
  if (P == 1) {
    for (int g = 0; g < G; ++g) {
      uint32_t o = gmax[(row_local < rows_per_block ? row_local : 0) * G + g];
      m = m > o ? m : o;
    }
  } else {
#pragma unroll
    for (int g = 0; g < 16; ++g) m = m > gmax[g] ? m : gmax[g];
  }
  // |v| < inf ? |v| : inf with NaN -> inf: any pattern >= +inf's is +inf.
  const float mf = m >= 0x7f800000u ? __builtin_huge_valf() : as_float(m);
  constexpr float qmax = BITS == 8 ? 127.0f : 7.0f;
  const float normal = mf * 0.0625f;
  const float safe = __builtin_fmaxf(normal, 1e-30f);
  const float scale = safe / qmax;
  const bool valid = scale < __builtin_huge_valf();
  const float inv = 0.0625f / scale;

#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int grp = grp0 + 16 * p;
    const bool on = active && grp < G;
#pragma unroll
    for (int k = 0; k < 16; ++k) buf[k * kPitch + L] = v[p][k];
    group_lds_order();
    float nat[16];
    const float4* rrow = reinterpret_cast<const float4*>(buf + L * kPitch);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float4 t = rrow[c];
      nat[4 * c] = t.x;
      nat[4 * c + 1] = t.y;
      nat[4 * c + 2] = t.z;
      nat[4 * c + 3] = t.w;
    }
    group_lds_order();
    if (on) store_group<BITS>(out, out + row * out_words, row, grp * 256 + 16 * L, width, nat, inv, valid);
  }
  if (active && grp0 == 0 && L == 0) scales_of<BITS>(out, rows, width, out_words)[row] = scale;
}

// Rows of G <= 16 groups, as prepare_kernel<1> but persistent: a workgroup
// walks row blocks (16 / G rows each) with a grid stride and fetches the next
// block's inputs before rotating and packing the current one, so HBM latency
// overlaps the work instead of being paid once per workgroup.
// The body runs as workgroup `block` of `nblocks` walking the row blocks.
template <int BITS, class Src>
__device__ __forceinline__ void prepare_loop_body(Src src, int64_t rows, int width, int out_words,
                                                  uint32_t* __restrict__ out, int64_t block, int64_t nblocks) {
  // 20 KiB: eight workgroups fill a CU's LDS. Each group's maximum goes to
  // the padding float of its first LDS row, which the transposes never touch.
  __shared__ __align__(16) float lds[16 * kGroupLds];
  uint32_t* gmax = reinterpret_cast<uint32_t*>(lds) + 16;
  const int tid = threadIdx.x;
  const int lg = tid >> 4;
  const int L = tid & 15;
  const int G = width >> 8;
  const int rows_per_block = 16 / G;
  const int row_local = lg / G;
  const int grp = lg - row_local * G;
  const bool lane_on = row_local < rows_per_block;
  const int64_t nblk = (rows + rows_per_block - 1) / rows_per_block;
  float* buf = lds + lg * kGroupLds;
  constexpr float qmax = BITS == 8 ? 127.0f : 7.0f;

  // The row and its input and output offsets advance by one grid stride per
  // block (additions, not the quarter-rate 64-bit multiplies per iteration).
  const int col = grp * 256 + 16 * L;
  const int64_t step = nblocks * rows_per_block;
  const int64_t in_step = step * width, out_step = step * out_words;
  int64_t blk = block;
  int64_t row = blk * rows_per_block + row_local;
  int64_t in_off = row * width, out_off = row * out_words;
  typename Src::Raw raw{};
  if (lane_on && row < rows) raw = src.fetch(in_off, col);
  for (; blk < nblk; blk += nblocks, row += step, in_off += in_step, out_off += out_step) {
    const bool on = lane_on && row < rows;
    float v[16];
    if (on) {
      src.convert(raw, v);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = 0.0f;
    }
    if (lane_on && row + step < rows) raw = src.fetch(in_off + in_step, col);
    radix4x2(v);  // strides 1 and 4
    float4* wrow = reinterpret_cast<float4*>(buf + L * kPitch);
#pragma unroll
    for (int c = 0; c < 4; ++c) wrow[c] = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
    group_lds_order();
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = buf[k * kPitch + L];
    group_lds_order();
    radix4x2(v);  // strides 16 and 64 (value k holds index L + 16k)
    uint32_t mbits = 0;
    if (on) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        uint32_t a = as_uint(v[k]) & 0x7fffffffu;
        mbits = mbits > a ? mbits : a;
      }
    }
    mbits = group_max16(mbits);
    if (L == 0) gmax[lg * kGroupLds] = mbits;
    __syncthreads();
    // Row r's scale and 1/16-scale by thread r of wave 0 (the other waves
    // skip the divisions), kept in floats 17 and 18 of group r's first LDS
    // row (padding the transposes never touch) and read after the next
    // barrier.
    if (threadIdx.x < rows_per_block) {
      const int r = threadIdx.x;
      uint32_t m = 0;
      for (int g = 0; g < G; ++g) {
        const uint32_t o = gmax[(r * G + g) * kGroupLds];
        m = m > o ? m : o;
      }
      const float mf = m >= 0x7f800000u ? __builtin_huge_valf() : as_float(m);
      const float normal = mf * 0.0625f;
      const float safe = __builtin_fmaxf(normal, 1e-30f);
      const float sc = safe / qmax;
      lds[r * kGroupLds + 17] = sc;
      lds[r * kGroupLds + 18] = 0.0625f / sc;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) buf[k * kPitch + L] = v[k];
    __syncthreads();
    const int srow = lane_on ? row_local : 0;
    const float scale = lds[srow * kGroupLds + 17];
    const float inv = lds[srow * kGroupLds + 18];
    const bool valid = scale < __builtin_huge_valf();
    float nat[16];
    const float4* rrow = reinterpret_cast<const float4*>(buf + L * kPitch);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float4 t = rrow[c];
      nat[4 * c] = t.x;
      nat[4 * c + 1] = t.y;
      nat[4 * c + 2] = t.z;
      nat[4 * c + 3] = t.w;
    }
    // The next iteration's first LDS writes (this group's rows, then gmax
    // after every wave has passed the barriers below) need no barrier here:
    // the scale slots are rewritten only after the next gmax barrier, which
    // every wave reaches after reading this iteration's scale.
    group_lds_order();
    if (on) {
      store_group<BITS>(out, out + out_off, row, col, width, nat, inv, valid);
      if (grp == 0 && L == 0) scales_of<BITS>(out, rows, width, out_words)[row] = scale;
    }
  }
}

template <int BITS, class Src>
__global__ __launch_bounds__(256) void prepare_loop_kernel(Src src, int64_t rows, int width, int out_words,
                                                           uint32_t* __restrict__ out) {
  prepare_loop_body<BITS, Src>(src, rows, width, out_words, out, blockIdx.x, gridDim.x);
}

// The router and the INT4 quantizer of the MoE input in one launch: the first
// route_blocks workgroups route the tokens (16 or 4 per workgroup), the others run the
// grid-stride quantizer. Neither needs the other's output, so they share the
// GPU instead of running one after the other.
// With `groups` non-NULL (at most 16 tokens at top-8: one routing
// workgroup) that workgroup also groups the routes it wrote (group_small).
// With `counts16` non-NULL (top-8) routing workgroup b also writes
// counts16[b][e], the number of its 16 tokens routed to expert e, for
// group_scatter_scan_kernel.
__global__ __launch_bounds__(256) void route_prepare_kernel(const void* __restrict__ logits, int dtype,
                                                            int64_t tokens, int experts, int topk,
                                                            float* __restrict__ routes, int64_t route_blocks,
                                                            PlainSource src, int width, int out_words,
                                                            uint32_t* __restrict__ out, float* groups, float* order,
                                                            int32_t* schedule, int bm, int* counts16) {
  if ((int64_t)blockIdx.x < route_blocks) {
    if (groups != nullptr) {  // topk 8, one routing workgroup: route_body16
      __shared__ int ids[128];
      route_impl::route_body16(logits, dtype, tokens, experts, topk, routes, 0, ids);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // ids written; the route stores may drain
      group_small(ids, (int)tokens, groups, order, schedule, bm);
      return;
    }
    if (counts16 != nullptr) {  // topk 8: the block's expert counts from its ids
      __shared__ int ids[128];
      __shared__ uint32_t masks16[128];  // bit i: token i of the block names the expert
      const int tid = threadIdx.x;
      if (tid < 128) masks16[tid] = 0u;
      route_impl::route_body16(logits, dtype, tokens, experts, topk, routes, blockIdx.x, ids);
      __syncthreads();
      const int64_t left = tokens - (int64_t)blockIdx.x * route_impl::kRouteTokens16;
      const int n = 8 * (int)(left < route_impl::kRouteTokens16 ? left : route_impl::kRouteTokens16);
      if (tid < n) {
        const int e = ids[tid];
        if (e >= 0 && e < 128) atomicOr(&masks16[e], 1u << (tid >> 3));
      }
      __syncthreads();
      if (tid < 128) counts16[(int64_t)blockIdx.x * 128 + tid] = __popc(masks16[tid]);
      return;
    }
    route_impl::route_block(logits, dtype, tokens, experts, topk, routes, blockIdx.x);
    return;
  }
  prepare_loop_body<4, PlainSource>(src, tokens, width, out_words, out, blockIdx.x - route_blocks,
                                    gridDim.x - route_blocks);
}

template <int BITS, class Src>
hipError_t launch_prepare_bits(const Src& src, int64_t rows, int width, int out_words,
                               uint32_t* out, hipStream_t stream) {
  const int G = width / 256;
  if (G <= 16 && !Src::kRowNorm) {
    const int per_block = 16 / G;
    const int64_t blocks = (rows + per_block - 1) / per_block;
    // Up to 8 resident workgroups per CU on 256 CUs; more row blocks than
    // that are walked by the grid stride.
    const unsigned grid = (unsigned)(blocks < 2048 ? blocks : 2048);
    if constexpr (!Src::kRowNorm)
      prepare_loop_kernel<BITS, Src><<<grid, 256, 0, stream>>>(src, rows, width, out_words, out);
  } else {
    const int passes = (G + 15) / 16;
    const unsigned grid = (unsigned)rows;
    switch (passes) {
#define CLEF_PREP_CASE(N) \
  case N: prepare_kernel<N, BITS, Src><<<grid, 256, 0, stream>>>(src, rows, width, out_words, out); break;
      CLEF_PREP_CASE(2)
      CLEF_PREP_CASE(3)
      CLEF_PREP_CASE(4)
      CLEF_PREP_CASE(5)
      CLEF_PREP_CASE(6)
      CLEF_PREP_CASE(7)
      CLEF_PREP_CASE(8)
#undef CLEF_PREP_CASE
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

// bits 4 or 8: packed codes of `stride` columns per row; bits 6: the tiled
// bf6 activation layout (f6_offset; stride == width).
template <class Src>
hipError_t launch_prepare_src(const Src& src, int64_t rows, int width, int stride, int bits,
                              uint32_t* out, hipStream_t stream) {
  if (bits == 6) return launch_prepare_bits<6>(src, rows, width, width * 3 / 16, out, stream);
  const int out_words = stride / (32 / bits);
  if (bits == 4) return launch_prepare_bits<4>(src, rows, width, out_words, out, stream);
  return launch_prepare_bits<8>(src, rows, width, out_words, out, stream);
}

// Q2 retile: word (n, q) of the row-major codes lands at
// ((n / 128) * blocks_k + q / 32) * 4096 + (n % 128) * 32 + q % 32.
// kernels/retile_codes.loom:2-5, 38-55. One thread moves 16 bytes; a
// workgroup writes one contiguous 16 KiB output block.
__global__ __launch_bounds__(256) void retile_kernel(const uint32_t* __restrict__ codes, int64_t rows,
                                                     int in_words, int blocks_k,
                                                     uint32_t* __restrict__ tiled) {
  const int64_t block = blockIdx.x;  // (n / 128) * blocks_k + q / 32
  const int64_t nb = block / blocks_k;
  const int kb = (int)(block - nb * blocks_k);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = threadIdx.x + 256 * j;  // 16-byte chunk within the block
    const int r = idx >> 3, c = idx & 7;
    const int64_t n = nb * 128 + r;
    const uint32_t* src = codes + n * in_words + kb * 32 + c * 4;
    uint4 w;
    if ((in_words & 3) == 0) {
      w = *reinterpret_cast<const uint4*>(src);
    } else {
      w = make_uint4(src[0], src[1], src[2], src[3]);
    }
    *reinterpret_cast<uint4*>(tiled + block * 4096 + idx * 4) = w;
  }
}

// Checkpoint tiling [rows/256][cols/64][256][64] <-> row-major [rows][cols]
// (src/checkpoint.rs:24-32, 63-106). Threads walk the tiled order in 16-byte
// chunks (8 bf16): element (tile, ks, r, c) is dense (tile*256 + r)*cols +
// ks*64 + c and tiled tile*256*cols + (ks*256 + r)*64 + c.
__global__ __launch_bounds__(256) void tile_permute_kernel(const uint16_t* __restrict__ src,
                                                           int64_t chunks, int cols, bool to_tiled,
                                                           uint16_t* __restrict__ dst) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const int c = (int)(q & 7) * 8;
  const int64_t rest = q >> 3;
  const int r = (int)(rest & 255);
  const int64_t rest2 = rest >> 8;
  const int ksteps = cols / 64;
  const int64_t tile = rest2 / ksteps;
  const int ks = (int)(rest2 - tile * ksteps);
  const int64_t dense = (tile * 256 + r) * cols + ks * 64 + c;
  const int64_t tiled = q * 8;
  if (to_tiled)
    *reinterpret_cast<uint4*>(dst + tiled) = *reinterpret_cast<const uint4*>(src + dense);
  else
    *reinterpret_cast<uint4*>(dst + dense) = *reinterpret_cast<const uint4*>(src + tiled);
}

}  // namespace

hipError_t launch_prepare(const uint16_t* x, int64_t rows, int width, int stride, int bits,
                          uint32_t* out, hipStream_t stream) {
  return launch_prepare_src(PlainSource{x}, rows, width, stride, bits, out, stream);
}

bool route_prepare_fusable(int width) { return width % 256 == 0 && width / 256 <= 16; }

bool route_group_fusable(int64_t tokens, int topk) { return topk == 8 && tokens >= 1 && tokens <= 16; }

hipError_t launch_route_prepare(const void* logits, int dtype, int64_t tokens, int experts, int topk,
                                float* routes, const uint16_t* x, int width, int stride, uint32_t* out,
                                hipStream_t stream, float* groups, float* order, int32_t* schedule, int bm,
                                int* counts16) {
  if (!route_prepare_fusable(width)) return hipErrorInvalidValue;
  if (groups != nullptr && !route_group_fusable(tokens, topk)) return hipErrorInvalidValue;
  if (counts16 != nullptr && (groups != nullptr || topk != 8)) return hipErrorInvalidValue;
  const int per_block = 16 / (width / 256);
  const int64_t blocks = (tokens + per_block - 1) / per_block;
  const int64_t prep = blocks < 2048 ? blocks : 2048;
  const int per = route_impl::route_tokens_per_block(topk);
  const int64_t route_blocks = (tokens + per - 1) / per;
  route_prepare_kernel<<<(unsigned)(route_blocks + prep), 256, 0, stream>>>(
      logits, dtype, tokens, experts, topk, routes, route_blocks, PlainSource{x}, width, stride / 8, out, groups, order,
      schedule, bm, counts16);
  return hipGetLastError();
}

hipError_t launch_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows, int width,
                                 int stride, int bits, uint32_t* out, hipStream_t stream) {
  return launch_prepare_src(SwigluSource{gate, up}, rows, width, stride, bits, out, stream);
}

hipError_t launch_prepare_attention_gate(const uint16_t* x, const uint16_t* q_gate, int64_t rows, int width,
                                         int stride, int bits, uint32_t* out, hipStream_t stream) {
  return launch_prepare_src(AttentionGateSource{x, q_gate}, rows, width, stride, bits, out, stream);
}

hipError_t launch_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int width, int stride,
                               int bits, uint32_t* out, uint16_t* normalized, hipStream_t stream) {
  if (width / 256 <= 16) return hipErrorInvalidValue;
  return launch_prepare_src(NormSource{x, weight, normalized}, rows, width, stride, bits, out, stream);
}

hipError_t launch_retile(const uint32_t* codes, int64_t rows, int in_words, int words,
                         uint32_t* tiled, hipStream_t stream) {
  const int blocks_k = words / 32;
  const int64_t blocks = (rows / 128) * blocks_k;
  retile_kernel<<<(unsigned)blocks, 256, 0, stream>>>(codes, rows, in_words, blocks_k, tiled);
  return hipGetLastError();
}

hipError_t launch_tile_permute(const uint16_t* src, int64_t rows, int cols, uint16_t* dst,
                               bool to_tiled, hipStream_t stream) {
  const int64_t chunks = rows * cols / 8;
  const int64_t blocks = (chunks + 255) / 256;
  tile_permute_kernel<<<(unsigned)blocks, 256, 0, stream>>>(src, chunks, cols, to_tiled, dst);
  return hipGetLastError();
}

}  // namespace clef
