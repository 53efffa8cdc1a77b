// G1 on bf6 operands for gfx950: the INT4 x INT4 projection of
// kernels/gemm_integer.loom:394-433 with both operands re-encoded, once, as
// 6-bit floats and multiplied by v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Exactness. bf6 is e3m2 (sign, 3 exponent bits with bias 3, 2 mantissa
// bits); every integer -8..7 is an e3m2 value (0, 1, 2, 3 = 1.5*2, 4, 5 =
// 1.25*4, 6 = 1.5*4, 7 = 1.75*4, 8 = 2^3), so each product of two codes is
// exact and the MFMA's f32 sum of them is the exact integer dot product as
// long as it stays below 2^24 (|dot| <= 64 K: K < 2^18). With the unit block
// scale (e8m0 127) the instruction computes exactly sum a * w. The G1
// epilogue then runs on f32(dot) itself, bit-identical to the INT4 path.
//
// Why: on gfx950 this MFMA takes 64 k per 32x32 tile in about the time the
// int8 MFMA takes 32 k (measured 35 against 32 cycles), and the operands
// need no unpacking: LDS holds them in the form the MFMA reads.
//
// Formats (this library's own; produced from the reference's packed
// activation and tiled weight by clef_i4_f6_activation / clef_i4_f6_weight):
//  * bf6 row: value k at bits 6k .. 6k+5 of the row, little-endian; K * 3/4
//    bytes per row (K % 128 == 0).
//  * bf6 activation: blocks of 128 rows x 128 k (96 bytes per row, 12 KiB)
//    at ((m / 128) * (K / 128) + k / 128) * 12288, row r of a block at
//    r * 96 (f6_offset); rows past M in the last block are padding. A
//    k-step's 256 rows are then two contiguous 12 KiB blocks: each 1 KiB DMA
//    instruction reads 8 whole 128-byte lines, where 96-byte pieces of
//    3072-byte rows would touch 1.5 lines each (3.7 % faster at M4096 K4096
//    N12288).
//  * bf6 tiled weight: the same blocks over n, with the 16-byte chunk c of
//    block row r stored at chunk c ^ ((r >> 3) & 1) (the LDS swizzle,
//    applied on the global side; the activation's is applied by the DMA's
//    per-lane offsets).
//
// Tile: 256 x 256 outputs per workgroup of 8 waves (2 x 4 waves of 128 rows x
// 64 columns), k-steps of 128 k (48 KiB of LDS per stage, three stages), a
// persistent grid walking tiles on the workgroup's XCD; while a k-step
// computes, the DMAs of the next two (running into the next tile's first)
// fill the other stages. Lane half h of a 32-row fragment reads bytes 48h .. 48h+47 of
// the row's 96 (k = 64h .. 64h+63): the first 24 are the operand of the
// k-step's first MFMA, the last 24 of its second; A and B use the same map,
// so the two MFMAs of a k-step together cover its 128 k exactly once.

#include <type_traits>

#include "common.hpp"
#include "gemm_dma.hpp"
#include "kernels.hpp"
#include "launch.hpp"
#include "silu_table.hpp"

namespace clef {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned f6_v2u __attribute__((ext_vector_type(2)));
typedef unsigned f6_v4u __attribute__((ext_vector_type(4)));

// 32 codes (four packed words, code j in nibble j % 8 of word j / 8) -> 32
// e3m2 values, value j at bits 6j of out[0..5].
__device__ __forceinline__ void f6_pack32(const uint32_t (&w)[4], uint32_t (&out)[6]) {
#pragma unroll
  for (int d = 0; d < 6; ++d) out[d] = 0;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const uint32_t v = e3m2_of_nibble((w[j >> 3] >> (4 * (j & 7))) & 15u);
    const int bit = 6 * j, d = bit >> 5, sh = bit & 31;
    out[d] |= v << sh;
    if (sh > 26) out[d + 1] |= v >> (32 - sh);
  }
}

// Packed activation (k_stride words per row) -> the bf6 activation layout
// (f6_offset); one thread per 32 codes.
__global__ __launch_bounds__(256) void f6_rows_kernel(const uint32_t* __restrict__ a, int a_words, int64_t rows,
                                                      int k, uint8_t* __restrict__ out) {
  const int groups = k / 32;
  const int64_t total = rows * groups;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / groups;
    const int g = (int)(t - r * groups);
    const uint4 in = *reinterpret_cast<const uint4*>(a + r * a_words + 4 * g);
    const uint32_t w[4] = {in.x, in.y, in.z, in.w};
    uint32_t o[6];
    f6_pack32(w, o);
    f6_v2u* dst = reinterpret_cast<f6_v2u*>(out + f6_offset(r, 32 * g, k));
    dst[0] = f6_v2u{o[0], o[1]};
    dst[1] = f6_v2u{o[2], o[3]};
    dst[2] = f6_v2u{o[4], o[5]};
  }
}

// Tiled INT4 weight (the reference layout: 128-row x 256-k blocks of 32 words
// per row) -> bf6 tiled weight (header comment); one thread per 32 codes.
__global__ __launch_bounds__(256) void f6_tiled_kernel(const uint32_t* __restrict__ w, int64_t n, int k,
                                                       uint8_t* __restrict__ out) {
  const int groups = k / 32;
  const int kb4 = k / 256, kb6 = k / 128;
  const int64_t total = n * groups;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = t / groups;
    const int g = (int)(t - row * groups);
    const int64_t panel = row / 128;
    const int r = (int)(row % 128);
    const int q = 4 * g;  // first word of the group in the row
    const uint4 in = *reinterpret_cast<const uint4*>(w + (panel * kb4 + q / 32) * 4096 + r * 32 + q % 32);
    const uint32_t wv[4] = {in.x, in.y, in.z, in.w};
    uint32_t o[6];
    f6_pack32(wv, o);
    uint8_t* blk = out + (panel * kb6 + g / 4) * 12288 + r * 96;
    const int s = (r >> 3) & 1;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const int off = 24 * (g % 4) + 8 * p;  // logical byte offset in the 96-byte row
      *reinterpret_cast<f6_v2u*>(blk + ((((off >> 4) ^ s)) << 4) + (off & 15)) = f6_v2u{o[2 * p], o[2 * p + 1]};
    }
  }
}

// Tile shape of the bf6 GEMM.
struct F6Tile {
  static constexpr int WM = 128, WN = 64, WAVES_M = 2, WAVES_N = 4;
  static constexpr int NW = WAVES_M * WAVES_N, THREADS = 64 * NW;
  static constexpr int BM = WM * WAVES_M, BN = WN * WAVES_N;  // 256 x 256
  static constexpr int TM = WM / 32, TN = WN / 32;              // fragments per wave
  static constexpr int ROW = 96;                                // bytes per row per k-step (128 k)
  static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;        // 48 KiB
  static constexpr int A_INST = A_BYTES / 1024 / NW;           // DMA instructions per wave per k-step
  static constexpr int B_INST = B_BYTES / 1024 / NW;
  static constexpr int NST = 3;                                 // LDS stages: prefetch distance 2
  static constexpr int INST = A_INST + B_INST;  // DMA instructions per wave per k-step
  static constexpr int EPI_WAVE = 32 * WN * 2;                  // staging bytes per wave (32 rows of WN bf16)
  static constexpr int SCALE_WAVE = 1024;                       // per-wave epilogue scales (768 bytes used)
  static constexpr int LDS = NST * STAGE_BYTES + NW * SCALE_WAVE;  // 152 KiB
  // fused gate/up: the SiLU window after the scales (exactly 160 KiB)
  static constexpr int LUT_OFF = LDS;
  static constexpr int LDS_GU = LUT_OFF + kSiluWinBytes;
  static_assert(NW * EPI_WAVE <= STAGE_BYTES, "the epilogue stages its output in one free stage");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "whole DMA instructions per wave");
  static_assert(BN % 128 == 0 && B_BYTES / 1024 % (BN / 128) == 0, "12 DMA instructions per 128-row panel");
};

// One k-step's operand of fragment rows `base` (+ lane row) for MFMA `mf`:
// 24 bytes = a 16-byte and an 8-byte read (mf 0) or an 8-byte and a 16-byte
// read (mf 1) at the lane's swizzled chunk offsets.
struct F6Offsets {
  int c0, c1, c2;  // byte offsets of logical chunks 3h, 3h+1, 3h+2 in the row
  __device__ __forceinline__ F6Offsets() {
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5, s = ((lane & 31) >> 3) & 1;
    c0 = ((3 * h) ^ s) << 4;
    c1 = ((3 * h + 1) ^ s) << 4;
    c2 = ((3 * h + 2) ^ s) << 4;
  }
  __device__ __forceinline__ v8i operand(const char* row, int mf) const {
    if (mf == 0) {
      const f6_v4u x = *reinterpret_cast<const f6_v4u*>(row + c0);
      const f6_v2u y = *reinterpret_cast<const f6_v2u*>(row + c1);
      return v8i{(int)x[0], (int)x[1], (int)x[2], (int)x[3], (int)y[0], (int)y[1], 0, 0};
    }
    const f6_v2u y = *reinterpret_cast<const f6_v2u*>(row + c1 + 8);
    const f6_v4u x = *reinterpret_cast<const f6_v4u*>(row + c2);
    return v8i{(int)y[0], (int)y[1], (int)x[0], (int)x[1], (int)x[2], (int)x[3], 0, 0};
  }
};

__device__ __forceinline__ v16f mfma_f6(v8i w, v8i a, v16f c) {
  // cbsz = blgp = 3: both operands e3m2; scale 127 (e8m0) = 1.0
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 3, 3, 0, 127, 0, 127);
}

// DMA addressing of one workgroup tile (fused gate/up: B rows 0..127 from
// the gate panel b_rsrc, 128..255 from the up panel b_rsrc2).
struct F6Tiles {
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc, b_rsrc2;
  int64_t m0;
  int n0;
};

// Per-lane DMA offsets of the A slots: slot ql of wave w moves 1 KiB of
// stage rows (instruction q = w + NW * ql, flat chunk f = 64 q + lane of the
// 256 x 6 stage chunks): row f / 6, stored chunk f % 6, which holds logical
// chunk (f % 6) ^ ((row >> 3) & 1), read from the row's 96 bytes in block
// row / 128 of the tile's two (kb k-steps of 12 KiB each); the k-step's
// block is the instruction's scalar offset. The 64 lanes of an instruction
// read one contiguous KiB.
__device__ __forceinline__ void f6_a_offsets(int kb, int (&voff)[F6Tile::A_INST]) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int ql = 0; ql < F6Tile::A_INST; ++ql) {
    const int f = 64 * (wave + F6Tile::NW * ql) + lane;
    const int row = f / 6, p = f % 6;
    voff[ql] = (row >> 7) * kb * 12288 + (row & 127) * F6Tile::ROW + ((p ^ ((row >> 3) & 1)) << 4);
  }
}

// Scales of a tile's epilogue into the wave's LDS block `sc` by 4-byte LDS
// DMA (64 per instruction): the wave's WM row scales at byte 0 (rows past M
// read as zero) and its WN column scales at byte 512.
struct F6Scales {
  __amdgpu_buffer_rsrc_t as_rsrc;  // the whole row-scale vector
  const float* ws;
  int64_t row0;  // first row of the wave's rows
  int col0;      // first column of the wave's columns
};
// Fused gate/up (GU): the wave's WN / 2 gate column scales at byte 512 and
// its WN / 2 up column scales at byte 768 (ws2), from column col0.
template <bool GU = false>
__device__ __forceinline__ void f6_issue_scales(char* __restrict__ sc, const F6Scales& s, const float* ws2 = nullptr) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < F6Tile::WM / 64; ++r)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.as_rsrc, (lds_ptr_t)(sc + 256 * r), 4, lane * 4,
                                             (int)((s.row0 + 64 * r) * 4), 0, 0);
  if constexpr (GU) {
    const __amdgpu_buffer_rsrc_t g_rsrc = make_rsrc(s.ws + s.col0, F6Tile::WN / 2 * 4);
    const __amdgpu_buffer_rsrc_t u_rsrc = make_rsrc(ws2 + s.col0, F6Tile::WN / 2 * 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(g_rsrc, (lds_ptr_t)(sc + 512), 4, lane * 4, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(u_rsrc, (lds_ptr_t)(sc + 768), 4, lane * 4, 0, 0, 0);
  } else {
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(s.ws + s.col0, F6Tile::WN * 4);
#pragma unroll
    for (int c = 0; c < F6Tile::WN / 64; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(sc + 512 + 256 * c), 4, lane * 4, 256 * c, 0, 0);
  }
}

// DMA instruction `slot` of this wave's share of k-step kt of tile `x` into
// `stage` (slots 0 .. A_INST - 1 move A rows, the rest B rows; together the
// slots are f6_issue). GU: the second 128-row panel comes from b_rsrc2.
template <bool GU = false>
__device__ __forceinline__ void f6_issue_slot(char* stage, const F6Tiles& x, const int (&voff_a)[F6Tile::A_INST],
                                              int kb, int kt, int slot) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (slot < F6Tile::A_INST) {
    const int q = wave + F6Tile::NW * slot;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(x.a_rsrc, (lds_ptr_t)(stage + q * 1024), 16, voff_a[slot], kt * 12288, 0,
                                             0);
  } else {
    const int q = wave + F6Tile::NW * (slot - F6Tile::A_INST);
    const int panel = q / 12, in_blk = (q % 12) * 1024;
    if constexpr (GU)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(panel == 0 ? x.b_rsrc : x.b_rsrc2,
                                               (lds_ptr_t)(stage + F6Tile::A_BYTES + q * 1024), 16, lane * 16,
                                               kt * 12288 + in_blk, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(x.b_rsrc, (lds_ptr_t)(stage + F6Tile::A_BYTES + q * 1024), 16,
                                               lane * 16, (panel * kb + kt) * 12288 + in_blk, 0, 0);
  }
}

// DMA of k-step kt of tile `x` into `stage` (all of this wave's slots).
template <bool GU = false>
__device__ __forceinline__ void f6_issue(char* stage, const F6Tiles& x, const int (&voff_a)[F6Tile::A_INST], int kb,
                                         int kt) {
#pragma unroll
  for (int slot = 0; slot < F6Tile::INST; ++slot) f6_issue_slot<GU>(stage, x, voff_a, kb, kt, slot);
}

// The two MFMA rounds of one k-step on stage `rd`, with the DMA of k-step
// `ks` of tile `x` into `nx` spread among the MFMAs: one instruction after
// every second MFMA from the fourth on. Issuing a DMA instruction can stall
// the wave while the memory pipeline is full; between MFMAs the stall hides
// under the MFMAs already issued, and the loads start earlier in the k-step
// than when all of them follow the MFMAs (measured 4 % faster over the
// M4096 K4096 N12288 projection).
// GU: weight fragment j of the wave starts at B row b_base + j * b_step (its
// gate and up fragments); otherwise b_step = 32 * ROW.
template <bool GU = false>
__device__ __forceinline__ void f6_compute(v16f (&acc)[F6Tile::TM][F6Tile::TN], const char* __restrict__ rd,
                                           const F6Offsets& o, int a_base, int b_base, char* __restrict__ nx,
                                           const F6Tiles& x, const int (&voff_a)[F6Tile::A_INST], int kb, int ks,
                                           int b_step = 32 * F6Tile::ROW) {
  using T = F6Tile;
  int slot = 0, idx = 0;
#pragma unroll
  for (int mf = 0; mf < 2; ++mf) {
    v8i fa[T::TM], fb[T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; ++i) fa[i] = o.operand(rd + a_base + i * 32 * T::ROW, mf);
#pragma unroll
    for (int j = 0; j < T::TN; ++j) fb[j] = o.operand(rd + T::A_BYTES + b_base + j * b_step, mf);
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        acc[i][j] = mfma_f6(fb[j], fa[i], acc[i][j]);
        if ((idx & 1) && idx >= 3 && slot < T::INST) {
          __builtin_amdgcn_sched_barrier(0);
          f6_issue_slot<GU>(nx, x, voff_a, kb, ks, slot);
          ++slot;
          __builtin_amdgcn_sched_barrier(0);
        }
        ++idx;
      }
  }
#pragma unroll
  for (; slot < T::INST; ++slot) f6_issue_slot<GU>(nx, x, voff_a, kb, ks, slot);
}

// Workgroup barrier that waits for this wave's LDS operations only (a
// __syncthreads() would also drain the DMA in flight for later k-steps).
__device__ __forceinline__ void f6_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// G1 value of f32(dot) (kernels/gemm_integer.loom:394-433): RN(RN(dot * ws)
// * as) + 0, finite values clamped to the bf16 finite range, then bf16.
__device__ __forceinline__ uint32_t g1_f6(float dot, float ws, float as) {
  float y = dot * ws;
  y = y * as;
  y = y + 0.0f;
  const float sat = __builtin_fmaxf(__builtin_fminf(y, kBf16Max), -kBf16Max);
  const float checked = __builtin_fabsf(y) < __builtin_huge_valf() ? sat : y;
  return f32_to_bf16(checked);
}

// Epilogue of one tile: G1 values staged per wave (32 rows at a time) and
// stored as 16-byte row pieces, the residual added on that pass. `asr` and
// `wsr` are the lane's row scales and column scales (loaded during the last
// k-step). Fast path when, over the wave's rows below M and its columns,
// every scale is finite and positive and 64 K max|ws| max|as| < bf16 max:
// the clamp cannot fire and the value is RN(RN(dot * ws) * as) + 0.
template <bool RESID>
__device__ __forceinline__ void f6_epilogue(const v16f (&acc)[F6Tile::TM][F6Tile::TN], int K, int64_t M, int N,
                                            int64_t m0, int n0, const uint16_t* __restrict__ residual,
                                            uint16_t* __restrict__ out, char* __restrict__ wlds,
                                            const char* __restrict__ sc) {
  using T = F6Tile;
  constexpr int kRowBytes = T::WN * 2, kLanesPerRow = T::WN / 8, kRowsPerRead = 64 / kLanesPerRow;
  constexpr int kReads = T::EPI_WAVE / 1024;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const float inf = __builtin_huge_valf();
  // the scales placed by f6_issue_scales
  float asr[T::TM];
  float4 wsr[T::TN][4];
#pragma unroll
  for (int i = 0; i < T::TM; ++i) asr[i] = *reinterpret_cast<const float*>(sc + (32 * i + lr) * 4);
#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) wsr[j][q] = *reinterpret_cast<const float4*>(sc + 512 + (32 * j + 8 * q + 4 * h) * 4);
  bool ok = true;
  float amax = 0.0f, wmax = 0.0f;
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    if (m0 + wm * T::WM + 32 * i + lr < M) {
      ok = ok & (asr[i] > 0.0f) & (asr[i] < inf);
      amax = __builtin_fmaxf(amax, asr[i]);
    }
  }
#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float w4[4] = {wsr[j][q].x, wsr[j][q].y, wsr[j][q].z, wsr[j][q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        ok = ok & (w4[t] > 0.0f) & (w4[t] < inf);
        wmax = __builtin_fmaxf(wmax, w4[t]);
      }
    }
  ok = ok & (wmax * amax * (64.0f * (float)K) < kBf16Max);
  const bool fast = __all(ok);
  const int64_t rows_here = M - m0 < T::BM ? M - m0 : T::BM;
  const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(out + m0 * N, (uint32_t)(rows_here * N * 2));
  const __amdgpu_buffer_rsrc_t res_rsrc =
      make_rsrc(RESID ? residual + m0 * N : out, RESID ? (uint32_t)(rows_here * N * 2) : 0u);
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    const float asv = asr[i];
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float w4[4] = {wsr[j][q].x, wsr[j][q].y, wsr[j][q].z, wsr[j][q].w};
        uint32_t p0, p1;
        if (fast) {
          float y[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) y[t] = acc[i][j][4 * q + t] * w4[t] * asv + 0.0f;
          p0 = pack_bf16x2(y[0], y[1]);
          p1 = pack_bf16x2(y[2], y[3]);
        } else {
          p0 = g1_f6(acc[i][j][4 * q + 0], w4[0], asv) | (g1_f6(acc[i][j][4 * q + 1], w4[1], asv) << 16);
          p1 = g1_f6(acc[i][j][4 * q + 2], w4[2], asv) | (g1_f6(acc[i][j][4 * q + 3], w4[3], asv) << 16);
        }
        const int chunk = 4 * j + q;  // 16-byte chunk of the wave row: columns 8 * chunk .. + 7
        *reinterpret_cast<f6_v2u*>(wlds + lr * kRowBytes + ((chunk ^ (lr & 7)) << 4) + 8 * h) = f6_v2u{p0, p1};
      }
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      const int lrow = lane / kLanesPerRow, row = kRowsPerRead * r + lrow, chunk = lane % kLanesPerRow;
      f6_v4u v = *reinterpret_cast<const f6_v4u*>(wlds + row * kRowBytes + ((chunk ^ (row & 7)) << 4));
      const int voff = ((wm * T::WM + lrow) * N + n0 + wn * T::WN + 8 * chunk) * 2;
      const int soff = (32 * i + kRowsPerRead * r) * N * 2;
      if (RESID) {
        const v4i rv = __builtin_amdgcn_raw_buffer_load_b128(res_rsrc, voff, soff, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t p = v[t], rr = (uint32_t)rv[t];
          v[t] = pack_bf16x2(bf16_lo(rr) + bf16_lo(p), bf16_hi(rr) + bf16_hi(p));
        }
      }
      store_b128(out_rsrc, voff + soff, v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]});
    }
  }
}

// Epilogue of the fused gate/up projection: h = S1(G1(gate), G1(up)) =
// bf16(silu_bf16(g) * u) for the wave's WN / 2 output columns, where the
// wave's weight fragment 0 holds gate rows and fragment 1 the up rows of the
// same columns (kernels/swiglu.loom:43-51 on the two G1 outputs, each rounded
// to bf16 first, as the separate gate, up and SwiGLU steps do). Staged per
// wave 32 rows at a time (64-byte rows, chunk q of row r at q ^ (r & 3)) and
// stored as 16-byte row pieces. The SiLU comes from the table window in LDS
// (silu_window_pair); values outside it take silu_bf16 on a wave-uniform
// branch.
__device__ __forceinline__ void f6_epilogue_gu(const v16f (&acc)[F6Tile::TM][F6Tile::TN], int K, int64_t M, int N,
                                               int64_t m0, int n0, uint16_t* __restrict__ out,
                                               char* __restrict__ wlds, const char* __restrict__ sc,
                                               const char* __restrict__ lut) {
  using T = F6Tile;
  constexpr int WC = T::WN / 2;  // output columns per wave
  constexpr int kRowBytes = WC * 2, kLanesPerRow = WC / 8, kRowsPerRead = 64 / kLanesPerRow;
  constexpr int kReads = 32 / kRowsPerRead;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const float inf = __builtin_huge_valf();
  float asr[T::TM];
#pragma unroll
  for (int i = 0; i < T::TM; ++i) asr[i] = *reinterpret_cast<const float*>(sc + (32 * i + lr) * 4);
  // fast path as in f6_epilogue, over the wave's rows and both column sets
  // (the clamp cannot fire: every G1 value is RN(RN(dot * ws) * as) + 0)
  bool ok = true;
  float amax = 0.0f, wmax = 0.0f;
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    if (m0 + wm * T::WM + 32 * i + lr < M) {
      ok = ok & (asr[i] > 0.0f) & (asr[i] < inf);
      amax = __builtin_fmaxf(amax, asr[i]);
    }
  }
  {
    // lane lr holds gate and up scale lr of the wave's 32 columns; the bound
    // takes the wave's largest column and row scales (a lane's values mix
    // rows and columns that other lanes checked)
    const float wgl = *reinterpret_cast<const float*>(sc + 512 + lr * 4);
    const float wul = *reinterpret_cast<const float*>(sc + 768 + lr * 4);
    ok = ok & (wgl > 0.0f) & (wgl < inf) & (wul > 0.0f) & (wul < inf);
    wmax = __builtin_fmaxf(wgl, wul);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      wmax = __builtin_fmaxf(wmax, __shfl_xor(wmax, off));
      amax = __builtin_fmaxf(amax, __shfl_xor(amax, off));
    }
  }
  ok = ok & (wmax * amax * (64.0f * (float)K) < kBf16Max);
  const bool fast = __all(ok);
  const int64_t rows_here = M - m0 < T::BM ? M - m0 : T::BM;
  const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(out + m0 * N, (uint32_t)(rows_here * N * 2));
  // this lane's 16 gate and 16 up column scales (columns 8q + 4h .. + 3)
  float4 wg[4], wu[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    wg[q] = *reinterpret_cast<const float4*>(sc + 512 + (8 * q + 4 * h) * 4);
    wu[q] = *reinterpret_cast<const float4*>(sc + 768 + (8 * q + 4 * h) * 4);
  }
  // one copy of the loop per path (a wave-uniform flag tested inside would be
  // re-tested per value, a scheduling barrier between the table reads)
  auto values = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) {
      const float asv = asr[i];
      // the fragment's 16 gate and up pairs first, their 32 table reads in
      // flight together, then one wave-uniform check for values the window
      // does not cover
      uint32_t gp[4][2], upv[4][2], act[4][2];
      uint32_t outside = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float g4[4] = {wg[q].x, wg[q].y, wg[q].z, wg[q].w};
        const float u4[4] = {wu[q].x, wu[q].y, wu[q].z, wu[q].w};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if constexpr (FAST) {
            gp[q][p] = pack_bf16x2(acc[i][0][4 * q + 2 * p] * g4[2 * p] * asv + 0.0f,
                                   acc[i][0][4 * q + 2 * p + 1] * g4[2 * p + 1] * asv + 0.0f);
            upv[q][p] = pack_bf16x2(acc[i][1][4 * q + 2 * p] * u4[2 * p] * asv + 0.0f,
                                    acc[i][1][4 * q + 2 * p + 1] * u4[2 * p + 1] * asv + 0.0f);
          } else {
            gp[q][p] = g1_f6(acc[i][0][4 * q + 2 * p], g4[2 * p], asv) |
                       (g1_f6(acc[i][0][4 * q + 2 * p + 1], g4[2 * p + 1], asv) << 16);
            upv[q][p] = g1_f6(acc[i][1][4 * q + 2 * p], u4[2 * p], asv) |
                        (g1_f6(acc[i][1][4 * q + 2 * p + 1], u4[2 * p + 1], asv) << 16);
          }
          act[q][p] = silu_window_pair<true>(gp[q][p], lut, outside);
        }
      }
      if (__any(outside != 0)) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            uint32_t fix = 0;
            silu_window_pair<true>(gp[q][p], lut, fix);
#pragma unroll
            for (int t = 0; t < 2; ++t)
              if ((fix >> (16 * t)) & 0x8000u) {
                const uint32_t gb = (gp[q][p] >> (16 * t)) & 0xFFFFu;
                const uint32_t sb = f32_to_bf16(silu_bf16(bf16_to_f32(gb)));
                act[q][p] = (act[q][p] & (0xFFFF0000u >> (16 * t))) | (sb << (16 * t));
              }
          }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t h0 =
            pack_bf16x2(bf16_lo(act[q][0]) * bf16_lo(upv[q][0]), bf16_hi(act[q][0]) * bf16_hi(upv[q][0]));
        const uint32_t h1 =
            pack_bf16x2(bf16_lo(act[q][1]) * bf16_lo(upv[q][1]), bf16_hi(act[q][1]) * bf16_hi(upv[q][1]));
        *reinterpret_cast<f6_v2u*>(wlds + lr * kRowBytes + ((q ^ (lr & 3)) << 4) + 8 * h) = f6_v2u{h0, h1};
      }
#pragma unroll
      for (int r = 0; r < kReads; ++r) {
        const int lrow = lane / kLanesPerRow, row = kRowsPerRead * r + lrow, chunk = lane % kLanesPerRow;
        const f6_v4u v = *reinterpret_cast<const f6_v4u*>(wlds + row * kRowBytes + ((chunk ^ (row & 3)) << 4));
        const int voff = ((wm * T::WM + 32 * i + row) * N + n0 + wn * WC + 8 * chunk) * 2;
        store_b128(out_rsrc, voff, v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]});
      }
    }
  };
  if (fast)
    values(std::true_type{});
  else
    values(std::false_type{});
}

// Persistent bf6 G1: workgroup b walks tiles b, b + grid, ... (grid a
// multiple of 8: all on its XCD, in the XCD-aware order of tile_of_block).
// Three LDS stages in a ring: k-step kt reads stage kt % 3 while the DMA of
// k-step kt + 2 fills stage (kt + 2) % 3; the last two k-steps of a tile load
// the next tile's first two, and k-step 0 the tile's scales (into the wave's
// own block). The epilogue stages its output in the stage the last k-step
// read, and its stores drain under the next tile's first k-step.
//
// GU (fused gate/up, benches/kernels/omni_gate_up_i4.loom's dense form): a
// tile is 256 rows x 128 output columns of h; its B stage holds the 128 gate
// rows (w) and the same 128 up rows (w2) of those columns, wave (wm, wn)
// multiplies gate rows 32 wn .. and up rows 128 + 32 wn .., and the epilogue
// writes h = S1(G1(gate), G1(up)) (f6_epilogue_gu); N is the width of h.
template <bool RESID, bool GU = false>
__global__ __launch_bounds__(F6Tile::THREADS) void gemm_f6_kernel(
    const uint8_t* __restrict__ a, const float* __restrict__ as, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, int64_t M, int N, int kb, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ out, int tiles_m, int tiles_n, const uint8_t* __restrict__ w2 = nullptr,
    const float* __restrict__ ws2 = nullptr) {
#if defined(__HIP_DEVICE_COMPILE__)
  using T = F6Tile;
  constexpr int TILE_N = GU ? T::BN / 2 : T::BN;  // output columns per tile
  extern __shared__ __align__(16) char lds[];
  const int total = tiles_m * tiles_n;  // below 2^31 (launch_gemm_f6_impl)
  int t = blockIdx.x;
  if (t >= total) return;
  auto tile = [&](int b) {
    int tm, tn;
    tile_of_block(b, total, tiles_m, tiles_n, tm, tn);
    F6Tiles x;
    x.m0 = (int64_t)tm * T::BM;
    x.n0 = tn * TILE_N;
    // the tile's one or two 128-row blocks of activation codes (a second
    // block past M does not exist: its loads fall outside the resource)
    const int blocks_here = M - x.m0 > 128 ? 2 : 1;
    x.a_rsrc = make_rsrc(a + (x.m0 >> 7) * kb * 12288, (uint32_t)(blocks_here * kb * 12288));
    x.b_rsrc = make_rsrc(w + (int64_t)(x.n0 / 128) * kb * 12288, (uint32_t)((TILE_N / 128) * kb * 12288));
    x.b_rsrc2 = GU ? make_rsrc(w2 + (int64_t)(x.n0 / 128) * kb * 12288, (uint32_t)(kb * 12288)) : x.b_rsrc;
    return x;
  };
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int lr = lane & 31;
  int voff_a[T::A_INST];
  f6_a_offsets(kb, voff_a);
  const F6Offsets o;
  const int a_base = (wm * T::WM + lr) * T::ROW;
  const int b_base = ((GU ? wn * (T::WN / 2) : wn * T::WN) + lr) * T::ROW;
  const int b_step = (GU ? T::BN / 2 : 32) * T::ROW;  // weight fragment 1: the up rows (GU)
  auto st = [&](int i) { return lds + i * T::STAGE_BYTES; };
  char* sc = lds + T::NST * T::STAGE_BYTES + wave * T::SCALE_WAVE;
  F6Scales scales;
  scales.as_rsrc = make_rsrc(as, (uint32_t)(M * 4));
  scales.ws = ws;

  F6Tiles cur = tile(t);
  const char* lut = lds + T::LUT_OFF;
  if constexpr (GU) {
    // the SiLU window: one KiB per wave (sign half wave / 4, KiB wave % 4)
    const __amdgpu_buffer_rsrc_t lut_rsrc = make_rsrc(g_silu_lut, kSiluLutSize * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        lut_rsrc, (lds_ptr_t)(lds + T::LUT_OFF + wave * 1024), 16, lane * 16,
        (wave >> 2) * (kSiluLutSize / 2) * 2 + kSiluWinSrc + (wave & 3) * 1024, 0, 0);
  }
  f6_issue<GU>(st(0), cur, voff_a, kb, 0);
  f6_issue<GU>(st(1), cur, voff_a, kb, 1);
  wait_vmcnt<0>();
  f6_lds_barrier();
  int rot = 0;  // ring position of the tile's k-step 0
  v16f acc[T::TM][T::TN];
  while (true) {
    const int t_next = t + (int)gridDim.x;
    const bool has_next = t_next < total;
    const F6Tiles nxt = tile(has_next ? t_next : t);  // the last tile re-reads its own
    scales.row0 = cur.m0 + wm * T::WM;
    scales.col0 = cur.n0 + wn * (GU ? T::WN / 2 : T::WN);
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = v16f{};
    // The tile's k-steps, the ring unrolled by three so that each step names
    // its stages statically (distinct restrict pointers of this one body: the
    // compiler then keeps the DMA in flight across the LDS reads). Every step
    // issues the same DMA (the k-step two ahead: this tile's, the next
    // tile's first two, or for the last tile a repeat of its own first two
    // into stages never read again) and ends with the same wait, so a step is
    // one straight block and its MFMAs stay ahead of its wait.
    auto tile_body = [&](char* __restrict__ r0, char* __restrict__ r1, char* __restrict__ r2,
                         char* __restrict__ scl) {
      auto step = [&](const char* rd, char* nx, int kt, auto scales_tag) {
        // The scales (k-step 0) before the stage DMA, so that the DMA group
        // is the last one issued (the wait below counts on it).
        if constexpr (decltype(scales_tag)::value) f6_issue_scales<GU>(scl, scales, ws2);
        __builtin_amdgcn_sched_barrier(0);
        const bool own = kt + 2 < kb;
        // the DMA's tile, selected field by field (scalar selects; a select
        // of the whole struct would go through scratch memory)
        F6Tiles src;
        src.a_rsrc = own ? cur.a_rsrc : nxt.a_rsrc;
        src.b_rsrc = own ? cur.b_rsrc : nxt.b_rsrc;
        src.b_rsrc2 = own ? cur.b_rsrc2 : nxt.b_rsrc2;
        f6_compute<GU>(acc, rd, o, a_base, b_base, nx, src, voff_a, kb, own ? kt + 2 : kt + 2 - kb, b_step);
        __builtin_amdgcn_sched_barrier(0);
        // k-step kt + 1 has landed once at most the DMA issued here is
        // outstanding (vector memory operations complete in issue order; at
        // k-step 0 this also drains the previous tile's stores)
        wait_vmcnt<T::INST>();
        f6_lds_barrier();
      };
      step(r0, r2, 0, std::true_type{});
      for (int kt0 = 1; kt0 < kb; kt0 += 3) {
        step(r1, r0, kt0, std::false_type{});
        if (kt0 + 1 < kb) step(r2, r1, kt0 + 1, std::false_type{});
        if (kt0 + 2 < kb) step(r0, r2, kt0 + 2, std::false_type{});
      }
    };
    tile_body(st(rot), st((rot + 1) % 3), st((rot + 2) % 3), sc);
    // the next tile's k-steps 0 and 1 and this tile's scales have landed
    wait_vmcnt<0>();
    char* staging = st((rot + kb - 1) % 3) + wave * T::EPI_WAVE;
    if constexpr (GU)
      f6_epilogue_gu(acc, kb * 128, M, N, cur.m0, cur.n0, out, staging, sc, lut);
    else
      f6_epilogue<RESID>(acc, kb * 128, M, N, cur.m0, cur.n0, residual, out, staging, sc);
    if (!has_next) break;
    // every wave is done with the staging stage before k-step 0 of the next
    // tile loads k-step 2 into it
    f6_lds_barrier();
    rot = (rot + kb) % 3;
    t = t_next;
    cur = nxt;
  }
  wait_vmcnt<0>();
#endif
}

// GU: w / ws the gate weight, w2 / ws2 the up weight, n the width of h
// (n % 128 == 0), out = h.
template <bool RESID, bool GU = false>
hipError_t launch_gemm_f6_impl(const uint8_t* a, const float* as, const uint8_t* w, const float* ws, int64_t m, int n,
                               int k, const uint16_t* residual, uint16_t* out, hipStream_t stream,
                               const uint8_t* w2 = nullptr, const float* ws2 = nullptr) {
  using T = F6Tile;
  constexpr int lds = GU ? T::LDS_GU : T::LDS;
  static_assert(lds <= 160 * 1024, "LDS per workgroup");
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&gemm_f6_kernel<RESID, GU>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, lds)) return e;
  int per_cu = 0, cus = 0;
  if (hipError_t e = resident_per_cu(cache, kern, T::THREADS, lds, per_cu, cus)) return e;
  const int tiles_n = n / (GU ? T::BN / 2 : T::BN);
  const int64_t tiles_m = (m + T::BM - 1) / T::BM;
  const int64_t total = tiles_m * tiles_n;
  if (total > kMaxTiles) return hipErrorInvalidValue;  // the kernel's 32-bit tile indices
  int64_t grid = (int64_t)cus * per_cu / 8 * 8;
  if (grid < 8) grid = 8;
  if (grid > total) grid = total;
  gemm_f6_kernel<RESID, GU><<<(unsigned)grid, T::THREADS, lds, stream>>>(
      a, as, w, ws, m, n, k / 128, residual, out, (int)tiles_m, tiles_n, w2, ws2);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_f6_rows(const uint32_t* a, int a_words, int64_t rows, int k, uint8_t* out, hipStream_t stream) {
  const int64_t total = rows * (k / 32);
  const int64_t blocks = (total + 255) / 256;
  f6_rows_kernel<<<(unsigned)(blocks < 8192 ? blocks : 8192), 256, 0, stream>>>(a, a_words, rows, k, out);
  return hipGetLastError();
}

hipError_t launch_f6_tiled(const uint32_t* w_tiled, int64_t n, int k, uint8_t* out, hipStream_t stream) {
  const int64_t total = n * (k / 32);
  const int64_t blocks = (total + 255) / 256;
  f6_tiled_kernel<<<(unsigned)(blocks < 8192 ? blocks : 8192), 256, 0, stream>>>(w_tiled, n, k, out);
  return hipGetLastError();
}

hipError_t launch_gemm_f6(const uint8_t* a, const float* as, const uint8_t* w, const float* ws, int64_t m, int n,
                          int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (residual) return launch_gemm_f6_impl<true>(a, as, w, ws, m, n, k, residual, out, stream);
  return launch_gemm_f6_impl<false>(a, as, w, ws, m, n, k, residual, out, stream);
}

hipError_t launch_gemm_f6_gate_up(const uint8_t* a, const float* as, const uint8_t* gate_w, const float* gate_s,
                                  const uint8_t* up_w, const float* up_s, int64_t m, int n, int k, uint16_t* h,
                                  hipStream_t stream) {
  return launch_gemm_f6_impl<false, true>(a, as, gate_w, gate_s, m, n, k, nullptr, h, stream, up_w, up_s);
}

}  // namespace clef
