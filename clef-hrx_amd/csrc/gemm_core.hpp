// Shared int4 x int4 -> i32 contraction core for gfx950 (dense and grouped
// expert GEMMs).
//
// Operands are the reference's packed codes (8 signed int4 per u32, nibble p =
// k offset p): activations row-major [rows][stride/8] words, weights in the
// retiled 128-row x 32-word blocks (kernels/retile_codes.loom:2-5). One
// k-step covers 256 k = 32 words = 128 bytes per row, which is exactly one
// retile block row, so a 128-row weight tile of one k-step is one contiguous
// 16 KiB block.
//
// Data flow per k-step: global (16-byte loads) -> registers -> LDS as nibbles
// (double-buffered) -> 8-byte LDS reads per MFMA fragment -> unpack to int8
// (16 * code) -> v_mfma_i32_16x16x64_i8 with i32 accumulation. Both operands
// use the same lane -> k map, so the i32 result is 256 times the exact code
// dot product; the epilogue shifts it back down (exact).
//
// LDS layout: row r of a tile is 128 bytes = 16 half-chunks of 8 bytes; half
// chunk h lives at position h ^ (r & 15), which keeps the 16 lanes of a
// fragment read on distinct banks. A 16-byte chunk c therefore sits at chunk
// position c ^ ((r >> 1) & 7) with its halves swapped when r is odd.
//
// MFMA roles are swapped (weights in the A slot, activations in the B slot) so
// that output lane l holds 4 consecutive columns n of one row m: one 8-byte
// store per fragment.
#pragma once

#include "common.hpp"

namespace clef {

template <int BM_, int BN_, int WM_, int WN_>
struct GemmTile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
  static_assert(WAVES_M * WAVES_N == 4, "four waves per workgroup");
  static_assert(WM % 16 == 0 && WN % 16 == 0 && BN % 128 == 0 && BM % 32 == 0, "tile shape");
  static constexpr int TM = WM / 16, TN = WN / 16;
  static constexpr int AL = BM * 8 / 256;  // 16-byte A chunks per thread per k-step
  static constexpr int BL = BN * 8 / 256;  // 16-byte B chunks per thread per k-step
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
};

__device__ __forceinline__ uint32_t chunk_offset(int r, int c) {
  return (uint32_t)(r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
}

__device__ __forceinline__ uint4 swap_halves_if(uint4 v, bool odd) {
  return odd ? make_uint4(v.z, v.w, v.x, v.y) : v;
}

__device__ __forceinline__ uint2 read_half(const char* region, int r, int h) {
  return *reinterpret_cast<const uint2*>(region + r * 128 + ((h ^ (r & 15)) << 3));
}

// Main loop. a_ptr[j]: this thread's A chunk for load slot j at k-step 0
// (advances 32 words per step). b_ptr[j]: same for B (advances 4096 words).
template <class T>
__device__ __forceinline__ void gemm_mainloop(const uint32_t* (&a_ptr)[T::AL],
                                              const uint32_t* (&b_ptr)[T::BL], int ksteps,
                                              char* lds, v4i (&acc)[T::TM][T::TN]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int g = lane >> 4, lr = lane & 15;

#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  uint4 ra[T::AL], rb[T::BL];
  auto load = [&](int kt) {
#pragma unroll
    for (int j = 0; j < T::AL; ++j) ra[j] = *reinterpret_cast<const uint4*>(a_ptr[j] + kt * 32);
#pragma unroll
    for (int j = 0; j < T::BL; ++j)
      rb[j] = *reinterpret_cast<const uint4*>(b_ptr[j] + (int64_t)kt * 4096);
  };
  auto store = [&](int stage) {
    char* sa = lds + stage * T::STAGE_BYTES;
    char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int j = 0; j < T::AL; ++j) {
      const int idx = tid + 256 * j;
      const int r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(sa + chunk_offset(r, c)) = swap_halves_if(ra[j], r & 1);
    }
#pragma unroll
    for (int j = 0; j < T::BL; ++j) {
      const int idx = tid + 256 * j;
      const int r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(sb + chunk_offset(r, c)) = swap_halves_if(rb[j], r & 1);
    }
  };

  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < ksteps; ++kt) {
    const int stage = kt & 1;
    if (kt + 1 < ksteps) load(kt + 1);
    const char* sa = lds + stage * T::STAGE_BYTES;
    const char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int h = 4 * g + s;  // words 8g+2s, 8g+2s+1 of the 32-word row
      v4i oa[T::TM], ob[T::TN];
#pragma unroll
      for (int i = 0; i < T::TM; ++i) {
        uint2 w = read_half(sa, wm * T::WM + 16 * i + lr, h);
        oa[i] = unpack_pair(w.x, w.y);
      }
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        uint2 w = read_half(sb, wn * T::WN + 16 * j + lr, h);
        ob[j] = unpack_pair(w.x, w.y);
      }
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma_i8(ob[j], oa[i], acc[i][j]);
    }
    if (kt + 1 < ksteps) store(stage ^ 1);
    __syncthreads();
  }
}

}  // namespace clef
