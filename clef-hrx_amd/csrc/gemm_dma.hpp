// int4 x int4 -> i32 contraction core with direct global->LDS loads (gfx950).
//
// Arithmetic: nibbles are unpacked to int8 bytes holding 16 * code and fed to
// v_mfma_i32_32x32x32_i8 with i32 accumulation. Both operands use one lane ->
// k map, so each i32 result is 256 times the exact code dot product (shifted
// back down, exactly, in the epilogue).
//
// Data movement:
//  * Global -> LDS by buffer_load_dwordx4 ... lds: a wave instruction moves 64
//    lanes x 16 bytes into 1 KiB of LDS with no VGPR staging. A lane's LDS
//    position is fixed (base + 16 * lane), so the XOR swizzle is realised on
//    the global side: physical chunk pc of row r holds logical chunk
//    pc ^ ((r >> 1) & 7). Rows past the operand's end read as zero (buffer
//    range).
//  * Two LDS stages of one 256-k step (128 bytes per row) each, one barrier
//    per step. The DMA for step k+2 is issued right after the barrier that
//    ends the reads of the buffer it overwrites.
//  * Fragments are read 16 bytes per lane (one swizzled chunk) covering two
//    32-k substeps, one chunk pair ahead, so the unpack of substep s+1
//    overlaps the MFMAs of substep s. The (r >> 1) & 7 swizzle measured
//    conflict-free for this 32-row read on gfx950 (r & 7 ran at 0.6x).
//
// k map (256-k step = 8 substeps of 32 k): lane half h = lane/32 of substep s
// takes words 2(s%2), 2(s%2)+1 of logical chunk 4h + s/2 of the 32-word row,
// for activations and weights alike.
//
// MFMA roles: weights in the A slot, activations in the B slot, so output
// lane l holds row m = l % 32 and, for register r, column
// 8(r/4) + 4(l/32) + r%4: four consecutive columns per register quad.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace clef {

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v2i __attribute__((ext_vector_type(2)));

template <int WM_, int WN_, int WAVES_M_, int WAVES_N_, bool HINT_ = true>
struct DmaTile {
  static constexpr int WM = WM_, WN = WN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr bool HINT = HINT_;
  static constexpr int NW = WAVES_M * WAVES_N;  // waves per workgroup
  static constexpr int THREADS = 64 * NW;
  static constexpr int BM = WM * WAVES_M, BN = WN * WAVES_N;
  static_assert(NW == 4 || NW == 8, "four or eight waves per workgroup");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BN % 128 == 0, "tile shape");
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "whole DMA instructions per wave");
  static constexpr int TM = WM / 32, TN = WN / 32;
  static constexpr int A_INST = BM / (8 * NW);  // DMA instructions per wave per k-step
  static constexpr int B_INST = BN / (8 * NW);
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = 2 * STAGE_BYTES;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(n) with the other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

__device__ __forceinline__ v16i mfma32_i8(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Logical 16-byte chunk (times 16) that DMA lane `lane` of wave `wave` moves:
// lane -> tile row r = 8q + lane/8, physical chunk lane%8, which holds logical
// chunk (lane%8) ^ g(r) with g(r) = (r >> 1) & 7 = ((q & 1) << 2) | (lane >> 4);
// q & 1 = wave & 1 for every DMA instruction of a wave (q = wave + NW * ql,
// NW even).
__device__ __forceinline__ int dma_chunk16(int wave, int lane) {
  return ((lane & 7) ^ ((((wave & 1) << 2) | (lane >> 4)) & 7)) * 16;
}

// A-operand DMA addressing: slot ql of wave w covers tile rows 8q .. 8q+7
// (q = w + NW * ql); voff_a[ql] is the lane's byte offset of its chunk at
// k-step 0 and the wave-uniform part is 8 * q * a_q_stride + kt * 128.
// Contiguous rows: a_rsrc starts at the tile's first row, voff_a[ql] =
// (lane/8) * row_bytes + chunk, a_q_stride = row_bytes. Gathered rows:
// voff_a[ql] = the lane's row offset in the whole buffer + chunk (or an
// out-of-range offset, which reads zeros), a_q_stride = 0.
//
// b_rsrc covers the tile's BN/128 retile block rows for all k-steps (block
// (b, kt) at (b * ksteps + kt) * 16 KiB).
template <class T>
__device__ __forceinline__ void dma_mainloop(__amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                             int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps,
                                             char* lds, v16i (&acc)[T::TM][T::TN]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep the
  // DMA scalar offsets and LDS bases in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;

#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};

  const int voff_b = (lane >> 3) * 128 + dma_chunk16(wave, lane);

  auto issue = [&](int kt, int stage) {
    char* sa = lds + stage * T::STAGE_BYTES;
    char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) {
      const int q = wave + T::NW * ql;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(sa + q * 1024), 16, voff_a[ql],
                                               8 * q * a_q_stride + kt * 128, 0, 0);
    }
#pragma unroll
    for (int ql = 0; ql < T::B_INST; ++ql) {
      const int q = wave + T::NW * ql;
      const int blk = (8 * q) >> 7, row_in = (8 * q) & 127;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_ptr_t)(sb + q * 1024), 16, voff_b,
                                               (blk * ksteps + kt) * 16384 + row_in * 128, 0, 0);
    }
  };

  // Chunk-pair read offsets (within a region) for pair p = substeps 2p, 2p+1.
  const int a_row = (wm * T::WM + lr) * 128;
  const int b_row = (wn * T::WN + lr) * 128;
  int offs[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) offs[p] = ((4 * h + p) ^ ((lr >> 1) & 7)) << 4;

  constexpr int NF = T::TM + T::TN;
  uint4 raw[2][NF];
  auto read = [&](int buf, int stage, int p) {
    const char* sa = lds + stage * T::STAGE_BYTES;
    const char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
      raw[buf][i] = *reinterpret_cast<const uint4*>(sa + a_row + i * 4096 + offs[p]);
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      raw[buf][T::TM + j] = *reinterpret_cast<const uint4*>(sb + b_row + j * 4096 + offs[p]);
  };

  v4i u[2][NF];
  auto unpack = [&](int dst, int buf, int half) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
      u[dst][f] = half == 0 ? unpack_pair(raw[buf][f].x, raw[buf][f].y)
                            : unpack_pair(raw[buf][f].z, raw[buf][f].w);
  };
  auto mma = [&](int src) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
  };

  // Scheduling of one substep: the chunk reads it issues first, then
  // {1 MFMA, VPM VALU} repeated, so the unpack (and address arithmetic) of
  // the next substep fills the MFMA shadow instead of trailing it.
  constexpr int MF = T::TM * T::TN;
  constexpr int VPM = (6 * NF + MF - 1) / MF + 1;
  auto hint = [&](auto reads) {
    if constexpr (T::HINT) {
      if constexpr (decltype(reads)::value > 0)
        __builtin_amdgcn_sched_group_barrier(0x100, decltype(reads)::value, 0);
#pragma unroll
      for (int q = 0; q < MF; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
      }
    }
  };

  // The steady-state body is branch-free (one basic block per k-step) so the
  // accumulators stay in place: the DMA for step kt + 2 and the read of step
  // kt + 1 are issued even past the last step. Those loads are range-checked
  // buffer reads (row padding or zeros, never a fault) into a stage that is
  // not read again; the final wait drains them before the epilogue.
  issue(0, 0);
  issue(1, 1);
  wait_vmcnt<T::A_INST + T::B_INST>();
  __syncthreads();
  read(0, 0, 0);
  unpack(0, 0, 0);

  for (int kt = 0; kt < ksteps; ++kt) {
    const int st = kt & 1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int cur = p & 1;
      // substep 2p: prefetch the next chunk pair, MFMAs on u[0], unpack the
      // odd half of this pair into u[1].
      if (p < 3) {
        read(cur ^ 1, st, p + 1);
      } else {
        wait_vmcnt<0>();
        __syncthreads();
        issue(kt + 2, st);
        read(cur ^ 1, st ^ 1, 0);
      }
      mma(0);
      unpack(1, cur, 1);
      hint(std::integral_constant<int, NF>{});
      // substep 2p+1: MFMAs on u[1], unpack the even half of the next pair.
      mma(1);
      unpack(0, cur ^ 1, 0);
      hint(std::integral_constant<int, 0>{});
    }
  }
  wait_vmcnt<0>();
}

}  // namespace clef
