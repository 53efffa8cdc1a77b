// int4 x int4 -> i32 contraction core with half-k-step LDS stages (gfx950).
//
// Same arithmetic, unpack, MFMA roles and lane -> k map as gemm_dma.hpp; what
// changes is the staging, so that two workgroups fit on one CU and each one's
// prologue and epilogue run under the other's MFMAs:
//  * a stage holds 128 k of every tile row: 64 bytes per row, four 16-byte
//    chunks. Of the eight chunks c of a row's 256-k step, stage half s holds
//    c = 4h + 2s + p' (h, p' in {0, 1}) at logical position L = 2h + p';
//    physical chunk pc of row r holds L = pc ^ ((r >> 2) & 3), measured
//    conflict-free for the 32-row ds_read_b128 on gfx950;
//  * two stages alternate: the DMA of half-step j + 1 is issued when half-step
//    j starts and drained when it ends (a barrier orders LDS DMA like any
//    other LDS write, so a deeper prefetch would be drained at the barrier
//    anyway); the second workgroup on the CU covers the DMA latency;
//  * a 4-wave workgroup owns BM x BN = (WM * WAVES_M) x (WN * WAVES_N); with
//    256 x 128 it needs 64 KiB of LDS (the epilogue's staged output tile), so
//    two workgroups share a CU.
//
// DMA lane map: one instruction moves 16 rows x 4 chunks; lane -> row
// 16q + lane/4, physical chunk lane%4, which holds logical
// L = (lane & 3) ^ ((lane >> 4) & 3) (the row's (r >> 2) & 3 is lane >> 4 for
// every 16-row group), i.e. global chunk 4(L >> 1) + (L & 1) + 2s.
#pragma once

#include <type_traits>

#include "gemm_dma.hpp"

namespace clef {

// SPLIT_B: the B tile is two panels of BN/2 rows from two buffers (rows
// [0, BN/2) from b_rsrc, [BN/2, BN) from b_rsrc2), and wave wn takes columns
// [wn * WN/2, +WN/2) of each half, so fragment j and j + TN/2 of a lane hold the
// same output column of the two panels (fused gate/up).
template <int WM_, int WN_, int WAVES_M_, int WAVES_N_, int SCHED_ = kSchedFree, bool SPLIT_B_ = false>
struct DmaHTile {
  static constexpr int WM = WM_, WN = WN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int SCHED = SCHED_;
  static constexpr bool SPLIT_B = SPLIT_B_;
  static constexpr int NW = WAVES_M * WAVES_N;
  static constexpr int THREADS = 64 * NW;
  static constexpr int BM = WM * WAVES_M, BN = WN * WAVES_N;
  static_assert(NW == 4 || NW == 8, "four or eight waves per workgroup");
  static_assert(WM % 32 == 0 && WN % 32 == 0 && BN % 128 == 0, "tile shape");
  static_assert(BM % (16 * NW) == 0 && BN % (16 * NW) == 0, "whole DMA instructions per wave");
  static constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(!SPLIT_B_ || (TN % 2 == 0 && BN % 256 == 0), "split B: whole 128-row panels per half");
  static constexpr int A_INST = BM / (16 * NW);  // DMA instructions per wave per half-step
  static constexpr int B_INST = BN / (16 * NW);
  static constexpr int INST = A_INST + B_INST;
  static constexpr int A_BYTES = BM * 64, B_BYTES = BN * 64;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int NSTAGE = 2;
  static constexpr int OUT_BYTES = NW * WM * WN * 2;  // staged bf16 output tile
  static constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES > OUT_BYTES ? NSTAGE * STAGE_BYTES : OUT_BYTES;
};

// Byte offset, within a row's 128-byte k-step block, of the chunk DMA lane
// `lane` moves for stage half 0 (stage half 1 adds 32, a wave-uniform term).
__device__ __forceinline__ int dmah_chunk16(int lane) {
  const int L = (lane & 3) ^ ((lane >> 4) & 3);
  return (4 * (L >> 1) + (L & 1)) * 16;
}

template <class T>
struct DmaHCore {
  static constexpr int NF = T::TM + T::TN;
  static constexpr int MF = T::TM * T::TN;
  int wave, voff_b, a_row;
  int b_row[T::TN];
  int offs[2];
  uint4 raw[2][NF];
  v4i u[2][NF];

  __device__ __forceinline__ DmaHCore() {
    const int lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
    const int h = lane >> 5, lr = lane & 31;
    voff_b = (lane >> 2) * 128 + dmah_chunk16(lane);
    a_row = (wm * T::WM + lr) * 64;
#pragma unroll
    for (int j = 0; j < T::TN; ++j) {
      const int col = T::SPLIT_B ? (j < T::TN / 2 ? 0 : T::BN / 2) + wn * (T::WN / 2) + 32 * (j % (T::TN / 2))
                                 : wn * T::WN + 32 * j;
      b_row[j] = (col + lr) * 64;
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) offs[p] = ((2 * h + p) ^ ((lr >> 2) & 3)) << 4;
  }

  // DMA of half-step j (k-step j / 2, stage half j % 2) into `stage`.
  // voff_a[ql]: the lane's row offset plus dmah_chunk16 (contiguous rows:
  // (lane / 4) * row_bytes + chunk with a_q_stride = row_bytes; gathered rows:
  // the row's offset in the whole buffer + chunk, a_q_stride = 0).
  // SPLIT_B: B slots of the second half read b_rsrc2 (their panel's blocks
  // counted from 0); the half a slot belongs to is fixed per slot index.
  __device__ __forceinline__ void issue(char* stage, __amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                        int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc,
                                        __amdgpu_buffer_rsrc_t b_rsrc2, int ksteps, int j) {
    issue_a(stage, a_rsrc, voff_a, a_q_stride, j);
    issue_b(stage, b_rsrc, b_rsrc2, ksteps, j);
  }
  // The activation rows (A_INST instructions) and the weight rows (B_INST)
  // of half-step j separately.
  __device__ __forceinline__ void issue_a(char* stage, __amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                          int a_q_stride, int j) {
    const int kt = j >> 1, half = (j & 1) * 32;
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) {
      const int q = wave + T::NW * ql;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(stage + q * 1024), 16, voff_a[ql],
                                               16 * q * a_q_stride + kt * 128 + half, 0, 0);
    }
  }
  __device__ __forceinline__ void issue_b(char* stage, __amdgpu_buffer_rsrc_t b_rsrc, __amdgpu_buffer_rsrc_t b_rsrc2,
                                          int ksteps, int j) {
    const int kt = j >> 1, half = (j & 1) * 32;
    char* sb = stage + T::A_BYTES;
#pragma unroll
    for (int ql = 0; ql < T::B_INST; ++ql) {
      const int q = wave + T::NW * ql;
      int blk = (16 * q) >> 7;
      const int row_in = (16 * q) & 127;
      bool second = false;
      if constexpr (T::SPLIT_B) {
        // q < NW * (ql + 1) and 16 q < 128 (ql + 1) * ...: the half follows from ql alone.
        second = ql >= T::B_INST / 2;
        blk -= second ? T::BN / 256 : 0;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(second ? b_rsrc2 : b_rsrc, (lds_ptr_t)(sb + q * 1024), 16, voff_b,
                                               (blk * ksteps + kt) * 16384 + row_in * 128 + half, 0, 0);
    }
  }

  // Chunk pair p of every fragment of `stage` -> raw[buf].
  __device__ __forceinline__ void read(const char* stage, int buf, int p) {
    const char* sb = stage + T::A_BYTES;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
      raw[buf][i] = *reinterpret_cast<const uint4*>(stage + a_row + i * 2048 + offs[p]);
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      raw[buf][T::TM + j] = *reinterpret_cast<const uint4*>(sb + b_row[j] + offs[p]);
  }

  __device__ __forceinline__ void unpack_one(int dst, int buf, int half, int f) {
    u[dst][f] = half == 0 ? unpack_pair(raw[buf][f].x, raw[buf][f].y) : unpack_pair(raw[buf][f].z, raw[buf][f].w);
  }
  __device__ __forceinline__ void unpack(int dst, int buf, int half) {
#pragma unroll
    for (int f = 0; f < NF; ++f) unpack_one(dst, buf, half, f);
  }

  // One substep on u[src] with the unpack of raw[buf] (half) into u[dst].
  template <bool UNPACK>
  __device__ __forceinline__ void substep(v16i (&acc)[T::TM][T::TN], int src, int dst, int buf, int half) {
    if constexpr (T::SCHED == kSchedPin) {
#pragma unroll
      for (int q = 0; q < MF; ++q) {
        const int i = q / T::TN, j = q % T::TN;
        acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
        if constexpr (UNPACK) {
#pragma unroll
          for (int f = 0; f < NF; ++f)
            if (f * MF / NF == q) unpack_one(dst, buf, half, f);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
      if constexpr (UNPACK) unpack(dst, buf, half);
    }
  }

  // Pair 0 of half-step from `rd` (already in raw[0], even half in u[0]) and
  // the prefetch of pair 1: leaves pair 1 in raw[1] and its even half in u[0].
  __device__ __forceinline__ void pair0(v16i (&acc)[T::TM][T::TN], const char* rd) {
    read(rd, 1, 1);
    substep<true>(acc, 0, 1, 0, 1);
    substep<true>(acc, 1, 0, 1, 0);
  }
};

// Half-step bodies; as in gemm_dma.hpp, the stage being loaded and the
// stage being read are distinct restrict pointers of one inlined call so that
// the outstanding DMA is not drained by the reads. COMPUTE = false runs the
// DMA and barrier schedule only (a wave whose rows are all past the end keeps
// the workgroup's barriers without spending MFMA work on them).

// Half-step 0: DMA of half-steps 0 and 1, pair 0 of half-step 0.
template <class T, bool COMPUTE>
__device__ __forceinline__ void dmah_first(DmaHCore<T>& c, v16i (&acc)[T::TM][T::TN], char* __restrict__ rd,
                                           char* __restrict__ dma, __amdgpu_buffer_rsrc_t a_rsrc,
                                           const int (&voff_a)[T::A_INST], int a_q_stride,
                                           __amdgpu_buffer_rsrc_t b_rsrc, __amdgpu_buffer_rsrc_t b_rsrc2,
                                           int ksteps) {
  c.issue(rd, a_rsrc, voff_a, a_q_stride, b_rsrc, b_rsrc2, ksteps, 0);
  c.issue(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, b_rsrc2, ksteps, 1);
  wait_vmcnt<T::INST>();
  __syncthreads();
  if constexpr (COMPUTE) {
    c.read(rd, 0, 0);
    c.unpack(0, 0, 0);
    c.pair0(acc, rd);
  }
  wait_vmcnt<0>();
  __syncthreads();
}

// Half-step j >= 1 reading `rd`: DMA of half-step j + 1 into `dma` (freed by
// half-step j - 1), the last pair of half-step j - 1 (registers only), pair 0
// of j; ends once half-step j + 1 has landed and every wave is done with `rd`.
template <class T, bool COMPUTE>
__device__ __forceinline__ void dmah_next(DmaHCore<T>& c, v16i (&acc)[T::TM][T::TN], const char* __restrict__ rd,
                                          char* __restrict__ dma, __amdgpu_buffer_rsrc_t a_rsrc,
                                          const int (&voff_a)[T::A_INST], int a_q_stride,
                                          __amdgpu_buffer_rsrc_t b_rsrc, __amdgpu_buffer_rsrc_t b_rsrc2, int ksteps,
                                          int j) {
  c.issue(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, b_rsrc2, ksteps, j + 1);
  if constexpr (COMPUTE) {
    c.read(rd, 0, 0);
    if constexpr (T::SCHED == kSchedPin) __builtin_amdgcn_sched_barrier(0);
    c.template substep<true>(acc, 0, 1, 1, 1);
    c.template substep<true>(acc, 1, 0, 0, 0);
    c.pair0(acc, rd);
  }
  wait_vmcnt<0>();
  __syncthreads();
}

// Full contraction over `ksteps` 256-k steps (2 * ksteps half-steps) into acc.
// Branch-free bodies: the last half-step also loads the half-step past the
// end (a range-checked buffer read: zeros, row padding or the next panel,
// never a fault) into the stage that is not read again, drained by its
// closing wait.
template <class T, bool COMPUTE = true>
__device__ __forceinline__ void dmah_mainloop(__amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                              int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc,
                                              __amdgpu_buffer_rsrc_t b_rsrc2, int ksteps, char* lds,
                                              v16i (&acc)[T::TM][T::TN]) {
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
  DmaHCore<T> c;
  dmah_first<T, COMPUTE>(c, acc, lds, lds + T::STAGE_BYTES, a_rsrc, voff_a, a_q_stride, b_rsrc, b_rsrc2, ksteps);
  for (int j = 1; j < 2 * ksteps; ++j) {
    char* rd = lds + (j & 1) * T::STAGE_BYTES;
    char* dma = lds + ((j & 1) ^ 1) * T::STAGE_BYTES;
    dmah_next<T, COMPUTE>(c, acc, rd, dma, a_rsrc, voff_a, a_q_stride, b_rsrc, b_rsrc2, ksteps, j);
  }
  if constexpr (COMPUTE) {
    c.template substep<true>(acc, 0, 1, 1, 1);
    c.template substep<false>(acc, 1, 0, 0, 0);
  }
}

}  // namespace clef
