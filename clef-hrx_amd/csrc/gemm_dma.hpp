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

// Main-loop instruction scheduling: the compiler's own order, interleaving
// hints (sched_group_barrier), or an order pinned by sched_barrier fences.
enum DmaSched { kSchedFree = 0, kSchedHint = 1, kSchedPin = 2 };

template <int WM_, int WN_, int WAVES_M_, int WAVES_N_, int SCHED_ = kSchedHint>
struct DmaTile {
  static constexpr int WM = WM_, WN = WN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int SCHED = SCHED_;
  static constexpr bool HINT = SCHED_ == kSchedHint;
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

// 16-byte buffer store with a zero scalar offset. A buffer store of more than
// 8 bytes reads its data VGPRs after issue, so a VALU write to them must not
// follow at once (one wait state). The compiler inserts that wait only for
// stores whose soffset is not an SGPR; with an SGPR soffset the data was
// measured to be overwritten on gfx950 (the last lanes of each 16-lane group
// stored the next value of the register). Callers fold any scalar part of
// the offset into `voff`.
__device__ __forceinline__ void store_b128(__amdgpu_buffer_rsrc_t rsrc, int voff, v4i v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, 0, 0);
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
//
// Per-lane state of the main loop: fragment registers, read offsets and the
// DMA addressing. Every LDS access takes its stage pointer as an argument so
// that the k-step bodies below can pass the stage being loaded and the stage
// being read as distinct restrict pointers.
template <class T>
struct DmaCore {
  static constexpr int NF = T::TM + T::TN;
  static constexpr int MF = T::TM * T::TN;
  int wave, voff_b, a_row, b_row;
  int offs[4];
  uint4 raw[2][NF];
  v4i u[2][NF];

  __device__ __forceinline__ DmaCore() {
    const int lane = threadIdx.x & 63;
    // Wave-uniform by construction; readfirstlane lets the compiler keep the
    // DMA scalar offsets and LDS bases in SGPRs.
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
    const int h = lane >> 5, lr = lane & 31;
    voff_b = (lane >> 3) * 128 + dma_chunk16(wave, lane);
    a_row = (wm * T::WM + lr) * 128;
    b_row = (wn * T::WN + lr) * 128;
#pragma unroll
    for (int p = 0; p < 4; ++p) offs[p] = ((4 * h + p) ^ ((lr >> 1) & 7)) << 4;
  }

  // DMA of k-step kt (A rows and B panel) into `stage`.
  __device__ __forceinline__ void issue(char* stage, __amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                        int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps, int kt) {
    char* sb = stage + T::A_BYTES;
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) {
      const int q = wave + T::NW * ql;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(stage + q * 1024), 16, voff_a[ql],
                                               8 * q * a_q_stride + kt * 128, 0, 0);
    }
#pragma unroll
    for (int ql = 0; ql < T::B_INST; ++ql) {
      const int q = wave + T::NW * ql;
      const int blk = (8 * q) >> 7, row_in = (8 * q) & 127;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_ptr_t)(sb + q * 1024), 16, voff_b,
                                               (blk * ksteps + kt) * 16384 + row_in * 128, 0, 0);
    }
  }

  // DMA instruction `idx` of k-step kt (A slots first, then B slots).
  __device__ __forceinline__ void issue_one(char* stage, __amdgpu_buffer_rsrc_t a_rsrc,
                                            const int (&voff_a)[T::A_INST], int a_q_stride,
                                            __amdgpu_buffer_rsrc_t b_rsrc, int ksteps, int kt, int idx) {
    if (idx < T::A_INST) {
      const int q = wave + T::NW * idx;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(stage + q * 1024), 16, voff_a[idx],
                                               8 * q * a_q_stride + kt * 128, 0, 0);
    } else {
      const int q = wave + T::NW * (idx - T::A_INST);
      const int blk = (8 * q) >> 7, row_in = (8 * q) & 127;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_ptr_t)(stage + T::A_BYTES + q * 1024), 16, voff_b,
                                               (blk * ksteps + kt) * 16384 + row_in * 128, 0, 0);
    }
  }

  // Chunk pair p of fragment f of `stage` -> raw[buf][f].
  __device__ __forceinline__ void read_one(const char* stage, int buf, int p, int f) {
    raw[buf][f] = f < T::TM ? *reinterpret_cast<const uint4*>(stage + a_row + f * 4096 + offs[p])
                            : *reinterpret_cast<const uint4*>(stage + T::A_BYTES + b_row + (f - T::TM) * 4096 + offs[p]);
  }

  // Chunk pair p (substeps 2p, 2p+1) of every fragment of `stage` -> raw[buf].
  __device__ __forceinline__ void read(const char* stage, int buf, int p) {
    const char* sb = stage + T::A_BYTES;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
      raw[buf][i] = *reinterpret_cast<const uint4*>(stage + a_row + i * 4096 + offs[p]);
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      raw[buf][T::TM + j] = *reinterpret_cast<const uint4*>(sb + b_row + j * 4096 + offs[p]);
  }

  __device__ __forceinline__ void unpack_one(int dst, int buf, int half, int f) {
    u[dst][f] = half == 0 ? unpack_pair(raw[buf][f].x, raw[buf][f].y) : unpack_pair(raw[buf][f].z, raw[buf][f].w);
  }
  __device__ __forceinline__ void unpack(int dst, int buf, int half) {
#pragma unroll
    for (int f = 0; f < NF; ++f) unpack_one(dst, buf, half, f);
  }
  __device__ __forceinline__ void mma(v16i (&acc)[T::TM][T::TN], int src) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
  }

  // One substep on u[src] with the unpack of raw[buf] (half) into u[dst] for
  // the next substep (UNPACK = false: MFMAs only).
  //  kSchedPin: MFMA q is followed by the unpack of the fragments assigned to
  //    it (fragment f after MFMA f * MF / NF), each group fenced, so the MFMA
  //    stream never waits behind a block of VALU.
  //  kSchedHint: `reads` chunk reads first, then {1 MFMA, VPM VALU} repeated.
  template <bool UNPACK, int READS>
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
      mma(acc, src);
      if constexpr (UNPACK) unpack(dst, buf, half);
      if constexpr (T::SCHED == kSchedHint) {
        constexpr int VPM = (6 * NF + MF - 1) / MF + 1;
        if constexpr (READS > 0) __builtin_amdgcn_sched_group_barrier(0x100, READS, 0);
#pragma unroll
        for (int q = 0; q < MF; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
        }
      }
    }
  }

  // Pinned substep with memory work spread over the MFMA slots: after MFMA q
  // come the unpacks assigned to q and `extra(q)` (the chunk reads and DMA
  // instructions given to that slot). A wave that issues its LDS reads in a
  // burst stalls its own MFMA issue (measured: 8 back-to-back ds_read per 16
  // MFMAs cost a third of the MFMA rate on one wave per SIMD); one or two per
  // slot cost almost nothing.
  template <bool UNPACK, class Extra>
  __device__ __forceinline__ void substep_spread(v16i (&acc)[T::TM][T::TN], int src, int dst, int buf, int half,
                                                 Extra extra) {
#pragma unroll
    for (int q = 0; q < MF; ++q) {
      const int i = q / T::TN, j = q % T::TN;
      acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
      extra(q);
      if constexpr (UNPACK) {
#pragma unroll
        for (int f = 0; f < NF; ++f)
          if (f * MF / NF == q) unpack_one(dst, buf, half, f);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // extra(q) that reads chunk pair p of `stage` into raw[rbuf], fragment f
  // after MFMA f * MF / NF.
  struct SpreadReads {
    DmaCore* c;
    const char* stage;
    int rbuf, p;
    __device__ __forceinline__ void operator()(int q) const {
#pragma unroll
      for (int f = 0; f < NF; ++f)
        if (f * MF / NF == q) c->read_one(stage, rbuf, p, f);
    }
  };
  struct NoExtra {
    __device__ __forceinline__ void operator()(int) const {}
  };

  // Pairs 0..2 of a k-step read from `rd` (pair 0 already in raw[0] and its
  // even half in u[0]): each prefetches the next chunk pair, runs its two
  // substeps and unpacks ahead. Leaves pair 3 in raw[1], its even half in u[0].
  __device__ __forceinline__ void pairs012(v16i (&acc)[T::TM][T::TN], const char* rd) {
    if constexpr (T::SCHED == kSchedPin) {
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const int cur = p & 1;
        substep_spread<true>(acc, 0, 1, cur, 1, SpreadReads{this, rd, cur ^ 1, p + 1});
        substep_spread<true>(acc, 1, 0, cur ^ 1, 0, NoExtra{});
      }
      return;
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const int cur = p & 1;
      read(rd, cur ^ 1, p + 1);
      substep<true, NF>(acc, 0, 1, cur, 1);
      substep<true, 0>(acc, 1, 0, cur ^ 1, 0);
    }
  }
};

// The k-step bodies. LDS DMA is tracked by the same counter as other vector
// memory operations, and the compiler makes an LDS read wait for every
// outstanding DMA it cannot prove disjoint from it. Passing the stage being
// loaded and the stage being read as distinct restrict pointers of one
// inlined call is that proof: the prefetch then stays in flight across the
// whole k-step instead of being drained at the first read.

// k-step 0: DMA of k-steps 0 and 1, then pairs 0..2 of k-step 0.
template <class T>
__device__ __forceinline__ void dma_kstep_first(DmaCore<T>& c, v16i (&acc)[T::TM][T::TN],
                                                char* __restrict__ rd, char* __restrict__ dma,
                                                __amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                                int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps) {
  c.issue(rd, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, 0);
  c.issue(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, 1);
  wait_vmcnt<T::A_INST + T::B_INST>();
  __syncthreads();
  c.read(rd, 0, 0);
  c.unpack(0, 0, 0);
  c.pairs012(acc, rd);
  wait_vmcnt<0>();
  __syncthreads();
}

// k-step kt >= 1: DMA of k-step kt + 1 into the stage freed by k-step kt - 1,
// the last pair of k-step kt - 1 (registers only), then pairs 0..2 of k-step
// kt from `rd`; ends once the DMA of kt + 1 has landed and every wave is done
// reading `rd`.
template <class T>
__device__ __forceinline__ void dma_kstep_next(DmaCore<T>& c, v16i (&acc)[T::TM][T::TN],
                                               const char* __restrict__ rd, char* __restrict__ dma,
                                               __amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                               int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps,
                                               int kt) {
  if constexpr (T::SCHED == kSchedPin) {
    // The DMA instructions and the reads of pair 0 ride on the MFMA slots of
    // the previous k-step's last substep.
    constexpr int INST = T::A_INST + T::B_INST, MF = DmaCore<T>::MF, NF = DmaCore<T>::NF;
    auto extra = [&](int q) {
#pragma unroll
      for (int d = 0; d < INST; ++d)
        if (d * MF / INST == q) c.issue_one(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, kt + 1, d);
#pragma unroll
      for (int f = 0; f < NF; ++f)
        if (f * MF / NF == q) c.read_one(rd, 0, 0, f);
    };
    c.template substep_spread<true>(acc, 0, 1, 1, 1, extra);
    c.template substep_spread<true>(acc, 1, 0, 0, 0, typename DmaCore<T>::NoExtra{});
  } else {
    c.issue(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, kt + 1);
    c.read(rd, 0, 0);
    c.template substep<true, DmaCore<T>::NF>(acc, 0, 1, 1, 1);
    c.template substep<true, 0>(acc, 1, 0, 0, 0);
  }
  c.pairs012(acc, rd);
  wait_vmcnt<0>();
  __syncthreads();
}

// Full contraction over `ksteps` 256-k steps into acc (zeroed here). The
// DMA of k-step kt + 1 is issued at the start of k-step kt and waited for at
// its end; two LDS stages alternate. The body is branch-free (one basic block
// per k-step) so the accumulators stay in place: the last k-step also loads
// k-step `ksteps`, a range-checked buffer read (row padding, zeros or the next
// panel, never a fault) into a stage that is not read again, drained by the
// final wait.
template <class T>
__device__ __forceinline__ void dma_mainloop(__amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                             int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps,
                                             char* lds, v16i (&acc)[T::TM][T::TN]) {
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
  DmaCore<T> c;
  dma_kstep_first<T>(c, acc, lds, lds + T::STAGE_BYTES, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps);
  for (int kt = 1; kt < ksteps; ++kt) {
    char* rd = lds + (kt & 1) * T::STAGE_BYTES;
    char* dma = lds + ((kt & 1) ^ 1) * T::STAGE_BYTES;
    dma_kstep_next<T>(c, acc, rd, dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, kt);
  }
  // Last pair of the last k-step.
  c.template substep<true, 0>(acc, 0, 1, 1, 1);
  c.template substep<false, 0>(acc, 1, 0, 0, 0);
}

// INT8 operands (h3_gemm_i8_256): a 16-byte chunk read is one MFMA operand as
// it stands (16 int8 values per lane; lanes 32..63 read the chunk four
// positions further on, so one substep covers chunks p and 4 + p, 32 k
// values), the 128-byte row of a k-step holds 128 k values in four substeps,
// and the accumulator is the dot product itself. The DMA and LDS layout are
// those of the INT4 core.
template <class T>
__device__ __forceinline__ void mma8(DmaCore<T>& c, v16i (&acc)[T::TM][T::TN], int buf) {
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      acc[i][j] = mfma32_i8(__builtin_bit_cast(v4i, c.raw[buf][T::TM + j]), __builtin_bit_cast(v4i, c.raw[buf][i]),
                            acc[i][j]);
}

// 128-k step kt read from `rd` while k-step kt + 1 is loaded into `dma`.
template <class T>
__device__ __forceinline__ void dma8_kstep(DmaCore<T>& c, v16i (&acc)[T::TM][T::TN], const char* __restrict__ rd,
                                           char* __restrict__ dma, __amdgpu_buffer_rsrc_t a_rsrc,
                                           const int (&voff_a)[T::A_INST], int a_q_stride,
                                           __amdgpu_buffer_rsrc_t b_rsrc, int ksteps, int kt) {
  c.issue(dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, kt + 1);
  c.read(rd, 0, 0);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if (p < 3) c.read(rd, (p + 1) & 1, p + 1);
    mma8<T>(c, acc, p & 1);
  }
  wait_vmcnt<0>();
  __syncthreads();
}

// Full INT8 contraction over `ksteps` 128-k steps into acc (zeroed here); the
// last step's prefetch reads past the operands into a stage that is not read
// again (range-checked, as in dma_mainloop).
template <class T>
__device__ __forceinline__ void dma8_mainloop(__amdgpu_buffer_rsrc_t a_rsrc, const int (&voff_a)[T::A_INST],
                                              int a_q_stride, __amdgpu_buffer_rsrc_t b_rsrc, int ksteps,
                                              char* lds, v16i (&acc)[T::TM][T::TN]) {
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
  DmaCore<T> c;
  c.issue(lds, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, 0);
  wait_vmcnt<0>();
  __syncthreads();
  for (int kt = 0; kt < ksteps; ++kt) {
    char* rd = lds + (kt & 1) * T::STAGE_BYTES;
    char* dma = lds + ((kt & 1) ^ 1) * T::STAGE_BYTES;
    dma8_kstep<T>(c, acc, rd, dma, a_rsrc, voff_a, a_q_stride, b_rsrc, ksteps, kt);
  }
}

}  // namespace clef
