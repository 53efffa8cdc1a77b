// Persistent int4 x int4 -> i32 tile loop (gfx950): one workgroup walks a
// sequence of output tiles with a continuous DMA stream.
//
// Same arithmetic, LDS layout, k map and MFMA roles as dma_mainloop
// (gemm_dma.hpp). What changes is the tile boundary:
//  * the last two k-steps of tile t issue the DMA for the first two stages of
//    the workgroup's next tile (instead of over-issuing past K), so the next
//    tile's data is in flight during tile t's epilogue;
//  * the epilogue (a callback) stores straight from the accumulators with
//    exactly EPI_STORES vector-memory instructions per wave (buffer stores;
//    rows past the end fall outside the buffer range and are dropped), and
//    k-step 0 of the next tile waits with vmcnt(EPI_STORES): the stage-1 DMA
//    it needs was issued before those stores, so the stores drain under the
//    next tile's MFMAs instead of stalling it;
//  * the prologue waits for both first stages, so the first tile's k-step 0
//    needs no different wait.
// Requires ksteps >= 2. Every k-step body is branch-free; k-step 0 is peeled
// so each loop body keeps one basic block (and the accumulators in place).
#pragma once

#include <type_traits>

#include "gemm_dma.hpp"

namespace clef {

// Tile addressing. The dense GEMM's A offsets do not depend on the tile
// (a_rsrc starts at the tile's first row), so only the two buffer resources
// change from tile to tile: voff_a is shared, a_q_stride = row bytes.
struct TileRsrc {
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  __device__ __forceinline__ int voff(int, int shared_voff) const { return shared_voff; }
};
// Grouped experts gather rows: per-slot lane offsets change with the tile.
template <int A_INST>
struct TileGather {
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  int voff_a[A_INST];
  __device__ __forceinline__ int voff(int ql, int) const { return voff_a[ql]; }
};

// get(t) -> Addr of tile t; epi(t, acc) stores tile t. Tiles first,
// first + step, ... < count.
template <class T, int EPI_STORES, class Addr, class Get, class Epi>
__device__ __forceinline__ void persistent_loop(int first, int step, int count, int ksteps, int shared_voff,
                                                int a_q_stride, char* lds, Get get, Epi epi) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const int voff_b = (lane >> 3) * 128 + dma_chunk16(wave, lane);

  auto issue = [&](const Addr& ta, int kt, int stage) {
    char* sa = lds + stage * T::STAGE_BYTES;
    char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) {
      const int q = wave + T::NW * ql;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ta.a_rsrc, (lds_ptr_t)(sa + q * 1024), 16,
                                               ta.voff(ql, shared_voff), 8 * q * a_q_stride + kt * 128, 0, 0);
    }
#pragma unroll
    for (int ql = 0; ql < T::B_INST; ++ql) {
      const int q = wave + T::NW * ql;
      const int blk = (8 * q) >> 7, row_in = (8 * q) & 127;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ta.b_rsrc, (lds_ptr_t)(sb + q * 1024), 16, voff_b,
                                               (blk * ksteps + kt) * 16384 + row_in * 128, 0, 0);
    }
  };

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
  v16i acc[T::TM][T::TN];
  auto mma = [&](int src) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma32_i8(u[src][T::TM + j], u[src][i], acc[i][j]);
  };

  // One k-step: stage st of the current tile; the DMA for two steps ahead
  // goes to `ahead` at step kt_ahead. The last k-step of a tile (LAST) skips
  // the read and unpack of the next tile's first chunk pair, which happen after
  // the epilogue, so they hold no registers across it.
  auto kstep = [&](auto wait_n, auto last, int st, const Addr& ahead, int kt_ahead) {
    constexpr bool LAST = decltype(last)::value;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int cur = p & 1;
      if (p < 3) {
        read(cur ^ 1, st, p + 1);
      } else {
        wait_vmcnt<decltype(wait_n)::value>();
        __syncthreads();
        issue(ahead, kt_ahead, st);
        if (!LAST) read(cur ^ 1, st ^ 1, 0);
      }
      mma(0);
      unpack(1, cur, 1);
      mma(1);
      if (!LAST || p < 3) unpack(0, cur ^ 1, 0);
    }
  };
  using Yes = std::integral_constant<bool, true>;
  using No = std::integral_constant<bool, false>;

  Addr cur = get(first);
  issue(cur, 0, 0);
  issue(cur, 1, 1);
  wait_vmcnt<0>();
  __syncthreads();
  read(0, 0, 0);
  unpack(0, 0, 0);

  int g = 0;  // k-steps done by this workgroup: LDS stage parity
  for (int t = first; t < count; t += step) {
    const Addr nxt = t + step < count ? get(t + step) : cur;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
    // k-step 0: the only outstanding ops younger than its stage-1 DMA are
    // the previous epilogue's stores.
    kstep(std::integral_constant<int, EPI_STORES>{}, No{}, g & 1, 2 < ksteps ? cur : nxt,
          2 < ksteps ? 2 : 2 - ksteps);
    for (int kt = 1; kt + 1 < ksteps; ++kt) {
      const bool in_tile = kt + 2 < ksteps;
      kstep(std::integral_constant<int, 0>{}, No{}, (g + kt) & 1, in_tile ? cur : nxt,
            in_tile ? kt + 2 : kt + 2 - ksteps);
    }
    kstep(std::integral_constant<int, 0>{}, Yes{}, (g + ksteps - 1) & 1, nxt, 1);
    g += ksteps;
    epi(t, acc);
    // First chunk pair of the next tile (its stage landed before the last
    // k-step's barrier).
    read(0, g & 1, 0);
    unpack(0, 0, 0);
    cur = nxt;
  }
  wait_vmcnt<0>();
}

}  // namespace clef
