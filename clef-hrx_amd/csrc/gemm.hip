// G1 dense INT4 GEMM and E1 grouped expert INT4 GEMM for gfx950.
//
// G1 (kernels/gemm_integer.loom:394-433, identical in gemm_integer_m128.loom
// and gemm_integer_wide_k.loom): acc = sum_k a[m][k] * w[n][k] exact in i32;
// y = RN(RN(f32(acc) * ws[n]) * as[m]) + 0; finite y clamped to the bf16
// finite range; out = bf16(y); residual variant out = bf16(f32(res) + f32(out)).
//
// E1 (kernels/omni_expert_i4.loom:113-125, 436-462): for expert e and slot i,
// route = groups[e][1+i], xr = input_routed ? route : route / topk,
// out[route][c] = bf16(RN(f32(acc) * RN(as[xr] * ws[e*n + c]))), no clamp.

#include <atomic>

#include "silu_table.hpp"
#include "gemm_dma.hpp"
#include "gemm_dmah.hpp"
#include "expert_persist.hpp"
#include "group.hpp"
#include "kernels.hpp"
#include "launch.hpp"
#include "route.hpp"

namespace clef {

namespace {

template <int SHIFT = 8>
__device__ __forceinline__ uint32_t g1_value(int32_t acc, float ws, float as) {
  float y = (float)(acc >> SHIFT) * ws;
  y = y * as;
  y = y + 0.0f;
  float sat = __builtin_fmaxf(__builtin_fminf(y, kBf16Max), -kBf16Max);
  float checked = __builtin_fabsf(y) < __builtin_huge_valf() ? sat : y;
  return f32_to_bf16(checked);
}

// G1 epilogue for the 32x32 MFMA layout (lane: row m = l % 32; register r:
// column 8(r/4) + 4(l/32) + r%4).
//
// Values: fast path, taken when the whole wave qualifies: acc = 256 * dot
// exactly, so f32(acc) * (ws * 2^-8) rounds exactly like f32(dot) * ws
// whenever ws * 2^-8 is exact (every scale the quantizer produces; checked
// per column), and the bf16-range clamp cannot fire when
// 98 * K * max|ws| * max|as| < bf16 max (infinite or NaN scales pass the clamp
// unchanged in the reference too). Otherwise the general path runs the
// reference sequence step by step.
//
// Stores: each wave stages its WM x WN bf16 tile in LDS (free after the main
// loop; 8-byte blocks XOR-swizzled by row) and writes it back as 16-byte row
// chunks, 8 lanes per 128-byte line; the residual is added on that pass.
template <class T, bool RESID, int SHIFT = 8>
__device__ __forceinline__ void dense_epilogue(const v16i (&acc)[T::TM][T::TN], const float* __restrict__ as,
                                               const float* __restrict__ ws, int64_t M, int N, int K,
                                               int64_t m0, int n0, const uint16_t* __restrict__ residual,
                                               uint16_t* __restrict__ out, char* lds) {
  static_assert(T::WN >= 64 && T::NW * T::WM * T::WN * 2 <= T::LDS_BYTES, "LDS staging of the output tile");
  constexpr int RP = T::WN * 2;        // staged row pitch, bytes
  constexpr int LPR = T::WN / 8;       // lanes per row on the store pass
  constexpr int RPP = 64 / LPR;        // rows per store pass
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const float inf = __builtin_huge_valf();
  // acc holds 2^SHIFT * dot: 256 * dot for INT4 (16 * code bytes), the dot
  // itself for INT8. |dot| <= qmax^2 * K; the bound keeps a factor 2 margin.
  constexpr float kShiftScale = (float)(1 << SHIFT), kUnshift = 1.0f / kShiftScale;
  constexpr float kProdBound = SHIFT == 8 ? 98.0f : 32258.0f;

  float asr[T::TM];
  float mas = 0.0f;
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    const int64_t m = m0 + wm * T::WM + 32 * i + lr;
    asr[i] = m < M ? as[m] : 0.0f;
    const float a = __builtin_fabsf(asr[i]);
    mas = __builtin_fmaxf(mas, a < inf ? a : 0.0f);
  }
  float4 wsr[T::TN][4];
  float mws = 0.0f;
  bool exact = true;
#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + wn * T::WN + 32 * j + 8 * q + 4 * h;
      wsr[j][q] = *reinterpret_cast<const float4*>(ws + n);
      const float w4[4] = {wsr[j][q].x, wsr[j][q].y, wsr[j][q].z, wsr[j][q].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        exact = exact && (w4[e] * kUnshift) * kShiftScale == w4[e];
        const float a = __builtin_fabsf(w4[e]);
        mws = __builtin_fmaxf(mws, a < inf ? a : 0.0f);
      }
    }
  const bool fast = __all(exact && mws * mas * (kProdBound * (float)K) < kBf16Max);

  // All waves are done reading the pipeline stages before LDS is reused.
  __syncthreads();
  char* tile = lds + wave * (T::WM * T::WN * 2);
  auto stage = [&](int row, int col, uint32_t p0, uint32_t p1) {
    const int blk = (col >> 2) ^ (row & 15);
    *reinterpret_cast<uint2*>(tile + row * RP + blk * 8) = make_uint2(p0, p1);
  };
  // one copy of the loops per path (a wave-uniform flag tested inside them
  // is re-tested per value, a scheduling barrier each time)
  auto values = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) {
      const float asv = asr[i];
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 32 * i + lr, col = 32 * j + 8 * q + 4 * h;
          const float4 wsv = wsr[j][q];
          uint32_t p0, p1;
          if constexpr (FAST) {
            const float w4[4] = {wsv.x, wsv.y, wsv.z, wsv.w};
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              y[e] = (float)acc[i][j][4 * q + e] * (w4[e] * kUnshift);
              y[e] = y[e] * asv;
              y[e] = y[e] + 0.0f;
            }
            p0 = pack_bf16x2(y[0], y[1]);
            p1 = pack_bf16x2(y[2], y[3]);
          } else {
            p0 = g1_value<SHIFT>(acc[i][j][4 * q + 0], wsv.x, asv) | (g1_value<SHIFT>(acc[i][j][4 * q + 1], wsv.y, asv) << 16);
            p1 = g1_value<SHIFT>(acc[i][j][4 * q + 2], wsv.z, asv) | (g1_value<SHIFT>(acc[i][j][4 * q + 3], wsv.w, asv) << 16);
          }
          stage(row, col, p0, p1);
        }
    }
  };
  if (fast)
    values(std::true_type{});
  else
    values(std::false_type{});
  // Each wave reads back only its own region; the LDS ops of a wave complete
  // in order, so no barrier is needed between the two phases.
  const int c = lane % LPR;
#pragma unroll
  for (int pass = 0; pass < T::WM / RPP; ++pass) {
    const int row = RPP * pass + lane / LPR;
    const int x = row & 15;
    uint4 v = *reinterpret_cast<const uint4*>(tile + row * RP + ((c ^ (x >> 1)) << 4));
    if (x & 1) v = make_uint4(v.z, v.w, v.x, v.y);
    const int64_t m = m0 + wm * T::WM + row;
    if (m >= M) continue;
    const int64_t at = m * N + n0 + wn * T::WN + 8 * c;
    if (RESID) {
      const uint4 r = *reinterpret_cast<const uint4*>(residual + at);
      const uint32_t rv[4] = {r.x, r.y, r.z, r.w};
      uint32_t ov[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ov[t] = pack_bf16x2(bf16_lo(rv[t]) + bf16_lo(ov[t]), bf16_hi(rv[t]) + bf16_hi(ov[t]));
      v = make_uint4(ov[0], ov[1], ov[2], ov[3]);
    }
    *reinterpret_cast<uint4*>(out + at) = v;
  }
}


template <class T, bool RESID>
__global__ __launch_bounds__(T::THREADS) void gemm_dma_kernel(
    const uint32_t* __restrict__ a, int a_words, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, int64_t M, int N, int kb,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ out, int tiles_m, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)  // buffer-resource builtins exist only in the device pass
  extern __shared__ __align__(16) char lds[];
  int tm, tn;
  tile_of_block((int)blockIdx.x, (int)gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * T::BM;
  const int n0 = tn * T::BN;
  const int64_t rows_here = M - m0 < T::BM ? M - m0 : T::BM;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a + m0 * a_words, (uint32_t)(rows_here * a_words * 4));
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(w + (int64_t)(n0 / 128) * kb * 4096, (uint32_t)((T::BN / 128) * kb * 16384));
  v16i acc[T::TM][T::TN];
  int voff_a[T::A_INST];
  {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) voff_a[ql] = (lane >> 3) * a_words * 4 + dma_chunk16(wave, lane);
  }
  dma_mainloop<T>(a_rsrc, voff_a, a_words * 4, b_rsrc, kb, lds, acc);
  dense_epilogue<T, RESID>(acc, as, ws, M, N, kb * 256, m0, n0, residual, out, lds);
#endif
}

// INT8 x INT8 (h3_gemm_i8_256, kernels/gemm_integer.loom:454-485): the same
// tiles, DMA and G1 epilogue; `ksteps` 128-k steps of int8 codes.
template <class T, bool RESID>
__global__ __launch_bounds__(T::THREADS) void gemm_dma8_kernel(
    const uint32_t* __restrict__ a, int a_words, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, int64_t M, int N, int ksteps,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ out, int tiles_m, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
  extern __shared__ __align__(16) char lds[];
  int tm, tn;
  tile_of_block((int)blockIdx.x, (int)gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * T::BM;
  const int n0 = tn * T::BN;
  const int64_t rows_here = M - m0 < T::BM ? M - m0 : T::BM;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a + m0 * a_words, (uint32_t)(rows_here * a_words * 4));
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(w + (int64_t)(n0 / 128) * ksteps * 4096, (uint32_t)((T::BN / 128) * ksteps * 16384));
  v16i acc[T::TM][T::TN];
  int voff_a[T::A_INST];
  {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) voff_a[ql] = (lane >> 3) * a_words * 4 + dma_chunk16(wave, lane);
  }
  dma8_mainloop<T>(a_rsrc, voff_a, a_words * 4, b_rsrc, ksteps, lds, acc);
  dense_epilogue<T, RESID, 0>(acc, as, ws, M, N, ksteps * 128, m0, n0, residual, out, lds);
#endif
}

// Scales and fast-path flag of a G1 tile epilogue (epi_scales_from_lds).
template <class T>
struct EpiScales {
  float asr[T::TM];
  float4 wsr[T::TN][4];
  bool fast;
};

typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Bytes of LDS each wave uses to turn one 32-row block of its accumulators
// into whole output rows (32 rows of WN bf16).
template <class T>
constexpr int kEpiWaveLds = 32 * T::WN * 2;

// Scales of the staged epilogue, brought into the wave's LDS block by 4-byte
// LDS DMA instructions (64 scales each) issued with the tile's last k-step:
// the wave's WM row scales at byte 0 (rows past M read as zero) and its WN
// column scales at byte 512. They land with the k-step's own DMA, so the epilogue reads
// them from LDS instead of waiting on global loads.
template <class T>
__device__ __forceinline__ void epi_scales_dma(char* __restrict__ wlds, const float* __restrict__ as,
                                               const float* __restrict__ ws, int64_t M, int64_t m0, int n0) {
  static_assert(T::WM % 64 == 0 && T::WM <= 128 && T::WN % 64 == 0 && T::WN <= 128, "scale slots");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int64_t r0 = m0 + wm * T::WM;
  const int64_t rows = M - r0 <= 0 ? 0 : (M - r0 < T::WM ? M - r0 : T::WM);
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(as + r0, (uint32_t)(rows * 4));
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(ws + n0 + wn * T::WN, T::WN * 4);
#pragma unroll
  for (int r = 0; r < T::WM / 64; ++r)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(wlds + 256 * r), 4, lane * 4, 256 * r, 0, 0);
#pragma unroll
  for (int c = 0; c < T::WN / 64; ++c)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(wlds + 512 + 256 * c), 4, lane * 4, 256 * c, 0,
                                             0);
}

// Reads the scales placed by epi_scales_dma. `fast` (wave-uniform) holds when,
// over the wave's rows below M and its columns, every scale is finite and
// positive, ws * 2^-8 is exact, the largest product stays below bf16 max
// (as in epi_scales_finish) and ws * 2^-8 * as >= 2^-126. Then a nonzero
// accumulator never rounds to zero, so the "+ 0" of the G1 epilogue (which
// only turns -0 into +0) is the identity and is left out. With `fast` the
// column scales are returned already multiplied by 2^-8.
template <class T>
__device__ __forceinline__ EpiScales<T> epi_scales_from_lds(const char* __restrict__ wlds, int K, int64_t M,
                                                            int64_t m0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const float inf = __builtin_huge_valf();
  EpiScales<T> e;
  bool ok = true;
  float amax = 0.0f, amin = inf, wmax = 0.0f, wmin = inf;
#pragma unroll
  // The staged store overwrites this block (other lanes' rows) after these
  // reads, so every scale is pinned in a register: the compiler may not
  // re-read it from LDS later (per thread the location looks unchanged).
  for (int i = 0; i < T::TM; ++i) {
    e.asr[i] = *reinterpret_cast<const float*>(wlds + (32 * i + lr) * 4);
    pin_vgpr(e.asr[i]);
    const float a = e.asr[i];
    if (m0 + wm * T::WM + 32 * i + lr < M) {
      ok = ok && a > 0.0f && a < inf;
      amax = __builtin_fmaxf(amax, a);
      amin = __builtin_fminf(amin, a);
    }
  }
#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      e.wsr[j][q] = *reinterpret_cast<const float4*>(wlds + 512 + (32 * j + 8 * q + 4 * h) * 4);
      pin_vgpr(e.wsr[j][q].x);
      pin_vgpr(e.wsr[j][q].y);
      pin_vgpr(e.wsr[j][q].z);
      pin_vgpr(e.wsr[j][q].w);
      const float w4[4] = {e.wsr[j][q].x, e.wsr[j][q].y, e.wsr[j][q].z, e.wsr[j][q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        ok = ok && w4[t] > 0.0f && w4[t] < inf && (w4[t] * 0.00390625f) * 256.0f == w4[t];
        wmax = __builtin_fmaxf(wmax, w4[t]);
        wmin = __builtin_fminf(wmin, w4[t]);
      }
    }
  ok = ok && wmax * amax * (98.0f * (float)K) < kBf16Max && (wmin * 0.00390625f) * amin >= 0x1p-126f;
  e.fast = __all(ok);
  if (e.fast) {
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        e.wsr[j][q].x *= 0.00390625f;
        e.wsr[j][q].y *= 0.00390625f;
        e.wsr[j][q].z *= 0.00390625f;
        e.wsr[j][q].w *= 0.00390625f;
      }
  }
  return e;
}

// G1 tile epilogue through a wave-private LDS block: for each 32-row block i
// the wave writes its bf16 results (8 bytes per lane per 4 columns, 16-byte
// chunks XOR-swizzled by row within each 128-byte line), reads them back as
// 16 bytes of one row per lane and stores whole row segments of WN columns
// (TM * TN * 2 stores of 16 bytes per lane instead of TM * TN * 4 stores of
// 8 bytes across 32 rows). LDS
// operations of one wave execute in order, so block i + 1 may overwrite the
// rows block i has read without a barrier. Scales come from
// epi_scales_from_lds. Same values as dense_epilogue.
template <class T, bool RESID>
__device__ __forceinline__ void staged_epilogue_store(const v16i (&acc)[T::TM][T::TN], const EpiScales<T>& e,
                                                      int64_t M, int N, int64_t m0, int n0,
                                                      const uint16_t* __restrict__ residual,
                                                      uint16_t* __restrict__ out, char* __restrict__ wlds) {
  static_assert(T::WN == 64 || T::WN == 128, "one or two 128-byte lines per wave row");
  constexpr int kRowBytes = T::WN * 2, kLanesPerRow = T::WN / 8, kRowsPerRead = 64 / kLanesPerRow;
  constexpr int kReads = kEpiWaveLds<T> / 1024;  // 16-byte reads per lane per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const int64_t rows_here = M - m0 < T::BM ? M - m0 : T::BM;
  const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(out + m0 * N, (uint32_t)(rows_here * N * 2));
  const __amdgpu_buffer_rsrc_t res_rsrc =
      make_rsrc(RESID ? residual + m0 * N : out, RESID ? (uint32_t)(rows_here * N * 2) : 0u);
  // The lane's part of every store offset (the blocks' rows go in the scalar
  // part). Opaque to the compiler: otherwise it keeps one precomputed sum per
  // store across the persistent loop, runs out of registers and reloads them
  // from scratch in this epilogue, each reload followed by a wait for all
  // outstanding memory operations (the next tile's DMA included).
  const int lrow = lane / kLanesPerRow, lchunk = lane % kLanesPerRow;
  int voff = ((wm * T::WM + lrow) * N + n0 + wn * T::WN + 8 * lchunk) * 2;
  asm volatile("" : "+v"(voff));
  // one copy of the loops per path: a wave-uniform flag tested inside them
  // is re-tested per value, and each test is a scheduling barrier
  auto values = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) {
      const float asv = e.asr[i];
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 wsv = e.wsr[j][q];
          uint32_t p0, p1;
          if constexpr (FAST) {
            const float w4[4] = {wsv.x, wsv.y, wsv.z, wsv.w};
            float y[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              y[t] = (float)acc[i][j][4 * q + t] * w4[t];
              y[t] = y[t] * asv;
            }
            p0 = pack_bf16x2(y[0], y[1]);
            p1 = pack_bf16x2(y[2], y[3]);
          } else {
            p0 = g1_value(acc[i][j][4 * q + 0], wsv.x, asv) | (g1_value(acc[i][j][4 * q + 1], wsv.y, asv) << 16);
            p1 = g1_value(acc[i][j][4 * q + 2], wsv.z, asv) | (g1_value(acc[i][j][4 * q + 3], wsv.w, asv) << 16);
          }
          const int chunk = 4 * j + q;  // 16-byte chunk of the row: columns 8 * chunk .. + 7
          *reinterpret_cast<v2u*>(wlds + lr * kRowBytes + ((chunk ^ (lr & 7)) << 4) + 8 * h) = v2u{p0, p1};
        }
#pragma unroll
      for (int r = 0; r < kReads; ++r) {
        const int row = kRowsPerRead * r + lrow, chunk = lchunk;
        v4u v = *reinterpret_cast<const v4u*>(wlds + row * kRowBytes + ((chunk ^ (row & 7)) << 4));
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
  };
  if (e.fast)
    values(std::true_type{});
  else
    values(std::false_type{});
}

// Last k-step of one tile and first k-step of the next, in one inlined body
// so that `last` (read by the last k-step, then refilled with the next tile's
// k-step 1) and `first` (filled with the next tile's k-step 0 during the last
// k-step) are distinct restrict pointers throughout:
//   DMA this tile's scales -> wlds and next k0 -> first; last k-step from
//   `last`; drain + barrier; DMA next k1 -> last; last pair; epilogue through
//   the wave's LDS block `wlds`;
//   k-step 0 of the next tile from `first`, then wait only for the k1 DMA:
//   the epilogue's stores, issued after it, keep draining under the MFMAs.
template <class T, bool RESID>
__device__ __forceinline__ void gemm_tile_turn(DmaCore<T>& c, v16i (&acc)[T::TM][T::TN], char* __restrict__ last,
                                               char* __restrict__ first, __amdgpu_buffer_rsrc_t a_cur,
                                               __amdgpu_buffer_rsrc_t b_cur, __amdgpu_buffer_rsrc_t a_next,
                                               __amdgpu_buffer_rsrc_t b_next, const int (&voff_a)[T::A_INST],
                                               int a_q_stride, int ksteps, const float* __restrict__ as,
                                               const float* __restrict__ ws, int64_t M, int N, int64_t m0, int n0,
                                               const uint16_t* __restrict__ residual, uint16_t* __restrict__ out,
                                               char* __restrict__ wlds, bool more) {
  (void)a_cur;
  (void)b_cur;
  constexpr int INST = T::A_INST + T::B_INST, MF = DmaCore<T>::MF, NF = DmaCore<T>::NF;
  epi_scales_dma<T>(wlds, as, ws, M, m0, n0);
  if constexpr (T::SCHED == kSchedPin) {
    // The next tile's k-step-0 DMA and the reads of pair 0 ride on the MFMA
    // slots of the previous k-step's last substep, as in dma_kstep_next.
    auto extra = [&](int q) {
#pragma unroll
      for (int d = 0; d < INST; ++d)
        if (more && d * MF / INST == q) c.issue_one(first, a_next, voff_a, a_q_stride, b_next, ksteps, 0, d);
#pragma unroll
      for (int f = 0; f < NF; ++f)
        if (f * MF / NF == q) c.read_one(last, 0, 0, f);
    };
    c.template substep_spread<true>(acc, 0, 1, 1, 1, extra);
    c.template substep_spread<true>(acc, 1, 0, 0, 0, typename DmaCore<T>::NoExtra{});
  } else {
    if (more) c.issue(first, a_next, voff_a, a_q_stride, b_next, ksteps, 0);
    c.read(last, 0, 0);
    c.template substep<true, NF>(acc, 0, 1, 1, 1);
    c.template substep<true, 0>(acc, 1, 0, 0, 0);
  }
  c.pairs012(acc, last);
  wait_vmcnt<0>();
  __syncthreads();
  if constexpr (T::SCHED == kSchedPin) {
    auto extra = [&](int q) {
#pragma unroll
      for (int d = 0; d < INST; ++d)
        if (more && d * MF / INST == q) c.issue_one(last, a_next, voff_a, a_q_stride, b_next, ksteps, 1, d);
    };
    c.template substep_spread<true>(acc, 0, 1, 1, 1, extra);
  } else {
    if (more) c.issue(last, a_next, voff_a, a_q_stride, b_next, ksteps, 1);
    c.template substep<true, 0>(acc, 0, 1, 1, 1);
  }
  c.template substep<false, 0>(acc, 1, 0, 0, 0);
  const EpiScales<T> e = epi_scales_from_lds<T>(wlds, ksteps * 256, M, m0);
  // The scheduler must not start the next tile's MFMAs (fresh accumulators)
  // while this tile's accumulators are still being stored.
  __builtin_amdgcn_sched_barrier(0);
  staged_epilogue_store<T, RESID>(acc, e, M, N, m0, n0, residual, out, wlds);
  __builtin_amdgcn_sched_barrier(0);
  if (!more) return;
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
  c.read(first, 0, 0);
  c.unpack(0, 0, 0);
  c.pairs012(acc, first);
  // VMEM ops complete in issue order: with at most EPI outstanding, the k1
  // DMA issued before the epilogue's EPI loads and stores has landed.
  constexpr int EPI = T::TM * (kEpiWaveLds<T> / 1024) * (RESID ? 2 : 1);
  wait_vmcnt<(EPI < 63 ? EPI : 63)>();
  __syncthreads();
}

// Persistent G1 on the DMA core: a workgroup walks tiles b, b + grid, ...
// (grid a multiple of 8, so all of a workgroup's tiles map to its XCD). The
// last k-step of a tile loads the next tile's k-step 0 into the free stage
// while it computes, the epilogue goes through a 4 KiB LDS block per wave
// above the two stages, and the next tile starts on data already in LDS; the
// epilogue's stores drain under the next tile's first k-step. Needs
// ksteps >= 2.
template <class T, bool RESID>
__global__ __launch_bounds__(T::THREADS) void gemm_dma_persist_kernel(
    const uint32_t* __restrict__ a, int a_words, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, int64_t M, int N, int kb,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ out, int tiles_m, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
  extern __shared__ __align__(16) char lds[];
  const int total = tiles_m * tiles_n;  // below 2^31 (launch_dma_persist)
  int t = blockIdx.x;
  if (t >= total) return;
  struct Tile {
    __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
    int64_t m0;
    int n0;
  };
  auto tile = [&](int b) {
    int tm, tn;
    tile_of_block(b, total, tiles_m, tiles_n, tm, tn);
    Tile x;
    x.m0 = (int64_t)tm * T::BM;
    x.n0 = tn * T::BN;
    const int64_t rows_here = M - x.m0 < T::BM ? M - x.m0 : T::BM;
    x.a_rsrc = make_rsrc(a + x.m0 * a_words, (uint32_t)(rows_here * a_words * 4));
    x.b_rsrc = make_rsrc(w + (int64_t)(x.n0 / 128) * kb * 4096, (uint32_t)((T::BN / 128) * kb * 16384));
    return x;
  };
  int voff_a[T::A_INST];
  {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) voff_a[ql] = (lane >> 3) * a_words * 4 + dma_chunk16(wave, lane);
  }
  const int a_q_stride = a_words * 4;
  DmaCore<T> c;
  v16i acc[T::TM][T::TN];
  Tile cur = tile(t);
  int64_t g = 0;  // k-steps done by this workgroup: the stage of k-step kt is (g + kt) & 1
  auto stage = [&](int64_t i) { return lds + (int)(i & 1) * T::STAGE_BYTES; };
  auto zero = [&] {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};
  };
  zero();
  dma_kstep_first<T>(c, acc, stage(0), stage(1), cur.a_rsrc, voff_a, a_q_stride, cur.b_rsrc, kb);
  while (true) {
    const int tn_next = t + (int)gridDim.x;
    const bool has_next = tn_next < total;
    for (int kt = 1; kt + 1 < kb; ++kt)
      dma_kstep_next<T>(c, acc, stage(g + kt), stage(g + kt + 1), cur.a_rsrc, voff_a, a_q_stride, cur.b_rsrc, kb,
                        kt);
    const Tile nxt = tile(has_next ? tn_next : t);
    gemm_tile_turn<T, RESID>(c, acc, stage(g + kb - 1), stage(g + kb), cur.a_rsrc, cur.b_rsrc, nxt.a_rsrc,
                             nxt.b_rsrc, voff_a, a_q_stride, kb, as, ws, M, N, cur.m0, cur.n0, residual, out,
                             lds + T::LDS_BYTES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * kEpiWaveLds<T>,
                             has_next);
    if (!has_next) break;
    g += kb;
    t = tn_next;
    cur = nxt;
  }
#endif
}

template <class T, bool RESID>
hipError_t launch_dma_persist(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                              int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  constexpr int kPersistLds = T::LDS_BYTES + T::NW * kEpiWaveLds<T>;
  static_assert(kPersistLds <= 160 * 1024, "LDS per workgroup");
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&gemm_dma_persist_kernel<T, RESID>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, kPersistLds)) return e;
  int per_cu = 0, cus = 0;
  if (hipError_t e = resident_per_cu(cache, kern, T::THREADS, kPersistLds, per_cu, cus)) return e;
  const int tiles_n = n / T::BN;
  const int64_t tiles_m = (m + T::BM - 1) / T::BM;
  const int64_t total = tiles_m * tiles_n;
  if (total > kMaxTiles) return hipErrorInvalidValue;  // the kernel's 32-bit tile indices
  int64_t grid = (int64_t)cus * per_cu / 8 * 8;
  if (grid < 8) grid = 8;
  if (grid > total) grid = total;
  gemm_dma_persist_kernel<T, RESID><<<(unsigned)grid, T::THREADS, kPersistLds, stream>>>(
      a, a_words, as, w, ws, m, n, k / 256, residual, out, (int)tiles_m, tiles_n);
  return hipGetLastError();
}

template <class T>
hipError_t launch_dma_persist_any(const uint32_t* a, int a_words, const float* as, const uint32_t* w,
                                  const float* ws, int64_t m, int n, int k, const uint16_t* residual, uint16_t* out,
                                  hipStream_t stream) {
  if (residual) return launch_dma_persist<T, true>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_dma_persist<T, false>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

template <class T, bool RESID>
hipError_t launch_dma(const uint32_t* a, int a_words, const float* as, const uint32_t* w,
                      const float* ws, int64_t m, int n, int k, const uint16_t* residual,
                      uint16_t* out, hipStream_t stream) {
  const void* kern = reinterpret_cast<const void*>(&gemm_dma_kernel<T, RESID>);
  static LaunchCache cache;
  if (hipError_t e = ensure_dynamic_lds(cache, kern, T::LDS_BYTES)) return e;
  const int tiles_n = n / T::BN;
  const int64_t tiles_m = (m + T::BM - 1) / T::BM;
  gemm_dma_kernel<T, RESID><<<(unsigned)(tiles_m * tiles_n), T::THREADS, T::LDS_BYTES, stream>>>(
      a, a_words, as, w, ws, m, n, k / 256, residual, out, (int)tiles_m, tiles_n);
  return hipGetLastError();
}

template <class T>
hipError_t launch_dma_any(const uint32_t* a, int a_words, const float* as, const uint32_t* w,
                          const float* ws, int64_t m, int n, int k, const uint16_t* residual,
                          uint16_t* out, hipStream_t stream) {
  if (residual) return launch_dma<T, true>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_dma<T, false>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

template <class T, bool RESID>
hipError_t launch_dma8(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                       int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&gemm_dma8_kernel<T, RESID>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, T::LDS_BYTES)) return e;
  const int tiles_n = n / T::BN;
  const int64_t tiles_m = (m + T::BM - 1) / T::BM;
  gemm_dma8_kernel<T, RESID><<<(unsigned)(tiles_m * tiles_n), T::THREADS, T::LDS_BYTES, stream>>>(
      a, a_words, as, w, ws, m, n, k / 128, residual, out, (int)tiles_m, tiles_n);
  return hipGetLastError();
}

template <class T>
hipError_t launch_dma8_any(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                           int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (residual) return launch_dma8<T, true>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_dma8<T, false>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

// G1 tiles: 128x128 on four 64x64 waves (compiler-hinted MFMA/unpack
// interleave), and 256x256 on eight 128x64 waves with the pinned schedule
// (one workgroup per tile, or persistent). INT8 uses the eight-wave tile with
// the compiler's own schedule.
using Dma128x128 = DmaTile<64, 64, 2, 2>;
using Dma256x256W8 = DmaTile<128, 64, 2, 4, kSchedFree>;
using Dma256x256W8Pin = DmaTile<128, 64, 2, 4, kSchedPin>;

// ---------------------------------------------------------------- experts

constexpr int kExpertBM = 128;

// Per-expert tile list: list[0] = tiles, then from list[HEAD] (expert, first
// slot) pairs for experts ascending and tiles of bm slots each. The expert
// GEMM schedule (int32, HEAD = kSchedEntries) also gets its work counters
// zeroed. With bm = 16, float output and HEAD = 1 the same walk is the
// reference task list R3 (kernels/omni_expert_tasks.loom:30-62).
template <class OutT, int HEAD>
__global__ __launch_bounds__(128) void tile_list_kernel(const float* __restrict__ groups,
                                                        int64_t tokens, int bm, OutT* __restrict__ list) {
  __shared__ int scan[128];
  if (HEAD > 1 && threadIdx.x < HEAD - 1) list[1 + threadIdx.x] = (OutT)0;
  const int e = threadIdx.x;
  const int count = (int)groups[(int64_t)e * (tokens + 1)];
  const int tiles = (count + bm - 1) / bm;
  scan[e] = tiles;
  __syncthreads();
  for (int off = 1; off < 128; off <<= 1) {
    const int v = e >= off ? scan[e - off] : 0;
    __syncthreads();
    scan[e] += v;
    __syncthreads();
  }
  // scan[e] is now the inclusive prefix: expert e owns tiles
  // scan[e] - tiles .. scan[e] - 1. Every thread writes entries; tile t's
  // expert is the first whose inclusive prefix exceeds t (one expert can own
  // hundreds of tiles under skewed routing).
  const int total = scan[127];
  for (int t = e; t < total; t += 128) {
    int lo = 0, hi = 127;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (scan[mid] > t)
        hi = mid;
      else
        lo = mid + 1;
    }
    const int first = lo > 0 ? scan[lo - 1] : 0;
    list[HEAD + 2 * t] = (OutT)lo;
    list[HEAD + 1 + 2 * t] = (OutT)((t - first) * bm);
  }
  if (e == 127) list[0] = (OutT)total;
}

// Grouped expert GEMM on the half-k-step core: 128 expert slots x 256 weight
// rows per workgroup, four 64 x 128 waves, two workgroups per CU.
//  GU = false: E1 over 256 output columns of one weight set.
//  GU = true:  the fused gate/up/SwiGLU producer: weight rows are 128 gate
//    rows and the same 128 up rows; each lane holds gate and up of the same
//    output column, applies E1 to both (bf16), then S1, and writes h.
// A wave whose 64 slots are all past the expert's count runs the DMA and
// barrier schedule only.
// Work items are (schedule tile, column block) pairs in expert-major order.
// Block b runs on XCD b % 8 (round-robin dispatch); XCD x takes the
// contiguous item range [x * C, (x + 1) * C), so the row tiles of one expert
// and weight panel run together on one XCD and share the panel in its L2.
// The grid is a multiple of 8 and covers 8 * C items. A rows are gathered:
// each DMA lane's offset is its slot's row (route / topk, or route for routed
// input); slots past the expert's count get an out-of-range offset (2^31 >=
// the buffer size, checked by the launcher) and read zeros.

using ExpertHTile = DmaHTile<64, 128, 2, 2, kSchedFree, false>;
using ExpertGUTile = DmaHTile<64, 128, 2, 2, kSchedFree, true>;
static_assert(ExpertHTile::BM == kExpertBM && ExpertGUTile::BM == kExpertBM, "expert schedule tile height");

// Dynamic LDS of expert_dmah_kernel: stages / staged output, the SiLU table
// (GU), the slots' routes and the tile's weight scales.
template <class T, bool GU>
constexpr int expert_lds_bytes() {
  constexpr int cols = GU ? T::BN / 2 : T::BN;
  constexpr int base = GU ? 2 * T::STAGE_BYTES + kSiluLutSize * 2
                          : (T::LDS_BYTES > 2 * T::STAGE_BYTES ? T::LDS_BYTES : 2 * T::STAGE_BYTES);
  return base + T::BM * 4 + (GU ? 2 : 1) * (cols * 4 > 1024 ? cols * 4 : 1024);
}

template <class T, bool GU>
__global__ __launch_bounds__(T::THREADS, 2) void expert_dmah_kernel(
    const uint32_t* __restrict__ a, int a_words, uint32_t a_bytes, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, const uint32_t* __restrict__ w2,
    const float* __restrict__ ws2, const float* __restrict__ groups, const int32_t* __restrict__ schedule,
    int64_t list_stride, int topk, int kb, int n, int input_routed, uint16_t* __restrict__ out, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
  extern __shared__ __align__(16) char lds[];
  const int64_t items = (int64_t)schedule[0] * tiles_n;
  const int64_t chunk = (items + 7) / 8;
  const int64_t local = blockIdx.x / 8;
  if (local >= chunk) return;
  const int64_t item = (blockIdx.x % 8) * chunk + local;
  if (item >= items) return;
  const int tile = (int)(item / tiles_n);
  const int tn = (int)(item - (int64_t)tile * tiles_n);
  const int e = schedule[kSchedEntries + 2 * tile];
  const int row0 = schedule[kSchedEntries + 1 + 2 * tile];
  const float* list = groups + (int64_t)e * list_stride;
  const int count = (int)list[0];
  constexpr int COLS = GU ? T::BN / 2 : T::BN;  // output columns per tile
  const int n0 = tn * COLS;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;

  // LDS: the two stages (the staged output tile reuses them), then for GU the
  // SiLU table, then per-tile metadata: the 128 slots' routes (int) and the
  // tile's weight scales (f32, COLS each for gate and up).
  constexpr int LUT_OFF = 2 * T::STAGE_BYTES;
  constexpr int META_OFF = GU ? LUT_OFF + kSiluLutSize * 2 : (T::LDS_BYTES > LUT_OFF ? T::LDS_BYTES : LUT_OFF);
  constexpr int WS_SLOT = COLS * 4 > 1024 ? COLS * 4 : 1024;
  int* routes_lds = reinterpret_cast<int*>(lds + META_OFF);
  char* ws_lds = lds + META_OFF + T::BM * 4;
  // Weight scales of the tile's columns by DMA (1 KiB per instruction).
  {
    // A DMA instruction writes 1 KiB whatever the source range (lanes past
    // it write zeros), so each scale vector gets a whole 1 KiB slot.
    constexpr int WS_INST = COLS * 4 / 1024 > 0 ? COLS * 4 / 1024 : 1;
    static_assert(COLS * 4 % 1024 == 0 || COLS * 4 == 512, "scale DMA granularity");
    const uint32_t ws_bytes = COLS * 4;
    const __amdgpu_buffer_rsrc_t ws_rsrc = make_rsrc(ws + (int64_t)e * n + n0, ws_bytes);
    const __amdgpu_buffer_rsrc_t ws2_rsrc = make_rsrc((GU ? ws2 : ws) + (int64_t)e * n + n0, ws_bytes);
    if (wave < WS_INST)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ws_rsrc, (lds_ptr_t)(ws_lds + wave * 1024), 16, lane * 16,
                                               wave * 1024, 0, 0);
    if (GU && wave >= 2 && wave < 2 + WS_INST)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ws2_rsrc, (lds_ptr_t)(ws_lds + WS_SLOT + (wave - 2) * 1024), 16,
                                               lane * 16, (wave - 2) * 1024, 0, 0);
  }
  int voff_a[T::A_INST];
#pragma unroll
  for (int ql = 0; ql < T::A_INST; ++ql) {
    const int r = 16 * (wave + T::NW * ql) + (lane >> 2);
    const int slot = row0 + r;
    int route = -1;
    if (slot < count) {
      route = (int)list[1 + slot];
      const int64_t xr = input_routed ? (int64_t)route : (int64_t)route / topk;
      voff_a[ql] = (int)(xr * a_words * 4) + dmah_chunk16(lane);
    } else {
      voff_a[ql] = (int)0x80000000u;
    }
    if ((lane & 3) == 0) routes_lds[r] = route;
  }
  // The SiLU table goes to LDS after the two stages; its DMA is issued before
  // the stages', so the main loop's first wait covers it.
  if constexpr (GU) {
    static_assert(LUT_OFF + kSiluLutSize * 2 <= T::LDS_BYTES, "SiLU table in LDS");
    const __amdgpu_buffer_rsrc_t lut_rsrc = make_rsrc(g_silu_lut, kSiluLutSize * 2);
#pragma unroll
    for (int i = 0; i < kSiluLutSize * 2 / 1024 / T::NW; ++i) {
      const int q = wave * (kSiluLutSize * 2 / 1024 / T::NW) + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(lut_rsrc, (lds_ptr_t)(lds + LUT_OFF + q * 1024), 16, lane * 16,
                                               q * 1024, 0, 0);
    }
  }
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, a_bytes);
  const int64_t blk0 = ((int64_t)e * n + n0) / 128;
  const uint32_t b_bytes = (uint32_t)((COLS / 128) * kb * 16384);
  const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(w + blk0 * kb * 4096, b_bytes);
  const __amdgpu_buffer_rsrc_t b_rsrc2 = GU ? make_rsrc(w2 + blk0 * kb * 4096, b_bytes) : b_rsrc;
  // Epilogue inputs that depend on a chain of loads (slot -> route -> scale)
  // are fetched before the main loop.
  const int h = lane >> 5, lr = lane & 31;
  float asr[T::TM];
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    const int slot = row0 + wm * T::WM + 32 * i + lr;
    asr[i] = 0.0f;
    if (slot < count) {
      const int64_t route = (int64_t)list[1 + slot];
      asr[i] = as[input_routed ? route : route / topk];
    }
  }
  v16i acc[T::TM][T::TN];
  if (row0 + wm * T::WM < count)
    dmah_mainloop<T, true>(a_rsrc, voff_a, 0, b_rsrc, b_rsrc2, kb, lds, acc);
  else
    dmah_mainloop<T, false>(a_rsrc, voff_a, 0, b_rsrc, b_rsrc2, kb, lds, acc);

  // Values -> bf16 tile in LDS (over the drained stages; rows of COLS * 2
  // bytes, 8-byte blocks XOR-swizzled by row), then whole 16-byte row pieces
  // to the routed output rows.
  static_assert(T::BM * COLS * 2 <= (GU ? 2 * T::STAGE_BYTES : T::LDS_BYTES), "staged output tile");
  constexpr int RP = COLS * 2;  // staged row pitch, bytes
  __syncthreads();              // every wave is done with the stages
  auto stage = [&](int row, int col, uint32_t p0, uint32_t p1) {
    const int blk = (col >> 2) ^ (row & 15);
    *reinterpret_cast<uint2*>(lds + row * RP + blk * 8) = make_uint2(p0, p1);
  };
  constexpr int JN = GU ? T::TN / 2 : T::TN;  // output fragments per lane row
  // f32(acc) is 256 * dot exactly (dot has at most 17 significant bits).
  // When every row and column scale of the tile is at least 2^-59, the row
  // scale taken times 2^-8 gives RN(asr * w) * 2^-8 exactly (all normal), so
  // RN(f32(acc) * RN(asr * 2^-8 * w)) = RN(dot * RN(asr * w)) and the shift
  // by 8 is not needed; otherwise the shift path runs. Only the gate/up
  // epilogue (two accumulators per output) gains more than the check costs.
  bool fast = false;
  if constexpr (GU) {
    constexpr float kMinScale = 0x1p-59f;
    bool ok = true;
#pragma unroll
    for (int i = 0; i < T::TM; ++i)  // rows past the group's end are never stored
      ok = ok && (row0 + wm * T::WM + 32 * i + lr >= count || asr[i] >= kMinScale);
    // each wave checks all of the tile's column scales (COLS per matrix)
#pragma unroll
    for (int c = lane; c < COLS; c += 64) {
      ok = ok && *reinterpret_cast<const float*>(ws_lds + c * 4) >= kMinScale;
      if constexpr (GU) ok = ok && *reinterpret_cast<const float*>(ws_lds + WS_SLOT + c * 4) >= kMinScale;
    }
    fast = __all(ok);
  }
  float asr8[T::TM];
#pragma unroll
  for (int i = 0; i < T::TM; ++i) asr8[i] = asr[i] * 0x1p-8f;
  // The epilogue body for one value of `fast` (wave-uniform, so one branch
  // instead of a select per value).
  auto values = [&](auto fast_tag) {
    constexpr bool FAST = decltype(fast_tag)::value;
    auto scaled = [&](int i, int jj, int r, float w) -> float {
      const int a = acc[i][jj][r];
      return FAST ? (float)a * (asr8[i] * w) : (float)(a >> 8) * (asr[i] * w);
    };
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wn * (GU ? T::WN / 2 : T::WN) + 32 * j + 8 * q + 4 * h;  // within the tile
        const float4 wsv = *reinterpret_cast<const float4*>(ws_lds + col * 4);
        float4 wsu = wsv;
        if constexpr (GU) wsu = *reinterpret_cast<const float4*>(ws_lds + WS_SLOT + col * 4);
        const float wg[4] = {wsv.x, wsv.y, wsv.z, wsv.w}, wu[4] = {wsu.x, wsu.y, wsu.z, wsu.w};
        float y[T::TM][4];
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t) y[i][t] = scaled(i, j, 4 * q + t, wg[t]);
        if constexpr (GU) {
          // bf16(g) two per register, SiLU from the LDS table for all 4 * TM
          // values at once (their reads overlap), then one wave-uniform branch
          // for the rare values outside the table, computed directly.
          uint32_t gp[T::TM][2];
          float act[T::TM][4];
          uint32_t outside = 0;
#pragma unroll
          for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              gp[i][p] = pack_bf16x2(y[i][2 * p], y[i][2 * p + 1]);
              // rows past the group's end (never stored) read as zero, which
              // lies outside the table: give them 1.0 instead
              if (row0 + wm * T::WM + 32 * i + lr >= count) gp[i][p] = 0x3F803F80u;
              const uint32_t off = silu_lut_offset2(gp[i][p], outside);
              act[i][2 * p] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(lds + LUT_OFF + (off & 0xFFFFu)));
              act[i][2 * p + 1] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(lds + LUT_OFF + (off >> 16)));
            }
          if (__any(outside != 0)) {
            // silu(+-0) = +-0 (integer dot products are often zero): those
            // directly, then the others outside the table only if there are any
            bool others = false;
#pragma unroll
            for (int i = 0; i < T::TM; ++i)
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const uint32_t gb = (t & 1) ? gp[i][t >> 1] >> 16 : gp[i][t >> 1] & 0xFFFFu;
                const bool out = ((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0;
                if (out && (gb & 0x7FFFu) == 0) act[i][t] = bf16_to_f32(gb);
                others = others | (out & ((gb & 0x7FFFu) != 0));
              }
            if (__any(others)) {
#pragma unroll
              for (int i = 0; i < T::TM; ++i)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                  const uint32_t gb = (t & 1) ? gp[i][t >> 1] >> 16 : gp[i][t >> 1] & 0xFFFFu;
                  if ((((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0) & ((gb & 0x7FFFu) != 0))
                    act[i][t] = silu_bf16(bf16_to_f32(gb));
                }
            }
          }
          // h = bf16(act * bf16(u)), u rounded two per register; the packing
          // below rounds h to bf16
#pragma unroll
          for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const uint32_t up = pack_bf16x2(scaled(i, j + JN, 4 * q + 2 * p, wu[2 * p]),
                                              scaled(i, j + JN, 4 * q + 2 * p + 1, wu[2 * p + 1]));
              y[i][2 * p] = act[i][2 * p] * bf16_lo(up);
              y[i][2 * p + 1] = act[i][2 * p + 1] * bf16_hi(up);
            }
        }
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
          stage(wm * T::WM + 32 * i + lr, col, pack_bf16x2(y[i][0], y[i][1]), pack_bf16x2(y[i][2], y[i][3]));
      }
  };
  if (GU && fast)
    values(std::true_type{});
  else
    values(std::false_type{});
  __syncthreads();
  constexpr int LPR = COLS / 8;              // lanes per row (16 bytes each)
  constexpr int RPP = T::THREADS / LPR;      // rows per pass
  const int c = threadIdx.x % LPR;
#pragma unroll
  for (int pass = 0; pass < T::BM / RPP; ++pass) {
    const int row = RPP * pass + threadIdx.x / LPR;
    const int route = routes_lds[row];
    if (route < 0) continue;
    const int x = row & 15;
    uint4 v = *reinterpret_cast<const uint4*>(lds + row * RP + ((c ^ (x >> 1)) << 4));
    if (x & 1) v = make_uint4(v.z, v.w, v.x, v.y);
    *reinterpret_cast<uint4*>(out + (int64_t)route * n + n0 + 8 * c) = v;
  }
#endif
}

template <class T, bool GU>
hipError_t launch_expert_dmah(const uint32_t* a, int a_words, int64_t a_bytes, const float* as, const uint32_t* w,
                              const float* ws, const uint32_t* w2, const float* ws2, const float* groups,
                              const int32_t* schedule, int64_t routes, int64_t list_stride, int topk, int k, int n,
                              int input_routed, uint16_t* out, hipStream_t stream);

// Small-M G1: with few activation rows the weight stream is the whole cost,
// and N / 128 workgroups walking all of K leave most of the GPU and of HBM
// idle. Here a workgroup of NW waves (16, or 8 with four row blocks) owns 32
// output columns and up to 32 * MT rows, and the waves split the k-steps
// between them. Each wave loads its 32
// weight rows and MT * 32 activation rows straight into registers (64 bytes
// per lane per row block per k-step: lane half h takes chunks 4h .. 4h+3 of
// the row's 128-byte k-step, the lane -> k map of the LDS cores) with the
// next k-step's loads in flight while the current one computes. The NW
// partial accumulators meet in LDS by integer atomic adds (exact in any
// order), and the G1 epilogue runs on the sums. I8: INT8 operands (k-steps of
// 128 k, the same 64 bytes per lane; each 16-byte chunk is an MFMA operand as
// it stands, and the accumulator is the dot product itself).
template <int MT, int NW, bool RESID, bool I8>
__global__ __launch_bounds__(NW * 64) void gemm_skinny_kernel(const uint32_t* __restrict__ a, int a_words,
                                                          const float* __restrict__ as, const uint32_t* __restrict__ w,
                                                          const float* __restrict__ ws, int64_t M, int N, int kb,
                                                          const uint16_t* __restrict__ residual,
                                                          uint16_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
  __shared__ int red[MT][16][64];  // [row block][accumulator register][lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 32;
  const int64_t m0 = (int64_t)blockIdx.y * (32 * MT);
  const int64_t rows = M - m0 < 32 * MT ? M - m0 : 32 * MT;
  for (int i = threadIdx.x; i < MT * 16 * 64; i += NW * 64) (&red[0][0][0])[i] = 0;

  // Weight row n0 + lr of k-step kt: tiled block (n / 128, kt), row n % 128.
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (int64_t)(n0 / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const int w_voff = ((n0 % 128) + lr) * 128 + 64 * h;
  // Activation rows past M read as zero (outside the resource's range).
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a + m0 * a_words, (uint32_t)(rows * a_words * 4));
  int a_voff[MT];
#pragma unroll
  for (int f = 0; f < MT; ++f) a_voff[f] = (32 * f + lr) * a_words * 4 + 64 * h;

  v16i acc[MT];
#pragma unroll
  for (int f = 0; f < MT; ++f) acc[f] = v16i{};
  v4i wr[2][4], ar[2][MT][4];
  auto load = [&](auto buf, int kt) {
    constexpr int B = decltype(buf)::value;
#pragma unroll
    for (int c = 0; c < 4; ++c) wr[B][c] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 16 * c, kt * 16384, 0);
#pragma unroll
    for (int f = 0; f < MT; ++f)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        ar[B][f][c] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff[f] + 16 * c, kt * 128, 0);
  };
  auto compute = [&](auto buf) {
    constexpr int B = decltype(buf)::value;
    if constexpr (I8) {
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int f = 0; f < MT; ++f) acc[f] = mfma32_i8(wr[B][p], ar[B][f][p], acc[f]);
      return;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const v4i& x = wr[B][p];
        const v4i uw = half ? unpack_pair(x.z, x.w) : unpack_pair(x.x, x.y);
#pragma unroll
        for (int f = 0; f < MT; ++f) {
          const v4i& y = ar[B][f][p];
          const v4i ua = half ? unpack_pair(y.z, y.w) : unpack_pair(y.x, y.y);
          acc[f] = mfma32_i8(uw, ua, acc[f]);
        }
      }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Epilogue item g = (row block f, register quad rq, lane) gives row
  // m0 + 32 f + lane % 32 and columns n0 + 8 rq + 4 (lane / 32) + 0..3. Its
  // scales (and residual) are fetched here, with the first loads, so their
  // latency is not paid again after the reduction; with more than one row
  // block there is no register room for them (the kernel would spill).
  constexpr int IPT = (MT * 256 + NW * 64 - 1) / (NW * 64);
  constexpr bool PRE = MT == 1;
  float e_as[IPT];
  float4 e_ws[IPT];
  uint2 e_res[IPT];
#pragma unroll
  for (int i = 0; i < IPT && PRE; ++i) {
    const int g = threadIdx.x + i * NW * 64;
    const int f = g >> 8, rq = (g >> 6) & 3, ln = g & 63;
    const int64_t m = m0 + 32 * f + (ln & 31);
    const int col = n0 + 8 * rq + 4 * (ln >> 5);
    const bool ok = g < MT * 256 && m < M;
    e_as[i] = ok ? as[m] : 0.0f;
    e_ws[i] = ok ? *reinterpret_cast<const float4*>(ws + col) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    e_res[i] = RESID && ok ? *reinterpret_cast<const uint2*>(residual + m * N + col) : make_uint2(0, 0);
  }
  const int k0 = wave * kb / NW, k1 = (wave + 1) * kb / NW;
  if (k0 < k1) {
    // The load after the last k-step repeats it (never used), so the body has
    // no branch around its loads and the waits stay exact.
    load(B0{}, k0);
    for (int kt = k0;;) {
      load(B1{}, kt + 1 < k1 ? kt + 1 : kt);
      compute(B0{});
      if (++kt >= k1) break;
      load(B0{}, kt + 1 < k1 ? kt + 1 : kt);
      compute(B1{});
      if (++kt >= k1) break;
    }
  }
  __syncthreads();  // reduction buffer zeroed
#pragma unroll
  for (int f = 0; f < MT; ++f)
#pragma unroll
    for (int r = 0; r < 16; ++r) atomicAdd(&red[f][r][lane], acc[f][r]);
  __syncthreads();

#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int g = threadIdx.x + i * NW * 64;
    const int f = g >> 8, rq = (g >> 6) & 3, ln = g & 63;
    const int64_t m = m0 + 32 * f + (ln & 31);
    if (g >= MT * 256 || m >= M) continue;
    const int col = n0 + 8 * rq + 4 * (ln >> 5);
    const float asv = PRE ? e_as[i] : as[m];
    const float4 wsv = PRE ? e_ws[i] : *reinterpret_cast<const float4*>(ws + col);
    constexpr int SH = I8 ? 0 : 8;
    uint32_t p0 = g1_value<SH>(red[f][4 * rq + 0][ln], wsv.x, asv) | (g1_value<SH>(red[f][4 * rq + 1][ln], wsv.y, asv) << 16);
    uint32_t p1 = g1_value<SH>(red[f][4 * rq + 2][ln], wsv.z, asv) | (g1_value<SH>(red[f][4 * rq + 3][ln], wsv.w, asv) << 16);
    uint16_t* dst = out + m * N + col;
    if (RESID) {
      const uint2 rv = PRE ? e_res[i] : *reinterpret_cast<const uint2*>(residual + m * N + col);
      p0 = pack_bf16x2(bf16_lo(rv.x) + bf16_lo(p0), bf16_hi(rv.x) + bf16_hi(p0));
      p1 = pack_bf16x2(bf16_lo(rv.y) + bf16_lo(p1), bf16_hi(rv.y) + bf16_hi(p1));
    }
    *reinterpret_cast<uint2*>(dst) = make_uint2(p0, p1);
  }
#endif
}

template <int MT, bool RESID, bool I8>
hipError_t launch_skinny(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                         int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  const int64_t groups = (m + 32 * MT - 1) / (32 * MT);
  if (groups > 65535) return hipErrorInvalidValue;
  constexpr int NW = MT == 4 ? 8 : 16;  // four row blocks need 256 VGPRs: two waves per SIMD
  gemm_skinny_kernel<MT, NW, RESID, I8><<<dim3((unsigned)(n / 32), (unsigned)groups), NW * 64, 0, stream>>>(
      a, a_words, as, w, ws, m, n, I8 ? k / 128 : k / 256, residual, out);
  return hipGetLastError();
}

template <bool RESID, bool I8>
hipError_t launch_skinny_m(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                           int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (m <= 32) return launch_skinny<1, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (m <= 64) return launch_skinny<2, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_skinny<4, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

template <bool I8 = false>
hipError_t launch_skinny_any(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                             int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (residual) return launch_skinny_m<true, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_skinny_m<false, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

// Decode-sized G1 (M <= MR <= 8) on the VALU. v_dot8_i32_i4 multiplies eight
// packed signed 4-bit codes pairwise and adds the products to an i32 exactly,
// so both operands are used as packed (no unpack, no MFMA): the kernel only
// has to stream the weight. A workgroup of NW waves owns RW output columns
// (weight rows n0 .. n0+RW-1); wave w takes k-steps w, w + NW, ..., U of them
// per round with all their loads in flight. Lane l reads 16 bytes (32 k) at
// k-segment l % 8 of weight rows l / 8 + 8j, j < RW / 8: one load
// instruction covers 8 whole 128-byte rows of a tiled block. The activation
// segment of row m is one 16-byte load; rows past M and k-steps past K read
// as zero (the weight's leave the buffer's range, so they move no data). The
// eight lanes of a row are summed by DPP and the waves' sums through LDS
// (integer adds: exact in any order), then the G1 epilogue runs on the totals.
// I8: INT8 codes (h3_gemm_i8_256's operands), v_dot4_i32_i8 on k-steps of
// 128 k; the layout and the 16 bytes per lane are the same.
template <int MR, int NW, int U, int RW, bool RESID, bool I8 = false>
__global__ __launch_bounds__(NW * 64) void gemm_decode_kernel(const uint32_t* __restrict__ a, int a_words,
                                                          const float* __restrict__ as, const uint32_t* __restrict__ w,
                                                          const float* __restrict__ ws, int64_t M, int N, int kb,
                                                          const uint16_t* __restrict__ residual,
                                                          uint16_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int J = RW / 8;
  static_assert(RW % 8 == 0 && 128 % RW == 0 && MR * RW <= NW * 64, "decode tile");
  // Every argument into SGPRs at once: one scalar round trip, where the
  // compiler would otherwise fetch each under the branch that first needs it.
  asm volatile("" ::"s"(a), "s"(as), "s"(w), "s"(ws), "s"(residual), "s"(out), "s"(M), "s"(a_words), "s"(N), "s"(kb));
  __shared__ int red[NW][MR][RW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int seg = lane & 7, r8 = lane >> 3;
  const int n0 = blockIdx.x * RW;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (int64_t)(n0 / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const int w_voff = ((n0 % 128) + r8) * 128 + 16 * seg;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, (uint32_t)(M * a_words * 4));
  const int a_voff = 16 * seg;
  // The epilogue's scales are fetched with the first loads, so their latency
  // is not paid again after the reduction.
  const int em = threadIdx.x / RW, er = threadIdx.x % RW;
  const bool epi = threadIdx.x < MR * RW && em < M;
  float e_ws = 0.0f, e_as = 0.0f;
  uint32_t e_res = 0;
  if (epi) {
    e_ws = ws[n0 + er];
    e_as = as[em];
    if (RESID) e_res = residual[(int64_t)em * N + n0 + er];
  }
  int acc[J][MR];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[j][m] = 0;
  for (int kt0 = wave; kt0 < kb; kt0 += NW * U) {
    v4i wv[U][J], av[U][MR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // k-steps past kb: the weight offset leaves the resource (reads 0)
      const int kt = kt0 + NW * u;
#pragma unroll
      for (int j = 0; j < J; ++j)
        wv[u][j] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 1024 * j, kt * 16384, 0);
#pragma unroll
      for (int m = 0; m < MR; ++m)
        av[u][m] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff + m * a_words * 4, (kt < kb ? kt : 0) * 128, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
          for (int c = 0; c < 4; ++c)
            acc[j][m] = I8 ? __builtin_amdgcn_sdot4(wv[u][j][c], av[u][m][c], acc[j][m], false)
                           : __builtin_amdgcn_sdot8(wv[u][j][c], av[u][m][c], acc[j][m], false);
  }
  // Sum the 8 segments of each row: lane xor 1 and xor 2 by DPP quad_perm
  // [1,0,3,2] and [2,3,0,1], then lane xor 4 by a swizzle; every lane of the
  // eight ends with the row's sum.
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      int v = acc[j][m];
      v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
      v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
      v += __builtin_amdgcn_ds_swizzle(v, 0x101F);  // bit mode: and 0x1F, or 0, xor 4
      if (seg == 0) red[wave][m][r8 + 8 * j] = v;
    }
  __syncthreads();
  if (epi) {
    int sum = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) sum += red[q][em][er];
    uint32_t v = g1_value<0>(sum, e_ws, e_as);
    if (RESID) v = f32_to_bf16(bf16_lo(e_res) + bf16_lo(v));
    out[(int64_t)em * N + n0 + er] = (uint16_t)v;
  }
#endif
}

template <int MR, bool RESID, bool I8>
hipError_t launch_decode_mr(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                            int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  // 16 columns and 8 waves per workgroup: N12288 gives 768 workgroups, three
  // per CU (32 columns gave 1.5 per CU and half the CUs twice the bytes).
  // Two k-steps per round where K has them (measured against one, and
  // against 4 or 16 waves: M1 N12288 K4096 2.9 us with the weight in the
  // last-level cache, 6.3 us streaming it from HBM).
  // Four per round for 32 k-steps or more (INT8 K4096) with at most two rows.
  const int kb = I8 ? k / 128 : k / 256;
  if (MR <= 2 && kb >= 32)
    gemm_decode_kernel<MR, 8, 4, 16, RESID, I8><<<(unsigned)(n / 16), 512, 0, stream>>>(a, a_words, as, w, ws, m, n,
                                                                                     kb, residual, out);
  else if (kb >= 16)
    gemm_decode_kernel<MR, 8, 2, 16, RESID, I8><<<(unsigned)(n / 16), 512, 0, stream>>>(a, a_words, as, w, ws, m, n,
                                                                                     kb, residual, out);
  else
    gemm_decode_kernel<MR, 8, 1, 16, RESID, I8><<<(unsigned)(n / 16), 512, 0, stream>>>(a, a_words, as, w, ws, m, n,
                                                                                     kb, residual, out);
  return hipGetLastError();
}

template <bool RESID, bool I8>
hipError_t launch_decode_m(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                           int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (m == 1) return launch_decode_mr<1, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (m == 2) return launch_decode_mr<2, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (m <= 4) return launch_decode_mr<4, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (m <= 8) return launch_decode_mr<8, RESID, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return hipErrorInvalidValue;
}

template <bool I8 = false>
hipError_t launch_decode(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                         int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  if (residual) return launch_decode_m<true, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_decode_m<false, I8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

// Mid-sized G1 with the K split inside the workgroup: output tiles of 32 MT
// activation rows x 32 NT columns, small enough that the grid covers the CUs
// (M512 N2048: 256 tiles of 64 x 64), and the tile's k-steps shared among its
// NW waves instead of walked by one set of waves. Each wave DMAs whole k-steps
// (activation rows and weight rows, 128 bytes each, swizzled as in the DMA
// cores: physical chunk c of row r holds logical chunk c ^ ((r >> 1) & 7))
// into its own LDS stages, so it only ever waits for its own loads; NB = 2
// keeps the next k-step's DMA in flight while one computes. The partial
// accumulators (256 x the dot products, exact) are then summed through LDS in
// wave order, and each thread runs the G1 epilogue on 8 consecutive columns of
// one row (16-byte stores); consecutive threads take consecutive rows, so
// their LDS reads are consecutive 16-byte slots.
template <int MT, int NT, int NW, int NB, bool RESID>
__global__ __launch_bounds__(NW * 64) void gemm_ksplit_kernel(const uint32_t* __restrict__ a, int a_words,
                                                          const float* __restrict__ as, const uint32_t* __restrict__ w,
                                                          const float* __restrict__ ws, int64_t M, int N, int kb,
                                                          const uint16_t* __restrict__ residual,
                                                          uint16_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 32 * MT, BN = 32 * NT;  // activation rows, weight rows of the tile
  constexpr int STAGE = (BM + BN) * 128;
  constexpr int NF = MT + NT;
  constexpr int CHUNKS = BM * NT * 4;        // 8-column row chunks of the tile
  constexpr int IPT = (CHUNKS + NW * 64 - 1) / (NW * 64);
  static_assert(NB * STAGE >= MT * NT * 4096, "a wave's accumulators fit its stages");
  // Every argument into SGPRs at once (one scalar round trip).
  asm volatile("" ::"s"(a), "s"(as), "s"(w), "s"(ws), "s"(residual), "s"(out), "s"(M), "s"(a_words), "s"(N), "s"(kb));
  __shared__ __align__(16) char lds[NW * NB * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * BN;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t rows = M - m0 < BM ? M - m0 : BM;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a + m0 * a_words, (uint32_t)(rows * a_words * 4));
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (int64_t)(n0 / 128) * kb * 4096, (uint32_t)(kb * 16384));
  // DMA instruction q moves rows 8q .. 8q+7; lane -> row 8q + lane / 8,
  // physical chunk lane % 8 = logical (lane % 8) ^ (((8q + lane / 8) >> 1) & 7),
  // which depends on q only through q & 1.
  const int c_even = ((lane & 7) ^ (lane >> 4)) * 16, c_odd = ((lane & 7) ^ (4 | (lane >> 4))) * 16;
  const int a_voff = (lane >> 3) * a_words * 4, w_voff = ((n0 & 127) + (lane >> 3)) * 128;

  // Epilogue chunk c of this thread: tile row c % BM, columns
  // 8 (c / BM) .. +7. Its scales (and residual) load now.
  float e_as[IPT];
  float4 e_ws[IPT][2];
  uint4 e_res[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int c = threadIdx.x + i * NW * 64;
    const int64_t m = m0 + c % BM;
    const int n = n0 + 8 * (c / BM);
    const bool ok = c < CHUNKS && m < M;
    e_as[i] = ok ? as[m] : 0.0f;
    e_ws[i][0] = ok ? *reinterpret_cast<const float4*>(ws + n) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    e_ws[i][1] = ok ? *reinterpret_cast<const float4*>(ws + n + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    e_res[i] = RESID && ok ? *reinterpret_cast<const uint4*>(residual + m * N + n) : make_uint4(0, 0, 0, 0);
  }

  char* my = lds + wave * NB * STAGE;
  auto issue = [&](char* stage, int kt) {
#pragma unroll
    for (int q = 0; q < MT * 4; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(stage + q * 1024), 16,
                                               a_voff + ((q & 1) ? c_odd : c_even), 8 * q * a_words * 4 + kt * 128,
                                               0, 0);
#pragma unroll
    for (int q = 0; q < NT * 4; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(stage + BM * 128 + q * 1024), 16,
                                               w_voff + ((q & 1) ? c_odd : c_even), kt * 16384 + q * 1024, 0, 0);
  };
  v16i acc[NT][MT];
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v16i{};
  auto compute = [&](const char* stage) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint4 raw[NF];
      const int off = lr * 128 + (((4 * h + p) ^ ((lr >> 1) & 7)) << 4);
#pragma unroll
      for (int f = 0; f < NF; ++f) raw[f] = *reinterpret_cast<const uint4*>(stage + f * 4096 + off);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        v4i u[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f)
          u[f] = half ? unpack_pair(raw[f].z, raw[f].w) : unpack_pair(raw[f].x, raw[f].y);
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
          for (int j = 0; j < MT; ++j) acc[i][j] = mfma32_i8(u[MT + i], u[j], acc[i][j]);
      }
    }
  };
  // k-steps wave, wave + NW, ...; with two stages the next one's DMA is in
  // flight while one computes (vector memory completes in issue order).
  const int steps = wave < kb ? (kb - 1 - wave) / NW + 1 : 0;
  if (steps > 0) {
    issue(my, wave);
    if (NB == 2 && steps > 1) issue(my + STAGE, wave + NW);
    for (int s = 0; s < steps; ++s) {
      char* stage = my + (NB == 2 ? (s & 1) * STAGE : 0);
      if (NB == 2 && s + 1 < steps)
        wait_vmcnt<4 * (MT + NT)>();
      else
        wait_vmcnt<0>();
      compute(stage);
      if (s + NB < steps) issue(stage, wave + NW * (s + NB));
    }
  }
  __syncthreads();  // every wave is done reading its stages
  // Partial sums: block b = i * MT + j, register quad rq, lane -> 16 bytes.
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        *reinterpret_cast<v4i*>(my + (((i * MT + j) * 4 + rq) * 64 + lane) * 16) =
            v4i{acc[i][j][4 * rq], acc[i][j][4 * rq + 1], acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]};
  __syncthreads();
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int c = threadIdx.x + i * NW * 64;
    const int rr = c % BM, cc = c / BM;
    const int64_t m = m0 + rr;
    if (c >= CHUNKS || m >= M) continue;
    const int n = n0 + 8 * cc;
    // columns 8 cc .. 8 cc + 3 and + 4 .. + 7: register quad cc % 4 of weight
    // block cc / 4, lane halves 0 and 1, lane rr % 32 of activation block rr / 32
    const int qd = (((cc >> 2) * MT + (rr >> 5)) * 4 + (cc & 3)) * 64 + (rr & 31);
    v4i lo = *reinterpret_cast<const v4i*>(lds + qd * 16);
    v4i hi = *reinterpret_cast<const v4i*>(lds + (qd + 32) * 16);
#pragma unroll
    for (int q = 1; q < NW; ++q) {
      lo += *reinterpret_cast<const v4i*>(lds + q * NB * STAGE + qd * 16);
      hi += *reinterpret_cast<const v4i*>(lds + q * NB * STAGE + (qd + 32) * 16);
    }
    const float4 w0 = e_ws[i][0], w1 = e_ws[i][1];
    const float av = e_as[i];
    uint32_t p[4] = {g1_value<8>(lo.x, w0.x, av) | (g1_value<8>(lo.y, w0.y, av) << 16),
                     g1_value<8>(lo.z, w0.z, av) | (g1_value<8>(lo.w, w0.w, av) << 16),
                     g1_value<8>(hi.x, w1.x, av) | (g1_value<8>(hi.y, w1.y, av) << 16),
                     g1_value<8>(hi.z, w1.z, av) | (g1_value<8>(hi.w, w1.w, av) << 16)};
    if (RESID) {
      const uint32_t rv[4] = {e_res[i].x, e_res[i].y, e_res[i].z, e_res[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) p[j] = pack_bf16x2(bf16_lo(rv[j]) + bf16_lo(p[j]), bf16_hi(rv[j]) + bf16_hi(p[j]));
    }
    *reinterpret_cast<uint4*>(out + m * N + n) = make_uint4(p[0], p[1], p[2], p[3]);
  }
#endif
}

template <int MT, int NT, int NW, int NB>
hipError_t launch_ksplit_t(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                           int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  const int64_t groups = (m + 32 * MT - 1) / (32 * MT);
  if (groups > 65535 || n % (32 * NT) != 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(n / (32 * NT)), (unsigned)groups);
  if (residual)
    gemm_ksplit_kernel<MT, NT, NW, NB, true><<<grid, NW * 64, 0, stream>>>(a, a_words, as, w, ws, m, n, k / 256,
                                                                          residual, out);
  else
    gemm_ksplit_kernel<MT, NT, NW, NB, false><<<grid, NW * 64, 0, stream>>>(a, a_words, as, w, ws, m, n, k / 256,
                                                                           residual, out);
  return hipGetLastError();
}

hipError_t launch_ksplit(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                         int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  // The largest tile that still gives about one per CU (>= 192 tiles), with
  // 32-row tiles when m <= 32 (a 64-row tile would be half padding); else
  // 32 x 32 tiles with two stages per wave. Measured (graph replay, us):
  // M512 N2048 K2048 64x64 5.7 (32x64 7.2, 32x32 9.9); M16 N12288 K4096
  // 32x64 4.7 (64x64 6.4); M64 N12288 K4096 64x64 6.9 (32x64 8.8); M64 N4096
  // K4096 32x32 4.5 (32x64 4.8); M32 N4096 K12288 32x32 6.8 (32x64 8.7).
  auto tiles = [&](int bm, int bn) { return (m + bm - 1) / bm * (n / bn); };
  if (m > 32 && tiles(64, 64) >= 192)
    return launch_ksplit_t<2, 2, 8, 1>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (tiles(32, 64) >= 192) return launch_ksplit_t<1, 2, 8, 1>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_ksplit_t<1, 1, 8, 2>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

// Grouped expert GEMM for few routed rows per expert (decode-sized batches),
// on the schedule's 32-slot tiles: the small-M scheme of gemm_skinny_kernel
// with gathered activation rows. A workgroup of min(16, k-steps) waves owns one
// tile and 32 output columns of the expert (GU: 32 gate and the same 32 up columns); the
// waves split the k-steps, load the expert's weight rows and the slots'
// activation rows (routed: route; else route / topk; slots past the group's
// end read zeros) into registers, and the partial sums meet in LDS by integer
// atomic adds. Epilogue: E1 as expert_dmah_kernel (and for GU, S1 on the bf16
// gate and up values), stored to the slots' routed rows.
template <bool GU>
__global__ __launch_bounds__(1024) void expert_skinny_kernel(
    const uint32_t* __restrict__ a, int a_words, uint32_t a_bytes, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, const uint32_t* __restrict__ w2,
    const float* __restrict__ ws2, const float* __restrict__ groups, const int32_t* __restrict__ schedule,
    int64_t list_stride, int topk, int kb, int n, int input_routed, uint16_t* __restrict__ out, int slices) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int NA = GU ? 2 : 1;
  const int NW = (int)blockDim.x >> 6;
  __shared__ int red[NA][16][64];  // [gate / up][accumulator register][lane]
  __shared__ int routes_s[32];
  // Without GU, the epilogue's scales are DMA'd by wave 0 under the k-steps
  // (lanes 32..63 read past their resources and land zeros in the upper
  // halves), so the epilogue makes no global round trip. (With GU the two
  // more addresses spill a register: 7.5 -> 8.2 us at 8 routed rows.)
  __shared__ __align__(16) float ws_s[64];  // column scales c0 .. c0 + 31
  __shared__ float as_s[64];                // row scales of the 32 slots
  // The item's schedule entry is read together with the tile count (every
  // launched item indexes inside the schedule buffer), so the exit test
  // costs no extra round trip.
  const int64_t item = blockIdx.x;
  const int tile = (int)(item / slices);
  const int c0 = (int)(item - (int64_t)tile * slices) * 32;  // first output column within the expert
  const int tiles = schedule[0];
  const int e = schedule[kSchedEntries + 2 * tile];
  const int row0 = schedule[kSchedEntries + 1 + 2 * tile];
  if (item >= (int64_t)tiles * slices || e < 0) return;  // e >= 0 in every listed tile
  const float* list = groups + (int64_t)e * list_stride;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 31, h = lane >> 5;
  // This lane's slot route, read through a resource bounded to the list (no
  // wait for the count first; entries past it are masked below).
  const int64_t cap = list_stride - 1 - row0;
  const __amdgpu_buffer_rsrc_t l_rsrc =
      make_rsrc(list + 1 + row0, (uint32_t)((cap < 32 ? (cap > 0 ? cap : 0) : 32) * 4));
  const float route_f = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(l_rsrc, lr * 4, 0, 0));
  const int count = (int)list[0];
  const int64_t nrow = (int64_t)e * n + c0;  // first weight row of the slice
  const int w_voff = (int)(nrow % 128 + lr) * 128 + 64 * h;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const __amdgpu_buffer_rsrc_t w2_rsrc = make_rsrc((GU ? w2 : w) + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  for (int i = threadIdx.x; i < NA * 16 * 64; i += NW * 64) (&red[0][0][0])[i] = 0;

  v16i acc[NA];
#pragma unroll
  for (int s = 0; s < NA; ++s) acc[s] = v16i{};
  v4i wr[2][NA][4], ar[2][4];
  auto load_w = [&](auto buf, int kt) {
    constexpr int B = decltype(buf)::value;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      wr[B][0][c] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 16 * c, kt * 16384, 0);
      if constexpr (GU) wr[B][1][c] = __builtin_amdgcn_raw_buffer_load_b128(w2_rsrc, w_voff + 16 * c, kt * 16384, 0);
    }
  };
  // The first k-step's weights go out right behind the route load; the
  // activation rows need the route (vector memory completes in issue order,
  // so waiting for the route leaves the weight loads in flight).
  const int k0 = wave * kb / NW, k1 = (wave + 1) * kb / NW;  // k0 < k1: NW <= kb
  load_w(std::integral_constant<int, 0>{}, k0);
  if (!GU && wave == 0)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(ws + nrow, 32 * 4), (lds_ptr_t)&ws_s[0], 4, lane * 4, 0, 0, 0);
  const int my_route = row0 + lr < count ? (int)route_f : -1;
  if (threadIdx.x < 32) routes_s[threadIdx.x] = my_route;
  const int64_t xr = input_routed ? (int64_t)my_route : (int64_t)my_route / topk;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, a_bytes);
  const int a_voff = my_route >= 0 ? (int)(xr * a_words * 4) + 64 * h : (int)0x80000000u;
  if (!GU && wave == 0)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(as, 0x7fffffff), (lds_ptr_t)&as_s[0], 4,
                                             my_route >= 0 && h == 0 ? (int)(xr * 4) : (int)0x80000000u, 0, 0, 0);
  auto load_a = [&](auto buf, int kt) {
    constexpr int B = decltype(buf)::value;
#pragma unroll
    for (int c = 0; c < 4; ++c) ar[B][c] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_voff + 16 * c, kt * 128, 0);
  };
  auto load = [&](auto buf, int kt) {
    load_w(buf, kt);
    load_a(buf, kt);
  };
  auto compute = [&](auto buf) {
    constexpr int B = decltype(buf)::value;
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const v4i& y = ar[B][p];
        const v4i ua = half ? unpack_pair(y.z, y.w) : unpack_pair(y.x, y.y);
#pragma unroll
        for (int s = 0; s < NA; ++s) {
          const v4i& x = wr[B][s][p];
          acc[s] = mfma32_i8(half ? unpack_pair(x.z, x.w) : unpack_pair(x.x, x.y), ua, acc[s]);
        }
      }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  load_a(B0{}, k0);
  for (int kt = k0;;) {
    load(B1{}, kt + 1 < k1 ? kt + 1 : kt);
    compute(B0{});
    if (++kt >= k1) break;
    load(B0{}, kt + 1 < k1 ? kt + 1 : kt);
    compute(B1{});
    if (++kt >= k1) break;
  }
  wait_vmcnt<0>();  // this wave's scale DMA has landed
  __syncthreads();  // reduction buffer zeroed, slot routes and scales written
#pragma unroll
  for (int s = 0; s < NA; ++s)
#pragma unroll
    for (int r = 0; r < 16; ++r) atomicAdd(&red[s][r][lane], acc[s][r]);
  __syncthreads();

  // Item g = (register quad rq, lane): slot lane % 32, columns
  // c0 + 8 rq + 4 (lane / 32) + 0..3.
  for (int g = threadIdx.x; g < 256; g += NW * 64) {
    const int rq = g >> 6, ln = g & 63;
    const int route = routes_s[ln & 31];
    if (route >= 0) {
      const int col = c0 + 8 * rq + 4 * (ln >> 5);
      const float asv = GU ? as[input_routed ? (int64_t)route : (int64_t)route / topk] : as_s[ln & 31];
      const float4 wg4 = GU ? *reinterpret_cast<const float4*>(ws + (int64_t)e * n + col)
                            : *reinterpret_cast<const float4*>(&ws_s[col - c0]);
      const float wg[4] = {wg4.x, wg4.y, wg4.z, wg4.w};
      float y[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) y[t] = (float)(red[0][4 * rq + t][ln] >> 8) * (asv * wg[t]);
      if constexpr (GU) {
        const float4 wu4 = *reinterpret_cast<const float4*>(ws2 + (int64_t)e * n + col);
        const float wu[4] = {wu4.x, wu4.y, wu4.z, wu4.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float g = as_float(pack_bf16x2(0.0f, y[t]));  // bf16(gate)
          const float u = (float)(red[1][4 * rq + t][ln] >> 8) * (asv * wu[t]);
          y[t] = silu_bf16(g) * bf16_round(u);
        }
      }
      *reinterpret_cast<uint2*>(out + (int64_t)route * n + col) =
          make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    }
  }
#endif
}

// Q1 (bits 4) of up to MR bf16 rows of G 256-value groups (G <= QG) into
// LDS, with prepare_loop_body's arithmetic (the same rotation, group maxima,
// scale and rounding, so the codes and scales are those clef_i4_prepare
// writes): row m's codes as packed words in qcodes[m] (32 words per group),
// its scale in qscale[m][0]. Thread (m, g, L) = (tid / (QG * 16),
// tid / 16 % QG, tid % 16), for tid < MR * QG * 16, takes values 16 L ..
// 16 L + 15 of group g of row m; row(m) gives the row's first element, or
// nullptr for a slot without a row. Every thread of the workgroup calls it
// (it holds barriers); the lanes of each 16-lane group stay together.
template <int MR, int QG, class RowFn>
__device__ __forceinline__ void q1_rows_lds(RowFn row, int G, float (*qbuf)[16 * 20], uint32_t* qmax_s,
                                            uint32_t (*qcodes)[QG * 32], float (*qscale)[2]) {
  const int tq = threadIdx.x, m = tq / (QG * 16), g = (tq / 16) % QG, L = tq & 15;
  const uint16_t* src = m < MR ? row(m) : nullptr;
  const bool on = m < MR && g < G && src != nullptr;
  float v[16];
  if (on) {
    const u4* p = reinterpret_cast<const u4*>(src + g * 256 + 16 * L);
    const u4 x0 = p[0], x1 = p[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = bf16_lo(xw[i]);
      v[2 * i + 1] = bf16_hi(xw[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.0f;
  }
  float* buf = qbuf[m < MR ? m * QG + g : 0];
  radix4x2(v);  // strides 1 and 4
  if (m < MR) {
    float4* wrow = reinterpret_cast<float4*>(buf + L * 20);
#pragma unroll
    for (int c = 0; c < 4; ++c) wrow[c] = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
  }
  __syncthreads();
  if (m < MR) {
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = buf[k * 20 + L];
  }
  __syncthreads();
  radix4x2(v);  // strides 16 and 64 (value k holds index L + 16 k)
  uint32_t mbits = 0;
  if (on) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t a = as_uint(v[k]) & 0x7fffffffu;
      mbits = mbits > a ? mbits : a;
    }
  }
  mbits = group_max16(mbits);
  if (m < MR && L == 0) qmax_s[m * QG + g] = mbits;
  if (m < MR) {
#pragma unroll
    for (int k = 0; k < 16; ++k) buf[k * 20 + L] = v[k];
  }
  __syncthreads();
  if (tq < MR) {
    // the row's scale and 1/16-scale (prepare_loop_body's steps)
    uint32_t mx = 0;
    for (int gg = 0; gg < G; ++gg) mx = mx > qmax_s[tq * QG + gg] ? mx : qmax_s[tq * QG + gg];
    const float mf = mx >= 0x7f800000u ? __builtin_huge_valf() : as_float(mx);
    const float normal = mf * 0.0625f;
    const float safe = __builtin_fmaxf(normal, 1e-30f);
    const float sc = safe / 7.0f;
    qscale[tq][0] = sc;
    qscale[tq][1] = 0.0625f / sc;
  }
  __syncthreads();
  if (on) {
    const float sc = qscale[m][0], inv = qscale[m][1];
    const bool valid = sc < __builtin_huge_valf();
    float nat[16];
    const float4* rrow = reinterpret_cast<const float4*>(buf + L * 20);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 t4 = rrow[c];
      nat[4 * c] = t4.x, nat[4 * c + 1] = t4.y, nat[4 * c + 2] = t4.z, nat[4 * c + 3] = t4.w;
    }
    qcodes[m][(g * 256 + 16 * L) / 8] = pack_codes<4>(nat, inv, valid);
    qcodes[m][(g * 256 + 16 * L) / 8 + 1] = pack_codes<4>(nat + 8, inv, valid);
  }
  __syncthreads();
}

// Grouped expert GEMM for schedule tiles of a few routed rows (decode
// batches: up to 32 tokens, where most experts hold one to three rows), on
// the VALU as gemm_decode_kernel: v_dot8_i32_i4 multiplies the packed codes
// as stored, and each load instruction reads 8 whole 128-byte weight rows
// (expert_skinny_kernel's MFMA layout reads 32 rows per instruction, 32
// bytes of each). A workgroup of NW waves owns one 32-slot tile and RW
// output columns of its expert (GU: RW gate and the same RW up columns);
// wave w takes k-steps w, w + NW, ...; lane l reads 16 bytes (32 k) at
// k-segment l % 8 of weight rows l / 8 + 8 j and the same segment of each
// slot's activation row (routed: row = route; else route / topk). The
// tile's slots are taken MR at a time. Segment sums by DPP and wave sums
// through LDS (exact integer adds), then expert_skinny_kernel's epilogue on
// the same integer dots: E1 = bf16(f32(dot) * RN(as * ws)), for GU S1 on the
// bf16 gate and up values, stored to the slots' routed rows.
//
// QH (the MoE layer's down projection): the activation is h itself, bf16
// rows [routes][K] (K <= kDecodeQhMaxK), and each pass quantizes its slots'
// rows into LDS with Q1's arithmetic (prepare_loop_body: the same rotation,
// group maxima, scale and rounding, so the codes and scales are those
// clef_i4_prepare writes) while the wave's first weight loads are in flight;
// the layer then needs no separate quantizer launch for h.
constexpr int kDecodeQhMaxK = 2048;
template <bool GU, int NW, int RW, int MR, bool QH = false>
__global__ __launch_bounds__(NW * 64) void expert_decode_kernel(
    const uint32_t* __restrict__ a, int a_words, uint32_t a_bytes, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, const uint32_t* __restrict__ w2,
    const float* __restrict__ ws2, const float* __restrict__ groups, const int32_t* __restrict__ schedule,
    int64_t list_stride, int topk, int kb, int n, int input_routed, uint16_t* __restrict__ out, int slices,
    const uint16_t* __restrict__ hq = nullptr) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int NA = GU ? 2 : 1, J = RW / 8;
  static_assert(RW % 8 == 0 && 128 % RW == 0, "decode tile");
  static_assert(!QH || (!GU && MR * (kDecodeQhMaxK / 256) * 16 <= NW * 64), "one thread per 16 values of h");
  __shared__ int red[NW][NA][MR][RW];
  // QH: the rotation buffers of each slot's groups (20-float rows, as the
  // quantizer), the groups' maxima, and the slots' codes and scales
  constexpr int QG = QH ? kDecodeQhMaxK / 256 : 1;
  __shared__ __align__(16) float qbuf[QH ? MR * QG : 1][16 * 20];
  __shared__ uint32_t qmax_s[QH ? MR * QG : 1];
  __shared__ __align__(16) uint32_t qcodes[QH ? MR : 1][QG * 32];
  __shared__ float qscale[QH ? MR : 1][2];
  // Every launched item indexes inside the schedule buffer (the launch
  // covers its largest tile count), so the entry is read with the count.
  const int64_t item = blockIdx.x;
  const int tile = (int)(item / slices);
  const int c0 = (int)(item - (int64_t)tile * slices) * RW;  // first output column within the expert
  const int tiles = schedule[0];
  const int e = schedule[kSchedEntries + 2 * tile];
  const int row0 = schedule[kSchedEntries + 1 + 2 * tile];
  if (item >= (int64_t)tiles * slices || e < 0) return;  // e >= 0 in every listed tile
  const float* list = groups + (int64_t)e * list_stride;
  const int count = (int)list[0];
  const int row_end = count < row0 + 32 ? count : row0 + 32;  // the tile's slots: row0 .. row_end - 1
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int seg = lane & 7, r8 = lane >> 3;
  const int64_t nrow = (int64_t)e * n + c0;  // first weight row of the slice (RW rows in one 128-row block)
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const __amdgpu_buffer_rsrc_t w2_rsrc = make_rsrc((GU ? w2 : w) + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const int w_voff = (int)(nrow % 128 + r8) * 128 + 16 * seg;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, a_bytes);
  for (int r0 = row0; r0 < row_end; r0 += MR) {
    // the pass's slots: routes (wave-uniform) and activation row offsets
    int route[MR], a_off[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      route[m] = r0 + m < row_end ? (int)list[1 + r0 + m] : -1;
      const int64_t xr = input_routed ? (int64_t)route[m] : (int64_t)route[m] / topk;
      a_off[m] = route[m] >= 0 ? (int)(xr * a_words * 4) + 16 * seg : (int)0x80000000u;
    }
    int acc[NA][J][MR];
#pragma unroll
    for (int s = 0; s < NA; ++s)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[s][j][m] = 0;
    v4i wv0[J];  // QH: the wave's first k-step's weights, issued before the quantization
    if constexpr (QH) {
#pragma unroll
      for (int j = 0; j < J; ++j)
        wv0[j] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 1024 * j, (wave < kb ? wave : 0) * 16384, 0);
      // Q1 of the pass's slots' h rows
      q1_rows_lds<MR, QG>(
          [&](int m) -> const uint16_t* {
            int rm = -1;  // slot m's route (selects: route[] stays in registers)
#pragma unroll
            for (int mm = 0; mm < MR; ++mm) rm = mm == m ? route[mm] : rm;
            return rm >= 0 ? hq + (int64_t)rm * (kb * 256) : nullptr;
          },
          kb, qbuf, qmax_s, qcodes, qscale);
    }
    for (int kt = wave; kt < kb; kt += NW) {
      v4i wv[NA][J], av[MR];
      if (QH && kt == wave) {
#pragma unroll
        for (int j = 0; j < J; ++j) wv[0][j] = wv0[j];
      } else {
#pragma unroll
        for (int j = 0; j < J; ++j) {
          wv[0][j] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 1024 * j, kt * 16384, 0);
          if constexpr (GU)
            wv[1][j] = __builtin_amdgcn_raw_buffer_load_b128(w2_rsrc, w_voff + 1024 * j, kt * 16384, 0);
        }
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if constexpr (QH) {
          const uint4 c4 = *reinterpret_cast<const uint4*>(&qcodes[m][kt * 32 + 4 * seg]);
          av[m] = v4i{(int)c4.x, (int)c4.y, (int)c4.z, (int)c4.w};
        } else {
          av[m] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, a_off[m], kt * 128, 0);
        }
      }
#pragma unroll
      for (int s = 0; s < NA; ++s)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[s][j][m] = __builtin_amdgcn_sdot8(wv[s][j][c], av[m][c], acc[s][j][m], false);
    }
    // the 8 segments of each row: lane xor 1 and xor 2 by DPP, xor 4 by a swizzle
#pragma unroll
    for (int s = 0; s < NA; ++s)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          int v = acc[s][j][m];
          v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
          v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
          v += __builtin_amdgcn_ds_swizzle(v, 0x101F);
          if (seg == 0) red[wave][s][m][r8 + 8 * j] = v;
        }
    __syncthreads();
    for (int t = threadIdx.x; t < MR * RW; t += NW * 64) {
      const int m = t / RW, c = t % RW;
      const int rt = r0 + m < row_end ? (int)list[1 + r0 + m] : -1;
      if (rt < 0) continue;
      int dot = 0, dot_u = 0;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        dot += red[q][0][m][c];
        if constexpr (GU) dot_u += red[q][NA - 1][m][c];
      }
      const float asv = QH ? qscale[m][0] : as[input_routed ? (int64_t)rt : (int64_t)rt / topk];
      float y = (float)dot * (asv * ws[nrow + c]);
      if constexpr (GU) {
        const float g = as_float(pack_bf16x2(0.0f, y));  // bf16(gate)
        const float u = (float)dot_u * (asv * ws2[nrow + c]);
        y = silu_bf16(g) * bf16_round(u);
      }
      out[(int64_t)rt * n + c0 + c] = (uint16_t)(pack_bf16x2(y, 0.0f) & 0xFFFFu);
    }
    __syncthreads();  // the partial sums are read before the next pass writes them
  }
#endif
}

// The MoE layer's router, Q1(x) and fused gate/up + SwiGLU for a few tokens
// at top-8 over 128 experts (decode), one launch: workgroup (t, r, slice)
// owns route slot r of token t and RW columns of h. Every workgroup routes
// the tokens itself (route_body16, the router's own code: the same ids;
// workgroup 0 also writes the routes and the combine order, order[t][j] =
// the slot with the j-th smallest expert id, as the grouping does), quantizes
// token t's x row into LDS (q1_rows_lds: the codes and scale
// clef_i4_prepare writes), and multiplies it with its expert's RW gate and
// RW up rows as expert_decode_kernel does (v_dot8_i32_i4, whole weight rows
// per load, k-steps split over the waves), then writes h = S1(E1(gate),
// E1(up)) for the slot's routed row. The redundant routing and Q1 cost less
// than the two launches and the grouping they replace up to a dozen tokens.
constexpr int kRouteGateUpMaxK = 2048;
template <int NW, int RW>
__global__ __launch_bounds__(NW * 64) void moe_route_gate_up_kernel(
    const void* __restrict__ logits, int dtype, int tokens, const uint16_t* __restrict__ x,
    const uint32_t* __restrict__ gw, const float* __restrict__ gs, const uint32_t* __restrict__ uw,
    const float* __restrict__ us, int kb, int n, int slices, float* __restrict__ routes,
    float* __restrict__ order, uint16_t* __restrict__ h) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int KT = 8, QG = kRouteGateUpMaxK / 256, J = RW / 8;
  static_assert(RW % 8 == 0 && 128 % RW == 0 && NW * 64 >= 256 && QG * 16 <= NW * 64, "decode tile");
  __shared__ int ids[16 * KT];
  __shared__ int red[NW][2][RW];
  __shared__ __align__(16) float qbuf[QG][16 * 20];
  __shared__ uint32_t qmax_s[QG];
  __shared__ __align__(16) uint32_t qcodes[1][QG * 32];
  __shared__ float qscale[1][2];
  const int per_token = KT * slices;
  const int t = (int)(blockIdx.x / per_token);
  const int rs = (int)(blockIdx.x - (int64_t)t * per_token);
  const int r = rs / slices, c0 = (rs - r * slices) * RW;
  // every thread takes part in the routing's row reductions (tokens <= 16)
  route_impl::route_body16(logits, dtype, tokens, 128, KT, routes, 0, ids, blockIdx.x == 0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int seg = lane & 7, r8 = lane >> 3;
  if (blockIdx.x == 0 && threadIdx.x < tokens * KT) {
    const int tt = threadIdx.x / KT, e = ids[threadIdx.x];
    int less = 0;
#pragma unroll
    for (int q = 0; q < KT; ++q) less += ids[tt * KT + q] < e ? 1 : 0;
    order[tt * KT + less] = (float)(threadIdx.x % KT);
  }
  // an invalid id (a logit row of NaN) names no expert: any in-range weights
  const int e = ids[t * KT + r] >= 0 && ids[t * KT + r] < 128 ? ids[t * KT + r] : 0;
  const int64_t nrow = (int64_t)e * n + c0;
  const __amdgpu_buffer_rsrc_t g_rsrc = make_rsrc(gw + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const __amdgpu_buffer_rsrc_t u_rsrc = make_rsrc(uw + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const int w_voff = (int)(nrow % 128 + r8) * 128 + 16 * seg;
  // the wave's first k-step's gate and up rows go out before the quantization
  v4i wv0[2][J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    wv0[0][j] = __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, w_voff + 1024 * j, (wave < kb ? wave : 0) * 16384, 0);
    wv0[1][j] = __builtin_amdgcn_raw_buffer_load_b128(u_rsrc, w_voff + 1024 * j, (wave < kb ? wave : 0) * 16384, 0);
  }
  q1_rows_lds<1, QG>([&](int) -> const uint16_t* { return x + (int64_t)t * (kb * 256); }, kb, qbuf, qmax_s, qcodes,
                     qscale);
  int acc[2][J];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[s2][j] = 0;
  for (int kt = wave; kt < kb; kt += NW) {
    v4i wv[2][J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (kt == wave) {
        wv[0][j] = wv0[0][j];
        wv[1][j] = wv0[1][j];
      } else {
        wv[0][j] = __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, w_voff + 1024 * j, kt * 16384, 0);
        wv[1][j] = __builtin_amdgcn_raw_buffer_load_b128(u_rsrc, w_voff + 1024 * j, kt * 16384, 0);
      }
    }
    const uint4 c4 = *reinterpret_cast<const uint4*>(&qcodes[0][kt * 32 + 4 * seg]);
    const int av[4] = {(int)c4.x, (int)c4.y, (int)c4.z, (int)c4.w};
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[s2][j] = __builtin_amdgcn_sdot8(wv[s2][j][c], av[c], acc[s2][j], false);
  }
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      int v = acc[s2][j];
      v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
      v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
      v += __builtin_amdgcn_ds_swizzle(v, 0x101F);
      if (seg == 0) red[wave][s2][r8 + 8 * j] = v;
    }
  __syncthreads();
  if (threadIdx.x < RW) {
    const int c = threadIdx.x;
    int dg = 0, du = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      dg += red[q][0][c];
      du += red[q][1][c];
    }
    const float asv = qscale[0][0];
    const float y = (float)dg * (asv * gs[nrow + c]);
    const float g = as_float(pack_bf16x2(0.0f, y));  // bf16(gate)
    const float u = (float)du * (asv * us[nrow + c]);
    const float hv = silu_bf16(g) * bf16_round(u);
    h[((int64_t)t * KT + r) * n + c0 + c] = (uint16_t)(pack_bf16x2(hv, 0.0f) & 0xFFFFu);
  }
#endif
}

// The MoE layer's down projection and combine for a few tokens at top-8
// (decode): workgroup (t, slice) owns token t's RW output columns. Its 8
// waves take the token's 8 route slots in combine order (order[t][j]: the
// slot with the j-th smallest expert id), wave j all k-steps of slot j's
// expert: each lane reads 16 bytes (32 k) at k-segment lane % 8 of weight row
// lane / 8 and the same segment of the slot's h row, quantized first into
// LDS with Q1's arithmetic (as expert_decode_kernel's QH). The segment sums
// meet by DPP; value j = E1 = bf16(f32(dot) * RN(as * ws)) of the slot goes
// to LDS, and each column's combine runs over the 8 values in order:
// acc = bf16(acc + bf16(v_j * p_j)) (combine_kernel's sequence), stored as
// bf16. One launch instead of the down projection and combine.
constexpr int kDownCombineMaxK = 1024;
template <int RW>
__global__ __launch_bounds__(512) void moe_down_combine_kernel(
    const uint16_t* __restrict__ h, const uint32_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ routes, const float* __restrict__ order, int kb, int n, int slices,
    uint16_t* __restrict__ out) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int KT = 8, QG = kDownCombineMaxK / 256, J = RW / 8;
  static_assert(RW % 8 == 0 && 128 % RW == 0 && KT * QG * 16 == 512, "one thread per 16 values of h");
  __shared__ __align__(16) float qbuf[KT * QG][16 * 20];
  __shared__ uint32_t qmax_s[KT * QG];
  __shared__ __align__(16) uint32_t qcodes[KT][QG * 32];
  __shared__ float qscale[KT][2];
  __shared__ float vals[KT][RW];
  const int t = (int)(blockIdx.x / slices);
  const int c0 = (int)(blockIdx.x - (int64_t)t * slices) * RW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // combine position j of this wave's slot
  const int seg = lane & 7, r8 = lane >> 3;
  const float* rt = routes + (int64_t)t * 2 * KT;
  // this wave's slot, its expert and weight rows
  const int slot = order_slot(order[(int64_t)t * KT + wave], KT);
  const int e_id = route_expert(rt[slot]);
  const int e = e_id >= 0 ? e_id : 0;  // a slot naming no expert: any in-range weights (unspecified output)
  const int64_t nrow = (int64_t)e * n + c0;
  const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(w + (nrow / 128) * kb * 4096, (uint32_t)(kb * 16384));
  const int w_voff = (int)(nrow % 128 + r8) * 128 + 16 * seg;
  v4i wv[QG][J];
#pragma unroll
  for (int kt = 0; kt < QG; ++kt)
#pragma unroll
    for (int j = 0; j < J; ++j)
      wv[kt][j] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_voff + 1024 * j, (kt < kb ? kt : 0) * 16384, 0);
  // Q1 of the token's 8 h rows (slot order)
  q1_rows_lds<KT, QG>([&](int m) -> const uint16_t* { return h + ((int64_t)t * KT + m) * (kb * 256); }, kb, qbuf,
                      qmax_s, qcodes, qscale);
  // the slot's dot products over every k-step (exact integer sums)
  int acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) acc[j] = 0;
#pragma unroll
  for (int kt = 0; kt < QG; ++kt) {
    if (kt >= kb) break;
    const uint4 c4 = *reinterpret_cast<const uint4*>(&qcodes[slot][kt * 32 + 4 * seg]);
    const int av[4] = {(int)c4.x, (int)c4.y, (int)c4.z, (int)c4.w};
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[j] = __builtin_amdgcn_sdot8(wv[kt][j][c], av[c], acc[j], false);
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int v = acc[j];
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    v += __builtin_amdgcn_ds_swizzle(v, 0x101F);
    if (seg == 0) {
      const int col = r8 + 8 * j;
      const float y = (float)v * (qscale[slot][0] * ws[nrow + col]);
      vals[wave][col] = bf16_to_f32(f32_to_bf16(y));  // the slot's E1 value, bf16
    }
  }
  __syncthreads();
  if (threadIdx.x < RW) {
    const int col = threadIdx.x;
    float acc2 = 0.0f;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const float p = rt[KT + order_slot(order[(int64_t)t * KT + j], KT)];
      acc2 = bf16_round(acc2 + bf16_round(vals[j][col] * p));
    }
    out[(int64_t)t * n + c0 + col] = (uint16_t)f32_to_bf16(acc2);
  }
#endif
}

template <bool GU>
hipError_t launch_expert_skinny(const uint32_t* a, int a_words, int64_t a_bytes, const float* as,
                                const uint32_t* w, const float* ws, const uint32_t* w2, const float* ws2,
                                const float* groups, const int32_t* schedule, int64_t routes, int64_t list_stride,
                                int topk, int k, int n, int input_routed, uint16_t* out, hipStream_t stream);

}  // namespace

int gemm_config_count() { return kGemmConfigs; }

hipError_t launch_gemm_i8(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                          int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream) {
  // At most 8 rows: the dot-product kernel (v_dot4_i32_i8); up to 32 the skinny kernel with one 32-row
  // block (graph replay, M1 N12288 K4096: 16.4 us against 24.2 for 128x128 tiles; at M64 the two-block
  // form loses to 128x128 tiles, 34.1 us against 24.7, on the 50 MB INT8 weight).
  if (m <= 8) return launch_decode<true>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (m <= 32) return launch_skinny_any<true>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  if (n % 256 == 0 && m >= 1024)
    return launch_dma8_any<Dma256x256W8>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
  return launch_dma8_any<Dma128x128>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
}

hipError_t launch_gemm_i4(const uint32_t* a, int a_words, const float* as, const uint32_t* w,
                          const float* ws, int64_t m, int n, int k, const uint16_t* residual,
                          uint16_t* out, int config, hipStream_t stream) {
  if (config < 0) {
    // 256x256 tiles (8 waves) once there are enough of them to give most CUs
    // one (measured: M2048 N4096 K4096 runs 33 us on 128x128 tiles against
    // 48 us on 128 tiles of 256x256), walked by a persistent grid that loads
    // each next tile's first k-steps under the current tile's last one
    // (M4096 N12288 K4096: 154 us against 160 us with one workgroup per
    // tile); 128x128 tiles otherwise.
    // Few rows: the weight stream dominates and 128x128 tiles give too few
    // workgroups, so the K-split skinny kernel (GPU time, graph replay:
    // M1 N4096 K4096 5.1 us against 17.4; M64 N12288 K4096 13.0 against
    // 17.8; M512 N2048 K2048 7.5 against 11.3; M128 N12288 K4096 29.1
    // against 18.3, where 96 tiles of 128x128 already cover most CUs).
    // At most 8 rows: the VALU dot-product kernel (graph replay, weight in
    // the last-level cache: M1 N12288 K4096 2.9 us against 8.4 for the
    // skinny kernel, M8 6.6 against 8.2; M8 N2048 K2048 3.3 against 3.8).
    // Up to 255 tiles of 128x128: the split-K tiles (M512 N2048 K2048 5.7 us
    // against 7.4 for the skinny kernel and 11.4 for 128x128 tiles; M128
    // N12288 K4096 12.6 against 18.3).
    const int64_t tiles256 = (m + 255) / 256 * (n / 256);
    const int64_t tiles128 = (m + 127) / 128 * (n / 128);
    if (m <= 8)
      config = kGemmDecode;
    else if (tiles128 < 256)
      config = kGemmKsplit;
    else
      config = (n % 256 == 0 && m >= 1024 && tiles256 >= 192) ? kGemmPersist256 : kGemmTile128;
  }
  // The 256x256 tiles need n % 256 == 0 (128x128 and skinny take any
  // n % 128 == 0); the persistent loop needs at least two k-steps.
  if ((config == kGemmTile256 || config == kGemmPersist256) && n % 256 != 0) config = kGemmTile128;
  if (config == kGemmPersist256 && k < 512) config = kGemmTile256;
  switch (config) {
    case kGemmTile128: return launch_dma_any<Dma128x128>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    case kGemmTile256: return launch_dma_any<Dma256x256W8Pin>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    case kGemmPersist256:
      return launch_dma_persist_any<Dma256x256W8Pin>(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    case kGemmSkinny: return launch_skinny_any(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    case kGemmDecode:
      if (m > 8) return launch_skinny_any(a, a_words, as, w, ws, m, n, k, residual, out, stream);
      return launch_decode(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    case kGemmKsplit: return launch_ksplit(a, a_words, as, w, ws, m, n, k, residual, out, stream);
    default: return hipErrorInvalidValue;
  }
}

// Routed rows up to which the grouped expert GEMMs use 32-slot tiles and
// expert_skinny_kernel (on average 16 rows per expert at 128 experts).
constexpr int64_t kExpertSkinnyRoutes = 2048;
constexpr int kExpertSkinnyBM = 32;

int expert_tile_rows(int64_t routes) { return routes <= kExpertSkinnyRoutes ? kExpertSkinnyBM : kExpertBM; }

// Tiles of the schedule: sum over experts of ceil(count / bm) <= routes / bm
// rounded up, plus one per expert with any route.
int64_t expert_max_tiles(int64_t routes) {
  const int bm = expert_tile_rows(routes);
  return (routes + bm - 1) / bm + (routes < 128 ? routes : 128);
}

// Routed rows up to which the grouped expert GEMMs run expert_decode_kernel
// on the 32-slot tiles: 32 tokens at top-8. Omni MoE layer by graph replay,
// weights in the last-level cache, against expert_skinny_kernel: 1 token
// 17.4 against 21.5 us, 2: 22.3 / 26.3, 4: 29.1 / 34.0, 8: 38.2 / 44.7, 16:
// 52.4 / 60.1, 32: 70.8 / 77.0; equal at 48 tokens, 96.4 against 85.5 at 64.
constexpr int64_t kExpertDecodeRoutes = 256;

namespace {
template <bool GU, int NW, int RW, int MR>
hipError_t launch_expert_decode_t(const uint32_t* a, int a_words, int64_t a_bytes, const float* as,
                                  const uint32_t* w, const float* ws, const uint32_t* w2, const float* ws2,
                                  const float* groups, const int32_t* schedule, int64_t routes, int64_t list_stride,
                                  int topk, int k, int n, int input_routed, uint16_t* out, hipStream_t stream) {
  if (a_bytes >= ((int64_t)1 << 31) || n % RW != 0) return hipErrorInvalidValue;
  const int slices = n / RW;
  const int64_t blocks = expert_max_tiles(routes) * slices;
  expert_decode_kernel<GU, NW, RW, MR><<<(unsigned)blocks, NW * 64, 0, stream>>>(
      a, a_words, (uint32_t)a_bytes, as, w, ws, w2, ws2, groups, schedule, list_stride, topk, k / 256, n,
      input_routed, out, slices);
  return hipGetLastError();
}

// MR: the slots a pass takes: one where an expert can have only one row (a
// token's top-k names distinct experts, so at most `routes / topk` rows),
// else two (8-slot passes were slower from 4 tokens on, 60.4 against 38.2 us
// at 8 tokens: most experts then hold 1 to 3 rows, and a pass costs its slots
// whether they are filled or not; experts with more rows take more passes).
// NW: one k-step per wave where K has at most 8 of them.
template <bool GU>
hipError_t launch_expert_decode(const uint32_t* a, int a_words, int64_t a_bytes, const float* as,
                                const uint32_t* w, const float* ws, const uint32_t* w2, const float* ws2,
                                const float* groups, const int32_t* schedule, int64_t routes, int64_t list_stride,
                                int topk, int k, int n, int input_routed, uint16_t* out, hipStream_t stream) {
  const int64_t rows = topk > 0 ? (routes + topk - 1) / topk : routes;
  const int kb = k / 256;
#define CLEF_DEC(NW, RW, MR)                                                                                      \
  return launch_expert_decode_t<GU, NW, RW, MR>(a, a_words, a_bytes, as, w, ws, w2, ws2, groups, schedule, routes, \
                                                list_stride, topk, k, n, input_routed, out, stream)
  constexpr int RW = GU ? 16 : 32;
  if (kb <= 4) {
    if (rows <= 1) CLEF_DEC(4, RW, 1);
    CLEF_DEC(4, RW, 2);
  }
  if (rows <= 1) CLEF_DEC(8, RW, 1);
  CLEF_DEC(8, RW, 2);
#undef CLEF_DEC
}

template <int NW, int MR>
hipError_t launch_expert_down_h_t(const uint16_t* h, const uint32_t* w, const float* ws, const float* groups,
                                  const int32_t* schedule, int64_t routes, int64_t list_stride, int topk, int k, int n,
                                  uint16_t* out, hipStream_t stream) {
  constexpr int RW = 32;
  const int slices = n / RW;
  const int64_t blocks = expert_max_tiles(routes) * slices;
  expert_decode_kernel<false, NW, RW, MR, true><<<(unsigned)blocks, NW * 64, 0, stream>>>(
      nullptr, 0, 0u, nullptr, w, ws, w, ws, groups, schedule, list_stride, topk, k / 256, n, 1, out, slices, h);
  return hipGetLastError();
}

template <bool GU>
hipError_t launch_expert_skinny(const uint32_t* a, int a_words, int64_t a_bytes, const float* as,
                                const uint32_t* w, const float* ws, const uint32_t* w2, const float* ws2,
                                const float* groups, const int32_t* schedule, int64_t routes, int64_t list_stride,
                                int topk, int k, int n, int input_routed, uint16_t* out, hipStream_t stream) {
  if (a_bytes >= ((int64_t)1 << 31) || n % 32 != 0) return hipErrorInvalidValue;
  if (routes <= kExpertDecodeRoutes)
    return launch_expert_decode<GU>(a, a_words, a_bytes, as, w, ws, w2, ws2, groups, schedule, routes, list_stride,
                                    topk, k, n, input_routed, out, stream);
  const int slices = n / 32;
  const int64_t blocks = expert_max_tiles(routes) * slices;
  const int waves = k / 256 < 16 ? k / 256 : 16;  // one k-step per wave at most needs no more waves
  expert_skinny_kernel<GU><<<(unsigned)blocks, 64 * waves, 0, stream>>>(a, a_words, (uint32_t)a_bytes, as, w, ws, w2,
                                                                   ws2, groups, schedule, list_stride, topk, k / 256,
                                                                   n, input_routed, out, slices);
  return hipGetLastError();
}
}  // namespace

namespace {
template <class T, bool GU>
hipError_t launch_expert_dmah(const uint32_t* a, int a_words, int64_t a_bytes, const float* as, const uint32_t* w,
                              const float* ws, const uint32_t* w2, const float* ws2, const float* groups,
                              const int32_t* schedule, int64_t routes, int64_t list_stride, int topk, int k, int n,
                              int input_routed, uint16_t* out, hipStream_t stream) {
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&expert_dmah_kernel<T, GU>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, expert_lds_bytes<T, GU>())) return e;
  const int tiles_n = n / (GU ? T::BN / 2 : T::BN);
  const int64_t blocks = 8 * ((expert_max_tiles(routes) * tiles_n + 7) / 8);
  expert_dmah_kernel<T, GU><<<(unsigned)blocks, T::THREADS, expert_lds_bytes<T, GU>(), stream>>>(
      a, a_words, (uint32_t)a_bytes, as, w, ws, w2, ws2, groups, schedule, list_stride, topk, k / 256, n, input_routed,
      out, tiles_n);
  return hipGetLastError();
}
}  // namespace


namespace {
// The persistent expert GEMM (expert_persist.hpp): kExpertWaves waves per
// workgroup (4: two workgroups per CU on 128 x 256 items; 8: one per CU on
// 128 x 512 items), a multiple of 8 workgroups so each XCD takes its range of
// items.
constexpr int kExpertWaves = 4;

template <bool GU, int NW = kExpertWaves>
hipError_t launch_expert_persist(const uint32_t* a, int a_words, int64_t a_bytes, const float* as, const uint32_t* w,
                                 const float* ws, const uint32_t* w2, const float* ws2, const float* groups,
                                 const int32_t* schedule, int64_t routes, int64_t list_stride, int topk, int k, int n,
                                 int input_routed, uint16_t* out, hipStream_t stream) {
  using P = ExpertPersist<GU, NW>;
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&expert_persist_kernel<GU, NW>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, P::LDS)) return e;
  int dev = 0, cus = 0;
  if (hipError_t e = current_device(dev)) return e;
  if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) return e;
  const int grid = cus * P::PER_CU >= 8 ? cus * P::PER_CU / 8 * 8 : 8;
  // Work counters: the schedule's first eight for the fused gate/up kernel,
  // the second eight for the other (each used by one launch per schedule).
  int32_t* claims = const_cast<int32_t*>(schedule) + kSchedClaims + (GU ? 0 : 8);
  expert_persist_kernel<GU, NW><<<(unsigned)grid, P::THREADS, P::LDS, stream>>>(
      a, a_words, (uint32_t)a_bytes, as, w, ws, w2, ws2, groups, schedule, list_stride, topk, k / 256, n,
      input_routed, out, n / P::COLS, claims);
  return hipGetLastError();
}

// The persistent kernel takes items of ExpertPersist::COLS output columns and
// needs at least two k-steps; other shapes run one workgroup per item
// (expert_dmah_kernel).
template <bool GU>
bool use_expert_persist(int k, int n, int64_t routes) {
  using P = ExpertPersist<GU, kExpertWaves>;
  return k / 256 * 2 >= P::MIN_HALF_STEPS && n % P::COLS == 0 &&
         routes * n * 2 <= ((int64_t)1 << 31) &&  // 32-bit store offsets
         expert_max_tiles(routes) * (n / P::COLS) < ((int64_t)1 << 31);  // 32-bit item indices
}
}  // namespace

hipError_t launch_expert_gate_up(const uint32_t* a, int a_words, const float* as, const uint32_t* gate_w,
                                 const float* gate_s, const uint32_t* up_w, const float* up_s, const float* groups,
                                 const int32_t* schedule, int64_t tokens, int topk, int k, int n, uint16_t* h,
                                 hipStream_t stream, int64_t list_stride) {
  const int64_t a_bytes = tokens * a_words * 4;
  const int64_t routes = tokens * topk;
  if (list_stride <= 0) list_stride = tokens + 1;
  if (a_bytes >= ((int64_t)1 << 31) || n % 128 != 0) return hipErrorInvalidValue;
  if (expert_tile_rows(routes) == kExpertSkinnyBM)
    return launch_expert_skinny<true>(a, a_words, a_bytes, as, gate_w, gate_s, up_w, up_s, groups, schedule, routes,
                                      list_stride, topk, k, n, 0, h, stream);
  if (use_expert_persist<true>(k, n, routes))
    return launch_expert_persist<true>(a, a_words, a_bytes, as, gate_w, gate_s, up_w, up_s, groups, schedule, routes,
                                       list_stride, topk, k, n, 0, h, stream);
  return launch_expert_dmah<ExpertGUTile, true>(a, a_words, a_bytes, as, gate_w, gate_s, up_w, up_s, groups,
                                                schedule, routes, list_stride, topk, k, n, 0, h, stream);
}

size_t expert_schedule_bytes(int64_t routes) {
  return (size_t)(kSchedEntries + 2 * expert_max_tiles(routes)) * sizeof(int32_t);
}

hipError_t launch_expert_schedule(const float* groups, int64_t tokens, int topk, int32_t* schedule,
                                  hipStream_t stream) {
  tile_list_kernel<int32_t, kSchedEntries><<<1, 128, 0, stream>>>(groups, tokens, expert_tile_rows(tokens * topk),
                                                                  schedule);
  return hipGetLastError();
}

hipError_t launch_expert_tasks(const float* groups, int64_t tokens, float* tasks, hipStream_t stream) {
  tile_list_kernel<float, 1><<<1, 128, 0, stream>>>(groups, tokens, 16, tasks);
  return hipGetLastError();
}

// Routed rows up to which the MoE layer's down projection quantizes its own
// h rows (launch_expert_down_h). Every column slice of a tile repeats its
// pass's quantization, which costs more than the quantizer launch it saves
// once experts take several passes. Omni MoE layer by graph replay, weights
// cached, against the separate quantizer: 1 token 15.8 against 17.7 us, 2:
// 21.2 / 22.6, 4: 30.0 / 30.2; 8: 39.4 / 38.7, 16: 56.5 / 52.9.
constexpr int64_t kExpertDownHRoutes = 32;

bool expert_down_h_fusable(int64_t routes, int k, int n) {
  return routes <= kExpertDownHRoutes && k % 256 == 0 && k <= kDecodeQhMaxK && n % 32 == 0;
}

// Tokens up to which the MoE layer runs moe_down_combine_kernel after the
// separate router and grouping. Each token reads its 8 experts' down weights
// itself (experts two tokens share are read twice), which the launches it
// saves outweigh up to here. Omni MoE layer by graph replay, weights cached,
// against the down projection (quantizing its own h rows up to 4 tokens) then
// combine: 1 token 14.3 against 15.8 us, 2: 19.0 / 21.1, 3: 22.6 / 24.8,
// 4: 27.1 / 29.1, 6: 32.0 / 33.3; 8: 38.5 / 38.3.
constexpr int64_t kDownCombineTokens = 6;
// Tokens up to which the layer is moe_route_gate_up_kernel then
// moe_down_combine_kernel (top-8 of 128 experts). Omni MoE layer (hidden
// 2048, inter 768) by graph replay, weights cached, against the router and
// grouping, expert_decode_kernel and moe_down_combine_kernel (up to 6 tokens)
// or the expert kernels then combine: 1 token 11.5 against 14.1 us, 4: 20.0 /
// 27.8, 6: 25.0 / 32.4, 7: 29.1 / 37.3, 8: 30.8 / 38.5, 10: 36.4 / 43.8,
// 12: 40.1 / 46.2; 16: 52.0 / 51.9.
constexpr int64_t kRouteGateUpTokens = 12;

bool down_combine_shape(int topk, int k, int n) {
  return topk == 8 && k % 256 == 0 && k <= kDownCombineMaxK && n % 8 == 0;
}

bool down_combine_fusable(int64_t tokens, int topk, int k, int n) {
  return tokens >= 1 && tokens <= kDownCombineTokens && down_combine_shape(topk, k, n);
}

bool route_gate_up_fusable(int64_t tokens, int topk, int experts, int k, int n) {
  return tokens >= 1 && tokens <= kRouteGateUpTokens && topk == 8 && experts == 128 && k % 256 == 0 &&
         k <= kRouteGateUpMaxK && n % 32 == 0 && down_combine_shape(topk, n, k);
}

hipError_t launch_route_gate_up(const void* logits, int dtype, int64_t tokens, const uint16_t* x,
                                const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                                const float* up_s, int k, int n, float* routes, float* order, uint16_t* h,
                                hipStream_t stream) {
  if (!route_gate_up_fusable(tokens, 8, 128, k, n)) return hipErrorInvalidValue;
  // 4 waves, 32 columns (graph replay of the layer at hidden 2048, inter 768,
  // 1-6 tokens: 11.4-25.3 us against 13.3-37.9 with 8 waves and 16 columns;
  // 64 columns or 2 waves within a microsecond either way)
  constexpr int NW = 4, RW = 32;
  const int slices = n / RW;
  moe_route_gate_up_kernel<NW, RW><<<(unsigned)(tokens * 8 * slices), NW * 64, 0, stream>>>(
      logits, dtype, (int)tokens, x, gate_w, gate_s, up_w, up_s, k / 256, n, slices, routes, order, h);
  return hipGetLastError();
}

hipError_t launch_down_combine(const uint16_t* h, const uint32_t* w, const float* ws, const float* routes,
                               const float* order, int64_t tokens, int topk, int k, int n, uint16_t* out,
                               hipStream_t stream) {
  if (tokens < 1 || tokens > kRouteGateUpTokens || !down_combine_shape(topk, k, n)) return hipErrorInvalidValue;
  // 16 columns per workgroup where they divide n (1-6 tokens: 0.5-2.5 us
  // less per layer than 8; 32 within half a microsecond of 16)
  auto go = [&](auto kernel, int width) {
    const int slices = n / width;
    kernel<<<(unsigned)(tokens * slices), 512, 0, stream>>>(h, w, ws, routes, order, k / 256, n, slices, out);
  };
  if (n % 16 == 0)
    go(moe_down_combine_kernel<16>, 16);
  else
    go(moe_down_combine_kernel<8>, 8);
  return hipGetLastError();
}

hipError_t launch_expert_down_h(const uint16_t* h, const uint32_t* w, const float* ws, const float* groups,
                                const int32_t* schedule, int64_t tokens, int topk, int k, int n, uint16_t* out,
                                hipStream_t stream) {
  const int64_t routes = tokens * topk;
  if (!expert_down_h_fusable(routes, k, n) || topk < 1) return hipErrorInvalidValue;
  const int64_t list_stride = tokens + 1;
  const bool one_row = tokens <= 1;  // a token's top-k names distinct experts
  if (k / 256 <= 4) {
    if (one_row) return launch_expert_down_h_t<4, 1>(h, w, ws, groups, schedule, routes, list_stride, topk, k, n, out, stream);
    return launch_expert_down_h_t<4, 2>(h, w, ws, groups, schedule, routes, list_stride, topk, k, n, out, stream);
  }
  if (one_row) return launch_expert_down_h_t<8, 1>(h, w, ws, groups, schedule, routes, list_stride, topk, k, n, out, stream);
  return launch_expert_down_h_t<8, 2>(h, w, ws, groups, schedule, routes, list_stride, topk, k, n, out, stream);
}

hipError_t launch_expert_i4(const uint32_t* a, int a_words, const float* as, const uint32_t* w,
                            const float* ws, const float* groups, const int32_t* schedule,
                            int64_t tokens, int topk, int k, int n, int input_routed, uint16_t* out,
                            hipStream_t stream, int64_t list_stride) {
  const int64_t routes = tokens * topk;
  const int64_t a_rows = input_routed ? routes : tokens;
  const int64_t a_bytes = a_rows * a_words * 4;
  if (list_stride <= 0) list_stride = tokens + 1;
  if (expert_tile_rows(routes) == kExpertSkinnyBM)
    return launch_expert_skinny<false>(a, a_words, a_bytes, as, w, ws, w, ws, groups, schedule, routes, list_stride,
                                       topk, k, n, input_routed, out, stream);
  // The callers reject activation operands of 2 GiB or more and n % 256 != 0.
  if (a_bytes >= ((int64_t)1 << 31) || n % 256 != 0) return hipErrorInvalidValue;
  if (use_expert_persist<false>(k, n, routes))
    return launch_expert_persist<false>(a, a_words, a_bytes, as, w, ws, w, ws, groups, schedule, routes, list_stride,
                                        topk, k, n, input_routed, out, stream);
  return launch_expert_dmah<ExpertHTile, false>(a, a_words, a_bytes, as, w, ws, w, ws, groups, schedule, routes,
                                                list_stride, topk, k, n, input_routed, out, stream);
}

}  // namespace clef
