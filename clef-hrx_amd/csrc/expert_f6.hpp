// Persistent grouped expert GEMM on bf6 operands (gfx950): E1 of
// kernels/omni_expert_i4.loom:113-125, 436-462 (and for GU the fused gate/up
// + SwiGLU of benches/kernels/omni_gate_up_i4.loom) with the INT4 codes of
// both operands re-encoded as e3m2 and multiplied by
// v_mfma_scale_f32_32x32x64_f8f6f4, as gemm_f6_kernel does for G1. Every
// product of two codes is exact and every partial sum an integer below 2^24
// (K < 2^18), so the f32 accumulator is f32(dot) exactly; E1 then runs on
// f32(dot) + 0 (the MFMA's -0 sums of all-zero rows made +0, as the integer
// accumulator gives) and equals the INT4 kernels' output bit for bit.
//
// Item, walk and pipeline as expert_persist_kernel: a work item is 128 slots
// (a schedule tile) x 256 weight rows (GU: 128 gate and the same 128 up rows),
// four waves of 64 x 128, two workgroups per CU walking per-XCD item ranges;
// two LDS stages of 128 k; the next item's schedule entry, route list and
// scales fetched during half-steps 1..3 and its first stage loaded under the
// current item's epilogue. Against the INT4 kernel a half-step issues half the
// MFMAs (64 k per instruction) and no unpack, and moves 1.5x the bytes
// (96-byte rows: activation rows from a bf6 quantizer, weights as
// clef_i4_f6_weight writes them). GU reads the SiLU table from global memory:
// the LDS of two workgroups holds their stages and item data only.
//
// Included by gemm_f6.hip after its bf6 helpers (F6Offsets, mfma_f6,
// f6_lds_barrier), at file scope.
#pragma once

#include "silu_table.hpp"

namespace clef {
namespace {

struct EF6Item {
  int e, row0, count, n0;
  bool valid;
};

template <bool GU>
struct ExpertF6 {
  static constexpr int NW = 4, THREADS = 64 * NW, WAVES_N = 2;
  static constexpr int WM = 64, WN = 128, TM = WM / 32, TN = WN / 32;
  static constexpr int BM = 128, BN = 256;
  static constexpr int COLS = GU ? BN / 2 : BN;  // output columns per item
  static constexpr int ROW = 96;                 // bytes per row per half-step (128 k)
  static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW;
  static constexpr int STAGE = A_BYTES + B_BYTES;  // 36 KiB
  static constexpr int A_INST = A_BYTES / 1024 / NW, B_INST = B_BYTES / 1024 / NW;
  static constexpr int INST = A_INST + B_INST;  // DMA instructions per wave per half-step
  static constexpr int PANEL_INST = B_INST / 2;  // of them in the first 128-row panel
  // Per-item metadata: slot routes, row scales, column scales (GU: gate, then
  // up 1 KiB further).
  static constexpr int M_ROUTES = 0, M_AS = 512, M_WS = 1024;
  static constexpr int WS_BYTES = GU ? 2048 : 1024;
  static constexpr int M_WS_UP = GU ? 1024 : 0;
  static constexpr int META = M_WS + WS_BYTES;
  static constexpr int META_OFF = 2 * STAGE;
  static constexpr int LDS = META_OFF + 2 * META;
  static_assert(2 * LDS <= 160 * 1024, "two workgroups per CU");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (2048 * NW) == 0, "whole DMA instructions per wave");
  static_assert(NW * WM * 64 <= STAGE, "epilogue staging: 4 KiB per wave in one stage");
  static constexpr int MIN_HALF_STEPS = 4;
};

// The 64-slot x 128-row wave tile's operands of round mf of a half-step from
// `stage`, and its MFMAs. Weight fragment j of wave column wn: GU rows (j < 2:
// gate, else up) 128 (j / 2) + 64 wn + 32 (j % 2), so fragments j and j + 2
// hold gate and up of the same output columns; otherwise rows 128 wn + 32 j.
template <bool GU>
__device__ __forceinline__ void ef6_round(v16f (&acc)[2][4], const char* __restrict__ stage, const F6Offsets& o,
                                          int a_row, int wn, int mf) {
  using P = ExpertF6<GU>;
  v8i fa[P::TM], fb[P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) fa[i] = o.operand(stage + a_row + i * 32 * P::ROW, mf);
#pragma unroll
  for (int j = 0; j < P::TN; ++j) {
    const int row = GU ? 128 * (j >> 1) + 64 * wn + 32 * (j & 1) : 128 * wn + 32 * j;
    fb[j] = o.operand(stage + P::A_BYTES + row * P::ROW + (threadIdx.x & 31) * P::ROW, mf);
  }
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma_f6(fb[j], fa[i], acc[i][j]);
}

template <bool GU>
__global__ __launch_bounds__(256, 2) void expert_f6_kernel(
    const uint8_t* __restrict__ a, int a_row_bytes, uint32_t a_bytes, const float* __restrict__ as,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, const uint8_t* __restrict__ w2,
    const float* __restrict__ ws2, const float* __restrict__ groups, const int32_t* __restrict__ schedule,
    int64_t list_stride, int topk, int kh, int n, int input_routed, uint16_t* __restrict__ out, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
  using P = ExpertF6<GU>;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / P::WAVES_N, wn = wave % P::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const int H = kh;  // half-steps per item

  // This workgroup's XCD range of items.
  const int xcd = blockIdx.x & 7;
  const int64_t total = (int64_t)schedule[0] * tiles_n;
  const int64_t chunk = (total + 7) / 8;
  const int64_t first = xcd * chunk;
  const int64_t mine = total - first < chunk ? (total - first > 0 ? total - first : 0) : chunk;
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, a_bytes);
  const uint32_t panel_bytes = (uint32_t)(kh * 12288);
  const __amdgpu_buffer_rsrc_t sched_rsrc = make_rsrc(schedule, 0x7fffffff);

  const int64_t per_xcd = gridDim.x / 8;
  int64_t claim_next = blockIdx.x / 8;
  auto claim = [&]() -> int {
    const int v = (int)claim_next;
    claim_next += per_xcd;
    return v;
  };
  auto fetch_entry = [&](int local, int& e_v, int& r_v, int& n0) {
    const int64_t it = first + local;
    const int tile = (int)(it / tiles_n);
    n0 = (int)(it - (int64_t)tile * tiles_n) * P::COLS;
    e_v = __builtin_amdgcn_raw_buffer_load_b32(sched_rsrc, 0, (1 + 2 * tile) * 4, 0);
    r_v = __builtin_amdgcn_raw_buffer_load_b32(sched_rsrc, 0, (2 + 2 * tile) * 4, 0);
  };
  // The expert's count, its route list from slot row0 (waves 0, 1) and the
  // item's column scales (waves 2, 3) into `meta`.
  auto fetch_lists = [&](int e, int row0, int n0, char* __restrict__ meta) -> int {
    const int cnt_v = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(groups + (int64_t)e * list_stride, 4), 0, 0, 0);
    if (wave < 2) {
      const int64_t cap = list_stride - 1 - row0;
      const __amdgpu_buffer_rsrc_t r_rsrc = make_rsrc(groups + (int64_t)e * list_stride + 1 + row0,
                                                      (uint32_t)((cap < 128 ? (cap > 0 ? cap : 0) : 128) * 4));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r_rsrc, (lds_ptr_t)(meta + P::M_ROUTES + 256 * wave), 4, lane * 4,
                                               256 * wave, 0, 0);
    } else if (GU || wave == 2) {
      // GU: wave 2 the gate scales, wave 3 the up scales (128 each); else
      // wave 2 the item's 256 scales (one 1 KiB instruction).
      const int part = wave - 2;
      const float* src = GU && part == 1 ? ws2 : ws;
      const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(src + (int64_t)e * n + n0, (uint32_t)(P::COLS * 4));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rsrc, (lds_ptr_t)(meta + P::M_WS + 1024 * part), 16, lane * 16, 0, 0,
                                               0);
    }
    return cnt_v;
  };
  // This lane's A DMA offsets (slot row f / 6 of instruction q, stored chunk
  // f % 6 holding logical chunk (f % 6) ^ ((row >> 3) & 1)) and, for waves
  // 0, 1, the slots' row scales into `meta`.
  auto fetch_rows = [&](int row0, int count, const char* __restrict__ routes_in, char* __restrict__ as_out,
                        int (&voff)[P::A_INST]) {
    const float* routes = reinterpret_cast<const float*>(routes_in);
#pragma unroll
    for (int ql = 0; ql < P::A_INST; ++ql) {
      const int f = 64 * (wave + P::NW * ql) + lane;
      const int r = f / 6, p = f % 6;
      const int64_t route = row0 + r < count ? (int64_t)routes[r] : 0;
      const int64_t xr = input_routed ? route : route / topk;
      voff[ql] = row0 + r < count ? (int)(xr * a_row_bytes) + ((p ^ ((r >> 3) & 1)) << 4) : (int)0x80000000u;
    }
    if (wave < 2) {
      const int rs = 64 * wave + lane;
      const int64_t rt = row0 + rs < count ? (int64_t)routes[rs] : 0;
      const int64_t xs = input_routed ? rt : rt / topk;
      const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(as, 0x7fffffff);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rsrc, (lds_ptr_t)(as_out + 256 * wave), 4,
                                               row0 + rs < count ? (int)(xs * 4) : (int)0x80000000u, 0, 0, 0);
    }
  };
  // The item's two 128-row weight panels (GU: gate and up rows n0.., else
  // rows n0 .. n0 + 255), each kh blocks of 12 KiB.
  auto b_rsrcs = [&](int e, int n0, __amdgpu_buffer_rsrc_t& b1, __amdgpu_buffer_rsrc_t& b2) {
    const int64_t p0 = ((int64_t)e * n + n0) / 128;
    b1 = make_rsrc(w + p0 * kh * 12288, panel_bytes);
    b2 = make_rsrc((GU ? w2 : w) + (GU ? p0 : p0 + 1) * kh * 12288, panel_bytes);
  };
  // DMA of half-step j into `stage`.
  auto issue = [&](char* stage, const int (&voff_a)[P::A_INST], __amdgpu_buffer_rsrc_t b1,
                   __amdgpu_buffer_rsrc_t b2, int j) {
#pragma unroll
    for (int ql = 0; ql < P::A_INST; ++ql) {
      const int q = wave + P::NW * ql;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_ptr_t)(stage + q * 1024), 16, voff_a[ql], j * 96, 0, 0);
    }
#pragma unroll
    for (int ql = 0; ql < P::B_INST; ++ql) {
      const int q = wave + P::NW * ql;  // ql < PANEL_INST: the first panel
      const int in_blk = (ql < P::PANEL_INST ? q : q - 12) * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ql < P::PANEL_INST ? b1 : b2,
                                               (lds_ptr_t)(stage + P::A_BYTES + q * 1024), 16, lane * 16,
                                               j * 12288 + in_blk, 0, 0);
    }
  };

  char* meta_cur = lds + P::META_OFF;
  char* meta_nxt = lds + P::META_OFF + P::META;
  EF6Item cur{};
  {
    const int local = claim();
    if (local >= mine) return;  // uniform: no item for this workgroup
    int e_v, r_v;
    fetch_entry(local, e_v, r_v, cur.n0);
    wait_vmcnt<0>();
    cur.e = __builtin_amdgcn_readfirstlane(e_v);
    cur.row0 = __builtin_amdgcn_readfirstlane(r_v);
    const int cnt_v = fetch_lists(cur.e, cur.row0, cur.n0, meta_cur);
    wait_vmcnt<0>();
    __syncthreads();
    cur.count = (int)__builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(cnt_v));
    cur.valid = true;
  }
  int voff_cur[P::A_INST];
  fetch_rows(cur.row0, cur.count, meta_cur + P::M_ROUTES, meta_cur + P::M_AS, voff_cur);
  __amdgpu_buffer_rsrc_t b_cur, b_cur2;
  b_rsrcs(cur.e, cur.n0, b_cur, b_cur2);
  const F6Offsets o;
  const int a_row = (wm * P::WM + lr) * P::ROW;
  char* st[2] = {lds, lds + P::STAGE};
  issue(st[0], voff_cur, b_cur, b_cur2, 0);
  wait_vmcnt<0>();
  f6_lds_barrier();

  v16f acc[P::TM][P::TN];
  while (true) {
    const bool active = cur.row0 + wm * P::WM < cur.count;  // wave-uniform: any of its 64 slots
#pragma unroll
    for (int i = 0; i < P::TM; ++i)
#pragma unroll
      for (int j = 0; j < P::TN; ++j) acc[i][j] = v16f{};

    EF6Item nxt{};
    int voff_nxt[P::A_INST];
#pragma unroll
    for (int ql = 0; ql < P::A_INST; ++ql) voff_nxt[ql] = (int)0x80000000u;
    int e_v = 0, r_v = 0, cnt_v = 0;

    // Half-step j reads stage j % 2 and loads half-step j + 1 into the other.
    auto main_loop = [&](char* __restrict__ r0, char* __restrict__ r1, char* __restrict__ mn) {
      auto half_step = [&](const char* rd, char* dma, int j) {
        if (j == 1) {
          const int local = claim();
          nxt.valid = local < mine;
          if (nxt.valid) fetch_entry(local, e_v, r_v, nxt.n0);
        }
        if (j == 2 && nxt.valid) {
          nxt.e = __builtin_amdgcn_readfirstlane(e_v);
          nxt.row0 = __builtin_amdgcn_readfirstlane(r_v);
          cnt_v = fetch_lists(nxt.e, nxt.row0, nxt.n0, mn);
        }
        if (j == 3 && nxt.valid) {
          nxt.count = (int)__builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(cnt_v));
          fetch_rows(nxt.row0, nxt.count, mn + P::M_ROUTES, mn + P::M_AS, voff_nxt);
        }
        if (j + 1 < H) issue(dma, voff_cur, b_cur, b_cur2, j + 1);
        if (active) {
          ef6_round<GU>(acc, rd, o, a_row, wn, 0);
          ef6_round<GU>(acc, rd, o, a_row, wn, 1);
        }
        wait_vmcnt<0>();
        f6_lds_barrier();
      };
      for (int j0 = 0; j0 < H; j0 += 2) {
        half_step(r0, r1, j0);
        if (j0 + 1 < H) half_step(r1, r0, j0 + 1);
      }
    };
    main_loop(st[0], st[1], meta_nxt);

    // The next item's half-step 0 goes where this item's half-step H would.
    char* nst0 = (H & 1) ? st[1] : st[0];
    char* stg = (H & 1) ? st[0] : st[1];  // the stage half-step H - 1 read
    __amdgpu_buffer_rsrc_t b_nxt = b_cur, b_nxt2 = b_cur2;
    if (nxt.valid) b_rsrcs(nxt.e, nxt.n0, b_nxt, b_nxt2);

    auto epilogue = [&](char* __restrict__ d0, char* __restrict__ stg_, const char* __restrict__ meta) {
      if (nxt.valid) issue(d0, voff_nxt, b_nxt, b_nxt2, 0);
      if (!active) {
        wait_vmcnt<0>();
        return;
      }
      const float* routes = reinterpret_cast<const float*>(meta + P::M_ROUTES);
      const float* asl = reinterpret_cast<const float*>(meta + P::M_AS);
      const float* wsl = reinterpret_cast<const float*>(meta + P::M_WS);
      const float* wsu = reinterpret_cast<const float*>(meta + P::M_WS + P::M_WS_UP);
      float asr[P::TM];
      bool valid_row[P::TM];
#pragma unroll
      for (int i = 0; i < P::TM; ++i) {
        const int r = wm * P::WM + 32 * i + lr;
        asr[i] = asl[r];
        valid_row[i] = cur.row0 + r < cur.count;
      }
      constexpr int RB = P::WM / 16;
      uint32_t dst[RB];
#pragma unroll
      for (int s = 0; s < RB; ++s) {
        const int r = wm * P::WM + 16 * s + (lane >> 2);
        const int route = (int)routes[r];
        dst[s] = cur.row0 + r < cur.count ? (uint32_t)(((int64_t)route * n + cur.n0) * 2) : 0x80000000u;
      }
      // Scales in [2^-59, 2^50] keep |E1| < 2^117: gate and up values are
      // finite, which the zero-gate handling below relies on.
      bool fast = false;
      if constexpr (GU) {
        auto in_range = [](float v) { return (v >= 0x1p-59f) & (v <= 0x1p50f); };
        bool ok = in_range(wsl[wn * 64 + lane]) & in_range(wsu[wn * 64 + lane]);
#pragma unroll
        for (int i = 0; i < P::TM; ++i) ok = ok & (!valid_row[i] | in_range(asr[i]));
        fast = __all(ok);
      }
      char* wst = stg_ + wave * (P::WM * 64);
      auto put = [&](int i, int q, uint32_t p0, uint32_t p1) {
        const int r = 32 * i + lr;
        *reinterpret_cast<uint2*>(wst + r * 64 + ((q ^ ((r >> 1) & 3)) << 4) + 8 * h) = make_uint2(p0, p1);
      };
      const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(out, 0x80000000u);
      auto flush = [&](int col0) {
        uint4 v[RB];
#pragma unroll
        for (int s = 0; s < RB; ++s) {
          const int r = 16 * s + (lane >> 2);
          v[s] = *reinterpret_cast<const uint4*>(wst + r * 64 + (((lane & 3) ^ ((r >> 1) & 3)) << 4));
        }
#pragma unroll
        for (int s = 0; s < RB; ++s)
          store_b128(out_rsrc, (int)(dst[s] + (col0 + 8 * (lane & 3)) * 2),
                     v4i{(int)v[s].x, (int)v[s].y, (int)v[s].z, (int)v[s].w});
      };
      // E1 of f32(dot): RN((dot + 0) * RN(as * ws))
      auto scaled = [&](int i, int jj, int r, float wv) -> float { return (acc[i][jj][r] + 0.0f) * (asr[i] * wv); };
      auto values = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        if constexpr (GU) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q0 = 0; q0 < 4; q0 += 2) {
              uint32_t gp[2][P::TM][2];
              uint32_t keep[2][P::TM][2];
              uint16_t act[2][P::TM][4];
              uint32_t outside = 0;
              float4 g4[2];
#pragma unroll
              for (int qq = 0; qq < 2; ++qq)
                g4[qq] = *reinterpret_cast<const float4*>(wsl + wn * 64 + 32 * j + 8 * (q0 + qq) + 4 * h);
#pragma unroll
              for (int qq = 0; qq < 2; ++qq) {
                const int q = q0 + qq;
                const float wg[4] = {g4[qq].x, g4[qq].y, g4[qq].z, g4[qq].w};
#pragma unroll
                for (int i = 0; i < P::TM; ++i)
#pragma unroll
                  for (int p = 0; p < 2; ++p) {
                    gp[qq][i][p] = pack_bf16x2(scaled(i, j, 4 * q + 2 * p, wg[2 * p]),
                                               scaled(i, j, 4 * q + 2 * p + 1, wg[2 * p + 1]));
                    if (!valid_row[i]) gp[qq][i][p] = 0x3F803F80u;
                    keep[qq][i][p] = FAST ? bf16x2_zero_keep(gp[qq][i][p]) : 0xFFFFFFFFu;
                    const uint32_t off = silu_lut_offset2(gp[qq][i][p], outside, keep[qq][i][p]);
                    const char* table = reinterpret_cast<const char*>(g_silu_lut);
                    act[qq][i][2 * p] = *reinterpret_cast<const uint16_t*>(table + (off & 0xFFFFu));
                    act[qq][i][2 * p + 1] = *reinterpret_cast<const uint16_t*>(table + (off >> 16));
                  }
              }
              __builtin_amdgcn_sched_barrier(0);
              if (__any(outside != 0)) {
                bool others = false;
#pragma unroll
                for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                  for (int i = 0; i < P::TM; ++i)
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                      const uint32_t gb = (t & 1) ? gp[qq][i][t >> 1] >> 16 : gp[qq][i][t >> 1] & 0xFFFFu;
                      const bool out_t = ((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0;
                      if (out_t && (gb & 0x7FFFu) == 0) act[qq][i][t] = (uint16_t)gb;
                      others = others | (out_t & ((gb & 0x7FFFu) != 0));
                    }
                if (__any(others)) {
#pragma unroll
                  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                    for (int i = 0; i < P::TM; ++i)
#pragma unroll
                      for (int t = 0; t < 4; ++t) {
                        const uint32_t gb = (t & 1) ? gp[qq][i][t >> 1] >> 16 : gp[qq][i][t >> 1] & 0xFFFFu;
                        if ((((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0) & ((gb & 0x7FFFu) != 0))
                          act[qq][i][t] = (uint16_t)(__builtin_bit_cast(uint32_t, silu_bf16(bf16_to_f32(gb))) >> 16);
                      }
                }
              }
#pragma unroll
              for (int qq = 0; qq < 2; ++qq) {
                const int q = q0 + qq;
                const float4 u4 = *reinterpret_cast<const float4*>(wsu + wn * 64 + 32 * j + 8 * q + 4 * h);
                const float wu[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
                for (int i = 0; i < P::TM; ++i) {
                  float y[4];
#pragma unroll
                  for (int p = 0; p < 2; ++p) {
                    const uint32_t up = pack_bf16x2(scaled(i, j + 2, 4 * q + 2 * p, wu[2 * p]),
                                                    scaled(i, j + 2, 4 * q + 2 * p + 1, wu[2 * p + 1]));
                    y[2 * p] = bf16_to_f32(act[qq][i][2 * p]) * bf16_lo(up);
                    y[2 * p + 1] = bf16_to_f32(act[qq][i][2 * p + 1]) * bf16_hi(up);
                  }
                  put(i, q, pack_bf16x2(y[0], y[1]) & keep[qq][i][0], pack_bf16x2(y[2], y[3]) & keep[qq][i][1]);
                }
              }
            }
            flush(wn * 64 + 32 * j);
          }
        } else {
#pragma unroll
          for (int j = 0; j < P::TN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int col = wn * P::WN + 32 * j + 8 * q + 4 * h;
              const float4 w4 = *reinterpret_cast<const float4*>(wsl + col);
              const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
              for (int i = 0; i < P::TM; ++i)
                put(i, q, pack_bf16x2(scaled(i, j, 4 * q, wv[0]), scaled(i, j, 4 * q + 1, wv[1])),
                    pack_bf16x2(scaled(i, j, 4 * q + 2, wv[2]), scaled(i, j, 4 * q + 3, wv[3])));
            }
            flush(wn * P::WN + 32 * j);
          }
        }
      };
      if (GU && fast)
        values(std::true_type{});
      else
        values(std::false_type{});
      // the next item's half-step 0 has landed once at most these stores are
      // outstanding (vector memory completes in issue order)
      constexpr int STORES = (GU ? P::TN / 2 : P::TN) * RB;
      static_assert(STORES < 64, "vmcnt range");
      wait_vmcnt<STORES>();
    };
    __builtin_amdgcn_sched_barrier(0);
    epilogue(nst0, stg, meta_cur);
    __builtin_amdgcn_sched_barrier(0);
    if (!nxt.valid) break;
    f6_lds_barrier();
    cur = nxt;
#pragma unroll
    for (int ql = 0; ql < P::A_INST; ++ql) voff_cur[ql] = voff_nxt[ql];
    b_cur = b_nxt;
    b_cur2 = b_nxt2;
    st[0] = nst0;
    st[1] = stg;
    char* m = meta_cur;
    meta_cur = meta_nxt;
    meta_nxt = m;
  }
  wait_vmcnt<0>();
#endif
}

template <bool GU>
hipError_t launch_expert_f6_impl(const uint8_t* a, int a_row_bytes, int64_t a_bytes, const float* as,
                                 const uint8_t* w, const float* ws, const uint8_t* w2, const float* ws2,
                                 const float* groups, const int32_t* schedule, int64_t list_stride, int topk, int k,
                                 int n, int input_routed, uint16_t* out, hipStream_t stream) {
  using P = ExpertF6<GU>;
  static LaunchCache cache;
  const void* kern = reinterpret_cast<const void*>(&expert_f6_kernel<GU>);
  if (hipError_t e = ensure_dynamic_lds(cache, kern, P::LDS)) return e;
  int dev = 0, cus = 0;
  if (hipError_t e = current_device(dev)) return e;
  if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) return e;
  const int grid = cus * 2 >= 8 ? cus * 2 / 8 * 8 : 8;
  expert_f6_kernel<GU><<<(unsigned)grid, P::THREADS, P::LDS, stream>>>(
      a, a_row_bytes, (uint32_t)a_bytes, as, w, ws, w2, ws2, groups, schedule, list_stride, topk, k / 128, n,
      input_routed, out, n / P::COLS);
  return hipGetLastError();
}

}  // namespace

// Shapes the bf6 expert kernel takes: K a multiple of 128 with at least four
// half-steps, n a multiple of the item width (GU: 128 output columns, else
// 256), activation bytes and route-row stores within 32-bit offsets.
bool expert_f6_supported(bool gu, int k, int n, int64_t a_bytes, int64_t routes) {
  return k % 128 == 0 && k / 128 >= ExpertF6<false>::MIN_HALF_STEPS && n % (gu ? 128 : 256) == 0 &&
         a_bytes < ((int64_t)1 << 31) && routes * n * 2 <= ((int64_t)1 << 31);
}

hipError_t launch_expert_f6(bool gu, const uint8_t* a, int a_row_bytes, int64_t a_bytes, const float* as,
                            const uint8_t* w, const float* ws, const uint8_t* w2, const float* ws2,
                            const float* groups, const int32_t* schedule, int64_t list_stride, int topk, int k, int n,
                            int input_routed, uint16_t* out, hipStream_t stream) {
  if (!expert_f6_supported(gu, k, n, a_bytes, (int64_t)(list_stride - 1) * topk)) return hipErrorInvalidValue;
  if (gu)
    return launch_expert_f6_impl<true>(a, a_row_bytes, a_bytes, as, w, ws, w2, ws2, groups, schedule, list_stride,
                                       topk, k, n, 0, out, stream);
  return launch_expert_f6_impl<false>(a, a_row_bytes, a_bytes, as, w, ws, w, ws, groups, schedule, list_stride, topk,
                                      k, n, input_routed, out, stream);
}

}  // namespace clef
