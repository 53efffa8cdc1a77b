// Persistent grouped expert GEMM for gfx950: one launch walks every active
// expert's work items (E1, kernels/omni_expert_i4.loom:113-125, 436-462, and
// for GU the fused gate/up + SwiGLU of benches/kernels/omni_gate_up_i4.loom).
//
// A work item is 128 expert slots (a tile of the schedule) x BN weight rows.
// The default layout (NW = 4) runs two 4-wave workgroups per CU on 128 x 256
// items (GU: 128 gate and the same 128 up rows, 128 output columns); waves
// form a 2 x 2 grid of 64 x 128 wave tiles, so each gathered activation row
// in LDS feeds two waves and each weight row two. NW = 8 runs one 8-wave
// workgroup per CU on 128 x 512 items with three stages. The contraction core
// (DmaHCore) is the half-k-step one of gemm_dmah.hpp: stages of 128 k (64
// bytes per row).
//
// Pipeline:
//  * NST LDS stages in a ring: half-step j reads stage j % NST while the DMA
//    of half-step j + NST - 1 fills stage (j + NST - 1) % NST (one barrier per
//    half-step); with two workgroups per CU, one's loads overlap the other's
//    MFMAs;
//  * the next item's schedule entry, route list, weight scales and row
//    scales are fetched during half-steps 1..3 of the current item, and its
//    first stages are DMA'd at the start of the current item's epilogue, so
//    an item starts on data already in LDS;
//  * items are (schedule tile, column block) pairs in expert-major order,
//    split into 8 contiguous per-XCD ranges (workgroup b runs on XCD b % 8);
//    the k-th workgroup of an XCD starts with item k of its range and then
//    claims the next unclaimed item from the XCD's counter, so the column
//    blocks of one tile run side by side and share its activation rows in the
//    XCD's L2. Claiming balances the two workgroups of a CU: the one
//    dispatched first wins instruction issue by age and runs its items about
//    twice as fast as the other while both compute, so equal static shares
//    left every CU with a tail of the slower workgroup running alone;
//  * the epilogue (E1, for GU then S1 with the SiLU table in LDS) goes out
//    in blocks of 32 output columns: each wave stages its 64 rows of a block
//    in the stage the item's last half-step read (free until the next item
//    starts) and stores 64-byte row pieces (buffer stores into an output of
//    at most 2 GiB), drained under the next item's first half-step.
//
// Every LDS region an inlined body touches while DMA is in flight is a
// distinct __restrict__ parameter of that body: the compiler then proves the
// reads disjoint from the DMA targets and keeps the loads in flight (it would
// otherwise wait for every outstanding DMA before each LDS read). The ring is
// therefore unrolled by NST so that each body names its stages statically.
//
// vmcnt accounting (vector memory operations complete in issue order): every
// extra load of a half-step (schedule entry, list, scales) is issued before
// that half-step's stage DMA, so "all but the last stage groups" also covers
// them.
#pragma once

#include "gemm_dmah.hpp"
#include "kernels.hpp"
#include "silu_table.hpp"

namespace clef {

// Two layouts: NW = 4 waves on 128 x 256 items (GU: 128 output columns),
// two stages, two workgroups per CU; NW = 8 waves on 128 x 512 items (GU:
// 256 output columns), three stages, one workgroup per CU.
template <bool GU, int NW_>
struct ExpertPersist {
  static constexpr int NW = NW_;
  using T = DmaHTile<64, 128, 2, NW / 2, kSchedPin, GU>;
  static_assert((NW == 4 || NW == 8) && T::BM == 128, "128-slot items on 4 or 8 waves");
  static constexpr int COLS = GU ? T::BN / 2 : T::BN;  // output columns per item
  static constexpr int STAGE = T::STAGE_BYTES;
  static constexpr int NST = NW == 8 ? 3 : 2;         // LDS stages: prefetch distance NST - 1
  static constexpr int DIST = NST - 1;
  static constexpr int INST = T::INST;                 // DMA instructions per wave per half-step
  static constexpr int PER_CU = NW == 8 ? 1 : 2;       // workgroups per CU
  // Per-item metadata block: slot routes (f32 ordinals), row scales (f32,
  // as[xr] or 0) and the item's column scales (f32; GU: gate at M_WS, up at
  // M_WS + 1 KiB: a scale DMA instruction writes a whole KiB).
  static constexpr int M_ROUTES = 0, M_AS = 512, M_WS = 1024;
  static constexpr int WS_BYTES = GU ? 2 * (COLS * 4 > 1024 ? COLS * 4 : 1024) : (COLS * 4 > 1024 ? COLS * 4 : 1024);
  static constexpr int M_WS_UP = GU ? WS_BYTES / 2 : 0;  // byte offset of the up scales from M_WS
  static constexpr int META = M_WS + WS_BYTES;
  static constexpr int LUT_OFF = NST * STAGE;
  static constexpr int LUT_BYTES = GU ? kSiluLutSize * 2 : 0;
  static constexpr int META_OFF = LUT_OFF + LUT_BYTES;
  static constexpr int CLAIM_OFF = META_OFF + 2 * META;  // the next item's index (16 bytes)
  static constexpr int LDS = CLAIM_OFF + 16;
  static_assert(LDS * PER_CU <= 160 * 1024, "workgroups per CU");
  static_assert(NW * T::WM * 64 <= STAGE, "epilogue staging: 4 KiB per wave in one stage");
  static constexpr int THREADS = T::THREADS;
  // Half-steps the pipeline needs: the next item is claimed and fetched
  // during half-steps 0..3 (K >= 512).
  static constexpr int MIN_HALF_STEPS = 4;
};

namespace {

// Workgroup barrier that waits for this wave's LDS operations only. A
// __syncthreads() also waits for every outstanding vector memory operation
// (its workgroup fence covers LDS DMA), which would drain the DMA of the
// stage two half-steps ahead at every barrier; the stage a half-step needs is
// waited for explicitly (wait_vmcnt) before this barrier. The "memory" clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Addressing of one work item (wave-uniform except voff_a).
struct ExpertItem {
  int e, row0, count, n0;
  bool valid;
};

template <bool GU, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 ? 1 : 2) void expert_persist_kernel(
    const uint32_t* __restrict__ a, int a_words, uint32_t a_bytes, const float* __restrict__ as,
    const uint32_t* __restrict__ w, const float* __restrict__ ws, const uint32_t* __restrict__ w2,
    const float* __restrict__ ws2, const float* __restrict__ groups, const int32_t* __restrict__ schedule,
    int64_t list_stride, int topk, int kb, int n, int input_routed,
    uint16_t* __restrict__ out, int tiles_n, int32_t* __restrict__ claims) {
#if defined(__HIP_DEVICE_COMPILE__)
  using P = ExpertPersist<GU, NW>;
  using T = typename P::T;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::WAVES_N, wn = wave % T::WAVES_N;
  const int h = lane >> 5, lr = lane & 31;
  const int H = 2 * kb;  // half-steps per item

  // This workgroup's XCD range of items.
  const int xcd = blockIdx.x & 7;
  // Item counts are below 2^31 (the launcher bounds tiles * tiles_n): 32-bit
  // arithmetic, which keeps the per-item index math off 64-bit division.
  const int total = schedule[0] * tiles_n;
  const int chunk = (total + 7) / 8;
  const int first = xcd * chunk;
  const int mine = total - first < chunk ? (total - first > 0 ? total - first : 0) : chunk;

  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(a, a_bytes);
  const uint32_t b_bytes = (uint32_t)((P::COLS / 128) * kb * 16384);
  // Whole-buffer resources for the item fetches: buffer loads are vector
  // memory operations whatever their address, so they follow the vmcnt
  // accounting (a uniform address would otherwise become a scalar load).
  const __amdgpu_buffer_rsrc_t sched_rsrc = make_rsrc(schedule, 0x7fffffff);

  // ---- fetch steps of an item; each is issued before a half-step's stage
  // DMA and its results are used one half-step later.
  // Step 0: the workgroup's next item in its XCD's range. Workgroup b starts
  // with item b / 8; later items come from the XCD's counter (zeroed with the
  // schedule), offset by the W = gridDim / 8 items handed out at the start.
  // Lane 0 of wave 0 issues the atomic during half-step 0 (a vector atomic,
  // covered by that half-step's vmcnt wait like the stage DMA issued after
  // it) and publishes the index in LDS before the half-step's barrier; every
  // wave reads it at half-step 1.
  const int per_xcd = gridDim.x / 8;
  int* claim_slot = reinterpret_cast<int*>(lds + P::CLAIM_OFF);
  int claimed = 0;
  auto claim_issue = [&]() {
    if (threadIdx.x == 0)
      claimed = per_xcd + __hip_atomic_fetch_add(claims + xcd, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto claim_publish = [&]() {
    if (threadIdx.x == 0) *claim_slot = claimed;
  };
  // Step 1: the schedule entry of item `local`.
  auto fetch_entry = [&](int local, int& e_v, int& r_v, int& n0) {
    const int it = first + local;
    const int tile = it / tiles_n;
    n0 = (it - tile * tiles_n) * P::COLS;
    e_v = __builtin_amdgcn_raw_buffer_load_b32(sched_rsrc, 0, (kSchedEntries + 2 * tile) * 4, 0);
    r_v = __builtin_amdgcn_raw_buffer_load_b32(sched_rsrc, 0, (kSchedEntries + 1 + 2 * tile) * 4, 0);
  };
  // Step 2: the expert's count (vector load), its route list from slot row0
  // (waves 0, 1: 64 routes each, 4 bytes per lane, zero past the list's
  // capacity) and the item's column scales (waves 2, 3: one KiB instruction
  // each, GU: gate and up) into `meta`.
  auto fetch_lists = [&](int e, int row0, int n0, char* __restrict__ meta) -> int {
    const int cnt_v = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(groups + (int64_t)e * list_stride, 4), 0, 0, 0);
    if (wave < 2) {
      const int64_t cap = list_stride - 1 - row0;
      const __amdgpu_buffer_rsrc_t r_rsrc = make_rsrc(groups + (int64_t)e * list_stride + 1 + row0,
                                                      (uint32_t)((cap < 128 ? (cap > 0 ? cap : 0) : 128) * 4));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r_rsrc, (lds_ptr_t)(meta + P::M_ROUTES + 256 * wave), 4, lane * 4,
                                               256 * wave, 0, 0);
    } else if (wave < 2 + (GU ? 2 : (P::COLS * 4 + 1023) / 1024)) {
      const int part = wave - 2;
      const float* src = GU ? (part == 0 ? ws : ws2) : ws;
      const int off = GU ? 0 : 256 * part;
      const uint32_t bytes = GU ? P::COLS * 4 : 1024;
      const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(src + (int64_t)e * n + n0 + off, bytes);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rsrc, (lds_ptr_t)(meta + P::M_WS + (GU ? P::M_WS_UP : 1024) * part),
                                               16, lane * 16, 0, 0, 0);
    }
    return cnt_v;
  };
  // Step 3: this lane's gathered A row offsets (the rows its DMA moves) and,
  // for waves 0, 1, the row scales as[xr] of 64 slots each into `meta` (zero
  // past the count).
  auto fetch_rows = [&](int row0, int count, const char* __restrict__ routes_in, char* __restrict__ as_out,
                        int (&voff)[T::A_INST]) {
    const float* routes = reinterpret_cast<const float*>(routes_in);
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) {
      const int r = 16 * (wave + NW * ql) + (lane >> 2);
      // ordinals are below 2^24 and the operand below 2 GiB: 32-bit math
      const int route = row0 + r < count ? (int)routes[r] : 0;
      const int xr = input_routed ? route : route / topk;
      voff[ql] = row0 + r < count ? xr * a_words * 4 + dmah_chunk16(lane) : (int)0x80000000u;
    }
    if (wave < 2) {
      const int rs = 64 * wave + lane;
      const int rt = row0 + rs < count ? (int)routes[rs] : 0;
      const int xs = input_routed ? rt : rt / topk;
      const __amdgpu_buffer_rsrc_t s_rsrc = make_rsrc(as, 0x7fffffff);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rsrc, (lds_ptr_t)(as_out + 256 * wave), 4,
                                               row0 + rs < count ? (int)(xs * 4) : (int)0x80000000u, 0, 0, 0);
    }
  };
  auto b_rsrcs = [&](int e, int n0, __amdgpu_buffer_rsrc_t& b1, __amdgpu_buffer_rsrc_t& b2) {
    const int64_t blk0 = ((int64_t)e * n + n0) / 128;
    b1 = make_rsrc(w + blk0 * kb * 4096, b_bytes);
    b2 = GU ? make_rsrc(w2 + blk0 * kb * 4096, b_bytes) : b1;
  };

  char* meta_cur = lds + P::META_OFF;
  char* meta_nxt = lds + P::META_OFF + P::META;

  // ---- prologue: the first item; the weight rows of its half-step 0 go
  // out with its route list (they need only the schedule entry), and the
  // SiLU table after the prologue (the first epilogue reads it).
  ExpertItem cur{};
  DmaHCore<T> c;
  // Stage ring: st[0] holds the item's half-step 0, st[1] half-step 1 (NST
  // == 3) or is free, st[NST - 1] is free.
  char* st[3] = {lds, lds + P::STAGE, lds + (P::NST - 1) * P::STAGE};
  __amdgpu_buffer_rsrc_t b_cur, b_cur2;
  {
    const int local = blockIdx.x / 8;
    if (local >= mine) return;  // uniform: no item for this workgroup, nothing in flight
    int e_v, r_v;
    fetch_entry(local, e_v, r_v, cur.n0);
    wait_vmcnt<0>();
    cur.e = __builtin_amdgcn_readfirstlane(e_v);
    cur.row0 = __builtin_amdgcn_readfirstlane(r_v);
    const int cnt_v = fetch_lists(cur.e, cur.row0, cur.n0, meta_cur);
    b_rsrcs(cur.e, cur.n0, b_cur, b_cur2);
    c.issue_b(st[0], b_cur, b_cur2, kb, 0);
    // the count, list and scales (issued before the weight rows) have landed
    wait_vmcnt<T::B_INST>();
    lds_barrier();
    cur.count = (int)__builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(cnt_v));
    cur.valid = true;
  }
  int voff_cur[T::A_INST];
  fetch_rows(cur.row0, cur.count, meta_cur + P::M_ROUTES, meta_cur + P::M_AS, voff_cur);
  c.issue_a(st[0], a_rsrc, voff_cur, 0, 0);
  if (P::DIST == 2) c.issue(st[1], a_rsrc, voff_cur, 0, b_cur, b_cur2, kb, 1);
  wait_vmcnt<(P::DIST - 1) * T::INST>();
  lds_barrier();
  if constexpr (GU) {
    // Landed by the end of half-step 0 (its wait covers every earlier load).
    const __amdgpu_buffer_rsrc_t lut_rsrc = make_rsrc(g_silu_lut, kSiluLutSize * 2);
#pragma unroll
    for (int i = 0; i < kSiluLutSize * 2 / 1024 / T::NW; ++i) {
      const int q = wave * (kSiluLutSize * 2 / 1024 / T::NW) + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(lut_rsrc, (lds_ptr_t)(lds + P::LUT_OFF + q * 1024), 16, lane * 16,
                                               q * 1024, 0, 0);
    }
  }

  v16i acc[T::TM][T::TN];
  const uint16_t* lut = reinterpret_cast<const uint16_t*>(lds + P::LUT_OFF);

  while (true) {
    const bool active = cur.row0 + wm * T::WM < cur.count;  // wave-uniform: any of its 64 slots
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) acc[i][j] = v16i{};

    // Next item (fetched during half-steps 0..3).
    ExpertItem nxt{};
    int voff_nxt[T::A_INST];
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) voff_nxt[ql] = (int)0x80000000u;
    int e_v = 0, r_v = 0, cnt_v = 0;

    // The item's half-steps, the ring unrolled by NST: half-step j reads
    // stage j % NST and loads half-step j + DIST into stage (j + DIST) % NST.
    auto main_loop = [&](char* __restrict__ r0, char* __restrict__ r1, char* __restrict__ r2,
                         char* __restrict__ mn) {
      auto half_step = [&](const char* rd, char* dma, int j) {
        if (j == 0) claim_issue();
        if (j == 1) {
          const int local = __builtin_amdgcn_readfirstlane(*claim_slot);
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
        const bool dma_now = j + P::DIST < H;
        if (dma_now) c.issue(dma, a_rsrc, voff_cur, 0, b_cur, b_cur2, kb, j + P::DIST);
        if (active) {
          c.read(rd, 0, 0);
          if (j == 0) {
            c.unpack(0, 0, 0);
          } else {
            // the last pair of half-step j - 1 (registers) under the read of pair 0
            c.template substep<true>(acc, 0, 1, 1, 1);
            c.template substep<true>(acc, 1, 0, 0, 0);
          }
          c.pair0(acc, rd);
        }
        // half-step j + 1 has landed once at most the groups issued after it
        // (DIST - 1 of them) are outstanding
        if (dma_now)
          wait_vmcnt<(P::DIST - 1) * P::INST>();
        else
          wait_vmcnt<0>();
        if (j == 0) claim_publish();
        lds_barrier();
      };
      if constexpr (P::NST == 3) {
        for (int j0 = 0; j0 < H; j0 += 3) {
          half_step(r0, r2, j0);
          if (j0 + 1 < H) half_step(r1, r0, j0 + 1);
          if (j0 + 2 < H) half_step(r2, r1, j0 + 2);
        }
      } else {
        for (int j0 = 0; j0 < H; j0 += 2) {
          half_step(r0, r1, j0);
          if (j0 + 1 < H) half_step(r1, r0, j0 + 1);
        }
      }
      if (active) {
        c.template substep<true>(acc, 0, 1, 1, 1);
        c.template substep<false>(acc, 1, 0, 0, 0);
      }
    };
    // The contraction at raised issue priority: the other workgroup's
    // epilogue on the same SIMDs then takes the issue slots the MFMA stream
    // leaves free instead of taking turns with it (measured 7 % faster for the
    // fused gate/up kernel at 4096 tokens, 3 % for the down projection).
    __builtin_amdgcn_s_setprio(2);
    main_loop(st[0], st[1], st[2], meta_nxt);
    __builtin_amdgcn_s_setprio(0);

    // The next item's stages: its half-step 0 goes where this item's
    // half-step H would (stage H % NST), and so on around the ring.
    const int rot = H % P::NST;
    char* nst[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int at = (rot + q) % P::NST;
      nst[q] = at == 0 ? st[0] : (at == 1 ? st[1] : st[2]);
    }
    __amdgpu_buffer_rsrc_t b_nxt = b_cur, b_nxt2 = b_cur2;
    if (nxt.valid) b_rsrcs(nxt.e, nxt.n0, b_nxt, b_nxt2);

    // Epilogue of the current item with the next item's loads in flight.
    // Values go out one block of 32 output columns at a time: each wave puts
    // its 64 rows x 32 columns (bf16) into its own 4 KiB of `stg` (the stage
    // the item's last half-step read, free until the next item's half-step 0
    // issues its DMA), reads them back as 64-byte row pieces and stores those
    // (one 16-byte store per lane, four lanes per row piece), so each store
    // request writes 64 contiguous bytes instead of 8.
    auto epilogue = [&](char* __restrict__ d0, char* __restrict__ d1, char* __restrict__ stg,
                        const char* __restrict__ meta, const char* __restrict__ table) {
      if (nxt.valid) {
        c.issue(d0, a_rsrc, voff_nxt, 0, b_nxt, b_nxt2, kb, 0);
        if (P::DIST == 2) c.issue(d1, a_rsrc, voff_nxt, 0, b_nxt, b_nxt2, kb, 1);
      }
      if (!active) {  // no slot of this wave is below the count: no stores
        wait_vmcnt<(P::DIST - 1) * P::INST>();
        return;
      }
      const float* routes = reinterpret_cast<const float*>(meta + P::M_ROUTES);
      const float* asl = reinterpret_cast<const float*>(meta + P::M_AS);
      const float* wsl = reinterpret_cast<const float*>(meta + P::M_WS);
      const float* wsu = reinterpret_cast<const float*>(meta + P::M_WS + P::M_WS_UP);
      float asr[T::TM], asr8[T::TM];
      bool valid_row[T::TM];
#pragma unroll
      for (int i = 0; i < T::TM; ++i) {
        const int r = wm * T::WM + 32 * i + lr;
        asr[i] = asl[r];
        asr8[i] = asr[i] * 0x1p-8f;
        valid_row[i] = cur.row0 + r < cur.count;
      }
      // Byte offset in `out` of the item's first output column in the rows
      // this lane stores (rows 16 s + lane / 4 of the wave's 64); rows past the
      // count get an offset past the output (stores dropped). Ordinals are
      // below 2^24, so the f32 list entries convert exactly to int.
      constexpr int RB = T::WM / 16;
      uint32_t dst[RB];
      // All RB route reads go out together and are pinned in registers before
      // the selects below (left to itself the compiler moves each read under
      // its row's condition: one LDS round trip per row).
      float route_f[RB];
#pragma unroll
      for (int s = 0; s < RB; ++s) {
        route_f[s] = routes[wm * T::WM + 16 * s + (lane >> 2)];
        pin_vgpr(route_f[s]);
      }
#pragma unroll
      for (int s = 0; s < RB; ++s) {
        const int r = wm * T::WM + 16 * s + (lane >> 2);
        // route * n + n0 < 2^30 (the launcher bounds routes * n * 2 by 2^31)
        dst[s] = cur.row0 + r < cur.count ? (uint32_t)(((int)route_f[s] * n + cur.n0) * 2) : 0x80000000u;
      }
      // f32(acc) is 256 * dot exactly. For GU, when every row and column
      // scale of the wave is at least 2^-59, RN(asr * 2^-8) * w is exact and
      // RN(f32(acc) * RN(asr * 2^-8 * w)) = RN(dot * RN(asr * w)): the shift
      // is left out (the down projection keeps it: one accumulator per
      // output gains less than the check costs).
      bool fast = false;
      if constexpr (GU) {
        // The wave's 64 gate and 64 up column scales, one of each per lane.
        // With every scale also at most 2^50, |E1| < 2^117 (acc < 2^25): no
        // gate or up value is infinite or NaN, which the zero handling below
        // relies on.
        auto in_range = [](float v) { return (v >= 0x1p-59f) & (v <= 0x1p50f); };
        bool ok = in_range(wsl[wn * 64 + lane]) & in_range(wsu[wn * 64 + lane]);
#pragma unroll
        for (int i = 0; i < T::TM; ++i) ok = ok & (!valid_row[i] | in_range(asr[i]));
        fast = __all(ok);
      }
      // This wave's staging rows: 64 bytes (32 columns) each, the 16-byte
      // chunk q of row r at chunk q ^ ((r / 2) % 4).
      char* wst = stg + wave * (T::WM * 64);
      auto put = [&](int i, int q, uint32_t p0, uint32_t p1) {
        const int r = 32 * i + lr;
        *reinterpret_cast<uint2*>(wst + r * 64 + ((q ^ ((r >> 1) & 3)) << 4) + 8 * h) = make_uint2(p0, p1);
      };
      // Every store instruction is issued (rows past the count fall outside
      // the resource), so each active wave issues exactly STORES of them.
      const __amdgpu_buffer_rsrc_t out_rsrc = make_rsrc(out, 0x80000000u);
      auto flush = [&](int col0) {  // col0: the block's first output column in the item
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
      auto values = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto scaled = [&](int i, int jj, int r, float wv) -> float {
          const int av = acc[i][jj][r];
          return FAST ? (float)av * (asr8[i] * wv) : (float)(av >> 8) * (asr[i] * wv);
        };
        if constexpr (GU) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q0 = 0; q0 < 4; q0 += 2) {
              // bf16(g) two per register and the table reads of 16 columns
              // first (their latencies overlap), then one wave-uniform branch
              // for values outside the table.
              uint32_t gp[2][T::TM][2];
              uint32_t keep[2][T::TM][2];  // FAST: bf16x2_zero_keep(gp)
              uint16_t act[2][T::TM][4];  // bf16 bits of silu(g)
              uint32_t outside = 0;
              float4 g4[2];  // gate column scales, read before the table
#pragma unroll
              for (int qq = 0; qq < 2; ++qq)
                g4[qq] = *reinterpret_cast<const float4*>(wsl + wn * 64 + 32 * j + 8 * (q0 + qq) + 4 * h);
#pragma unroll
              for (int qq = 0; qq < 2; ++qq) {
                const int q = q0 + qq;
                const float wg[4] = {g4[qq].x, g4[qq].y, g4[qq].z, g4[qq].w};
#pragma unroll
                for (int i = 0; i < T::TM; ++i)
#pragma unroll
                  for (int p = 0; p < 2; ++p) {
                    gp[qq][i][p] = pack_bf16x2(scaled(i, j, 4 * q + 2 * p, wg[2 * p]),
                                               scaled(i, j, 4 * q + 2 * p + 1, wg[2 * p + 1]));
                    // rows past the count (never stored) read as zero, which
                    // lies outside the table: give them 1.0 instead
                    if (!valid_row[i]) gp[qq][i][p] = 0x3F803F80u;
                    // FAST: g = +-0 (integer dot products are often zero) is
                    // not flagged: the table gives silu(+-2), of g's sign, and
                    // masking the product to its sign gives +-0 * bf16(u)
                    // exactly (u is finite)
                    keep[qq][i][p] = FAST ? bf16x2_zero_keep(gp[qq][i][p]) : 0xFFFFFFFFu;
                    const uint32_t off = silu_lut_offset2(gp[qq][i][p], outside, keep[qq][i][p]);
                    act[qq][i][2 * p] = *reinterpret_cast<const uint16_t*>(table + (off & 0xFFFFu));
                    act[qq][i][2 * p + 1] = *reinterpret_cast<const uint16_t*>(table + (off >> 16));
                  }
              }
              __builtin_amdgcn_sched_barrier(0);
              if (__any(outside != 0)) {
                // silu(+-0) = +-0 (integer dot products are often zero):
                // those directly, then the others outside the table only if
                // there are any
                bool others = false;
#pragma unroll
                for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                  for (int i = 0; i < T::TM; ++i)
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                      const uint32_t gb = (t & 1) ? gp[qq][i][t >> 1] >> 16 : gp[qq][i][t >> 1] & 0xFFFFu;
                      const bool out = ((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0;
                      if (out && (gb & 0x7FFFu) == 0) act[qq][i][t] = (uint16_t)gb;
                      others = others | (out & ((gb & 0x7FFFu) != 0));
                    }
                if (__any(others)) {
#pragma unroll
                  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                    for (int i = 0; i < T::TM; ++i)
#pragma unroll
                      for (int t = 0; t < 4; ++t) {
                        const uint32_t gb = (t & 1) ? gp[qq][i][t >> 1] >> 16 : gp[qq][i][t >> 1] & 0xFFFFu;
                        if ((((gb - ((uint32_t)kSiluLutExp0 << 7)) & 0x7000u) != 0) & ((gb & 0x7FFFu) != 0))
                          act[qq][i][t] = (uint16_t)(__builtin_bit_cast(uint32_t, silu_bf16(bf16_to_f32(gb))) >> 16);
                      }
                }
              }
              // h = bf16(silu(g) * bf16(u)); the packing rounds h to bf16
#pragma unroll
              for (int qq = 0; qq < 2; ++qq) {
                const int q = q0 + qq;
                const float4 u4 = *reinterpret_cast<const float4*>(wsu + wn * 64 + 32 * j + 8 * q + 4 * h);
                const float wu[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
                for (int i = 0; i < T::TM; ++i) {
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
          // The column scales of block j + 1 are read while block j is
          // converted and stored, so each block waits for LDS once (its
          // staged rows) instead of once per scale read.
          float4 w4[2][4];
          auto load_scales = [&](int j, float4 (&dst4)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              dst4[q] = *reinterpret_cast<const float4*>(wsl + wn * T::WN + 32 * j + 8 * q + 4 * h);
          };
          load_scales(0, w4[0]);
#pragma unroll
          for (int j = 0; j < T::TN; ++j) {
            if (j + 1 < T::TN) load_scales(j + 1, w4[(j + 1) & 1]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float4 c4 = w4[j & 1][q];
              const float wv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
              for (int i = 0; i < T::TM; ++i)
                put(i, q, pack_bf16x2(scaled(i, j, 4 * q, wv[0]), scaled(i, j, 4 * q + 1, wv[1])),
                    pack_bf16x2(scaled(i, j, 4 * q + 2, wv[2]), scaled(i, j, 4 * q + 3, wv[3])));
            }
            flush(wn * T::WN + 32 * j);
          }
        }
      };
      if (GU && fast)
        values(std::true_type{});
      else
        values(std::false_type{});
      // The next item's half-step 0 has landed once at most its half-step 1
      // group and these stores are outstanding (in issue order).
      constexpr int STORES = (GU ? T::TN / 2 : T::TN) * RB;
      constexpr int AFTER = (P::DIST - 1) * P::INST + STORES;
      static_assert(AFTER < 64, "vmcnt range");
      wait_vmcnt<AFTER>();
    };
    // No MFMA of the next item (fresh accumulators) may move into the epilogue.
    __builtin_amdgcn_sched_barrier(0);
    epilogue(nst[0], nst[1], nst[P::NST - 1], meta_cur, reinterpret_cast<const char*>(lut));
    __builtin_amdgcn_sched_barrier(0);
    if (!nxt.valid) break;
    // Every wave waited for its part of the next item's half-step 0 in the
    // epilogue; its half-step 1 and this epilogue's stores drain under the
    // next item's half-step 0 (the vmcnt wait at its end covers them).
    lds_barrier();
    cur = nxt;
#pragma unroll
    for (int ql = 0; ql < T::A_INST; ++ql) voff_cur[ql] = voff_nxt[ql];
    b_cur = b_nxt;
    b_cur2 = b_nxt2;
#pragma unroll
    for (int q = 0; q < 3; ++q) st[q] = nst[q];
    char* m = meta_cur;
    meta_cur = meta_nxt;
    meta_nxt = m;
  }
  wait_vmcnt<0>();
#endif
}

}  // namespace

}  // namespace clef
