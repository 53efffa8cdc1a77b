// Omni MoE routing, grouping, SwiGLU and combine for gfx950.
//
// R1 router (kernels/omni_route.loom:84-146): per token, topk rounds of
// "largest remaining logit, ties -> lowest expert id", the selected slot reset
// to -FLT_MAX; routes[t][r] = f32(id), then p_j = exp(v_j - v_0) summed in
// rank order and routes[t][topk+j] = f32(bf16(p_j / sum)).
// R2 grouping (kernels/omni_group_routes.loom:43-82 and the ordered variant
// kernels/omni_group_routes_ordered.loom:50-87): groups[e][0] = count,
// groups[e][1+i] = f32(t*topk + r) for the i-th token (ascending) routed to e
// at rank r; order[t][#(ids < e)] = r.
// S1 (kernels/swiglu.loom:43-51) and C1 (kernels/omni_combine_ordered.loom:51-79,
// kernels/omni_combine.loom:50-77).
#include "common.hpp"
#include "kernels.hpp"
#include "group.hpp"
#include "route.hpp"

namespace clef {

namespace {

__global__ __launch_bounds__(256) void route_kernel(const void* __restrict__ logits, int dtype,
                                                    int64_t tokens, int experts, int topk,
                                                    float* __restrict__ routes) {
  route_impl::route_block(logits, dtype, tokens, experts, topk, routes, blockIdx.x);
}

// ---------------------------------------------------------------- grouping
//
// Three passes over blocks of 64 tokens (one wave, one token per lane):
//   count:   64-bit lane mask per expert (LDS atomic OR), block counts per
//            expert -> workspace [blocks][128]
//   scan:    per expert, exclusive prefix over blocks; counts -> groups[e][0]
//   scatter: rank of (t, r) within expert e = block prefix + popcount of the
//            block's mask below this lane
// Every position is computed, not claimed, so the lists are in ascending
// token order exactly. One-wave blocks give T/64 workgroups: enough to spread
// the scattered writes over the whole GPU. Up to 512 tokens at top-8 one
// workgroup runs all three passes (group_single_kernel).

constexpr int kGroupBlock = 64;

// True when slot r is the last slot of this token naming its expert.
__device__ __forceinline__ bool last_slot(const float* rt, int topk, int r, int e) {
  for (int q = r + 1; q < topk; ++q)
    if (route_expert(rt[q]) == e) return false;
  return true;
}

// KT > 0: topk == KT, the token's KT route ids loaded together before the
// atomics; KT == 0: any topk.
template <int KT>
__device__ void build_masks(const float* __restrict__ routes, int64_t tokens, int topk,
                            unsigned long long* masks /* [128] */) {
  const int lane = threadIdx.x;
  masks[lane] = 0ull;
  masks[64 + lane] = 0ull;
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * kGroupBlock + lane;
  if (t < tokens) {
    const float* rt = routes + t * 2 * topk;
    if constexpr (KT > 0) {
      int ex[KT];
#pragma unroll
      for (int r = 0; r < KT; ++r) ex[r] = route_expert(rt[r]);
#pragma unroll
      for (int r = 0; r < KT; ++r)
        if (ex[r] >= 0) atomicOr(&masks[ex[r]], 1ull << lane);
    } else {
      for (int r = 0; r < topk; ++r) {
        const int e = route_expert(rt[r]);
        if (e >= 0) atomicOr(&masks[e], 1ull << lane);
      }
    }
  }
  __syncthreads();
}

template <int KT>
__global__ __launch_bounds__(64) void group_count_kernel(const float* __restrict__ routes, int64_t tokens,
                                                         int topk, int* __restrict__ block_counts) {
  __shared__ unsigned long long masks[128];
  build_masks<KT>(routes, tokens, topk, masks);
  const int lane = threadIdx.x;
  int* dst = block_counts + (int64_t)blockIdx.x * 128;
  dst[lane] = __popcll(masks[lane]);
  dst[64 + lane] = __popcll(masks[64 + lane]);
}

// One workgroup of 1024 threads: 8 threads per expert, each summing a
// contiguous run of blocks, then an 8-way scan. With `schedule` non-NULL it
// also writes the expert GEMM's tile list: [count] then (expert, first slot)
// pairs, tiles of `bm` slots, experts ascending.
__global__ __launch_bounds__(1024) void group_scan_kernel(int* __restrict__ block_counts, int64_t blocks,
                                                          int64_t tokens, float* __restrict__ groups,
                                                          int32_t* __restrict__ schedule, int bm) {
  __shared__ int part[8][128];
  __shared__ int tiles_scan[129];
  const int e = threadIdx.x & 127, j = threadIdx.x >> 7;
  const int64_t per = (blocks + 7) / 8;
  const int64_t b0 = j * per < blocks ? j * per : blocks;
  const int64_t b1 = b0 + per < blocks ? b0 + per : blocks;
  // The run's counts are read 8 at a time (independent loads in flight
  // together), summed, then rewritten as exclusive prefixes.
  int sum = 0;
  for (int64_t b = b0; b < b1; b += 8) {
    int c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = b + u < b1 ? block_counts[(b + u) * 128 + e] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += c[u];
  }
  part[j][e] = sum;
  __syncthreads();
  int run = 0;
  for (int q = 0; q < j; ++q) run += part[q][e];
  for (int64_t b = b0; b < b1; b += 8) {
    int c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = b + u < b1 ? block_counts[(b + u) * 128 + e] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (b + u < b1) {
        block_counts[(b + u) * 128 + e] = run;
        run += c[u];
      }
  }
  if (j == 7) groups[(int64_t)e * (tokens + 1)] = (float)run;
  if (schedule == nullptr) return;
  write_tile_schedule(run, j == 7, e, bm, tiles_scan, schedule);  // run of thread j == 7 is e's count
}

// The same scan with one 256-thread workgroup per expert, for many blocks
// (above kGroupScanWideBlocks one workgroup's serial runs dominate: 34 us at
// 65536 tokens). Workgroup e scans expert e's column of block counts (each
// thread a contiguous run of blocks, then a workgroup scan of the run sums)
// and writes groups[e][0]. The tile schedule, which needs every expert's
// count, is written by group_scatter_kernel after this launch (a workgroup
// that finished last and wrote it here needed device-scope fences in every
// workgroup: 18 us against 6 us without the schedule at 65536 tokens).
constexpr int64_t kGroupScanWideBlocks = 64;

__global__ __launch_bounds__(256) void group_scan_wide_kernel(int* __restrict__ block_counts, int64_t blocks,
                                                              int64_t tokens, float* __restrict__ groups) {
  __shared__ int wave_sums[4];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t per = (blocks + 255) / 256;
  const int64_t b0 = tid * per < blocks ? tid * per : blocks;
  const int64_t b1 = b0 + per < blocks ? b0 + per : blocks;
  int sum = 0;
  for (int64_t b = b0; b < b1; b += 8) {
    int c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = b + u < b1 ? block_counts[(b + u) * 128 + e] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += c[u];
  }
  // exclusive prefix of the run sums over the workgroup
  int incl = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wave_sums[wave] = incl;
  __syncthreads();
  int run = incl - sum;
  for (int w = 0; w < wave; ++w) run += wave_sums[w];
  const int total = wave_sums[0] + wave_sums[1] + wave_sums[2] + wave_sums[3];
  for (int64_t b = b0; b < b1; b += 8) {
    int c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = b + u < b1 ? block_counts[(b + u) * 128 + e] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (b + u < b1) {
        block_counts[(b + u) * 128 + e] = run;
        run += c[u];
      }
  }
  if (tid == 0) groups[(int64_t)e * (tokens + 1)] = (float)total;
}

// KT > 0: topk == KT, the token's route ids held in registers; KT == 0: any
// topk, read from memory. With `schedule` non-NULL (after the wide scan)
// every workgroup also takes the experts' counts from groups[e][0], forms
// the tiles' prefix (one wave, two experts per lane) and writes its share of
// the schedule entries, one per thread of the grid.
template <int KT>
__global__ __launch_bounds__(64) void group_scatter_kernel(const float* __restrict__ routes, int64_t tokens,
                                                           int topk, const int* __restrict__ block_offsets,
                                                           float* __restrict__ groups, float* __restrict__ order,
                                                           int bm, int32_t* __restrict__ schedule) {
  __shared__ unsigned long long masks[128];
  __shared__ int first[129];
  if constexpr (KT > 0) {
    // Every global load at once: the token's route ids, the block's 128
    // list offsets (to LDS) and, for the tile schedule, the experts' counts.
    // One round trip instead of ids -> offsets.
    const int lane = threadIdx.x;
    const int64_t t = (int64_t)blockIdx.x * kGroupBlock + lane;
    const bool live = t < tokens;
    float id[KT];
#pragma unroll
    for (int r = 0; r < KT; ++r) id[r] = live ? routes[t * 2 * KT + r] : -1.0f;
    __shared__ int offs[128];
    const int* offsets = block_offsets + (int64_t)blockIdx.x * 128;
    const int o0 = offsets[lane], o1 = offsets[64 + lane];
    int c0 = 0, c1 = 0;
    if (schedule != nullptr) {
      c0 = (int)groups[(int64_t)(2 * lane) * (tokens + 1)];
      c1 = (int)groups[(int64_t)(2 * lane + 1) * (tokens + 1)];
    }
    masks[lane] = 0ull;
    masks[64 + lane] = 0ull;
    offs[lane] = o0;
    offs[64 + lane] = o1;
    if (schedule != nullptr) {
      const int t0 = (c0 + bm - 1) / bm, t1 = (c1 + bm - 1) / bm;
      int incl = t0 + t1;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
      }
      first[2 * lane] = incl - t0 - t1;
      first[2 * lane + 1] = incl - t1;
      if (lane == 63) {
        first[128] = incl;
        if (blockIdx.x == 0) schedule[0] = incl;
      }
      if (blockIdx.x == 0 && lane < kSchedEntries - kSchedClaims) schedule[kSchedClaims + lane] = 0;
    }
    __syncthreads();
    int ex[KT];
#pragma unroll
    for (int r = 0; r < KT; ++r) {
      ex[r] = route_expert(id[r]);
      if (ex[r] >= 0) atomicOr(&masks[ex[r]], 1ull << lane);
    }
    __syncthreads();
    if (schedule != nullptr)
      tile_entries(first, bm, (int)(blockIdx.x * 64 + threadIdx.x), (int)(gridDim.x * 64), schedule);
    if (!live) return;
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int r = 0; r < KT; ++r) {
      const int e = ex[r];
      bool last = e >= 0;
#pragma unroll
      for (int q = r + 1; q < KT; ++q) last = last && ex[q] != e;
      if (!last) continue;
      const int rank = offs[e] + __popcll(masks[e] & below);
      groups[(int64_t)e * (tokens + 1) + 1 + rank] = (float)(t * KT + r);
      if (order) {
        int less = 0;
#pragma unroll
        for (int q = 0; q < KT; ++q) less += id[q] < (float)e ? 1 : 0;
        order[t * KT + less] = (float)r;
      }
    }
    return;
  }
  if (schedule != nullptr) {
    const int l = threadIdx.x;
    const int t0 = ((int)groups[(int64_t)(2 * l) * (tokens + 1)] + bm - 1) / bm;
    const int t1 = ((int)groups[(int64_t)(2 * l + 1) * (tokens + 1)] + bm - 1) / bm;
    int incl = t0 + t1;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (l >= off) incl += o;
    }
    first[2 * l] = incl - t0 - t1;
    first[2 * l + 1] = incl - t1;
    if (l == 63) {
      first[128] = incl;
      if (blockIdx.x == 0) schedule[0] = incl;
    }
    if (blockIdx.x == 0 && l < kSchedEntries - kSchedClaims) schedule[kSchedClaims + l] = 0;
  }
  build_masks<KT>(routes, tokens, topk, masks);  // its barriers also order `first`
  if (schedule != nullptr)
    tile_entries(first, bm, (int)(blockIdx.x * 64 + threadIdx.x), (int)(gridDim.x * 64), schedule);
  const int lane = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * kGroupBlock + lane;
  if (t >= tokens) return;
  const float* rt = routes + t * 2 * topk;
  const unsigned long long below = (1ull << lane) - 1ull;
  const int* offsets = block_offsets + (int64_t)blockIdx.x * 128;
  for (int r = 0; r < topk; ++r) {
    const int e = route_expert(rt[r]);
    if (e < 0 || !last_slot(rt, topk, r, e)) continue;
    const int rank = offsets[e] + __popcll(masks[e] & below);
    groups[(int64_t)e * (tokens + 1) + 1 + rank] = (float)(t * topk + r);
    if (order) {
      int less = 0;
      for (int q = 0; q < topk; ++q) less += rt[q] < (float)e ? 1 : 0;
      order[t * topk + less] = (float)r;
    }
  }
}

// The scan and the scatter of top-8 routes in one launch, from counts16
// [rows16][128] (tokens of 16-token block r routed to expert e, written by
// the router): workgroup b (1024 threads) handles the 64-token block b.
// Its 32 row groups of 32 threads each read every 16-token count row with
// 16-byte loads (thread q of a group four experts), keeping the sum of the
// rows of earlier tokens (r < 4b: the list offsets of this block) and of
// all rows (the experts' counts); the 32 partial sums meet in LDS. Wave 0
// then lists the block's tokens as group_scatter_kernel<8> does (masks of
// 64 tokens, rank = offset + popcount below), every workgroup writes its
// share of the tile schedule from the counts, and workgroup 0 writes
// groups[e][0]. Same outputs as the count, scan and scatter launches.
__global__ __launch_bounds__(1024) void group_scatter_scan_kernel(const float* __restrict__ routes, int64_t tokens,
                                                                  const int* __restrict__ counts16, int64_t rows16,
                                                                  float* __restrict__ groups, float* __restrict__ order,
                                                                  int bm, int32_t* __restrict__ schedule) {
  constexpr int KT = 8, RG = 32, U = 8;
  __shared__ int part[2][RG][128];
  __shared__ unsigned long long masks[128];
  __shared__ int offs[128];
  __shared__ int first[129];
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t t = (int64_t)blockIdx.x * kGroupBlock + lane;
  const bool live = tid < 64 && t < tokens;
  float id[KT];
#pragma unroll
  for (int r = 0; r < KT; ++r) id[r] = live ? routes[t * 2 * KT + r] : -1.0f;
  if (tid < 128) masks[tid] = 0ull;
  {
    const int g = tid / 32, q = tid % 32;
    const int64_t split = (int64_t)blockIdx.x * (kGroupBlock / 16);
    int pre[4] = {0, 0, 0, 0}, tot[4] = {0, 0, 0, 0};
    for (int64_t r0 = g; r0 < rows16; r0 += RG * U) {
      int4 c[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t r = r0 + (int64_t)RG * u;
        c[u] = r < rows16 ? *reinterpret_cast<const int4*>(counts16 + r * 128 + 4 * q) : make_int4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool early = r0 + (int64_t)RG * u < split;
        tot[0] += c[u].x, tot[1] += c[u].y, tot[2] += c[u].z, tot[3] += c[u].w;
        if (early) pre[0] += c[u].x, pre[1] += c[u].y, pre[2] += c[u].z, pre[3] += c[u].w;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part[0][g][4 * q + i] = pre[i];
      part[1][g][4 * q + i] = tot[i];
    }
  }
  __syncthreads();
  // threads 0..127: expert tid's count (tile_prefix's holders); 128..255:
  // the list offset of this block for expert tid - 128
  int count = 0;
  if (tid < 256) {
    const int e = tid & 127;
    int sum = 0;
#pragma unroll
    for (int g = 0; g < RG; ++g) sum += part[tid < 128 ? 1 : 0][g][e];
    if (tid < 128)
      count = sum;
    else
      offs[e] = sum;
  }
  if (blockIdx.x == 0 && tid < 128) groups[(int64_t)tid * (tokens + 1)] = (float)count;
  tile_prefix(count, tid < 128, tid & 127, bm, first);
  if (blockIdx.x == 0 && tid == 0) schedule[0] = first[128];
  if (blockIdx.x == 0 && tid < kSchedEntries - kSchedClaims) schedule[kSchedClaims + tid] = 0;
  tile_entries(first, bm, (int)(blockIdx.x * 1024 + tid), (int)(gridDim.x * 1024), schedule);
  if (tid >= 64) return;
  int ex[KT];
#pragma unroll
  for (int r = 0; r < KT; ++r) {
    ex[r] = route_expert(id[r]);
    if (ex[r] >= 0) atomicOr(&masks[ex[r]], 1ull << lane);
  }
  // one wave: its LDS operations complete in order
  if (!live) return;
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int r = 0; r < KT; ++r) {
    const int e = ex[r];
    bool last = e >= 0;
#pragma unroll
    for (int q = r + 1; q < KT; ++q) last = last && ex[q] != e;
    if (!last) continue;
    const int rank = offs[e] + __popcll(masks[e] & below);
    groups[(int64_t)e * (tokens + 1) + 1 + rank] = (float)(t * KT + r);
    if (order) {
      int less = 0;
#pragma unroll
      for (int q = 0; q < KT; ++q) less += id[q] < (float)e ? 1 : 0;
      order[t * KT + less] = (float)r;
    }
  }
}

// The three passes in one workgroup of 16 waves for up to 512 tokens at
// top-8: one launch instead of three, where each pass is a few microseconds
// of latency. (Beyond that the scattered list writes of a single CU cost more
// than the launches saved: 31 us against 16 us at 4096 tokens.) Wave w takes
// the 64-token blocks w, w + 16, ...; each lane keeps its tokens' route ids
// in registers from the first pass to the last. A block's expert masks are
// built in the wave's own 1 KiB of LDS (LDS operations of one wave execute in
// order, so no barrier is needed between clearing, OR-ing and reading them),
// once to count and once to scatter; block counts and their prefixes stay in
// LDS. Same outputs as group_count_kernel, group_scan_kernel and
// group_scatter_kernel<8>.
constexpr int kGroupSingleTokens = 512;
constexpr int kGroupSingleWaves = 16;
constexpr int kGroupSingleBlocks = kGroupSingleTokens / kGroupBlock;  // 8
constexpr int kGroupCountScanBlocks = 16;                               // 1024 tokens

// NB: blocks of 64 tokens it takes (8: up to 512 tokens, all three passes;
// 16: up to 1024 tokens without the scatter, the blocks' prefixes written to
// `block_offsets` for group_scatter_kernel<8>: one launch for count and scan).
template <int NB, bool SCATTER>
__global__ __launch_bounds__(1024) void group_single_kernel(const float* __restrict__ routes, int64_t tokens,
                                                            float* __restrict__ groups, float* __restrict__ order,
                                                            int32_t* __restrict__ schedule, int bm,
                                                            int* __restrict__ block_offsets) {
  constexpr int KT = 8;
  constexpr int kGroupSinglePer = (NB + kGroupSingleWaves - 1) / kGroupSingleWaves;  // blocks per wave
  __shared__ unsigned long long masks[kGroupSingleWaves][128];
  __shared__ int offs[NB][128];
  __shared__ int part[8][128];
  __shared__ int tiles_scan[129];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int blocks = (int)((tokens + kGroupBlock - 1) / kGroupBlock);
  float id[kGroupSinglePer][KT];
  int ex[kGroupSinglePer][KT];
#pragma unroll
  for (int s = 0; s < kGroupSinglePer; ++s) {
    const int64_t t = (int64_t)(wave + kGroupSingleWaves * s) * kGroupBlock + lane;
    if (t < tokens) {
#pragma unroll
      for (int r = 0; r < KT; ++r) id[s][r] = routes[t * 2 * KT + r];
    } else {
#pragma unroll
      for (int r = 0; r < KT; ++r) id[s][r] = -1.0f;
    }
#pragma unroll
    for (int r = 0; r < KT; ++r) ex[s][r] = route_expert(id[s][r]);
  }
  unsigned long long* m = masks[wave];
  auto build = [&](int s) {
    m[lane] = 0ull;
    m[64 + lane] = 0ull;
#pragma unroll
    for (int r = 0; r < KT; ++r)
      if (ex[s][r] >= 0) atomicOr(&m[ex[s][r]], 1ull << lane);
  };
  // counts
#pragma unroll
  for (int s = 0; s < kGroupSinglePer; ++s) {
    const int b = wave + kGroupSingleWaves * s;
    if (b >= blocks) break;
    build(s);
    offs[b][lane] = __popcll(m[lane]);
    offs[b][64 + lane] = __popcll(m[64 + lane]);
  }
  __syncthreads();
  // per expert, exclusive prefix over blocks (8 threads per expert, each a
  // contiguous run of blocks)
  {
    const int e = threadIdx.x & 127, j = threadIdx.x >> 7;
    const int per = (blocks + 7) / 8;
    const int b0 = j * per < blocks ? j * per : blocks;
    const int b1 = b0 + per < blocks ? b0 + per : blocks;
    int sum = 0;
    for (int b = b0; b < b1; ++b) sum += offs[b][e];
    part[j][e] = sum;
    __syncthreads();
    int run = 0;
    for (int q = 0; q < j; ++q) run += part[q][e];
    for (int b = b0; b < b1; ++b) {
      const int c = offs[b][e];
      offs[b][e] = run;
      run += c;
    }
    if (j == 7) groups[(int64_t)e * (tokens + 1)] = (float)run;
    if (!SCATTER)
      for (int b = b0; b < b1; ++b) block_offsets[b * 128 + e] = offs[b][e];
    if (schedule != nullptr) write_tile_schedule(run, j == 7, e, bm, tiles_scan, schedule);
  }
  if (!SCATTER) return;
  __syncthreads();
  // scatter
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int s = 0; s < kGroupSinglePer; ++s) {
    const int b = wave + kGroupSingleWaves * s;
    if (b >= blocks) break;
    build(s);
    const int64_t t = (int64_t)b * kGroupBlock + lane;
    if (t >= tokens) continue;
#pragma unroll
    for (int r = 0; r < KT; ++r) {
      const int e = ex[s][r];
      bool last = e >= 0;
#pragma unroll
      for (int q = r + 1; q < KT; ++q) last = last && ex[s][q] != e;
      if (!last) continue;
      const int rank = offs[b][e] + __popcll(m[e] & below);
      groups[(int64_t)e * (tokens + 1) + 1 + rank] = (float)(t * KT + r);
      if (order) {
        int less = 0;
#pragma unroll
        for (int q = 0; q < KT; ++q) less += id[s][q] < (float)e ? 1 : 0;
        order[t * KT + less] = (float)r;
      }
    }
  }
}

// ---------------------------------------------------------------- S1, C1

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ gate,
                                                     const uint16_t* __restrict__ up, int64_t n,
                                                     uint16_t* __restrict__ h) {
  const int64_t i8 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i8 + 8 <= n) {
    const uint4 g = *reinterpret_cast<const uint4*>(gate + i8);
    const uint4 u = *reinterpret_cast<const uint4*>(up + i8);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t hw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = f32_to_bf16(swiglu1(bf16_lo(gw[q]), bf16_lo(uw[q])));
      const uint32_t hi = f32_to_bf16(swiglu1(bf16_hi(gw[q]), bf16_hi(uw[q])));
      hw[q] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(h + i8) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  } else {
    for (int64_t i = i8; i < n; ++i)
      h[i] = (uint16_t)f32_to_bf16(swiglu1(bf16_to_f32(gate[i]), bf16_to_f32(up[i])));
  }
}

// One thread per (token, 8 columns).
// KT > 0: topk == KT; the ranks, their probabilities and all KT value chunks
// are loaded before the ordered accumulation, so a thread waits for memory
// twice instead of once per rank. KT == 0: any topk, rank by rank.
template <int KT>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ values,
                                                      const float* __restrict__ routes,
                                                      const float* __restrict__ order, int64_t tokens,
                                                      int width, int topk, uint16_t* __restrict__ out) {
  const int chunks = width / 8;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= tokens * chunks) return;
  const int64_t t = id / chunks;
  const int c = (int)(id - t * chunks) * 8;
  const float* rt = routes + t * 2 * topk;
  float acc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
  if constexpr (KT > 0) {
    int rank[KT];
    if (order) {
#pragma unroll
      for (int j = 0; j < KT; ++j) rank[j] = order_slot(order[t * KT + j], KT);
    } else {
      float ids[KT];
#pragma unroll
      for (int r = 0; r < KT; ++r) ids[r] = rt[r];
      float prev = -1.0f;
#pragma unroll
      for (int j = 0; j < KT; ++j) {
        float best = 1000000.0f;
        int rk = 0;
#pragma unroll
        for (int r = 0; r < KT; ++r)
          if (ids[r] > prev && ids[r] < best) {
            best = ids[r];
            rk = r;
          }
        prev = best;
        rank[j] = rk;
      }
    }
    float p[KT];
    uint4 v[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      p[j] = rt[KT + rank[j]];
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(values + ((t * KT + rank[j]) * width + c)));
      v[j] = make_uint4(q.x, q.y, q.z, q.w);
    }
#pragma unroll
    for (int j = 0; j < KT; ++j) {
      const uint32_t vw[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] = bf16_round(acc[2 * q] + bf16_round(bf16_lo(vw[q]) * p[j]));
        acc[2 * q + 1] = bf16_round(acc[2 * q + 1] + bf16_round(bf16_hi(vw[q]) * p[j]));
      }
    }
    uint32_t ow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) ow[q] = f32_to_bf16(acc[2 * q]) | (f32_to_bf16(acc[2 * q + 1]) << 16);
    *reinterpret_cast<uint4*>(out + t * width + c) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    return;
  }
  float prev = -1.0f;
  for (int j = 0; j < topk; ++j) {
    int rank;
    if (order) {
      rank = order_slot(order[t * topk + j], topk);
    } else {
      // j-th smallest expert id (kernels/omni_combine.loom:50-77).
      float best = 1000000.0f;
      rank = 0;
      for (int r = 0; r < topk; ++r)
        if (rt[r] > prev && rt[r] < best) {
          best = rt[r];
          rank = r;
        }
      prev = best;
    }
    const float p = rt[topk + rank];
    const uint4 v = *reinterpret_cast<const uint4*>(values + ((t * topk + rank) * width + c));
    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] = bf16_round(acc[2 * q] + bf16_round(bf16_lo(vw[q]) * p));
      acc[2 * q + 1] = bf16_round(acc[2 * q + 1] + bf16_round(bf16_hi(vw[q]) * p));
    }
  }
  uint32_t ow[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) ow[q] = f32_to_bf16(acc[2 * q]) | (f32_to_bf16(acc[2 * q + 1]) << 16);
  *reinterpret_cast<uint4*>(out + t * width + c) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

}  // namespace

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Router gate projection: logits[t][e] = bf16(sum_k x[t][k] * w[e][k]) with
// f32 accumulation on the bf16 MFMA -- the bf16 linear that produces the
// Omni router logits (src/omni.rs:764 -> Engine::linear, src/ops.rs:95-175,
// kernels/gemm_bf16_reference.loom). One workgroup per 32 tokens; wave w
// computes experts 32w..32w+31 (x in the MFMA A slot, so lane l holds expert
// 32w + l%32 for tokens 8(i/4) + 4(l/32) + i%4, i < 16). No barriers: waves
// past the expert count leave at once.
__global__ __launch_bounds__(256) void router_gate_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w, int64_t tokens,
                                                          int hidden, int experts, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e0 = wave * 32;
  if (e0 >= experts) return;
  const int64_t t0 = (int64_t)blockIdx.x * 32;
  const int r = lane & 31, kb = (lane >> 5) * 8;
  const bool tok_ok = t0 + r < tokens;
  const uint16_t* xa = x + (tok_ok ? t0 + r : 0) * (int64_t)hidden + kb;
  const uint16_t* wb = w + (int64_t)(e0 + r) * hidden + kb;
  v16f acc = {};
  // hidden % 64 == 0: four 16-k MFMAs per iteration, their loads issued first
  for (int k = 0; k < hidden; k += 64) {
    u4 a[4], b[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      a[s] = tok_ok ? *reinterpret_cast<const u4*>(xa + k + 16 * s) : u4{0u, 0u, 0u, 0u};
      b[s] = *reinterpret_cast<const u4*>(wb + k + 16 * s);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a[s]),
                                                    __builtin_bit_cast(bf16x8_t, b[s]), acc, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t t = t0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (t < tokens) out[t * experts + e0 + r] = (uint16_t)f32_to_bf16(acc[i]);
  }
}

hipError_t launch_router_gate(const uint16_t* x, const uint16_t* w, int64_t tokens, int hidden, int experts,
                              uint16_t* out, hipStream_t stream) {
  const int64_t blocks = (tokens + 31) / 32;
  if (blocks == 0) return hipSuccess;
  router_gate_kernel<<<(unsigned)blocks, 256, 0, stream>>>(x, w, tokens, hidden, experts, out);
  return hipGetLastError();
}

hipError_t launch_route(const void* logits, int dtype, int64_t tokens, int experts, int topk,
                        float* routes, hipStream_t stream) {
  const int per = route_impl::route_tokens_per_block(topk);
  const int64_t blocks = (tokens + per - 1) / per;
  route_kernel<<<(unsigned)blocks, 256, 0, stream>>>(logits, dtype, tokens, experts, topk, routes);
  return hipGetLastError();
}

// Tokens up to which the MoE layer groups from the router's per-16-token
// counts (route_prepare_kernel, then group_scatter_scan_kernel) instead of
// the count, scan and scatter launches. Every workgroup of the second
// launch reads all ceil(tokens / 16) count rows (512 bytes each).
constexpr int64_t kGroupCountedTokens = 8192;

bool group_counted_fusable(int64_t tokens, int topk) {
  return topk == 8 && tokens > kGroupCountScanBlocks * kGroupBlock && tokens <= kGroupCountedTokens;
}

size_t group_workspace_bytes(int64_t tokens) {
  const int64_t blocks = (tokens + kGroupBlock - 1) / kGroupBlock;
  return (size_t)blocks * 128 * sizeof(int);
}

size_t group_counted_bytes(int64_t tokens) { return (size_t)((tokens + 15) / 16) * 128 * sizeof(int); }

namespace {
__global__ __launch_bounds__(256) void route_slots_kernel(const float* __restrict__ routes, int64_t slots_n,
                                                          int topk, float* __restrict__ slots) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= slots_n) return;
  const int64_t t = j / topk;
  slots[2 * j] = routes[t * 2 * topk + (j - t * topk)];
  slots[2 * j + 1] = 0.0f;
}
}  // namespace

hipError_t launch_route_slots(const float* routes, int64_t tokens, int topk, float* slots, hipStream_t stream) {
  const int64_t n = tokens * topk;
  route_slots_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(routes, n, topk, slots);
  return hipGetLastError();
}

hipError_t launch_group_routes(const float* routes, int64_t tokens, int topk, float* groups,
                               float* order, void* workspace, hipStream_t stream, int32_t* schedule,
                               int schedule_bm) {
  if (topk == 8 && tokens <= kGroupSingleTokens) {
    group_single_kernel<kGroupSingleBlocks, true><<<1, 1024, 0, stream>>>(routes, tokens, groups, order, schedule,
                                                                          schedule_bm, nullptr);
    return hipGetLastError();
  }
  const int64_t blocks = (tokens + kGroupBlock - 1) / kGroupBlock;
  int* counts = static_cast<int*>(workspace);
  if (topk == 8 && blocks <= kGroupCountScanBlocks) {
    group_single_kernel<kGroupCountScanBlocks, false><<<1, 1024, 0, stream>>>(routes, tokens, groups, order,
                                                                              schedule, schedule_bm, counts);
    group_scatter_kernel<8><<<(unsigned)blocks, 64, 0, stream>>>(routes, tokens, topk, counts, groups, order,
                                                                 schedule_bm, nullptr);
    return hipGetLastError();
  }
  if (topk == 8)
    group_count_kernel<8><<<(unsigned)blocks, 64, 0, stream>>>(routes, tokens, topk, counts);
  else
    group_count_kernel<0><<<(unsigned)blocks, 64, 0, stream>>>(routes, tokens, topk, counts);
  const bool wide = blocks > kGroupScanWideBlocks;
  if (wide)
    group_scan_wide_kernel<<<128, 256, 0, stream>>>(counts, blocks, tokens, groups);
  else
    group_scan_kernel<<<1, 1024, 0, stream>>>(counts, blocks, tokens, groups, schedule, schedule_bm);
  int32_t* scatter_schedule = wide ? schedule : nullptr;
  if (topk == 8)
    group_scatter_kernel<8><<<(unsigned)blocks, 64, 0, stream>>>(routes, tokens, topk, counts, groups, order,
                                                                 schedule_bm, scatter_schedule);
  else
    group_scatter_kernel<0><<<(unsigned)blocks, 64, 0, stream>>>(routes, tokens, topk, counts, groups, order,
                                                                 schedule_bm, scatter_schedule);
  return hipGetLastError();
}

hipError_t launch_group_counted(const float* routes, int64_t tokens, const int* counts16, float* groups,
                                float* order, int32_t* schedule, int schedule_bm, hipStream_t stream) {
  if (!group_counted_fusable(tokens, 8) || schedule == nullptr) return hipErrorInvalidValue;
  const int64_t blocks = (tokens + kGroupBlock - 1) / kGroupBlock;
  group_scatter_scan_kernel<<<(unsigned)blocks, 1024, 0, stream>>>(routes, tokens, counts16, (tokens + 15) / 16,
                                                                   groups, order, schedule_bm, schedule);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h,
                         hipStream_t stream) {
  const int64_t threads = (n + 7) / 8;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks == 0) return hipSuccess;
  swiglu_kernel<<<(unsigned)blocks, 256, 0, stream>>>(gate, up, n, h);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* values, const float* routes, const float* order,
                          int64_t tokens, int width, int topk, uint16_t* out, hipStream_t stream) {
  const int64_t threads = tokens * (width / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks == 0) return hipSuccess;
  if (topk == 8)
    combine_kernel<8><<<(unsigned)blocks, 256, 0, stream>>>(values, routes, order, tokens, width, topk, out);
  else
    combine_kernel<0><<<(unsigned)blocks, 256, 0, stream>>>(values, routes, order, tokens, width, topk, out);
  return hipGetLastError();
}

}  // namespace clef
