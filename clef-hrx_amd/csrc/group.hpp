// Grouping helpers shared by the grouping kernels and the router launch
// (kernels/omni_group_routes.loom:43-82, kernels/omni_group_routes_ordered.loom:50-87):
// groups[e][0] = count, groups[e][1+i] = f32(t*topk + r) for the i-th token
// (ascending) routed to e at rank r, a token naming e in several slots listed
// once at its last such slot; order[t][#(ids < e)] = r; and the grouped
// expert GEMM's tile schedule.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace clef {

// Expert id of route slot r, or -1 when the slot names no expert in 0..127
// (the oracle compares (int32_t)id against each expert).
__device__ __forceinline__ int route_expert(float id) {
  return (id > -1.0f && id < 128.0f) ? (int)id : -1;
}

// Slot named by combine-order entry `o` of a token with `topk` slots. The
// grouping writes an entry for each expert a token names, so a token naming
// an expert twice or naming none (logit rows with NaN, or with fewer than
// topk values above -FLT_MAX) leaves entries unwritten; an entry outside
// [0, topk) then reads slot 0, never memory past the token's rows. Such a
// token's output is unspecified, as in the reference.
__device__ __forceinline__ int order_slot(float o, int topk) { return o >= 0.0f && o < (float)topk ? (int)o : 0; }

// The expert GEMM's tile list from the experts' counts: tiles of bm slots,
// schedule = [total] then (expert, first slot) per tile, experts ascending.
//
// tile_prefix: `holder` threads (one per expert e) pass e's count; every
// thread of the workgroup calls it. The tile counts' exclusive prefix is one
// wave's scan, two experts per lane, between two barriers; afterwards
// first[e] is expert e's first tile and first[128] the total.
__device__ inline void tile_prefix(int count, bool holder, int e, int bm, int* first /* [129] */) {
  if (holder) first[e] = (count + bm - 1) / bm;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    const int t0 = first[2 * l], t1 = first[2 * l + 1];
    int incl = t0 + t1;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (l >= off) incl += o;
    }
    first[2 * l] = incl - t0 - t1;
    first[2 * l + 1] = incl - t1;
    if (l == 63) first[128] = incl;
  }
  __syncthreads();
}

// Schedule entries t = t0, t0 + stride, ... below first[128]: tile t's
// expert is the last one whose first tile is at or below t (experts without
// tiles share the next one's first tile and are passed over).
__device__ __forceinline__ void tile_entries(const int* first, int bm, int t0, int stride,
                                             int32_t* __restrict__ schedule) {
  const int total = first[128];
  for (int t = t0; t < total; t += stride) {
    int lo = 0, hi = 127;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (first[mid] <= t)
        lo = mid;
      else
        hi = mid - 1;
    }
    schedule[kSchedEntries + 2 * t] = lo;
    schedule[kSchedEntries + 1 + 2 * t] = (t - first[lo]) * bm;
  }
}

// The whole schedule from one workgroup (few tiles: up to 4096 tokens).
__device__ inline void write_tile_schedule(int count, bool holder, int e, int bm, int* first /* [129] */,
                                    int32_t* __restrict__ schedule) {
  tile_prefix(count, holder, e, bm, first);
  if (threadIdx.x == 0) schedule[0] = first[128];
  if (threadIdx.x < kSchedEntries - kSchedClaims) schedule[kSchedClaims + threadIdx.x] = 0;
  tile_entries(first, bm, threadIdx.x, blockDim.x, schedule);
}

// Grouping of at most 16 tokens at top-8 by the 256-thread workgroup that
// has just routed them, from their expert ids in LDS (ids[8t + r], written
// before the caller's barrier): slot i is listed when it is its token's last
// slot naming its expert; bit i of expert e's 128-bit mask marks it, so its
// list position is the popcount below it (ascending token order) and e's
// count the mask's popcount. The same tables as the three-pass grouping.
__device__ inline void group_small(const int* ids, int tokens, float* __restrict__ groups, float* __restrict__ order,
                                   int32_t* __restrict__ schedule, int bm) {
  __shared__ unsigned long long masks[2][128];
  __shared__ int first[129];
  const int tid = threadIdx.x;
  const int n = tokens * 8;
  int e = -1;
  bool listed = false;
  if (tid < n) {
    e = ids[tid];
    e = e >= 0 && e < 128 ? e : -1;
    listed = e >= 0;
    for (int q = tid + 1; q <= (tid | 7); ++q) listed = listed && ids[q] != e;
  }
  if (tid < 128) {
    masks[0][tid] = 0ull;
    masks[1][tid] = 0ull;
  }
  __syncthreads();
  if (listed) atomicOr(&masks[tid >> 6][e], 1ull << (tid & 63));
  __syncthreads();
  if (listed) {
    const unsigned long long below = (1ull << (tid & 63)) - 1ull;
    const int rank = tid < 64 ? __popcll(masks[0][e] & below) : __popcll(masks[0][e]) + __popcll(masks[1][e] & below);
    groups[(int64_t)e * (tokens + 1) + 1 + rank] = (float)tid;
    if (order != nullptr) {
      const int t = tid >> 3;
      int less = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) less += ids[8 * t + q] < e ? 1 : 0;
      order[8 * t + less] = (float)(tid & 7);
    }
  }
  int count = 0;
  if (tid < 128) {
    count = __popcll(masks[0][tid]) + __popcll(masks[1][tid]);
    groups[(int64_t)tid * (tokens + 1)] = (float)count;
  }
  if (schedule != nullptr) write_tile_schedule(count, tid < 128, tid & 127, bm, first, schedule);
}

}  // namespace clef
