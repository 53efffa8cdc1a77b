// R1 router body (kernels/omni_route.loom:84-146), shared by route_kernel and
// the launch that runs the router beside the activation quantizer: per token,
// topk rounds of "largest remaining logit, ties -> lowest expert id", the
// selected slot reset to -FLT_MAX; routes[t][r] = f32(id), then
// p_j = exp(v_j - v_0) summed in rank order and
// routes[t][topk+j] = f32(bf16(p_j / sum)).
#pragma once

#include "common.hpp"

namespace clef {
namespace route_impl {

constexpr float kNegMax = -3.402823466e38f;
constexpr int kInvalidId = 2147483647;

// Wave-wide reductions with every lane active: within each row of 16 lanes by
// DPP (quad_perm [1,0,3,2] and [2,3,0,1], then row_ror 4 and 8: every lane
// ends with its row's result), then across the four rows by readlane. Each
// step is a few cycles, against an LDS round trip per step for a
// ds_bpermute shuffle. Max and min are exact in any order.
template <int CTRL>
__device__ __forceinline__ int dpp_row(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float wave_max(float v) {
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0xB1>((int)as_uint(v))));
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x4E>((int)as_uint(v))));
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x124>((int)as_uint(v))));
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x128>((int)as_uint(v))));
  const int b = (int)as_uint(v);
  const float r0 = as_float((uint32_t)__builtin_amdgcn_readlane(b, 0));
  const float r1 = as_float((uint32_t)__builtin_amdgcn_readlane(b, 16));
  const float r2 = as_float((uint32_t)__builtin_amdgcn_readlane(b, 32));
  const float r3 = as_float((uint32_t)__builtin_amdgcn_readlane(b, 48));
  return __builtin_fmaxf(__builtin_fmaxf(r0, r1), __builtin_fmaxf(r2, r3));
}

__device__ __forceinline__ int wave_min(int v) {
  int o = dpp_row<0xB1>(v);
  v = o < v ? o : v;
  o = dpp_row<0x4E>(v);
  v = o < v ? o : v;
  o = dpp_row<0x124>(v);
  v = o < v ? o : v;
  o = dpp_row<0x128>(v);
  v = o < v ? o : v;
  const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  const int a = r0 < r1 ? r0 : r1, c = r2 < r3 ? r2 : r3;
  return a < c ? a : c;
}

// One wave per token, four tokens per 256-thread workgroup `block`; lane l
// holds expert slots 2l and 2l+1 (E <= 128).
__device__ __forceinline__ void route_body(const void* __restrict__ logits, int dtype, int64_t tokens,
                                           int experts, int topk, float* __restrict__ routes, int64_t block) {
  const int lane = threadIdx.x & 63;
  const int64_t t = block * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;
  float v[2];
  bool valid[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int e = 2 * lane + s;
    valid[s] = e < experts;
    if (!valid[s]) {
      v[s] = kNegMax;
    } else if (dtype == 0) {
      v[s] = bf16_to_f32(static_cast<const uint16_t*>(logits)[t * experts + e]);
    } else {
      v[s] = static_cast<const float*>(logits)[t * experts + e];
    }
  }
  float* out = routes + t * 2 * topk;
  // Rank r is kept by lane r % 64 (slot r / 64): selected value and id.
  float rv[2] = {0.0f, 0.0f};
  int rid[2] = {0, 0};
  for (int r = 0; r < topk; ++r) {
    const float best = wave_max(__builtin_fmaxf(v[0], v[1]));
    int cand = kInvalidId;
    if (valid[1] && v[1] == best) cand = 2 * lane + 1;
    if (valid[0] && v[0] == best) cand = 2 * lane;
    const int id = wave_min(cand);
    if (lane == (r & 63)) {
      rv[r >> 6] = best;
      rid[r >> 6] = id;
    }
    if (id == 2 * lane) v[0] = kNegMax;
    if (id == 2 * lane + 1) v[1] = kNegMax;
  }
  // exp of every rank in parallel, the sum in rank order (as the reference's
  // sequential loop), the divisions in parallel.
  const float vmax = as_float((uint32_t)__builtin_amdgcn_readlane((int)as_uint(rv[0]), 0));
  float p[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) p[s] = 64 * s + lane < topk ? cephes_expf(rv[s] - vmax) : 0.0f;
  float sum = 0.0f;
  const int pb0 = (int)as_uint(p[0]), pb1 = (int)as_uint(p[1]);
  for (int r = 0; r < topk; ++r)  // r is wave-uniform: readlane of lane r % 64
    sum = sum + as_float((uint32_t)__builtin_amdgcn_readlane(r < 64 ? pb0 : pb1, r & 63));
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = 64 * s + lane;
    if (r < topk) {
      out[r] = (float)rid[s];
      out[topk + r] = bf16_round(p[s] / sum);
    }
  }
}

// Reductions over one 16-lane DPP row (every lane ends with the row's result).
__device__ __forceinline__ float row_max(float v) {
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0xB1>((int)as_uint(v))));
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x4E>((int)as_uint(v))));
  v = __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x124>((int)as_uint(v))));
  return __builtin_fmaxf(v, as_float((uint32_t)dpp_row<0x128>((int)as_uint(v))));
}

__device__ __forceinline__ int row_min(int v) {
  int o = dpp_row<0xB1>(v);
  v = o < v ? o : v;
  o = dpp_row<0x4E>(v);
  v = o < v ? o : v;
  o = dpp_row<0x124>(v);
  v = o < v ? o : v;
  o = dpp_row<0x128>(v);
  return o < v ? o : v;
}

// Tokens per 256-thread workgroup of route_body16.
constexpr int kRouteTokens16 = 16;

// The same router with 16 lanes per token (topk <= 16): each 16-lane DPP row
// of a wave routes one token, four per wave, and lane i of the row holds
// expert slots 8i .. 8i+7. A rank is a row maximum (fmaxf: the order of the
// maxima does not matter, NaN is ignored), the lowest valid slot holding it
// (a row minimum of candidate ids) and that slot reset to -FLT_MAX: a third
// of the instructions per token of the one-wave-per-token body, whose
// reductions span 64 lanes for two slots each. Rank r is kept by lane r of
// the row; the softmax sum runs in rank order over the row's lanes.
// With `ids` non-NULL the ranks' expert ids also go to LDS: ids[8 * (token in
// the block) + rank] (topk <= 8).
__device__ __forceinline__ void route_body16(const void* __restrict__ logits, int dtype, int64_t tokens,
                                             int experts, int topk, float* __restrict__ routes, int64_t block,
                                             int* ids = nullptr, bool write_routes = true) {
  const int lane = threadIdx.x & 63, li = lane & 15;
  const int64_t t = block * kRouteTokens16 + (threadIdx.x >> 4);
  const bool live = t < tokens;  // every lane stays on for the row reductions
  const int e0 = 8 * li;
  float v[8];
  bool valid[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) valid[j] = e0 + j < experts;
  // 16-byte loads when every row starts on a 16-byte boundary (the C ABI
  // requires a 16-byte aligned logits pointer); element loads otherwise.
  if (live && dtype == 0 && experts % 8 == 0 && e0 < experts) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(logits) + t * experts + e0);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_lo(w[j]);
      v[2 * j + 1] = bf16_hi(w[j]);
    }
  } else if (live && dtype == 1 && experts % 4 == 0 && e0 < experts) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(logits) + t * experts + e0);
    const float4 a = p[0];
    const float4 b = e0 + 4 < experts ? p[1] : make_float4(kNegMax, kNegMax, kNegMax, kNegMax);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = e0 + j;
      if (!live || e >= experts)
        v[j] = kNegMax;
      else if (dtype == 0)
        v[j] = bf16_to_f32(static_cast<const uint16_t*>(logits)[t * experts + e]);
      else
        v[j] = static_cast<const float*>(logits)[t * experts + e];
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (!valid[j]) v[j] = kNegMax;
  float rv = 0.0f;  // this lane's rank (r == li): value and id
  int rid = 0;
  for (int r = 0; r < topk; ++r) {
    float m = v[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) m = __builtin_fmaxf(m, v[j]);
    const float best = row_max(m);
    int cand = kInvalidId;
#pragma unroll
    for (int j = 7; j >= 0; --j)
      if (valid[j] && v[j] == best) cand = e0 + j;
    const int id = row_min(cand);
    if (li == r) {
      rv = best;
      rid = id;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (id == e0 + j) v[j] = kNegMax;
  }
  // exp of every rank in parallel, the sum in rank order (the reference's
  // sequential loop) from the row's lanes, the divisions in parallel.
  const int row0 = lane & 48;
  const float vmax = __shfl(rv, row0, 64);
  const float p = li < topk ? cephes_expf(rv - vmax) : 0.0f;
  float sum = 0.0f;
  for (int r = 0; r < topk; ++r) sum = sum + __shfl(p, row0 + r, 64);
  if (live && li < topk) {
    if (write_routes) {
      float* out = routes + t * 2 * topk;
      out[li] = (float)rid;
      out[topk + li] = bf16_round(p / sum);
    }
    if (ids != nullptr) ids[8 * (threadIdx.x >> 4) + li] = rid;
  }
}

// Tokens per 256-thread workgroup for a topk, and the body that routes them.
__host__ __device__ __forceinline__ int route_tokens_per_block(int topk) { return topk <= 16 ? kRouteTokens16 : 4; }

__device__ __forceinline__ void route_block(const void* __restrict__ logits, int dtype, int64_t tokens, int experts,
                                            int topk, float* __restrict__ routes, int64_t block) {
  if (topk <= 16)
    route_body16(logits, dtype, tokens, experts, topk, routes, block);
  else
    route_body(logits, dtype, tokens, experts, topk, routes, block);
}

}  // namespace route_impl
}  // namespace clef
