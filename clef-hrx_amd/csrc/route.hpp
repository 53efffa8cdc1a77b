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

}  // namespace route_impl
}  // namespace clef
