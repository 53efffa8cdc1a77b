// Launchers of the gfx950 kernels (internal to the library; the public
// boundary is include/clef_i4.h). Each returns the launch's hipError_t and
// assumes the caller already checked every shape and alignment precondition.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace clef {

// bf6 activation layout (this library's own, the bf6 weight's block shape
// without its swizzle): blocks of 128 rows x 128 k, each 12 KiB of 96-byte
// rows (value k of a row at bits 6k of its 96 bytes, little-endian), block
// (r / 128, k / 128) at byte ((r / 128) * (K / 128) + k / 128) * 12288, row
// r % 128 of a block at (r % 128) * 96. Rows of the last block past `rows`
// are padding that no kernel writes and the GEMMs never store. The f32 row
// scales of a prepared buffer follow the codes.
constexpr int64_t f6_codes_bytes(int64_t rows, int64_t width) { return (rows + 127) / 128 * 128 * width * 3 / 4; }
constexpr int64_t f6_offset(int64_t row, int64_t col, int64_t width) {
  return ((row >> 7) * (width >> 7) + (col >> 7)) * 12288 + (row & 127) * 96 + (col & 127) * 3 / 4;
}

hipError_t launch_prepare(const uint16_t* x, int64_t rows, int width, int stride, int bits,
                          uint32_t* out, hipStream_t stream);
// The router and the INT4 quantizer of `x` ([tokens][width], stride as
// launch_prepare) in one launch; only for widths the grid-stride quantizer
// takes (route_prepare_fusable).
bool route_prepare_fusable(int width);
// With `groups` non-NULL (route_group_fusable) the routing workgroup also
// writes the grouping tables and tile schedule (tiles of `bm` slots), as
// launch_group_routes would. With `counts16` non-NULL (top-8) it writes the
// per-16-token expert counts launch_group_counted reads.
bool route_group_fusable(int64_t tokens, int topk);
hipError_t launch_route_prepare(const void* logits, int dtype, int64_t tokens, int experts, int topk,
                                float* routes, const uint16_t* x, int width, int stride, uint32_t* out,
                                hipStream_t stream, float* groups = nullptr, float* order = nullptr,
                                int32_t* schedule = nullptr, int bm = 0, int* counts16 = nullptr);
hipError_t launch_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows, int width,
                                 int stride, int bits, uint32_t* out, hipStream_t stream);
hipError_t launch_prepare_attention_gate(const uint16_t* x, const uint16_t* q_gate, int64_t rows, int width,
                                         int stride, int bits, uint32_t* out, hipStream_t stream);
hipError_t launch_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int width, int stride,
                               int bits, uint32_t* out, uint16_t* normalized, hipStream_t stream);
hipError_t launch_retile(const uint32_t* codes, int64_t rows, int in_words, int words,
                         uint32_t* tiled, hipStream_t stream);
hipError_t launch_tile_permute(const uint16_t* src, int64_t rows, int cols, uint16_t* dst,
                               bool to_tiled, hipStream_t stream);

hipError_t launch_gemm_i4(const uint32_t* a, int a_words, const float* a_scales,
                          const uint32_t* w_tiled, const float* w_scales, int64_t m, int n, int k,
                          const uint16_t* residual, uint16_t* out, int config, hipStream_t stream);
// INT8 x INT8 G1 (codes 4 per word, weights tiled as retile_codes with bits 8).
hipError_t launch_gemm_i8(const uint32_t* a, int a_words, const float* as, const uint32_t* w, const float* ws,
                          int64_t m, int n, int k, const uint16_t* residual, uint16_t* out, hipStream_t stream);
// bf6 (e3m2) operands for G1 (gemm_f6.hip): packed activation rows -> bf6
// rows of k * 3/4 bytes; tiled INT4 weight -> bf6 tiled weight; the GEMM on
// them (k % 128 == 0, n % 256 == 0).
hipError_t launch_f6_rows(const uint32_t* a, int a_words, int64_t rows, int k, uint8_t* out, hipStream_t stream);
hipError_t launch_f6_tiled(const uint32_t* w_tiled, int64_t n, int k, uint8_t* out, hipStream_t stream);
hipError_t launch_gemm_f6(const uint8_t* a, const float* as, const uint8_t* w, const float* ws, int64_t m, int n,
                          int k, const uint16_t* residual, uint16_t* out, hipStream_t stream);
// Gate and up projections with SwiGLU on the bf6 forms: h [m][n] (n % 128 == 0).
hipError_t launch_gemm_f6_gate_up(const uint8_t* a, const float* as, const uint8_t* gate_w, const float* gate_s,
                                  const uint8_t* up_w, const float* up_s, int64_t m, int n, int k, uint16_t* h,
                                  hipStream_t stream);
// Records msg as clef_last_error() of this thread; returns CLEF_EINVAL.
int set_last_error(const char* msg);
// G1 tile configurations (clef_i4_gemm_config): 128x128 tiles, 256x256
// tiles with one workgroup per tile, 256x256 tiles walked by a persistent
// grid, and the K-split small-M kernel.
enum GemmConfig {
  kGemmTile128 = 0,
  kGemmTile256 = 1,
  kGemmPersist256 = 2,
  kGemmSkinny = 3,
  kGemmDecode = 4,
  kGemmKsplit = 5,
  kGemmConfigs = 6
};
int gemm_config_count();

hipError_t launch_router_gate(const uint16_t* x, const uint16_t* w, int64_t tokens, int hidden, int experts,
                              uint16_t* out, hipStream_t stream);
hipError_t launch_route(const void* logits, int dtype, int64_t tokens, int experts, int topk,
                        float* routes, hipStream_t stream);
size_t group_workspace_bytes(int64_t tokens);
// The grouping of top-8 routes from the per-16-token expert counts that
// launch_route_prepare wrote (counts16 [ceil(tokens / 16)][128] int32,
// group_counted_bytes): the scan and the scatter in one launch, with the same
// outputs as launch_group_routes. For group_counted_fusable token counts.
bool group_counted_fusable(int64_t tokens, int topk);
size_t group_counted_bytes(int64_t tokens);
hipError_t launch_group_counted(const float* routes, int64_t tokens, const int* counts16, float* groups,
                                float* order, int32_t* schedule, int schedule_bm, hipStream_t stream);
// With `schedule` non-NULL the scan also writes the grouped expert GEMM's tile
// schedule (as launch_expert_schedule, tiles of schedule_bm slots).
hipError_t launch_group_routes(const float* routes, int64_t tokens, int topk, float* groups,
                               float* order, void* workspace, hipStream_t stream,
                               int32_t* schedule = nullptr, int schedule_bm = 0);
hipError_t launch_expert_tasks(const float* groups, int64_t tokens, float* tasks,
                               hipStream_t stream);

// Tile schedule of the grouped expert GEMM: int32 [kSchedEntries + 2 *
// max_tiles], tiles of expert_tile_rows(routes) slots for `routes` routed rows
// (tokens * topk): 32-slot tiles for few routed rows, 128-slot tiles
// otherwise. The expert GEMM launches pick their kernel by the same rule, so a
// schedule must be built for the routes count the GEMMs are launched with.
// Layout: [0] the tile count; [kSchedClaims, +16) the work counters of the
// persistent expert kernels (eight per launch, one per XCD: the fused gate/up
// kernel uses the first eight, the other the second eight), zeroed by every
// writer of [0]; tile t's expert and first slot at [kSchedEntries + 2t] and
// [kSchedEntries + 2t + 1].
constexpr int kSchedClaims = 1, kSchedEntries = 17;
int expert_tile_rows(int64_t routes);
int64_t expert_max_tiles(int64_t routes);
size_t expert_schedule_bytes(int64_t routes);
hipError_t launch_expert_schedule(const float* groups, int64_t tokens, int topk, int32_t* schedule,
                                  hipStream_t stream);
// `list_stride` is the row pitch of `groups` in floats: tokens + 1 for the
// reference's table (0 selects it), more for a table that lists every route
// slot (ungrouped, duplicates included).
// The MoE layer's down projection for few routed rows straight from the
// bf16 h rows [tokens * topk][k] (quantized per pass inside the kernel, the
// codes and scales equal to launch_prepare's): launch_prepare of h then
// launch_expert_i4 (input_routed 1) in one launch, with the same output.
bool expert_down_h_fusable(int64_t routes, int k, int n);
// The MoE layer's down projection and combine for a few tokens at top-8
// (down_combine_fusable) in one launch, from the bf16 h rows [tokens * 8][k], the routes and
// the combine order the grouping wrote: launch_prepare of h, launch_expert_i4
// (input_routed 1) and launch_combine in one, with the same output.
bool down_combine_fusable(int64_t tokens, int topk, int k, int n);
// The MoE layer's router, Q1(x) and fused gate/up + SwiGLU for as many tokens
// (top-8 of 128 experts) in one launch: the routes and the combine order as
// launch_route and the grouping write them, and h [tokens * 8][n] as
// launch_expert_gate_up writes it. route_gate_up_fusable (k = hidden, n =
// inter) holds when the whole layer runs as this launch then
// launch_down_combine, which accepts these token counts too.
bool route_gate_up_fusable(int64_t tokens, int topk, int experts, int k, int n);
hipError_t launch_route_gate_up(const void* logits, int dtype, int64_t tokens, const uint16_t* x,
                                const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                                const float* up_s, int k, int n, float* routes, float* order, uint16_t* h,
                                hipStream_t stream);
hipError_t launch_down_combine(const uint16_t* h, const uint32_t* w, const float* ws, const float* routes,
                               const float* order, int64_t tokens, int topk, int k, int n, uint16_t* out,
                               hipStream_t stream);
hipError_t launch_expert_down_h(const uint16_t* h, const uint32_t* w, const float* ws, const float* groups,
                                const int32_t* schedule, int64_t tokens, int topk, int k, int n, uint16_t* out,
                                hipStream_t stream);
hipError_t launch_expert_i4(const uint32_t* a, int a_words, const float* a_scales,
                            const uint32_t* w_tiled, const float* w_scales, const float* groups,
                            const int32_t* schedule, int64_t tokens, int topk, int k, int n,
                            int input_routed, uint16_t* out, hipStream_t stream, int64_t list_stride = 0);

// Fused gate/up expert GEMMs with SwiGLU: h[route][c] = S1(E1(gate), E1(up)),
// routed rows gathered from `a` by route / topk; n % 128 == 0.
hipError_t launch_expert_gate_up(const uint32_t* a, int a_words, const float* as, const uint32_t* gate_w,
                                 const float* gate_s, const uint32_t* up_w, const float* up_s, const float* groups,
                                 const int32_t* schedule, int64_t tokens, int topk, int k, int n, uint16_t* h,
                                 hipStream_t stream, int64_t list_stride = 0);

// Every route slot of `routes` ([tokens][2 * topk]) as a one-slot token:
// slots[j] = (routes[j / topk][j % topk], 0) for j < tokens * topk. Grouping
// slots with topk 1 lists every slot naming an expert, duplicates included,
// under its ordinal j = t * topk + r.
hipError_t launch_route_slots(const float* routes, int64_t tokens, int topk, float* slots, hipStream_t stream);

hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h,
                         hipStream_t stream);
hipError_t launch_combine(const uint16_t* values, const float* routes, const float* order,
                          int64_t tokens, int width, int topk, uint16_t* out, hipStream_t stream);

}  // namespace clef
