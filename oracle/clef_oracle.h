/*
 * CPU oracle for the clef-hrx INT4 quantized-matmul and Omni INT4 MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the CPU
 * baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never links or calls it.
 *
 * Every function restates the reference arithmetic in plain C (IEEE f32,
 * round-to-nearest-even, no FMA contraction) and cites the reference file:line
 * it follows. Layouts are the reference's:
 *   packed activation: u32 [rows][stride/(32/bits)] codes, then rows f32 scales
 *   tiled weight codes: 128-row x 32-word blocks (kernels/retile_codes.loom:2-5)
 *   routes: f32 [T][2*topk] (ids then probabilities)
 *   groups: f32 [128][T+1] (count, then route ordinals), order f32 [T][topk]
 *
 * Return value 0 = success, negative = precondition violation (message via
 * orc_last_error()).
 */
#ifndef CLEF_ORACLE_H
#define CLEF_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* orc_last_error(void);

/* scalar helpers */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
float orc_expf(float x);
void orc_rotate256(float* group);

/* Q1: Hadamard-rotated per-row quantizer (bits 4 or 8). */
int orc_prepare(const uint16_t* x, int64_t rows, int32_t width, int32_t stride,
                int32_t bits, uint32_t* out);
/* Q1 after S1 (fused SwiGLU producer). */
int orc_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows,
                       int32_t width, int32_t stride, int32_t bits, uint32_t* out);
/* Q1 after the attention gate: x [rows][width], q_gate [rows][2*width]. */
int orc_prepare_attention_gate(const uint16_t* x, const uint16_t* q_gate, int64_t rows,
                               int32_t width, int32_t stride, int32_t bits, uint32_t* out);
/* Q1 after the named RMSNorm (width 5120); normalized may be NULL. */
int orc_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width,
                     int32_t stride, int32_t bits, uint32_t* out, uint16_t* normalized);
/* Named RMSNorm alone (weight offset 1, eps 1e-6, width 5120). */
int orc_rms_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width,
                 uint16_t* out);
/* Q2: row-major packed codes -> 128x32-word tiles. */
int orc_retile(const uint32_t* codes, int64_t rows, int32_t in_words,
               int32_t cols, int32_t bits, uint32_t* tiled);
/* G1: i32 accumulators only (row-major [m][n]). */
int orc_gemm_acc(const uint32_t* a, int32_t k_stride, const uint32_t* w_tiled,
                 int64_t m, int32_t n, int32_t k, int32_t bits, int32_t* acc);
/* G1: full projection, bf16 out, optional residual (may be NULL). */
int orc_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales,
             const uint32_t* w_tiled, const float* w_scales, int64_t m,
             int32_t n, int32_t k, int32_t bits, const uint16_t* residual,
             uint16_t* out);
/* R1: top-k router. dtype 0 = bf16 logits, 1 = f32 logits. */
int orc_route(const void* logits, int32_t dtype, int64_t tokens, int32_t experts,
              int32_t topk, float* routes);
/* R2: stable per-expert route lists (+ optional ascending-expert rank order). */
int orc_group_routes(const float* routes, int64_t tokens, int32_t topk,
                     float* groups, float* order);
/* R3: compact (expert, 16-row tile) task list. */
int orc_expert_tasks(const float* groups, int64_t tokens, float* tasks);
/* E1: grouped INT4 expert projection, out bf16 [tokens*topk][n]. */
int orc_expert_i4(const uint32_t* a, int32_t stride, const float* a_scales,
                  const uint32_t* w_tiled, const float* w_scales,
                  const float* groups, int64_t tokens, int32_t topk, int32_t k,
                  int32_t n, int32_t input_routed, uint16_t* out);
/* S1: SwiGLU with the reference's BF16 materialization. */
void orc_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h);
/* C1: weighted combine in ascending expert order; order may be NULL. */
int orc_expert_i4_ungrouped(const uint32_t* a, int32_t stride, const float* a_scales,
                            const uint32_t* w_tiled, const float* w_scales, const float* routes,
                            int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                            uint16_t* out);
int orc_combine(const uint16_t* values, const float* routes, const float* order,
                int64_t tokens, int32_t width, int32_t topk, uint16_t* out);
/* MoE block: route -> group -> Q1 -> E1 gate/up -> S1 -> Q1 -> E1 down -> C1. */
int orc_moe_layer(const uint16_t* x, const void* logits, int32_t logits_dtype,
                  int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                  int32_t topk, const uint32_t* gate_w, const float* gate_s,
                  const uint32_t* up_w, const float* up_s,
                  const uint32_t* down_w, const float* down_s,
                  float* routes_out, uint16_t* out);
/* checkpoint 256x64 tile layout (src/checkpoint.rs:63-106) */
int orc_tile_rows(const uint16_t* src, int64_t rows, int32_t cols, uint16_t* dst);
int orc_untile_rows(const uint16_t* src, int64_t rows, int32_t cols, uint16_t* dst);

/* number of OpenMP threads the oracle uses (for the CPU baseline report) */
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
