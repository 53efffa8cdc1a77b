/*
 * clef_i4.h - C ABI of the MI355X (gfx950) INT4 quantized-matmul and Omni INT4
 * MoE hot path.
 *
 * Drop-in boundary for the reference's crate-internal operator API. Each
 * entry point names the reference function it replaces (paths relative to the
 * reference repository). Memory layouts are the reference's, byte for byte:
 *
 *   bf16 tensors          uint16_t bit patterns, row-major
 *   packed activation     uint32_t [rows][stride/(32/bits)] codes (8 int4 or
 *                         4 int8 per word, low bits first), then rows f32
 *                         scales (src/quantized.rs:656-664)
 *   tiled weight codes    128-row x 32-word blocks:
 *                         word (n, q) -> ((n/128)*(K/256) + q/32)*4096
 *                                        + (n%128)*32 + q%32
 *                         (kernels/retile_codes.loom:2-5)
 *   routes                float [T][2*topk]: expert ids, then probabilities
 *   groups                float [128][T+1]: count, then route ordinals t*topk+r
 *   order                 float [T][topk]: rank of the j-th smallest expert id
 *   tasks                 float [1 + 2*(ceil(T*topk/16) + 127)]
 *
 * Conventions:
 *   - Every pointer argument is a device pointer owned by the caller, 16-byte
 *     aligned. Outputs are written, never allocated. No entry point allocates
 *     device memory; scratch comes from the caller's workspace (size query
 *     functions below).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default
 *     stream) and is asynchronous. Calls on distinct streams are independent.
 *   - Return 0 on success; CLEF_EINVAL (-1) when a precondition fails, with
 *     the reference's message (or a message of this library where the
 *     reference has no check) from clef_last_error(); a positive value is the
 *     hipError_t of a failed launch.
 *   - clef_last_error() is per calling thread.
 */
#ifndef CLEF_I4_H
#define CLEF_I4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* clef_stream_t;

#define CLEF_OK 0
#define CLEF_EINVAL (-1)

/* Message of the last failed call on this thread ("" if none). */
const char* clef_last_error(void);

/* ABI version of this header (major * 100 + minor). */
int clef_abi_version(void);

/* Identity of the sources the library was built from: the first 16 hex
 * digits of the SHA-256 of the files of clef-hrx_amd/csrc (sorted by name),
 * this header and the library's Makefile. Has no counterpart in the reference (whose kernels are
 * compiled at run time); lets a caller detect a library that is stale against
 * its source tree. */
const char* clef_build_id(void);

/* ------------------------------------------------------------------ Q1/Q2 */

/* Activation/weight stride rule: width + (width % 1024 == 0 ? 512/bits : 0).
 * Replaces the stride computation at src/quantized.rs:161-166. */
int32_t clef_i4_activation_stride(int32_t width, int32_t bits);

/* Words of one packed buffer: rows * (stride/(32/bits) + 1). */
int64_t clef_i4_prepared_words(int64_t rows, int32_t stride, int32_t bits);

/* Hadamard-rotated per-row quantizer (bits 4 or 8) into the packed layout.
 * Padding words [width/(32/bits), stride/(32/bits)) of each row are not
 * written. Replaces quantized::prepare / prepare_inputs
 * (src/quantized.rs:574-686) and the h3_prepare_plain_tiled_i4/_i8 kernels
 * (kernels/prepare_integer_single.loom, prepare_integer.loom,
 * prepare_integer_register.loom:317-352).
 * Preconditions (src/quantized.rs:640-649): bits in {4,8}, 256 <= width <=
 * 32768, width % 256 == 0, 1 <= rows <= 1048576, width <= stride <= 65536,
 * stride % (512/bits) == 0 -> else "unsupported rotated integer operand". */
int clef_i4_prepare(const uint16_t* x, int64_t rows, int32_t width, int32_t stride, int32_t bits,
                    uint32_t* out, clef_stream_t stream);

/* SwiGLU fused into the quantizer: quantizes bf16(swiglu(gate, up)) with the
 * rounding of a materialized SwiGLU. Replaces prepare_with_inputs([gate, up])
 * / h3_prepare_swiglu_i4 (src/quantized.rs:406-439, 605-613;
 * kernels/prepare_integer_register.loom:155-172, 353-368). Same
 * preconditions as clef_i4_prepare. */
int clef_i4_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows, int32_t width,
                           int32_t stride, int32_t bits, uint32_t* out, clef_stream_t stream);

/* Attention output gated by the sigmoid of its query-gate half, fused into
 * the quantizer: quantizes bf16(x * bf16(1 / (1 + exp(-g)))) where g for
 * column c is column (c/256)*512 + 256 + c%256 of q_gate (bf16
 * [rows][2*width]: query and gate share each 512-column head block).
 * Replaces prepare_attention_gate_with_source / h3_prepare_attention_gate_i4
 * (src/quantized.rs:440-468, 615-635; kernels/prepare_integer_register.loom:
 * 137-155). Same preconditions as clef_i4_prepare. */
int clef_i4_prepare_attention_gate(const uint16_t* attention, const uint16_t* q_gate, int64_t rows,
                                   int32_t width, int32_t stride, int32_t bits, uint32_t* out,
                                   clef_stream_t stream);

/* Size in u32 words of clef_i4_prepare_norm's output: rows * (stride/(32/bits)
 * + 1), plus, when store is nonzero, the padding to a 128-byte boundary and
 * the bf16 normalized rows [rows][width] (src/quantized.rs:731-740). -1 for
 * bits other than 4 and 8. */
int64_t clef_i4_prepare_norm_words(int64_t rows, int32_t width, int32_t stride, int32_t bits,
                                   int32_t store);

/* Named RMSNorm (weight offset 1, eps 1e-6) fused into the quantizer:
 * r = bf16(fma(x * inv, weight + 1, 0)) with inv = 1/sqrt(sum(x^2)/width +
 * 1e-6), then Q1 of r. With store nonzero the bf16 rows r are also written
 * after the packed codes and scales, at the first 128-byte boundary. Replaces
 * prepare_norm_with_source / prepare_norm_store_with_source and
 * h3_prepare_norm[_store]_i4/_i8 (src/quantized.rs:687-779;
 * kernels/prepare_integer_register.loom:63-80, 112-134). The reference sums
 * the squares in an order of its compiler's choosing and uses an approximate
 * rsqrt; here the order is fixed (documented in csrc/prepare.hip) and sqrt
 * and division are correctly rounded. Preconditions (src/quantized.rs:
 * 721-731): width == 5120, bits in {4,8}, 1 <= rows <= 1048576, width <=
 * stride <= 65536, stride % (512/bits) == 0 -> else "unsupported normalized
 * packing shape". */
int clef_i4_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width,
                         int32_t stride, int32_t bits, int32_t store, uint32_t* out,
                         clef_stream_t stream);

/* Row-major packed codes [rows][in_words] -> tiled blocks, dropping padding.
 * Replaces quantized::retile_codes (src/quantized.rs:542-572) and
 * kernels/retile_codes.loom. Preconditions: rows % 128 == 0, words =
 * cols/(32/bits) with words % 32 == 0, in_words >= words -> else
 * "unsupported packed weight shape for tiling". */
int clef_i4_retile(const uint32_t* codes, int64_t rows, int32_t in_words, int32_t cols, int32_t bits,
                   uint32_t* tiled, clef_stream_t stream);

/* Bytes of scratch clef_i4_pack_weight needs (the row-major packed staging). */
size_t clef_i4_pack_weight_workspace_bytes(int64_t rows, int32_t cols, int32_t bits);

/* bf16 weight [rows][cols] (logical row order) -> tiled codes
 * [rows*cols/(32/bits)] words and f32 scales [rows]: quantize with the
 * activation stride, retile, keep one scale per row. Replaces the packing
 * half of Engine::load_quantized_weight (src/quantized.rs:147-234) after its
 * CPU untile. Preconditions: rows % 256 == 0 && cols % 256 == 0 ->
 * "unsupported quantized weight shape"; then those of prepare and retile. */
int clef_i4_pack_weight(const uint16_t* w, int64_t rows, int32_t cols, int32_t bits, uint32_t* tiled,
                        float* scales, void* workspace, size_t workspace_bytes,
                        clef_stream_t stream);

/* 256x64-tiled checkpoint layout [rows/256][cols/64][256][64] <-> logical
 * rows. Replace checkpoint::untile_rows / tile_rows (src/checkpoint.rs:63-106,
 * 24-32). Preconditions: rows % 256 == 0, cols % 64 == 0 -> "tiled layout
 * requires 256-row and 64-column multiples". */
int clef_untile_rows(const uint16_t* tiled, int64_t rows, int32_t cols, uint16_t* out,
                     clef_stream_t stream);
int clef_tile_rows(const uint16_t* dense, int64_t rows, int32_t cols, uint16_t* out,
                   clef_stream_t stream);

/* ------------------------------------------------------------------ G1 */

/* INT4 x INT4 -> i32 dense GEMM with the reference epilogue
 * out[m][n] = bf16(sat(RN(RN(f32(acc) * w_scales[n]) * a_scales[m]) + 0)),
 * plus residual (bf16 [m][n], nullable): out = bf16(res + out).
 * `a` points at the packed activation codes (row pitch k_stride/8 words) and
 * `a_scales` at its scales. Replaces Engine::project_prepared
 * (src/quantized.rs:470-537) and h3_gemm_i4_256[_residual]
 * (kernels/gemm_integer.loom, gemm_integer_m128.loom, gemm_integer_wide_k.loom).
 * Preconditions: m >= 1, n % 128 == 0, k % 256 == 0, k >= 256, k_stride >= k,
 * k_stride % 32 == 0 -> "unsupported integer projection shape". */
int clef_i4_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales, const uint32_t* w_tiled,
                 const float* w_scales, int64_t m, int32_t n, int32_t k, const uint16_t* residual,
                 uint16_t* out, clef_stream_t stream);

/* INT8 x INT8 -> i32 dense GEMM with the same epilogue, for INT8-packed
 * activations (clef_i4_prepare with bits 8: 4 codes per word, row pitch
 * k_stride/4 words) and INT8 weights (clef_i4_pack_weight with bits 8).
 * Replaces the bits = 8 dispatch of Engine::project_prepared
 * (src/quantized.rs:486-497) and h3_gemm_i8_256 (kernels/gemm_integer.loom:
 * 444-485). Preconditions: m >= 1, n % 128 == 0, k % 256 == 0, k >= 256,
 * k_stride >= k, k_stride % 64 == 0 -> "unsupported integer projection shape". */
int clef_i8_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales, const uint32_t* w_tiled,
                 const float* w_scales, int64_t m, int32_t n, int32_t k, const uint16_t* residual,
                 uint16_t* out, clef_stream_t stream);

/* Same, with an explicit tile configuration (0..clef_i4_gemm_configs()-1;
 * -1 = automatic): 0 = 128x128 tiles, 1 = 256x256 tiles (one workgroup per
 * tile), 2 = 256x256 tiles on a persistent grid, 3 = the K-split small-M
 * kernel, 4 = the VALU dot-product kernel for m <= 8 (3 for larger m),
 * 5 = small tiles with the K split among a workgroup's waves. Configurations 1 and 2 fall back to 0 when n % 256 != 0, and 2 to 1
 * when k < 512. For tuning and tests. */
int clef_i4_gemm_config(const uint32_t* a, int32_t k_stride, const float* a_scales,
                        const uint32_t* w_tiled, const float* w_scales, int64_t m, int32_t n,
                        int32_t k, const uint16_t* residual, uint16_t* out, int32_t config,
                        clef_stream_t stream);
int clef_i4_gemm_configs(void);

/* bf6 form of G1's operands (no counterpart in the reference: a gfx950
 * re-encoding of the same INT4 codes). Every code -8..7 is exact in bf6
 * (e3m2), so v_mfma_scale_f32_32x32x64_f8f6f4 on these operands gives the
 * exact integer dot products, and clef_i4_gemm_f6 returns exactly what
 * clef_i4_gemm returns for the operands they were made from, with no
 * unpacking in the GEMM and twice the int8 MFMA's k per instruction.
 * - clef_i4_f6_activation: packed activation codes (as clef_i4_gemm's `a`,
 *   row pitch k_stride/8 words) -> the bf6 activation layout: blocks of 128
 *   rows x 128 k (12 KiB of 96-byte rows; value k of a row at bits 6k of
 *   its 96 bytes) at ((row/128)*(k/128) + k/128)*12288, row r % 128 of a
 *   block at (r % 128)*96; rows past `rows` in the last block are padding
 *   (not written): ceil(rows/128)*128*k*3/4 bytes. Preconditions: rows >= 1,
 *   k % 128 == 0, k_stride >= k, k_stride % 32 == 0 -> "unsupported integer
 *   projection shape"; 16-byte aligned pointers.
 * - clef_i4_f6_weight: tiled weight codes (clef_i4_retile, bits 4, [n][k])
 *   -> bf6 tiled weight: 128-row x 128-k blocks of 96-byte rows (12 KiB) at
 *   ((row/128)*(k/128) + k/128)*12288, the 16-byte chunk c of block row r
 *   stored at chunk c ^ ((r >> 3) & 1); n*k*3/4 bytes. Preconditions:
 *   n % 128 == 0, k % 256 == 0 -> "unsupported integer projection shape".
 * - clef_i4_prepare_f6 / clef_i4_prepare_swiglu_f6: Q1 (as clef_i4_prepare /
 *   clef_i4_prepare_swiglu with bits 4) writing the codes in the bf6
 *   activation layout directly: ceil(rows/128)*128*width*3/4 bytes of codes,
 *   then rows f32 scales (at that byte); clef_i4_f6_prepared_bytes gives the
 *   size. Same codes and scales as clef_i4_prepare then
 *   clef_i4_f6_activation, in one pass.
 *   Preconditions as clef_i4_prepare (width % 256 == 0, 256 <= width <=
 *   32768, 1 <= rows <= 2^20 -> "unsupported rotated integer operand").
 * - clef_i4_gemm_f6: G1 on them, with clef_i4_gemm's epilogue and residual.
 *   Preconditions: m >= 1, n % 256 == 0, k % 256 == 0, 256 <= k <= 32768
 *   (the quantizer's widest row; the f32 sums of the bf6 products are exact
 *   integers there) -> "unsupported integer projection shape"; 16-byte
 *   aligned pointers. */
int clef_i4_f6_activation(const uint32_t* a, int32_t k_stride, int64_t rows, int32_t k, uint8_t* out,
                          clef_stream_t stream);
int clef_i4_f6_weight(const uint32_t* w_tiled, int64_t n, int32_t k, uint8_t* out, clef_stream_t stream);
int64_t clef_i4_f6_prepared_bytes(int64_t rows, int32_t width);
int clef_i4_prepare_f6(const uint16_t* x, int64_t rows, int32_t width, uint8_t* out, clef_stream_t stream);
int clef_i4_prepare_swiglu_f6(const uint16_t* gate, const uint16_t* up, int64_t rows, int32_t width,
                              uint8_t* out, clef_stream_t stream);
int clef_i4_gemm_f6(const uint8_t* a_f6, const float* a_scales, const uint8_t* w_f6, const float* w_scales,
                    int64_t m, int32_t n, int32_t k, const uint16_t* residual, uint16_t* out,
                    clef_stream_t stream);

/* The dense MLP's gate and up projections with SwiGLU in one GEMM on the bf6
 * forms: h[m][n] = S1(G1(a, gate), G1(a, up)) = bf16(silu_bf16(g) * u), g
 * and u each G1's bf16 output. Replaces the two project_prepared calls and
 * the SwiGLU step of the reference's dense MLP (src/quantized.rs:399-401
 * then project_swiglu :406-439, whose fused quantizer rounds the same h to
 * bf16 before quantizing; kernels/swiglu.loom:43-51): h equals
 * clef_swiglu(clef_i4_gemm_f6(a, gate), clef_i4_gemm_f6(a, up)) bit for
 * bit, and clef_i4_prepare_f6(h) equals clef_i4_prepare_swiglu_f6 of those
 * two outputs. Reads the activation tile once for both projections and
 * writes h instead of gate and up. Preconditions: those of clef_i4_gemm_f6
 * with n % 128 == 0 (gate and up weights both [n][k], bf6 tiled) ->
 * "unsupported integer projection shape"; 16-byte aligned pointers. */
int clef_i4_gemm_f6_gate_up(const uint8_t* a_f6, const float* a_scales, const uint8_t* gate_f6,
                            const float* gate_scales, const uint8_t* up_f6, const float* up_scales, int64_t m,
                            int32_t n, int32_t k, uint16_t* h, clef_stream_t stream);

/* Bytes of scratch clef_i4_project needs (the packed activation). */
size_t clef_i4_project_workspace_bytes(int64_t m, int32_t k);

/* Quantize x [m][k] with the weight's stride (clef_i4_activation_stride(k,
 * 4)) and run G1. Replaces Engine::project_quantized /
 * project_quantized_with_residual (src/quantized.rs:235-303). */
int clef_i4_project(const uint16_t* x, int64_t m, int32_t k, const uint32_t* w_tiled,
                    const float* w_scales, int32_t n, const uint16_t* residual, uint16_t* out,
                    void* workspace, size_t workspace_bytes, clef_stream_t stream);

/* The same projection on the bf6 form of the codes (no counterpart in the
 * reference): x quantized straight into bf6 (clef_i4_prepare_f6) into the
 * workspace, then clef_i4_gemm_f6 with the bf6 weight (clef_i4_f6_weight of
 * the 4-bit tiled weight) and its f32 scales. Same bf16 output as
 * clef_i4_project bit for bit. Preconditions: those of clef_i4_prepare_f6 and
 * clef_i4_gemm_f6; workspace_bytes >= clef_i4_project_f6_workspace_bytes(m, k)
 * -> "workspace too small". */
size_t clef_i4_project_f6_workspace_bytes(int64_t m, int32_t k);
int clef_i4_project_f6(const uint16_t* x, int64_t m, int32_t k, const uint8_t* w_f6, const float* w_scales,
                       int32_t n, const uint16_t* residual, uint16_t* out, void* workspace,
                       size_t workspace_bytes, clef_stream_t stream);

/* ------------------------------------------------------------------ MoE */

/* Top-k router: ties -> lowest expert id, softmax over the selected logits,
 * probabilities rounded to bf16. logits_dtype 0 = bf16, 1 = f32.
 * Replaces Engine::omni_route (src/omni.rs:170-190), kernels/omni_route.loom.
 * Preconditions: 0 < topk <= experts <= 128 -> "invalid expert router shape";
 * 1 <= tokens <= 2^24; logits 16-byte aligned (rows are read as 16-byte
 * pieces where their length allows) -> the alignment message. */
int clef_moe_route(const void* logits, int32_t logits_dtype, int64_t tokens, int32_t experts,
                   int32_t topk, float* routes, clef_stream_t stream);

/* Bytes of scratch clef_moe_group_routes needs. */
size_t clef_moe_group_workspace_bytes(int64_t tokens);

/* Stable per-expert route lists (128 experts) and, when `order` is non-NULL,
 * the ascending-expert rank order. Replaces Engine::omni_group_routes /
 * omni_group_routes_ordered (src/omni.rs:192-245) and
 * kernels/omni_group_routes.loom, omni_group_routes_ordered.loom. The
 * reference caps tokens at 2048 per chunk (src/omni.rs:11); this library
 * accepts up to 1048576 tokens in one call (every stage is row-local), while
 * the f32-encoded route ordinals t*topk+r stay exact (below 2^24).
 * Preconditions: 1 <= tokens <= 1048576, 1 <= topk <= 128, tokens * topk <=
 * 16777216 -> "unsupported Omni route grouping shape". */
int clef_moe_group_routes(const float* routes, int64_t tokens, int32_t topk, float* groups,
                          float* order, void* workspace, size_t workspace_bytes,
                          clef_stream_t stream);

/* Compact task list: tasks[0] = count, then (expert, 16*tile) pairs for
 * experts ascending. Replaces the omni_expert_tasks dispatch of
 * Engine::omni_compact_routes (src/omni.rs:126-169) and
 * kernels/omni_expert_tasks.loom. tasks holds 1 + 2*(ceil(T*8/16)+127)
 * floats. */
int clef_moe_expert_tasks(const float* groups, int64_t tokens, float* tasks, clef_stream_t stream);

/* Bytes of scratch clef_moe_expert_i4 needs (its tile schedule). */
size_t clef_moe_expert_workspace_bytes(int64_t tokens, int32_t topk);

/* Grouped INT4 expert GEMM over all 128 experts:
 * out[route][c] = bf16(RN(f32(acc) * RN(a_scales[xr] * w_scales[e*n + c]))),
 * xr = input_routed ? route : route/topk. `a` is the packed activation (row
 * pitch stride/8 words, rows = tokens or tokens*topk), w_tiled the 128
 * experts' codes concatenated as [128*n][k]. Output bf16 [tokens*topk][n].
 * Replaces Engine::omni_expert_impl / omni_expert_inputs
 * (src/omni.rs:289-534) and kernels/omni_expert_i4.loom,
 * omni_expert_i4_k128_down.loom, omni_expert_i4_compact.loom.
 * Preconditions: 1 <= tokens <= 1048576, 1 <= topk <= 128 -> "invalid
 * grouped expert routes"; tokens * topk <= 16777216 -> "unsupported Omni
 * route grouping shape"; k % 256 == 0 && n % 256 == 0 && k, n >= 256 &&
 * stride >= k && stride % 32 == 0 -> "unsupported Omni expert tile shape";
 * the packed codes of `a` (rows * stride / 2 bytes) below 2 GiB -> "expert
 * activation operand of 2 GiB or more ...". `groups` must hold lists as
 * clef_moe_group_routes writes them (counts <= tokens, route ordinals below
 * tokens * topk): the ordinals address output rows and are not checked. */
int clef_moe_expert_i4(const uint32_t* a, int32_t stride, const float* a_scales,
                       const uint32_t* w_tiled, const float* w_scales, const float* groups,
                       int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                       uint16_t* out, void* workspace, size_t workspace_bytes,
                       clef_stream_t stream);

/* Bytes of scratch clef_moe_expert_i4_ungrouped needs (0 for shapes it
 * rejects). */
size_t clef_moe_expert_ungrouped_workspace_bytes(int64_t tokens, int32_t topk);

/* The expert GEMM without a groups table: for every route slot (t, r) whose
 * expert id e = (int)routes[t][r] names one of the 128 experts, row
 * t * topk + r of `out` gets the E1 values of expert e, with every slot
 * computed on its own (duplicate experts of one token included), as the
 * reference's ungrouped kernel computes them. Slots naming no expert (the
 * reference assumes there are none) leave their rows unwritten. Replaces
 * Engine::omni_expert (src/omni.rs:280-288: omni_expert_impl with groups =
 * None) and kernels/omni_expert.loom:86-150, whose f32 FMA dot is exact on
 * integer codes, so results equal clef_moe_expert_i4's bit for bit. The
 * slots are grouped into the workspace (topk-1 grouping of the slots), then
 * the grouped kernels run. Preconditions: those of clef_moe_expert_i4. */
int clef_moe_expert_i4_ungrouped(const uint32_t* a, int32_t stride, const float* a_scales,
                                 const uint32_t* w_tiled, const float* w_scales, const float* routes,
                                 int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                                 uint16_t* out, void* workspace, size_t workspace_bytes, clef_stream_t stream);

/* Fused gate/up expert GEMMs with SwiGLU: for every routed row r of every
 * expert e, h[r][c] = bf16(bf16(g/(1+exp(-g))) * u) where g and u are the E1
 * outputs (as clef_moe_expert_i4, input_routed = 0) of gate_w and up_w for
 * column c. One pass over the gathered activation rows feeds both weight
 * sets; h (bf16 [tokens*topk][n]) is bit-equal to clef_moe_expert_i4 twice
 * followed by clef_swiglu. Replaces Engine::omni_gate_up (src/omni.rs:300-372)
 * and benches/kernels/omni_gate_up_i4.loom. Workspace: as clef_moe_expert_i4.
 * Preconditions: 1 <= tokens <= 1048576, 1 <= topk <= 128 -> "fused gate/up
 * requires regular grouped routes"; tokens * topk <= 16777216 ->
 * "unsupported Omni route grouping shape"; k % 256 == 0, n % 128 == 0 (the
 * tiled weight layout's 128-row panels; the reference accepts n % 64 == 0),
 * stride >= k, stride % 32 == 0 -> "incompatible fused expert weights";
 * tokens * stride / 2 < 2 GiB -> "expert activation operand of 2 GiB or
 * more ...". */
int clef_moe_expert_gate_up_i4(const uint32_t* a, int32_t stride, const float* a_scales,
                               const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                               const float* up_s, const float* groups, int64_t tokens, int32_t topk,
                               int32_t k, int32_t n, uint16_t* h, void* workspace,
                               size_t workspace_bytes, clef_stream_t stream);

/* h = bf16(bf16(g/(1+exp(-g))) * u) elementwise over n values. Replaces
 * Engine::swiglu (src/ops.rs:9-29) and kernels/swiglu.loom. Precondition:
 * n >= 0 -> "SwiGLU shape/dtype mismatch". */
int clef_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h,
                clef_stream_t stream);

/* Weighted combine in ascending expert order with a bf16 rounding per step.
 * `order` NULL selects the unordered variant (ascending ids found from the
 * routes). Replaces Engine::omni_combine / omni_combine_ordered
 * (src/omni.rs:246-278, 535-556) and kernels/omni_combine.loom,
 * omni_combine_ordered.loom. Preconditions: width % 8 == 0, 1 <= topk <=
 * 128, tokens >= 1 -> "unsupported ordered Omni accumulation". An order
 * entry outside [0, topk) (the grouping leaves entries unwritten for a
 * token that names an expert twice or none) reads slot 0; such a token's
 * output is unspecified. */
int clef_moe_combine(const uint16_t* values, const float* routes, const float* order,
                     int64_t tokens, int32_t width, int32_t topk, uint16_t* out,
                     clef_stream_t stream);

/* Bytes of scratch clef_moe_layer needs. */
size_t clef_moe_layer_workspace_bytes(int64_t tokens, int32_t hidden, int32_t inter,
                                      int32_t topk);

/* Omni INT4 MoE block: route -> ordered grouping -> quantize x (shared by
 * gate and up) -> gate and up expert GEMMs -> SwiGLU -> quantize h per routed
 * row -> down expert GEMM (routed input) -> ordered combine. Output bf16
 * [tokens][hidden]; routes_out (nullable) receives the routes. Replaces the
 * MoE half of omni::forward_layers_cached (src/omni.rs:760-857) without the
 * bf16 router-gate projection (logits are an input) and without the residual
 * add. Preconditions: experts == 128 -> "Omni MoE requires 128 experts";
 * hidden, inter % 256 == 0; then those of the stages (logits 16-byte
 * aligned, as clef_moe_route), including the 2 GiB
 * bound on the packed x (tokens rows) and packed h (tokens * topk rows): the
 * reference runs at most 2048 tokens per call (src/omni.rs:11), and callers
 * with more tokens than the bound allows split them into chunks. */
int clef_moe_layer(const uint16_t* x, const void* logits, int32_t logits_dtype, int64_t tokens,
                   int32_t hidden, int32_t inter, int32_t experts, int32_t topk,
                   const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                   const float* up_s, const uint32_t* down_w, const float* down_s,
                   float* routes_out, uint16_t* out, void* workspace, size_t workspace_bytes,
                   clef_stream_t stream);

/* Bytes of the static scratch of clef_moe_layer_static: 32 MiB per device. */
#define CLEF_MOE_STATIC_SCRATCH_BYTES ((size_t)32 << 20)

/* clef_moe_layer without a workspace argument: allocates nothing (no
 * hipMalloc, hipFree or allocating library call) and takes its intermediates
 * from a static device array of CLEF_MOE_STATIC_SCRATCH_BYTES, one per device,
 * which the library holds from the first call on a device until the process
 * ends. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same preconditions and results as
 * clef_moe_layer, plus clef_moe_layer_workspace_bytes(tokens, hidden, inter,
 * topk) <= CLEF_MOE_STATIC_SCRATCH_BYTES (about 650 tokens at hidden 2048,
 * inter 768, top-8) -> "MoE layer needs N bytes of scratch; ...". Nothing
 * in the scratch needs to start at zero (every intermediate is written before
 * it is read). Every call on one device shares that device's scratch, and it
 * keeps the last call's contents: calls that overlap on one device (on
 * different streams, or from different host threads) race and must be
 * ordered by the caller. The first call on a device looks up the scratch's
 * device address with that device current, so call it with the device of
 * `stream` current. */
int clef_moe_layer_static(const uint16_t* x, const void* logits, int32_t logits_dtype, int64_t tokens,
                          int32_t hidden, int32_t inter, int32_t experts, int32_t topk,
                          const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                          const float* up_s, const uint32_t* down_w, const float* down_s,
                          float* routes_out, uint16_t* out, clef_stream_t stream);

/* Router gate projection: logits[t][e] = bf16(sum_k x[t][k] * gate_w[e][k])
 * with f32 accumulation (bf16 MFMA), x bf16 [tokens][hidden], gate_w bf16
 * [experts][hidden] row-major, logits bf16 [tokens][experts] -- the input of
 * clef_moe_route. Replaces the Omni MoE block's e.project(norm, "mlp.gate")
 * (src/omni.rs:764) through Engine::linear (src/ops.rs:95-175,
 * kernels/gemm_bf16_reference.loom). The summation order differs from the
 * reference's WMMA order, so results agree within f32 rounding, not bit for
 * bit. Preconditions: tokens >= 1, hidden % 64 == 0, 32 <= experts <= 128,
 * experts % 32 == 0 -> "linear shape/dtype mismatch". */
int clef_moe_router_logits(const uint16_t* x, const uint16_t* gate_w, int64_t tokens, int32_t hidden,
                           int32_t experts, uint16_t* logits, clef_stream_t stream);

/* ------------------------------------------------------- packed cache */

/* Key of a packed-weight cache entry (src/packed_cache.rs:24-33): the weight
 * name and extent, the compiler and target identities, and the source bytes
 * (host memory, hashed with SHA-256). The packing definition's hash is
 * supplied by the library. */
typedef struct clef_pack_key {
  const char* name;
  int64_t rows;
  int64_t cols;
  int32_t bits;
  const char* compiler;
  const char* target;
  const void* source;
  size_t source_bytes;
} clef_pack_key;

/* Path of the entry of `key` under `directory`: hex SHA-256 of the compact
 * JSON key + ".pack" (src/packed_cache.rs:101-105). Host-only, no device
 * work. */
int clef_pack_cache_path(const char* directory, const clef_pack_key* key, char* path, size_t path_bytes);

/* Reads the "CLFPACK1" entry of `key` into host buffers of exactly
 * rows*cols*bits/8 code bytes and rows*4 scale bytes. *hit = 0 and CLEF_OK
 * when there is no entry (a miss). Replaces PackedWeightCache::read
 * (src/packed_cache.rs:106-145) with its checks and messages: "invalid
 * packed-cache extent", "truncated packed-cache prefix", "invalid
 * packed-cache magic", "oversized packed-cache header", "packed-cache length
 * mismatch", "packed-cache key mismatch", "packed-cache checksum mismatch:
 * <path>". */
int clef_pack_cache_read(const char* directory, const clef_pack_key* key, void* codes, size_t codes_bytes,
                         void* scales, size_t scales_bytes, int32_t* hit);

/* Writes the entry of `key` atomically (temporary file, then rename).
 * Replaces PackedWeightCache::write (src/packed_cache.rs:146-190);
 * "packed-cache data size mismatch" when the buffers do not match the key's
 * extent. */
int clef_pack_cache_write(const char* directory, const clef_pack_key* key, const void* codes, size_t codes_bytes,
                          const void* scales, size_t scales_bytes);

#ifdef __cplusplus
}
#endif

#endif /* CLEF_I4_H */
