// C ABI of the gfx950 INT4 path (include/clef_i4.h): argument checks with the
// reference's predicates and messages, then stream-ordered launches. The
// composite entry points (pack_weight, project, moe_layer) are the host side
// of the reference's operators: Engine::load_quantized_weight
// (src/quantized.rs:147-234), Engine::project_quantized (:235-303) and the
// MoE block of omni::forward_layers_cached (src/omni.rs:760-857).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "../../include/clef_i4.h"
#include "kernels.hpp"

namespace {

thread_local char g_error[1024] = "";

int fail(const char* msg) {
  std::snprintf(g_error, sizeof g_error, "%s", msg);
  return CLEF_EINVAL;
}

int hip_status(hipError_t e) {
  if (e == hipSuccess) return CLEF_OK;
  std::snprintf(g_error, sizeof g_error, "HIP error %d: %s", (int)e, hipGetErrorString(e));
  return (int)e;
}

bool aligned(const void* p, size_t a) { return p && (reinterpret_cast<uintptr_t>(p) % a) == 0; }

hipStream_t hs(clef_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

constexpr const char* kAlign = "device pointer is NULL or not 16-byte aligned";
constexpr const char* kWorkspace = "workspace too small";

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Quantizer preconditions, src/quantized.rs:640-649.
int check_prepare(int64_t rows, int32_t width, int32_t stride, int32_t bits) {
  if (!((bits == 4 || bits == 8) && width >= 256 && width <= 32768 && width % 256 == 0 && rows >= 1 &&
        rows <= 1048576 && stride >= width && stride <= 65536 && stride % (512 / bits) == 0))
    return fail("unsupported rotated integer operand");
  return CLEF_OK;
}

int check_gemm(int64_t m, int32_t n, int32_t k, int32_t k_stride) {
  if (!(m >= 1 && n >= 128 && n % 128 == 0 && k >= 256 && k % 256 == 0 && k_stride >= k &&
        k_stride % 32 == 0))
    return fail("unsupported integer projection shape");
  return CLEF_OK;
}

int64_t prepared_words(int64_t rows, int32_t stride, int32_t bits) {
  return rows * (stride / (32 / bits) + 1);
}

int32_t stride_for(int32_t width, int32_t bits) {
  return width + (width % 1024 == 0 ? 512 / bits : 0);
}

}  // namespace

namespace clef {
int set_last_error(const char* msg) { return fail(msg); }
}  // namespace clef

extern "C" {

const char* clef_last_error(void) { return g_error; }

int clef_abi_version(void) { return 100; }

int32_t clef_i4_activation_stride(int32_t width, int32_t bits) { return stride_for(width, bits); }

int64_t clef_i4_prepared_words(int64_t rows, int32_t stride, int32_t bits) {
  if (bits != 4 && bits != 8) return -1;
  return prepared_words(rows, stride, bits);
}

int clef_i4_prepare(const uint16_t* x, int64_t rows, int32_t width, int32_t stride, int32_t bits,
                    uint32_t* out, clef_stream_t stream) {
  if (int rc = check_prepare(rows, width, stride, bits)) return rc;
  if (!aligned(x, 16) || !aligned(out, 16)) return fail(kAlign);
  return hip_status(clef::launch_prepare(x, rows, width, stride, bits, out, hs(stream)));
}

int clef_i4_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows, int32_t width,
                           int32_t stride, int32_t bits, uint32_t* out, clef_stream_t stream) {
  if (int rc = check_prepare(rows, width, stride, bits)) return rc;
  if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, 16)) return fail(kAlign);
  return hip_status(clef::launch_prepare_swiglu(gate, up, rows, width, stride, bits, out, hs(stream)));
}

int clef_i4_prepare_attention_gate(const uint16_t* attention, const uint16_t* q_gate, int64_t rows,
                                   int32_t width, int32_t stride, int32_t bits, uint32_t* out,
                                   clef_stream_t stream) {
  if (int rc = check_prepare(rows, width, stride, bits)) return rc;
  if (!aligned(attention, 16) || !aligned(q_gate, 16) || !aligned(out, 16)) return fail(kAlign);
  return hip_status(
      clef::launch_prepare_attention_gate(attention, q_gate, rows, width, stride, bits, out, hs(stream)));
}

namespace {
// Byte offset of the stored normalized rows: the packed words rounded up to
// 128 bytes (src/quantized.rs:733-734).
int64_t norm_offset_bytes(int64_t rows, int32_t stride, int32_t bits) {
  return (prepared_words(rows, stride, bits) * 4 + 127) / 128 * 128;
}
}  // namespace

int64_t clef_i4_prepare_norm_words(int64_t rows, int32_t width, int32_t stride, int32_t bits,
                                   int32_t store) {
  if ((bits != 4 && bits != 8) || rows < 0 || width < 0) return -1;
  if (!store) return prepared_words(rows, stride, bits);
  return norm_offset_bytes(rows, stride, bits) / 4 + rows * width / 2;
}

int clef_i4_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width,
                         int32_t stride, int32_t bits, int32_t store, uint32_t* out,
                         clef_stream_t stream) {
  if (!(width == 5120 && (bits == 4 || bits == 8) && rows >= 1 && rows <= 1048576 && stride >= width &&
        stride <= 65536 && stride % (512 / bits) == 0))
    return fail("unsupported normalized packing shape");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 16)) return fail(kAlign);
  uint16_t* normalized =
      store ? reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(out) + norm_offset_bytes(rows, stride, bits))
            : nullptr;
  return hip_status(
      clef::launch_prepare_norm(x, weight, rows, width, stride, bits, out, normalized, hs(stream)));
}

int clef_i4_retile(const uint32_t* codes, int64_t rows, int32_t in_words, int32_t cols, int32_t bits,
                   uint32_t* tiled, clef_stream_t stream) {
  if (bits != 4 && bits != 8) return fail("unsupported packed weight shape for tiling");
  const int32_t words = cols / (32 / bits);
  // src/quantized.rs:550-558.
  if (!(rows > 0 && rows % 128 == 0 && cols > 0 && cols % (32 / bits) == 0 && words % 32 == 0 &&
        in_words >= words))
    return fail("unsupported packed weight shape for tiling");
  if (!aligned(codes, 16) || !aligned(tiled, 16)) return fail(kAlign);
  return hip_status(clef::launch_retile(codes, rows, in_words, words, tiled, hs(stream)));
}

size_t clef_i4_pack_weight_workspace_bytes(int64_t rows, int32_t cols, int32_t bits) {
  if ((bits != 4 && bits != 8) || rows < 0 || cols < 0) return 0;
  return align256((size_t)prepared_words(rows, stride_for(cols, bits), bits) * 4);
}

int clef_i4_pack_weight(const uint16_t* w, int64_t rows, int32_t cols, int32_t bits, uint32_t* tiled,
                        float* scales, void* workspace, size_t workspace_bytes,
                        clef_stream_t stream) {
  if (!(rows > 0 && cols > 0 && rows % 256 == 0 && cols % 256 == 0))
    return fail("unsupported quantized weight shape");
  const int32_t stride = stride_for(cols, bits);
  if (int rc = check_prepare(rows, cols, stride, bits)) return rc;
  if (!aligned(w, 16) || !aligned(tiled, 16) || !aligned(scales, 4) || !aligned(workspace, 16))
    return fail(kAlign);
  if (workspace_bytes < clef_i4_pack_weight_workspace_bytes(rows, cols, bits)) return fail(kWorkspace);
  uint32_t* staging = static_cast<uint32_t*>(workspace);
  const int32_t words = stride / (32 / bits);
  if (int rc = hip_status(clef::launch_prepare(w, rows, cols, stride, bits, staging, hs(stream))))
    return rc;
  if (int rc = hip_status(clef::launch_retile(staging, rows, words, cols / (32 / bits), tiled, hs(stream))))
    return rc;
  return hip_status(hipMemcpyAsync(scales, staging + rows * words, (size_t)rows * 4,
                                   hipMemcpyDeviceToDevice, hs(stream)));
}

int clef_untile_rows(const uint16_t* tiled, int64_t rows, int32_t cols, uint16_t* out,
                     clef_stream_t stream) {
  if (!(rows > 0 && cols > 0 && rows % 256 == 0 && cols % 64 == 0))
    return fail("tiled layout requires 256-row and 64-column multiples");
  if (!aligned(tiled, 16) || !aligned(out, 16)) return fail(kAlign);
  return hip_status(clef::launch_tile_permute(tiled, rows, cols, out, false, hs(stream)));
}

int clef_tile_rows(const uint16_t* dense, int64_t rows, int32_t cols, uint16_t* out,
                   clef_stream_t stream) {
  if (!(rows > 0 && cols > 0 && rows % 256 == 0 && cols % 64 == 0))
    return fail("tiled layout requires 256-row and 64-column multiples");
  if (!aligned(dense, 16) || !aligned(out, 16)) return fail(kAlign);
  return hip_status(clef::launch_tile_permute(dense, rows, cols, out, true, hs(stream)));
}

int clef_i4_gemm_configs(void) { return clef::gemm_config_count(); }

int clef_i4_gemm_config(const uint32_t* a, int32_t k_stride, const float* a_scales,
                        const uint32_t* w_tiled, const float* w_scales, int64_t m, int32_t n,
                        int32_t k, const uint16_t* residual, uint16_t* out, int32_t config,
                        clef_stream_t stream) {
  if (int rc = check_gemm(m, n, k, k_stride)) return rc;
  if (config < -1 || config >= clef::gemm_config_count()) return fail("unknown GEMM tile configuration");
  if (!aligned(a, 16) || !aligned(a_scales, 4) || !aligned(w_tiled, 16) || !aligned(w_scales, 16) ||
      !aligned(out, 16) || (residual && !aligned(residual, 16)))
    return fail(kAlign);
  return hip_status(clef::launch_gemm_i4(a, k_stride / 8, a_scales, w_tiled, w_scales, m, n, k,
                                         residual, out, config, hs(stream)));
}

int clef_i4_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales, const uint32_t* w_tiled,
                 const float* w_scales, int64_t m, int32_t n, int32_t k, const uint16_t* residual,
                 uint16_t* out, clef_stream_t stream) {
  return clef_i4_gemm_config(a, k_stride, a_scales, w_tiled, w_scales, m, n, k, residual, out, -1,
                             stream);
}

int clef_i8_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales, const uint32_t* w_tiled,
                 const float* w_scales, int64_t m, int32_t n, int32_t k, const uint16_t* residual,
                 uint16_t* out, clef_stream_t stream) {
  if (int rc = check_gemm(m, n, k, k_stride)) return rc;
  if (k_stride % 64 != 0) return fail("unsupported integer projection shape");
  if (!aligned(a, 16) || !aligned(w_tiled, 16) || !aligned(w_scales, 16) || !aligned(out, 16) ||
      (residual && !aligned(residual, 16)))
    return fail(kAlign);
  return hip_status(
      clef::launch_gemm_i8(a, k_stride / 4, a_scales, w_tiled, w_scales, m, n, k, residual, out, hs(stream)));
}

size_t clef_i4_project_workspace_bytes(int64_t m, int32_t k) {
  if (m < 0 || k < 0) return 0;
  return align256((size_t)prepared_words(m, stride_for(k, 4), 4) * 4);
}

int clef_i4_project(const uint16_t* x, int64_t m, int32_t k, const uint32_t* w_tiled,
                    const float* w_scales, int32_t n, const uint16_t* residual, uint16_t* out,
                    void* workspace, size_t workspace_bytes, clef_stream_t stream) {
  const int32_t stride = stride_for(k, 4);
  if (int rc = check_prepare(m, k, stride, 4)) return rc;
  if (int rc = check_gemm(m, n, k, stride)) return rc;
  if (!aligned(x, 16) || !aligned(workspace, 16) || !aligned(w_tiled, 16) || !aligned(w_scales, 16) ||
      !aligned(out, 16) || (residual && !aligned(residual, 16)))
    return fail(kAlign);
  if (workspace_bytes < clef_i4_project_workspace_bytes(m, k)) return fail(kWorkspace);
  uint32_t* packed = static_cast<uint32_t*>(workspace);
  if (int rc = hip_status(clef::launch_prepare(x, m, k, stride, 4, packed, hs(stream)))) return rc;
  const float* a_scales = reinterpret_cast<const float*>(packed + m * (stride / 8));
  return hip_status(clef::launch_gemm_i4(packed, stride / 8, a_scales, w_tiled, w_scales, m, n, k,
                                         residual, out, -1, hs(stream)));
}

int clef_moe_route(const void* logits, int32_t logits_dtype, int64_t tokens, int32_t experts,
                   int32_t topk, float* routes, clef_stream_t stream) {
  // src/omni.rs:171-174.
  if (!(topk > 0 && topk <= experts && experts <= 128)) return fail("invalid expert router shape");
  if (logits_dtype != 0 && logits_dtype != 1) return fail("invalid router logits dtype");
  if (tokens < 1 || tokens > 16777216) return fail("invalid expert router shape");
  if (!aligned(logits, 4) || !aligned(routes, 4)) return fail(kAlign);
  return hip_status(clef::launch_route(logits, logits_dtype, tokens, experts, topk, routes, hs(stream)));
}

int clef_moe_router_logits(const uint16_t* x, const uint16_t* gate_w, int64_t tokens, int32_t hidden,
                           int32_t experts, uint16_t* logits, clef_stream_t stream) {
  if (!(tokens >= 1 && hidden >= 64 && hidden % 64 == 0 && experts >= 32 && experts <= 128 && experts % 32 == 0))
    return fail("linear shape/dtype mismatch");
  if (!aligned(x, 16) || !aligned(gate_w, 16) || !aligned(logits, 2)) return fail(kAlign);
  return hip_status(clef::launch_router_gate(x, gate_w, tokens, hidden, experts, logits, hs(stream)));
}

size_t clef_moe_group_workspace_bytes(int64_t tokens) {
  if (tokens < 1) return 0;
  return align256(clef::group_workspace_bytes(tokens));
}

int clef_moe_group_routes(const float* routes, int64_t tokens, int32_t topk, float* groups,
                          float* order, void* workspace, size_t workspace_bytes,
                          clef_stream_t stream) {
  // src/omni.rs:194-197, with the chunk cap raised.
  if (!(tokens >= 1 && tokens <= 1048576 && topk >= 1 && topk <= 128))
    return fail("unsupported Omni route grouping shape");
  if (!aligned(routes, 4) || !aligned(groups, 4) || (order && !aligned(order, 4)) ||
      !aligned(workspace, 16))
    return fail(kAlign);
  if (workspace_bytes < clef_moe_group_workspace_bytes(tokens)) return fail(kWorkspace);
  return hip_status(clef::launch_group_routes(routes, tokens, topk, groups, order, workspace, hs(stream)));
}

int clef_moe_expert_tasks(const float* groups, int64_t tokens, float* tasks, clef_stream_t stream) {
  if (!(tokens >= 1 && tokens <= 1048576)) return fail("unsupported compact Omni routes");
  if (!aligned(groups, 4) || !aligned(tasks, 4)) return fail(kAlign);
  return hip_status(clef::launch_expert_tasks(groups, tokens, tasks, hs(stream)));
}

size_t clef_moe_expert_workspace_bytes(int64_t tokens, int32_t topk) {
  if (tokens < 1 || topk < 1) return 0;
  return align256(clef::expert_schedule_bytes(tokens * topk));
}

int clef_moe_expert_i4(const uint32_t* a, int32_t stride, const float* a_scales,
                       const uint32_t* w_tiled, const float* w_scales, const float* groups,
                       int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                       uint16_t* out, void* workspace, size_t workspace_bytes,
                       clef_stream_t stream) {
  if (!(tokens >= 1 && tokens <= 1048576 && topk >= 1 && topk <= 128))
    return fail("invalid grouped expert routes");
  // src/omni.rs:461-466.
  if (!(k % 256 == 0 && n % 256 == 0 && k >= 256 && n >= 256 && stride >= k && stride % 32 == 0))
    return fail("unsupported Omni expert tile shape");
  if (!aligned(a, 16) || !aligned(a_scales, 4) || !aligned(w_tiled, 16) || !aligned(w_scales, 16) ||
      !aligned(groups, 4) || !aligned(out, 16) || !aligned(workspace, 16))
    return fail(kAlign);
  if (workspace_bytes < clef_moe_expert_workspace_bytes(tokens, topk)) return fail(kWorkspace);
  int32_t* schedule = static_cast<int32_t*>(workspace);
  if (int rc = hip_status(clef::launch_expert_schedule(groups, tokens, topk, schedule, hs(stream)))) return rc;
  return hip_status(clef::launch_expert_i4(a, stride / 8, a_scales, w_tiled, w_scales, groups, schedule,
                                           tokens, topk, k, n, input_routed ? 1 : 0, out, hs(stream)));
}

int clef_moe_expert_gate_up_i4(const uint32_t* a, int32_t stride, const float* a_scales, const uint32_t* gate_w,
                               const float* gate_s, const uint32_t* up_w, const float* up_s,
                               const float* groups, int64_t tokens, int32_t topk, int32_t k, int32_t n,
                               uint16_t* h, void* workspace, size_t workspace_bytes, clef_stream_t stream) {
  // src/omni.rs:309-320, 333-344.
  if (!(tokens >= 1 && tokens <= 1048576 && topk >= 1 && topk <= 128))
    return fail("fused gate/up requires regular grouped routes");
  if (!(k % 256 == 0 && k >= 256 && n % 128 == 0 && n >= 128 && stride >= k && stride % 32 == 0 &&
        tokens * (int64_t)(stride / 8) * 4 < ((int64_t)1 << 31)))
    return fail("incompatible fused expert weights");
  if (!aligned(a, 16) || !aligned(a_scales, 4) || !aligned(gate_w, 16) || !aligned(gate_s, 16) ||
      !aligned(up_w, 16) || !aligned(up_s, 16) || !aligned(groups, 4) || !aligned(h, 16) ||
      !aligned(workspace, 16))
    return fail(kAlign);
  if (workspace_bytes < clef_moe_expert_workspace_bytes(tokens, topk)) return fail(kWorkspace);
  int32_t* schedule = static_cast<int32_t*>(workspace);
  if (int rc = hip_status(clef::launch_expert_schedule(groups, tokens, topk, schedule, hs(stream)))) return rc;
  return hip_status(clef::launch_expert_gate_up(a, stride / 8, a_scales, gate_w, gate_s, up_w, up_s, groups,
                                                schedule, tokens, topk, k, n, h, hs(stream)));
}

int clef_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h, clef_stream_t stream) {
  if (n < 0) return fail("SwiGLU shape/dtype mismatch");
  if (n == 0) return CLEF_OK;
  if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(h, 16)) return fail(kAlign);
  return hip_status(clef::launch_swiglu(gate, up, n, h, hs(stream)));
}

int clef_moe_combine(const uint16_t* values, const float* routes, const float* order,
                     int64_t tokens, int32_t width, int32_t topk, uint16_t* out,
                     clef_stream_t stream) {
  // src/omni.rs:253-262.
  if (!(tokens >= 1 && width >= 8 && width % 8 == 0 && topk >= 1 && topk <= 128))
    return fail("unsupported ordered Omni accumulation");
  if (!aligned(values, 16) || !aligned(routes, 4) || (order && !aligned(order, 4)) || !aligned(out, 16))
    return fail(kAlign);
  return hip_status(clef::launch_combine(values, routes, order, tokens, width, topk, out, hs(stream)));
}

}  // extern "C"

namespace {

// Workspace carve-up of the MoE block; offsets are 256-byte aligned.
struct MoeLayout {
  size_t routes, groups, order, group_ws, schedule, ax, gate, up, ah, values, total;
};

MoeLayout moe_layout(int64_t tokens, int32_t hidden, int32_t inter, int32_t topk) {
  MoeLayout l{};
  const int64_t routed = tokens * topk;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at += align256(bytes);
    return here;
  };
  l.routes = take((size_t)tokens * 2 * topk * 4);
  l.groups = take((size_t)128 * (tokens + 1) * 4);
  l.order = take((size_t)routed * 4);
  l.group_ws = take(clef::group_workspace_bytes(tokens));
  l.schedule = take(clef::expert_schedule_bytes(routed));
  l.ax = take((size_t)prepared_words(tokens, stride_for(hidden, 4), 4) * 4);
  l.gate = take((size_t)routed * inter * 2);
  l.up = take((size_t)routed * inter * 2);
  l.ah = take((size_t)prepared_words(routed, stride_for(inter, 4), 4) * 4);
  l.values = take((size_t)routed * hidden * 2);
  l.total = at;
  return l;
}

}  // namespace

extern "C" {

size_t clef_moe_layer_workspace_bytes(int64_t tokens, int32_t hidden, int32_t inter, int32_t topk) {
  if (tokens < 1 || hidden < 1 || inter < 1 || topk < 1) return 0;
  return moe_layout(tokens, hidden, inter, topk).total;
}

int clef_moe_layer(const uint16_t* x, const void* logits, int32_t logits_dtype, int64_t tokens,
                   int32_t hidden, int32_t inter, int32_t experts, int32_t topk,
                   const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                   const float* up_s, const uint32_t* down_w, const float* down_s,
                   float* routes_out, uint16_t* out, void* workspace, size_t workspace_bytes,
                   clef_stream_t stream) {
  if (experts != 128) return fail("Omni MoE requires 128 experts");
  if (!(topk >= 1 && topk <= experts)) return fail("invalid expert router shape");
  if (!(tokens >= 1 && tokens <= 1048576 && tokens * topk <= 16777216))
    return fail("unsupported Omni route grouping shape");
  if (!(hidden % 256 == 0 && inter % 256 == 0 && hidden >= 256 && inter >= 256))
    return fail("unsupported Omni expert tile shape");
  const int32_t sx = stride_for(hidden, 4), sh = stride_for(inter, 4);
  if (int rc = check_prepare(tokens, hidden, sx, 4)) return rc;
  if (int rc = check_prepare(tokens * topk, inter, sh, 4)) return rc;
  if (!aligned(x, 16) || !aligned(logits, 4) || !aligned(gate_w, 16) || !aligned(gate_s, 16) ||
      !aligned(up_w, 16) || !aligned(up_s, 16) || !aligned(down_w, 16) || !aligned(down_s, 16) ||
      !aligned(out, 16) || !aligned(workspace, 256) || (routes_out && !aligned(routes_out, 4)))
    return fail(kAlign);
  const MoeLayout l = moe_layout(tokens, hidden, inter, topk);
  if (workspace_bytes < l.total) return fail(kWorkspace);
  char* ws = static_cast<char*>(workspace);
  float* routes = routes_out ? routes_out : reinterpret_cast<float*>(ws + l.routes);
  float* groups = reinterpret_cast<float*>(ws + l.groups);
  float* order = reinterpret_cast<float*>(ws + l.order);
  int32_t* schedule = reinterpret_cast<int32_t*>(ws + l.schedule);
  uint32_t* ax = reinterpret_cast<uint32_t*>(ws + l.ax);
  uint16_t* gate = reinterpret_cast<uint16_t*>(ws + l.gate);
  uint16_t* up = reinterpret_cast<uint16_t*>(ws + l.up);
  uint32_t* ah = reinterpret_cast<uint32_t*>(ws + l.ah);
  uint16_t* values = reinterpret_cast<uint16_t*>(ws + l.values);
  const int64_t routed = tokens * topk;
  const float* axs = reinterpret_cast<const float*>(ax + tokens * (sx / 8));
  const float* ahs = reinterpret_cast<const float*>(ah + routed * (sh / 8));
  hipStream_t s = hs(stream);

#define CLEF_STEP(call) \
  if (int rc = hip_status(call)) return rc
  if (clef::route_prepare_fusable(hidden)) {  // router and the quantizer of x side by side
    CLEF_STEP(clef::launch_route_prepare(logits, logits_dtype, tokens, experts, topk, routes, x, hidden, sx, ax, s));
    CLEF_STEP(clef::launch_group_routes(routes, tokens, topk, groups, order, ws + l.group_ws, s, schedule,
                                        clef::expert_tile_rows(routed)));
  } else {
    CLEF_STEP(clef::launch_route(logits, logits_dtype, tokens, experts, topk, routes, s));
    CLEF_STEP(clef::launch_group_routes(routes, tokens, topk, groups, order, ws + l.group_ws, s, schedule,
                                        clef::expert_tile_rows(routed)));
    CLEF_STEP(clef::launch_prepare(x, tokens, hidden, sx, 4, ax, s));
  }
  if (tokens * (int64_t)(sx / 8) * 4 < ((int64_t)1 << 31)) {
    // Gate and up share one pass over the gathered x rows and SwiGLU runs in
    // their epilogue; h is then quantized per routed row. Bit-equal to the
    // separate gate, up, swiglu and prepare (each lane applies the same E1
    // rounding and S1 to the same bf16 values).
    CLEF_STEP(clef::launch_expert_gate_up(ax, sx / 8, axs, gate_w, gate_s, up_w, up_s, groups, schedule, tokens,
                                          topk, hidden, inter, gate, s));
    CLEF_STEP(clef::launch_prepare(gate, routed, inter, sh, 4, ah, s));
  } else {
    CLEF_STEP(clef::launch_expert_i4(ax, sx / 8, axs, gate_w, gate_s, groups, schedule, tokens, topk,
                                     hidden, inter, 0, gate, s));
    CLEF_STEP(clef::launch_expert_i4(ax, sx / 8, axs, up_w, up_s, groups, schedule, tokens, topk,
                                     hidden, inter, 0, up, s));
    // SwiGLU fused into the quantizer of h: bit-equal to swiglu then prepare
    // (src/quantized.rs:1189-1266).
    CLEF_STEP(clef::launch_prepare_swiglu(gate, up, routed, inter, sh, 4, ah, s));
  }
  CLEF_STEP(clef::launch_expert_i4(ah, sh / 8, ahs, down_w, down_s, groups, schedule, tokens, topk,
                                   inter, hidden, 1, values, s));
  CLEF_STEP(clef::launch_combine(values, routes, order, tokens, hidden, topk, out, s));
#undef CLEF_STEP
  return CLEF_OK;
}

}  // extern "C"
