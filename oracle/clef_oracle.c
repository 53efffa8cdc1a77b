/*
 * CPU oracle for the clef-hrx INT4 quantized-matmul and Omni INT4 MoE path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline. The
 * product library never links or calls this file.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off). Plain IEEE f32
 * arithmetic; no FMA contraction except the explicit fmaf() in orc_expf.
 *
 * Pinning (what checks each function independently of this file):
 *   orc_rotate256     H.H^T = 256 I, Kronecker-product matrix (tests)
 *   orc_prepare       closed forms (e_0 row, constant rows), the reference test
 *                     oracle's formula on its own inputs, identity-weight KAT
 *   orc_retile        the retile formula on index-valued words
 *   orc_gemm(_acc)    int64 brute-force dot, power-of-two-scale closed forms,
 *                     identity-weight KAT, saturation/NaN cases
 *   orc_route         stable descending sort of the logits (ties -> lowest id)
 *   orc_group_routes  brute-force list construction, total-order sort of ids
 *   orc_expert_tasks  brute-force task list
 *   orc_expert_i4     dense oracle (orc_gemm_acc) restricted to routed rows
 *   orc_expert_i4_ungrouped  orc_expert_i4 on duplicate-free routes; the
 *                     dense oracle on every slot (duplicates included)
 *   orc_swiglu        float64 SiLU within one bf16 step per rounding
 *   orc_combine       the reference's sparse MoE test formula
 *   orc_expf          float64 exp, <= 2 ulp
 *   orc_prepare_attention_gate  Q1 of the float64-checked gate product (tests)
 *   orc_prepare_norm  = Q1(orc_rms_norm) bit for bit; orc_rms_norm against a
 *                     float64 RMSNorm within one bf16 step (tests)
 * exp bits: the reference uses expf<afn>, whose bits are those of the gfx1151
 * hardware approximation; orc_expf is the Cephes expf method (S. L. Moshier,
 * Cephes Math Library, expf.c), which the HIP kernels evaluate with the same
 * steps. Agreement with the reference's exp bits is therefore "parity
 * unpinned" beyond the float64 accuracy bound.
 */
#include "clef_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_error[256];

static int fail(const char* msg) {
    snprintf(g_error, sizeof g_error, "%s", msg);
    return -1;
}

const char* orc_last_error(void) { return g_error; }

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* f32 -> bf16 round-to-nearest-even; NaN stays NaN (quiet).
 * kernels/common.loom:29-35 (scalar.fptrunc f32 to bf16). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float bf16_round(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* Cephes expf (Moshier): Cody-Waite reduction by ln 2 with C1 = 0.693359375,
 * C2 = -2.12194440e-4, then the degree-5 minimax polynomial of expf.c.
 * Stands in for the reference's expf<afn> (kernels/swiglu.loom:46,
 * kernels/omni_route.loom:131). */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972076416015625f) return 0.0f;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float r2 = r * r;
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    return ldexpf(p, (int)n);
}

/* 256-point radix-4 rotation, strides 1,4,16,64, this exact op order.
 * src/quantized.rs:801-824 (test oracle `rotated`);
 * kernels/prepare_integer_single.loom:87-248. */
void orc_rotate256(float* g) {
    static const int strides[4] = {1, 4, 16, 64};
    for (int si = 0; si < 4; ++si) {
        int s = strides[si];
        for (int base = 0; base < 256; base += 4 * s) {
            for (int i = 0; i < s; ++i) {
                int j = base + i;
                float a = g[j], b = g[j + s], c = g[j + 2 * s], d = g[j + 3 * s];
                float s01 = a + b, s23 = c + d, d01 = a - b, d23 = c - d;
                g[j] = s01 + d23;
                g[j + s] = s01 - d23;
                g[j + 2 * s] = d01 + s23;
                g[j + 3 * s] = s23 - d01;
            }
        }
    }
}

/* Preconditions of prepare_inputs (src/quantized.rs:634-649). */
static int check_prepare(int64_t rows, int32_t width, int32_t stride, int32_t bits) {
    if (!((bits == 4 || bits == 8) && width >= 256 && width <= 32768 && width % 256 == 0 &&
          rows >= 1 && rows <= 1048576 && stride >= width && stride <= 65536 &&
          stride % (512 / bits) == 0))
        return fail("unsupported rotated integer operand");
    return 0;
}

/* Quantize one already-materialized f32 row (Q1 steps 2-5).
 * kernels/prepare_integer_single.loom:222-286; src/quantized.rs:990-1004. */
static void quantize_row(float* v, int32_t width, int32_t bits, uint32_t* words, float* scale_out) {
    for (int g = 0; g < width; g += 256) orc_rotate256(v + g);
    float m = 0.0f;
    for (int i = 0; i < width; ++i) {
        float a = fabsf(v[i]);
        float checked = a < INFINITY ? a : INFINITY; /* NaN -> +inf */
        m = fmaxf(m, checked);
    }
    const float qmax = bits == 8 ? 127.0f : 7.0f;
    float normal = m * 0.0625f;
    float safe = fmaxf(normal, 1e-30f);
    float scale = safe / qmax;
    int valid = scale < INFINITY;
    float inv = 0.0625f / scale;
    const int per_word = 32 / bits;
    const uint32_t mask = bits == 8 ? 0xffu : 0xfu;
    for (int w = 0; w < width / per_word; ++w) {
        uint32_t word = 0;
        for (int p = 0; p < per_word; ++p) {
            float scaled = v[w * per_word + p] * inv;
            float s = valid ? scaled : 0.0f;
            float r = rintf(s);
            float lo = fmaxf(r, -qmax);
            float hi = fminf(lo, qmax);
            int code = (int)hi;
            word |= ((uint32_t)code & mask) << (p * bits);
        }
        words[w] = word;
    }
    *scale_out = scale;
}

/* Q1. Storage: codes [rows][stride/(32/bits)] then rows f32 scales
 * (src/quantized.rs:656-664). Padding words past width are left untouched. */
int orc_prepare(const uint16_t* x, int64_t rows, int32_t width, int32_t stride, int32_t bits,
                uint32_t* out) {
    if (check_prepare(rows, width, stride, bits)) return -1;
    const int64_t words = stride / (32 / bits);
    float* scales = (float*)(out + rows * words);
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * width);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            for (int i = 0; i < width; ++i) v[i] = orc_bf16_to_f32(x[r * width + i]);
            quantize_row(v, width, bits, out + r * words, &scales[r]);
        }
        free(v);
    }
    return 0;
}

/* S1 then Q1 with both BF16 materializations
 * (kernels/prepare_integer_register.loom:155-172). */
int orc_prepare_swiglu(const uint16_t* gate, const uint16_t* up, int64_t rows, int32_t width,
                       int32_t stride, int32_t bits, uint32_t* out) {
    if (check_prepare(rows, width, stride, bits)) return -1;
    const int64_t words = stride / (32 / bits);
    float* scales = (float*)(out + rows * words);
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * width);
        uint16_t* h = (uint16_t*)malloc(sizeof(uint16_t) * width);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            orc_swiglu(gate + r * width, up + r * width, width, h);
            for (int i = 0; i < width; ++i) v[i] = orc_bf16_to_f32(h[i]);
            quantize_row(v, width, bits, out + r * words, &scales[r]);
        }
        free(h);
        free(v);
    }
    return 0;
}

/* Attention-gate producer then Q1 (kernels/prepare_integer_register.loom:137-155;
 * src/quantized.rs:440-468, 626-635): the gate of column c is column
 * (c/256)*512 + 256 + c%256 of the [rows][2*width] q_gate row (query and gate
 * share each 512-column head block), s = bf16(1 / (1 + exp(-g))) and the
 * packed value is bf16(x * s). */
int orc_prepare_attention_gate(const uint16_t* x, const uint16_t* q_gate, int64_t rows, int32_t width,
                               int32_t stride, int32_t bits, uint32_t* out) {
    if (check_prepare(rows, width, stride, bits)) return -1;
    const int64_t words = stride / (32 / bits);
    float* scales = (float*)(out + rows * words);
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * width);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            for (int c = 0; c < width; ++c) {
                const float g = orc_bf16_to_f32(q_gate[r * 2 * width + (c / 256) * 512 + 256 + c % 256]);
                const float e = orc_expf(-g);
                const float sig = bf16_round(1.0f / (1.0f + e));
                v[c] = bf16_round(orc_bf16_to_f32(x[r * width + c]) * sig);
            }
            quantize_row(v, width, bits, out + r * words, &scales[r]);
        }
        free(v);
    }
    return 0;
}

/* Inverse RMS of one 5120-wide row in the fixed summation order of the fused
 * producer kernel: thread t of 256 (group g = t/16 and g + 16, lane l = t%16)
 * sums fma(x, x, acc) over columns g*256 + 16l .. +15 of each of its groups in
 * turn; each 64-thread wave adds across lanes by the butterfly
 * s[l] += s[l ^ o] for o = 32, 16, ..., 1; the four wave sums are added in wave
 * order. The reference reduces in an order of its compiler's choosing
 * (kernels/prepare_integer_register.loom:63-80: workgroup.reduce<addf>) and
 * uses an approximate rsqrt; here inv = 1 / sqrt(ss / 5120 + 1e-6) with
 * correctly rounded sqrt and division. */
static float norm_row_inv(const uint16_t* x, int32_t width) {
    float s[256];
    const int groups = width / 256;
    for (int t = 0; t < 256; ++t) {
        const int g = t / 16, l = t % 16;
        float acc = 0.0f;
        for (int p = 0; p < 2; ++p) {
            const int grp = g + 16 * p;
            if (grp >= groups) continue;
            for (int i = 0; i < 16; ++i) {
                const float v = orc_bf16_to_f32(x[grp * 256 + 16 * l + i]);
                acc = fmaf(v, v, acc);
            }
        }
        s[t] = acc;
    }
    float wave[4];
    for (int w = 0; w < 4; ++w) {
        float* a = s + 64 * w;
        for (int o = 32; o >= 1; o >>= 1) {
            float b[64];
            for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ o];
            memcpy(a, b, sizeof(b));
        }
        wave[w] = a[0];
    }
    const float ss = ((wave[0] + wave[1]) + wave[2]) + wave[3];
    const float var = ss / (float)width;
    const float ve = var + 1e-6f;
    return 1.0f / sqrtf(ve);
}

/* Named-RMSNorm producer then Q1 (kernels/prepare_integer_register.loom:63-80,
 * 112-134; src/quantized.rs:713-779): width 5120, weight offset 1, eps 1e-6.
 * n = x * inv, r = fma(n, w + 1, 0), the packed value is bf16(r); when
 * normalized is not NULL the bf16 values are also written there ([rows][5120]). */
int orc_prepare_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width,
                     int32_t stride, int32_t bits, uint32_t* out, uint16_t* normalized) {
    if (!(width == 5120 && (bits == 4 || bits == 8) && rows >= 1 && rows <= 1048576 && stride >= width &&
          stride <= 65536 && stride % (512 / bits) == 0))
        return fail("unsupported normalized packing shape");
    const int64_t words = stride / (32 / bits);
    float* scales = (float*)(out + rows * words);
#pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * width);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const uint16_t* xr = x + r * width;
            const float inv = norm_row_inv(xr, width);
            for (int c = 0; c < width; ++c) {
                const float n = orc_bf16_to_f32(xr[c]) * inv;
                const float nw = orc_bf16_to_f32(weight[c]) + 1.0f;
                const uint16_t h = orc_f32_to_bf16(fmaf(n, nw, 0.0f));
                if (normalized) normalized[r * width + c] = h;
                v[c] = orc_bf16_to_f32(h);
            }
            quantize_row(v, width, bits, out + r * words, &scales[r]);
        }
        free(v);
    }
    return 0;
}

/* Unfused named RMSNorm (kernels/norm.loom:57-95 without bias, weight offset
 * 1): the same inverse RMS as orc_prepare_norm, out = bf16(fma(x * inv, w + 1, 0)).
 * The fused producer must equal Q1 of this output. */
int orc_rms_norm(const uint16_t* x, const uint16_t* weight, int64_t rows, int32_t width, uint16_t* out) {
    if (width != 5120 || rows < 1) return fail("norm dimensions");
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * width;
        const float inv = norm_row_inv(xr, width);
        for (int c = 0; c < width; ++c) {
            const float n = orc_bf16_to_f32(xr[c]) * inv;
            out[r * width + c] = orc_f32_to_bf16(fmaf(n, orc_bf16_to_f32(weight[c]) + 1.0f, 0.0f));
        }
    }
    return 0;
}

/* Q2 retile: word (n, q) -> ((n/128)*blocks_k + q/32)*4096 + (n%128)*32 + q%32.
 * kernels/retile_codes.loom:2-5,38-55; preconditions src/quantized.rs:550-558. */
int orc_retile(const uint32_t* codes, int64_t rows, int32_t in_words, int32_t cols, int32_t bits,
               uint32_t* tiled) {
    const int64_t words = cols / (32 / bits);
    if (!(rows % 128 == 0 && words % 32 == 0 && in_words >= words && rows > 0))
        return fail("unsupported packed weight shape for tiling");
    const int64_t blocks_k = words / 32;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < rows; ++n)
        for (int64_t q = 0; q < words; ++q)
            tiled[((n / 128) * blocks_k + q / 32) * 4096 + (n % 128) * 32 + q % 32] =
                codes[n * in_words + q];
    return 0;
}

/* Signed code k of a packed word stream (bits 4: 8 per word, bits 8: 4 per word). */
static inline int code_at(const uint32_t* row_words, int k, int bits) {
    const int per_word = 32 / bits;
    uint32_t w = row_words[k / per_word];
    int shift = (k % per_word) * bits;
    return (int32_t)(w << (32 - bits - shift)) >> (32 - bits);
}

/* Unpack one tiled weight row to int8. */
static void unpack_tiled_row(const uint32_t* w_tiled, int64_t n, int32_t k, int32_t bits,
                             int8_t* dst) {
    const int per_word = 32 / bits;
    const int64_t words = k / per_word, blocks_k = words / 32;
    for (int64_t q = 0; q < words; ++q) {
        uint32_t w = w_tiled[((n / 128) * blocks_k + q / 32) * 4096 + (n % 128) * 32 + q % 32];
        for (int p = 0; p < per_word; ++p) {
            int shift = p * bits;
            dst[q * per_word + p] = (int8_t)((int32_t)(w << (32 - bits - shift)) >> (32 - bits));
        }
    }
}

static void unpack_row(const uint32_t* row_words, int32_t k, int32_t bits, int8_t* dst) {
    for (int i = 0; i < k; ++i) dst[i] = (int8_t)code_at(row_words, i, bits);
}

static int32_t dot_i8(const int8_t* a, const int8_t* b, int32_t k) {
    int32_t s = 0;
    for (int32_t i = 0; i < k; ++i) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

static int check_gemm(int64_t m, int32_t n, int32_t k, int32_t k_stride, int32_t bits) {
    if (!((bits == 4 || bits == 8) && m >= 1 && n >= 128 && n % 128 == 0 && k >= 256 &&
          k % 256 == 0 && k_stride >= k && k_stride % (32 / bits) == 0))
        return fail("unsupported integer projection shape");
    return 0;
}

/* G1 accumulators: acc[m][n] = sum_k a[m][k] * w[n][k] in exact i32.
 * kernels/gemm_integer.loom:199-272 (K loop), src/quantized.rs:1048-1066. */
int orc_gemm_acc(const uint32_t* a, int32_t k_stride, const uint32_t* w_tiled, int64_t m,
                 int32_t n, int32_t k, int32_t bits, int32_t* acc) {
    if (check_gemm(m, n, k, k_stride, bits)) return -1;
    const int64_t a_words = k_stride / (32 / bits);
    int8_t* wu = (int8_t*)malloc((size_t)n * k);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < n; ++c) unpack_tiled_row(w_tiled, c, k, bits, wu + c * k);
#pragma omp parallel
    {
        int8_t* au = (int8_t*)malloc((size_t)k);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            unpack_row(a + r * a_words, k, bits, au);
            for (int64_t c = 0; c < n; ++c) acc[r * n + c] = dot_i8(au, wu + c * k, k);
        }
        free(au);
    }
    free(wu);
    return 0;
}

/* G1 epilogue: y = RN(RN(f32(acc)*ws[n])*as[m]) + 0; clamp finite y to the
 * BF16 finite range; bf16 RNE; residual: bf16(f32(res) + f32(out)).
 * kernels/gemm_integer.loom:394-433. */
static inline uint16_t g1_epilogue(int32_t acc, float ws, float as, const uint16_t* residual) {
    const float bmax = 3.3895313892515355e38f;
    float y = (float)acc * ws;
    y = y * as;
    y = y + 0.0f;
    float sat = fmaxf(fminf(y, bmax), -bmax);
    float checked = fabsf(y) < INFINITY ? sat : y;
    uint16_t out = orc_f32_to_bf16(checked);
    if (residual) out = orc_f32_to_bf16(orc_bf16_to_f32(*residual) + orc_bf16_to_f32(out));
    return out;
}

int orc_gemm(const uint32_t* a, int32_t k_stride, const float* a_scales, const uint32_t* w_tiled,
             const float* w_scales, int64_t m, int32_t n, int32_t k, int32_t bits,
             const uint16_t* residual, uint16_t* out) {
    if (check_gemm(m, n, k, k_stride, bits)) return -1;
    const int64_t a_words = k_stride / (32 / bits);
    int8_t* wu = (int8_t*)malloc((size_t)n * k);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < n; ++c) unpack_tiled_row(w_tiled, c, k, bits, wu + c * k);
#pragma omp parallel
    {
        int8_t* au = (int8_t*)malloc((size_t)k);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; ++r) {
            unpack_row(a + r * a_words, k, bits, au);
            for (int64_t c = 0; c < n; ++c) {
                int32_t acc = dot_i8(au, wu + c * k, k);
                out[r * n + c] = g1_epilogue(acc, w_scales[c], a_scales[r],
                                             residual ? residual + r * n + c : NULL);
            }
        }
        free(au);
    }
    free(wu);
    return 0;
}

/* R1 router, one token: kernels/omni_route.loom:40-146. Max by maxNum with
 * invalid slots at -FLT_MAX, ties -> lowest expert id (no match -> 2^31-1),
 * selected slot reset to -FLT_MAX; then exp(v - v0) summed in rank order and
 * bf16-rounded probabilities. */
static void route_token(const float* logits, int32_t experts, int32_t topk, float* out) {
    const float neg = -3.402823466e38f;
    float vals[128];
    for (int e = 0; e < 128; ++e) vals[e] = e < experts ? logits[e] : neg;
    for (int r = 0; r < topk; ++r) {
        float best = vals[0];
        for (int e = 1; e < 128; ++e) best = fmaxf(best, vals[e]);
        uint32_t id = 2147483647u;
        for (int e = 0; e < experts; ++e)
            if (vals[e] == best) {
                id = (uint32_t)e;
                break;
            }
        out[r] = (float)(int32_t)id;
        out[topk + r] = best;
        if (id < 128) vals[id] = neg;
    }
    const float vmax = out[topk];
    float sum = 0.0f;
    for (int j = 0; j < topk; ++j) {
        float p = orc_expf(out[topk + j] - vmax);
        out[topk + j] = p;
        sum = sum + p;
    }
    for (int j = 0; j < topk; ++j) out[topk + j] = bf16_round(out[topk + j] / sum);
}

/* Engine::omni_route preconditions: src/omni.rs:170-190. */
int orc_route(const void* logits, int32_t dtype, int64_t tokens, int32_t experts, int32_t topk,
              float* routes) {
    if (!(topk > 0 && topk <= experts && experts <= 128)) return fail("invalid expert router shape");
    if (dtype != 0 && dtype != 1) return fail("invalid router logits dtype");
#pragma omp parallel
    {
        float row[128];
#pragma omp for schedule(static)
        for (int64_t t = 0; t < tokens; ++t) {
            for (int e = 0; e < experts; ++e)
                row[e] = dtype == 0 ? orc_bf16_to_f32(((const uint16_t*)logits)[t * experts + e])
                                    : ((const float*)logits)[t * experts + e];
            route_token(row, experts, topk, routes + t * 2 * topk);
        }
    }
    return 0;
}

/* R2: per expert e (128 of them), groups[e][0] = count, groups[e][1+i] =
 * f32(t*topk + r) for the i-th token (ascending) whose LAST rank r with id e
 * matches; order[t][#(ids < e)] = r. kernels/omni_group_routes.loom:43-82,
 * kernels/omni_group_routes_ordered.loom:50-87. */
int orc_group_routes(const float* routes, int64_t tokens, int32_t topk, float* groups,
                     float* order) {
    if (!(tokens >= 1 && topk >= 1 && topk <= 128)) return fail("unsupported Omni route grouping shape");
    const int64_t stride = tokens + 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int e = 0; e < 128; ++e) {
        int64_t count = 0;
        for (int64_t t = 0; t < tokens; ++t) {
            const float* rt = routes + t * 2 * topk;
            int rank = topk, less = 0;
            for (int r = 0; r < topk; ++r) {
                if ((int32_t)rt[r] == e) rank = r;
                if (rt[r] < (float)e) ++less;
            }
            if (rank < topk) {
                groups[e * stride + 1 + count] = (float)(int32_t)(t * topk + rank);
                if (order) order[t * topk + less] = (float)rank;
                ++count;
            }
        }
        groups[e * stride] = (float)(int32_t)count;
    }
    return 0;
}

/* R3: tasks[0] = total, then (e, 16*tile) for e ascending, tile <
 * ceil(count_e/16). kernels/omni_expert_tasks.loom:30-62. */
int orc_expert_tasks(const float* groups, int64_t tokens, float* tasks) {
    const int64_t stride = tokens + 1;
    int64_t total = 0;
    for (int e = 0; e < 128; ++e) {
        int64_t count = (int32_t)groups[e * stride];
        for (int64_t tile = 0; tile < (count + 15) / 16; ++tile) {
            tasks[1 + 2 * total] = (float)e;
            tasks[2 + 2 * total] = (float)(int32_t)(16 * tile);
            ++total;
        }
    }
    tasks[0] = (float)(int32_t)total;
    return 0;
}

/* E1: out[route][c] = bf16(RN(f32(acc) * RN(as[xr] * ws[e*n + c]))), xr =
 * input_routed ? route : route/topk. kernels/omni_expert_i4.loom:113-125,
 * 436-462; kernels/omni_expert.loom:86-146. Preconditions src/omni.rs:386-399,
 * 461-466 (k, n multiples of 256). */
int orc_expert_i4(const uint32_t* a, int32_t stride, const float* a_scales,
                  const uint32_t* w_tiled, const float* w_scales, const float* groups,
                  int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                  uint16_t* out) {
    if (!(k % 256 == 0 && n % 256 == 0 && k >= 256 && n >= 256 && stride >= k && stride % 8 == 0 &&
          tokens >= 1 && topk >= 1))
        return fail("unsupported Omni expert tile shape");
    const int64_t estride = tokens + 1, a_words = stride / 8;
#pragma omp parallel
    {
        int8_t* wu = (int8_t*)malloc((size_t)n * k);
        int8_t* au = (int8_t*)malloc((size_t)k);
#pragma omp for schedule(dynamic, 1)
        for (int e = 0; e < 128; ++e) {
            int64_t count = (int32_t)groups[e * estride];
            if (count == 0) continue;
            for (int64_t c = 0; c < n; ++c)
                unpack_tiled_row(w_tiled, (int64_t)e * n + c, k, 4, wu + c * k);
            for (int64_t i = 0; i < count; ++i) {
                int64_t route = (int32_t)groups[e * estride + 1 + i];
                int64_t xr = input_routed ? route : route / topk;
                unpack_row(a + xr * a_words, k, 4, au);
                float as = a_scales[xr];
                for (int64_t c = 0; c < n; ++c) {
                    int32_t acc = dot_i8(au, wu + c * k, k);
                    float s = as * w_scales[(int64_t)e * n + c];
                    out[route * n + c] = orc_f32_to_bf16((float)acc * s);
                }
            }
        }
        free(au);
        free(wu);
    }
    return 0;
}

/* Ungrouped E1 (Engine::omni_expert, src/omni.rs:280-288;
 * kernels/omni_expert.loom:86-150): every route slot (t, r) on its own, no
 * groups table. The expert is (int)routes[t][r] (slots naming no expert in
 * 0..127 are skipped); the dot is the exact integer sum the reference's f32
 * FMA chain reaches on integer codes; out[t*topk + r][c] =
 * bf16(RN(f32(dot) * RN(as[xr] * ws[e*n + c]))). */
int orc_expert_i4_ungrouped(const uint32_t* a, int32_t stride, const float* a_scales,
                            const uint32_t* w_tiled, const float* w_scales, const float* routes,
                            int64_t tokens, int32_t topk, int32_t k, int32_t n, int32_t input_routed,
                            uint16_t* out) {
    if (!(k % 256 == 0 && n % 256 == 0 && k >= 256 && n >= 256 && stride >= k && stride % 8 == 0 &&
          tokens >= 1 && topk >= 1))
        return fail("unsupported Omni expert tile shape");
    const int64_t a_words = stride / 8;
#pragma omp parallel
    {
        int8_t* wu = (int8_t*)malloc((size_t)k);
        int8_t* au = (int8_t*)malloc((size_t)k);
#pragma omp for schedule(dynamic, 16)
        for (int64_t slot = 0; slot < tokens * topk; ++slot) {
            const int64_t t = slot / topk, r = slot % topk;
            const float id = routes[t * 2 * topk + r];
            if (!(id > -1.0f && id < 128.0f)) continue;
            const int64_t e = (int32_t)id;
            const int64_t xr = input_routed ? slot : t;
            unpack_row(a + xr * a_words, k, 4, au);
            for (int64_t c = 0; c < n; ++c) {
                unpack_tiled_row(w_tiled, e * n + c, k, 4, wu);
                float s = a_scales[xr] * w_scales[e * n + c];
                out[slot * n + c] = orc_f32_to_bf16((float)dot_i8(au, wu, k) * s);
            }
        }
        free(au);
        free(wu);
    }
    return 0;
}

/* S1: h = bf16(f32(bf16(g / (1 + exp(-g)))) * u). kernels/swiglu.loom:43-51. */
void orc_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h) {
    for (int64_t i = 0; i < n; ++i) {
        float g = orc_bf16_to_f32(gate[i]);
        float u = orc_bf16_to_f32(up[i]);
        float e = orc_expf(-g);
        float d = 1.0f + e;
        float act = g / d;
        float r = bf16_round(act);
        h[i] = orc_f32_to_bf16(r * u);
    }
}

/* C1: acc = 0; for ranks in ascending expert id: acc = bf16(acc +
 * bf16(values[8t+rank][c] * p_rank)); out = bf16(acc).
 * kernels/omni_combine_ordered.loom:51-79 (order table),
 * kernels/omni_combine.loom:50-77 (selection by ascending id). */
int orc_combine(const uint16_t* values, const float* routes, const float* order, int64_t tokens,
                int32_t width, int32_t topk, uint16_t* out) {
    if (!(width % 8 == 0 && topk >= 1 && topk <= 128)) return fail("unsupported ordered Omni accumulation");
#pragma omp parallel
    {
        int ranks[128];
#pragma omp for schedule(static)
        for (int64_t t = 0; t < tokens; ++t) {
            const float* rt = routes + t * 2 * topk;
            if (order) {
                for (int j = 0; j < topk; ++j) ranks[j] = (int32_t)order[t * topk + j];
            } else {
                float prev = -1.0f;
                for (int j = 0; j < topk; ++j) {
                    float best = 1000000.0f;
                    int at = 0;
                    for (int r = 0; r < topk; ++r)
                        if (rt[r] > prev && rt[r] < best) {
                            best = rt[r];
                            at = r;
                        }
                    ranks[j] = at;
                    prev = best;
                }
            }
            for (int32_t c = 0; c < width; ++c) {
                float acc = 0.0f;
                for (int j = 0; j < topk; ++j) {
                    int rank = ranks[j];
                    float v = orc_bf16_to_f32(values[(t * topk + rank) * width + c]);
                    float p = rt[topk + rank];
                    float prod = bf16_round(v * p);
                    acc = bf16_round(acc + prod);
                }
                out[t * width + c] = orc_f32_to_bf16(acc);
            }
        }
    }
    return 0;
}

/* Omni INT4 MoE block, src/omni.rs:762-857 (fast defaults: ordered grouping,
 * shared packing, materialized SwiGLU): route -> group(ordered) -> Q1(x) ->
 * E1 gate, E1 up -> S1 -> Q1(h) -> E1 down (routed) -> C1. The stride rule
 * is src/quantized.rs:161-166. */
int orc_moe_layer(const uint16_t* x, const void* logits, int32_t logits_dtype, int64_t tokens,
                  int32_t hidden, int32_t inter, int32_t experts, int32_t topk,
                  const uint32_t* gate_w, const float* gate_s, const uint32_t* up_w,
                  const float* up_s, const uint32_t* down_w, const float* down_s,
                  float* routes_out, uint16_t* out) {
    if (experts != 128) return fail("Omni MoE requires 128 experts");
    const int32_t sx = hidden + (hidden % 1024 == 0 ? 128 : 0);
    const int32_t sh = inter + (inter % 1024 == 0 ? 128 : 0);
    const int64_t routes_n = tokens * topk;
    int rc = 0;
    float* routes = routes_out ? routes_out : (float*)malloc(sizeof(float) * tokens * 2 * topk);
    float* groups = (float*)malloc(sizeof(float) * 128 * (tokens + 1));
    float* order = (float*)malloc(sizeof(float) * routes_n);
    uint32_t* ax = (uint32_t*)malloc(sizeof(uint32_t) * tokens * (sx / 8 + 1));
    uint16_t* gate = (uint16_t*)malloc(sizeof(uint16_t) * routes_n * inter);
    uint16_t* up = (uint16_t*)malloc(sizeof(uint16_t) * routes_n * inter);
    uint32_t* ah = (uint32_t*)malloc(sizeof(uint32_t) * routes_n * (sh / 8 + 1));
    uint16_t* values = (uint16_t*)malloc(sizeof(uint16_t) * routes_n * hidden);
    if (!(groups && order && ax && gate && up && ah && values && routes)) {
        rc = fail("oracle allocation failed");
        goto done;
    }
    if ((rc = orc_route(logits, logits_dtype, tokens, experts, topk, routes))) goto done;
    if ((rc = orc_group_routes(routes, tokens, topk, groups, order))) goto done;
    if ((rc = orc_prepare(x, tokens, hidden, sx, 4, ax))) goto done;
    const float* axs = (const float*)(ax + tokens * (sx / 8));
    if ((rc = orc_expert_i4(ax, sx, axs, gate_w, gate_s, groups, tokens, topk, hidden, inter, 0, gate)))
        goto done;
    if ((rc = orc_expert_i4(ax, sx, axs, up_w, up_s, groups, tokens, topk, hidden, inter, 0, up)))
        goto done;
    orc_swiglu(gate, up, routes_n * inter, gate); /* in place: h overwrites gate */
    if ((rc = orc_prepare(gate, routes_n, inter, sh, 4, ah))) goto done;
    const float* ahs = (const float*)(ah + routes_n * (sh / 8));
    if ((rc = orc_expert_i4(ah, sh, ahs, down_w, down_s, groups, tokens, topk, inter, hidden, 1,
                            values)))
        goto done;
    rc = orc_combine(values, routes, order, tokens, hidden, topk, out);
done:
    if (!routes_out) free(routes);
    free(groups);
    free(order);
    free(ax);
    free(gate);
    free(up);
    free(ah);
    free(values);
    return rc;
}

/* [rows][cols] bf16 <-> [rows/256][cols/64][256][64]; src/checkpoint.rs:63-106. */
static int permute_tiles(const uint16_t* src, int64_t rows, int32_t cols, uint16_t* dst, int to_tiled) {
    if (!(rows > 0 && cols > 0 && rows % 256 == 0 && cols % 64 == 0))
        return fail("tiled layout requires 256-row and 64-column multiples");
    const int64_t k_steps = cols / 64;
#pragma omp parallel for schedule(static)
    for (int64_t tile = 0; tile < rows / 256; ++tile)
        for (int64_t ks = 0; ks < k_steps; ++ks)
            for (int64_t r = 0; r < 256; ++r) {
                int64_t dense = (tile * 256 + r) * cols + ks * 64;
                int64_t tiled = tile * 256 * cols + (ks * 256 + r) * 64;
                if (to_tiled)
                    memcpy(dst + tiled, src + dense, 128);
                else
                    memcpy(dst + dense, src + tiled, 128);
            }
    return 0;
}

int orc_tile_rows(const uint16_t* src, int64_t rows, int32_t cols, uint16_t* dst) {
    return permute_tiles(src, rows, cols, dst, 1);
}

int orc_untile_rows(const uint16_t* src, int64_t rows, int32_t cols, uint16_t* dst) {
    return permute_tiles(src, rows, cols, dst, 0);
}
