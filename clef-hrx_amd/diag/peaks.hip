// Device ceilings that bound the INT4 path on this GPU, printed as one JSON
// line for bench.py (`bench.py --only peaks`):
//   - v_mfma_i32_32x32x32_i8 issued back to back from registers (8
//     independent accumulators per wave, 4 waves per SIMD), for several
//     operand forms: the board's power limit lowers the clock as operand bit
//     activity rises, so the sustainable rate depends on the data;
//   - v_mfma_scale_f32_32x32x64_f8f6f4 on bf6 operands (unit scales) the
//     same way, zeros and the e3m2 form of the same gaussian int4 codes;
//   - the shader clock under that load (s_memtime cycles against the 100 MHz
//     s_memrealtime counter, read by one wave);
//   - HBM streaming read, write and copy over 1 GiB buffers (well past the
//     256 MiB last-level cache).
// Build: make -C clef-hrx_amd diag (lib/peaks).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

__device__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Operand forms: 0 zeros; 1 random bytes; 2 int4 codes as 16 * code with
// codes round(2z) of a normal z clamped to +-7 (the form the INT4 kernels
// feed the MFMA).
template <int FORM>
__global__ __launch_bounds__(256) void mfma_kernel(int iters, int* out, unsigned long long* clock) {
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  v4i a, b;
  for (int i = 0; i < 4; ++i) {
    uint32_t ra = mix(t * 8 + i), rb = mix(t * 8 + 4 + i);
    if (FORM == 0) ra = rb = 0;
    if (FORM == 2) {
      uint32_t wa = 0, wb = 0;
      for (int q = 0; q < 4; ++q) {
        const uint32_t h1 = mix(t * 64 + i * 8 + q), h2 = mix(t * 64 + i * 8 + q + 4);
        const float u1 = (h1 >> 8) * (1.0f / 16777216.0f) + 1e-7f, u2 = (h2 >> 8) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        const int c1 = (int)rintf(fminf(fmaxf(2.0f * r * cosf(6.2831853f * u2), -7.0f), 7.0f));
        const int c2 = (int)rintf(fminf(fmaxf(2.0f * r * sinf(6.2831853f * u2), -7.0f), 7.0f));
        wa |= ((uint32_t)(c1 * 16) & 0xffu) << (8 * q);
        wb |= ((uint32_t)(c2 * 16) & 0xffu) << (8 * q);
      }
      ra = wa;
      rb = wb;
    }
    a[i] = (int)ra;
    b[i] = (int)rb;
  }
  v16i acc[8];
  for (int j = 0; j < 8; ++j) acc[j] = v16i{};
  unsigned long long c0 = 0, r0 = 0;
  const bool timer = blockIdx.x == 0 && threadIdx.x < 64;
  if (timer) {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[j], 0, 0, 0);
  int s = 0;
  for (int j = 0; j < 8; ++j)
    for (int e = 0; e < 16; ++e) s ^= acc[j][e];
  if (s == 0x7fffffff) out[t] = s;  // keeps the MFMAs live; never true in practice
  if (timer && threadIdx.x == 0) {
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    clock[0] = c1 - c0;
    clock[1] = r1 - r0;
  }
}

// A gaussian int4 code: round(2z) of a normal z, clamped to +-7.
__device__ int gaussian_code(uint32_t seed) {
  const uint32_t h1 = mix(seed), h2 = mix(seed ^ 0x9e3779b9u);
  const float u1 = (h1 >> 8) * (1.0f / 16777216.0f) + 1e-7f, u2 = (h2 >> 8) * (1.0f / 16777216.0f);
  const float r = sqrtf(-2.0f * logf(u1));
  return (int)rintf(fminf(fmaxf(2.0f * r * cosf(6.2831853f * u2), -7.0f), 7.0f));
}

// e3m2 bits of an integer code -7..7.
__device__ uint32_t e3m2_code(int c) {
  const uint32_t mag[8] = {0x00, 0x0C, 0x10, 0x12, 0x14, 0x15, 0x16, 0x17};
  return c < 0 ? (mag[-c] | 0x20u) : mag[c];
}

// bf6 operand forms: 0 zeros; 1 the e3m2 codes of gaussian int4 codes, 32
// per lane in six words (value j at bits 6j).
template <int FORM>
__global__ __launch_bounds__(256) void mfma_f6_kernel(int iters, int* out, unsigned long long* clock) {
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;
  v8i a = v8i{}, b = v8i{};
  if (FORM == 1) {
    for (int j = 0; j < 32; ++j) {
      const uint32_t ea = e3m2_code(gaussian_code(t * 64 + j)), eb = e3m2_code(gaussian_code(t * 64 + 32 + j));
      const int bit = 6 * j, d = bit >> 5, sh = bit & 31;
      a[d] |= (int)(ea << sh);
      b[d] |= (int)(eb << sh);
      if (sh > 26) {
        a[d + 1] |= (int)(ea >> (32 - sh));
        b[d + 1] |= (int)(eb >> (32 - sh));
      }
    }
  }
  v16f acc[8];
  for (int j = 0; j < 8; ++j) acc[j] = v16f{};
  unsigned long long c0 = 0, r0 = 0;
  const bool timer = blockIdx.x == 0 && threadIdx.x < 64;
  if (timer) {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[j], 3, 3, 0, 127, 0, 127);
  float s = 0.0f;
  for (int j = 0; j < 8; ++j)
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  if (s == 12345.678f) out[t] = 1;  // keeps the MFMAs live; never true in practice
  if (timer && threadIdx.x == 0) {
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    clock[0] = c1 - c0;
    clock[1] = r1 - r0;
  }
}

__global__ void read_kernel(const u4* __restrict__ p, size_t n, u4* out) {
  u4 acc = {0, 0, 0, 0};
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) acc += p[i];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) out[0] = acc;
}
__global__ void write_kernel(u4* __restrict__ p, size_t n) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = u4{(unsigned)i, 1u, 2u, 3u};
}
__global__ void copy_kernel(const u4* __restrict__ s, u4* __restrict__ d, size_t n) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) d[i] = s[i];
}

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                \
      return 1;                                                                   \
    }                                                                             \
  } while (0)

}  // namespace

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  int* out;
  unsigned long long* clk;
  CHECK(hipMalloc(&out, (size_t)cus * 16 * 256 * sizeof(int)));
  CHECK(hipMalloc(&clk, 2 * sizeof(unsigned long long)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  const int blocks = cus * 4;  // 4 waves per SIMD
  const int iters = 40000;
  std::printf("{\"cus\": %d, \"mfma\": {", cus);
  const char* names[3] = {"zeros", "random_bytes", "int4_16x_gaussian_codes"};
  for (int f = 0; f < 3; ++f) {
    auto launch = [&](int it) {
      if (f == 0) mfma_kernel<0><<<blocks, 256>>>(it, out, clk);
      if (f == 1) mfma_kernel<1><<<blocks, 256>>>(it, out, clk);
      if (f == 2) mfma_kernel<2><<<blocks, 256>>>(it, out, clk);
    };
    for (int w = 0; w < 3; ++w) launch(iters);  // past the power-management transient
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0));
    launch(iters);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    unsigned long long c[2];
    CHECK(hipMemcpy(c, clk, sizeof(c), hipMemcpyDeviceToHost));
    const double ops = (double)blocks * 4 * iters * 8 * 32.0 * 32 * 32 * 2;
    const double mhz = c[1] ? (double)c[0] / (double)c[1] * 100.0 : 0.0;
    std::printf("%s\"%s\": {\"tops\": %.1f, \"pct_of_5000\": %.1f, \"sclk_mhz\": %.0f}", f ? ", " : "", names[f],
                ops / ms / 1e9, ops / ms / 1e9 / 50.0, mhz);
  }
  std::printf("}, \"mfma_bf6\": {");
  const char* names6[2] = {"zeros", "int4_gaussian_codes_as_e3m2"};
  for (int f = 0; f < 2; ++f) {
    const int it6 = iters / 2;
    auto launch = [&](int it) {
      if (f == 0) mfma_f6_kernel<0><<<blocks, 256>>>(it, out, clk);
      if (f == 1) mfma_f6_kernel<1><<<blocks, 256>>>(it, out, clk);
    };
    for (int w = 0; w < 3; ++w) launch(it6);
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0));
    launch(it6);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    unsigned long long c[2];
    CHECK(hipMemcpy(c, clk, sizeof(c), hipMemcpyDeviceToHost));
    const double ops = (double)blocks * 4 * it6 * 8 * 32.0 * 32 * 64 * 2;
    const double mhz = c[1] ? (double)c[0] / (double)c[1] * 100.0 : 0.0;
    std::printf("%s\"%s\": {\"tops\": %.1f, \"pct_of_10100\": %.1f, \"sclk_mhz\": %.0f}", f ? ", " : "",
                names6[f], ops / ms / 1e9, ops / ms / 1e9 / 101.0, mhz);
  }
  std::printf("}, \"hbm_gbs\": {");
  const size_t bytes = 1ull << 30, n = bytes / 16;
  u4 *a, *b, *o;
  CHECK(hipMalloc(&a, bytes));
  CHECK(hipMalloc(&b, bytes));
  CHECK(hipMalloc(&o, 64));
  CHECK(hipMemset(a, 1, bytes));
  CHECK(hipMemset(b, 2, bytes));
  const int grid = cus * 8;
  const char* hb[3] = {"read", "write", "copy"};
  for (int f = 0; f < 3; ++f) {
    auto launch = [&] {
      if (f == 0) read_kernel<<<grid, 256>>>(a, n, o);
      if (f == 1) write_kernel<<<grid, 256>>>(b, n);
      if (f == 2) copy_kernel<<<grid, 256>>>(a, b, n);
    };
    launch();
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0));
    for (int r = 0; r < 5; ++r) launch();
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double moved = (f == 2 ? 2.0 : 1.0) * (double)bytes;
    std::printf("%s\"%s\": %.1f", f ? ", " : "", hb[f], moved / (ms / 5) / 1e6);
  }
  std::printf("}}\n");
  CHECK(hipFree(a));
  CHECK(hipFree(b));
  CHECK(hipFree(o));
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  return 0;
}
