// mllm_ops.hip -- operator-level kernels and their C ABI (include/mllm.h).
//
// These replace the exports of engine/kernels.rs (gemv_f32, gemv_q8, gemv_q4,
// rms_norm, silu_mul, kernel_version) and the Q4 branch of
// engine/weights.js dequantizeToF32, plus the group-32 Q8 and batched Q4
// variants the benchmark needs.  All pointers are device pointers.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "mllm_device.h"
#include "mllm_host.h"

using namespace mllm;

// ---------------------------------------------------------------- errors
namespace mllm {
static thread_local std::string g_err = "no error";

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
  return set_error(e == hipErrorOutOfMemory ? MLLM_ERR_OOM : MLLM_ERR_HIP, "%s failed: %s (%s:%d)", what,
                   hipGetErrorString(e), file, line);
}

void clear_error() { g_err = "no error"; }
}  // namespace mllm

extern "C" const char *mllm_last_error(void) { return mllm::g_err.c_str(); }
extern "C" int mllm_kernel_version(void) { return 1; }

// ---------------------------------------------------------------- Q4 GEMV
// Tiles of rows_per_tile rows; each workgroup stages the m vectors once and
// walks tiles grid-stride.  y[t][rows] row-major.
__global__ __launch_bounds__(WG) void k_gemv_q4(Q4Mat W, const float *__restrict__ x, float *__restrict__ y,
                                                 int m, int rows_per_tile, int ntiles) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const int ng = W.cols >> 5;
  float *xs = smem;
  float *xsum = xs + m * ng * XS;
  float *part = xsum + m * ng;
  stage_plain(x, W.cols, m, W.cols, xs, xsum);
  const int gfirst = threadIdx.x % ng, gstep = WG % ng;
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int row0 = tile * rows_per_tile;
    const int nr = min(rows_per_tile, W.rows - row0);
    gemv_q4_rows(W, row0, nr, m, xs, xsum, ng, gfirst, gstep, part, y + row0, W.rows);
  }
}

// One launch over `count` same-shape matrices: blockIdx.y selects the matrix.
__global__ __launch_bounds__(WG) void k_gemv_q4_batched(const uint8_t *const *__restrict__ packed,
                                                         const float *const *__restrict__ scale,
                                                         const float *const *__restrict__ xv, float *const *__restrict__ yv,
                                                         int rows, int cols, int rows_per_tile, int ntiles) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const int b = blockIdx.y;
  Q4Mat W{reinterpret_cast<const uint4 *>(packed[b]), scale[b], rows, cols};
  const int ng = cols >> 5;
  float *xs = smem;
  float *xsum = xs + ng * XS;
  float *part = xsum + ng;
  stage_plain(xv[b], cols, 1, cols, xs, xsum);
  const int gfirst = threadIdx.x % ng, gstep = WG % ng;
  float *y = yv[b];
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int row0 = tile * rows_per_tile;
    gemv_q4_rows(W, row0, min(rows_per_tile, rows - row0), 1, xs, xsum, ng, gfirst, gstep, part, y + row0, rows);
  }
}

// ---------------------------------------------------------------- Q8 GEMV
// 16-byte chunk = 16 int8 weights.  per_row: one scale per row applied to the
// row sum (kernels.rs:41-57); otherwise one scale per 32 (two chunks).
__global__ __launch_bounds__(WG) void k_gemv_q8(const uint4 *__restrict__ q, const float *__restrict__ scale,
                                                 const float *__restrict__ x, float *__restrict__ y, int rows, int cols,
                                                 int per_row, int rows_per_tile, int ntiles) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const int ng = cols >> 5, nc = cols >> 4;  // groups of 32, chunks of 16
  float *xs = smem;
  float *xsum16 = xs + ng * XS;
  float *part = xsum16 + nc;
  stage_rows(x, cols, 1, cols, xs);
  __syncthreads();
  for (int c = threadIdx.x; c < nc; c += WG) {
    const float *p = xs + (c >> 1) * XS + (c & 1) * 16;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) s += p[k];
    xsum16[c] = s;
  }
  __syncthreads();
  const int tid = threadIdx.x;
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int row0 = tile * rows_per_tile;
    const int nr = min(rows_per_tile, rows - row0);
    const int nch = nr * nc;
    const size_t cbase = (size_t)row0 * nc;
    for (int c = tid; c < nch; c += WG) {
      const uint4 w = q[cbase + c];
      const int cc = c % nc;
      const float d = q8_chunk_dot(w, xs + (cc >> 1) * XS + (cc & 1) * 16) - 128.f * xsum16[cc];
      part[c] = per_row ? d : d * scale[(cbase + c) >> 1];
    }
    __syncthreads();
    for (int r = tid; r < nr; r += WG) {
      const float *p = part + r * nc;
      float acc = 0.f;
      for (int k = 0; k < nc; ++k) acc += p[k];
      y[row0 + r] = per_row ? acc * scale[row0 + r] : acc;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- f32 GEMV
// One wavefront per row, lanes over float4s, fixed-pattern wave reduction.
__global__ __launch_bounds__(WG) void k_gemv_f32(const float *__restrict__ w, const float *__restrict__ x,
                                                  float *__restrict__ y, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (WG / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *wr = w + (size_t)row * cols;
  float acc = 0.f;
  if ((cols & 3) == 0) {
    for (int k = lane * 4; k < cols; k += 256) {
      const float4 a = *reinterpret_cast<const float4 *>(wr + k);
      const float4 b = *reinterpret_cast<const float4 *>(x + k);
      acc = __builtin_fmaf(a.x, b.x, acc);
      acc = __builtin_fmaf(a.y, b.y, acc);
      acc = __builtin_fmaf(a.z, b.z, acc);
      acc = __builtin_fmaf(a.w, b.w, acc);
    }
  } else {
    for (int k = lane; k < cols; k += 64) acc = __builtin_fmaf(wr[k], x[k], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// ---------------------------------------------------------------- elementwise
__global__ __launch_bounds__(WG) void k_rms_norm(int n, const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ out, float eps) {
  __shared__ float red[4];
  const float *xo = x + (size_t)blockIdx.x * n;
  float *oo = out + (size_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += WG) ss = __builtin_fmaf(xo[i], xo[i], ss);
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += WG) oo[i] = xo[i] * inv * w[i];
}

__global__ __launch_bounds__(WG) void k_silu_mul(int n, float *__restrict__ a, const float *__restrict__ b) {
  const int i = blockIdx.x * WG + threadIdx.x;
  if (i < n) {
    const float v = a[i];
    a[i] = (v / (1.0f + expf(-v))) * b[i];
  }
}

// One thread per packed byte: two weights, each (nib - 8) * sc rounded once.
__global__ __launch_bounds__(WG) void k_dequant_q4(const uint8_t *__restrict__ packed, const float *__restrict__ scale,
                                                    float *__restrict__ out, size_t nbytes, int cols) {
  const size_t i = (size_t)blockIdx.x * WG + threadIdx.x;
  if (i >= nbytes) return;
  const int b = packed[i];
  const size_t e = 2 * i;
  const size_t row = e / cols;
  const int col = (int)(e - row * cols);
  const float sc = scale[row * (cols >> 5) + (col >> 5)];
  float2 v;
  v.x = (float)((b & 15) - 8) * sc;
  v.y = (float)((b >> 4) - 8) * sc;
  *reinterpret_cast<float2 *>(out + e) = v;
}

// ---------------------------------------------------------------- host side
namespace {

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

int device_wg_cap() {
  static int cap = 0;
  if (!cap) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                hipSuccess && cus > 0)
      cap = cus * 8;
    else
      cap = 2048;
  }
  return cap;
}

constexpr int kMaxCols = 16384;  // staged x must fit LDS: 144 B per 32 columns
constexpr int kMaxTok = 8;       // tokens per gemm launch

size_t q4_lds_bytes(int m, int ng) { return sizeof(float) * ((size_t)m * ng * XS + (size_t)m * ng + (size_t)m * SUB_CH); }

template <typename K>
int launch_dyn(K kernel, dim3 grid, size_t lds, hipStream_t st, const char *name) {
  if (lds > 64 * 1024) MLLM_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  (void)name;
  return 0;
}

int check_q4_shape(int m, int n, int group) {
  MLLM_CHECK(m > 0 && n > 0, "invalid shape m=%d n=%d", m, n);
  if (group != 32) return set_error(MLLM_ERR_UNSUPPORTED, "group %d unsupported (only 32)", group);
  MLLM_CHECK(n % 32 == 0, "n=%d not a multiple of 32", n);
  if (n > kMaxCols) return set_error(MLLM_ERR_UNSUPPORTED, "n=%d exceeds %d", n, kMaxCols);
  return 0;
}

int q4_gemm(int t, int m, int n, const uint8_t *packed, const float *scale, const float *x, float *y,
            hipStream_t st) {
  const int ng = n / 32;
  const int rpt = SUB_CH / ng > 0 ? SUB_CH / ng : 1;
  const int ntiles = (m + rpt - 1) / rpt;
  const int grid = ntiles < device_wg_cap() ? ntiles : device_wg_cap();
  Q4Mat W{reinterpret_cast<const uint4 *>(packed), scale, m, n};
  for (int t0 = 0; t0 < t; t0 += kMaxTok) {
    const int mt = t - t0 < kMaxTok ? t - t0 : kMaxTok;
    const size_t lds = q4_lds_bytes(mt, ng);
    if (int rc = launch_dyn(k_gemv_q4, grid, lds, st, "k_gemv_q4")) return rc;
    hipLaunchKernelGGL(k_gemv_q4, dim3(grid), dim3(WG), lds, st, W, x + (size_t)t0 * n, y + (size_t)t0 * m, mt, rpt,
                       ntiles);
    MLLM_HIP(hipGetLastError());
  }
  return 0;
}

}  // namespace

extern "C" int mllm_gemv_q4(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x,
                            float *y, void *stream) {
  if (int rc = check_q4_shape(m, n, group)) return rc;
  MLLM_CHECK(packed && scale && x && y, "null pointer");
  MLLM_CHECK((((uintptr_t)packed | (uintptr_t)x) & 15) == 0, "packed and x must be 16-byte aligned");
  return q4_gemm(1, m, n, packed, scale, x, y, as_stream(stream));
}

extern "C" int mllm_gemm_q4(int t, int m, int n, const uint8_t *packed, const float *scale, int group, const float *x,
                            float *y, void *stream) {
  if (int rc = check_q4_shape(m, n, group)) return rc;
  MLLM_CHECK(t > 0, "t=%d", t);
  MLLM_CHECK(packed && scale && x && y, "null pointer");
  MLLM_CHECK((((uintptr_t)packed | (uintptr_t)x) & 15) == 0, "packed and x must be 16-byte aligned");
  return q4_gemm(t, m, n, packed, scale, x, y, as_stream(stream));
}

extern "C" int mllm_gemv_q4_batched(int count, int m, int n, const uint8_t *const *packed, const float *const *scale,
                                    const float *const *x, float *const *y, void *stream) {
  if (int rc = check_q4_shape(m, n, 32)) return rc;
  MLLM_CHECK(count > 0 && count <= 65535, "count=%d", count);
  MLLM_CHECK(packed && scale && x && y, "null pointer");
  const int ng = n / 32;
  const int rpt = SUB_CH / ng > 0 ? SUB_CH / ng : 1;
  const int ntiles = (m + rpt - 1) / rpt;
  int gx = device_wg_cap() / count;
  if (gx < 1) gx = 1;
  if (gx > ntiles) gx = ntiles;
  const size_t lds = q4_lds_bytes(1, ng);
  hipStream_t st = as_stream(stream);
  if (int rc = launch_dyn(k_gemv_q4_batched, dim3(gx, count), lds, st, "k_gemv_q4_batched")) return rc;
  hipLaunchKernelGGL(k_gemv_q4_batched, dim3(gx, count), dim3(WG), lds, st, packed, scale, x, y, m, n, rpt, ntiles);
  MLLM_HIP(hipGetLastError());
  return 0;
}

static int q8_common(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, int per_row,
                     hipStream_t st) {
  MLLM_CHECK(m > 0 && n > 0 && n % 32 == 0, "invalid shape m=%d n=%d (n %% 32 == 0 required)", m, n);
  if (n > kMaxCols) return set_error(MLLM_ERR_UNSUPPORTED, "n=%d exceeds %d", n, kMaxCols);
  MLLM_CHECK(q && scale && x && y, "null pointer");
  MLLM_CHECK((((uintptr_t)q | (uintptr_t)x) & 15) == 0, "q and x must be 16-byte aligned");
  const int nc = n / 16, ng = n / 32;
  const int rpt = SUB_CH / nc > 0 ? SUB_CH / nc : 1;
  const int ntiles = (m + rpt - 1) / rpt;
  const int grid = ntiles < device_wg_cap() ? ntiles : device_wg_cap();
  const size_t lds = sizeof(float) * ((size_t)ng * XS + nc + (size_t)rpt * nc);
  if (int rc = launch_dyn(k_gemv_q8, grid, lds, st, "k_gemv_q8")) return rc;
  hipLaunchKernelGGL(k_gemv_q8, dim3(grid), dim3(WG), lds, st, reinterpret_cast<const uint4 *>(q), scale, x, y, m, n,
                     per_row, rpt, ntiles);
  MLLM_HIP(hipGetLastError());
  return 0;
}

extern "C" int mllm_gemv_q8(int m, int n, const int8_t *q, const float *scale, const float *x, float *y,
                            void *stream) {
  return q8_common(m, n, q, scale, x, y, 1, as_stream(stream));
}

extern "C" int mllm_gemv_q8_g32(int m, int n, const int8_t *q, const float *scale, const float *x, float *y,
                                void *stream) {
  return q8_common(m, n, q, scale, x, y, 0, as_stream(stream));
}

extern "C" int mllm_gemv_f32(int m, int n, const float *w, const float *x, float *y, void *stream) {
  MLLM_CHECK(m > 0 && n > 0, "invalid shape m=%d n=%d", m, n);
  MLLM_CHECK(w && x && y, "null pointer");
  MLLM_CHECK((n & 3) != 0 || (((uintptr_t)w | (uintptr_t)x) & 15) == 0, "w and x must be 16-byte aligned");
  const int rows_per_wg = WG / 64;
  hipLaunchKernelGGL(k_gemv_f32, dim3((m + rows_per_wg - 1) / rows_per_wg), dim3(WG), 0, as_stream(stream), w, x, y,
                     m, n);
  MLLM_HIP(hipGetLastError());
  return 0;
}

extern "C" int mllm_rms_norm(int n, const float *x, const float *w, float *out, int tokens, float eps, void *stream) {
  MLLM_CHECK(n > 0 && tokens > 0, "invalid shape n=%d tokens=%d", n, tokens);
  MLLM_CHECK(x && w && out, "null pointer");
  hipLaunchKernelGGL(k_rms_norm, dim3(tokens), dim3(WG), 0, as_stream(stream), n, x, w, out, eps);
  MLLM_HIP(hipGetLastError());
  return 0;
}

extern "C" int mllm_silu_mul(int n, float *a, const float *b, void *stream) {
  MLLM_CHECK(n > 0, "invalid n=%d", n);
  MLLM_CHECK(a && b, "null pointer");
  hipLaunchKernelGGL(k_silu_mul, dim3((n + WG - 1) / WG), dim3(WG), 0, as_stream(stream), n, a, b);
  MLLM_HIP(hipGetLastError());
  return 0;
}

extern "C" int mllm_dequant_q4(int m, int n, const uint8_t *packed, const float *scale, int group, float *out,
                               void *stream) {
  MLLM_CHECK(m > 0 && n > 0, "invalid shape m=%d n=%d", m, n);
  if (group != 32) return set_error(MLLM_ERR_UNSUPPORTED, "group %d unsupported (only 32)", group);
  MLLM_CHECK(n % 32 == 0, "n=%d not a multiple of 32", n);
  MLLM_CHECK(packed && scale && out, "null pointer");
  MLLM_CHECK(((uintptr_t)out & 7) == 0, "out must be 8-byte aligned");
  const size_t nbytes = (size_t)m * n / 2;
  hipLaunchKernelGGL(k_dequant_q4, dim3((unsigned)((nbytes + WG - 1) / WG)), dim3(WG), 0, as_stream(stream), packed,
                     scale, out, nbytes, n);
  MLLM_HIP(hipGetLastError());
  return 0;
}
