// mllm_ops.hip -- operator-level kernels and their C ABI (include/mllm.h).
//
// These replace the exports of engine/kernels.rs (gemv_f32, gemv_q8, gemv_q4,
// rms_norm, silu_mul, kernel_version) and the Q4 branch of
// engine/weights.js dequantizeToF32, plus the group-32 Q8 and batched Q4
// variants the benchmark needs.  All pointers are device pointers.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
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
// The activations are taken as Q6 records (24-bit integers per 32-element
// group, mllm_device.h): one v_dot8 per 8 weights and digit plane, exact in
// int32; a group adds (float)dot * sx * w_scale to its row.
//
// Work split (q4_gemv_tile): each row of a pass sits on one segment of L
// lanes, lane l taking groups l, l + L, ... (K of them), so a row's sum
// stays in registers (the lane's groups in order, then a DPP / swizzle tree
// over the segment), in an order that depends only on ng.
constexpr int GX_BATCH = 4;          // float4s of x per thread loaded ahead of the weights
// The Q4 weights are loaded with the non-temporal policy: every byte of a
// matrix is read once per launch, so its lines need not displace what the
// caches hold (x, the scales, the other launches' data).  Measured on the
// lm_head shape: 8.06 -> 7.78 us cold, 75% -> 83% of HBM peak when 32
// matrices share a launch.  The Q8 weights keep the default policy: with
// twice the bytes per group, the same change made the Q8 lm_head slower
// (10.9 -> 12.0 us cold).
constexpr int CP_NT = 2;             // cache-policy operand: non-temporal

// x through buffer loads, like the weights: vector-memory loads of one kind
// complete in issue order, so the staging waits for x alone (vmcnt) while the
// weights are in flight.  A load through a generic pointer is a flat load,
// which may complete out of order with them: the compiler then waits for every
// load in flight before the first use of x.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_rsrc(const float *x) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float4 x_ld4(__amdgpu_buffer_rsrc_t r, int q) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, q * 16, 0, 0));
}
// Called once the weights' loads are issued: from here on x is the value in
// these registers, so the compiler cannot load it again behind the weights
// (it would rather re-load x than keep it live across them, and the staging
// would then wait for every weight).
__device__ __forceinline__ void x_pin(float4 (&xv)[GX_BATCH]) {
#pragma unroll
  for (int i = 0; i < GX_BATCH; ++i) asm volatile("" : "+v"(xv[i].x), "+v"(xv[i].y), "+v"(xv[i].z), "+v"(xv[i].w));
}

// Sum over lpr (a power of two <= 64) neighbouring lanes; whole lpr-lane
// segments are active.
__device__ __forceinline__ float seg_sum(float a, int lpr) {
  if (lpr > 1) a += dpp_f<0xB1>(a);    // lane ^ 1
  if (lpr > 2) a += dpp_f<0x4E>(a);    // lane ^ 2
  if (lpr > 4) a += dpp_f<0x141>(a);   // mirror within 8
  if (lpr > 8) a += dpp_f<0x140>(a);   // mirror within 16
  if (lpr > 16) a += __shfl_xor(a, 16);
  if (lpr > 32) a += __shfl_xor(a, 32);
  return a;
}

struct GemvGeom {
  int rows, cols, m;  // matrix shape; tokens
  int rpp, lpr;       // rows per pass; lanes per row sum (power of two <= 64)
  int ystride;        // y[t * ystride + r]
};

// The first maximum of the rows this thread wrote (one token), for the
// argmax launches: (value, row) under amax_better, NaN rows left out, and
// whether row 0 is NaN.
struct RowMax {
  float v = -INFINITY;
  int i = 0x7fffffff;
  bool nan0 = false;
};

// One tile (P passes of rpp rows) of y = W x for m tokens.  Each row's
// groups sit in one segment of L = G.lpr lanes (a power of two <= 64, L >=
// ng / K): lane l of a segment takes groups l, l + L, ... (K of them), so a
// row's sum is formed in registers, lane partials first (in group order),
// then the DPP / swizzle tree over the segment, with no LDS pass and no
// barrier after the dots.  The order depends only on ng (L and K follow
// from it), so a row carries the same bits whatever the workgroup size, the
// passes per tile or the launch (single, batched, argmax).
template <int WGT, int P, int K, bool AMX = false>
__device__ __forceinline__ void q4_gemv_tile(const uint8_t *__restrict__ packed, const float *__restrict__ scale,
                                             const float *__restrict__ x, float *__restrict__ y, const GemvGeom &G,
                                             int tile, uint32_t *lds, RowMax *rm = nullptr) {
  const int ng = G.cols >> 5, nq = G.cols >> 2, nx = G.m * nq, L = G.lpr;
  const int RT = G.rpp * P;
  uint32_t *rec = lds;  // [m][ng][Q6R]
  const int t = threadIdx.x;
  const int rr = t / L, l = t - rr * L;
  const int row0 = tile * RT;
  // x ahead of the weights: loads retire in order, so the staging below
  // waits for x alone while the weights are in flight
  const __amdgpu_buffer_rsrc_t rx = x_rsrc(x);
  float4 xv[GX_BATCH];
#pragma unroll
  for (int i = 0; i < GX_BATCH; ++i) {
    const int q = t + i * WGT;
    xv[i] = x_ld4(rx, q < nx ? q : 0);
  }
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(packed), (short)0,
                                                                      0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scale), (short)0,
                                                                      0x7fffffff, 0x00020000);
  uint4 w[P * K];
  float s[P * K];
  const int last = G.rows - 1;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = min(row0 + p * G.rpp + rr, last);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const uint32_t c = (uint32_t)(row * ng + min(l + j * L, ng - 1));  // lanes past the row: a valid chunk, unused
      w[p * K + j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(c * 16), 0, CP_NT));
      s[p * K + j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(c * 4), 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);  // pass p's loads (weights, scales) before pass p + 1's
  }
  x_pin(xv);
#pragma unroll
  for (int i = 0; i < GX_BATCH; ++i)
    if (i * WGT < nx) q6_stage_col(xv[i], t + i * WGT < nx, t + i * WGT, rec);
  for (int base = GX_BATCH * WGT; base < nx; base += WGT) {
    const int q = base + t;
    q6_stage_col(x_ld4(rx, q < nx ? q : 0), q < nx, q, rec);
  }
  __syncthreads();
  const int nr = min(RT, G.rows - row0);
  for (int tok = 0; tok < G.m; ++tok) {
    // the lane's groups in order (group l + jL of every pass, one record in
    // registers at a time), then each pass's segment tree
    float acc[P];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const bool ok = l + j * L < ng;
      const Q6Rec xr = q6_load(rec + (tok * ng + min(l + j * L, ng - 1)) * Q6R);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const float d = q4_dot6(w[p * K + j], xr, s[p * K + j]);
        acc[p] = j == 0 ? (ok ? d : 0.f) : (ok ? acc[p] + d : acc[p]);
        if (K == 1) __builtin_amdgcn_sched_barrier(0);  // chunk by chunk: each dot waits only for its own loads
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const float a = seg_sum(acc[p], L);
      const int rl = p * G.rpp + rr;
      if (l == 0 && rl < nr) {
        y[tok * G.ystride + row0 + rl] = a;
        if (AMX) {
          const int row = row0 + rl;
          if (amax_better(a, row, rm->v, rm->i)) {  // false for a NaN row
            rm->v = a;
            rm->i = row;
          }
          if (row == 0) rm->nan0 = a != a;
        }
      }
    }
  }
}

template <int WGT, int P, int K>
__global__ __launch_bounds__(WGT) void k_gemv_q4(const uint8_t *__restrict__ packed, const float *__restrict__ scale,
                                                 const float *__restrict__ x, float *__restrict__ y, GemvGeom G) {
  extern __shared__ float4 smem4[];
  q4_gemv_tile<WGT, P, K>(packed, scale, x, y, G, blockIdx.x, reinterpret_cast<uint32_t *>(smem4));
}

// One launch over same-shape matrices: blockIdx.y selects the matrix.
template <int WGT, int P, int K>
__global__ __launch_bounds__(WGT) void k_gemv_q4_batched(const uint8_t *const *__restrict__ packed,
                                                         const float *const *__restrict__ scale,
                                                         const float *const *__restrict__ xv,
                                                         float *const *__restrict__ yv, GemvGeom G) {
  extern __shared__ float4 smem4[];
  const int b = blockIdx.y;
  q4_gemv_tile<WGT, P, K>(packed[b], scale[b], xv[b], yv[b], G, blockIdx.x, reinterpret_cast<uint32_t *>(smem4));
}

// y = W x (one token) and the first index of its maximum, in one launch
// (infer.js:597-600 + argmax, infer.js:240-250: best = 0, bestV = y[0], then
// every later row that is strictly larger; a NaN row never wins, and a NaN
// y[0] keeps index 0).  Each workgroup reduces its tile's rows to a (value,
// row) pair in the scratch buffer; the last workgroup to finish (a counter in
// the scratch) reduces the pairs and writes the index.  Scratch layout
// (bytes): [0, 4) the counter, which every completed launch leaves at 0;
// [4, 8) row 0 is NaN (tile 0 writes it); [64, 64 + 4 ntiles) the tiles'
// values, then ntiles rows.  Two launches that share a scratch buffer must
// not overlap.
constexpr size_t kAmxHead = 64;
__host__ __device__ constexpr size_t amx_scratch_bytes(int ntiles) { return kAmxHead + 8 * (size_t)ntiles; }

template <int WGT, int P, int K>
__global__ __launch_bounds__(WGT) void k_gemv_q4_argmax(const uint8_t *__restrict__ packed,
                                                        const float *__restrict__ scale, const float *__restrict__ x,
                                                        float *__restrict__ y, GemvGeom G, unsigned char *scratch,
                                                        int32_t *out) {
  extern __shared__ float4 smem4[];
  __shared__ float wv[WGT / 64];
  __shared__ int wi[WGT / 64], last;
  unsigned *cnt = reinterpret_cast<unsigned *>(scratch);
  int *nan0 = reinterpret_cast<int *>(scratch + 4);
  float *tv = reinterpret_cast<float *>(scratch + kAmxHead);
  int *ti = reinterpret_cast<int *>(scratch + kAmxHead + 4 * (size_t)gridDim.x);
  RowMax rm;
  q4_gemv_tile<WGT, P, K, true>(packed, scale, x, y, G, blockIdx.x, reinterpret_cast<uint32_t *>(smem4), &rm);
  const int t = threadIdx.x;
  float v = rm.v;
  int i = rm.i;
  wave_argmax(v, i);
  if ((t & 63) == 0) {
    wv[t >> 6] = v;
    wi[t >> 6] = i;
  }
  if (blockIdx.x == 0 && t == 0) coh_sti(nan0, 0, rm.nan0 ? 1 : 0);  // thread 0 of tile 0 summed row 0
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < WGT / 64; ++w)
      if (amax_better(wv[w], wi[w], v, i)) {
        v = wv[w];
        i = wi[w];
      }
    coh_stf(tv, 4u * blockIdx.x, v);
    coh_sti(ti, 4u * blockIdx.x, i);
    wait_stores();  // the pair (and nan0) are visible before the count is
    last = atomicAdd(cnt, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  v = -INFINITY;
  i = 0x7fffffff;
  for (int k = t; k < (int)gridDim.x; k += WGT) {
    const float kv = coh_ldf(tv, 4u * k);
    const int ki = coh_ldi(ti, 4u * k);
    if (amax_better(kv, ki, v, i)) {
      v = kv;
      i = ki;
    }
  }
  wave_argmax(v, i);
  __syncthreads();
  if ((t & 63) == 0) {
    wv[t >> 6] = v;
    wi[t >> 6] = i;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < WGT / 64; ++w)
      if (amax_better(wv[w], wi[w], v, i)) {
        v = wv[w];
        i = wi[w];
      }
    // every row NaN leaves i at INT_MAX; row 0 NaN wins in any case
    *out = coh_ldi(nan0, 0) || i == 0x7fffffff ? 0 : i;
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- Q8 GEMV (integer dots)
// The activations as 24-bit integers per 32-element group, xi = rint(x *
// Q3MAX / amax) with sx = amax / Q3MAX (the rounding of the Q4 path's Q6
// records, |xi| <= Q3MAX), split into three signed bytes, xi = 65536 h +
// 256 m + l (l, m the low bytes sign-extended; |xi| <= Q3MAX keeps h in
// [-128, 127]).  A group's record (Q6R dwords, as a Q6 record) holds the h,
// m and l planes at dwords 0-7, 8-15 and 16-23 (byte e of the plane is
// element e, the weights' byte order) and sx at dword 24.  One v_dot4 per
// 4 weights and plane, exact in int32 (a plane's sum is at most 32 * 127 *
// 128 in magnitude); the planes combine exactly in 64 bits (the group's dot
// reaches 32 * 127 * Q3MAX, past int32), converted to float once.  The
// group adds ((float)dot * sx) * w_scale to its row (g32), or the row sum is
// multiplied by the row's scale (kernels.rs:41-57).
constexpr float Q3MAX = 8355000.0f;

// A row staged by one thread per float4 column q (as q6_stage_col).
__device__ __forceinline__ void q3_stage_col(float4 y, bool in, int q, uint32_t *rec0) {
  if (!in) y = make_float4(0.f, 0.f, 0.f, 0.f);
  const float a = max8(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  const float inv = a > 0.f ? Q3MAX * __builtin_amdgcn_rcpf(a) : 0.f;
  const float v[4] = {y.x, y.y, y.z, y.w};
  uint32_t ph = 0, pm = 0, pl = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int xi = (int)__builtin_rintf(v[e] * inv);
    const int l = (int)(int8_t)(xi & 0xFF);
    const int r1 = (xi - l) >> 8;
    const int m = (int)(int8_t)(r1 & 0xFF);
    const int h = (r1 - m) >> 8;
    ph |= (uint32_t)(h & 0xFF) << (8 * e);
    pm |= (uint32_t)(m & 0xFF) << (8 * e);
    pl |= (uint32_t)(l & 0xFF) << (8 * e);
  }
  if (!in) return;
  uint32_t *rec = rec0 + (q >> 3) * Q6R;
  const int j = q & 7;  // elements 4j .. 4j+3 of the group: dword j of each plane
  rec[j] = ph;
  rec[8 + j] = pm;
  rec[16 + j] = pl;
  if (j == 0) rec[24] = __float_as_uint(a * (1.0f / Q3MAX));
}

// One group (32 int8 weights in wa, wb) against a Q3 record in registers.
__device__ __forceinline__ float q8_dot3(const uint4 wa, const uint4 wb, const Q6Rec &r, float ws) {
  const int wd[8] = {(int)wa.x, (int)wa.y, (int)wa.z, (int)wa.w, (int)wb.x, (int)wb.y, (int)wb.z, (int)wb.w};
  int H = 0, M = 0, L = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    H = __builtin_amdgcn_sdot4(wd[j], (int)r.d[j], H, false);
    M = __builtin_amdgcn_sdot4(wd[j], (int)r.d[8 + j], M, false);
    L = __builtin_amdgcn_sdot4(wd[j], (int)r.d[16 + j], L, false);
  }
  const long long dot = (long long)H * 65536 + (long long)M * 256 + (long long)L;
  return ((float)dot * r.sx) * ws;
}

// One tile of y = W x (one token) for Q8 weights, 32-byte chunks: thread t
// takes group t % ng of row t / ng of each pass, and the rows are summed from
// LDS partials (lane l of a row's lpr lanes adds float4s 4l, 4l + 4 lpr, ...,
// then a segment tree).
template <int WGT, int P, bool PERROW>
__device__ __forceinline__ void q8_gemv_tile(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                             const float *__restrict__ x, float *__restrict__ y, const GemvGeom &G,
                                             int tile, uint32_t *lds) {
  const int ng = G.cols >> 5, nq = G.cols >> 2, nx = nq;
  const int ngp = 4 * ((ng + 3) >> 2), RT = G.rpp * P;
  uint32_t *rec = lds;                                    // [ng][Q6R]
  float *part = reinterpret_cast<float *>(lds + ng * Q6R);  // [RT][ngp]
  const int t = threadIdx.x;
  const int rr0 = t / ng;
  const bool act = rr0 < G.rpp;
  const int rr = act ? rr0 : 0, g = act ? t - rr0 * ng : 0;
  const int row0 = tile * RT;
  const __amdgpu_buffer_rsrc_t rx = x_rsrc(x);
  float4 xv[GX_BATCH];
#pragma unroll
  for (int i = 0; i < GX_BATCH; ++i) {
    const int qq = t + i * WGT;
    xv[i] = x_ld4(rx, qq < nx ? qq : 0);
  }
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(q), (short)0, 0x7fffffff,
                                                                      0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scale), (short)0,
                                                                      0x7fffffff, 0x00020000);
  uint4 wa[P], wb[P];
  float s[P];
  const int last = G.rows - 1;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = min(row0 + p * G.rpp + rr, last);
    const uint32_t c = (uint32_t)(row * ng + g);
    wa[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(c * 32), 0, 0));
    wb[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(c * 32 + 16), 0, 0));
    s[p] = PERROW ? 1.f : __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(c * 4), 0, 0));
    __builtin_amdgcn_sched_barrier(0);  // chunk p's loads before chunk p + 1's
  }
  x_pin(xv);
#pragma unroll
  for (int i = 0; i < GX_BATCH; ++i)
    if (i * WGT < nx) q3_stage_col(xv[i], t + i * WGT < nx, t + i * WGT, rec);
  for (int base = GX_BATCH * WGT; base < nx; base += WGT) {
    const int qq = base + t;
    q3_stage_col(x_ld4(rx, qq < nx ? qq : 0), qq < nx, qq, rec);
  }
  __syncthreads();
  if (act) {
    const Q6Rec xr = q6_load(rec + g * Q6R);
    float *pp = part + rr * ngp + g;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      pp[p * G.rpp * ngp] = q8_dot3(wa[p], wb[p], xr, s[p]);  // chunk by chunk: each dot waits only for its own loads
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  // row sums
  const int nr = min(RT, G.rows - row0);
  for (int i = t; i < RT * G.lpr; i += WGT) {
    const int r = i / G.lpr, l = i - r * G.lpr;
    float a = 0.f;
    for (int gi = 4 * l; gi < ng; gi += 4 * G.lpr) {
      const float4 v = *reinterpret_cast<const float4 *>(part + r * ngp + gi);
      a += ((v.x + (gi + 1 < ng ? v.y : 0.f)) + ((gi + 2 < ng ? v.z : 0.f) + (gi + 3 < ng ? v.w : 0.f)));
    }
    a = seg_sum(a, G.lpr);
    if (l == 0 && r < nr) y[row0 + r] = PERROW ? a * scale[row0 + r] : a;
  }
}

template <int WGT, int P, bool PERROW>
__global__ __launch_bounds__(WGT) void k_gemv_q8i(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                  const float *__restrict__ x, float *__restrict__ y, GemvGeom G) {
  extern __shared__ float4 smem4[];
  q8_gemv_tile<WGT, P, PERROW>(q, scale, x, y, G, blockIdx.x, reinterpret_cast<uint32_t *>(smem4));
}

// One launch over same-shape Q8 matrices: blockIdx.y selects the matrix.
template <int WGT, int P, bool PERROW>
__global__ __launch_bounds__(WGT) void k_gemv_q8i_batched(const int8_t *const *__restrict__ q,
                                                          const float *const *__restrict__ scale,
                                                          const float *const *__restrict__ xv,
                                                          float *const *__restrict__ yv, GemvGeom G) {
  extern __shared__ float4 smem4[];
  const int b = blockIdx.y;
  q8_gemv_tile<WGT, P, PERROW>(q[b], scale[b], xv[b], yv[b], G, blockIdx.x, reinterpret_cast<uint32_t *>(smem4));
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

constexpr int kMaxCols = 16384;              // staged x must fit LDS
constexpr int kMaxTok = 8;                   // tokens per gemm launch
constexpr size_t kQ4LdsMax = 96 * 1024;      // LDS budget of one Q4 GEMV workgroup

struct Q4Plan {
  int wgt, rpp, lpr, ngp;
};
#ifndef MLLM_Q4_WG_PER_CU
#define MLLM_Q4_WG_PER_CU 4  // workgroups per CU that the tile plan aims for
#endif
long q4_target() { return (long)MLLM_Q4_WG_PER_CU * (device_wg_cap() / 8); }

// Geometry of the Q8 GEMV (q8_gemv_tile) for a shape and matrix count:
// workgroup size, rows per pass (one group per thread, a row's groups on
// neighbouring threads), lanes per row sum of the LDS partials.  256-thread
// workgroups up to 256 groups per row; 512 above that, and also for long rows
// (>= 64 groups) where even one-pass tiles of 256 threads leave the launch
// below its workgroup target: every workgroup stages all of x, and twice the
// rows share that staging.  The per-row arithmetic and its summation order do
// not depend on the workgroup size.
Q4Plan q4_plan(int cols, int rows, int count) {
  const int ng = cols / 32;
  Q4Plan p;
  p.wgt = ng <= 256 ? 256 : 512;
  if (p.wgt == 256 && ng >= 64 && (long)((rows + 256 / ng - 1) / (256 / ng)) * count < q4_target()) p.wgt = 512;
  p.rpp = p.wgt / ng;
  p.lpr = 1;
  while (p.lpr < 64 && p.lpr * 4 < ng) p.lpr <<= 1;
  p.ngp = 4 * ((ng + 3) / 4);
  return p;
}
size_t q4_lds_bytes(const Q4Plan &pl, int ng, int m, int P) {
  return sizeof(float) * ((size_t)m * ng * Q6R + (size_t)m * pl.rpp * P * pl.ngp);
}
// Passes per tile: the largest P in {8, 4, 2, 1} that still gives at least
// the target number of workgroups, so every load of a launch is in flight at
// once while the per-workgroup staging of x is spread over several passes.
int q4_pick_p(int rows, int rpp, int count) {
  const long target = q4_target();
  int P = 8;
  while (P > 1 && (long)((rows + rpp * P - 1) / (rpp * P)) * count < target) P >>= 1;
  return P;
}

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

template <int WGT, int P, int K>
int q4_launch_one(dim3 grid, size_t lds, hipStream_t st, const uint8_t *packed, const float *scale, const float *x,
                  float *y, const GemvGeom &G) {
  if (int rc = launch_dyn(k_gemv_q4<WGT, P, K>, grid, lds, st, "k_gemv_q4")) return rc;
  hipLaunchKernelGGL((k_gemv_q4<WGT, P, K>), grid, dim3(WGT), lds, st, packed, scale, x, y, G);
  MLLM_HIP(hipGetLastError());
  return 0;
}

template <int WGT, int P, int K>
int q4_launch_batched(dim3 grid, size_t lds, hipStream_t st, const uint8_t *const *packed, const float *const *scale,
                      const float *const *x, float *const *y, const GemvGeom &G) {
  if (int rc = launch_dyn(k_gemv_q4_batched<WGT, P, K>, grid, lds, st, "k_gemv_q4_batched")) return rc;
  hipLaunchKernelGGL((k_gemv_q4_batched<WGT, P, K>), grid, dim3(WGT), lds, st, packed, scale, x, y, G);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// Geometry of the Q4 GEMV (q4_gemv_tile): a row's ng groups on one segment
// of L lanes (a power of two), K <= 8 groups per lane, rpp = wgt / L rows per
// pass.  (L, K) wastes the fewest lane slots L K - ng; among equals, segments
// of at most 16 lanes (reduced by DPP alone) and then the longer segment.
// 256-thread workgroups, 512 for rows of 64 groups or more when the launch
// still has a workgroup per CU: every workgroup stages all of x, and twice
// the rows then share that staging (stacked 960 x 2560: 12.4 -> 11.5 us).  L
// and K follow from ng alone, so a row's summation order does not depend on
// the tile plan or the launch.
struct Q4SegPlan {
  int wgt, L, K, rpp;
};
Q4SegPlan q4_seg_plan(int cols, int rows, int count) {
  const int ng = cols / 32;
  Q4SegPlan p;
  p.L = 64;
  p.K = (ng + 63) / 64;  // ng <= 512: K <= 8
  for (const int L : {32, 1, 2, 4, 8, 16}) {  // later entries win ties
    const int K = (ng + L - 1) / L;
    if (K <= 8 && L * K - ng <= p.L * p.K - ng) {
      p.L = L;
      p.K = K;
    }
  }
  const long tiles512 = (long)((rows + 512 / p.L - 1) / (512 / p.L)) * count;
  p.wgt = ng >= 64 && tiles512 >= device_wg_cap() / 8 ? 512 : 256;
  p.rpp = p.wgt / p.L;
  return p;
}
// Passes per tile: the largest P in {8, 4, 2, 1} with at most 8 chunks per
// thread that still gives the launch its workgroup target: 2 per CU for one
// matrix, 8 per CU for a batched launch (measured, graph-replayed: stacked
// 960 x 2560 13.4 -> 11.5 us with 8 per CU instead of 4; one cold lm_head
// launch 7.8 -> 7.5 us with 2 per CU instead of 4: fewer, longer tiles, so
// fewer workgroups stage x).
int q4_seg_pick_p(const Q4SegPlan &pl, int rows, int count) {
  const long target = count > 1 ? 2L * q4_target() : q4_target() / 2;
  int P = 8;
  while (P > 1 && (P * pl.K > 8 || (long)((rows + pl.rpp * P - 1) / (pl.rpp * P)) * count < target)) P >>= 1;
  return P;
}
size_t q4_seg_lds(int ng, int m) { return sizeof(uint32_t) * (size_t)m * ng * Q6R; }

// Run F<WGT, P, K>(args...) for the runtime (wgt, P, K) of a Q4 plan (P * K <= 8).
#define MLLM_Q4K_PK(F, W, P, K, ...)                                                                       \
  ((K) == 1   ? ((P) == 8   ? F<W, 8, 1>(__VA_ARGS__)                                                       \
                 : (P) == 4 ? F<W, 4, 1>(__VA_ARGS__)                                                       \
                 : (P) == 2 ? F<W, 2, 1>(__VA_ARGS__)                                                       \
                            : F<W, 1, 1>(__VA_ARGS__))                                                      \
   : (K) == 2 ? ((P) == 4 ? F<W, 4, 2>(__VA_ARGS__) : (P) == 2 ? F<W, 2, 2>(__VA_ARGS__) : F<W, 1, 2>(__VA_ARGS__)) \
   : (K) == 3 ? ((P) == 2 ? F<W, 2, 3>(__VA_ARGS__) : F<W, 1, 3>(__VA_ARGS__))                              \
   : (K) == 4 ? ((P) == 2 ? F<W, 2, 4>(__VA_ARGS__) : F<W, 1, 4>(__VA_ARGS__))                              \
   : (K) == 5 ? F<W, 1, 5>(__VA_ARGS__)                                                                     \
   : (K) == 6 ? F<W, 1, 6>(__VA_ARGS__)                                                                     \
   : (K) == 7 ? F<W, 1, 7>(__VA_ARGS__)                                                                     \
              : F<W, 1, 8>(__VA_ARGS__))
#define MLLM_Q4K_DISPATCH(F, wgt, P, K, ...) \
  ((wgt) == 256 ? MLLM_Q4K_PK(F, 256, P, K, __VA_ARGS__) : MLLM_Q4K_PK(F, 512, P, K, __VA_ARGS__))

// Run F<WGT, P>(args...) for the runtime (wgt, P) of a plan.
#define MLLM_Q4_DISPATCH(F, wgt, P, ...)                                     \
  ((wgt) == 256 ? ((P) == 8 ? F<256, 8>(__VA_ARGS__)                         \
                   : (P) == 4 ? F<256, 4>(__VA_ARGS__)                       \
                   : (P) == 2 ? F<256, 2>(__VA_ARGS__)                       \
                              : F<256, 1>(__VA_ARGS__))                      \
                : ((P) == 8 ? F<512, 8>(__VA_ARGS__)                         \
                   : (P) == 4 ? F<512, 4>(__VA_ARGS__)                       \
                   : (P) == 2 ? F<512, 2>(__VA_ARGS__)                       \
                              : F<512, 1>(__VA_ARGS__)))

template <int WGT, int P, int K>
int q4_launch_argmax(dim3 grid, size_t lds, hipStream_t st, const uint8_t *packed, const float *scale, const float *x,
                     float *y, const GemvGeom &G, unsigned char *scratch, int32_t *out) {
  if (int rc = launch_dyn(k_gemv_q4_argmax<WGT, P, K>, grid, lds, st, "k_gemv_q4_argmax")) return rc;
  hipLaunchKernelGGL((k_gemv_q4_argmax<WGT, P, K>), grid, dim3(WGT), lds, st, packed, scale, x, y, G, scratch, out);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// The GEMV + argmax plan: the tiles of mllm_gemv_q4 for one token, so y is
// bit-identical to mllm_gemv_q4's.
struct AmxPlan {
  Q4SegPlan pl;
  int P, ntiles;
};
AmxPlan amx_plan(int m, int n) {
  AmxPlan a;
  a.pl = q4_seg_plan(n, m, 1);
  a.P = q4_seg_pick_p(a.pl, m, 1);
  a.ntiles = (m + a.pl.rpp * a.P - 1) / (a.pl.rpp * a.P);
  return a;
}

int gemv_q4_argmax_run(const AmxPlan &a, int m, int n, const uint8_t *packed, const float *scale, const float *x,
                       float *y, int32_t *out, unsigned char *scratch, hipStream_t st) {
  const GemvGeom G{m, n, 1, a.pl.rpp, a.pl.L, m};
  return MLLM_Q4K_DISPATCH(q4_launch_argmax, a.pl.wgt, a.P, a.pl.K, dim3(a.ntiles), q4_seg_lds(n / 32, 1), st, packed,
                           scale, x, y, G, scratch, out);
}

int check_argmax_args(int m, int n, int group, const uint8_t *packed, const float *scale, const float *x, float *y,
                      int32_t *argmax) {
  if (int rc = check_q4_shape(m, n, group)) return rc;
  MLLM_CHECK(packed && scale && x && y && argmax, "null pointer");
  MLLM_CHECK((((uintptr_t)packed | (uintptr_t)x) & 15) == 0, "packed and x must be 16-byte aligned");
  MLLM_CHECK((size_t)m * n / 2 < (1ull << 31), "matrix of %zu bytes exceeds 2 GiB", (size_t)m * n / 2);
  return 0;
}

// The library's argmax scratch, one buffer per device, allocated on the first
// call that needs it and grown (after the device is idle) when a call needs
// more; its counter is zeroed once at allocation.
constexpr int kMaxDevices = 64;
struct DevScratch {
  unsigned char *p = nullptr;
  size_t bytes = 0;
};
DevScratch g_amx_scratch[kMaxDevices];
std::mutex g_amx_mu;

int amx_scratch_for(int dev, size_t need, unsigned char **out) {
  std::lock_guard<std::mutex> lk(g_amx_mu);
  DevScratch &d = g_amx_scratch[dev];
  if (d.bytes < need) {
    if (d.p) {
      MLLM_HIP(hipDeviceSynchronize());
      MLLM_HIP(hipFree(d.p));
      d.p = nullptr;
      d.bytes = 0;
    }
    const size_t bytes = need < 65536 ? 65536 : need;
    MLLM_HIP(hipMalloc(reinterpret_cast<void **>(&d.p), bytes));
    MLLM_HIP(hipMemset(d.p, 0, bytes));
    d.bytes = bytes;
  }
  *out = d.p;
  return 0;
}

int q4_gemm(int t, int m, int n, const uint8_t *packed, const float *scale, const float *x, float *y,
            hipStream_t st) {
  MLLM_CHECK((size_t)m * n / 2 < (1ull << 31), "matrix of %zu bytes exceeds 2 GiB", (size_t)m * n / 2);
  const int ng = n / 32;
  const Q4SegPlan pl = q4_seg_plan(n, m, 1);
  const int P = q4_seg_pick_p(pl, m, 1);
  const int ntiles = (m + pl.rpp * P - 1) / (pl.rpp * P);
  for (int t0 = 0; t0 < t;) {
    int mt = t - t0 < kMaxTok ? t - t0 : kMaxTok;
    while (mt > 1 && q4_seg_lds(ng, mt) > kQ4LdsMax) --mt;
    const GemvGeom G{m, n, mt, pl.rpp, pl.L, m};
    if (int rc = MLLM_Q4K_DISPATCH(q4_launch_one, pl.wgt, P, pl.K, dim3(ntiles), q4_seg_lds(ng, mt), st, packed, scale,
                                   x + (size_t)t0 * n, y + (size_t)t0 * m, G))
      return rc;
    t0 += mt;
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
  MLLM_CHECK((size_t)m * n / 2 < (1ull << 31), "matrix of %zu bytes exceeds 2 GiB", (size_t)m * n / 2);
  const int ng = n / 32;
  const Q4SegPlan pl = q4_seg_plan(n, m, count);
  const int P = q4_seg_pick_p(pl, m, count);
  const int ntiles = (m + pl.rpp * P - 1) / (pl.rpp * P);
  const GemvGeom G{m, n, 1, pl.rpp, pl.L, m};
  return MLLM_Q4K_DISPATCH(q4_launch_batched, pl.wgt, P, pl.K, dim3(ntiles, count), q4_seg_lds(ng, 1), as_stream(stream),
                           packed, scale, x, y, G);
}

extern "C" int mllm_gemv_q4_argmax(int m, int n, const uint8_t *packed, const float *scale, int group,
                                   const float *x, float *y, int32_t *argmax, void *stream) {
  if (int rc = check_argmax_args(m, n, group, packed, scale, x, y, argmax)) return rc;
  int dev = 0;
  MLLM_HIP(hipGetDevice(&dev));
  MLLM_CHECK(dev >= 0 && dev < kMaxDevices, "device %d beyond %d", dev, kMaxDevices);
  const AmxPlan a = amx_plan(m, n);
  unsigned char *scratch = nullptr;
  if (int rc = amx_scratch_for(dev, amx_scratch_bytes(a.ntiles), &scratch)) return rc;
  return gemv_q4_argmax_run(a, m, n, packed, scale, x, y, argmax, scratch, as_stream(stream));
}

namespace mllm {
size_t gemv_q4_argmax_scratch(int m, int n) { return amx_scratch_bytes(amx_plan(m, n).ntiles); }

int gemv_q4_argmax_into(int m, int n, const uint8_t *packed, const float *scale, const float *x, float *y,
                        int32_t *argmax, unsigned char *scratch, hipStream_t st) {
  if (int rc = check_argmax_args(m, n, 32, packed, scale, x, y, argmax)) return rc;
  MLLM_CHECK(scratch != nullptr, "null argmax scratch");
  return gemv_q4_argmax_run(amx_plan(m, n), m, n, packed, scale, x, y, argmax, scratch, st);
}
}  // namespace mllm

// ---------------------------------------------------------------- no-allocation variant
// mllm_gemv_q4_argmax_noalloc keeps the argmax scratch in a file-scope device
// array of fixed size instead of memory the library allocates: every call on
// a device shares that device's copy, which keeps the last call's contents
// (the counter, which every completed call leaves at 0, is the only part read
// before it is written).  Calls that overlap on one device race.  In host code
// `scratch` names a host-side stand-in, not the device array: its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is passed to kernels.
constexpr size_t kNoallocScratchBytes = 128 * 1024;
constexpr int kNoallocMaxTiles = (int)((kNoallocScratchBytes - kAmxHead) / 8);
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
unsigned char *g_noalloc_ptr[kMaxDevices];
std::mutex g_noalloc_mu;

int noalloc_scratch(int dev, unsigned char **out) {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void *p = nullptr;
    MLLM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(MLLM_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
    g_noalloc_ptr[dev] = static_cast<unsigned char *>(p);
  }
  *out = g_noalloc_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int mllm_gemv_q4_argmax_noalloc(int m, int n, const uint8_t *packed, const float *scale, int group,
                                           const float *x, float *y, int32_t *argmax, void *stream) {
  if (int rc = check_argmax_args(m, n, group, packed, scale, x, y, argmax)) return rc;
  const AmxPlan a = amx_plan(m, n);
  if (a.ntiles > kNoallocMaxTiles)
    return set_error(MLLM_ERR_UNSUPPORTED,
                     "m=%d n=%d needs %d argmax tiles; the no-allocation scratch (%zu bytes) holds at most %d", m, n,
                     a.ntiles, kNoallocScratchBytes, kNoallocMaxTiles);
  int dev = 0;
  MLLM_HIP(hipGetDevice(&dev));
  MLLM_CHECK(dev >= 0 && dev < kMaxDevices, "device %d beyond %d", dev, kMaxDevices);
  unsigned char *sp = nullptr;
  if (int rc = noalloc_scratch(dev, &sp)) return rc;
  return gemv_q4_argmax_run(a, m, n, packed, scale, x, y, argmax, sp, as_stream(stream));
}

template <int WGT, int P>
int q8_launch(dim3 grid, size_t lds, hipStream_t st, const int8_t *q, const float *scale, const float *x, float *y,
              const GemvGeom &G, int per_row) {
  if (per_row) {
    if (int rc = launch_dyn(k_gemv_q8i<WGT, P, true>, grid, lds, st, "k_gemv_q8i")) return rc;
    hipLaunchKernelGGL((k_gemv_q8i<WGT, P, true>), grid, dim3(WGT), lds, st, q, scale, x, y, G);
  } else {
    if (int rc = launch_dyn(k_gemv_q8i<WGT, P, false>, grid, lds, st, "k_gemv_q8i")) return rc;
    hipLaunchKernelGGL((k_gemv_q8i<WGT, P, false>), grid, dim3(WGT), lds, st, q, scale, x, y, G);
  }
  MLLM_HIP(hipGetLastError());
  return 0;
}

template <int WGT, int P>
int q8_launch_batched(dim3 grid, size_t lds, hipStream_t st, const int8_t *const *q, const float *const *scale,
                      const float *const *x, float *const *y, const GemvGeom &G) {
  if (int rc = launch_dyn(k_gemv_q8i_batched<WGT, P, false>, grid, lds, st, "k_gemv_q8i_batched")) return rc;
  hipLaunchKernelGGL((k_gemv_q8i_batched<WGT, P, false>), grid, dim3(WGT), lds, st, q, scale, x, y, G);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// The Q8 GEMVs on integer dots, with the Q4 path's tile plan (the chunk of a
// (row, group) is 32 bytes instead of 16).
static int q8_common(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, int per_row,
                     hipStream_t st) {
  MLLM_CHECK(m > 0 && n > 0 && n % 32 == 0, "invalid shape m=%d n=%d (n %% 32 == 0 required)", m, n);
  if (n > kMaxCols) return set_error(MLLM_ERR_UNSUPPORTED, "n=%d exceeds %d", n, kMaxCols);
  MLLM_CHECK(q && scale && x && y, "null pointer");
  MLLM_CHECK((((uintptr_t)q | (uintptr_t)x) & 15) == 0, "q and x must be 16-byte aligned");
  MLLM_CHECK((size_t)m * n < (1ull << 31), "matrix of %zu bytes exceeds 2 GiB", (size_t)m * n);
  const int ng = n / 32;
  const Q4Plan pl = q4_plan(n, m, 1);
  const int P = q4_pick_p(m, pl.rpp, 1);
  const int ntiles = (m + pl.rpp * P - 1) / (pl.rpp * P);
  const GemvGeom G{m, n, 1, pl.rpp, pl.lpr, m};
  return MLLM_Q4_DISPATCH(q8_launch, pl.wgt, P, dim3(ntiles), q4_lds_bytes(pl, ng, 1, P), st, q, scale, x, y, G,
                          per_row);
}

extern "C" int mllm_gemv_q8(int m, int n, const int8_t *q, const float *scale, const float *x, float *y,
                            void *stream) {
  return q8_common(m, n, q, scale, x, y, 1, as_stream(stream));
}

extern "C" int mllm_gemv_q8_g32(int m, int n, const int8_t *q, const float *scale, const float *x, float *y,
                                void *stream) {
  return q8_common(m, n, q, scale, x, y, 0, as_stream(stream));
}

extern "C" int mllm_gemv_q8_g32_batched(int count, int m, int n, const int8_t *const *q, const float *const *scale,
                                        const float *const *x, float *const *y, void *stream) {
  MLLM_CHECK(m > 0 && n > 0 && n % 32 == 0, "invalid shape m=%d n=%d (n %% 32 == 0 required)", m, n);
  if (n > kMaxCols) return set_error(MLLM_ERR_UNSUPPORTED, "n=%d exceeds %d", n, kMaxCols);
  MLLM_CHECK(count > 0 && count <= 65535, "count=%d", count);
  MLLM_CHECK(q && scale && x && y, "null pointer");
  MLLM_CHECK((size_t)m * n < (1ull << 31), "matrix of %zu bytes exceeds 2 GiB", (size_t)m * n);
  // the tile plan chosen for the whole batch; a row's sum depends only on
  // its group count (lpr), so each matrix's rows come out as mllm_gemv_q8_g32's
  const int ng = n / 32;
  const Q4Plan pl = q4_plan(n, m, count);
  const int P = q4_pick_p(m, pl.rpp, count);
  const int ntiles = (m + pl.rpp * P - 1) / (pl.rpp * P);
  const GemvGeom G{m, n, 1, pl.rpp, pl.lpr, m};
  return MLLM_Q4_DISPATCH(q8_launch_batched, pl.wgt, P, dim3(ntiles, count), q4_lds_bytes(pl, ng, 1, P),
                          as_stream(stream), q, scale, x, y, G);
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
