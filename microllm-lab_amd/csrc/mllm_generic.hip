// mllm_generic.hip -- the decode step for models whose matrices are not all
// Q4 group-32 (infer.js:313-346 binds each matrix by its own storage; the
// reference's GPU engine packs Q8, f16 and bf16 models as they are,
// webgpu.js:902-973, and runs them through the same step with a per-kind
// weight load, webgpu.js:141-260).
//
// One token per step, a few kernels per layer:
//   k_g_embed    the token's row of the tied lm_head in its storage
//                (infer.js:360-420: quantised rows de-scaled by gpt2's
//                scale_factors) + gpt2's learned position
//   k_g_gemv     norm (RMSNorm / LayerNorm) of the input row as a prologue,
//                then one wave per weight row: 8-column chunks of any
//                storage kind dotted with the staged row, the wave's sum,
//                and an epilogue: store (+ bias), residual add (+ bias),
//                SwiGLU over the w1 / w3 rows, or bias + GELU-tanh
//   k_g_attn     one workgroup per query head: rotate-half RoPE of its q
//                and of its KV group's new k (infer.js:208-225) in LDS, the
//                group's first head writes k / v to the KV cache (the
//                engine's layout); scores over the cache, the softmax of
//                infer.js:227-238, P.V (infer.js:466-495)
//   k_g_argmax   first maximum (infer.js:240-250), or argmaxGpt2
//                (infer.js:252-287) in gpt2 chains
// These matrices are read once per token, as by the Q4 engine, at the
// bytes their storage takes (f32 4, f16 / bf16 2, Q8 1 per weight).  A
// step's position and token come from a device cursor (GCursor) that the
// step's first kernel advances, so the host replays one captured graph per
// token.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "mllm_device.h"
#include "mllm_generic.h"
#include "mllm_host.h"

namespace mllm {
namespace {

constexpr int GHD = 64;   // head dimension
constexpr int GT = 256;   // threads per workgroup
constexpr int GAT = 1024;  // threads of the argmax workgroup
enum { G_STORE = 0, G_RESID = 1, G_SWIGLU = 2, G_GELU = 3 };
enum { GN_NONE = 0, GN_RMS = 1, GN_LN = 2 };

// Chained calls stop once an EOS was emitted.
__device__ __forceinline__ bool stopped(const GCursor *c) {
  return c && *reinterpret_cast<const volatile int *>(&c->done) != 0;
}

__device__ __forceinline__ float f16_bits(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }
__device__ __forceinline__ float bf16_bits(uint32_t h) { return __uint_as_float(h << 16); }

// Columns 8c .. 8c+7 of row r as floats (w) and the chunk's scale (Q8
// group-32 and Q4: the group's; 1 otherwise -- per-row Q8 scales the row's sum).
__device__ __forceinline__ float load8(const GMat &W, int r, int c, float (&w)[8]) {
  const size_t e0 = (size_t)r * W.cols + 8 * (size_t)c;
  switch (W.kind) {
  case MLLM_F32: {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(W.w) + e0);
    const float4 a = p[0], b = p[1];
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    return 1.f;
  }
  case MLLM_F16:
  case MLLM_BF16: {
    const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(W.w) + e0);
    const uint32_t p[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      w[2 * k] = W.kind == MLLM_F16 ? f16_bits(p[k] & 0xffffu) : bf16_bits(p[k] & 0xffffu);
      w[2 * k + 1] = W.kind == MLLM_F16 ? f16_bits(p[k] >> 16) : bf16_bits(p[k] >> 16);
    }
    return 1.f;
  }
  case MLLM_Q8:
  case MLLM_Q8G32: {
    const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const int8_t *>(W.w) + e0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      w[k] = (float)(int8_t)(u.x >> (8 * k));
      w[4 + k] = (float)(int8_t)(u.y >> (8 * k));
    }
    return W.kind == MLLM_Q8G32 ? W.s[(size_t)r * (W.cols >> 5) + (c >> 2)] : 1.f;
  }
  default: {  // MLLM_Q4: byte k holds element 2k (low nibble) and 2k + 1, stored as q + 8
    const uint32_t u = *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(W.w) + e0 / 2);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      w[2 * k] = (float)((int)((u >> (8 * k)) & 15u) - 8);
      w[2 * k + 1] = (float)((int)((u >> (8 * k + 4)) & 15u) - 8);
    }
    return W.s[(size_t)r * (W.cols / W.group) + (8 * c) / W.group];
  }
  }
}

__device__ __forceinline__ float dot8(const GMat &W, int r, int c, const float *xs) {
  float w[8];
  const float sc = load8(W, r, c, w);
  const float4 xa = *reinterpret_cast<const float4 *>(xs + 8 * c), xb = *reinterpret_cast<const float4 *>(xs + 8 * c + 4);
  float d = w[0] * xa.x;
  d = __builtin_fmaf(w[1], xa.y, d);
  d = __builtin_fmaf(w[2], xa.z, d);
  d = __builtin_fmaf(w[3], xa.w, d);
  d = __builtin_fmaf(w[4], xb.x, d);
  d = __builtin_fmaf(w[5], xb.y, d);
  d = __builtin_fmaf(w[6], xb.z, d);
  d = __builtin_fmaf(w[7], xb.w, d);
  return d * sc;
}

struct GemvArgs {
  GMat W, W3;          // W3: the up rows of G_SWIGLU
  const float *x;      // input row [W.cols]
  const float *gains;  // norm gains (LayerNorm: gamma || beta) or null
  float eps;           // RMSNorm eps (LayerNorm: 1e-5, infer.js:145)
  const float *bias;   // per output row, or null
  float *y;            // output row [W.rows]; G_RESID adds to it
  int rpw;             // rows per wave
  const GCursor *cur;
  int lm;              // 1: y is the logits, row cur->i when cur->rows (verify)
};

// Dynamic LDS: W.cols + 4 floats.
template <int EPI, int NORM>
__global__ __launch_bounds__(GT) void k_g_gemv(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  if (stopped(a.cur)) return;
  const int K = a.W.cols;
  float *y = a.y + (a.lm && a.cur->rows ? (size_t)a.cur->i * a.W.rows : 0);
  float *red = xs + K;
  if (NORM == GN_NONE) {
    for (int i = tid(); i < K; i += GT) xs[i] = a.x[i];
  } else {
    // infer.js:133-164 (sums in a fixed order: per thread, then the block tree)
    float s1 = 0.f;
    for (int i = tid(); i < K; i += GT) {
      const float v = a.x[i];
      s1 += NORM == GN_RMS ? v * v : v;
    }
    s1 = block_sum<GT>(s1, red);
    if (NORM == GN_RMS) {
      const float r = 1.0f / sqrtf(s1 / (float)K + a.eps);
      for (int i = tid(); i < K; i += GT) xs[i] = a.x[i] * r * a.gains[i];
    } else {
      const float mean = s1 / (float)K;
      float s2 = 0.f;
      for (int i = tid(); i < K; i += GT) {
        const float d = a.x[i] - mean;
        s2 += d * d;
      }
      s2 = block_sum<GT>(s2, red);
      const float r = 1.0f / sqrtf(s2 / (float)K + 1e-5f);
      for (int i = tid(); i < K; i += GT) xs[i] = (a.x[i] - mean) * r * a.gains[i] + a.gains[K + i];
    }
  }
  __syncthreads();
  const int lane = tid() & 63, wv = tid() >> 6, nc = K >> 3;
  const int r0 = (blockIdx.x * (GT / 64) + wv) * a.rpw;
  for (int k = 0; k < a.rpw; ++k) {
    const int r = r0 + k;
    if (r >= a.W.rows) break;  // uniform in the wave
    float acc = 0.f, acc3 = 0.f;
    for (int c = lane; c < nc; c += 64) {
      acc += dot8(a.W, r, c, xs);
      if (EPI == G_SWIGLU) acc3 += dot8(a.W3, r, c, xs);
    }
    acc = wave_sum(acc);
    if (EPI == G_SWIGLU) acc3 = wave_sum(acc3);
    if (lane != 0) continue;
    if (a.W.kind == MLLM_Q8) acc *= a.W.s[r];
    if (EPI == G_SWIGLU && a.W3.kind == MLLM_Q8) acc3 *= a.W3.s[r];
    if (EPI == G_STORE) {
      y[r] = a.bias ? acc + a.bias[r] : acc;
    } else if (EPI == G_RESID) {
      y[r] = y[r] + (a.bias ? acc + a.bias[r] : acc);
    } else if (EPI == G_SWIGLU) {
      y[r] = (acc / (1.0f + expf(-acc))) * acc3;  // infer.js:175-181
    } else {
      const float v = a.bias ? acc + a.bias[r] : acc;  // infer.js:166-172
      y[r] = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    }
  }
}

__device__ __forceinline__ size_t g_kv_index(const GArgs &A, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * A.NKV + h) * A.max_seq + pos) * GHD;
}

// The step's start: position and token index from the cursor (advanced for
// the next step), the input token (chained calls: the previous argmax),
// its embedding row.
__global__ __launch_bounds__(GT) void k_g_embed(GArgs A) {
  GCursor *cur = A.cur;
  if (stopped(cur)) return;
  const int D = A.D, pos = cur->pos_next, ti = cur->i_next;
  const int id = cur->chain ? cur->tok : A.ids[ti];
  __syncthreads();  // every thread has read the cursor
  if (tid() == 0) {
    cur->pos = pos;
    cur->i = ti;
    cur->pos_next = pos + 1;
    cur->i_next = ti + 1;
  }
  const GMat &W = A.lm;
  const bool quant = W.kind == MLLM_Q8 || W.kind == MLLM_Q8G32 || W.kind == MLLM_Q4;
  for (int c = tid(); c < (D >> 3); c += GT) {
    float w[8];
    const float sc = load8(W, id, c, w);
    const float rs = W.kind == MLLM_Q8 ? W.s[id] : sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * c + e;
      float v = quant ? w[e] * rs : w[e];
      if (A.arch == 1) {
        if (quant && A.sf) v = v / A.sf[i];
        v = v + A.wpe[(size_t)min(pos, A.max_seq - 1) * D + i];
      }
      A.x[i] = v;
    }
  }
}

__device__ __forceinline__ void kv_row(const GArgs &A, size_t off, float (&r)[GHD]) {
  if (A.kv_fp16) {
    const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const __half *>(A.kv) + off);
#pragma unroll
    for (int k = 0; k < GHD / 8; ++k) {
      const uint4 u = p[k];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[8 * k + 2 * e] = f16_bits(w[e] & 0xffffu);
        r[8 * k + 2 * e + 1] = f16_bits(w[e] >> 16);
      }
    }
  } else {
    const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(A.kv) + off);
#pragma unroll
    for (int k = 0; k < GHD / 4; ++k) {
      const float4 u = p[k];
      r[4 * k] = u.x, r[4 * k + 1] = u.y, r[4 * k + 2] = u.z, r[4 * k + 3] = u.w;
    }
  }
}

// One head's rotated component d (rotate-half on the first rope_dim
// components: out[d] = x[d] cos[d] + rot[d] sin[d], rot = (-x[half .. rd),
// x[0 .. half))).
__device__ __forceinline__ float rope_at(const GArgs &A, const float *hd, int d, int pos) {
  const int rd = A.rope_dim, half = rd >> 1;
  if (A.arch != 0 || d >= rd) return hd[d];
  const float c = A.rope_cos[(size_t)pos * rd + d], sn = A.rope_sin[(size_t)pos * rd + d];
  return d < half ? hd[d] * c + (-hd[d + half]) * sn : hd[d] * c + hd[d - half] * sn;
}

// Dynamic LDS: 3 x 64 (q, the new k and v) + max_seq (weights) + 256 (P.V
// partials) + 4 floats.  The new position's k and v are used from LDS (as
// the cache holds them: f16-rounded for an f16 cache), so the heads of a
// group do not wait for the one that writes them to the cache.
__global__ __launch_bounds__(GT) void k_g_attn(GArgs A, int li) {
  extern __shared__ __attribute__((aligned(16))) float sa[];
  if (stopped(A.cur)) return;
  const int pos = A.cur->pos, rep = A.NH / A.NKV;
  const int h = blockIdx.x, kvh = h / rep, n = pos + 1;
  float *qs = sa, *kn = sa + GHD, *vn = kn + GHD, *p = vn + GHD;
  float *part = p + ((A.max_seq + 3) & ~3), *red = part + GT;
  const size_t kb = g_kv_index(A, li, 0, kvh, 0), vb = g_kv_index(A, li, 1, kvh, 0);
  if (tid() < GHD) {
    const int d = tid();
    const float *k = A.qkv + A.D + kvh * GHD, *v = A.qkv + A.D + A.NKV * GHD + kvh * GHD;
    qs[d] = rope_at(A, A.qkv + h * GHD, d, pos);
    float kr = rope_at(A, k, d, pos), vr = v[d];
    if (A.kv_fp16) {
      const __half kh = __float2half_rn(kr), vh = __float2half_rn(vr);
      kr = __half2float(kh);
      vr = __half2float(vh);
      if (h % rep == 0) {
        reinterpret_cast<__half *>(A.kv)[kb + (size_t)pos * GHD + d] = kh;
        reinterpret_cast<__half *>(A.kv)[vb + (size_t)pos * GHD + d] = vh;
      }
    } else if (h % rep == 0) {
      reinterpret_cast<float *>(A.kv)[kb + (size_t)pos * GHD + d] = kr;
      reinterpret_cast<float *>(A.kv)[vb + (size_t)pos * GHD + d] = vr;
    }
    kn[d] = kr;
    vn[d] = vr;
  }
  __syncthreads();
  float mx = -INFINITY;
  for (int j = tid(); j < n; j += GT) {
    float kr[GHD];
    if (j == pos) {
#pragma unroll
      for (int e = 0; e < GHD; ++e) kr[e] = kn[e];
    } else {
      kv_row(A, kb + (size_t)j * GHD, kr);
    }
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < GHD; ++e) d = __builtin_fmaf(qs[e], kr[e], d);
    d *= A.attn_scale;
    p[j] = d;
    mx = fmaxf(mx, d);
  }
  mx = block_max<GT>(mx, red);
  float s = 0.f;
  for (int j = tid(); j < n; j += GT) {
    const float e = expf(p[j] - mx);
    p[j] = e;
    s += e;
  }
  s = block_sum<GT>(s, red);  // (its barriers also order the p[] writes before the reads below)
  const float inv = 1.0f / s;
  const int d = tid() & (GHD - 1), sl = tid() / GHD;
  float o = 0.f;
  for (int j = sl; j < n; j += GT / GHD) {
    const size_t off = vb + (size_t)j * GHD + d;
    const float vv = j == pos ? vn[d]
                              : (A.kv_fp16 ? __half2float(reinterpret_cast<const __half *>(A.kv)[off])
                                           : reinterpret_cast<const float *>(A.kv)[off]);
    o = __builtin_fmaf(p[j] * inv, vv, o);
  }
  part[tid()] = o;
  __syncthreads();
  if (tid() < GHD) A.att[h * GHD + tid()] = (part[tid()] + part[GHD + tid()]) + (part[2 * GHD + tid()] + part[3 * GHD + tid()]);
}

// First maximum of the step's logits row (infer.js:240-250: NaN never
// wins, and a NaN in slot 0 keeps index 0); in a gpt2 chain argmaxGpt2
// over the history (infer.js:252-287: trigram-banned ids -1e9, ids among
// the last 32 scaled by 1/1.15 or 1.15, then the first strict maximum from
// -inf).  Dynamic LDS: 2 + 32 + max_seq ints.
__global__ __launch_bounds__(GAT) void k_g_argmax(GArgs A) {
  extern __shared__ int lists[];
  GCursor *cur = A.cur;
  if (stopped(cur)) return;
  const int row = cur->rows ? cur->i : 0, chained = cur->chain;
  const float *lg = A.logits + (size_t)row * A.V;
  const bool rule = chained && cur->gpt2_rule;
  int *nb = lists, *nr = lists + 1, *rec = lists + 2, *ban = lists + 34;
  const int nh = chained ? cur->n_hist + cur->emitted : 0;
  const int *hist = A.hist;
  if (rule) {
    if (tid() == 0) {
      *nb = 0;
      int k = 0;
      for (int h = max(0, nh - 32); h < nh; ++h) rec[k++] = hist[h];
      *nr = k;
    }
    __syncthreads();
    if (nh >= 2) {
      const int t1 = hist[nh - 2], t2 = hist[nh - 1];
      for (int h = tid(); h < nh - 2; h += GAT)
        if (hist[h] == t1 && hist[h + 1] == t2) ban[atomicAdd(nb, 1)] = hist[h + 2];
    }
    __syncthreads();
  }
  const int nban = rule ? *nb : 0, nrec = rule ? *nr : 0;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid(); i < A.V; i += GAT) {
    float v = lg[i];
    if (rule) {
      for (int k = 0; k < nban; ++k)
        if (ban[k] == i) {
          v = -1e9f;
          break;
        }
      if (v > -1e8f)
        for (int k = 0; k < nrec; ++k)
          if (rec[k] == i) {
            v = v > 0.f ? v / 1.15f : v * 1.15f;
            break;
          }
    }
    // candidates: values above -inf (NaN and -inf never displace a maximum)
    if (v > -INFINITY && amax_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  wave_argmax(bv, bi);
  __shared__ float wv_v[GAT / 64];
  __shared__ int wv_i[GAT / 64];
  if ((tid() & 63) == 0) {
    wv_v[tid() >> 6] = bv;
    wv_i[tid() >> 6] = bi;
  }
  __syncthreads();
  if (tid() != 0) return;
  for (int w = 1; w < GAT / 64; ++w)
    if (amax_better(wv_v[w], wv_i[w], bv, bi)) {
      bv = wv_v[w];
      bi = wv_i[w];
    }
  int best = bi == 0x7fffffff ? 0 : bi;  // nothing above -inf: index 0 (both rules)
  if (!rule && isnan(lg[0])) best = 0;   // infer.js:241-243 starts from logits[0]
  A.res[row] = best;
  if (chained) {
    A.hist[nh] = best;
    cur->tok = best;
    cur->emitted = cur->emitted + 1;
    if (best == cur->eos) cur->done = 1;
  }
}

// Rows per wave: about 2048 workgroups for the largest matrices.
int g_rpw(int rows) { return std::max(1, (rows + 4 * 2048 - 1) / (4 * 2048)); }

template <int EPI, int NORM>
int launch_gemv(const GemvArgs &a, hipStream_t s) {
  const int rpw = g_rpw(a.W.rows);
  GemvArgs b = a;
  b.rpw = rpw;
  const int grid = (a.W.rows + 4 * rpw - 1) / (4 * rpw);
  const size_t lds = sizeof(float) * ((size_t)a.W.cols + 4);
  hipLaunchKernelGGL((k_g_gemv<EPI, NORM>), dim3(grid), dim3(GT), lds, s, b);
  return 0;
}

GemvArgs gemv_args(const GMat &W, const float *x, const float *gains, float eps, const float *bias, float *y,
                   const GCursor *cur) {
  GemvArgs a{};
  a.W = W;
  a.x = x;
  a.gains = gains;
  a.eps = eps;
  a.bias = bias;
  a.y = y;
  a.cur = cur;
  return a;
}

}  // namespace

bool g_kind_supported(int kind, int group) {
  switch (kind) {
  case MLLM_F32:
  case MLLM_F16:
  case MLLM_BF16:
  case MLLM_Q8: return true;
  case MLLM_Q8G32: return group == 32;
  case MLLM_Q4: return group >= 8 && group % 8 == 0;
  default: return false;
  }
}

int g_gemv(const GMat &W, const float *x, float *y, hipStream_t s) {
  MLLM_CHECK(g_kind_supported(W.kind, W.group) && W.cols % 8 == 0 && (W.kind != MLLM_Q4 || W.cols % W.group == 0),
             "matrix storage %d (group %d, %d columns) unsupported", W.kind, W.group, W.cols);
  MLLM_CHECK(W.cols <= 16000, "%d columns exceed the staged row", W.cols);
  launch_gemv<G_STORE, GN_NONE>(gemv_args(W, x, nullptr, 0.f, nullptr, y, nullptr), s);
  MLLM_HIP(hipGetLastError());
  return 0;
}

int g_step(const GArgs &A, bool lm, hipStream_t s) {
  const bool gpt2 = A.arch == 1;
  const GCursor *cur = A.cur;
  hipLaunchKernelGGL(k_g_embed, dim3(1), dim3(GT), 0, s, A);
  const size_t att_lds = sizeof(float) * (3 * GHD + ((A.max_seq + 3) & ~3) + GT + 4);
  for (int li = 0; li < A.L; ++li) {
    const GLayer &w = A.layers[li];
    if (!(w.dbg & 1)) {
      GemvArgs q = gemv_args(w.qkv, A.x, w.n1, A.eps, w.qkv_b, A.qkv, cur);
      if (gpt2)
        launch_gemv<G_STORE, GN_LN>(q, s);
      else
        launch_gemv<G_STORE, GN_RMS>(q, s);
      hipLaunchKernelGGL(k_g_attn, dim3(A.NH), dim3(GT), att_lds, s, A, li);
      launch_gemv<G_RESID, GN_NONE>(gemv_args(w.proj, A.att, nullptr, 0.f, w.proj_b, A.x, cur), s);
    }
    if (!(w.dbg & 2)) {
      if (gpt2) {
        launch_gemv<G_GELU, GN_LN>(gemv_args(w.w1, A.x, w.n2, A.eps, w.fc_b, A.h, cur), s);
      } else {
        GemvArgs u = gemv_args(w.w1, A.x, w.n2, A.eps, nullptr, A.h, cur);
        u.W3 = w.w3;
        launch_gemv<G_SWIGLU, GN_RMS>(u, s);
      }
      launch_gemv<G_RESID, GN_NONE>(gemv_args(w.w2, A.h, nullptr, 0.f, w.mproj_b, A.x, cur), s);
    }
  }
  if (lm) {
    GemvArgs f = gemv_args(A.lm, A.x, A.norm_f, A.eps, nullptr, A.logits, cur);
    f.lm = 1;
    if (gpt2)
      launch_gemv<G_STORE, GN_LN>(f, s);
    else
      launch_gemv<G_STORE, GN_RMS>(f, s);
    hipLaunchKernelGGL(k_g_argmax, dim3(1), dim3(GAT), sizeof(int) * (34 + (size_t)A.max_seq), s, A);
  }
  MLLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace mllm
