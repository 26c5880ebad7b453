// mllm_prefill.hip -- batched prompt processing for forwardPrompt
// (infer.js:553-577): a chunk of T prompt tokens goes through every layer as
// a handful of wide kernels instead of 16-token passes of the decode phases.
//
// Q4 GEMMs on int8 matrix cores.  Activations are quantised per token to
// 16-bit integers, xi = rint(x * 32639 / amax) (amax = max |x| of the
// token's row; sx = amax / 32639), and split into two signed bytes,
// xi = 256 * hi + lo with lo = the low byte sign-extended (|xi| <= 32639
// keeps hi within [-127, 127]).  With the weights as signed nibbles q - 8 the
// group's dot product is exact in int32:
//   sum_k (q_k - 8) xi_k = 256 * sum_k (q_k - 8) hi_k + sum_k (q_k - 8) lo_k,
// two v_mfma_i32_32x32x32_i8 per 32-row x 32-token x 32-column group (K =
// 32 = one Q4 group).  The group's float contribution is added as
//   acc = fma((float)dot, w_scale, acc)
// in group order, and the row is multiplied by sx at the end.  The VALU
// epilogue (three operations per output and group) bounds these GEMMs, not
// the matrix cores.
//
// Operand layouts (v_mfma_i32_32x32x32_i8, checked on gfx950): A (the
// activations) lane l holds row l % 32 (a token), 16 bytes of k; B (the
// weights) lane l holds column l % 32 (a weight row), the same 16 k; D lane l
// value v is (row 8(v/4) + 4(l/32) + v%4, column l % 32).  Only the pairing of
// A's and B's k matters, so lane half hh = l / 32 takes the group's elements
// 16hh .. 16hh+15 in the order its weight bytes unpack: the low nibbles of
// packed bytes 8hh .. 8hh+3 (elements 0, 2, 4, 6), of bytes 8hh+4 .. 8hh+7
// (elements 8 .. 14), then the high nibbles of each (elements 1 .. 7 and
// 9 .. 15, odd).  The activation planes are stored in that order, 64 bytes
// per (token, group): hi of half 0, hi of half 1, lo of half 0, lo of half 1.
//
// Attention: causal, f32, one (64-query block, query head) per workgroup,
// 64-key blocks staged in LDS with an online softmax (running max and sum,
// rescaled per block); the softmax of infer.js:422-504 without the decode
// path's single pass.
//
// Per layer: norm + quantise, QKV GEMM (bias or RoPE, K/V to the cache, q to
// a buffer), attention, quantise, O GEMM (+ residual), norm + quantise,
// gate/up GEMM (SwiGLU; gpt2 fc + GELU), quantise, down GEMM (+ residual).
// The last layer stops after its QKV GEMM: only its K and V are needed.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>

#include "mllm_device.h"
#include "mllm_host.h"
#include "mllm_prefill.h"

namespace mllm {
namespace {

constexpr int PX_MAX = 32639;   // |xi| bound of the 16-bit activations
constexpr int PX_GROUP = 64;    // bytes per (token, group) of the planes
constexpr int PF_HD = 64;       // head dimension
constexpr int AQ = 64, AK = 64; // attention query and key block
constexpr int KS = 68;          // LDS row stride (floats) of the key / weight tiles

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum { EPI_QKV = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_GELU = 3 };
enum { NORM_RMS = 0, NORM_LN = 1, NORM_NONE = 2 };

__device__ __forceinline__ size_t pf_kv_index(const PfArgs &A, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * A.NKV + h) * A.max_seq + pos) * PF_HD;
}

// ---------------------------------------------------------------- embedding
// Token t's row of the tied lm_head, dequantised (infer.js:360-393); gpt2
// divides by scale_factors (when present) and adds the learned position.
__global__ __launch_bounds__(WG) void k_pf_embed(PfArgs A, int n, int pos0) {
  const int t = blockIdx.x, D = A.D, ng = D >> 5;
  const int tok = A.ids[t];
  const int pos = min(pos0 + t, A.max_seq - 1);
  const uint8_t *row = A.emb.q + (size_t)tok * (D >> 1);
  for (int q = threadIdx.x; q < (D >> 2); q += WG) {
    const unsigned short b2 = *reinterpret_cast<const unsigned short *>(row + 2 * q);
    const float s = A.emb.s[(size_t)tok * ng + (q >> 3)];
    float4 e = make_float4((float)((int)(b2 & 15) - 8) * s, (float)((int)((b2 >> 4) & 15) - 8) * s,
                           (float)((int)((b2 >> 8) & 15) - 8) * s, (float)((int)(b2 >> 12) - 8) * s);
    if (A.arch == 1) {
      if (A.sf) {
        const float4 f = reinterpret_cast<const float4 *>(A.sf)[q];
        e = make_float4(e.x / f.x, e.y / f.y, e.z / f.z, e.w / f.w);
      }
      const float4 w = reinterpret_cast<const float4 *>(A.wpe + (size_t)pos * D)[q];
      e = make_float4(e.x + w.x, e.y + w.y, e.z + w.z, e.w + w.w);
    }
    reinterpret_cast<float4 *>(A.x + (size_t)t * D)[q] = e;
  }
}

// ---------------------------------------------------------------- norm + quantise
// One token row of K floats per workgroup: optional RMSNorm / LayerNorm
// (the decode engine's formulas), then the 16-bit planes and the scale.
template <int NORM>
__global__ __launch_bounds__(WG) void k_pf_quant(const float *src, int K, const float *g, float eps, uint8_t *px,
                                                 float *sx) {
  extern __shared__ float ys[];  // K floats
  __shared__ float red[WG / 64];
  const int t = blockIdx.x, nq = K >> 2, ng = K >> 5;
  const float4 *xr = reinterpret_cast<const float4 *>(src + (size_t)t * K);
  float4 *y4 = reinterpret_cast<float4 *>(ys);
  const float inv_k = 1.0f / (float)K;
  float s1 = 0.f;
  for (int q = tid(); q < nq; q += WG) {
    const float4 v = xr[q];
    y4[q] = v;
    if (NORM == NORM_RMS) s1 += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    if (NORM == NORM_LN) s1 += (v.x + v.y) + (v.z + v.w);
  }
  if (NORM == NORM_RMS) {
    const float r = __builtin_amdgcn_rsqf(block_sum<WG>(s1, red) * inv_k + eps);
    const float4 *g4 = reinterpret_cast<const float4 *>(g);
    for (int q = tid(); q < nq; q += WG) {
      const float4 v = y4[q], w = g4[q];
      y4[q] = make_float4(v.x * r * w.x, v.y * r * w.y, v.z * r * w.z, v.w * r * w.w);
    }
  } else if (NORM == NORM_LN) {
    const float mean = block_sum<WG>(s1, red) * inv_k;
    float s2 = 0.f;
    for (int q = tid(); q < nq; q += WG) {
      const float4 v = y4[q];
      const float4 d = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
      s2 += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
    }
    const float r = __builtin_amdgcn_rsqf(block_sum<WG>(s2, red) * inv_k + 1e-5f);
    const float4 *g4 = reinterpret_cast<const float4 *>(g);
    for (int q = tid(); q < nq; q += WG) {
      const float4 v = y4[q], w = g4[q], b = g4[nq + q];
      const float4 d = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
      y4[q] = make_float4(__builtin_fmaf(d.x * r, w.x, b.x), __builtin_fmaf(d.y * r, w.y, b.y),
                          __builtin_fmaf(d.z * r, w.z, b.z), __builtin_fmaf(d.w * r, w.w, b.w));
    }
  }
  float am = 0.f;
  for (int q = tid(); q < nq; q += WG) {
    const float4 v = y4[q];
    am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  am = block_max<WG>(am, red);  // its barriers also order the y4 stores above
  const float inv = am > 0.f ? (float)PX_MAX / am : 0.f;
  if (tid() == 0) sx[t] = am / (float)PX_MAX;
  uint8_t *rowp = px + (size_t)t * ng * PX_GROUP;
  for (int q = tid(); q < nq; q += WG) {
    const float4 v = y4[q];
    const int x0 = (int)__builtin_rintf(v.x * inv), x1 = (int)__builtin_rintf(v.y * inv);
    const int x2 = (int)__builtin_rintf(v.z * inv), x3 = (int)__builtin_rintf(v.w * inv);
    // signed split: lo = low byte sign-extended, hi = (x - lo) / 256
    const int l0 = (int)(signed char)(x0 & 255), l1 = (int)(signed char)(x1 & 255);
    const int l2 = (int)(signed char)(x2 & 255), l3 = (int)(signed char)(x3 & 255);
    const int h0 = (x0 - l0) >> 8, h1 = (x1 - l1) >> 8, h2 = (x2 - l2) >> 8, h3 = (x3 - l3) >> 8;
    // elements e0 .. e0+3 of group q/8: half e0/16; even elements at bytes
    // p, p+1 of the half, odd ones at p+8, p+9
    const int e0 = 4 * (q & 7), hh = e0 >> 4, kk = e0 & 15;
    const int p = (kk >> 3) * 4 + ((kk & 7) >> 1);
    uint8_t *rec = rowp + (q >> 3) * PX_GROUP + 16 * hh;
    *reinterpret_cast<unsigned short *>(rec + p) = (unsigned short)((h0 & 255) | ((h2 & 255) << 8));
    *reinterpret_cast<unsigned short *>(rec + 8 + p) = (unsigned short)((h1 & 255) | ((h3 & 255) << 8));
    *reinterpret_cast<unsigned short *>(rec + 32 + p) = (unsigned short)((l0 & 255) | ((l2 & 255) << 8));
    *reinterpret_cast<unsigned short *>(rec + 40 + p) = (unsigned short)((l1 & 255) | ((l3 & 255) << 8));
  }
}

// ---------------------------------------------------------------- Q4 GEMM
// A wave computes two 32-row sub-tiles (sub-tile 1 is either the next 32
// rows of the same matrix -- a 64-row head of attn.qkv, 64 rows of the
// others -- or the same rows of a second matrix: mlp.w3 beside mlp.w1) for
// 32 tokens.  Workgroup: 4 waves on consecutive row ranges, one token tile.
struct PfGemm {
  const uint8_t *q0, *q1;
  const float *s0, *s1;
  int rows;   // rows of each matrix
  int off1;   // row offset of sub-tile 1 in its matrix (32 or 0)
  int rstep;  // rows per wave (64 or 32)
  int ng;     // groups per row
  int n;      // tokens
  int li, pos0;
  const float *bias0, *bias1;  // per row of each matrix, or null
  float *out;                  // EPI_RESID: the residual rows; SWIGLU/GELU: the MLP activation
  int ldo;
};

__device__ __forceinline__ v4i pf_unpack(uint2 w) {
  // nibble q -> signed byte q - 8: (q + 0x78) ^ 0x80, no carry between bytes
  const uint32_t e0 = w.x & 0x0F0F0F0Fu, e1 = w.y & 0x0F0F0F0Fu;
  const uint32_t o0 = (w.x >> 4) & 0x0F0F0F0Fu, o1 = (w.y >> 4) & 0x0F0F0F0Fu;
  v4i r;
  r.x = (int)((e0 + 0x78787878u) ^ 0x80808080u);
  r.y = (int)((e1 + 0x78787878u) ^ 0x80808080u);
  r.z = (int)((o0 + 0x78787878u) ^ 0x80808080u);
  r.w = (int)((o1 + 0x78787878u) ^ 0x80808080u);
  return r;
}

struct GemmLd {
  uint2 w0, w1;
  float c0, c1;
  v4i ah, al;
};

template <int EPI>
__global__ __launch_bounds__(WG) void k_pf_gemm(PfArgs A, PfGemm G) {
  const int wv = tid() >> 6, lane = tid() & 63, j = lane & 31, hh = lane >> 5;
  const int R = (blockIdx.x * (WG / 64) + wv) * G.rstep;
  if (R >= G.rows) return;  // no barriers below
  const int T0 = blockIdx.y * 32;
  const int ng = G.ng;
  const int ra = min(R + j, G.rows - 1), rb = min(R + G.off1 + j, G.rows - 1);
  const uint8_t *wa = G.q0 + (size_t)ra * ng * 16 + 8 * hh;
  const uint8_t *wb = G.q1 + (size_t)rb * ng * 16 + 8 * hh;
  const float *sa = G.s0 + (size_t)ra * ng, *sb = G.s1 + (size_t)rb * ng;
  const uint8_t *xa = A.px + (size_t)min(T0 + j, G.n - 1) * ng * PX_GROUP + 16 * hh;
  auto load = [&](int g) {
    GemmLd L;
    L.w0 = *reinterpret_cast<const uint2 *>(wa + 16 * g);
    L.w1 = *reinterpret_cast<const uint2 *>(wb + 16 * g);
    L.c0 = sa[g];
    L.c1 = sb[g];
    L.ah = *reinterpret_cast<const v4i *>(xa + PX_GROUP * g);
    L.al = *reinterpret_cast<const v4i *>(xa + PX_GROUP * g + 32);
    return L;
  };
  float acc0[16], acc1[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.f;
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  GemmLd cur = load(0);
  for (int g = 0; g < ng; ++g) {
    const GemmLd nxt = load(min(g + 1, ng - 1));
    const v4i b0 = pf_unpack(cur.w0), b1 = pf_unpack(cur.w1);
    const v16i h0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.ah, b0, zero, 0, 0, 0);
    const v16i l0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.al, b0, zero, 0, 0, 0);
    const v16i h1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.ah, b1, zero, 0, 0, 0);
    const v16i l1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.al, b1, zero, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc0[v] = __builtin_fmaf((float)(h0[v] * 256 + l0[v]), cur.c0, acc0[v]);
      acc1[v] = __builtin_fmaf((float)(h1[v] * 256 + l1[v]), cur.c1, acc1[v]);
    }
    cur = nxt;
  }
  // epilogue: value v is token T0 + 8(v/4) + 4hh + v%4, rows ra / rb
  const int r0 = R + j, r1 = R + G.off1 + j;
  const bool in0 = r0 < G.rows, in1 = r1 < G.rows;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int t = T0 + 8 * (v >> 2) + 4 * hh + (v & 3);
    if (t >= G.n) continue;
    const float s = A.sx[t];
    float y0 = acc0[v] * s, y1 = acc1[v] * s;
    if (EPI == EPI_QKV) {
      // rows R .. R+63 are one head: query head, K head or V head
      const int head = R >> 6, pos = G.pos0 + t;
      if (G.bias0) {
        y0 = y0 + G.bias0[r0];
        y1 = y1 + G.bias0[r1];
      } else if (head < A.NH + A.NKV) {
        // rotate-half RoPE: d = j pairs with d + 32 (infer.js:208-225)
        const float *cs = A.rope_cos + (size_t)pos * PF_HD, *sn = A.rope_sin + (size_t)pos * PF_HD;
        const float a = y0, b = y1;
        y0 = __builtin_fmaf(a, cs[j], (-b) * sn[j]);
        y1 = __builtin_fmaf(b, cs[32 + j], a * sn[32 + j]);
      }
      if (head < A.NH) {
        float *qd = A.q + (size_t)t * A.D + head * PF_HD;
        qd[j] = y0;
        qd[32 + j] = y1;
      } else {
        const bool is_k = head < A.NH + A.NKV;
        const int kvh = is_k ? head - A.NH : head - A.NH - A.NKV;
        const size_t k = pf_kv_index(A, G.li, is_k ? 0 : 1, kvh, pos);
        if (A.kv_fp16) {
          __half *kv = reinterpret_cast<__half *>(A.kv) + k;
          kv[j] = __float2half_rn(y0);
          kv[32 + j] = __float2half_rn(y1);
        } else {
          float *kv = reinterpret_cast<float *>(A.kv) + k;
          kv[j] = y0;
          kv[32 + j] = y1;
        }
      }
    } else if (EPI == EPI_RESID) {
      float *xr = G.out + (size_t)t * G.ldo;
      if (in0) xr[r0] = xr[r0] + (G.bias0 ? y0 + G.bias0[r0] : y0);
      if (in1) xr[r1] = xr[r1] + (G.bias0 ? y1 + G.bias0[r1] : y1);
    } else if (EPI == EPI_SWIGLU) {
      // sub-tile 0: gate rows, sub-tile 1: the same units' up rows
      if (in0) G.out[(size_t)t * G.ldo + r0] = (y0 / (1.0f + expf(-y0))) * y1;
    } else {  // EPI_GELU
      float *hr = G.out + (size_t)t * G.ldo;
      if (G.bias0) {
        y0 = y0 + G.bias0[r0 < G.rows ? r0 : 0];
        y1 = y1 + G.bias0[r1 < G.rows ? r1 : 0];
      }
      if (in0) hr[r0] = 0.5f * y0 * (1.0f + tanhf(0.7978845608028654f * (y0 + 0.044715f * y0 * y0 * y0)));
      if (in1) hr[r1] = 0.5f * y1 * (1.0f + tanhf(0.7978845608028654f * (y1 + 0.044715f * y1 * y1 * y1)));
    }
  }
}

// ---------------------------------------------------------------- attention
// Workgroup (query block, query head): 64 queries x 64 dimensions in LDS;
// per 64-key block, S = Q K^T (thread (ti, tj): queries 4ti .. 4ti+3, keys
// tj + 16b), the online softmax over the 16 threads of a query row, then
// O += P V (thread (ti, tj): queries 4ti .. 4ti+3, dimensions 4tj .. 4tj+3).
__global__ __launch_bounds__(WG) void k_pf_attn(PfArgs A, int li, int n, int pos0) {
  __shared__ float Qs[AQ * PF_HD];
  __shared__ float KP[AK * KS];  // keys, then the block's weights P
  __shared__ float Vs[AK * PF_HD];
  const int hq = blockIdx.y, qb = gridDim.x - 1 - blockIdx.x;  // the longest rows first
  const int T0 = qb * AQ;
  const int kvh = hq / (A.NH / A.NKV);
  const int ti = tid() >> 4, tj = tid() & 15;
  // the query block (zeros past the chunk)
  for (int i = tid(); i < AQ * PF_HD / 4; i += WG) {
    const int r = i >> 4, c = i & 15;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (T0 + r < n) v = reinterpret_cast<const float4 *>(A.q + (size_t)(T0 + r) * A.D + hq * PF_HD)[c];
    reinterpret_cast<float4 *>(Qs)[i] = v;
  }
  const int qlast = pos0 + min(T0 + AQ, n) - 1;  // last key any query of the block sees
  const int nkb = qlast / AK + 1;
  const size_t kbase = pf_kv_index(A, li, 0, kvh, 0), vbase = pf_kv_index(A, li, 1, kvh, 0);
  float m[4], l[4], o[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    m[a] = -INFINITY;
    l[a] = 0.f;
    o[a][0] = o[a][1] = o[a][2] = o[a][3] = 0.f;
  }
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * AK;
    __syncthreads();  // the previous block's P and V are consumed
    for (int i = tid(); i < AK * PF_HD / 4; i += WG) {
      const int r = i >> 4, c = i & 15;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (k0 + r <= qlast) {
        const size_t ko = kbase + (size_t)(k0 + r) * PF_HD + 4 * c, vo = vbase + (size_t)(k0 + r) * PF_HD + 4 * c;
        if (A.kv_fp16) {
          const __half *h = reinterpret_cast<const __half *>(A.kv);
          const uint2 ku = *reinterpret_cast<const uint2 *>(h + ko), vu = *reinterpret_cast<const uint2 *>(h + vo);
          const __half2 k01 = *reinterpret_cast<const __half2 *>(&ku.x), k23 = *reinterpret_cast<const __half2 *>(&ku.y);
          const __half2 v01 = *reinterpret_cast<const __half2 *>(&vu.x), v23 = *reinterpret_cast<const __half2 *>(&vu.y);
          kv = make_float4(__low2float(k01), __high2float(k01), __low2float(k23), __high2float(k23));
          vv = make_float4(__low2float(v01), __high2float(v01), __low2float(v23), __high2float(v23));
        } else {
          const float *f = reinterpret_cast<const float *>(A.kv);
          kv = *reinterpret_cast<const float4 *>(f + ko);
          vv = *reinterpret_cast<const float4 *>(f + vo);
        }
      }
      *reinterpret_cast<float4 *>(KP + r * KS + 4 * c) = kv;
      reinterpret_cast<float4 *>(Vs)[i] = vv;
    }
    __syncthreads();
    float s[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a) s[a][0] = s[a][1] = s[a][2] = s[a][3] = 0.f;
#pragma unroll 4
    for (int d = 0; d < PF_HD; d += 4) {
      float4 qa[4], kk[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) qa[a] = *reinterpret_cast<const float4 *>(Qs + (4 * ti + a) * PF_HD + d);
#pragma unroll
      for (int b = 0; b < 4; ++b) kk[b] = *reinterpret_cast<const float4 *>(KP + (tj + 16 * b) * KS + d);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          float z = s[a][b];
          z = __builtin_fmaf(qa[a].x, kk[b].x, z);
          z = __builtin_fmaf(qa[a].y, kk[b].y, z);
          z = __builtin_fmaf(qa[a].z, kk[b].z, z);
          z = __builtin_fmaf(qa[a].w, kk[b].w, z);
          s[a][b] = z;
        }
    }
    __syncthreads();  // every thread is done with the keys: KP becomes P
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int qpos = pos0 + T0 + 4 * ti + a;
      float mb = -INFINITY;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        s[a][b] = k0 + tj + 16 * b <= qpos ? s[a][b] * A.attn_scale : -INFINITY;
        mb = fmaxf(mb, s[a][b]);
      }
      // the 16 threads of the row are lanes 16k .. 16k+15 of the wave
      mb = fmaxf(mb, __shfl_xor(mb, 8, 16));
      mb = fmaxf(mb, __shfl_xor(mb, 4, 16));
      mb = fmaxf(mb, __shfl_xor(mb, 2, 16));
      mb = fmaxf(mb, __shfl_xor(mb, 1, 16));
      const float mn = fmaxf(m[a], mb);  // finite: key 0 is in block 0 for every query
      const float alpha = expf(m[a] - mn);
      float ps = 0.f;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float p = expf(s[a][b] - mn);
        KP[(4 * ti + a) * KS + tj + 16 * b] = p;
        ps += p;
      }
      ps += __shfl_xor(ps, 8, 16);
      ps += __shfl_xor(ps, 4, 16);
      ps += __shfl_xor(ps, 2, 16);
      ps += __shfl_xor(ps, 1, 16);
      l[a] = l[a] * alpha + ps;
      m[a] = mn;
#pragma unroll
      for (int c = 0; c < 4; ++c) o[a][c] *= alpha;
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < AK; k += 4) {
      float4 pa[4], vk[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) pa[a] = *reinterpret_cast<const float4 *>(KP + (4 * ti + a) * KS + k);
#pragma unroll
      for (int u = 0; u < 4; ++u) vk[u] = *reinterpret_cast<const float4 *>(Vs + (k + u) * PF_HD + 4 * tj);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float pp[4] = {pa[a].x, pa[a].y, pa[a].z, pa[a].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          o[a][0] = __builtin_fmaf(pp[u], vk[u].x, o[a][0]);
          o[a][1] = __builtin_fmaf(pp[u], vk[u].y, o[a][1]);
          o[a][2] = __builtin_fmaf(pp[u], vk[u].z, o[a][2]);
          o[a][3] = __builtin_fmaf(pp[u], vk[u].w, o[a][3]);
        }
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int t = T0 + 4 * ti + a;
    if (t < n)
      *reinterpret_cast<float4 *>(A.att + (size_t)t * A.D + hq * PF_HD + 4 * tj) =
          make_float4(o[a][0] / l[a], o[a][1] / l[a], o[a][2] / l[a], o[a][3] / l[a]);
  }
}

// ---------------------------------------------------------------- host
template <int NORM>
void launch_quant(const PfArgs &A, const float *src, int K, const float *g, int n, hipStream_t s) {
  hipLaunchKernelGGL(k_pf_quant<NORM>, dim3(n), dim3(WG), (size_t)K * sizeof(float), s, src, K, g, A.eps, A.px, A.sx);
}

template <int EPI>
void launch_gemm(const PfArgs &A, const PfGemm &G, hipStream_t s) {
  const int per_wg = (WG / 64) * G.rstep;
  hipLaunchKernelGGL(k_pf_gemm<EPI>, dim3((G.rows + per_wg - 1) / per_wg, (G.n + 31) / 32), dim3(WG), 0, s, A, G);
}

PfGemm gemm_same(const PfMat &W, int n, const float *bias, float *out, int ldo) {
  PfGemm G{};
  G.q0 = G.q1 = W.q;
  G.s0 = G.s1 = W.s;
  G.rows = W.rows;
  G.off1 = 32;
  G.rstep = 64;
  G.ng = W.cols >> 5;
  G.n = n;
  G.bias0 = G.bias1 = bias;
  G.out = out;
  G.ldo = ldo;
  return G;
}

}  // namespace

size_t pf_buffer_bytes(const PfArgs &A, int tc) {
  const size_t kmax = (size_t)(A.D > A.FF ? A.D : A.FF);
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  return al(sizeof(int32_t) * tc) + 3 * al(sizeof(float) * tc * A.D) + al(sizeof(float) * tc * A.FF) +
         al(sizeof(float) * tc) + al((size_t)tc * (kmax / 32) * PX_GROUP);
}

void pf_carve(PfArgs &A, void *base, int tc) {
  const size_t kmax = (size_t)(A.D > A.FF ? A.D : A.FF);
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  uint8_t *p = static_cast<uint8_t *>(base);
  A.tc = tc;
  A.ids = reinterpret_cast<int32_t *>(p);
  p += al(sizeof(int32_t) * tc);
  A.x = reinterpret_cast<float *>(p);
  p += al(sizeof(float) * tc * A.D);
  A.q = reinterpret_cast<float *>(p);
  p += al(sizeof(float) * tc * A.D);
  A.att = reinterpret_cast<float *>(p);
  p += al(sizeof(float) * tc * A.D);
  A.h = reinterpret_cast<float *>(p);
  p += al(sizeof(float) * tc * A.FF);
  A.sx = reinterpret_cast<float *>(p);
  p += al(sizeof(float) * tc);
  A.px = p;
}

int pf_layers(const PfArgs &A, const int32_t *ids, int n, int pos0, hipStream_t s) {
  if (n <= 0) return 0;
  MLLM_CHECK(n <= A.tc && pos0 >= 0 && pos0 + n <= A.max_seq, "prefill chunk of %d tokens at %d out of range", n,
             pos0);
  MLLM_CHECK(A.D == A.NH * PF_HD && A.D % 64 == 0 && A.FF % 64 == 0 && A.D <= 16384 && A.FF <= 16384,
             "prefill shapes unsupported (d_model %d, d_ff %d)", A.D, A.FF);
  MLLM_HIP(hipMemcpyAsync(A.ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
  const bool gpt2 = A.arch == 1;
  hipLaunchKernelGGL(k_pf_embed, dim3(n), dim3(WG), 0, s, A, n, pos0);
  const int nqb = (n + AQ - 1) / AQ;
  for (int li = 0; li < A.L; ++li) {
    const PfLayer &W = A.layers[li];
    if (gpt2)
      launch_quant<NORM_LN>(A, A.x, A.D, W.n1, n, s);
    else
      launch_quant<NORM_RMS>(A, A.x, A.D, W.n1, n, s);
    PfGemm G = gemm_same(W.qkv, n, gpt2 ? W.qkv_b : nullptr, nullptr, 0);
    G.li = li;
    G.pos0 = pos0;
    launch_gemm<EPI_QKV>(A, G, s);
    if (li == A.L - 1) break;  // the last layer's K and V are all the cache needs
    hipLaunchKernelGGL(k_pf_attn, dim3(nqb, A.NH), dim3(WG), 0, s, A, li, n, pos0);
    launch_quant<NORM_NONE>(A, A.att, A.D, nullptr, n, s);
    launch_gemm<EPI_RESID>(A, gemm_same(W.proj, n, gpt2 ? W.proj_b : nullptr, A.x, A.D), s);
    if (gpt2)
      launch_quant<NORM_LN>(A, A.x, A.D, W.n2, n, s);
    else
      launch_quant<NORM_RMS>(A, A.x, A.D, W.n2, n, s);
    if (gpt2) {
      launch_gemm<EPI_GELU>(A, gemm_same(W.w1, n, W.fc_b, A.h, A.FF), s);
    } else {
      PfGemm U{};
      U.q0 = W.w1.q;
      U.s0 = W.w1.s;
      U.q1 = W.w3.q;
      U.s1 = W.w3.s;
      U.rows = W.w1.rows;
      U.off1 = 0;
      U.rstep = 32;
      U.ng = W.w1.cols >> 5;
      U.n = n;
      U.out = A.h;
      U.ldo = A.FF;
      launch_gemm<EPI_SWIGLU>(A, U, s);
    }
    launch_quant<NORM_NONE>(A, A.h, A.FF, nullptr, n, s);
    launch_gemm<EPI_RESID>(A, gemm_same(W.w2, n, gpt2 ? W.mproj_b : nullptr, A.x, A.D), s);
  }
  MLLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace mllm
