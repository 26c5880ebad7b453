// mllm_prefill.hip -- batched prompt processing for forwardPrompt
// (infer.js:553-577): a chunk of T prompt tokens goes through every layer as
// a handful of wide kernels instead of 16-token passes of the decode phases.
//
// Q4 GEMMs on the f16 matrix cores with exact operands.  Each token's row
// is scaled by a power of two, 2^-e with e = ilogb(max |x|) - 14 (so the
// row's largest element lands in [2^14, 2^15), far from the f16 limits), and
// every scaled element x' is split into three f16 pieces,
//   p1 = f16(x'),  p2 = f16(x' - p1),  p3 = f16(x' - p1 - p2),
// whose sum is x' exactly (24 significant bits in three 11-bit pieces; only
// elements below 2^-16 of the row's max can lose bits, at 2^-39 of it).  The
// weights q - 8 of a Q4 group are small integers, exact in f16: the packed
// nibbles become f16 pairs 1024 + q with one v_perm_b32 against 0x64 bytes,
// then one packed f16 add of -1032.  A group (K = 32) is six
// v_mfma_f32_32x32x16_f16 per 32-row x 32-token sub-tile (three pieces x two
// K halves) chained in one f32 accumulator z, so the group's dot with the
// exact activations costs no integer combine; the epilogue is
//   acc = fma(z, w_scale, acc)
// in group order, one VALU operation per output and group, and the token's
// 2^e is applied once after the last group.  The matrix cores and the
// weight conversion then bound these GEMMs about equally.
//
// Operand layouts (v_mfma_f32_32x32x16_f16, checked on gfx950): A (the
// activations) lane l holds row l % 32 (a token) and 8 halves of k; B (the
// weights) lane l holds column l % 32 (a weight row) and the same 8 k; D
// lane l value v is (row 8(v/4) + 4(l/32) + v%4, column l % 32).  Only the
// pairing of A's and B's k matters: lane half hh = l / 32 holds the group's
// elements 16hh .. 16hh+15 (its 8 packed bytes), the first K half of the
// group takes elements 0 2 4 6 1 3 5 7 of those (the nibble order the
// conversion gives), the second 8 10 12 14 9 11 13 15.  The activation
// pieces are stored in that order, PXG bytes per (32-token tile, group):
// piece p, K half m at ((2p + m) * 64 + lane) * 16; after a tile's groups,
// its 32 tokens' exponents e.
//
// Attention: causal, one (32-query tile, KV head) per workgroup, 32-key
// blocks staged in LDS, S = Q K^T and O = P V on the f16 matrix cores with
// hi/lo splits for f32 accuracy, an online softmax (running max and sum,
// rescaled per block); the softmax of infer.js:422-504.
//
// Per layer: norm + quantise, QKV GEMM (bias or RoPE, K/V to the cache, q to
// a buffer), attention, quantise, O GEMM (+ residual), norm + quantise,
// gate/up GEMM (SwiGLU; gpt2 fc + GELU), quantise, down GEMM (+ residual).
// The last layer stops after its QKV GEMM: only its K and V are needed.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "mllm_device.h"
#include "mllm_host.h"
#include "mllm_prefill.h"

namespace mllm {
namespace {

// Workgroups of one token tile on one XCD (workgroup b runs on XCD b % 8):
// the GEMMs (MLLM_PF_XCD), the quantise kernels (MLLM_PF_XCDQ) and the
// attention (MLLM_PF_XCDA) put relative tile r on XCD r % 8.
#ifndef MLLM_PF_XCD
#define MLLM_PF_XCD 1
#endif
#ifndef MLLM_PF_XCDQ
#define MLLM_PF_XCDQ 1
#endif
#ifndef MLLM_PF_XCDA
#define MLLM_PF_XCDA 1
#endif
constexpr int PXG = 6 * 1024;  // bytes per (32-token tile, group): 3 pieces x 2 K halves x 64 lanes x 16
constexpr int PX_TOK = 128;    // after a tile's groups: its 32 tokens' exponents (int)
constexpr int PF_HD = 64;      // head dimension

// bytes per 32-token tile of activations with K columns
__host__ __device__ constexpr size_t px_tile_bytes(int K) { return (size_t)(K >> 5) * PXG + PX_TOK; }

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

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
// One token row of K floats per wave (tokens t0 .. t1-1): optional RMSNorm /
// LayerNorm (the decode engine's formulas), then the row's exponent and the
// three f16 pieces of every scaled element.  Wave reductions only.
template <int NORM>
__device__ __forceinline__ float4 pf_norm_col(const float4 *xr, const float4 *g4, int nq, int q, float r, float mean) {
  const float4 v = xr[q];
  if (NORM == NORM_RMS) {
    const float4 w = g4[q];
    return make_float4(v.x * r * w.x, v.y * r * w.y, v.z * r * w.z, v.w * r * w.w);
  }
  if (NORM == NORM_LN) {
    const float4 w = g4[q], b = g4[nq + q];
    const float4 d = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
    return make_float4(__builtin_fmaf(d.x * r, w.x, b.x), __builtin_fmaf(d.y * r, w.y, b.y),
                       __builtin_fmaf(d.z * r, w.z, b.z), __builtin_fmaf(d.w * r, w.w, b.w));
  }
  return v;
}

template <int NORM>
__device__ __forceinline__ void pf_norm_stats(const float4 *xr, int K, float eps, float &r, float &mean) {
  const int lane = tid() & 63, nq = K >> 2;
  const float inv_k = 1.0f / (float)K;
  r = 1.f;
  mean = 0.f;
  if (NORM == NORM_RMS) {
    float s1 = 0.f;
    for (int q = lane; q < nq; q += 64) {
      const float4 v = xr[q];
      s1 += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    r = __builtin_amdgcn_rsqf(wave_sum(s1) * inv_k + eps);
  } else if (NORM == NORM_LN) {
    float s1 = 0.f;
    for (int q = lane; q < nq; q += 64) {
      const float4 v = xr[q];
      s1 += (v.x + v.y) + (v.z + v.w);
    }
    mean = wave_sum(s1) * inv_k;
    float s2 = 0.f;
    for (int q = lane; q < nq; q += 64) {
      const float4 v = xr[q];
      const float4 d = make_float4(v.x - mean, v.y - mean, v.z - mean, v.w - mean);
      s2 += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
    }
    r = __builtin_amdgcn_rsqf(wave_sum(s2) * inv_k + 1e-5f);
  }
}

// Lane u of the wave owns (group u / 2, half u % 2) of the row -- 16
// consecutive elements, PPL such units per lane (K <= 1024 PPL) -- held in
// registers from one load.  A workgroup is QT waves: QT consecutive tokens
// of one 32-token tile.  The units' pieces (three pieces x two K halves of
// 16 bytes each) go to LDS first, unit u of token jj at u * qstr(QT) +
// ((2p + m) QT + jj) * 16 (padded so the 64 lanes' writes spread over the
// banks); then the workgroup copies them out so that the QT tokens' records
// of each (unit, piece, half) -- QT * 16 contiguous bytes of the GEMM operand
// layout, one whole 128-byte line at QT = 8 -- go out together.
__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
  const v2h v = {a, b};
  return __builtin_bit_cast(uint32_t, v);
}

// The three f16 pieces of x (x = p[0] + p[1] + p[2] exactly for the scaled
// rows, see the file comment); each conversion rounds to nearest.
__device__ __forceinline__ void pf_split3(float x, _Float16 (&p)[3]) {
  p[0] = (_Float16)x;
  const float r1 = x - (float)p[0];
  p[1] = (_Float16)r1;
  p[2] = (_Float16)(r1 - (float)p[1]);
}

// QT tokens (waves) per quantise workgroup: 8, or 4 where 8 tokens' records
// of a long row would not fit the LDS; qstr: LDS bytes per unit (its 6 x QT
// records, padded)
__host__ __device__ constexpr int qstr(int qt) { return 6 * qt * 16 + 16; }

// Token t's row (one wave, t < t1): the norm, the exponent (to the tile's
// exponent slot jt) and the unit records into the workgroup's LDS (token
// slot jj).
template <int NORM, int PPL, int QT>
__device__ __forceinline__ void pf_quant_row(const float *src, int K, const float *g, float eps, int t, int jj,
                                             int jt, uint8_t *tb, uint8_t *qs) {
  const int lane = tid() & 63, nu = K >> 4, ng = K >> 5;
  const float4 *xr = reinterpret_cast<const float4 *>(src + (size_t)t * K);
  const float4 *g4 = reinterpret_cast<const float4 *>(g);
  const float inv_k = 1.0f / (float)K;
  float4 y[PPL][4];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int u = lane + 64 * i;
#pragma unroll
    for (int c = 0; c < 4; ++c) y[i][c] = u < nu ? xr[4 * u + c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (NORM == NORM_RMS) {
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 v = y[i][c];
        s1 += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      }
    const float r = __builtin_amdgcn_rsqf(wave_sum(s1) * inv_k + eps);
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int u = lane + 64 * i;
      if (u < nu)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 v = y[i][c], w = g4[4 * u + c];
          y[i][c] = make_float4(v.x * r * w.x, v.y * r * w.y, v.z * r * w.z, v.w * r * w.w);
        }
    }
  } else if (NORM == NORM_LN) {
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) s1 += (y[i][c].x + y[i][c].y) + (y[i][c].z + y[i][c].w);
    const float mean = wave_sum(s1) * inv_k;
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int u = lane + 64 * i;
      if (u < nu)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 d = make_float4(y[i][c].x - mean, y[i][c].y - mean, y[i][c].z - mean, y[i][c].w - mean);
          s2 += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
    }
    const float r = __builtin_amdgcn_rsqf(wave_sum(s2) * inv_k + 1e-5f);
    const int nq = K >> 2;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int u = lane + 64 * i;
      if (u < nu)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 w = g4[4 * u + c], b = g4[nq + 4 * u + c];
          const float4 d = make_float4(y[i][c].x - mean, y[i][c].y - mean, y[i][c].z - mean, y[i][c].w - mean);
          y[i][c] = make_float4(__builtin_fmaf(d.x * r, w.x, b.x), __builtin_fmaf(d.y * r, w.y, b.y),
                                __builtin_fmaf(d.z * r, w.z, b.z), __builtin_fmaf(d.w * r, w.w, b.w));
        }
    }
  }
  // the row's exponent: its largest element scaled into [2^14, 2^15)
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < PPL; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v = y[i][c];  // zero past the row
      am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  am = wave_max(am);
  const int e = am > 0.f && am <= 3.4e38f ? __builtin_amdgcn_frexp_expf(am) - 1 - 14 : 0;
  if (lane == 0) reinterpret_cast<int *>(tb + (size_t)ng * PXG)[jt] = e;
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int u = lane + 64 * i;
    if (u >= nu) continue;
    // element order per K half: 0 2 4 6 1 3 5 7 (then + 8)
    const float4 *yc = y[i];
    _Float16 pc[16][3];
    const float ev[16] = {yc[0].x, yc[0].z, yc[1].x, yc[1].z, yc[0].y, yc[0].w, yc[1].y, yc[1].w,
                          yc[2].x, yc[2].z, yc[3].x, yc[3].z, yc[2].y, yc[2].w, yc[3].y, yc[3].w};
#pragma unroll
    for (int k = 0; k < 16; ++k) pf_split3(__builtin_amdgcn_ldexpf(ev[k], -e), pc[k]);
    uint8_t *rec = qs + (size_t)u * qstr(QT) + 16 * jj;
#pragma unroll
    for (int pi = 0; pi < 3; ++pi)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const _Float16(*q)[3] = pc + 8 * m;
        *reinterpret_cast<v4u *>(rec + (size_t)(2 * pi + m) * QT * 16) =
            v4u{pack_h2(q[0][pi], q[1][pi]), pack_h2(q[2][pi], q[3][pi]), pack_h2(q[4][pi], q[5][pi]),
                pack_h2(q[6][pi], q[7][pi])};
      }
  }
}

template <int NORM, int PPL, int QT>
__global__ __launch_bounds__(QT * 64) void k_pf_quant(const float *src, int K, const float *g, float eps,
                                                      uint8_t *px, int t0, int t1) {
  extern __shared__ float4 qsm4[];
  uint8_t *qs = reinterpret_cast<uint8_t *>(qsm4);
  // workgroup -> (tile rt, token slot); with MLLM_PF_XCDQ a tile's workgroups
  // run on the XCD that the GEMMs give it (relative tile rt on XCD rt % 8)
  int bq = blockIdx.x, rt = bq / (32 / QT), jslot = bq % (32 / QT);
  if (MLLM_PF_XCDQ && gridDim.x % (8 * (32 / QT)) == 0) {
    const int k = bq >> 3;
    rt = (bq & 7) + 8 * (k / (32 / QT));
    jslot = k % (32 / QT);
  }
  const int jj = tid() >> 6, j0 = QT * jslot;
  const int tile = t0 / 32 + rt, t = tile * 32 + j0 + jj;
  const int nu = K >> 4;
  uint8_t *tb = px + (size_t)tile * px_tile_bytes(K);
  if (t < t1) pf_quant_row<NORM, PPL, QT>(src, K, g, eps, t, jj, j0 + jj, tb, qs);  // wave-uniform
  __syncthreads();
  // the records out: unit u = (group u / 2, half hh = u % 2), piece p, K half
  // m, token jj at tile + (u / 2) PXG + (2p + m) 1024 + 16 (32 hh + j0 + jj)
  // (tokens past t1 carry whatever the LDS held: the GEMMs never use them)
  const int nrec = nu * 6 * QT;
  for (int f = tid(); f < nrec; f += QT * 64) {
    const int r = f % QT, pm = (f / QT) % 6, u = f / (6 * QT);
    const v4u v = *reinterpret_cast<const v4u *>(qs + (size_t)u * qstr(QT) + (pm * QT + r) * 16);
    *reinterpret_cast<v4u *>(tb + (size_t)(u >> 1) * PXG + pm * 1024 + 16 * (32 * (u & 1) + j0 + r)) = v;
  }
}

// The final norm of token t's row (one wave) into xn.
template <int NORM>
__global__ __launch_bounds__(64) void k_pf_final(const float *x, int K, int t, const float *g, float eps, float *xn) {
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)t * K);
  float r, mean;
  pf_norm_stats<NORM>(xr, K, eps, r, mean);
  for (int q = tid(); q < (K >> 2); q += 64)
    reinterpret_cast<float4 *>(xn)[q] = pf_norm_col<NORM>(xr, reinterpret_cast<const float4 *>(g), K >> 2, q, r, mean);
}

// ---------------------------------------------------------------- Q4 GEMM
// A wave computes two 32-row sub-tiles (sub-tile 1 is either the next 32
// rows of the same matrix -- a 64-row head of attn.qkv, 64 rows of the
// others -- or the same rows of a second matrix: mlp.w3 beside mlp.w1) for
// 32 tokens.  Workgroup: GWG / 64 waves, one token tile; with KS > 1, KS waves
// share a row range and take consecutive slices of the groups, and their
// sums are added in slice order through LDS (deterministic) before the
// epilogue -- more waves for the GEMMs with few row ranges.
struct PfGemm {
  const uint8_t *q0, *q1;
  const float *s0, *s1;
  int rows;   // rows of each matrix
  int off1;   // row offset of sub-tile 1 in its matrix (32 or 0)
  int rstep;  // rows per wave (64 or 32)
  int ng;     // groups per row
  int n;      // tokens
  int tt0;    // first token tile
  int li, pos0;
  const float *bias0, *bias1;  // per row of each matrix, or null
  float *out;                  // EPI_RESID: the residual rows; SWIGLU/GELU: the MLP activation
  int ldo;
};

// Eight packed nibbles q (one dword of a lane's weight operand, elements
// 0 .. 7 in nibble order) as the f16 values q - 8 in the order 0 2 4 6 1 3 5 7:
// each byte pair becomes the f16 pair 1024 + q by one v_perm_b32 against
// 0x64 high bytes, then one packed add of -1032 (exact: integers below 2048).
__device__ __forceinline__ v8h pf_w8(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu, k64 = 0x64646464u;
  const v2h off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const v2h a = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, k64, 0x00050004u)) + off;  // elements 0 2
  const v2h b = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(lo, k64, 0x00070006u)) + off;  // 4 6
  const v2h c = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, k64, 0x00050004u)) + off;  // 1 3
  const v2h d = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(hi, k64, 0x00070006u)) + off;  // 5 7
  return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}

#ifndef MLLM_PF_GPF
#define MLLM_PF_GPF 3
#endif
constexpr int GPF = MLLM_PF_GPF;  // groups of loads in flight per wave
#ifndef MLLM_PF_GWG
#define MLLM_PF_GWG 256
#endif
constexpr int GWG = MLLM_PF_GWG;  // threads per GEMM workgroup (waves sharing one token tile)

struct Pieces {
  v8h p0a, p0b, p1a, p1b, p2a, p2b;  // piece 0 .. 2, K half a / b
};

struct GemmLd {
  uint2 w0, w1;
  float c0, c1;
  Pieces x;
};

constexpr int PF_NGMAX = 128;  // groups per row (d_model, d_ff <= 4096)

// One sub-tile's group: the exact dot of the group's weights with the three
// pieces, chained in one f32 accumulator, then acc += dot * w_scale for the
// lane's 16 tokens.
__device__ __forceinline__ void pf_group_acc(const Pieces &x, uint2 w, float c, float (&acc)[16]) {
  const v8h b0 = pf_w8(w.x), b1 = pf_w8(w.y);
  v16f z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p0a, b0, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p0b, b1, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p1a, b0, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p1b, b1, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p2a, b0, z, 0, 0, 0);
  z = __builtin_amdgcn_mfma_f32_32x32x16_f16(x.p2b, b1, z, 0, 0, 0);
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = __builtin_fmaf(z[v], c, acc[v]);
}

template <int EPI, int KS>
__global__ __launch_bounds__(GWG) void k_pf_gemm(PfArgs A, PfGemm G) {
  __shared__ float red[KS > 1 ? GWG * 32 : 1];
  const int wv = tid() >> 6, lane = tid() & 63, j = lane & 31, hh = lane >> 5;
  const int ks = wv % KS;
  // workgroup -> (row range bx, token tile by); with MLLM_PF_XCD the
  // workgroups of one token tile sit on one XCD (workgroup b runs on XCD b % 8,
  // each with its own L2), so the tile's activation pieces are fetched into one
  // L2 and read there by every row range (a bijection when the tiles divide
  // over the eight XCDs)
  int bx = blockIdx.x, by = blockIdx.y;
  if (MLLM_PF_XCD && gridDim.y % 8 == 0) {
    const int b = bx + (int)gridDim.x * by, k = b >> 3;
    by = (b & 7) + 8 * (k / (int)gridDim.x);
    bx = k % (int)gridDim.x;
  }
  const int R = (bx * (GWG / 64 / KS) + wv / KS) * G.rstep;
  const bool active = R < G.rows;
  const int T0 = (G.tt0 + by) * 32;
  const int ng = G.ng, gb = ng * ks / KS, ge = ng * (ks + 1) / KS;  // this wave's groups
  // tiled operands (every row tile and token tile whole): per group, the
  // wave's weights are 512 contiguous bytes, its scales 128, the tile's
  // activation pieces 6 x 1024
  const size_t ta = (size_t)(R >> 5) * ng, tb = (size_t)((R + G.off1) >> 5) * ng;
  const uint8_t *wa = G.q0 + ta * 512 + 8 * lane, *wb = G.q1 + tb * 512 + 8 * lane;
  const float *sa = G.s0 + ta * 32 + j, *sb = G.s1 + tb * 32 + j;
  const uint8_t *xt = A.px + (size_t)(G.tt0 + by) * px_tile_bytes(32 * ng), *xa = xt + 16 * lane;
  auto load = [&](int g) {
    GemmLd L;
    L.w0 = *reinterpret_cast<const uint2 *>(wa + 512 * g);
    L.w1 = *reinterpret_cast<const uint2 *>(wb + 512 * g);
    L.c0 = sa[32 * g];
    L.c1 = sb[32 * g];
    const v4u *xg = reinterpret_cast<const v4u *>(xa + (size_t)PXG * g);
    L.x.p0a = __builtin_bit_cast(v8h, xg[0]);
    L.x.p0b = __builtin_bit_cast(v8h, xg[64]);
    L.x.p1a = __builtin_bit_cast(v8h, xg[128]);
    L.x.p1b = __builtin_bit_cast(v8h, xg[192]);
    L.x.p2a = __builtin_bit_cast(v8h, xg[256]);
    L.x.p2b = __builtin_bit_cast(v8h, xg[320]);
    return L;
  };
  float acc0[16], acc1[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.f;
  // the loads of group g + GPF go out before group g is computed
  GemmLd ring[GPF];
  if (active) {
    // (groups past ge are loaded and not used: the tiled matrices and the
    // activation tiles carry GPF groups of padding)
#pragma unroll
    for (int i = 0; i < GPF; ++i) ring[i] = load(gb + i);
    for (int g0 = gb; g0 < ge; g0 += GPF)
#pragma unroll
      for (int i = 0; i < GPF; ++i) {
        if (g0 + i >= ge) break;
        const GemmLd cur = ring[i];
        ring[i] = load(g0 + i + GPF);
        pf_group_acc(cur.x, cur.w0, cur.c0, acc0);
        pf_group_acc(cur.x, cur.w1, cur.c1, acc1);
      }
  }
  if (KS > 1) {
    // partials value-major in 16-byte quads, red4[q * GWG + thread]: the 64
    // lanes of a wave touch 1 KiB of consecutive LDS per access, so no two
    // lanes of a pass share a bank
    v4f *red4 = reinterpret_cast<v4f *>(red);
    if (ks > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        red4[q * GWG + tid()] = v4f{acc0[4 * q], acc0[4 * q + 1], acc0[4 * q + 2], acc0[4 * q + 3]};
        red4[(4 + q) * GWG + tid()] = v4f{acc1[4 * q], acc1[4 * q + 1], acc1[4 * q + 2], acc1[4 * q + 3]};
      }
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k = 1; k < KS; ++k) {
      const int o = tid() + 64 * k;  // the same lane of slice k's wave
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4f a = red4[q * GWG + o], b = red4[(4 + q) * GWG + o];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0[4 * q + e] = acc0[4 * q + e] + a[e];
          acc1[4 * q + e] = acc1[4 * q + e] + b[e];
        }
      }
    }
  }
  if (!active) return;
  // epilogue: value v is token T0 + 8(v/4) + 4hh + v%4, rows r0 / r1; the
  // token's exponent undoes its row scaling (exact)
  const int r0 = R + j, r1 = R + G.off1 + j;
  const bool in0 = r0 < G.rows, in1 = r1 < G.rows;
  int ex[16];
  {
    const int4 *et = reinterpret_cast<const int4 *>(xt + (size_t)ng * PXG) + hh;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int4 e4 = et[2 * k];
      ex[4 * k] = e4.x;
      ex[4 * k + 1] = e4.y;
      ex[4 * k + 2] = e4.z;
      ex[4 * k + 3] = e4.w;
    }
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int t = T0 + 8 * (v >> 2) + 4 * hh + (v & 3);
    if (t >= G.n) continue;
    float y0 = __builtin_amdgcn_ldexpf(acc0[v], ex[v]), y1 = __builtin_amdgcn_ldexpf(acc1[v], ex[v]);
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
// Workgroup (32-query tile, KV head), one wave per query head of the KV
// head (GQA: the waves share the staged keys and values).  Per 32-key block,
// on the f16 matrix cores (v_mfma_f32_32x32x16_f16, f32 accumulation):
//   S^T = K Q^T   A = the keys (lane: key j, 8 dimensions), B = the queries;
//                 out lane (query j, half hh) holds keys 8(v/4) + 4hh + v%4
//   O^T += V^T P^T  A = the values transposed (lane: dimension j), B = the
//                 weights P straight from the S^T registers: slot s of half
//                 hh is key 8(s/4) + 4hh + s%4 (+16 for the block's second
//                 half), so V^T takes the same keys per slot
// so every lane holds one query's scores and output column, and the online
// softmax (running max and sum, per-block rescaling) needs one exchange with
// the lane 32 apart.  f32 accuracy from f16 operands: the scaled query and
// the weights are split as hi + lo halves (v = hi + lo to ~2^-22), and so are
// f32 keys and values (an f16 cache is exact as is); the dropped lo x lo
// terms are below 2^-40 relative.  The scores are formed in the log2 domain
// (the query scaled by attn_scale * log2 e) for v_exp_f32.
constexpr int QTL = 32;   // queries per wave
constexpr int KROW = 72;  // halves per staged key row (64 + pad)

// Eight consecutive cache values as loaded (f16: one 16-byte load, f32: two),
// widened to f32 when staged.
struct Raw8 {
  uint4 a, b;
};
template <bool F32>
__device__ __forceinline__ Raw8 load8(const PfArgs &A, size_t off) {
  Raw8 r;
  if (F32) {
    r.a = *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(A.kv) + off);
    r.b = *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(A.kv) + off + 4);
  } else {
    r.a = *reinterpret_cast<const uint4 *>(reinterpret_cast<const __half *>(A.kv) + off);
    r.b = make_uint4(0u, 0u, 0u, 0u);
  }
  return r;
}
template <bool F32>
__device__ __forceinline__ void widen8(const Raw8 &r, float (&v)[8]) {
  if (F32) {
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const __half2 h = *reinterpret_cast<const __half2 *>(&w[i]);
      v[2 * i] = __low2float(h);
      v[2 * i + 1] = __high2float(h);
    }
  }
}
constexpr int SCH = 4;   // staged 8-value chunks per thread and super-block (32 NSET keys x 8 chunks, >= 64 NSET threads)

// The tile's key blocks are dealt round-robin to NSET sets of waves (block
// NSET i + s to set s; a wave per query head in each set), each set keeping
// its own running (max, sum, output); at the end sets 1 .. NSET-1 hand theirs
// to set 0 through LDS, which merges them in set order.  A super-block is the
// NSET blocks the sets take at once.  NSET = 2 puts 2 rep waves on the 4
// SIMDs (two SIMDs run two of a KV head's three query-head waves and the
// others one); NSET = 4 with rep 3 puts three waves on every SIMD and takes
// twice the keys per staging round.  (NSET = 4 needs rep <= 3 and the f16
// cache: 4 rep waves of an f32 cache's registers would not fit.)
template <bool SPLIT_KV, int NSET>
__global__ __launch_bounds__(NSET == 4 ? 768 : 512) void k_pf_attn(PfArgs A, int li, int n, int pos0, int tt0) {
  constexpr int KSB = 32 * NSET;    // keys per super-block
  constexpr int VROW = KSB + 4;     // halves per staged value column (KSB keys + pad)
  constexpr int MAXREP = NSET == 4 ? 3 : 4;
  constexpr int KB_BYTES = KSB * KROW * 2, VB_BYTES = PF_HD * VROW * 2;
  constexpr int STAGE = (SPLIT_KV ? 2 : 1) * (KB_BYTES + VB_BYTES);
  constexpr int MERGE = (NSET - 1) * MAXREP * 64 * 34 * 4;  // sets 1.. x heads x 64 lanes x (32 outputs, max, sum)
  __shared__ __attribute__((aligned(16))) uint8_t smem[STAGE > MERGE ? STAGE : MERGE];
  _Float16 *Kh = reinterpret_cast<_Float16 *>(smem), *Vh = Kh + KSB * KROW;
  _Float16 *Kl = Vh + PF_HD * VROW, *Vl = Kl + KSB * KROW;  // SPLIT_KV only
  const int rep = A.NH / A.NKV;
  // the longest tiles first; with MLLM_PF_XCDA relative tile r runs on XCD
  // r % 8, where the GEMMs put it
  int rtile = gridDim.x - 1 - blockIdx.x, kvh = blockIdx.y;
  if (MLLM_PF_XCDA && gridDim.x % 8 == 0) {
    const int b = blockIdx.x + gridDim.x * blockIdx.y, k = b >> 3;
    rtile = (b & 7) + 8 * ((int)gridDim.x / 8 - 1 - k / (int)gridDim.y);
    kvh = k % (int)gridDim.y;
  }
  const int T0 = (tt0 + rtile) * QTL;
  const int lane = tid() & 63, j = lane & 31, hh = lane >> 5;
  const int wv = tid() >> 6, set = wv / rep, hsel = wv - set * rep;
  const int hq = kvh * rep + hsel;
  v8h qh[4], ql[4];
  {
    const float c = A.attn_scale * 1.4426950408889634f;
    const float *qr = A.q + (size_t)min(T0 + j, n - 1) * A.D + hq * PF_HD + 8 * hh;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = qr[16 * m + i] * c;
        const _Float16 h = (_Float16)v;
        qh[m][i] = h;
        ql[m][i] = (_Float16)(v - (float)h);
      }
  }
  const int qpos = pos0 + T0 + j;
  const int qlast = pos0 + min(T0 + QTL, n) - 1;  // last key any query of the tile sees
  const int nsb = qlast / KSB + 1;
  const size_t kbase = pf_kv_index(A, li, 0, kvh, 0), vbase = pf_kv_index(A, li, 1, kvh, 0);
  float m_run = -INFINITY, l_run = 0.f;
  v16f o0, o1;
#pragma unroll
  for (int v = 0; v < 16; ++v) o0[v] = o1[v] = 0.f;
  // chunks c = tid + i * blockDim (key c / 8 of the super-block, dimensions
  // 8 (c % 8) .. +7), loaded one super-block ahead of their use
  Raw8 rk[SCH], rv[SCH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int c = tid() + i * (int)blockDim.x, kk = c >> 3, d0 = (c & 7) * 8;
      if (c < KSB * 8 && k0 + kk <= qlast) {
        rk[i] = load8<SPLIT_KV>(A, kbase + (size_t)(k0 + kk) * PF_HD + d0);
        rv[i] = load8<SPLIT_KV>(A, vbase + (size_t)(k0 + kk) * PF_HD + d0);
      } else {
        rk[i].a = rk[i].b = rv[i].a = rv[i].b = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  fetch(0);
  for (int sb = 0; sb < nsb; ++sb) {
    __syncthreads();  // the previous super-block is consumed
#pragma unroll
    for (int ci = 0; ci < SCH; ++ci) {
      const int c = tid() + ci * (int)blockDim.x, kk = c >> 3, d0 = (c & 7) * 8;
      if (c >= KSB * 8) break;
      if (SPLIT_KV) {
        float kv[8], vv[8];
        widen8<true>(rk[ci], kv);
        widen8<true>(rv[ci], vv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const _Float16 kh = (_Float16)kv[i], vh = (_Float16)vv[i];
          Kh[kk * KROW + d0 + i] = kh;
          Vh[(d0 + i) * VROW + kk] = vh;
          Kl[kk * KROW + d0 + i] = (_Float16)(kv[i] - (float)kh);
          Vl[(d0 + i) * VROW + kk] = (_Float16)(vv[i] - (float)vh);
        }
      } else {  // an f16 cache is staged as is
        *reinterpret_cast<uint4 *>(Kh + kk * KROW + d0) = rk[ci].a;
        const uint32_t w[4] = {rv[ci].a.x, rv[ci].a.y, rv[ci].a.z, rv[ci].a.w};
        unsigned short *vt = reinterpret_cast<unsigned short *>(Vh);
#pragma unroll
        for (int i = 0; i < 8; ++i) vt[(d0 + i) * VROW + kk] = (unsigned short)(w[i >> 1] >> (16 * (i & 1)));
      }
    }
    if (sb + 1 < nsb) fetch((sb + 1) * KSB);
    __syncthreads();
    const int k0 = sb * KSB + 32 * set;  // this set's block
    if (k0 > qlast) continue;            // past every query of the tile (uniform)
    const int kr = 32 * set;             // its rows / columns in the staged super-block
    v16f s;
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const v8h ka = *reinterpret_cast<const v8h *>(Kh + (kr + j) * KROW + 16 * m + 8 * hh);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[m], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, ql[m], s, 0, 0, 0);
      if (SPLIT_KV) {
        const v8h kl = *reinterpret_cast<const v8h *>(Kl + (kr + j) * KROW + 16 * m + 8 * hh);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[m], s, 0, 0, 0);
      }
    }
    float mx = -INFINITY;
    if (k0 + 31 > pos0 + T0) {  // the block reaches past a query of the tile: mask
#pragma unroll
      for (int v = 0; v < 16; ++v)
        if (k0 + 8 * (v >> 2) + 4 * hh + (v & 3) > qpos) s[v] = -INFINITY;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m_run, mx);
    // a query with no key yet in this set: everything stays zero
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mref);
    v8h ph[2], pl[2];
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = __builtin_amdgcn_exp2f(s[v] - mref);
      ps += p;
      const _Float16 h = (_Float16)p;
      ph[v >> 3][v & 7] = h;
      pl[v >> 3][v & 7] = (_Float16)(p - (float)h);
    }
    ps += __shfl_xor(ps, 32);
    l_run = l_run * alpha + ps;
    // rescale the outputs unless no lane's running max moved (alpha = 1)
    if (__builtin_amdgcn_read_exec() & __ballot(mn != m_run)) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        o0[v] *= alpha;
        o1[v] *= alpha;
      }
    }
    m_run = mn;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kc = kr + 16 * u + 4 * hh;
      const v4h a0 = *reinterpret_cast<const v4h *>(Vh + j * VROW + kc);
      const v4h a1 = *reinterpret_cast<const v4h *>(Vh + j * VROW + kc + 8);
      const v4h b0 = *reinterpret_cast<const v4h *>(Vh + (32 + j) * VROW + kc);
      const v4h b1 = *reinterpret_cast<const v4h *>(Vh + (32 + j) * VROW + kc + 8);
      const v8h va = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      const v8h vb = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph[u], o0, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl[u], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb, ph[u], o1, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb, pl[u], o1, 0, 0, 0);
      if (SPLIT_KV) {
        const v4h c0 = *reinterpret_cast<const v4h *>(Vl + j * VROW + kc);
        const v4h c1 = *reinterpret_cast<const v4h *>(Vl + j * VROW + kc + 8);
        const v4h d0 = *reinterpret_cast<const v4h *>(Vl + (32 + j) * VROW + kc);
        const v4h d1 = *reinterpret_cast<const v4h *>(Vl + (32 + j) * VROW + kc + 8);
        o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_shufflevector(c0, c1, 0, 1, 2, 3, 4, 5, 6, 7), ph[u], o0,
                                                    0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_shufflevector(d0, d1, 0, 1, 2, 3, 4, 5, 6, 7), ph[u], o1,
                                                    0, 0, 0);
      }
    }
  }
  // merge: sets 1 .. NSET-1 hand (outputs, max, sum) to set 0 through LDS
  // (slot (s - 1, head, lane)); set 0 adds them in set order
  float *const mrg0 = reinterpret_cast<float *>(smem) + (size_t)(hsel * 64 + lane) * 34;
  constexpr size_t MSET = (size_t)MAXREP * 64 * 34;  // floats per set's slots
  __syncthreads();  // the staging area is free
  if (set > 0) {
    float *mrg = mrg0 + (set - 1) * MSET;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      mrg[v] = o0[v];
      mrg[16 + v] = o1[v];
    }
    mrg[32] = m_run;
    mrg[33] = l_run;
  }
  __syncthreads();
  if (set == 0 && T0 + j < n) {
    float M = m_run;  // finite: set 0 holds key 0
#pragma unroll
    for (int s = 1; s < NSET; ++s) M = fmaxf(M, mrg0[(s - 1) * MSET + 32]);
    float a[NSET];
    a[0] = __builtin_amdgcn_exp2f(m_run - M);
    float l = l_run * a[0];
#pragma unroll
    for (int s = 1; s < NSET; ++s) {
      a[s] = __builtin_amdgcn_exp2f(mrg0[(s - 1) * MSET + 32] - M);
      l = l + mrg0[(s - 1) * MSET + 33] * a[s];
    }
    float *out = A.att + (size_t)(T0 + j) * A.D + hq * PF_HD + 4 * hh;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float r[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r0 = o0[4 * g + e] * a[0], r1 = o1[4 * g + e] * a[0];
#pragma unroll
        for (int s = 1; s < NSET; ++s) {
          r0 = r0 + mrg0[(s - 1) * MSET + 4 * g + e] * a[s];
          r1 = r1 + mrg0[(s - 1) * MSET + 16 + 4 * g + e] * a[s];
        }
        r[e] = r0 / l;
        r[4 + e] = r1 / l;
      }
      *reinterpret_cast<float4 *>(out + 8 * g) = make_float4(r[0], r[1], r[2], r[3]);
      *reinterpret_cast<float4 *>(out + 32 + 8 * g) = make_float4(r[4], r[5], r[6], r[7]);
    }
  }
}

// ---------------------------------------------------------------- weight tiling
// The prefill GEMMs read a tiled copy of each Q4 matrix: for row tile rt
// (rows 32 rt .. 32 rt + 31) and group g, the 64 lanes' 8-byte weight
// operands in lane order (lane 32 hh + j: bytes 8hh .. 8hh+7 of the group in
// row 32 rt + j), then separately the 32 rows' scales.
__global__ __launch_bounds__(WG) void k_pf_tile(PfMat W, uint8_t *q, float *s) {
  const int ng = W.cols >> 5;
  const size_t units = (size_t)(W.rows >> 5) * ng * 64;  // (row tile, group, lane)
  for (size_t u = (size_t)blockIdx.x * WG + tid(); u < units; u += (size_t)gridDim.x * WG) {
    const int lane = (int)(u & 63), j = lane & 31, hh = lane >> 5;
    const size_t tg = u >> 6;  // rt * ng + g
    const int g = (int)(tg % ng), r = (int)(tg / ng) * 32 + j;
    const uint8_t *src = W.q + (size_t)r * ng * 16 + 16 * g + 8 * hh;
    *reinterpret_cast<uint2 *>(q + u * 8) = *reinterpret_cast<const uint2 *>(src);
    if (hh == 0) s[tg * 32 + j] = W.s[(size_t)r * ng + g];
  }
}

// ---------------------------------------------------------------- host
// One quantise instance: past 64 KB of LDS a kernel needs the opt-in, made
// once per instance.
template <int NORM, int PPL, int QT>
void quant_launch(dim3 grid, size_t lds, hipStream_t s, const PfArgs &A, const float *src, int K, const float *g,
                  int t0, int t1) {
  static bool opted = false;
  if (lds > 64 * 1024 && !opted)
    opted = hipFuncSetAttribute(reinterpret_cast<const void *>(k_pf_quant<NORM, PPL, QT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  hipLaunchKernelGGL((k_pf_quant<NORM, PPL, QT>), grid, dim3(QT * 64), lds, s, src, K, g, A.eps, A.px, t0, t1);
}

template <int NORM>
void launch_quant(const PfArgs &A, const float *src, int K, const float *g, int t0, int t1, hipStream_t s) {
  // QT tokens per workgroup (t0 is a multiple of 32); the LDS holds the QT
  // tokens' records of every unit: (K / 16) * qstr(QT) bytes, 125 KB at
  // K = 2560 with QT = 8, at most 100 KB at K = 4096 with QT = 4
  const int qt = (K >> 4) * qstr(8) <= 160 * 1024 ? 8 : 4;
  const dim3 grid(((t1 - t0 + 31) / 32) * (32 / qt));
  const size_t lds = (size_t)(K >> 4) * qstr(qt);
  if (K <= 1024)
    quant_launch<NORM, 1, 8>(grid, lds, s, A, src, K, g, t0, t1);
  else if (K <= 2048)
    quant_launch<NORM, 2, 8>(grid, lds, s, A, src, K, g, t0, t1);
  else if (qt == 8)
    quant_launch<NORM, 4, 8>(grid, lds, s, A, src, K, g, t0, t1);
  else
    quant_launch<NORM, 4, 4>(grid, lds, s, A, src, K, g, t0, t1);
}

#ifndef MLLM_PF_WAVES
#define MLLM_PF_WAVES 1024
#endif
#ifndef MLLM_PF_MINSLICE
#define MLLM_PF_MINSLICE 8
#endif
// Group slices per row range (KS, 1, 2 or 4): doubled while the launch has
// fewer than MLLM_PF_WAVES row waves and every slice keeps MLLM_PF_MINSLICE
// groups (1024 and 8 measured best: 2048 or 4096 waves gave longer prompts).
template <int EPI>
void launch_gemm(const PfArgs &A, const PfGemm &G, hipStream_t s) {
  const int tt = (G.n + 31) / 32 - G.tt0, rw = (G.rows + G.rstep - 1) / G.rstep;
  int ks = 1;
  while (ks < 4 && rw * tt * ks < MLLM_PF_WAVES && G.ng / (2 * ks) >= MLLM_PF_MINSLICE) ks *= 2;
  const int per_wg = (GWG / 64 / ks) * G.rstep;
  const dim3 grid((G.rows + per_wg - 1) / per_wg, tt);
  if (ks == 1) hipLaunchKernelGGL((k_pf_gemm<EPI, 1>), grid, dim3(GWG), 0, s, A, G);
  if (ks == 2) hipLaunchKernelGGL((k_pf_gemm<EPI, 2>), grid, dim3(GWG), 0, s, A, G);
  if (ks == 4) hipLaunchKernelGGL((k_pf_gemm<EPI, 4>), grid, dim3(GWG), 0, s, A, G);
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

size_t pf_tiled_bytes(const PfMat &W) {
  // + GPF groups of padding after the scales (read ahead, never used)
  const size_t packed = ((size_t)W.rows * W.cols / 2 + 255) & ~(size_t)255;
  return (packed + (size_t)W.rows * (W.cols / 32) * sizeof(float) + GPF * 512 + 255) & ~(size_t)255;
}

int pf_tile(const PfMat &W, void *dst, PfMat *out, hipStream_t s) {
  MLLM_CHECK(W.rows % 32 == 0 && W.cols % 32 == 0, "matrix %d x %d cannot be tiled", W.rows, W.cols);
  uint8_t *q = static_cast<uint8_t *>(dst);
  float *sc = reinterpret_cast<float *>(q + (((size_t)W.rows * W.cols / 2 + 255) & ~(size_t)255));
  const size_t units = (size_t)(W.rows / 32) * (W.cols / 32) * 64;
  const int blocks = (int)std::min<size_t>((units + WG - 1) / WG, 4096);
  hipLaunchKernelGGL(k_pf_tile, dim3(blocks), dim3(WG), 0, s, W, q, sc);
  MLLM_HIP(hipGetLastError());
  *out = PfMat{q, sc, W.rows, W.cols};
  return 0;
}

bool pf_supported(const PfArgs &A) {
  return A.D == A.NH * PF_HD && A.NH % A.NKV == 0 && A.NH / A.NKV <= 4 && A.FF % 64 == 0 &&
         A.D <= 32 * PF_NGMAX && A.FF <= 32 * PF_NGMAX;
}

size_t pf_buffer_bytes(const PfArgs &A, int tc) {
  const size_t kmax = (size_t)(A.D > A.FF ? A.D : A.FF);
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  // + GPF groups of padding after the last tile (read ahead, never used)
  return al(sizeof(int32_t) * tc) + 3 * al(sizeof(float) * tc * A.D) + al(sizeof(float) * tc * A.FF) +
         al(gemv_q4_argmax_scratch(A.emb.rows, A.emb.cols)) +
         al((size_t)((tc + 31) / 32) * px_tile_bytes((int)kmax) + (size_t)GPF * PXG);
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
  A.amx = p;
  p += al(gemv_q4_argmax_scratch(A.emb.rows, A.emb.cols));
  A.px = p;
}

int pf_layers(const PfArgs &A, const int32_t *ids, int n, int pos0, bool last, hipStream_t s) {
  if (n <= 0) return 0;
  MLLM_CHECK(n <= A.tc && pos0 >= 0 && pos0 + n <= A.max_seq, "prefill chunk of %d tokens at %d out of range", n,
             pos0);
  MLLM_CHECK(pf_supported(A), "prefill shapes unsupported (d_model %d, d_ff %d, %d heads, %d KV heads)", A.D, A.FF,
             A.NH, A.NKV);
  MLLM_HIP(hipMemcpyAsync(A.ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
  const bool gpt2 = A.arch == 1;
  hipLaunchKernelGGL(k_pf_embed, dim3(n), dim3(WG), 0, s, A, n, pos0);
  const int nqt = (n + QTL - 1) / QTL, rep = A.NH / A.NKV;
  for (int li = 0; li < A.L; ++li) {
    const PfLayer &W = A.layers[li];
    if (gpt2)
      launch_quant<NORM_LN>(A, A.x, A.D, W.n1, 0, n, s);
    else
      launch_quant<NORM_RMS>(A, A.x, A.D, W.n1, 0, n, s);
    PfGemm G = gemm_same(W.qkv, n, gpt2 ? W.qkv_b : nullptr, nullptr, 0);
    G.li = li;
    G.pos0 = pos0;
    launch_gemm<EPI_QKV>(A, G, s);
    // the last layer: only the K and V, or (for the prompt's last token) the
    // rest of it for the last token tile alone
    const bool final_layer = li == A.L - 1;
    if (final_layer && !last) break;
    const int tt0 = final_layer ? nqt - 1 : 0, t0 = tt0 * QTL;
    if (A.kv_fp16 && rep <= 3)
      hipLaunchKernelGGL((k_pf_attn<false, 4>), dim3(nqt - tt0, A.NKV), dim3(256 * rep), 0, s, A, li, n, pos0, tt0);
    else if (A.kv_fp16)
      hipLaunchKernelGGL((k_pf_attn<false, 2>), dim3(nqt - tt0, A.NKV), dim3(128 * rep), 0, s, A, li, n, pos0, tt0);
    else
      hipLaunchKernelGGL((k_pf_attn<true, 2>), dim3(nqt - tt0, A.NKV), dim3(128 * rep), 0, s, A, li, n, pos0, tt0);
    launch_quant<NORM_NONE>(A, A.att, A.D, nullptr, t0, n, s);
    PfGemm O = gemm_same(W.proj, n, gpt2 ? W.proj_b : nullptr, A.x, A.D);
    O.tt0 = tt0;
    launch_gemm<EPI_RESID>(A, O, s);
    if (gpt2)
      launch_quant<NORM_LN>(A, A.x, A.D, W.n2, t0, n, s);
    else
      launch_quant<NORM_RMS>(A, A.x, A.D, W.n2, t0, n, s);
    if (gpt2) {
      PfGemm F = gemm_same(W.w1, n, W.fc_b, A.h, A.FF);
      F.tt0 = tt0;
      launch_gemm<EPI_GELU>(A, F, s);
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
      U.tt0 = tt0;
      U.out = A.h;
      U.ldo = A.FF;
      launch_gemm<EPI_SWIGLU>(A, U, s);
    }
    launch_quant<NORM_NONE>(A, A.h, A.FF, nullptr, t0, n, s);
    PfGemm Dn = gemm_same(W.w2, n, gpt2 ? W.mproj_b : nullptr, A.x, A.D);
    Dn.tt0 = tt0;
    launch_gemm<EPI_RESID>(A, Dn, s);
  }
  if (last) {
    // the final norm of the last token, then the lm_head and the greedy
    // argmax in one launch (the standalone Q4 GEMV's rows, infer.js:240-250's
    // first maximum)
    float *xn = A.att;  // free once the layers are done
    if (gpt2)
      hipLaunchKernelGGL(k_pf_final<NORM_LN>, dim3(1), dim3(64), 0, s, A.x, A.D, n - 1, A.norm_f, A.eps, xn);
    else
      hipLaunchKernelGGL(k_pf_final<NORM_RMS>, dim3(1), dim3(64), 0, s, A.x, A.D, n - 1, A.norm_f, A.eps, xn);
    if (int rc = gemv_q4_argmax_into(A.emb.rows, A.emb.cols, A.emb.q, A.emb.s, xn, A.logits, A.res, A.amx, s))
      return rc;
  }
  MLLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace mllm
