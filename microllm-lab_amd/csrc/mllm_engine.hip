// mllm_engine.hip -- the fused single-token Q4 decode step on MI355X and the
// engine-level C ABI (PetitGPT API of engine/infer.js:289-647).
//
// One decode step = L x [QKV, ATTN, O, UP, DOWN] + LM + ARGMAX phases
// (engine/infer.js:579-601; the reference GPU runs the same graph as 244
// dispatches, engine/webgpu-metal.js:1242-1322):
//   QKV   (one workgroup per 64-row head tile of blocks.i.attn.qkv)
//         prologue: embed (layer 0) or load x; RMSNorm/LayerNorm in LDS
//         epilogue: bias (gpt2), RoPE (llama), q -> scratch, k/v -> KV cache
//   ATTN  (one workgroup per (token, 256-position split, head))
//         scores, split-local softmax statistics and P.V -> partials (m, l, acc)
//   O     prologue: combine the splits -> attention output; epilogue x += W_o.att
//   UP    prologue: norm2; gate and up rows of the same index -> silu(g)*u
//         (gpt2: fc + bias -> GELU-tanh)
//   DOWN  epilogue x += W_2.h (+ bias)
//   LM    prologue: final norm; logits + per-tile argmax (gpt2 chain: 3-gram
//         block and repetition penalty of infer.js:252-287)
//   ARGMAX one workgroup: first maximum over tiles; chained decode feeds it
//         back as the next input token (CHAIN_TOK, webgpu-metal.js:609-610).
//
// Execution: mode 0 runs every phase of a pass (or of n chained steps) in one
// persistent cooperative kernel with a grid barrier between phases; mode 1
// launches one kernel per phase and replays a captured HIP graph per chained
// step.  Both modes run the same per-item device code.
//
// Every per-token computation (norm, GEMV row, attention split, combine,
// argmax) runs the same instruction sequence whatever the number of tokens in
// the pass, so a row of the multi-token verify pass is bit-identical to the
// single-token decode of that position.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "mllm_device.h"
#include "mllm_host.h"

namespace mllm {

constexpr int HD = 64;    // head dimension of every supported config
constexpr int ACH = 256;  // positions per attention split (one per thread)
constexpr int MAXT = 16;  // tokens per pass (upper bound; LDS sets the real one)
constexpr int APS = 68;   // floats per attention partial: m, l, pad, pad, acc[64]
constexpr unsigned kSpinLimit = 1u << 22;

enum Phase { PH_QKV = 0, PH_ATTN, PH_O, PH_UP, PH_DOWN, PH_LM, PH_ARGMAX, PH_COUNT };

struct LayerW {
  Q4Mat qkv, proj, w1, w3, w2;  // gpt2: w1 = mlp.fc, w2 = mlp.proj
  const float *n1, *n2;         // RMS gains; gpt2: LayerNorm gamma || beta
  const float *qkv_b, *proj_b, *fc_b, *mproj_b;
};

// Device-resident description of the current pass; every phase reads it.
struct PassState {
  int pos0;      // position of token 0
  int ntok;      // tokens in the pass
  int lm_rows;   // 0: no lm_head, 1: last token only, 2: every token
  int chain;     // chained decode: ARGMAX feeds tok[0] and advances pos0
  int eos;       // chain stop id (-1: none)
  int done;      // chain reached eos
  int n_hist;    // tokens in hist[] (gpt2 argmax history / chain output)
  int err;       // barrier time-out
  int tok[MAXT];
  int res[MAXT];  // argmax per lm row
};

struct DecParams {
  int arch, L, D, NH, NKV, FF, V, max_seq, rd, kv_fp16, nsplit_max;
  float eps, attn_scale;
  const LayerW *layers;
  Q4Mat lm;
  const float *norm_f, *wpe, *sf, *rope_cos, *rope_sin;
  float *x;     // [MAXT][D] residual stream
  float *q;     // [MAXT][NH*HD] queries after RoPE
  void *kv;     // [L][2][NKV][max_seq][HD] (f32 or f16)
  float *attp;  // [MAXT][NH][nsplit_max][APS]
  float *ff;    // [MAXT][FF]
  float *logits;  // [MAXT][V]
  float *amv;     // [MAXT][lm_items]
  int *ami;
  int lm_items, lm_rpt, o_rpt, up_rpt, dn_rpt;
  PassState *st;
  int *hist;      // [max_seq + 1]
  unsigned *bar;  // grid barrier: count, generation
};

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ int skew(int i) { return (i >> 5) * XS + (i & 31); }

__device__ __forceinline__ size_t kv_index(const DecParams &P, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * P.NKV + h) * P.max_seq + pos) * HD;
}

// Normalise m staged raw vectors in place (skewed layout): RMSNorm
// (infer.js:134-143) or LayerNorm (infer.js:147-164, eps 1e-5).
__device__ void norm_staged(const DecParams &P, float *xs, int m, const float *w, float *red) {
  const int D = P.D, ng = D >> 5;
  for (int t = 0; t < m; ++t) {
    float *xt = xs + t * ng * XS;
    if (P.arch == 1) {
      float s = 0.f;
      for (int i = threadIdx.x; i < D; i += WG) s += xt[skew(i)];
      const float mean = block_sum(s, red) / (float)D;
      float v = 0.f;
      for (int i = threadIdx.x; i < D; i += WG) {
        const float d = xt[skew(i)] - mean;
        v = __builtin_fmaf(d, d, v);
      }
      const float inv = 1.0f / sqrtf(block_sum(v, red) / (float)D + 1e-5f);
      for (int i = threadIdx.x; i < D; i += WG) {
        const int k = skew(i);
        xt[k] = __builtin_fmaf((xt[k] - mean) * inv, w[i], w[D + i]);
      }
    } else {
      float s = 0.f;
      for (int i = threadIdx.x; i < D; i += WG) s = __builtin_fmaf(xt[skew(i)], xt[skew(i)], s);
      const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + P.eps);
      for (int i = threadIdx.x; i < D; i += WG) {
        const int k = skew(i);
        xt[k] = xt[k] * inv * w[i];
      }
    }
  }
  __syncthreads();
}

// LDS carve-up shared by the GEMV phases.
struct Lds {
  float *xs, *xsum, *part, *out, *red;
};

__device__ __forceinline__ Lds carve(float *smem, int m, int ng, int out_floats) {
  Lds s;
  s.red = smem;  // 16 floats
  s.xs = smem + 16;
  s.xsum = s.xs + m * ng * XS;
  s.part = s.xsum + m * ng;
  s.out = s.part + m * SUB_CH;
  (void)out_floats;
  return s;
}

// ---------------------------------------------------------------- phases
__device__ void phase_qkv(const DecParams &P, int li, int item, float *smem) {
  const PassState &S = *P.st;
  const int m = S.ntok, D = P.D, ng = D >> 5;
  Lds s = carve(smem, m, ng, m * HD);
  const LayerW &Lw = P.layers[li];
  // stage the residual stream (layer 0: embed it, infer.js:360-420)
  for (int t = 0; t < m; ++t) {
    float *xt = s.xs + t * ng * XS;
    if (li == 0) {
      const int tok = S.tok[t];
      const uint8_t *row = reinterpret_cast<const uint8_t *>(P.lm.q) + (size_t)tok * (D >> 1);
      const float *sc = P.lm.s + (size_t)tok * ng;
      const int pos = min(S.pos0 + t, P.max_seq - 1);
      for (int i = threadIdx.x; i < D; i += WG) {
        const int b = row[i >> 1];
        float v = (float)(((i & 1) ? (b >> 4) : (b & 15)) - 8) * sc[i >> 5];
        if (P.arch == 1) {
          if (P.sf) v = v / P.sf[i];
          v = v + P.wpe[(size_t)pos * D + i];
        }
        xt[skew(i)] = v;
        if (item == 0) P.x[(size_t)t * D + i] = v;
      }
    } else {
      for (int i = threadIdx.x; i < D; i += WG) xt[skew(i)] = P.x[(size_t)t * D + i];
    }
  }
  __syncthreads();
  norm_staged(P, s.xs, m, Lw.n1, s.red);
  stage_group_sums(s.xs, s.xsum, m, ng);
  gemv_q4_rows(Lw.qkv, item * HD, HD, m, s.xs, s.xsum, ng, threadIdx.x % ng, WG % ng, s.part, s.out, HD);
  // epilogue
  const bool is_q = item < P.NH, is_k = !is_q && item < P.NH + P.NKV;
  const int kvh = is_q ? 0 : (is_k ? item - P.NH : item - P.NH - P.NKV);
  const int half = P.rd >> 1;
  for (int e = threadIdx.x; e < m * HD; e += WG) {
    const int t = e / HD, d = e - t * HD;
    float v = s.out[e];
    if (P.arch == 1) {
      v = v + Lw.qkv_b[item * HD + d];
    } else if (!(!is_q && !is_k) && d < P.rd) {
      const int pos = S.pos0 + t;
      const float mate = d < half ? -s.out[t * HD + d + half] : s.out[t * HD + d - half];
      v = __builtin_fmaf(v, P.rope_cos[(size_t)pos * P.rd + d], mate * P.rope_sin[(size_t)pos * P.rd + d]);
    }
    if (is_q) {
      P.q[(size_t)t * P.NH * HD + item * HD + d] = v;
    } else {
      const size_t k = kv_index(P, li, is_k ? 0 : 1, kvh, S.pos0 + t) + d;
      if (P.kv_fp16)
        reinterpret_cast<__half *>(P.kv)[k] = __float2half_rn(v);
      else
        reinterpret_cast<float *>(P.kv)[k] = v;
    }
  }
}

__device__ void phase_attn(const DecParams &P, int li, int item, float *smem) {
  const PassState &S = *P.st;
  const int per_tok = P.NH * P.nsplit_max;
  const int t = item / per_tok;
  const int rem = item - t * per_tok;
  const int sp = rem / P.NH, h = rem - sp * P.NH;
  if (t >= S.ntok) return;
  const int pos = S.pos0 + t;
  const int s0 = sp * ACH;
  if (s0 > pos) return;
  const int cnt = min(ACH, pos + 1 - s0);
  const int kvh = h / (P.NH / P.NKV);
  float *qs = smem;       // 64
  float *es = qs + HD;    // 256
  float *pv = es + ACH;   // 4 x 64
  float *red = pv + 4 * HD;
  if (threadIdx.x < HD) qs[threadIdx.x] = P.q[(size_t)t * P.NH * HD + h * HD + threadIdx.x];
  __syncthreads();
  const size_t kbase = kv_index(P, li, 0, kvh, s0), vbase = kv_index(P, li, 1, kvh, s0);
  float score = -INFINITY;
  const int i = threadIdx.x;
  if (i < cnt) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (P.kv_fp16) {
      const uint4 *kr = reinterpret_cast<const uint4 *>(reinterpret_cast<const __half *>(P.kv) + kbase + (size_t)i * HD);
#pragma unroll
      for (int j = 0; j < HD / 8; ++j) {
        const uint4 u = kr[j];
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        const float2 f2 = __half22float2(hp[2]), f3 = __half22float2(hp[3]);
        a0 = __builtin_fmaf(qs[8 * j + 0], f0.x, a0);
        a1 = __builtin_fmaf(qs[8 * j + 1], f0.y, a1);
        a2 = __builtin_fmaf(qs[8 * j + 2], f1.x, a2);
        a3 = __builtin_fmaf(qs[8 * j + 3], f1.y, a3);
        a0 = __builtin_fmaf(qs[8 * j + 4], f2.x, a0);
        a1 = __builtin_fmaf(qs[8 * j + 5], f2.y, a1);
        a2 = __builtin_fmaf(qs[8 * j + 6], f3.x, a2);
        a3 = __builtin_fmaf(qs[8 * j + 7], f3.y, a3);
      }
    } else {
      const float4 *kr = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(P.kv) + kbase + (size_t)i * HD);
#pragma unroll
      for (int j = 0; j < HD / 4; ++j) {
        const float4 k4 = kr[j];
        a0 = __builtin_fmaf(qs[4 * j + 0], k4.x, a0);
        a1 = __builtin_fmaf(qs[4 * j + 1], k4.y, a1);
        a2 = __builtin_fmaf(qs[4 * j + 2], k4.z, a2);
        a3 = __builtin_fmaf(qs[4 * j + 3], k4.w, a3);
      }
    }
    score = ((a0 + a1) + (a2 + a3)) * P.attn_scale;
  }
  const float mx = block_max(score, red);
  const float e = i < cnt ? expf(score - mx) : 0.f;
  es[i] = e;
  const float l = block_sum(e, red);  // contains the barrier that publishes es[]
  const int d = threadIdx.x & (HD - 1), g4 = threadIdx.x >> 6;
  float acc = 0.f;
  if (P.kv_fp16) {
    const __half *vr = reinterpret_cast<const __half *>(P.kv) + vbase + d;
    for (int k = g4; k < cnt; k += 4) acc = __builtin_fmaf(es[k], __half2float(vr[(size_t)k * HD]), acc);
  } else {
    const float *vr = reinterpret_cast<const float *>(P.kv) + vbase + d;
    for (int k = g4; k < cnt; k += 4) acc = __builtin_fmaf(es[k], vr[(size_t)k * HD], acc);
  }
  pv[g4 * HD + d] = acc;
  __syncthreads();
  float *dst = P.attp + ((size_t)(t * P.NH + h) * P.nsplit_max + sp) * APS;
  if (threadIdx.x < HD) dst[4 + threadIdx.x] = (pv[threadIdx.x] + pv[HD + threadIdx.x]) +
                                               (pv[2 * HD + threadIdx.x] + pv[3 * HD + threadIdx.x]);
  if (threadIdx.x == 0) {
    dst[0] = mx;
    dst[1] = l;
  }
}

__device__ void phase_o(const DecParams &P, int li, int item, float *smem) {
  const PassState &S = *P.st;
  const int m = S.ntok, D = P.D, ng = D >> 5;
  const int row0 = item * P.o_rpt;
  const int nr = min(P.o_rpt, D - row0);
  Lds s = carve(smem, m, ng, m * P.o_rpt);
  // combine the attention splits (flash-decoding merge, splits in order)
  for (int t = 0; t < m; ++t) {
    const int ns = (S.pos0 + t) / ACH + 1;
    for (int e = threadIdx.x; e < D; e += WG) {
      const int h = e >> 6, d = e & 63;
      const float *p = P.attp + (size_t)(t * P.NH + h) * P.nsplit_max * APS;
      float M = p[0];
      for (int k = 1; k < ns; ++k) M = fmaxf(M, p[k * APS]);
      float l = 0.f, a = 0.f;
      for (int k = 0; k < ns; ++k) {
        const float w = expf(p[k * APS] - M);
        l = __builtin_fmaf(p[k * APS + 1], w, l);
        a = __builtin_fmaf(p[k * APS + 4 + d], w, a);
      }
      s.xs[t * ng * XS + skew(e)] = a / l;
    }
  }
  __syncthreads();
  stage_group_sums(s.xs, s.xsum, m, ng);
  const LayerW &Lw = P.layers[li];
  gemv_q4_rows(Lw.proj, row0, nr, m, s.xs, s.xsum, ng, threadIdx.x % ng, WG % ng, s.part, s.out, P.o_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    float y = s.out[t * P.o_rpt + r];
    if (P.arch == 1) y = y + Lw.proj_b[row0 + r];
    float &x = P.x[(size_t)t * D + row0 + r];
    x = x + y;
  }
}

__device__ void phase_up(const DecParams &P, int li, int item, float *smem) {
  const PassState &S = *P.st;
  const int m = S.ntok, D = P.D, ng = D >> 5;
  const int row0 = item * P.up_rpt;
  const int nr = min(P.up_rpt, P.FF - row0);
  Lds s = carve(smem, m, ng, 2 * m * P.up_rpt);
  const LayerW &Lw = P.layers[li];
  for (int t = 0; t < m; ++t)
    for (int i = threadIdx.x; i < D; i += WG) s.xs[t * ng * XS + skew(i)] = P.x[(size_t)t * D + i];
  __syncthreads();
  norm_staged(P, s.xs, m, Lw.n2, s.red);
  stage_group_sums(s.xs, s.xsum, m, ng);
  const int gf = threadIdx.x % ng, gs = WG % ng;
  float *og = s.out, *ou = s.out + m * P.up_rpt;
  gemv_q4_rows(Lw.w1, row0, nr, m, s.xs, s.xsum, ng, gf, gs, s.part, og, P.up_rpt);
  if (P.arch == 1) {
    for (int e = threadIdx.x; e < m * nr; e += WG) {
      const int t = e / nr, r = e - t * nr;
      const float v = og[t * P.up_rpt + r] + Lw.fc_b[row0 + r];
      P.ff[(size_t)t * P.FF + row0 + r] =
          0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    }
    return;
  }
  gemv_q4_rows(Lw.w3, row0, nr, m, s.xs, s.xsum, ng, gf, gs, s.part, ou, P.up_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    const float g = og[t * P.up_rpt + r];
    P.ff[(size_t)t * P.FF + row0 + r] = (g / (1.0f + expf(-g))) * ou[t * P.up_rpt + r];
  }
}

__device__ void phase_down(const DecParams &P, int li, int item, float *smem) {
  const PassState &S = *P.st;
  const int m = S.ntok, D = P.D, ngf = P.FF >> 5;
  const int row0 = item * P.dn_rpt;
  const int nr = min(P.dn_rpt, D - row0);
  Lds s = carve(smem, m, ngf, m * P.dn_rpt);
  const LayerW &Lw = P.layers[li];
  stage_plain(P.ff, P.FF, m, P.FF, s.xs, s.xsum);
  gemv_q4_rows(Lw.w2, row0, nr, m, s.xs, s.xsum, ngf, threadIdx.x % ngf, WG % ngf, s.part, s.out, P.dn_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    float y = s.out[t * P.dn_rpt + r];
    if (P.arch == 1) y = y + Lw.mproj_b[row0 + r];
    float &x = P.x[(size_t)t * D + row0 + r];
    x = x + y;
  }
}

// argmaxGpt2 (infer.js:252-287) adjustment of one logit given the banned and
// recent token lists built in LDS.
__device__ __forceinline__ float gpt2_adjust(float v, int i, const int *ban, int nban, const int *rec, int nrec) {
  for (int k = 0; k < nban; ++k)
    if (ban[k] == i) return -1e9f;
  if (v > -1e8f)
    for (int k = 0; k < nrec; ++k)
      if (rec[k] == i) return v > 0.f ? v / 1.15f : v * 1.15f;
  return v;
}

__device__ void phase_lm(const DecParams &P, int item, float *smem) {
  const PassState &S = *P.st;
  if (S.lm_rows == 0) return;
  const int m_all = S.ntok;
  const int tb = S.lm_rows == 1 ? m_all - 1 : 0;
  const int m = m_all - tb;
  const int D = P.D, ng = D >> 5;
  const int row0 = item * P.lm_rpt;
  const int nr = min(P.lm_rpt, P.V - row0);
  Lds s = carve(smem, m, ng, m * P.lm_rpt);
  int *lists = reinterpret_cast<int *>(s.out + m * P.lm_rpt);  // [0]: nban, [1]: nrec, [2..34): rec, then ban
  const bool penal = P.arch == 1 && S.chain;
  if (penal && threadIdx.x == 0) {
    // infer.js:252-287 over hist[0..n): banned = tokens that would repeat the
    // last 3-gram, recent = the last 32 tokens.
    const int n = S.n_hist;
    int nrec = 0, nban = 0;
    for (int h = max(0, n - 32); h < n; ++h) lists[2 + nrec++] = P.hist[h];
    if (n >= 2) {
      const int t1 = P.hist[n - 2], t2 = P.hist[n - 1];
      for (int h = 0; h < n - 2; ++h)
        if (P.hist[h] == t1 && P.hist[h + 1] == t2) lists[34 + nban++] = P.hist[h + 2];
    }
    lists[0] = nban;
    lists[1] = nrec;
  }
  for (int t = 0; t < m; ++t)
    for (int i = threadIdx.x; i < D; i += WG) s.xs[t * ng * XS + skew(i)] = P.x[(size_t)(tb + t) * D + i];
  __syncthreads();
  norm_staged(P, s.xs, m, P.norm_f, s.red);
  stage_group_sums(s.xs, s.xsum, m, ng);
  gemv_q4_rows(P.lm, row0, nr, m, s.xs, s.xsum, ng, threadIdx.x % ng, WG % ng, s.part, s.out, P.lm_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    P.logits[(size_t)(tb + t) * P.V + row0 + r] = s.out[t * P.lm_rpt + r];
  }
  if (threadIdx.x < 64) {
    const int nban = penal ? lists[0] : 0, nrec = penal ? lists[1] : 0;
    for (int t = 0; t < m; ++t) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int r = threadIdx.x; r < nr; r += 64) {
        float v = s.out[t * P.lm_rpt + r];
        if (penal) v = gpt2_adjust(v, row0 + r, lists + 34, nban, lists + 2, nrec);
        if (amax_better(v, row0 + r, bv, bi)) {
          bv = v;
          bi = row0 + r;
        }
      }
      wave_argmax(bv, bi);
      if (threadIdx.x == 0) {
        P.amv[(size_t)(tb + t) * P.lm_items + item] = bv;
        P.ami[(size_t)(tb + t) * P.lm_items + item] = bi;
      }
    }
  }
}

__device__ void phase_argmax(const DecParams &P, float *smem) {
  PassState &S = *P.st;
  if (S.lm_rows == 0) return;
  const int tb = S.lm_rows == 1 ? S.ntok - 1 : 0;
  float *rv = smem;
  int *ri = reinterpret_cast<int *>(smem + 4);
  for (int t = tb; t < S.ntok; ++t) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int k = threadIdx.x; k < P.lm_items; k += WG) {
      const float v = P.amv[(size_t)t * P.lm_items + k];
      const int i = P.ami[(size_t)t * P.lm_items + k];
      if (amax_better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
    wave_argmax(bv, bi);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      rv[threadIdx.x >> 6] = bv;
      ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = rv[0];
      int i = ri[0];
      for (int w = 1; w < 4; ++w)
        if (amax_better(rv[w], ri[w], v, i)) {
          v = rv[w];
          i = ri[w];
        }
      S.res[t] = i;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && S.chain) {
    const int tok = S.res[S.ntok - 1];
    P.hist[S.n_hist] = tok;
    S.n_hist = S.n_hist + 1;
    S.tok[0] = tok;
    S.pos0 = S.pos0 + 1;
    if (tok == S.eos) S.done = 1;
  }
}

__device__ __forceinline__ int phase_items(const DecParams &P, int ph, int m) {
  switch (ph) {
  case PH_QKV: return P.NH + 2 * P.NKV;
  case PH_ATTN: return m * P.NH * P.nsplit_max;
  case PH_O: return (P.D + P.o_rpt - 1) / P.o_rpt;
  case PH_UP: return (P.FF + P.up_rpt - 1) / P.up_rpt;
  case PH_DOWN: return (P.D + P.dn_rpt - 1) / P.dn_rpt;
  case PH_LM: return P.lm_items;
  default: return 1;
  }
}

__device__ __forceinline__ void run_item(const DecParams &P, int ph, int li, int item, float *smem) {
  switch (ph) {
  case PH_QKV: phase_qkv(P, li, item, smem); break;
  case PH_ATTN: phase_attn(P, li, item, smem); break;
  case PH_O: phase_o(P, li, item, smem); break;
  case PH_UP: phase_up(P, li, item, smem); break;
  case PH_DOWN: phase_down(P, li, item, smem); break;
  case PH_LM: phase_lm(P, item, smem); break;
  default: phase_argmax(P, smem); break;
  }
  __syncthreads();
}

// ---------------------------------------------------------------- kernels
// Mode 1: one kernel per phase (grid = items of that phase).
__global__ __launch_bounds__(WG) void k_phase(DecParams P, int ph, int li) {
  extern __shared__ float4 smem4[];
  if (P.st->done) return;
  run_item(P, ph, li, blockIdx.x, reinterpret_cast<float *>(smem4));
}

// Grid barrier for the persistent kernel: arrival counter + generation word
// at agent scope; the last arriver resets the counter and bumps the
// generation.  The spin is bounded: on time-out it records st->err and every
// later barrier of the launch returns at once, so the grid always drains.
__device__ __forceinline__ void grid_barrier(const DecParams &P, unsigned nblocks, unsigned &gen) {
  __syncthreads();
  if (threadIdx.x == 0) {
    if (__hip_atomic_load(&P.st->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      const unsigned old = __hip_atomic_fetch_add(&P.bar[0], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if (old == nblocks - 1) {
        __hip_atomic_store(&P.bar[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&P.bar[1], gen + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        unsigned spins = 0;
        while (__hip_atomic_load(&P.bar[1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == gen) {
          if (++spins > kSpinLimit) {
            __hip_atomic_store(&P.st->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
    }
    gen += 1;
    __atomic_thread_fence(__ATOMIC_ACQUIRE);
  }
  __syncthreads();
}

// Mode 0: every phase of `steps` passes in one cooperative launch.
__global__ __launch_bounds__(WG) void k_persistent(DecParams P, int steps) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const unsigned nb = gridDim.x;
  unsigned gen = __hip_atomic_load(&P.bar[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int step = 0; step < steps; ++step) {
    if (__hip_atomic_load(&P.st->done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    const int m = P.st->ntok;
    for (int li = 0; li < P.L; ++li) {
      for (int ph = PH_QKV; ph <= PH_DOWN; ++ph) {
        const int n = phase_items(P, ph, m);
        for (int it = blockIdx.x; it < n; it += nb) run_item(P, ph, li, it, smem);
        grid_barrier(P, nb, gen);
      }
    }
    if (P.st->lm_rows) {
      for (int it = blockIdx.x; it < P.lm_items; it += nb) run_item(P, PH_LM, 0, it, smem);
      grid_barrier(P, nb, gen);
      if (blockIdx.x == 0) run_item(P, PH_ARGMAX, 0, 0, smem);
      grid_barrier(P, nb, gen);
    }
  }
}

}  // namespace mllm

// ====================================================================== host
using namespace mllm;

struct mllm_model {
  mllm_config cfg{};
  int device = 0, num_cus = 0;
  hipStream_t stream = nullptr;
  uint8_t *d_payload = nullptr;
  uint64_t payload_bytes = 0;
  LayerW *d_layers = nullptr;
  std::vector<LayerW> layers;
  struct Named {
    std::string name;
    int storage, rows, cols;
    const void *data;
    const float *scale;
  };
  std::vector<Named> tensors;
  float *d_rope_cos = nullptr, *d_rope_sin = nullptr;
  float *d_x = nullptr, *d_q = nullptr, *d_attp = nullptr, *d_ff = nullptr, *d_logits = nullptr, *d_amv = nullptr;
  int *d_ami = nullptr, *d_hist = nullptr;
  void *d_kv = nullptr;
  PassState *d_st = nullptr;
  unsigned *d_bar = nullptr;
  PassState *h_st = nullptr;  // pinned
  float *d_gemv_x = nullptr, *d_gemv_y = nullptr;
  DecParams P{};
  int cache_len = 0;
  int exec_mode = 0;
  int max_pass = 1;
  size_t lds_max = 0;
  int persist_grid = 0;
  uint64_t device_bytes = 0;
  hipGraphExec_t chain_graph = nullptr;
  std::vector<void *> allocs;
};

namespace {

int dev_alloc(mllm_model *M, void **p, size_t bytes) {
  MLLM_HIP(hipMalloc(p, bytes));
  M->allocs.push_back(*p);
  M->device_bytes += bytes;
  return 0;
}

size_t lds_for(const mllm_config &c, int m) {
  // Largest LDS carve over the phases for m tokens (floats).
  const int ngd = c.d_model / 32, ngf = c.d_ff / 32;
  const size_t base = 16;
  auto gemv = [&](int ng, int outf) { return base + (size_t)m * ng * XS + (size_t)m * ng + (size_t)m * SUB_CH + outf; };
  const int rpt_d = SUB_CH / ngd, rpt_f = SUB_CH / ngf;
  size_t f = 0;
  f = std::max(f, gemv(ngd, m * HD));                    // qkv
  f = std::max(f, gemv(ngd, m * rpt_d));                 // o
  f = std::max(f, gemv(ngd, 2 * m * rpt_d));             // up
  f = std::max(f, gemv(ngf, m * rpt_f));                 // down
  f = std::max(f, gemv(ngd, m * rpt_d + 34 + c.max_seq_len));  // lm + argmax lists
  f = std::max(f, (size_t)(HD + ACH + 4 * HD + 16));      // attn
  return f * sizeof(float);
}

const mllm_model::Named *find(const mllm_model *M, const std::string &n) {
  for (auto &t : M->tensors)
    if (t.name == n) return &t;
  return nullptr;
}

int get_q4(mllm_model *M, const std::string &n, int rows, int cols, Q4Mat *out) {
  const auto *t = find(M, n);
  if (!t) return set_error(MLLM_ERR_INVALID, "missing tensor %s", n.c_str());
  if (t->storage != MLLM_Q4)
    return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s: storage %d unsupported by the decode engine (q4 only)",
                     n.c_str(), t->storage);
  if (t->rows != rows || t->cols != cols)
    return set_error(MLLM_ERR_INVALID, "tensor %s has shape [%d,%d], expected [%d,%d]", n.c_str(), t->rows, t->cols,
                     rows, cols);
  if (((uintptr_t)t->data & 15) != 0) return set_error(MLLM_ERR_INVALID, "tensor %s is not 16-byte aligned", n.c_str());
  *out = Q4Mat{reinterpret_cast<const uint4 *>(t->data), t->scale, rows, cols};
  return 0;
}

int get_f32(mllm_model *M, const std::string &n, size_t count, const float **out, bool required = true) {
  const auto *t = find(M, n);
  if (!t) {
    *out = nullptr;
    return required ? set_error(MLLM_ERR_INVALID, "missing tensor %s", n.c_str()) : 0;
  }
  if (t->storage != MLLM_F32 || (size_t)t->rows * t->cols < count)
    return set_error(MLLM_ERR_INVALID, "tensor %s must be f32 with >= %zu elements", n.c_str(), count);
  *out = reinterpret_cast<const float *>(t->data);
  return 0;
}

int upload_state(mllm_model *M) {
  MLLM_HIP(hipMemcpyAsync(M->d_st, M->h_st, sizeof(PassState), hipMemcpyHostToDevice, M->stream));
  return 0;
}

int launch_phase(mllm_model *M, int ph, int li, int m) {
  const DecParams &P = M->P;
  int n = 1;
  switch (ph) {
  case PH_QKV: n = P.NH + 2 * P.NKV; break;
  case PH_ATTN: n = m * P.NH * P.nsplit_max; break;
  case PH_O: n = (P.D + P.o_rpt - 1) / P.o_rpt; break;
  case PH_UP: n = (P.FF + P.up_rpt - 1) / P.up_rpt; break;
  case PH_DOWN: n = (P.D + P.dn_rpt - 1) / P.dn_rpt; break;
  case PH_LM: n = P.lm_items; break;
  default: n = 1;
  }
  hipLaunchKernelGGL(k_phase, dim3(n), dim3(WG), M->lds_max, M->stream, M->P, ph, li);
  MLLM_HIP(hipGetLastError());
  return 0;
}

int enqueue_pass_phases(mllm_model *M, int m, bool lm) {
  for (int li = 0; li < M->cfg.n_layers; ++li)
    for (int ph = PH_QKV; ph <= PH_DOWN; ++ph)
      if (int rc = launch_phase(M, ph, li, m)) return rc;
  if (lm) {
    if (int rc = launch_phase(M, PH_LM, 0, m)) return rc;
    if (int rc = launch_phase(M, PH_ARGMAX, 0, m)) return rc;
  }
  return 0;
}

int launch_persistent(mllm_model *M, int steps) {
  void *args[] = {&M->P, &steps};
  MLLM_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(k_persistent), dim3(M->persist_grid), dim3(WG),
                                      args, M->lds_max, M->stream));
  return 0;
}

int check_device_err(mllm_model *M) {
  int err = 0;
  MLLM_HIP(hipMemcpy(&err, &M->d_st->err, sizeof(int), hipMemcpyDeviceToHost));
  if (err) {
    int zero = 0;
    MLLM_HIP(hipMemcpy(&M->d_st->err, &zero, sizeof(int), hipMemcpyHostToDevice));
    MLLM_HIP(hipMemset(M->d_bar, 0, 2 * sizeof(unsigned)));
    return set_error(MLLM_ERR_DEVICE, "decode kernel grid barrier timed out");
  }
  return 0;
}

// Run one pass of m tokens starting at pos0.  lm_rows: 0 none, 1 last, 2 all.
int run_pass(mllm_model *M, const int32_t *ids, int m, int pos0, int lm_rows) {
  PassState &s = *M->h_st;
  memset(&s, 0, sizeof s);
  s.pos0 = pos0;
  s.ntok = m;
  s.lm_rows = lm_rows;
  s.eos = -1;
  for (int i = 0; i < m; ++i) s.tok[i] = ids[i];
  if (int rc = upload_state(M)) return rc;
  if (M->exec_mode == 0) {
    if (int rc = launch_persistent(M, 1)) return rc;
  } else {
    if (int rc = enqueue_pass_phases(M, m, lm_rows != 0)) return rc;
  }
  MLLM_HIP(hipStreamSynchronize(M->stream));
  return check_device_err(M);
}

int check_ids(const mllm_model *M, const int32_t *ids, int n) {
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= M->cfg.vocab_size)
      return set_error(MLLM_ERR_INVALID, "token id %d out of range [0, %d)", ids[i], M->cfg.vocab_size);
  return 0;
}

std::vector<float> build_rope_table(const mllm_config &c, int hd, bool sin_table, int *rd_out) {
  // infer.js:185-206: inv[i] rounded to f32, freq in fp64, cos/sin rounded to f32.
  int rd = (int)floor(hd * c.rope_pct);
  rd -= rd % 2;
  const int half = rd / 2;
  std::vector<float> inv(half > 0 ? half : 1);
  for (int i = 0; i < half; ++i) inv[i] = (float)(1.0 / pow(c.rope_theta, (2.0 * i) / rd));
  std::vector<float> tab((size_t)c.max_seq_len * (rd > 0 ? rd : 1));
  for (int t = 0; t < c.max_seq_len; ++t)
    for (int i = 0; i < half; ++i) {
      const double f = (double)t * (double)inv[i];
      const float v = sin_table ? (float)sin(f) : (float)cos(f);
      tab[(size_t)t * rd + i] = v;
      tab[(size_t)t * rd + half + i] = v;
    }
  *rd_out = rd;
  return tab;
}

}  // namespace

extern "C" int mllm_model_create(const mllm_config *cfg, const void *payload, uint64_t payload_nbytes,
                                 const mllm_tensor *tensors, int n_tensors, mllm_model **out) {
  MLLM_CHECK(cfg && payload && tensors && out && n_tensors > 0, "null argument");
  *out = nullptr;
  const mllm_config &c = *cfg;
  MLLM_CHECK(c.arch == 0 || c.arch == 1, "arch %d", c.arch);
  MLLM_CHECK(c.n_layers > 0 && c.d_model > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.d_ff > 0 &&
                 c.vocab_size > 0 && c.max_seq_len > 0,
             "invalid config");
  MLLM_CHECK(c.d_model % c.n_heads == 0 && c.n_heads % c.n_kv_heads == 0, "heads do not divide");
  if (c.d_model / c.n_heads != HD)
    return set_error(MLLM_ERR_UNSUPPORTED, "head_dim %d unsupported (64 only)", c.d_model / c.n_heads);
  if (c.d_model % 32 || c.d_ff % 32 || c.d_model > 4096 || c.d_ff > 16384)
    return set_error(MLLM_ERR_UNSUPPORTED, "d_model %d / d_ff %d unsupported", c.d_model, c.d_ff);
  if (c.arch == 1 && c.n_kv_heads != c.n_heads) return set_error(MLLM_ERR_INVALID, "gpt2 needs n_kv_heads == n_heads");

  mllm_model *M = new mllm_model();
  M->cfg = c;
  auto fail = [&](int rc) {
    mllm_model_destroy(M);
    return rc;
  };
  if (hipGetDevice(&M->device) != hipSuccess) return fail(set_error(MLLM_ERR_HIP, "no HIP device"));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, M->device) != hipSuccess) return fail(set_error(MLLM_ERR_HIP, "device props"));
  M->num_cus = prop.multiProcessorCount;
  if (hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "stream create"));

  // weights: the payload as-is (16-byte aligned tensors, PGW1 layout)
  M->payload_bytes = payload_nbytes;
  if (int rc = dev_alloc(M, (void **)&M->d_payload, payload_nbytes)) return fail(rc);
  if (hipMemcpy(M->d_payload, payload, payload_nbytes, hipMemcpyHostToDevice) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "payload upload"));
  for (int i = 0; i < n_tensors; ++i) {
    const mllm_tensor &t = tensors[i];
    if (!t.name) return fail(set_error(MLLM_ERR_INVALID, "tensor %d has no name", i));
    if (t.offset + t.nbytes > payload_nbytes || t.scale_offset + t.scale_nbytes > payload_nbytes)
      return fail(set_error(MLLM_ERR_INVALID, "tensor %s exceeds the payload", t.name));
    const bool scaled = t.storage == MLLM_Q4 || t.storage == MLLM_Q8 || t.storage == MLLM_Q8G32;
    M->tensors.push_back({t.name, t.storage, t.rows, t.cols, M->d_payload + t.offset,
                          scaled ? reinterpret_cast<const float *>(M->d_payload + t.scale_offset) : nullptr});
  }

  const int D = c.d_model, FF = c.d_ff, NH = c.n_heads, NKV = c.n_kv_heads, V = c.vocab_size, L = c.n_layers;
  const int kvd = NKV * HD;
  M->layers.resize(L);
  for (int i = 0; i < L; ++i) {
    LayerW &w = M->layers[i];
    memset(&w, 0, sizeof w);
    const std::string b = "blocks." + std::to_string(i) + ".";
    int rc = get_q4(M, b + "attn.qkv", D + 2 * kvd, D, &w.qkv);
    if (!rc) rc = get_q4(M, b + "attn.proj", D, D, &w.proj);
    if (c.arch == 1) {
      if (!rc) rc = get_q4(M, b + "mlp.fc", FF, D, &w.w1);
      if (!rc) rc = get_q4(M, b + "mlp.proj", D, FF, &w.w2);
      if (!rc) rc = get_f32(M, b + "ln1", 2 * D, &w.n1);
      if (!rc) rc = get_f32(M, b + "ln2", 2 * D, &w.n2);
      if (!rc) rc = get_f32(M, b + "attn.qkv_bias", D + 2 * kvd, &w.qkv_b);
      if (!rc) rc = get_f32(M, b + "attn.proj_bias", D, &w.proj_b);
      if (!rc) rc = get_f32(M, b + "mlp.fc_bias", FF, &w.fc_b);
      if (!rc) rc = get_f32(M, b + "mlp.proj_bias", D, &w.mproj_b);
    } else {
      if (!rc) rc = get_q4(M, b + "mlp.w1", FF, D, &w.w1);
      if (!rc) rc = get_q4(M, b + "mlp.w3", FF, D, &w.w3);
      if (!rc) rc = get_q4(M, b + "mlp.w2", D, FF, &w.w2);
      if (!rc) rc = get_f32(M, b + "norm1", D, &w.n1);
      if (!rc) rc = get_f32(M, b + "norm2", D, &w.n2);
    }
    if (rc) return fail(rc);
  }
  DecParams &P = M->P;
  P.arch = c.arch;
  P.L = L;
  P.D = D;
  P.NH = NH;
  P.NKV = NKV;
  P.FF = FF;
  P.V = V;
  P.max_seq = c.max_seq_len;
  P.kv_fp16 = c.kv_fp16 ? 1 : 0;
  P.eps = c.norm_eps > 0 ? c.norm_eps : 1e-6f;
  P.attn_scale = (float)(1.0 / sqrt((double)HD));
  P.nsplit_max = (c.max_seq_len + ACH - 1) / ACH;
  if (int rc = get_q4(M, "lm_head", V, D, &P.lm)) return fail(rc);
  if (c.arch == 1) {
    int rc = get_f32(M, "ln_f", 2 * D, &P.norm_f);
    if (!rc) rc = get_f32(M, "wpe", (size_t)c.max_seq_len * D, &P.wpe);
    if (!rc) rc = get_f32(M, "scale_factors", D, &P.sf, false);
    if (rc) return fail(rc);
  } else {
    if (int rc = get_f32(M, "norm_f", D, &P.norm_f)) return fail(rc);
  }
  if (c.arch == 0) {
    int rd = 0;
    std::vector<float> cs = build_rope_table(c, HD, false, &rd), sn = build_rope_table(c, HD, true, &rd);
    P.rd = rd;
    if (int rc = dev_alloc(M, (void **)&M->d_rope_cos, cs.size() * 4)) return fail(rc);
    if (int rc = dev_alloc(M, (void **)&M->d_rope_sin, sn.size() * 4)) return fail(rc);
    if (hipMemcpy(M->d_rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(M->d_rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return fail(set_error(MLLM_ERR_HIP, "rope upload"));
    P.rope_cos = M->d_rope_cos;
    P.rope_sin = M->d_rope_sin;
  }
  if (int rc = dev_alloc(M, (void **)&M->d_layers, sizeof(LayerW) * L)) return fail(rc);
  if (hipMemcpy(M->d_layers, M->layers.data(), sizeof(LayerW) * L, hipMemcpyHostToDevice) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "layer table upload"));
  P.layers = M->d_layers;

  // tiles
  const int ngd = D / 32, ngf = FF / 32;
  P.o_rpt = std::max(1, SUB_CH / ngd);
  P.up_rpt = std::max(1, SUB_CH / ngd);
  P.dn_rpt = std::max(1, SUB_CH / ngf);
  P.lm_rpt = std::max(1, SUB_CH / ngd);
  P.lm_items = (V + P.lm_rpt - 1) / P.lm_rpt;

  // pass size bound by LDS (160 KiB on gfx950)
  const size_t lds_cap = (size_t)prop.sharedMemPerBlock > 0 ? (size_t)prop.sharedMemPerBlock : 65536;
  int mp = 1;
  while (mp < MAXT && lds_for(c, mp + 1) <= lds_cap) ++mp;
  M->max_pass = mp;
  M->lds_max = lds_for(c, mp);
  if (M->lds_max > lds_cap) return fail(set_error(MLLM_ERR_UNSUPPORTED, "model needs more LDS than the device has"));

  // activations, KV cache, scratch
  const size_t kv_elems = (size_t)L * 2 * NKV * c.max_seq_len * HD;
  int rc = dev_alloc(M, (void **)&M->d_x, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_q, sizeof(float) * MAXT * NH * HD);
  if (!rc) rc = dev_alloc(M, &M->d_kv, kv_elems * (c.kv_fp16 ? 2 : 4));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_attp, sizeof(float) * MAXT * NH * P.nsplit_max * APS);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_ff, sizeof(float) * MAXT * FF);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_logits, sizeof(float) * MAXT * (size_t)V);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_amv, sizeof(float) * MAXT * P.lm_items);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_ami, sizeof(int) * MAXT * P.lm_items);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_hist, sizeof(int) * (c.max_seq_len + 1));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_st, sizeof(PassState));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_bar, 64);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_x, sizeof(float) * std::max(FF, D) * 4);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_y, sizeof(float) * std::max((size_t)V, (size_t)std::max(FF, D + 2 * kvd)));
  if (rc) return fail(rc);
  if (hipHostMalloc((void **)&M->h_st, sizeof(PassState), hipHostMallocDefault) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "pinned state"));
  if (hipMemset(M->d_bar, 0, 64) != hipSuccess || hipMemset(M->d_st, 0, sizeof(PassState)) != hipSuccess ||
      hipMemset(M->d_kv, 0, kv_elems * (c.kv_fp16 ? 2 : 4)) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "memset"));
  P.x = M->d_x;
  P.q = M->d_q;
  P.kv = M->d_kv;
  P.attp = M->d_attp;
  P.ff = M->d_ff;
  P.logits = M->d_logits;
  P.amv = M->d_amv;
  P.ami = M->d_ami;
  P.hist = M->d_hist;
  P.st = M->d_st;
  P.bar = M->d_bar;

  if (M->lds_max > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(k_persistent), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)M->lds_max) != hipSuccess ||
        hipFuncSetAttribute(reinterpret_cast<const void *>(k_phase), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)M->lds_max) != hipSuccess)
      return fail(set_error(MLLM_ERR_HIP, "LDS attribute"));
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_persistent), WG,
                                                   M->lds_max) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  M->persist_grid = M->num_cus * std::min(per_cu, 1);
  *out = M;
  clear_error();
  return 0;
}

extern "C" int mllm_model_destroy(mllm_model *M) {
  if (!M) return 0;
  if (M->stream) hipStreamSynchronize(M->stream);
  if (M->chain_graph) hipGraphExecDestroy(M->chain_graph);
  for (void *p : M->allocs) hipFree(p);
  if (M->h_st) hipHostFree(M->h_st);
  if (M->stream) hipStreamDestroy(M->stream);
  delete M;
  return 0;
}

extern "C" int mllm_reset_cache(mllm_model *M) {
  MLLM_CHECK(M, "null model");
  M->cache_len = 0;
  return 0;
}

extern "C" int mllm_cache_len(const mllm_model *M) { return M ? M->cache_len : -1; }

extern "C" int mllm_set_cache_len(mllm_model *M, int len) {
  MLLM_CHECK(M, "null model");
  MLLM_CHECK(len >= 0 && len <= M->cfg.max_seq_len, "cache length %d out of range", len);
  M->cache_len = len;
  return 0;
}

extern "C" int mllm_max_pass_tokens(const mllm_model *M) { return M ? M->max_pass : 0; }

extern "C" int mllm_set_exec_mode(mllm_model *M, int mode) {
  MLLM_CHECK(M, "null model");
  MLLM_CHECK(mode == 0 || mode == 1, "exec mode %d", mode);
  M->exec_mode = mode;
  return 0;
}

extern "C" uint64_t mllm_model_device_bytes(const mllm_model *M) { return M ? M->device_bytes : 0; }

static int fetch_outputs(mllm_model *M, int row, int nrows, float *logits, int32_t *argmax) {
  if (logits)
    MLLM_HIP(hipMemcpy(logits, M->d_logits + (size_t)row * M->cfg.vocab_size,
                       sizeof(float) * (size_t)nrows * M->cfg.vocab_size, hipMemcpyDeviceToHost));
  if (argmax) MLLM_HIP(hipMemcpy(argmax, &M->d_st->res[row], sizeof(int32_t) * nrows, hipMemcpyDeviceToHost));
  return 0;
}

extern "C" int mllm_forward_prompt(mllm_model *M, const int32_t *ids, int n, float *logits, int32_t *argmax) {
  MLLM_CHECK(M && ids, "null argument");
  MLLM_CHECK(n > 0 && n <= M->cfg.max_seq_len, "prompt length %d out of range", n);
  if (int rc = check_ids(M, ids, n)) return rc;
  int last_rows = 0;
  for (int p0 = 0; p0 < n; p0 += M->max_pass) {
    const int m = std::min(M->max_pass, n - p0);
    const bool last = p0 + m == n;
    if (int rc = run_pass(M, ids + p0, m, p0, last ? 1 : 0)) return rc;
    last_rows = m;
  }
  M->cache_len = n;
  return fetch_outputs(M, last_rows - 1, 1, logits, argmax);
}

extern "C" int mllm_forward_decode(mllm_model *M, int32_t id, float *logits, int32_t *argmax) {
  MLLM_CHECK(M, "null model");
  MLLM_CHECK(M->cache_len < M->cfg.max_seq_len, "KV cache full (%d)", M->cache_len);
  if (int rc = check_ids(M, &id, 1)) return rc;
  if (int rc = run_pass(M, &id, 1, M->cache_len, 1)) return rc;
  M->cache_len += 1;
  return fetch_outputs(M, 0, 1, logits, argmax);
}

extern "C" int mllm_forward_verify(mllm_model *M, const int32_t *ids, int n, int32_t *argmax, float *logits) {
  MLLM_CHECK(M && ids, "null argument");
  MLLM_CHECK(n > 0 && n <= M->max_pass, "verify length %d out of range [1, %d]", n, M->max_pass);
  MLLM_CHECK(M->cache_len + n <= M->cfg.max_seq_len, "verify pass exceeds the context");
  if (int rc = check_ids(M, ids, n)) return rc;
  if (int rc = run_pass(M, ids, n, M->cache_len, 2)) return rc;
  M->cache_len += n;
  return fetch_outputs(M, 0, n, logits, argmax);
}

extern "C" int mllm_decode_chain(mllm_model *M, int32_t first, int n_steps, int32_t eos_id, const int32_t *hist,
                                 int n_hist, int32_t *out_ids, int *n_out) {
  MLLM_CHECK(M && out_ids && n_out, "null argument");
  MLLM_CHECK(n_steps > 0, "n_steps %d", n_steps);
  MLLM_CHECK(M->cache_len + n_steps <= M->cfg.max_seq_len, "chain exceeds the context");
  MLLM_CHECK(n_hist >= 0 && n_hist + n_steps <= M->cfg.max_seq_len, "history too long");
  MLLM_CHECK(n_hist == 0 || hist, "null history");
  if (int rc = check_ids(M, &first, 1)) return rc;
  if (n_hist) MLLM_HIP(hipMemcpyAsync(M->d_hist, hist, sizeof(int32_t) * n_hist, hipMemcpyHostToDevice, M->stream));
  PassState &s = *M->h_st;
  memset(&s, 0, sizeof s);
  s.pos0 = M->cache_len;
  s.ntok = 1;
  s.lm_rows = 1;
  s.chain = 1;
  s.eos = eos_id;
  s.n_hist = n_hist;
  s.tok[0] = first;
  if (int rc = upload_state(M)) return rc;
  if (M->exec_mode == 0) {
    if (int rc = launch_persistent(M, n_steps)) return rc;
  } else {
    if (!M->chain_graph) {
      hipGraph_t g;
      MLLM_HIP(hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal));
      int rc = enqueue_pass_phases(M, 1, true);
      hipError_t e = hipStreamEndCapture(M->stream, &g);
      if (rc) return rc;
      MLLM_HIP(e);
      e = hipGraphInstantiate(&M->chain_graph, g, nullptr, nullptr, 0);
      hipGraphDestroy(g);
      MLLM_HIP(e);
    }
    for (int i = 0; i < n_steps; ++i) MLLM_HIP(hipGraphLaunch(M->chain_graph, M->stream));
  }
  MLLM_HIP(hipStreamSynchronize(M->stream));
  if (int rc = check_device_err(M)) return rc;
  MLLM_HIP(hipMemcpy(&s, M->d_st, sizeof(PassState), hipMemcpyDeviceToHost));
  const int emitted = s.n_hist - n_hist;
  MLLM_HIP(hipMemcpy(out_ids, M->d_hist + n_hist, sizeof(int32_t) * emitted, hipMemcpyDeviceToHost));
  *n_out = emitted;
  M->cache_len += emitted;
  return 0;
}

extern "C" int mllm_model_gemv(mllm_model *M, const char *name, const float *x, float *y) {
  MLLM_CHECK(M && name && x && y, "null argument");
  const auto *t = find(M, name);
  if (!t) return set_error(MLLM_ERR_INVALID, "missing tensor %s", name);
  MLLM_CHECK(t->rows >= 1 && t->cols >= 1, "tensor %s is not a matrix", name);
  const size_t xin = sizeof(float) * std::max(M->cfg.d_ff, M->cfg.d_model) * 4;
  const size_t yout = sizeof(float) * std::max((size_t)M->cfg.vocab_size,
                                               (size_t)std::max(M->cfg.d_ff, M->cfg.d_model + 2 * M->cfg.n_kv_heads * HD));
  if (sizeof(float) * t->cols > xin || sizeof(float) * t->rows > yout)
    return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s too large for model.gemv", name);
  MLLM_HIP(hipMemcpy(M->d_gemv_x, x, sizeof(float) * t->cols, hipMemcpyHostToDevice));
  int rc;
  switch (t->storage) {
  case MLLM_Q4:
    rc = mllm_gemv_q4(t->rows, t->cols, (const uint8_t *)t->data, t->scale, 32, M->d_gemv_x, M->d_gemv_y, M->stream);
    break;
  case MLLM_Q8:
    rc = mllm_gemv_q8(t->rows, t->cols, (const int8_t *)t->data, t->scale, M->d_gemv_x, M->d_gemv_y, M->stream);
    break;
  case MLLM_Q8G32:
    rc = mllm_gemv_q8_g32(t->rows, t->cols, (const int8_t *)t->data, t->scale, M->d_gemv_x, M->d_gemv_y, M->stream);
    break;
  case MLLM_F32:
    rc = mllm_gemv_f32(t->rows, t->cols, (const float *)t->data, M->d_gemv_x, M->d_gemv_y, M->stream);
    break;
  default: return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s storage %d", name, t->storage);
  }
  if (rc) return rc;
  MLLM_HIP(hipStreamSynchronize(M->stream));
  MLLM_HIP(hipMemcpy(y, M->d_gemv_y, sizeof(float) * t->rows, hipMemcpyDeviceToHost));
  return 0;
}
