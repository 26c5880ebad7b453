// mllm_engine.hip -- the fused single-token Q4 decode step on MI355X and the
// engine-level C ABI (PetitGPT API of engine/infer.js:289-647).
//
// One decode step = L x [QKV, ATTN, O, UP, DOWN] + LM + ARGMAX phases
// (engine/infer.js:579-601; the reference GPU runs the same graph as 244
// dispatches, engine/webgpu-metal.js:1242-1322):
//   QKV   16-row tiles of blocks.i.attn.qkv holding RoPE partner rows d, d+32
//         prologue: embed (layer 0) or load x; RMSNorm/LayerNorm in LDS
//         epilogue: bias (gpt2), RoPE (llama), q -> scratch, k/v -> KV cache
//   ATTN  (one workgroup per (token, 256-position split, head))
//         scores, split-local softmax statistics and P.V -> partials (m, l, acc)
//   O     prologue: combine the splits -> attention output; epilogue x += W_o.att
//   UP    prologue: norm2; gate and up rows of the same index -> silu(g)*u
//         (gpt2: fc + bias -> GELU-tanh)
//   DOWN  epilogue x += W_2.h (+ bias)
//   LM    prologue: final norm; grid-stride row tiles with the next tile's
//         weights in flight; logits + per-tile argmax (gpt2 chain: 3-gram
//         block and repetition penalty of infer.js:252-287)
//   ARGMAX one workgroup: first maximum over tiles; chained decode feeds it
//         back as the next input token (CHAIN_TOK, webgpu-metal.js:609-610).
// Every GEMV phase issues its weight loads before it stages the activations,
// so the two memory latencies overlap.
//
// Execution: mode 1 (default) replays a HIP graph of one kernel per phase;
// mode 2 launches the same kernels directly; mode 0 runs all phases in one
// persistent cooperative kernel with a grid barrier between phases.  All
// modes run the same per-item device code.
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
constexpr int TC = 2;     // tile capacity of the decode phases: TC * WG chunks
#ifndef MLLM_TILE_TARGET
#define MLLM_TILE_TARGET 320
#endif
#ifndef MLLM_LM_TILES_PER_WG
#define MLLM_LM_TILES_PER_WG 1
#endif
constexpr int TILE_TARGET = MLLM_TILE_TARGET;  // chunks per GEMV tile (~0.15 us of VALU on one CU)
constexpr int QSPLIT = 4;         // QKV tiles per head
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
  int err;       // barrier / flag-wait time-out
  int bad_tok;   // ARGMAX found no finite maximum (chain fed token 0 instead)
  int epoch;     // mode 3: epoch of the launch's first step
  int tok[MAXT];
  int res[MAXT];  // argmax per lm row
};

struct DecParams {
  int arch, L, D, NH, NKV, FF, V, max_seq, kv_fp16, nsplit_max;
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
  float *amv;     // [MAXT][lm_tiles]
  int *ami;
  int o_rpt, up_rpt, dn_rpt, lm_rpt, lm_tiles, lm_grid;
  PassState *st;
  int *hist;      // [max_seq + 1]
  unsigned *bar;  // grid barrier: count, generation
  // mode 3 item flags: per layer [qkv | attn | o | up | down], then lm[grid], argmax
  int *flags;
  int fl_stride, fl_qkv, fl_attn, fl_o, fl_up, fl_down, fl_lm, fl_argmax;
  int n_o, n_up, n_down;
};

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ int skew(int i) { return (i >> 5) * XS + (i & 31); }

__device__ __forceinline__ size_t kv_index(const DecParams &P, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * P.NKV + h) * P.max_seq + pos) * HD;
}

// Norm gains (and LayerNorm betas) of this thread's elements i = tid + k*WG,
// loaded into registers up front (d_model <= 1024).
struct Gains {
  float g[4], b[4];
};

__device__ __forceinline__ Gains load_gains(const DecParams &P, const float *w) {
  Gains G;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = threadIdx.x + k * WG;
    if (i < P.D) {
      G.g[k] = w[i];
      G.b[k] = P.arch == 1 ? w[P.D + i] : 0.f;
    }
  }
  return G;
}

// Normalise m staged raw vectors in place (skewed layout): RMSNorm
// (infer.js:134-143) or LayerNorm (infer.js:147-164, eps 1e-5).
__device__ void norm_staged(const DecParams &P, float *xs, int m, const Gains &G, float *red) {
  const int D = P.D, ng = D >> 5;
  for (int t = 0; t < m; ++t) {
    float *xt = xs + t * ng * XS;
    if (P.arch == 1) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) s += xt[skew(i)];
      }
      const float mean = block_sum(s, red) / (float)D;
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) {
          const float d = xt[skew(i)] - mean;
          v = __builtin_fmaf(d, d, v);
        }
      }
      const float inv = 1.0f / sqrtf(block_sum(v, red) / (float)D + 1e-5f);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) {
          const int j = skew(i);
          xt[j] = __builtin_fmaf((xt[j] - mean) * inv, G.g[k], G.b[k]);
        }
      }
    } else {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) s = __builtin_fmaf(xt[skew(i)], xt[skew(i)], s);
      }
      const float inv = 1.0f / sqrtf(block_sum(s, red) / (float)D + P.eps);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) {
          const int j = skew(i);
          xt[j] = xt[j] * inv * G.g[k];
        }
      }
    }
  }
  __syncthreads();
}

// Stage the residual stream rows [t0, t0+m) of P.x, normalise them with
// the prefetched gains, and form the group sums.
__device__ __forceinline__ void stage_normed(const DecParams &P, int t0, int m, const Gains &G, float *xs,
                                             float *xsum, float *red) {
  const int D = P.D, ng = D >> 5;
  stage_rows(P.x + (size_t)t0 * D, D, m, D, xs);
  __syncthreads();
  norm_staged(P, xs, m, G, red);
  stage_group_sums(xs, xsum, m, ng);
}

// LDS carve-up shared by the GEMV phases (floats):
// red[16] | xs[m][ng][XS] | xsum[m][ng] | part[m][TC*WG] | out[...]
struct Lds {
  float *red, *xs, *xsum, *part, *out;
};

__device__ __forceinline__ Lds carve(float *smem, int m, int ng) {
  Lds s;
  s.red = smem;
  s.xs = smem + 16;
  s.xsum = s.xs + m * ng * XS;
  s.part = s.xsum + m * ng;
  s.out = s.part + m * TC * WG;
  return s;
}

// ---------------------------------------------------------------- dataflow
// Mode 3 orders work items with per-item completion flags instead of kernel
// boundaries or grid barriers.  An item's flag holds the epoch (step number)
// it last completed; a consumer waits until every producer flag it depends on
// (up to three contiguous ranges) has reached the current epoch.  Wave 0
// polls with agent-scope loads and takes an acquire fence; the producer
// publishes with an agent-scope release store after a workgroup barrier.
// Waits are bounded: on time-out st->err is set and every later wait of the
// launch returns at once, so the grid always drains.
struct Dep {
  const int *f[3];
  int n[3];
  int ep;
};

__device__ __forceinline__ void dep_wait(const DecParams &P, const Dep &d) {
  if (d.n[0] + d.n[1] + d.n[2] == 0) return;
  if (threadIdx.x < 64) {
    unsigned spins = 0;
    for (;;) {
      bool ok = true;
#pragma unroll
      for (int r = 0; r < 3; ++r)
        for (int k = threadIdx.x; k < d.n[r]; k += 64)
          ok &= __hip_atomic_load(d.f[r] + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= d.ep;
      if (__all(ok)) break;
      if (++spins > kSpinLimit || __hip_atomic_load(&P.st->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        if (threadIdx.x == 0) __hip_atomic_store(&P.st->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

__device__ __forceinline__ void dep_signal(int *flag, int ep) {
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(flag, ep, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- phases
__device__ void phase_qkv(const DecParams &P, const LayerW &Lw, int m, int li, int item, const Dep &dep,
                          float *smem) {
  const int D = P.D, ng = D >> 5;
  const int head = item / QSPLIT, quarter = item - head * QSPLIT;
  const int ra = head * HD + quarter * 8, rb = ra + 32;  // RoPE partners d and d + 32
  const int nch = 16 * ng;
  TileRegs<TC> R;
  tile_load<TC>(Lw.qkv, ra, 8, rb, ng, nch, R);
  const Gains G = load_gains(P, Lw.n1);
  dep_wait(P, dep);
  Lds s = carve(smem, m, ng);
  const PassState &S = *P.st;
  const int pos0 = S.pos0;
  // this thread's epilogue element (m * 16 <= WG): its RoPE table entries or
  // bias, fetched before the staging so the epilogue does not wait for them
  const bool is_q = head < P.NH, is_k = !is_q && head < P.NH + P.NKV;
  const int e_own = threadIdx.x, t_own = e_own >> 4, r_own = e_own & 15;
  const int d_own = quarter * 8 + (r_own & 7) + (r_own >> 3) * 32;
  float c_own = 0.f, s_own = 0.f, b_own = 0.f;
  if (e_own < m * 16) {
    if (P.arch == 1) {
      b_own = Lw.qkv_b[head * HD + d_own];
    } else if (is_q || is_k) {
      const size_t ri = (size_t)(pos0 + t_own) * HD + d_own;
      c_own = P.rope_cos[ri];
      s_own = P.rope_sin[ri];
    }
  }
  if (li == 0) {
    // embed (infer.js:360-420): dequantised tied lm_head row; gpt2 divides by
    // scale_factors and adds the learned position.  Item 0 writes the residual.
    for (int t = 0; t < m; ++t) {
      float *xt = s.xs + t * ng * XS;
      const int tok = min(max(S.tok[t], 0), P.V - 1);  // host and ARGMAX keep it in range
      const uint8_t *row = reinterpret_cast<const uint8_t *>(P.lm.q) + (size_t)tok * (D >> 1);
      const float *sc = P.lm.s + (size_t)tok * ng;
      const int pos = min(pos0 + t, P.max_seq - 1);
      int bv[4];
      float sv[4], sfv[4], pv4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // D <= 1024: at most 4 elements per thread, loads first
        const int i = threadIdx.x + k * WG;
        if (i < D) {
          bv[k] = row[i >> 1];
          sv[k] = sc[i >> 5];
          if (P.arch == 1) {
            sfv[k] = P.sf ? P.sf[i] : 1.f;
            pv4[k] = P.wpe[(size_t)pos * D + i];
          }
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < D) {
          float v = (float)(((i & 1) ? (bv[k] >> 4) : (bv[k] & 15)) - 8) * sv[k];
          if (P.arch == 1) {
            if (P.sf) v = v / sfv[k];
            v = v + pv4[k];
          }
          xt[skew(i)] = v;
          if (item == 0) P.x[(size_t)t * D + i] = v;
        }
      }
    }
    __syncthreads();
    norm_staged(P, s.xs, m, G, s.red);
    stage_group_sums(s.xs, s.xsum, m, ng);
  } else {
    stage_normed(P, 0, m, G, s.xs, s.xsum, s.red);
  }
  tile_compute<TC>(R, 16, ng, nch, m, s.xs, s.xsum, threadIdx.x % ng, WG % ng, s.part, s.out, 16);
  // epilogue: tile row r < 8 is head dim d = quarter*8 + r, r >= 8 is d + 32
  const int kvh = is_q ? 0 : (is_k ? head - P.NH : head - P.NH - P.NKV);
  if (e_own < m * 16) {
    const int e = e_own, t = t_own, r = r_own, d = d_own;
    float v = s.out[e];
    const int pos = pos0 + t;
    if (P.arch == 1) {
      v = v + b_own;
    } else if (is_q || is_k) {
      const float mate = r < 8 ? -s.out[e + 8] : s.out[e - 8];
      v = __builtin_fmaf(v, c_own, mate * s_own);
    }
    if (is_q) {
      P.q[(size_t)t * P.NH * HD + head * HD + d] = v;
    } else {
      const size_t k = kv_index(P, li, is_k ? 0 : 1, kvh, pos) + d;
      if (P.kv_fp16)
        reinterpret_cast<__half *>(P.kv)[k] = __float2half_rn(v);
      else
        reinterpret_cast<float *>(P.kv)[k] = v;
    }
  }
}

// One (token, split, head) item.  After pos arrives, every load of the item
// (q, the K rows, the V rows) is issued at once: thread i owns key i of the
// split; thread (kg, d4) owns V[kg + 16j][4*d4 .. 4*d4+3] for j < 16.
__device__ void phase_attn(const DecParams &P, int m, int li, int item, const Dep &dep, float *smem) {
  dep_wait(P, dep);
  const int per_tok = P.NH * P.nsplit_max;
  const int t = item / per_tok;
  const int rem = item - t * per_tok;
  const int sp = rem / P.NH, h = rem - sp * P.NH;
  if (t >= m) return;
  const int pos = P.st->pos0 + t;
  const int s0 = sp * ACH;
  if (s0 > pos) return;
  const int cnt = min(ACH, pos + 1 - s0);
  const int kvh = h / (P.NH / P.NKV);
  float *qs = smem;        // 64
  float *es = qs + HD;     // 256
  float *pv = es + ACH;    // 16 x 64
  float *red = pv + 16 * HD;
  const size_t kbase = kv_index(P, li, 0, kvh, s0), vbase = kv_index(P, li, 1, kvh, s0);
  const int i = threadIdx.x;
  const int d4 = threadIdx.x & 15, kg = threadIdx.x >> 4;
  float4 kr[HD / 4];
  float4 vr[16];
  if (threadIdx.x < HD) qs[threadIdx.x] = P.q[(size_t)t * P.NH * HD + h * HD + threadIdx.x];
  if (P.kv_fp16) {
    const __half *kvh16 = reinterpret_cast<const __half *>(P.kv);
    if (i < cnt) {
      const uint4 *row = reinterpret_cast<const uint4 *>(kvh16 + kbase + (size_t)i * HD);
#pragma unroll
      for (int j = 0; j < HD / 8; ++j) {
        const uint4 u = row[j];
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        const float2 f2 = __half22float2(hp[2]), f3 = __half22float2(hp[3]);
        kr[2 * j] = make_float4(f0.x, f0.y, f1.x, f1.y);
        kr[2 * j + 1] = make_float4(f2.x, f2.y, f3.x, f3.y);
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int k = kg + 16 * j;
      if (k < cnt) {
        const uint2 u = *reinterpret_cast<const uint2 *>(kvh16 + vbase + (size_t)k * HD + 4 * d4);
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        vr[j] = make_float4(f0.x, f0.y, f1.x, f1.y);
      }
    }
  } else {
    const float *kv32 = reinterpret_cast<const float *>(P.kv);
    if (i < cnt) {
      const float4 *row = reinterpret_cast<const float4 *>(kv32 + kbase + (size_t)i * HD);
#pragma unroll
      for (int j = 0; j < HD / 4; ++j) kr[j] = row[j];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int k = kg + 16 * j;
      if (k < cnt) vr[j] = *reinterpret_cast<const float4 *>(kv32 + vbase + (size_t)k * HD + 4 * d4);
    }
  }
  __syncthreads();
  float score = -INFINITY;
  if (i < cnt) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      a0 = __builtin_fmaf(qs[4 * j + 0], kr[j].x, a0);
      a1 = __builtin_fmaf(qs[4 * j + 1], kr[j].y, a1);
      a2 = __builtin_fmaf(qs[4 * j + 2], kr[j].z, a2);
      a3 = __builtin_fmaf(qs[4 * j + 3], kr[j].w, a3);
    }
    score = ((a0 + a1) + (a2 + a3)) * P.attn_scale;
  }
  const float mx = block_max(score, red);
  es[i] = i < cnt ? expf(score - mx) : 0.f;
  const float l = block_sum(es[i], red);  // contains the barrier that publishes es[]
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int k = kg + 16 * j;
    if (k < cnt) {
      const float e = es[k];
      acc.x = __builtin_fmaf(e, vr[j].x, acc.x);
      acc.y = __builtin_fmaf(e, vr[j].y, acc.y);
      acc.z = __builtin_fmaf(e, vr[j].z, acc.z);
      acc.w = __builtin_fmaf(e, vr[j].w, acc.w);
    }
  }
  *reinterpret_cast<float4 *>(pv + kg * HD + 4 * d4) = acc;
  __syncthreads();
  float *dst = P.attp + ((size_t)(t * P.NH + h) * P.nsplit_max + sp) * APS;
  if (threadIdx.x < HD) {
    float a = 0.f;
    for (int g = 0; g < 16; ++g) a += pv[g * HD + threadIdx.x];
    dst[4 + threadIdx.x] = a;
  }
  if (threadIdx.x == 0) {
    dst[0] = mx;
    dst[1] = l;
  }
}

__device__ void phase_o(const DecParams &P, const LayerW &Lw, int m, int item, const Dep &dep, float *smem) {
  const int D = P.D, ng = D >> 5;
  const int row0 = item * P.o_rpt;
  const int nr = min(P.o_rpt, D - row0);
  TileRegs<TC> R;
  tile_load<TC>(Lw.proj, row0, nr, 0, ng, nr * ng, R);
  dep_wait(P, dep);
  const int pos0 = P.st->pos0;
  // the residual this thread will update, fetched with the weights
  const int e0 = threadIdx.x;
  const bool own = e0 < m * nr;
  const int et = own ? e0 / nr : 0, er = own ? e0 - et * nr : 0;
  const float xres = own ? P.x[(size_t)et * D + row0 + er] : 0.f;
  const float bres = own && P.arch == 1 ? Lw.proj_b[row0 + er] : 0.f;
  Lds s = carve(smem, m, ng);
  // combine the attention splits (flash-decoding merge, splits in order);
  // split 0's values for this thread's (up to 4) elements are loaded first
  for (int t = 0; t < m; ++t) {
    const int ns = (pos0 + t) / ACH + 1;
    float m0[4], l0[4], a0[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // D <= 1024
      const int e = threadIdx.x + k * WG;
      if (e < D) {
        const float *p = P.attp + (size_t)(t * P.NH + (e >> 6)) * P.nsplit_max * APS;
        m0[k] = p[0];
        l0[k] = p[1];
        a0[k] = p[4 + (e & 63)];
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = threadIdx.x + k * WG;
      if (e < D) {
        const int h = e >> 6, d = e & 63;
        const float *p = P.attp + (size_t)(t * P.NH + h) * P.nsplit_max * APS;
        float M = m0[k];
        for (int j = 1; j < ns; ++j) M = fmaxf(M, p[j * APS]);
        const float w0 = expf(m0[k] - M);
        float l = __builtin_fmaf(l0[k], w0, 0.f), a = __builtin_fmaf(a0[k], w0, 0.f);
        for (int j = 1; j < ns; ++j) {
          const float w = expf(p[j * APS] - M);
          l = __builtin_fmaf(p[j * APS + 1], w, l);
          a = __builtin_fmaf(p[j * APS + 4 + d], w, a);
        }
        s.xs[t * ng * XS + skew(e)] = a / l;
      }
    }
  }
  __syncthreads();
  stage_group_sums(s.xs, s.xsum, m, ng);
  tile_compute<TC>(R, nr, ng, nr * ng, m, s.xs, s.xsum, threadIdx.x % ng, WG % ng, s.part, s.out, P.o_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    float y = s.out[t * P.o_rpt + r];
    if (P.arch == 1) y = y + (e == e0 ? bres : Lw.proj_b[row0 + r]);
    const float x = e == e0 ? xres : P.x[(size_t)t * D + row0 + r];
    P.x[(size_t)t * D + row0 + r] = x + y;
  }
}

__device__ void phase_up(const DecParams &P, const LayerW &Lw, int m, int item, const Dep &dep, float *smem) {
  const int D = P.D, ng = D >> 5;
  const int row0 = item * P.up_rpt;
  const int nr = min(P.up_rpt, P.FF - row0);
  const bool gpt2 = P.arch == 1;
  TileRegs<TC> Rg, Ru;
  tile_load<TC>(Lw.w1, row0, nr, 0, ng, nr * ng, Rg);
  if (!gpt2) tile_load<TC>(Lw.w3, row0, nr, 0, ng, nr * ng, Ru);
  const Gains G = load_gains(P, Lw.n2);
  const bool own = (int)threadIdx.x < m * nr;
  const float fcb = gpt2 && own ? Lw.fc_b[row0 + threadIdx.x % nr] : 0.f;
  dep_wait(P, dep);
  Lds s = carve(smem, m, ng);
  stage_normed(P, 0, m, G, s.xs, s.xsum, s.red);
  const int gf = threadIdx.x % ng, gs = WG % ng;
  float *og = s.out, *ou = s.out + m * P.up_rpt;
  tile_compute<TC>(Rg, nr, ng, nr * ng, m, s.xs, s.xsum, gf, gs, s.part, og, P.up_rpt);
  if (gpt2) {
    for (int e = threadIdx.x; e < m * nr; e += WG) {
      const int t = e / nr, r = e - t * nr;
      const float v = og[t * P.up_rpt + r] + (e == (int)threadIdx.x ? fcb : Lw.fc_b[row0 + r]);
      P.ff[(size_t)t * P.FF + row0 + r] =
          0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    }
    return;
  }
  tile_compute<TC>(Ru, nr, ng, nr * ng, m, s.xs, s.xsum, gf, gs, s.part, ou, P.up_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    const float g = og[t * P.up_rpt + r];
    P.ff[(size_t)t * P.FF + row0 + r] = (g / (1.0f + expf(-g))) * ou[t * P.up_rpt + r];
  }
}

__device__ void phase_down(const DecParams &P, const LayerW &Lw, int m, int item, const Dep &dep, float *smem) {
  const int D = P.D, ngf = P.FF >> 5;
  const int row0 = item * P.dn_rpt;
  const int nr = min(P.dn_rpt, D - row0);
  TileRegs<TC> R;
  tile_load<TC>(Lw.w2, row0, nr, 0, ngf, nr * ngf, R);
  dep_wait(P, dep);
  const int e0 = threadIdx.x;
  const bool own = e0 < m * nr;
  const int et = own ? e0 / nr : 0, er = own ? e0 - et * nr : 0;
  const float xres = own ? P.x[(size_t)et * D + row0 + er] : 0.f;
  const float bres = own && P.arch == 1 ? Lw.mproj_b[row0 + er] : 0.f;
  Lds s = carve(smem, m, ngf);
  stage_plain(P.ff, P.FF, m, P.FF, s.xs, s.xsum);
  tile_compute<TC>(R, nr, ngf, nr * ngf, m, s.xs, s.xsum, threadIdx.x % ngf, WG % ngf, s.part, s.out, P.dn_rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    float y = s.out[t * P.dn_rpt + r];
    if (P.arch == 1) y = y + (e == e0 ? bres : Lw.mproj_b[row0 + r]);
    const float x = e == e0 ? xres : P.x[(size_t)t * D + row0 + r];
    P.x[(size_t)t * D + row0 + r] = x + y;
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

// One lm_head tile whose weights are in R: logits rows [r0, r0+nr) of the m
// tokens from tb, then the tile's first maximum per token (gpt2 chain: with
// the argmaxGpt2 adjustments).
__device__ __forceinline__ void lm_tile(const DecParams &P, const TileRegs<TC> &R, int tile, int tb, int m,
                                        const Lds &s, bool penal, const int *lists, int nban, int nrec) {
  const int ng = P.D >> 5, rpt = P.lm_rpt;
  const int r0 = tile * rpt, nr = min(rpt, P.V - r0);
  tile_compute<TC>(R, nr, ng, nr * ng, m, s.xs, s.xsum, threadIdx.x % ng, WG % ng, s.part, s.out, rpt);
  for (int e = threadIdx.x; e < m * nr; e += WG) {
    const int t = e / nr, r = e - t * nr;
    P.logits[(size_t)(tb + t) * P.V + r0 + r] = s.out[t * rpt + r];
  }
  if (threadIdx.x < 64) {
    for (int t = 0; t < m; ++t) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int r = threadIdx.x; r < nr; r += 64) {
        float v = s.out[t * rpt + r];
        if (penal) v = gpt2_adjust(v, r0 + r, lists + 34, nban, lists + 2, nrec);
        if (amax_better(v, r0 + r, bv, bi)) {
          bv = v;
          bi = r0 + r;
        }
      }
      wave_argmax(bv, bi);
      if (threadIdx.x == 0) {
        P.amv[(size_t)(tb + t) * P.lm_tiles + tile] = bv;
        P.ami[(size_t)(tb + t) * P.lm_tiles + tile] = bi;
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void lm_load(const DecParams &P, int tile, TileRegs<TC> &R) {
  if (tile < P.lm_tiles) {
    const int ng = P.D >> 5, r0 = tile * P.lm_rpt, nr = min(P.lm_rpt, P.V - r0);
    tile_load<TC>(P.lm, r0, nr, 0, ng, nr * ng, R);
  }
}

// lm_head over row tiles wg, wg + nwg, ...; the next tile's weights are
// loaded while the current one is computed (two register sets used in
// turn, each with constant indices so both stay in VGPRs).
__device__ void phase_lm(const DecParams &P, int m_all, int wg, int nwg, const Dep &dep, float *smem) {
  const PassState &S = *P.st;
  const int lm_rows = S.lm_rows;
  if (lm_rows == 0 || wg >= P.lm_tiles) return;
  const int tb = lm_rows == 1 ? m_all - 1 : 0;
  const int m = m_all - tb;
  const int D = P.D, ng = D >> 5, rpt = P.lm_rpt;
  TileRegs<TC> Ra, Rb;
  int tile = wg;
  lm_load(P, tile, Ra);
  const Gains G = load_gains(P, P.norm_f);
  dep_wait(P, dep);
  Lds s = carve(smem, m, ng);
  int *lists = reinterpret_cast<int *>(s.out + m * rpt);  // [0]: nban, [1]: nrec, [2..34): rec, then ban
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
  stage_normed(P, tb, m, G, s.xs, s.xsum, s.red);
  const int nban = penal ? lists[0] : 0, nrec = penal ? lists[1] : 0;
  while (tile < P.lm_tiles) {
    lm_load(P, tile + nwg, Rb);
    lm_tile(P, Ra, tile, tb, m, s, penal, lists, nban, nrec);
    tile += nwg;
    if (tile >= P.lm_tiles) break;
    lm_load(P, tile + nwg, Ra);
    lm_tile(P, Rb, tile, tb, m, s, penal, lists, nban, nrec);
    tile += nwg;
  }
}

__device__ void phase_argmax(const DecParams &P, const Dep &dep, float *smem) {
  dep_wait(P, dep);
  PassState &S = *P.st;
  if (S.lm_rows == 0) return;
  const int tb = S.lm_rows == 1 ? S.ntok - 1 : 0;
  float *rv = smem;
  int *ri = reinterpret_cast<int *>(smem + 4);
  for (int t = tb; t < S.ntok; ++t) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = 0; base < P.lm_tiles; base += 16 * WG) {
      float vv[16];
      int iv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {  // all loads of the batch before any compare
        const int k = base + threadIdx.x + j * WG;
        if (k < P.lm_tiles) {
          vv[j] = P.amv[(size_t)t * P.lm_tiles + k];
          iv[j] = P.ami[(size_t)t * P.lm_tiles + k];
        }
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int k = base + threadIdx.x + j * WG;
        if (k < P.lm_tiles && amax_better(vv[j], iv[j], bv, bi)) {
          bv = vv[j];
          bi = iv[j];
        }
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
    int tok = S.res[S.ntok - 1];
    if (tok < 0 || tok >= P.V) {  // no finite maximum (non-finite logits)
      S.bad_tok = 1;
      tok = 0;
    }
    P.hist[S.n_hist] = tok;
    S.n_hist = S.n_hist + 1;
    S.tok[0] = tok;
    S.pos0 = S.pos0 + 1;
    if (tok == S.eos) S.done = 1;
  }
}

__host__ __device__ __forceinline__ int phase_items(const DecParams &P, int ph, int m) {
  switch (ph) {
  case PH_QKV: return (P.NH + 2 * P.NKV) * QSPLIT;
  case PH_ATTN: return m * P.NH * P.nsplit_max;
  case PH_O: return (P.D + P.o_rpt - 1) / P.o_rpt;
  case PH_UP: return (P.FF + P.up_rpt - 1) / P.up_rpt;
  case PH_DOWN: return (P.D + P.dn_rpt - 1) / P.dn_rpt;
  case PH_LM: return P.lm_grid;
  default: return 1;
  }
}

__device__ __forceinline__ void run_item(const DecParams &P, const LayerW &Lw, int ph, int m, int li, int item,
                                         int nitems, const Dep &dep, float *smem) {
  switch (ph) {
  case PH_QKV: phase_qkv(P, Lw, m, li, item, dep, smem); break;
  case PH_ATTN: phase_attn(P, m, li, item, dep, smem); break;
  case PH_O: phase_o(P, Lw, m, item, dep, smem); break;
  case PH_UP: phase_up(P, Lw, m, item, dep, smem); break;
  case PH_DOWN: phase_down(P, Lw, m, item, dep, smem); break;
  case PH_LM: phase_lm(P, m, item, nitems, dep, smem); break;
  default: phase_argmax(P, dep, smem); break;
  }
  __syncthreads();
}

// ---------------------------------------------------------------- kernels
// Modes 1 and 2: one kernel per phase (grid = items of that phase).
// The layer's weight pointers come in as a kernel argument, so the first
// weight loads do not wait for a table lookup.  One symbol per phase so
// profilers report the phases apart.
template <int PH>
__global__ __launch_bounds__(WG) void k_phase(DecParams P, LayerW Lw, int li, int m) {
  extern __shared__ float4 smem4[];
  if (P.st->done) return;
  const Dep none{};
  run_item(P, Lw, PH, m, li, blockIdx.x, gridDim.x, none, reinterpret_cast<float *>(smem4));
}

using PhaseKernel = void (*)(DecParams, LayerW, int, int);
static const PhaseKernel kPhaseKernels[PH_COUNT] = {k_phase<PH_QKV>, k_phase<PH_ATTN>, k_phase<PH_O>,
                                                    k_phase<PH_UP>,  k_phase<PH_DOWN>, k_phase<PH_LM>,
                                                    k_phase<PH_ARGMAX>};

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
      const LayerW Lw = P.layers[li];
      const Dep none{};
      for (int ph = PH_QKV; ph <= PH_DOWN; ++ph) {
        const int n = phase_items(P, ph, m);
        for (int it = blockIdx.x; it < n; it += nb) run_item(P, Lw, ph, m, li, it, n, none, smem);
        grid_barrier(P, nb, gen);
      }
    }
    if (P.st->lm_rows) {
      const LayerW none{};
      const Dep nodep{};
      run_item(P, none, PH_LM, m, 0, blockIdx.x, nb, nodep, smem);
      grid_barrier(P, nb, gen);
      if (blockIdx.x == 0) run_item(P, none, PH_ARGMAX, m, 0, 0, 1, nodep, smem);
      grid_barrier(P, nb, gen);
    }
  }
}

// Mode 3: every item of `steps` passes in one cooperative launch, ordered by
// per-item flags.  Item dependencies (producer ranges):
//   QKV(l)   <- DOWN(l-1), all items       (layer 0: previous step's ARGMAX)
//   ATTN(l)  <- QKV(l) tiles of the query head, its K head and its V head
//   O(l)     <- ATTN(l), all items of the pass
//   UP(l)    <- O(l);  DOWN(l) <- UP(l);  LM <- DOWN(L-1);  ARGMAX <- LM
// Each workgroup also waits for the previous step's ARGMAX before starting a
// step, so a chain that hit eos is seen by every workgroup at the same step.
__global__ __launch_bounds__(WG) void k_dataflow(DecParams P, int steps) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const int nb = gridDim.x, wg = blockIdx.x;
  const int base = __hip_atomic_load(&P.st->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int *const argmax_flag = P.flags + P.fl_argmax;
  for (int step = 0; step < steps; ++step) {
    const int ep = base + step;
    if (step > 0) {
      const Dep d{{argmax_flag, nullptr, nullptr}, {1, 0, 0}, ep - 1};
      dep_wait(P, d);
      if (__hip_atomic_load(&P.st->done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
    const int m = P.st->ntok;
    const int n_attn = m * P.NH * P.nsplit_max;
    for (int li = 0; li < P.L; ++li) {
      const LayerW Lw = P.layers[li];
      int *const fl = P.flags + (size_t)li * P.fl_stride;
      const int *const prev_down = li > 0 ? fl - P.fl_stride + P.fl_down : nullptr;
      for (int ph = PH_QKV; ph <= PH_DOWN; ++ph) {
        const int n = phase_items(P, ph, m);
        for (int it = wg; it < n; it += nb) {
          Dep d{{nullptr, nullptr, nullptr}, {0, 0, 0}, ep};
          int *mine = nullptr;
          switch (ph) {
          case PH_QKV:
            if (li > 0) {
              d.f[0] = prev_down;
              d.n[0] = P.n_down;
            }
            mine = fl + P.fl_qkv + it;
            break;
          case PH_ATTN: {
            const int h = (it % (P.NH * P.nsplit_max)) % P.NH;
            const int kvh = h / (P.NH / P.NKV);
            d.f[0] = fl + P.fl_qkv + h * QSPLIT;
            d.f[1] = fl + P.fl_qkv + (P.NH + kvh) * QSPLIT;
            d.f[2] = fl + P.fl_qkv + (P.NH + P.NKV + kvh) * QSPLIT;
            d.n[0] = d.n[1] = d.n[2] = QSPLIT;
            mine = fl + P.fl_attn + it;
            break;
          }
          case PH_O:
            d.f[0] = fl + P.fl_attn;
            d.n[0] = n_attn;
            mine = fl + P.fl_o + it;
            break;
          case PH_UP:
            d.f[0] = fl + P.fl_o;
            d.n[0] = P.n_o;
            mine = fl + P.fl_up + it;
            break;
          default:
            d.f[0] = fl + P.fl_up;
            d.n[0] = P.n_up;
            mine = fl + P.fl_down + it;
            break;
          }
          run_item(P, Lw, ph, m, li, it, n, d, smem);
          dep_signal(mine, ep);
        }
      }
    }
    if (P.st->lm_rows) {
      const LayerW none{};
      const Dep dl{{P.flags + (size_t)(P.L - 1) * P.fl_stride + P.fl_down, nullptr, nullptr}, {P.n_down, 0, 0}, ep};
      run_item(P, none, PH_LM, m, 0, wg, nb, dl, smem);
      dep_signal(P.flags + P.fl_lm + wg, ep);
      if (wg == 0) {
        const Dep da{{P.flags + P.fl_lm, nullptr, nullptr}, {nb, 0, 0}, ep};
        run_item(P, none, PH_ARGMAX, m, 0, 0, 1, da, smem);
      }
    }
    if (wg == 0) dep_signal(argmax_flag, ep);
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
  int exec_mode = 1;
  int max_pass = 1;
  size_t lds_max = 0;
  int persist_grid = 0;
  int flow_grid = 0;
  int epoch = 0;  // mode 3: last epoch used
  uint64_t device_bytes = 0;
  hipGraphExec_t chain_graph = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;  // around the kernels of the last call
  std::vector<hipEvent_t> prof_ev;          // mllm_profile_decode
  float last_ms = 0.f;
  int last_tokens = 0;
  std::vector<void *> allocs;
};

namespace {

int dev_alloc(mllm_model *M, void **p, size_t bytes) {
  MLLM_HIP(hipMalloc(p, bytes));
  M->allocs.push_back(*p);
  M->device_bytes += bytes;
  return 0;
}

// Tile rows per item: about TILE_TARGET chunks, at most TC * WG.
int tile_rows(int ng, int per_row_mats = 1) { return std::max(1, TILE_TARGET / (ng * per_row_mats)); }

// Dynamic LDS (bytes) of a pass of m tokens: the largest phase carve.
size_t lds_for(const DecParams &P, int m) {
  const int ngd = P.D / 32, ngf = P.FF / 32;
  auto gemv = [&](int ng, size_t outf) {
    return 16 + (size_t)m * ng * XS + (size_t)m * ng + (size_t)m * TC * WG + outf;
  };
  size_t f = 0;
  f = std::max(f, gemv(ngd, (size_t)m * 16));                                     // qkv
  f = std::max(f, gemv(ngd, (size_t)m * P.o_rpt));                                // o
  f = std::max(f, gemv(ngd, (size_t)2 * m * P.up_rpt));                           // up
  f = std::max(f, gemv(ngf, (size_t)m * P.dn_rpt));                               // down
  f = std::max(f, gemv(ngd, (size_t)m * P.lm_rpt + 34 + (size_t)P.max_seq));     // lm + argmax lists
  f = std::max(f, (size_t)(HD + ACH + 16 * HD + 16));                             // attn
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
  const int n = phase_items(M->P, ph, m);
  const LayerW Lw = ph <= PH_DOWN ? M->layers[li] : LayerW{};
  hipLaunchKernelGGL(kPhaseKernels[ph], dim3(n), dim3(WG), lds_for(M->P, m), M->stream, M->P, Lw, li, m);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// The chained decode step as an explicit graph: one kernel node per phase in
// a linear chain (built with node APIs rather than stream capture).
int build_chain_graph(mllm_model *M) {
  hipGraph_t g;
  MLLM_HIP(hipGraphCreate(&g, 0));
  hipGraphNode_t prev = nullptr;
  const size_t lds = lds_for(M->P, 1);
  int m = 1;
  auto add = [&](int ph, int li) -> int {
    LayerW Lw = ph <= PH_DOWN ? M->layers[li] : LayerW{};
    void *args[] = {&M->P, &Lw, &li, &m};
    hipKernelNodeParams kp;
    memset(&kp, 0, sizeof kp);
    kp.func = reinterpret_cast<void *>(kPhaseKernels[ph]);
    kp.gridDim = dim3(phase_items(M->P, ph, 1));
    kp.blockDim = dim3(WG);
    kp.sharedMemBytes = (unsigned)lds;
    kp.kernelParams = args;
    hipGraphNode_t node;
    MLLM_HIP(hipGraphAddKernelNode(&node, g, prev ? &prev : nullptr, prev ? 1 : 0, &kp));
    prev = node;
    return 0;
  };
  int rc = 0;
  for (int li = 0; li < M->cfg.n_layers && !rc; ++li)
    for (int ph = PH_QKV; ph <= PH_DOWN && !rc; ++ph) rc = add(ph, li);
  if (!rc) rc = add(PH_LM, 0);
  if (!rc) rc = add(PH_ARGMAX, 0);
  if (!rc) {
    hipError_t e = hipGraphInstantiate(&M->chain_graph, g, nullptr, nullptr, 0);
    if (e != hipSuccess) rc = hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
  }
  (void)hipGraphDestroy(g);
  return rc;
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

int launch_dataflow(mllm_model *M, int steps, int m) {
  M->h_st->epoch = M->epoch + 1;
  if (int rc = upload_state(M)) return rc;
  void *args[] = {&M->P, &steps};
  MLLM_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(k_dataflow), dim3(M->flow_grid), dim3(WG), args,
                                      lds_for(M->P, m), M->stream));
  M->epoch += steps;
  return 0;
}

int launch_persistent(mllm_model *M, int steps, int m) {
  void *args[] = {&M->P, &steps};
  MLLM_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(k_persistent), dim3(M->persist_grid), dim3(WG),
                                      args, lds_for(M->P, m), M->stream));
  return 0;
}

int check_device_err(mllm_model *M) {
  int err[2] = {0, 0};
  MLLM_HIP(hipMemcpy(err, &M->d_st->err, sizeof(err), hipMemcpyDeviceToHost));
  if (err[0] || err[1]) {
    int zero[2] = {0, 0};
    MLLM_HIP(hipMemcpy(&M->d_st->err, zero, sizeof(zero), hipMemcpyHostToDevice));
    MLLM_HIP(hipMemset(M->d_bar, 0, 2 * sizeof(unsigned)));
    return set_error(MLLM_ERR_DEVICE, err[0] ? "decode kernel grid barrier timed out"
                                             : "chained decode produced no finite maximum logit");
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
  MLLM_HIP(hipEventRecord(M->ev0, M->stream));
  if (M->exec_mode == 3) {
    if (int rc = launch_dataflow(M, 1, m)) return rc;
  } else if (M->exec_mode == 0) {
    if (int rc = launch_persistent(M, 1, m)) return rc;
  } else {
    if (int rc = enqueue_pass_phases(M, m, lm_rows != 0)) return rc;
  }
  MLLM_HIP(hipEventRecord(M->ev1, M->stream));
  MLLM_HIP(hipStreamSynchronize(M->stream));
  MLLM_HIP(hipEventElapsedTime(&M->last_ms, M->ev0, M->ev1));
  M->last_tokens = m;
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
  if (c.d_model > 1024) return set_error(MLLM_ERR_UNSUPPORTED, "d_model %d unsupported (<= 1024)", c.d_model);
  if (c.arch == 0 && (int)floor(HD * c.rope_pct) != HD)
    return set_error(MLLM_ERR_UNSUPPORTED, "partial rotary (ropePct %g) unsupported", c.rope_pct);

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
  if (hipEventCreate(&M->ev0) != hipSuccess || hipEventCreate(&M->ev1) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "event create"));

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
  P.o_rpt = tile_rows(ngd);
  P.up_rpt = tile_rows(ngd, c.arch == 1 ? 1 : 2);
  P.dn_rpt = tile_rows(ngf);
  P.lm_rpt = tile_rows(ngd);
  P.lm_tiles = (V + P.lm_rpt - 1) / P.lm_rpt;
  // MLLM_LM_TILES_PER_WG = 1: one tile per workgroup, every tile's loads in
  // flight at once; larger values trade workgroups for the register double
  // buffer of phase_lm.
  P.lm_grid = (P.lm_tiles + MLLM_LM_TILES_PER_WG - 1) / MLLM_LM_TILES_PER_WG;
  // every GEMV tile must fit the TC * WG chunk registers of a workgroup
  const int cap = TC * WG;
  if (16 * ngd > cap || P.o_rpt * ngd > cap || P.up_rpt * ngd > cap || P.dn_rpt * ngf > cap || P.lm_rpt * ngd > cap)
    return fail(set_error(MLLM_ERR_UNSUPPORTED, "tile exceeds %d chunks (d_model %d, d_ff %d)", cap, D, FF));

  // pass size bound by LDS (160 KiB on gfx950)
  const size_t lds_cap = (size_t)prop.sharedMemPerBlock > 0 ? (size_t)prop.sharedMemPerBlock : 65536;
  int mp = 1;
  while (mp < MAXT && lds_for(P, mp + 1) <= lds_cap) ++mp;
  M->max_pass = mp;
  M->lds_max = lds_for(P, mp);
  if (M->lds_max > lds_cap) return fail(set_error(MLLM_ERR_UNSUPPORTED, "model needs more LDS than the device has"));

  // activations, KV cache, scratch
  const size_t kv_elems = (size_t)L * 2 * NKV * c.max_seq_len * HD;
  int rc = dev_alloc(M, (void **)&M->d_x, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_q, sizeof(float) * MAXT * NH * HD);
  if (!rc) rc = dev_alloc(M, &M->d_kv, kv_elems * (c.kv_fp16 ? 2 : 4));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_attp, sizeof(float) * MAXT * NH * P.nsplit_max * APS);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_ff, sizeof(float) * MAXT * FF);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_logits, sizeof(float) * MAXT * (size_t)V);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_amv, sizeof(float) * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_ami, sizeof(int) * MAXT * P.lm_tiles);
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
    bool ok = hipFuncSetAttribute(reinterpret_cast<const void *>(k_persistent),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->lds_max) == hipSuccess;
    for (int ph = 0; ph < PH_COUNT; ++ph)
      ok = ok && hipFuncSetAttribute(reinterpret_cast<const void *>(kPhaseKernels[ph]),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->lds_max) == hipSuccess;
    if (!ok) return fail(set_error(MLLM_ERR_HIP, "LDS attribute"));
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_persistent), WG,
                                                   M->lds_max) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  M->persist_grid = M->num_cus * std::min(per_cu, 1);
  {
    bool ok = true;
    if (M->lds_max > 64 * 1024)
      ok = hipFuncSetAttribute(reinterpret_cast<const void *>(k_dataflow), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)M->lds_max) == hipSuccess;
    int fcu = 0;
    if (!ok || hipOccupancyMaxActiveBlocksPerMultiprocessor(&fcu, reinterpret_cast<const void *>(k_dataflow), WG,
                                                             M->lds_max) != hipSuccess || fcu < 1)
      fcu = 1;
    M->flow_grid = M->num_cus * std::min(fcu, 2);
  }
  // mode 3 flags: per layer [qkv | attn | o | up | down], then lm[grid], argmax
  {
    DecParams &Q = M->P;
    const int n_qkv = (Q.NH + 2 * Q.NKV) * QSPLIT;
    Q.n_o = (Q.D + Q.o_rpt - 1) / Q.o_rpt;
    Q.n_up = (Q.FF + Q.up_rpt - 1) / Q.up_rpt;
    Q.n_down = (Q.D + Q.dn_rpt - 1) / Q.dn_rpt;
    Q.fl_qkv = 0;
    Q.fl_attn = n_qkv;
    Q.fl_o = Q.fl_attn + MAXT * Q.NH * Q.nsplit_max;
    Q.fl_up = Q.fl_o + Q.n_o;
    Q.fl_down = Q.fl_up + Q.n_up;
    Q.fl_stride = Q.fl_down + Q.n_down;
    Q.fl_lm = Q.L * Q.fl_stride;
    Q.fl_argmax = Q.fl_lm + M->flow_grid;
    const size_t nflags = (size_t)Q.fl_argmax + 1;
    if (int rc = dev_alloc(M, (void **)&Q.flags, nflags * sizeof(int))) return fail(rc);
    if (hipMemset(Q.flags, 0, nflags * sizeof(int)) != hipSuccess) return fail(set_error(MLLM_ERR_HIP, "memset"));
  }
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
  for (hipEvent_t e : M->prof_ev) (void)hipEventDestroy(e);
  if (M->ev0) hipEventDestroy(M->ev0);
  if (M->ev1) hipEventDestroy(M->ev1);
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
  MLLM_CHECK(mode >= 0 && mode <= 3, "exec mode %d", mode);
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
  MLLM_HIP(hipEventRecord(M->ev0, M->stream));
  if (M->exec_mode == 3) {
    if (int rc = launch_dataflow(M, n_steps, 1)) return rc;
  } else if (M->exec_mode == 0) {
    if (int rc = launch_persistent(M, n_steps, 1)) return rc;
  } else if (M->exec_mode == 2) {
    for (int i = 0; i < n_steps; ++i)
      if (int rc = enqueue_pass_phases(M, 1, true)) return rc;
  } else {
    if (!M->chain_graph)
      if (int rc = build_chain_graph(M)) return rc;
    for (int i = 0; i < n_steps; ++i) MLLM_HIP(hipGraphLaunch(M->chain_graph, M->stream));
  }
  MLLM_HIP(hipEventRecord(M->ev1, M->stream));
  MLLM_HIP(hipStreamSynchronize(M->stream));
  MLLM_HIP(hipEventElapsedTime(&M->last_ms, M->ev0, M->ev1));
  if (int rc = check_device_err(M)) return rc;
  MLLM_HIP(hipMemcpy(&s, M->d_st, sizeof(PassState), hipMemcpyDeviceToHost));
  const int emitted = s.n_hist - n_hist;
  MLLM_HIP(hipMemcpy(out_ids, M->d_hist + n_hist, sizeof(int32_t) * emitted, hipMemcpyDeviceToHost));
  *n_out = emitted;
  M->last_tokens = emitted;
  M->cache_len += emitted;
  return 0;
}

extern "C" int mllm_profile_decode(mllm_model *M, int32_t first, int n_steps, float *phase_us) {
  MLLM_CHECK(M && phase_us, "null argument");
  MLLM_CHECK(n_steps > 0, "n_steps %d", n_steps);
  MLLM_CHECK(M->cache_len + n_steps <= M->cfg.max_seq_len, "profile run exceeds the context");
  if (int rc = check_ids(M, &first, 1)) return rc;
  const int L = M->cfg.n_layers;
  const int per_step = L * 5 + 2;
  if ((int)M->prof_ev.size() < 2 * per_step) {
    for (hipEvent_t e : M->prof_ev) (void)hipEventDestroy(e);
    M->prof_ev.assign(2 * per_step, nullptr);
    for (auto &e : M->prof_ev) MLLM_HIP(hipEventCreate(&e));
  }
  PassState &s = *M->h_st;
  memset(&s, 0, sizeof s);
  s.pos0 = M->cache_len;
  s.ntok = 1;
  s.lm_rows = 1;
  s.chain = 1;
  s.eos = -1;
  s.tok[0] = first;
  if (int rc = upload_state(M)) return rc;
  double sum[PH_COUNT] = {0};
  int cnt[PH_COUNT] = {0};
  for (int step = 0; step < n_steps; ++step) {
    int k = 0;
    std::vector<int> phs;
    for (int li = 0; li < L; ++li)
      for (int ph = PH_QKV; ph <= PH_DOWN; ++ph, ++k) {
        MLLM_HIP(hipEventRecord(M->prof_ev[2 * k], M->stream));
        if (int rc = launch_phase(M, ph, li, 1)) return rc;
        MLLM_HIP(hipEventRecord(M->prof_ev[2 * k + 1], M->stream));
        phs.push_back(ph);
      }
    for (int ph = PH_LM; ph <= PH_ARGMAX; ++ph, ++k) {
      MLLM_HIP(hipEventRecord(M->prof_ev[2 * k], M->stream));
      if (int rc = launch_phase(M, ph, 0, 1)) return rc;
      MLLM_HIP(hipEventRecord(M->prof_ev[2 * k + 1], M->stream));
      phs.push_back(ph);
    }
    MLLM_HIP(hipStreamSynchronize(M->stream));
    for (int j = 0; j < k; ++j) {
      float ms = 0;
      MLLM_HIP(hipEventElapsedTime(&ms, M->prof_ev[2 * j], M->prof_ev[2 * j + 1]));
      sum[phs[j]] += ms;
      cnt[phs[j]] += 1;
    }
  }
  if (int rc = check_device_err(M)) return rc;
  MLLM_HIP(hipMemcpy(&s, M->d_st, sizeof(PassState), hipMemcpyDeviceToHost));
  M->cache_len += n_steps;
  for (int ph = 0; ph < PH_COUNT; ++ph) phase_us[ph] = cnt[ph] ? (float)(sum[ph] / cnt[ph] * 1000.0) : 0.f;
  return 0;
}

extern "C" int mllm_last_timing(const mllm_model *M, float *gpu_ms, int *n_tokens) {
  MLLM_CHECK(M, "null model");
  if (gpu_ms) *gpu_ms = M->last_ms;
  if (n_tokens) *n_tokens = M->last_tokens;
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
