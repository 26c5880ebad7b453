// mllm_engine.hip -- the fused single-token Q4 decode step on MI355X and the
// engine-level C ABI (PetitGPT API of engine/infer.js:289-647).
//
// One decode step = L x [QKV, ATTN, MLP] + FINAL + LM + ARGMAX kernels
// (the graph of engine/infer.js:579-601; the reference GPU runs it as 244
// dispatches, engine/webgpu-metal.js:1242-1322):
//   QKV    16-row tiles of blocks.i.attn.qkv holding RoPE partner rows d, d+32
//          prologue: embed (layer 0) or x = xb + sum of the previous layer's
//          down-projection partials; RMSNorm/LayerNorm in LDS
//          epilogue: bias (gpt2), RoPE (llama), q -> scratch, k/v -> KV cache
//   ATTN   one workgroup per (token, 256-position split, head): scores,
//          split-local softmax statistics and P.V.  The last split of a
//          (token, head) to finish (the only one below 256 positions) merges
//          the splits and multiplies the head's attention output by its
//          64-column slice of attn.proj: a per-head partial of W_o . att.
//   MLP    one workgroup per 64 hidden units: x = xa + sum of the per-head
//          partials (+ proj bias), norm2, gate and up rows of its units ->
//          silu(g)*u (gpt2: fc + bias -> GELU-tanh), then those units'
//          64-column slice of the down projection: a per-chunk partial of
//          W_2 . h
//   FINAL  per token: x = xb + the down partials (+ bias), final norm
//   LM     grid-stride row tiles of the tied lm_head with the next tile's
//          weights in flight; logits + per-tile argmax (gpt2 chain: 3-gram
//          block and repetition penalty of infer.js:252-287)
//   ARGMAX one workgroup: first maximum over tiles; chained decode feeds it
//          back as the next input token (CHAIN_TOK, webgpu-metal.js:609-610).
// The split-K partials are summed by their consumer in a fixed order, so
// every result is deterministic.  Every GEMV issues its weight loads before
// it stages its activations, so the two memory latencies overlap.
//
// Execution: mode 1 (default) replays a HIP graph of one kernel per phase;
// mode 2 launches the same kernels directly.  Both run the same kernels.  (A
// persistent kernel with grid barriers between phases measured slower than
// graph replay here: one barrier over 256 workgroups cost ~17 us against
// ~1.6 us per graph node.)
//
// Every per-token computation (norm, GEMV row, attention split, merge, the
// partial sums, argmax) runs the same instruction sequence whatever the
// number of tokens in the pass, so a row of the multi-token verify pass is
// bit-identical to the single-token decode of that position.
#include <hip/hip_ext.h>
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

#ifndef MLLM_LM_TILES_PER_WG
#define MLLM_LM_TILES_PER_WG 1
#endif

constexpr int HD = 64;     // head dimension of every supported config
constexpr int ACH = 256;   // positions per attention split (one per thread)
constexpr int MAXT = 16;   // tokens per pass (upper bound; LDS sets the real one)
constexpr int APS = 68;    // floats per attention partial: m, l, pad, pad, acc[64]
constexpr int TC = 2;      // chunk registers per thread of an LM tile (TC * WG chunks)
// Threads per workgroup of each phase.  The QKV, MLP and FINAL phases are
// chains of dependent steps (loads, reductions, small GEMVs) inside few
// workgroups: 1024 threads put four waves on every SIMD of the CU, so each
// step's latency is shared out instead of serialised in one wave per SIMD.
constexpr int QT = 1024;   // QKV
constexpr int AT = 1024;   // ATTN: four threads per key of a 256-key split
constexpr int MT = 1024;   // MLP
constexpr int FT = 1024;   // FINAL
constexpr int LT = WG;     // LM, ARGMAX
constexpr int TILE_TARGET = 320;  // chunks per LM tile (~0.15 us of VALU on one CU)
constexpr int QSPLIT = 4;  // QKV tiles per head
constexpr int UNITS = 64;  // hidden units per MLP item (two 32-column groups of mlp.w2)
constexpr int SC = 2;      // chunk registers per thread of an ATTN head slice (SC * AT chunks)
constexpr int MC = 2;      // chunk registers per thread of the MLP tiles and slices (MC * MT chunks)
constexpr int QC = 1;      // chunk registers per thread of a QKV tile (QC * QT chunks)
constexpr int PB = 8;      // partials per block of the fixed-order partial sums
constexpr int NBMAX = 8;   // blocks per partial sum (<= PB * NBMAX partials: heads, 64-unit chunks)

enum Phase { PH_QKV = 0, PH_ATTN, PH_MLP, PH_FINAL, PH_LM, PH_ARGMAX, PH_COUNT };

struct LayerW {
  Q4Mat qkv, proj, w1, w3, w2;  // gpt2: w1 = mlp.fc, w2 = mlp.proj
  const float *n1, *n2;         // RMS gains; gpt2: LayerNorm gamma || beta
  const float *qkv_b, *proj_b, *fc_b, *mproj_b;
  const float *prev_mproj_b;    // gpt2: the previous layer's mlp.proj bias
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
  int err;       // device-side error flag (reported by the next host check)
  int bad_tok;   // ARGMAX found no finite maximum (chain fed token 0 instead)
  int tok[MAXT];
  int res[MAXT];  // argmax per lm row
};

struct DecParams {
  int arch, L, D, NH, NKV, FF, V, max_seq, kv_fp16, nsplit_max, nchunk;
  float eps, attn_scale;
  const LayerW *layers;
  Q4Mat lm;
  const float *norm_f, *wpe, *sf, *rope_cos, *rope_sin;
  const float *last_mproj_b;  // gpt2: mlp.proj bias of the last layer
  float *xa;      // [MAXT][D] residual entering the attention block
  float *xb;      // [MAXT][D] residual entering the MLP block
  float *opart;   // [MAXT][NH][D] per-head partials of W_o . att
  float *dpart;   // [MAXT][nchunk][D] per-chunk partials of W_2 . h
  float *xn;      // [MAXT][D] final-normed rows for the lm_head
  float *q;       // [MAXT][NH*HD] queries after RoPE
  void *kv;       // [L][2][NKV][max_seq][HD] (f32 or f16)
  float *attp;    // [MAXT][NH][nsplit_max][APS]
  unsigned *cnt;  // [MAXT][NH] finished splits of the current layer
  float *logits;  // [MAXT][V]
  float *amv;     // [MAXT][lm_tiles]
  int *ami;
  int lm_rpt, lm_tiles, lm_grid;
  PassState *st;
  int *hist;      // [max_seq + 1]
};

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ int skew(int i) { return (i >> 5) * XS + (i & 31); }

// LDS regions read or written as float4 start on a 16-byte boundary.
__host__ __device__ __forceinline__ size_t al4(size_t n) { return (n + 3) & ~(size_t)3; }

__device__ __forceinline__ size_t kv_index(const DecParams &P, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * P.NKV + h) * P.max_seq + pos) * HD;
}

// Norm gains (and LayerNorm betas) of this thread's elements i = tid + k*NT,
// loaded into registers up front (d_model <= 1024).
template <int NT>
struct Gains {
  static constexpr int K = (1024 + NT - 1) / NT;
  float g[K], b[K];
};

template <int NT>
__device__ __forceinline__ Gains<NT> load_gains(const DecParams &P, const float *w) {
  Gains<NT> G;
#pragma unroll
  for (int k = 0; k < Gains<NT>::K; ++k) {
    const int i = min((int)threadIdx.x + k * NT, P.D - 1);  // branch-free load; lanes past D unused
    G.g[k] = w[i];
    G.b[k] = P.arch == 1 ? w[P.D + i] : 0.f;
  }
  return G;
}

// Block-wide sum of one value per thread (NT threads, <= 16 waves) into
// every thread: each wave reduces its 64 values with DPP, wave 0 folds the
// wave results in order (lanes w < NT/64, DPP row sum), and the total goes
// back through LDS.  red needs 17 floats.
template <int NT>
__device__ __forceinline__ float block_sum_fast(float v, float *red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const float r = row16_sum(v);
  const float w = (readlane_f(r, 0) + readlane_f(r, 16)) + (readlane_f(r, 32) + readlane_f(r, 48));
  if (lane == 0) red[wv] = w;
  __syncthreads();
  if (wv == 0) {
    const float t = row16_sum(lane < NT / 64 ? red[lane] : 0.f);
    if (lane == 0) red[16] = t;
  }
  __syncthreads();
  return red[16];
}

// Normalise m staged raw vectors in place (skewed layout) and write their
// group sums xsum[t*ng + g]: RMSNorm (infer.js:134-143) or LayerNorm
// (infer.js:147-164, eps 1e-5).  Thread i owns element i (d_model <= NT);
// the group sums come from the normalised values of each 32-lane half-wave
// (two DPP rows).  1/sqrt is the hardware reciprocal square root.
template <int NT>
__device__ void norm_staged(const DecParams &P, float *xs, float *xsum, float *red, int m, const Gains<NT> &G) {
  static_assert(NT >= 1024, "one element per thread (d_model <= 1024)");
  const int D = P.D, ng = D >> 5, lane = threadIdx.x & 63, i = threadIdx.x;
  const float inv_d = 1.0f / (float)D;
  for (int t = 0; t < m; ++t) {
    float *xt = xs + t * ng * XS;
    const float x = i < D ? xt[skew(i)] : 0.f;
    float y;
    if (P.arch == 1) {
      const float mean = block_sum_fast<NT>(x, red) * inv_d;
      const float d = i < D ? x - mean : 0.f;
      const float var = block_sum_fast<NT>(d * d, red) * inv_d;
      y = __builtin_fmaf(d * __builtin_amdgcn_rsqf(var + 1e-5f), G.g[0], G.b[0]);
    } else {
      const float ss = block_sum_fast<NT>(x * x, red) * inv_d;
      y = x * __builtin_amdgcn_rsqf(ss + P.eps) * G.g[0];
    }
    if (i >= D) y = 0.f;
    if (i < D) xt[skew(i)] = y;
    const float r = row16_sum(y);
    const float ga = readlane_f(r, 0) + readlane_f(r, 16), gb = readlane_f(r, 32) + readlane_f(r, 48);
    if ((lane == 0 || lane == 32) && i < D) xsum[t * ng + (i >> 5)] = lane == 0 ? ga : gb;
    __syncthreads();
  }
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Residual rows t = t0 .. t0+m-1:
//   x[t] = base[t] + (((B_0 + B_1) + ... + B_{nb-1}) + bias)
// where B_b sums parts[t][p] for p in [b*PB, min(np, (b+1)*PB)) in ascending
// p (from +0).  The rows go to the skewed LDS layout xs[t - t0] and, when
// `out` is set, to out[t].  The order of every addition is fixed by np alone.
// Each thread loads two (block, float4-column) items per round before adding,
// so a round costs one memory latency.  blk needs nb * D floats of LDS.
// The first round of token t0 is loaded by resid_prefetch, which a phase
// calls before it issues its weight loads: loads retire in issue order, so
// activations issued first can be consumed while the weights still stream.
// U items per thread per round: two with 256 threads, one with 1024.
template <int NT>
struct ResidPre {
  static constexpr int U = NT >= 1024 ? 1 : 2;
  float4 v[U][PB];
  float4 xb, bb;
};

// Branch-free loads: an item or partial past the end reads partial 0 of
// column 0 (valid memory) and resid_add leaves it out.
template <int NT, int U>
__device__ __forceinline__ void resid_load(const float4 *pt, int nq, int np, int nitems, int i0, float4 (&v)[U][PB]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int it = i0 + u * NT;
    const int b = it / nq, c = it - b * nq;
#pragma unroll
    for (int k = 0; k < PB; ++k) {
      const int p = b * PB + k;
      const bool ok = it < nitems && p < np;
      v[u][k] = pt[ok ? (size_t)p * nq + c : 0];
    }
  }
}

// The loaded registers are consumed on every lane (only the store is
// conditional): a load consumed inside a divergent branch leaves the
// compiler unsure it has completed, and it then waits for every load in
// flight before the register is reused.
template <int NT, int U>
__device__ __forceinline__ void resid_add(int nq, int np, int nitems, int i0, const float4 (&v)[U][PB], float *blk) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int it = i0 + u * NT;
    const int b = it / nq;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < PB; ++k) {
      const float4 w = v[u][k];
      const bool use = b * PB + k < np;
      a = add4(a, make_float4(use ? w.x : 0.f, use ? w.y : 0.f, use ? w.z : 0.f, use ? w.w : 0.f));
    }
    if (it < nitems) reinterpret_cast<float4 *>(blk)[it] = a;
  }
}

template <int NT>
__device__ __forceinline__ void resid_prefetch(const float *base, const float *parts, int np, const float *bias, int t0,
                                               int D, ResidPre<NT> &R) {
  const int nq = D >> 2, nb = (np + PB - 1) / PB;
  const int q = min((int)threadIdx.x, nq - 1);  // D <= 1024: one float4 column per thread (branch-free)
  R.xb = reinterpret_cast<const float4 *>(base + (size_t)t0 * D)[q];
  // unconditional load (of base itself when there is no bias): a load in a
  // branch leaves the compiler unsure whether it is pending, and it then
  // waits for every load in flight at the next reuse of its register
  R.bb = reinterpret_cast<const float4 *>(bias ? bias : base)[q];
  resid_load<NT, ResidPre<NT>::U>(reinterpret_cast<const float4 *>(parts + (size_t)t0 * np * D), nq, np, nq * nb,
                                  threadIdx.x, R.v);
}

// Block sums of row t (all rounds but the prefetched one when skip_first is
// set), then the row itself: xs[tt] and out[t].
template <int NT>
__device__ __forceinline__ void resid_row(const float *parts, int np, int t, int tt, int D, float4 xb, float4 bb,
                                          bool has_bias, bool skip_first, float *xs, float *out, float *blk) {
  constexpr int U = ResidPre<NT>::U;
  const int nq = D >> 2, ng = D >> 5, nb = (np + PB - 1) / PB, nitems = nq * nb;
  const float4 *pt = reinterpret_cast<const float4 *>(parts + (size_t)t * np * D);
  for (int i0 = threadIdx.x + (skip_first ? U * NT : 0); i0 < nitems; i0 += U * NT) {
    float4 v[U][PB];
    resid_load<NT, U>(pt, nq, np, nitems, i0, v);
    resid_add<NT, U>(nq, np, nitems, i0, v, blk);
  }
  __syncthreads();
  // every lane combines (column clamped), only the stores are conditional:
  // xb and bb are loads and are consumed outside any branch
  const int q = min((int)threadIdx.x, nq - 1);
  const float4 *b4 = reinterpret_cast<const float4 *>(blk);
  float4 s = b4[q];
  // fixed trip count: a runtime loop here made the compiler wait for every
  // load in flight (the weights) before entering it
#pragma unroll
  for (int b = 1; b < NBMAX; ++b)
    if (b < nb) s = add4(s, b4[b * nq + q]);
  if (has_bias) s = add4(s, bb);
  const float4 v = add4(xb, s);
  if ((int)threadIdx.x < nq) {
    const int i = 4 * q;
    *reinterpret_cast<float4 *>(xs + (tt * ng + (i >> 5)) * XS + (i & 31)) = v;
    if (out) reinterpret_cast<float4 *>(out + (size_t)t * D)[q] = v;
  }
  __syncthreads();
}

template <int NT>
__device__ void stage_residual(const float *base, const float *parts, int np, const float *bias, int t0, int m,
                               int D, float *xs, float *out, float *blk, const ResidPre<NT> &R) {
  const int nq = D >> 2, nb = (np + PB - 1) / PB;
  const float4 bb = R.bb;
  // token t0: its first round is in R
  resid_add<NT, ResidPre<NT>::U>(nq, np, nq * nb, threadIdx.x, R.v, blk);
  resid_row<NT>(parts, np, t0, 0, D, R.xb, bb, bias != nullptr, true, xs, out, blk);
  for (int tt = 1; tt < m; ++tt) {
    const int t = t0 + tt;
    const float4 xb = reinterpret_cast<const float4 *>(base + (size_t)t * D)[min((int)threadIdx.x, nq - 1)];
    resid_row<NT>(parts, np, t, tt, D, xb, bb, bias != nullptr, false, xs, out, blk);
  }
}

// One token's GEMV over a row tile held in registers (chunk c = tid + k*NT
// of rows ng groups wide, c < nch): out[r] for r < nch / ng, with the
// arithmetic of tile_compute (bit-identical rows).
template <int C, int NT>
__device__ __forceinline__ void gemv_tok(const TileRegs<C> &R, int nch, int ng, const float *xs, const float *xsum,
                                         float *part, float *out) {
  int g = threadIdx.x % ng;
  const int gstep = NT % ng;
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const int c = threadIdx.x + k * NT;
    if (c < nch) part[c] = (q4_chunk_dot(R.w[k], xs + g * XS) - 8.f * xsum[g]) * R.s[k];
    g += gstep;
    if (g >= ng) g -= ng;
  }
  __syncthreads();
  for (int r = threadIdx.x; r < nch / ng; r += NT) out[r] = row_sum(part + r * ng, ng);
  __syncthreads();
}

// A two-group column slice of a matrix with ng groups per row: chunk
// c = 2r + j (r < rows, j < 2) is row r, group g0 + j.
template <int C, int NT>
__device__ __forceinline__ void slice_load(const Q4Mat &W, int g0, int rows, TileRegs<C> &R) {
  const int ng = W.cols >> 5;
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const int c = min((int)threadIdx.x + k * NT, 2 * rows - 1);  // branch-free; extra lanes unused
    const size_t gc = (size_t)(c >> 1) * ng + g0 + (c & 1);
    R.w[k] = W.q[gc];
    R.s[k] = W.s[gc];
  }
}

// The slice against two staged groups v (skewed, 2 x XS) with sums vsum[2]:
// out[r] = part(group g0) + part(group g0 + 1), the row_sum order of two
// groups.  Neighbouring lanes hold the pair; every lane takes part in the
// shuffle.
template <int C, int NT>
__device__ __forceinline__ void slice_gemv(const TileRegs<C> &R, int rows, const float *v, const float *vsum,
                                           float *out) {
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const int c = threadIdx.x + k * NT;
    const int j = c & 1;
    float p = 0.f;
    if (c < 2 * rows) p = (q4_chunk_dot(R.w[k], v + j * XS) - 8.f * vsum[j]) * R.s[k];
    const float sum = p + lane_xor1(p);
    if (c < 2 * rows && j == 0) out[c >> 1] = sum;
  }
}

// ---------------------------------------------------------------- phases
__device__ void phase_qkv(const DecParams &P, const LayerW &Lw, int m, int li, int item, bool done, float *smem) {
  const int D = P.D, ng = D >> 5;
  const int head = item / QSPLIT, quarter = item - head * QSPLIT;
  const int ra = head * HD + quarter * 8, rb = ra + 32;  // RoPE partners d and d + 32
  const int nch = 16 * ng;
  const PassState &S = *P.st;
  const int pos0 = S.pos0;
  // activations first (the embedding row, or the residual and the previous
  // layer's partials), then the weight tile
  const bool gpt2 = P.arch == 1;
  constexpr int K = Gains<QT>::K;  // elements per thread (d_model <= 1024)
  int bv[K];
  float sv[K], sfv[K], pv4[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    bv[k] = 0;
    sv[k] = 0.f;
    sfv[k] = 1.f;
    pv4[k] = 0.f;
  }
  ResidPre<QT> RP;
  if (li == 0) {
    // embed (infer.js:360-420): dequantised tied lm_head row; gpt2 divides by
    // scale_factors and adds the learned position.  Loads of token 0 here.
    const int tok = min(max(S.tok[0], 0), P.V - 1);  // host and ARGMAX keep it in range
    const uint8_t *row = reinterpret_cast<const uint8_t *>(P.lm.q) + (size_t)tok * (D >> 1);
    const float *sc = P.lm.s + (size_t)tok * ng;
    const int pos = min(pos0, P.max_seq - 1);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int i = min((int)threadIdx.x + k * QT, D - 1);  // branch-free; lanes past D unused
      bv[k] = row[i >> 1];
      sv[k] = sc[i >> 5];
      if (gpt2) {
        sfv[k] = P.sf ? P.sf[i] : 1.f;
        pv4[k] = P.wpe[(size_t)pos * D + i];
      }
    }
  } else {
    resid_prefetch<QT>(P.xb, P.dpart, P.nchunk, gpt2 ? Lw.prev_mproj_b : nullptr, 0, D, RP);
  }
  // loads retire in issue order: everything the prologue reads goes out
  // before the weight tile, so the prologue never waits for the weights
  const Gains<QT> G = load_gains<QT>(P, Lw.n1);
  TileRegs<QC> R;
  tile_load<QC, QT>(Lw.qkv, ra, 8, rb, ng, nch, R);
  if (done) return;  // a chained decode that reached eos: loads only, no stores
  float *red = smem, *xs = red + 20, *xsum = xs + m * ng * XS, *part = xsum + m * ng, *out = part + m * nch;
  float *blk = smem + al4(20 + (size_t)m * ng * XS + m * ng + m * nch + m * 16);
  // this thread's epilogue element (m * 16 <= QT): its RoPE table entries or
  // bias, fetched before the staging so the epilogue does not wait for them
  const bool is_q = head < P.NH, is_k = !is_q && head < P.NH + P.NKV;
  const int e_own = threadIdx.x, t_own = e_own >> 4, r_own = e_own & 15;
  const int d_own = quarter * 8 + (r_own & 7) + (r_own >> 3) * 32;
  // unconditional loads (gpt2: the bias twice; llama: the RoPE tables, also
  // for V rows that do not use them; positions clamped for lanes past m * 16)
  const size_t ri = (size_t)min(pos0 + t_own, P.max_seq - 1) * HD + d_own;
  const float *pc = gpt2 ? Lw.qkv_b + head * HD + d_own : P.rope_cos + ri;
  const float *ps = gpt2 ? pc : P.rope_sin + ri;
  const float c_own = *pc, s_own = *ps;
  const float b_own = c_own;
  if (li == 0) {
    // item 0 writes xa
    for (int t = 0; t < m; ++t) {
      float *xt = xs + t * ng * XS;
      if (t > 0) {
        const int tok = min(max(S.tok[t], 0), P.V - 1);
        const uint8_t *row = reinterpret_cast<const uint8_t *>(P.lm.q) + (size_t)tok * (D >> 1);
        const float *sc = P.lm.s + (size_t)tok * ng;
        const int pos = min(pos0 + t, P.max_seq - 1);
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int i = min((int)threadIdx.x + k * QT, D - 1);
          bv[k] = row[i >> 1];
          sv[k] = sc[i >> 5];
          if (gpt2) {
            sfv[k] = P.sf ? P.sf[i] : 1.f;
            pv4[k] = P.wpe[(size_t)pos * D + i];
          }
        }
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = threadIdx.x + k * QT;
        if (i < D) {
          float v = (float)(((i & 1) ? (bv[k] >> 4) : (bv[k] & 15)) - 8) * sv[k];
          if (gpt2) {
            if (P.sf) v = v / sfv[k];
            v = v + pv4[k];
          }
          xt[skew(i)] = v;
          if (item == 0) P.xa[(size_t)t * D + i] = v;
        }
      }
    }
    __syncthreads();
  } else {
    stage_residual<QT>(P.xb, P.dpart, P.nchunk, gpt2 ? Lw.prev_mproj_b : nullptr, 0, m, D, xs,
                       item == 0 ? P.xa : nullptr, blk, RP);
  }
  norm_staged<QT>(P, xs, xsum, red, m, G);
  tile_compute<QC, QT>(R, 16, ng, nch, m, xs, xsum, threadIdx.x % ng, QT % ng, part, out, 16);
  // epilogue: tile row r < 8 is head dim d = quarter*8 + r, r >= 8 is d + 32
  const int kvh = is_q ? 0 : (is_k ? head - P.NH : head - P.NH - P.NKV);
  if (e_own < m * 16) {
    const int e = e_own, t = t_own, r = r_own, d = d_own;
    float v = out[e];
    const int pos = pos0 + t;
    if (P.arch == 1) {
      v = v + b_own;
    } else if (is_q || is_k) {
      const float mate = r < 8 ? -out[e + 8] : out[e - 8];
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

// One (token, split, head) item, 1024 threads.  Every load of the item (q,
// the K rows, the V rows) is issued at once: the score of key p of the split
// is formed by the four lanes 4p .. 4p+3 (16 dimensions each, joined with
// DPP); thread (kg, d4) owns V[kg + 64j][4*d4 .. 4*d4+3] for j < 4.  The last
// split of (token, head) to finish -- counted in P.cnt; a single split is its
// own last -- merges the splits (flash-decoding merge in split order) and
// writes the head's partial of the attention output projection to P.opart.
__device__ void phase_attn(const DecParams &P, const LayerW &Lw, int m, int li, int item, bool done, float *smem) {
  const int per_tok = P.NH * P.nsplit_max;
  const int t = item / per_tok;
  const int rem = item - t * per_tok;
  const int sp = rem / P.NH, h = rem - sp * P.NH;
  if (t >= m || done) return;
  const int pos = P.st->pos0 + t;
  const int s0 = sp * ACH;
  if (s0 > pos) return;
  const int ns = pos / ACH + 1;
  const bool solo = ns == 1;
  const int D = P.D;
  TileRegs<SC> Ro;
  const int cnt = min(ACH, pos + 1 - s0);
  const int kvh = h / (P.NH / P.NKV);
  float *qs = smem;            // 64
  float *es = qs + HD;         // 256: exp weights
  float *sc = es + ACH;        // 256: scores
  float *pv = sc + ACH;        // 64 x 64
  float *pv2 = pv + 64 * HD;   // 4 x 64
  float *red = pv2 + 4 * HD;   // 16
  float *own = red + 16;       // 64: this split's P.V
  float *att = own + HD;       // 2 x XS: merged head output, skewed
  float *asum = att + 2 * XS;  // 2
  int *flag = reinterpret_cast<int *>(asum + 2);
  const size_t kbase = kv_index(P, li, 0, kvh, s0), vbase = kv_index(P, li, 1, kvh, s0);
  const int kp = threadIdx.x >> 2, ku = threadIdx.x & 3;  // key of the split, quarter of its dimensions
  const int d4 = threadIdx.x & 15, kg = threadIdx.x >> 4;
  float4 kr[4];
  float4 vr[4];
  if (threadIdx.x < HD) qs[threadIdx.x] = P.q[(size_t)t * P.NH * HD + h * HD + threadIdx.x];
  // K/V loads only for keys below cnt (at short contexts most lanes have
  // none; duplicated clamped loads measured slower here)
  if (P.kv_fp16) {
    const __half *kvh16 = reinterpret_cast<const __half *>(P.kv);
    if (kp < cnt) {
      const uint4 *row = reinterpret_cast<const uint4 *>(kvh16 + kbase + (size_t)kp * HD + 16 * ku);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint4 u = row[j];
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        const float2 f2 = __half22float2(hp[2]), f3 = __half22float2(hp[3]);
        kr[2 * j] = make_float4(f0.x, f0.y, f1.x, f1.y);
        kr[2 * j + 1] = make_float4(f2.x, f2.y, f3.x, f3.y);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = kg + 64 * j;
      if (k < cnt) {
        const uint2 u = *reinterpret_cast<const uint2 *>(kvh16 + vbase + (size_t)k * HD + 4 * d4);
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        vr[j] = make_float4(f0.x, f0.y, f1.x, f1.y);
      }
    }
  } else {
    const float *kv32 = reinterpret_cast<const float *>(P.kv);
    if (kp < cnt) {
      const float4 *row = reinterpret_cast<const float4 *>(kv32 + kbase + (size_t)kp * HD + 16 * ku);
#pragma unroll
      for (int j = 0; j < 4; ++j) kr[j] = row[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = kg + 64 * j;
      if (k < cnt) vr[j] = *reinterpret_cast<const float4 *>(kv32 + vbase + (size_t)k * HD + 4 * d4);
    }
  }
  if (solo) slice_load<SC, AT>(Lw.proj, 2 * h, D, Ro);  // W_o columns of this head, behind the K/V loads
  __syncthreads();
  float part = 0.f;
  if (kp < cnt) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    const float *qq = qs + 16 * ku;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a0 = __builtin_fmaf(qq[4 * j + 0], kr[j].x, a0);
      a1 = __builtin_fmaf(qq[4 * j + 1], kr[j].y, a1);
      a2 = __builtin_fmaf(qq[4 * j + 2], kr[j].z, a2);
      a3 = __builtin_fmaf(qq[4 * j + 3], kr[j].w, a3);
    }
    part = (a0 + a1) + (a2 + a3);
  }
  // the four quarters: (q0 + q1) + (q2 + q3) in every lane of the quad
  part = part + dpp_f<0xB1>(part);
  part = part + dpp_f<0x4E>(part);
  const float score = kp < cnt ? part * P.attn_scale : -INFINITY;
  // softmax statistics, reduced by every wave itself (no cross-wave
  // exchange): the scores, then the weights, go through LDS once each
  const int lane = threadIdx.x & 63;
  if (ku == 0) sc[kp] = score;
  __syncthreads();
  float ml = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) ml = fmaxf(ml, sc[lane + 64 * j]);  // -inf past cnt
  const float mx = wave_max(ml);
  const float e = kp < cnt ? expf(score - mx) : 0.f;
  if (ku == 0) es[kp] = e;
  __syncthreads();
  float ll = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ll += es[lane + 64 * j];
  const float l = wave_sum(ll);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = kg + 64 * j;
    if (k < cnt) {
      const float ek = es[k];
      acc.x = __builtin_fmaf(ek, vr[j].x, acc.x);
      acc.y = __builtin_fmaf(ek, vr[j].y, acc.y);
      acc.z = __builtin_fmaf(ek, vr[j].z, acc.z);
      acc.w = __builtin_fmaf(ek, vr[j].w, acc.w);
    }
  }
  *reinterpret_cast<float4 *>(pv + kg * HD + 4 * d4) = acc;
  __syncthreads();
  if (threadIdx.x < 4 * HD) {  // key groups 16q .. 16q+15 of dimension d
    const int d = threadIdx.x & (HD - 1), q = threadIdx.x >> 6;
    float a = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) a += pv[(16 * q + g) * HD + d];
    pv2[q * HD + d] = a;
  }
  __syncthreads();
  if (threadIdx.x < HD) own[threadIdx.x] = (pv2[threadIdx.x] + pv2[HD + threadIdx.x]) +
                                           (pv2[2 * HD + threadIdx.x] + pv2[3 * HD + threadIdx.x]);
  const float *parts = P.attp + (size_t)(t * P.NH + h) * P.nsplit_max * APS;
  if (!solo) {
    // publish this split, then count it; the last one merges
    float *dst = P.attp + ((size_t)(t * P.NH + h) * P.nsplit_max + sp) * APS;
    __syncthreads();
    if (threadIdx.x < HD) dst[4 + threadIdx.x] = own[threadIdx.x];
    if (threadIdx.x == 0) {
      dst[0] = mx;
      dst[1] = l;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned *c = P.cnt + t * P.NH + h;
      const unsigned arrived = atomicAdd(c, 1u);
      flag[0] = arrived == (unsigned)(ns - 1);
      if (flag[0]) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!flag[0]) return;
    __threadfence();
    slice_load<SC, AT>(Lw.proj, 2 * h, D, Ro);
  }
  __syncthreads();
  if (threadIdx.x < HD) {
    const int d = threadIdx.x;
    float v;
    if (solo) {
      v = own[d] / l;  // the merge below with one split: weight expf(0) = 1
    } else {
      float M = sp == 0 ? mx : parts[0];
      for (int j = 1; j < ns; ++j) M = fmaxf(M, j == sp ? mx : parts[j * APS]);
      const float m0 = sp == 0 ? mx : parts[0], l0 = sp == 0 ? l : parts[1], a0 = sp == 0 ? own[d] : parts[4 + d];
      const float w0 = expf(m0 - M);
      float ls = __builtin_fmaf(l0, w0, 0.f), as = __builtin_fmaf(a0, w0, 0.f);
      for (int j = 1; j < ns; ++j) {
        const float mj = j == sp ? mx : parts[j * APS];
        const float lj = j == sp ? l : parts[j * APS + 1];
        const float aj = j == sp ? own[d] : parts[j * APS + 4 + d];
        const float w = expf(mj - M);
        ls = __builtin_fmaf(lj, w, ls);
        as = __builtin_fmaf(aj, w, as);
      }
      v = as / ls;
    }
    att[skew(d)] = v;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) s += att[threadIdx.x * XS + k];
    asum[threadIdx.x] = s;
  }
  __syncthreads();
  slice_gemv<SC, AT>(Ro, D, att, asum, P.opart + (size_t)(t * P.NH + h) * D);
}

// Hidden units [item*UNITS, (item+1)*UNITS): gate/up (or fc) rows, the
// activation, then the units' two-group slice of the down projection.
__device__ void phase_mlp(const DecParams &P, const LayerW &Lw, int m, int item, bool done, float *smem) {
  const int D = P.D, ng = D >> 5;
  const bool gpt2 = P.arch == 1;
  const int r0 = item * UNITS;
  const int nch = UNITS * ng;
  ResidPre<MT> RP;
  resid_prefetch<MT>(P.xa, P.opart, P.NH, gpt2 ? Lw.proj_b : nullptr, 0, D, RP);
  const Gains<MT> G = load_gains<MT>(P, Lw.n2);  // before the weights (loads retire in issue order)
  // gate/up chunk c = tid + j*S (S = (MT / ng) * ng): every chunk of a thread
  // is group tid % ng, so its activations are read from LDS once
  const int S = (MT / ng) * ng;
  TileRegs<MC> Rg, Ru, Rd;
  tile_load_strided<MC>(Lw.w1, r0, UNITS, ng, S, Rg);
  if (!gpt2) tile_load_strided<MC>(Lw.w3, r0, UNITS, ng, S, Ru);
  if (done) return;
  // unconditional load (llama reads its norm gains instead and ignores it)
  const float fcb = (gpt2 ? Lw.fc_b + r0 : Lw.n2)[threadIdx.x & (UNITS - 1)];
  float *red = smem, *xs = red + 20, *xsum = xs + m * ng * XS, *part = xsum + m * ng;  // part: gate || up
  float *hs = smem + al4(20 + (size_t)m * ng * XS + m * ng + 2 * nch);
  float *hsum = hs + m * 2 * XS, *blk = hsum + al4(2 * m);
  stage_residual<MT>(P.xa, P.opart, P.NH, gpt2 ? Lw.proj_b : nullptr, 0, m, D, xs, item == 0 ? P.xb : nullptr, blk,
                     RP);
  norm_staged<MT>(P, xs, xsum, red, m, G);
  slice_load<MC, MT>(Lw.w2, 2 * item, D, Rd);  // needed last: behind everything the prologue reads
  const int g = threadIdx.x % ng;
  for (int t = 0; t < m; ++t) {
    // gate and up chunk partials of this token in one pass (the arithmetic
    // of tile_compute), one barrier, then wave 0 (unit r = lane) forms the
    // rows, the activation and the two group sums of h
    float xr[32];
    load_group(xs + (t * ng + g) * XS, xr);
    const float xsg = 8.f * xsum[t * ng + g];
#pragma unroll
    for (int k = 0; k < MC; ++k) {
      const int c = threadIdx.x + k * S;
      if ((int)threadIdx.x < S && c < nch) {
        float dg, du;
        q4_chunk_dot2_reg(Rg.w[k], gpt2 ? Rg.w[k] : Ru.w[k], xr, dg, du);
        part[c] = (dg - xsg) * Rg.s[k];
        if (!gpt2) part[nch + c] = (du - xsg) * Ru.s[k];
      }
    }
    __syncthreads();
    if (threadIdx.x < UNITS) {  // exactly wave 0
      const int r = threadIdx.x;
      const float gv = row_sum(part + r * ng, ng);
      float h;
      if (gpt2) {
        const float v = gv + fcb;
        h = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
      } else {
        h = (gv / (1.0f + expf(-gv))) * row_sum(part + nch + r * ng, ng);
      }
      hs[t * 2 * XS + skew(r)] = h;
      const float rs = row16_sum(h);
      const float ga = readlane_f(rs, 0) + readlane_f(rs, 16), gb = readlane_f(rs, 32) + readlane_f(rs, 48);
      if (r == 0) hsum[2 * t] = ga;
      if (r == 32) hsum[2 * t + 1] = gb;
    }
    __syncthreads();
  }
  for (int t = 0; t < m; ++t)
    slice_gemv<MC, MT>(Rd, D, hs + t * 2 * XS, hsum + 2 * t, P.dpart + ((size_t)t * P.nchunk + item) * D);
}

// Item t: the residual after the last layer, final norm -> xn[t] (only the
// rows the lm_head reads).
__device__ void phase_final(const DecParams &P, int m, int item, bool done, float *smem) {
  const PassState &S = *P.st;
  if (S.lm_rows == 0 || done) return;
  const int tb = S.lm_rows == 1 ? m - 1 : 0;
  const int t = item;
  if (t < tb || t >= m) return;
  const int D = P.D, ng = D >> 5;
  ResidPre<FT> RP;
  resid_prefetch<FT>(P.xb, P.dpart, P.nchunk, P.arch == 1 ? P.last_mproj_b : nullptr, t, D, RP);
  const Gains<FT> G = load_gains<FT>(P, P.norm_f);
  // red: 20 floats; xsum: ng <= 32 (unused by the lm_head)
  float *red = smem, *xsum = smem + 20, *xs = smem + 52, *blk = xs + ng * XS;
  stage_residual<FT>(P.xb, P.dpart, P.nchunk, P.arch == 1 ? P.last_mproj_b : nullptr, t, 1, D, xs, nullptr, blk, RP);
  norm_staged<FT>(P, xs, xsum, red, 1, G);
  for (int i = threadIdx.x; i < D; i += FT) P.xn[(size_t)t * D + i] = xs[skew(i)];
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

struct LmLds {
  float *xs, *xsum, *part, *out;
  int *lists;
};

// One lm_head tile whose weights are in R: logits rows [r0, r0+nr) of the m
// tokens from tb, then the tile's first maximum per token (gpt2 chain: with
// the argmaxGpt2 adjustments).
__device__ __forceinline__ void lm_tile(const DecParams &P, const TileRegs<TC> &R, int tile, int tb, int m,
                                        const LmLds &s, bool penal, int nban, int nrec) {
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
        if (penal) v = gpt2_adjust(v, r0 + r, s.lists + 34, nban, s.lists + 2, nrec);
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
__device__ void phase_lm(const DecParams &P, int m_all, int wg, int nwg, bool done, float *smem) {
  if (wg >= P.lm_tiles) return;
  const PassState &S = *P.st;
  const int lm_rows = S.lm_rows;
  if (lm_rows == 0 || done) return;
  const int tb = lm_rows == 1 ? m_all - 1 : 0;
  const int m = m_all - tb;
  const int D = P.D, ng = D >> 5, rpt = P.lm_rpt;
  // the normed rows first, then the weights (loads retire in issue order)
  float4 xv[4];
  stage_rows_load<LT>(P.xn + (size_t)tb * D, D, m, D, 0, xv);
  TileRegs<TC> Ra, Rb;
  int tile = wg;
  lm_load(P, tile, Ra);
  LmLds s;
  s.xs = smem;
  s.xsum = s.xs + m * ng * XS;
  s.part = s.xsum + m * ng;
  s.out = s.part + m * TC * WG;
  s.lists = reinterpret_cast<int *>(s.out + m * rpt);  // [0]: nban, [1]: nrec, [2..34): rec, then ban
  const bool penal = P.arch == 1 && S.chain;
  if (penal && threadIdx.x == 0) {
    // infer.js:252-287 over hist[0..n): banned = tokens that would repeat the
    // last 3-gram, recent = the last 32 tokens.
    const int n = S.n_hist;
    int nrec = 0, nban = 0;
    for (int h = max(0, n - 32); h < n; ++h) s.lists[2 + nrec++] = P.hist[h];
    if (n >= 2) {
      const int t1 = P.hist[n - 2], t2 = P.hist[n - 1];
      for (int h = 0; h < n - 2; ++h)
        if (P.hist[h] == t1 && P.hist[h + 1] == t2) s.lists[34 + nban++] = P.hist[h + 2];
    }
    s.lists[0] = nban;
    s.lists[1] = nrec;
  }
  stage_rows_store<LT>(m, D, 0, xv, s.xs);
  stage_rows<LT>(P.xn + (size_t)tb * D, D, m, D, s.xs, 4 * LT);
  __syncthreads();
  stage_group_sums(s.xs, s.xsum, m, ng);
  const int nban = penal ? s.lists[0] : 0, nrec = penal ? s.lists[1] : 0;
  while (tile < P.lm_tiles) {
    lm_load(P, tile + nwg, Rb);
    lm_tile(P, Ra, tile, tb, m, s, penal, nban, nrec);
    tile += nwg;
    if (tile >= P.lm_tiles) break;
    lm_load(P, tile + nwg, Ra);
    lm_tile(P, Rb, tile, tb, m, s, penal, nban, nrec);
    tile += nwg;
  }
}

__device__ void phase_argmax(const DecParams &P, bool done, float *smem) {
  PassState &S = *P.st;
  if (S.lm_rows == 0 || done) return;
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
        vv[j] = -INFINITY;
        iv[j] = 0x7fffffff;
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
  case PH_MLP: return P.nchunk;
  case PH_FINAL: return m;
  case PH_LM: return P.lm_grid;
  default: return 1;
  }
}

// done: the chained decode already emitted eos.  Each phase still issues
// its first loads (they do not depend on the pass state, whose load then
// overlaps them) but stores nothing.
__device__ __forceinline__ void run_item(const DecParams &P, const LayerW &Lw, int ph, int m, int li, int item,
                                         int nitems, bool done, float *smem) {
  switch (ph) {
  case PH_QKV: phase_qkv(P, Lw, m, li, item, done, smem); break;
  case PH_ATTN: phase_attn(P, Lw, m, li, item, done, smem); break;
  case PH_MLP: phase_mlp(P, Lw, m, item, done, smem); break;
  case PH_FINAL: phase_final(P, m, item, done, smem); break;
  case PH_LM: phase_lm(P, m, item, nitems, done, smem); break;
  default: phase_argmax(P, done, smem); break;
  }
}

// ---------------------------------------------------------------- kernels
// Modes 1 and 2: one kernel per phase (grid = items of that phase).
// The layer's weight pointers come in as a kernel argument, so the first
// weight loads do not wait for a table lookup.  One symbol per phase so
// profilers report the phases apart.
__host__ __device__ constexpr int phase_threads(int ph) {
  return ph == PH_QKV ? QT : ph == PH_ATTN ? AT : ph == PH_MLP ? MT : ph == PH_FINAL ? FT : LT;
}

// ONE = 1: the single-token instance (m is the constant 1, so the token
// loops vanish); the decode step runs it.  ONE = 0 takes m from the argument.
// Both run the same per-token code.
template <int PH, int ONE>
__global__ __launch_bounds__(phase_threads(PH)) void k_phase(DecParams P, LayerW Lw, int li, int m) {
  extern __shared__ float4 smem4[];
  const bool done = P.st->done != 0;
  run_item(P, Lw, PH, ONE ? 1 : m, li, blockIdx.x, gridDim.x, done, reinterpret_cast<float *>(smem4));
}

using PhaseKernel = void (*)(DecParams, LayerW, int, int);
static const PhaseKernel kPhaseKernels[2][PH_COUNT] = {
    {k_phase<PH_QKV, 0>, k_phase<PH_ATTN, 0>, k_phase<PH_MLP, 0>, k_phase<PH_FINAL, 0>, k_phase<PH_LM, 0>,
     k_phase<PH_ARGMAX, 0>},
    {k_phase<PH_QKV, 1>, k_phase<PH_ATTN, 1>, k_phase<PH_MLP, 1>, k_phase<PH_FINAL, 1>, k_phase<PH_LM, 1>,
     k_phase<PH_ARGMAX, 1>}};
static const char *const kPhaseNames[PH_COUNT] = {"QKV", "ATTN", "MLP", "FINAL", "LM", "ARGMAX"};

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
  float *d_logits = nullptr;
  int *d_hist = nullptr;
  PassState *d_st = nullptr;
  PassState *h_st = nullptr;  // pinned
  float *d_gemv_x = nullptr, *d_gemv_y = nullptr;
  DecParams P{};
  int cache_len = 0;
  int exec_mode = 1;
  int max_pass = 1;
  size_t lds_max = 0;
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

// LM tile rows: about TILE_TARGET chunks, at most TC * WG.
int lm_tile_rows(int ng) { return std::max(1, std::min(TILE_TARGET, TC * WG) / ng); }

// Dynamic LDS floats of each phase for a pass of m tokens (the carve-ups in
// the phase functions).
size_t lds_floats(const DecParams &P, int ph, int m) {
  const size_t ngd = P.D / 32, D = P.D;
  const size_t blk_o = (size_t)((P.NH + PB - 1) / PB) * D, blk_d = (size_t)((P.nchunk + PB - 1) / PB) * D;
  switch (ph) {
  case PH_QKV: return al4(20 + m * ngd * XS + m * ngd + m * 16 * ngd + m * 16) + blk_d;
  case PH_ATTN: return HD + 2 * ACH + 64 * HD + 4 * HD + 16 + HD + 2 * XS + 2 + 4;
  case PH_MLP:
    return al4(20 + m * ngd * XS + m * ngd + 2 * UNITS * ngd) + (size_t)m * 2 * XS + al4(2 * m) + blk_o;
  case PH_FINAL: return 52 + ngd * XS + blk_d;
  case PH_LM: return m * ngd * XS + m * ngd + (size_t)m * TC * WG + (size_t)m * P.lm_rpt + 34 + P.max_seq;
  default: return 16;
  }
}

size_t lds_for(const DecParams &P, int m) {
  size_t f = 0;
  for (int ph = 0; ph < PH_COUNT; ++ph) f = std::max(f, lds_floats(P, ph, m));
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

// f32 tensor of at least `count` elements; `vec4` tensors are read as float4
// and must be 16-byte aligned.
int get_f32(mllm_model *M, const std::string &n, size_t count, const float **out, bool required = true,
            bool vec4 = false) {
  const auto *t = find(M, n);
  if (!t) {
    *out = nullptr;
    return required ? set_error(MLLM_ERR_INVALID, "missing tensor %s", n.c_str()) : 0;
  }
  if (t->storage != MLLM_F32 || (size_t)t->rows * t->cols < count)
    return set_error(MLLM_ERR_INVALID, "tensor %s must be f32 with >= %zu elements", n.c_str(), count);
  if (vec4 && ((uintptr_t)t->data & 15) != 0)
    return set_error(MLLM_ERR_INVALID, "tensor %s is not 16-byte aligned", n.c_str());
  *out = reinterpret_cast<const float *>(t->data);
  return 0;
}

int upload_state(mllm_model *M) {
  MLLM_HIP(hipMemcpyAsync(M->d_st, M->h_st, sizeof(PassState), hipMemcpyHostToDevice, M->stream));
  return 0;
}

// With events e0/e1 the launch goes through hipExtLaunchKernel, which stamps
// the kernel's own begin and end (the same interval a kernel trace reports).
int launch_phase(mllm_model *M, int ph, int li, int m, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr) {
  const int n = phase_items(M->P, ph, m);
  LayerW Lw = ph <= PH_MLP ? M->layers[li] : LayerW{};
  if (e0 && e1) {
    DecParams P = M->P;
    int li_ = li, m_ = m;
    void *args[] = {&P, &Lw, &li_, &m_};
    MLLM_HIP(hipExtLaunchKernel(reinterpret_cast<const void *>(kPhaseKernels[m == 1][ph]), dim3(n),
                                dim3(phase_threads(ph)), args,
                                lds_for(M->P, m), M->stream, e0, e1, 0));
    return 0;
  }
  hipLaunchKernelGGL(kPhaseKernels[m == 1][ph], dim3(n), dim3(phase_threads(ph)), lds_for(M->P, m), M->stream, M->P,
                     Lw, li, m);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// The phases of one pass in order: (phase, layer) pairs.
std::vector<std::pair<int, int>> pass_phases(const mllm_model *M, bool lm) {
  std::vector<std::pair<int, int>> v;
  for (int li = 0; li < M->cfg.n_layers; ++li)
    for (int ph = PH_QKV; ph <= PH_MLP; ++ph) v.emplace_back(ph, li);
  if (lm)
    for (int ph = PH_FINAL; ph <= PH_ARGMAX; ++ph) v.emplace_back(ph, 0);
  return v;
}

// The chained decode step as an explicit graph: one kernel node per phase in
// a linear chain (built with node APIs rather than stream capture).
int build_chain_graph(mllm_model *M) {
  hipGraph_t g;
  MLLM_HIP(hipGraphCreate(&g, 0));
  hipGraphNode_t prev = nullptr;
  const size_t lds = lds_for(M->P, 1);
  int m = 1;
  int rc = 0;
  for (const auto &pl : pass_phases(M, true)) {
    int ph = pl.first, li = pl.second;
    LayerW Lw = ph <= PH_MLP ? M->layers[li] : LayerW{};
    void *args[] = {&M->P, &Lw, &li, &m};
    hipKernelNodeParams kp;
    memset(&kp, 0, sizeof kp);
    kp.func = reinterpret_cast<void *>(kPhaseKernels[1][ph]);
    kp.gridDim = dim3(phase_items(M->P, ph, 1));
    kp.blockDim = dim3(phase_threads(ph));
    kp.sharedMemBytes = (unsigned)lds;
    kp.kernelParams = args;
    hipGraphNode_t node;
    hipError_t e = hipGraphAddKernelNode(&node, g, prev ? &prev : nullptr, prev ? 1 : 0, &kp);
    if (e != hipSuccess) {
      rc = hip_fail(e, "hipGraphAddKernelNode", __FILE__, __LINE__);
      break;
    }
    prev = node;
  }
  if (!rc) {
    hipError_t e = hipGraphInstantiate(&M->chain_graph, g, nullptr, nullptr, 0);
    if (e != hipSuccess) rc = hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
  }
  (void)hipGraphDestroy(g);
  return rc;
}

int enqueue_pass_phases(mllm_model *M, int m, bool lm) {
  for (const auto &pl : pass_phases(M, lm))
    if (int rc = launch_phase(M, pl.first, pl.second, m)) return rc;
  return 0;
}

int check_device_err(mllm_model *M) {
  int err[2] = {0, 0};
  MLLM_HIP(hipMemcpy(err, &M->d_st->err, sizeof(err), hipMemcpyDeviceToHost));
  if (err[0] || err[1]) {
    int zero[2] = {0, 0};
    MLLM_HIP(hipMemcpy(&M->d_st->err, zero, sizeof(zero), hipMemcpyHostToDevice));
    return set_error(MLLM_ERR_DEVICE, err[0] ? "decode kernel reported an error"
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
  if (int rc = enqueue_pass_phases(M, m, lm_rows != 0)) return rc;
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
  if (c.d_model % 32 || c.d_model > 1024)
    return set_error(MLLM_ERR_UNSUPPORTED, "d_model %d unsupported (a multiple of 32, <= 1024)", c.d_model);
  if (c.d_ff % UNITS || c.d_ff > UNITS * PB * NBMAX)
    return set_error(MLLM_ERR_UNSUPPORTED, "d_ff %d unsupported (a multiple of %d, <= %d)", c.d_ff, UNITS,
                     UNITS * PB * NBMAX);
  if (c.n_heads > PB * NBMAX) return set_error(MLLM_ERR_UNSUPPORTED, "n_heads %d > %d", c.n_heads, PB * NBMAX);
  if (c.arch == 1 && c.n_kv_heads != c.n_heads) return set_error(MLLM_ERR_INVALID, "gpt2 needs n_kv_heads == n_heads");
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
      if (!rc) rc = get_f32(M, b + "attn.proj_bias", D, &w.proj_b, true, true);
      if (!rc) rc = get_f32(M, b + "mlp.fc_bias", FF, &w.fc_b);
      if (!rc) rc = get_f32(M, b + "mlp.proj_bias", D, &w.mproj_b, true, true);
      w.prev_mproj_b = i > 0 ? M->layers[i - 1].mproj_b : nullptr;
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
  P.nchunk = FF / UNITS;
  P.eps = c.norm_eps > 0 ? c.norm_eps : 1e-6f;
  P.attn_scale = (float)(1.0 / sqrt((double)HD));
  P.nsplit_max = (c.max_seq_len + ACH - 1) / ACH;
  if (int rc = get_q4(M, "lm_head", V, D, &P.lm)) return fail(rc);
  if (c.arch == 1) {
    int rc = get_f32(M, "ln_f", 2 * D, &P.norm_f);
    if (!rc) rc = get_f32(M, "wpe", (size_t)c.max_seq_len * D, &P.wpe);
    if (!rc) rc = get_f32(M, "scale_factors", D, &P.sf, false);
    if (rc) return fail(rc);
    P.last_mproj_b = M->layers[L - 1].mproj_b;
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

  // tiles: QKV 16 rows x ng <= QC * QT chunks (d_model <= 1024); the MLP
  // tiles and slices fit MC * MT chunks (UNITS x ng and 2 x d_model), an
  // attention head's W_o slice SC * AT chunks
  const int ngd = D / 32;
  P.lm_rpt = lm_tile_rows(ngd);
  P.lm_tiles = (V + P.lm_rpt - 1) / P.lm_rpt;
  // MLLM_LM_TILES_PER_WG = 1: one tile per workgroup, every tile's loads in
  // flight at once; larger values trade workgroups for the register double
  // buffer of phase_lm.
  P.lm_grid = (P.lm_tiles + MLLM_LM_TILES_PER_WG - 1) / MLLM_LM_TILES_PER_WG;
  if (16 * ngd > QC * QT || UNITS * ngd > MC * ((MT / ngd) * ngd) || 2 * D > MC * MT || 2 * D > SC * AT ||
      16 * ngd > TC * LT)
    return fail(set_error(MLLM_ERR_UNSUPPORTED, "tiles exceed the chunk registers (d_model %d)", D));

  // pass size bound by LDS (160 KiB on gfx950)
  const size_t lds_cap = (size_t)prop.sharedMemPerBlock > 0 ? (size_t)prop.sharedMemPerBlock : 65536;
  int mp = 1;
  while (mp < MAXT && lds_for(P, mp + 1) <= lds_cap) ++mp;
  M->max_pass = mp;
  M->lds_max = lds_for(P, mp);
  if (M->lds_max > lds_cap) return fail(set_error(MLLM_ERR_UNSUPPORTED, "model needs more LDS than the device has"));

  // activations, KV cache, scratch
  const size_t kv_elems = (size_t)L * 2 * NKV * c.max_seq_len * HD;
  int rc = dev_alloc(M, (void **)&P.xa, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.xb, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.opart, sizeof(float) * MAXT * NH * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.dpart, sizeof(float) * MAXT * P.nchunk * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.xn, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.q, sizeof(float) * MAXT * NH * HD);
  if (!rc) rc = dev_alloc(M, &P.kv, kv_elems * (c.kv_fp16 ? 2 : 4));
  if (!rc) rc = dev_alloc(M, (void **)&P.attp, sizeof(float) * MAXT * NH * P.nsplit_max * APS);
  if (!rc) rc = dev_alloc(M, (void **)&P.cnt, sizeof(unsigned) * MAXT * NH);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_logits, sizeof(float) * MAXT * (size_t)V);
  if (!rc) rc = dev_alloc(M, (void **)&P.amv, sizeof(float) * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&P.ami, sizeof(int) * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_hist, sizeof(int) * (c.max_seq_len + 1));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_st, sizeof(PassState));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_x, sizeof(float) * std::max(FF, D) * 4);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_y, sizeof(float) * std::max((size_t)V, (size_t)std::max(FF, D + 2 * kvd)));
  if (rc) return fail(rc);
  if (hipHostMalloc((void **)&M->h_st, sizeof(PassState), hipHostMallocDefault) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "pinned state"));
  if (hipMemset(M->d_st, 0, sizeof(PassState)) != hipSuccess ||
      hipMemset(P.cnt, 0, sizeof(unsigned) * MAXT * NH) != hipSuccess ||
      hipMemset(P.kv, 0, kv_elems * (c.kv_fp16 ? 2 : 4)) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "memset"));
  P.logits = M->d_logits;
  P.hist = M->d_hist;
  P.st = M->d_st;

  if (M->lds_max > 64 * 1024) {
    bool ok = true;
    for (int one = 0; one < 2; ++one)
      for (int ph = 0; ph < PH_COUNT; ++ph)
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void *>(kPhaseKernels[one][ph]),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->lds_max) == hipSuccess;
    if (!ok) return fail(set_error(MLLM_ERR_HIP, "LDS attribute"));
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
  MLLM_CHECK(mode == 1 || mode == 2, "exec mode %d (1: graph replay, 2: direct launches)", mode);
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
  if (M->exec_mode == 2) {
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
  const auto phases = pass_phases(M, true);
  const int per_step = (int)phases.size();
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
    for (int k = 0; k < per_step; ++k)
      if (int rc = launch_phase(M, phases[k].first, phases[k].second, 1, M->prof_ev[2 * k], M->prof_ev[2 * k + 1]))
        return rc;
    MLLM_HIP(hipStreamSynchronize(M->stream));
    for (int k = 0; k < per_step; ++k) {
      float ms = 0;
      MLLM_HIP(hipEventElapsedTime(&ms, M->prof_ev[2 * k], M->prof_ev[2 * k + 1]));
      sum[phases[k].first] += ms;
      cnt[phases[k].first] += 1;
    }
  }
  if (int rc = check_device_err(M)) return rc;
  MLLM_HIP(hipMemcpy(&s, M->d_st, sizeof(PassState), hipMemcpyDeviceToHost));
  M->cache_len += n_steps;
  for (int ph = 0; ph < PH_COUNT; ++ph) phase_us[ph] = cnt[ph] ? (float)(sum[ph] / cnt[ph] * 1000.0) : 0.f;
  return 0;
}

extern "C" const char *mllm_phase_name(int phase) {
  return phase >= 0 && phase < PH_COUNT ? kPhaseNames[phase] : nullptr;
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
