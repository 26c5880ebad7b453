// mllm_engine.hip -- the fused single-token Q4 decode step on MI355X and the
// engine-level C ABI (PetitGPT API of engine/infer.js:289-647).
//
// One decode step = L x [QKV, ATTN, MLP] + FINAL + LM + ARGMAX (the graph
// of engine/infer.js:579-601; the reference GPU runs it as 244 dispatches,
// engine/webgpu-metal.js:1242-1322):
//   QKV    (multi-token passes) one head's 64 q, k or v rows per workgroup;
//          prologue: embed (layer 0) or the residual sum of the previous
//          layer's down-projection partials, then RMSNorm/LayerNorm;
//          epilogue: bias (gpt2), RoPE (llama), q -> scratch, k/v -> KV cache
//   ATTN   one workgroup per (token, 256-position split, head): scores,
//          split-local softmax statistics and P.V; the last split of a
//          (token, head) merges the splits and multiplies the head output by
//          its 64-column slice of attn.proj, a per-head partial of W_o . att.
//          At one token (decode) the head's q/k/v rows are computed inside
//          the item itself (QKV fused in): residual sum, norm, q/k/v GEMV,
//          RoPE, KV-cache write, then attention.
//   MLP    one workgroup per 64 hidden units: residual sum of the per-head
//          partials (+ proj bias), norm2, gate and up rows of its units ->
//          silu(g)*u (gpt2: fc + bias -> GELU-tanh), then those units'
//          64-column slice of the down projection: a per-chunk partial of
//          W_2 . h
//   FINAL  per token: residual sum of the down partials (+ bias), final norm
//   LM     row tiles of the tied lm_head; logits + per-tile argmax (gpt2
//          chain: 3-gram block and repetition penalty of infer.js:252-287)
//   ARGMAX first maximum over tiles; chained decode feeds it back as the
//          next input token (CHAIN_TOK, webgpu-metal.js:609-610).
// The split-K partials are summed by their consumer in a fixed order, so
// every result is deterministic.  Every GEMV issues its weight loads before
// it stages its activations, so the two memory latencies overlap.  The GEMVs
// take their activations as 24-bit integer records per 32-element group and
// use 4-bit dot products (Q6 records, mllm_device.h).
//
// Execution modes, all running the same per-item device code:
//   3 (default where the device co-schedules one 1024-thread workgroup per
//     CU) one persistent cooperative kernel per decode call or chain; items
//     are ordered by per-item epoch flags, not barriers (k_flow below);
//   1 a HIP graph of one kernel per phase, replayed per token;
//   2 the phase kernels launched directly (for profilers).
// Multi-token passes (prefill, verify) always run the phase kernels.
//
// Every per-token computation (norm, GEMV row, attention split, merge, the
// partial sums, argmax) runs the same instruction sequence whatever the
// number of tokens in the pass, so a row of the multi-token verify pass is
// bit-identical to the single-token decode of that position.
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "mllm_device.h"
#include "mllm_host.h"
#include "mllm_generic.h"
#include "mllm_prefill.h"

namespace mllm {

#ifndef MLLM_LM_TILES_PER_WG
#define MLLM_LM_TILES_PER_WG 1
#endif

constexpr int HD = 64;     // head dimension of every supported config
constexpr int ACH = 256;   // positions per attention split (one per thread)
constexpr int MAXT = 16;   // tokens per pass (upper bound; LDS sets the real one)
constexpr int APS = 68;    // floats per attention partial: m, l, pad, pad, acc[64]
constexpr int APT = 66;    // tagged pairs per attention partial of the persistent kernels: m, l, acc[64]
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
constexpr int NWV = 16;    // waves of a 1024-thread workgroup: token t's serial work runs on wave t % NWV
constexpr int UNITS = 64;  // hidden units per MLP item (two 32-column groups of mlp.w2)
constexpr int SC = 2;      // chunk registers per thread of an ATTN head slice (SC * AT chunks)
constexpr int MC = 2;      // chunk registers per thread of the MLP tiles and slices (MC * MT chunks)
constexpr int QC = 2;      // chunk registers per thread of a QKV item: one head, 64 rows (QC * QT chunks)
// Chunk registers per thread of the fused q/k/v tile of a decode attention
// item (3 x 64 rows x d_model/32 chunks over 1024 threads): 4 up to d_model
// 672, 5 up to 832, 6 up to 1024.  The kernels are instantiated for each.
// (chunk c of the tile is taken by thread c % S, S = ng * (1024 / ng) the
// largest multiple of ng that fits the workgroup, so all of a thread's
// chunks are of one group)
constexpr int fixed_stride(int ng) { return (1024 / ng) * ng; }
constexpr int aqc_for(int ng) {
  return (3 * HD * ng + fixed_stride(ng) - 1) / fixed_stride(ng) <= 4
             ? 4
             : (3 * HD * ng + fixed_stride(ng) - 1) / fixed_stride(ng);
}
constexpr int FTC = 4;     // chunk registers per thread of a persistent-kernel lm_head tile (FTC * 1024 chunks)
constexpr int PB = 8;      // partials per block of the fixed-order partial sums
constexpr int NBMAX = 8;   // blocks per partial sum (<= PB * NBMAX partials: heads, 64-unit chunks)

enum Phase { PH_QKV = 0, PH_ATTN, PH_MLP, PH_FINAL, PH_LM, PH_ARGMAX, PH_COUNT };

struct LayerW {
  Q4Mat qkv, proj, w1, w3, w2;  // gpt2: w1 = mlp.fc, w2 = mlp.proj
  const float *n1, *n2;         // RMS gains; gpt2: LayerNorm gamma || beta
  const float *qkv_b, *proj_b, *fc_b, *mproj_b;
  const float *prev_mproj_b;    // gpt2: the previous layer's mlp.proj bias
  int dbg;                      // debug knobs (mllm_set_debug): bit 0 the attention block adds nothing to the
                                // residual, bit 1 the MLP block adds nothing (its projection writes zero partials)
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
  int tag0;      // tag base of a kernel-per-phase pass (below every later persistent-kernel tag)
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
  uint2 *xa;      // [MAXT][D] tagged residual entering the attention block
  uint2 *xb;      // [MAXT][D] tagged residual entering the MLP block
  uint2 *opart;   // [MAXT][NH][D] per-head partials of W_o . att, tagged pairs
  uint2 *dpart;   // [MAXT][nchunk][D] per-chunk partials of W_2 . h, tagged pairs
  float *xn;      // [MAXT][D] final-normed rows for the lm_head
  uint2 *rec;     // [2][MAXT][D/32 * Q6R] verify step: normed rows as tagged Q6 record dwords (attention, MLP)
  uint2 *qkvr;    // [L][MAXT][(NH + 2 NKV) * HD] verify step: q/k/v rows as tagged pairs, per layer
  float *q;       // [MAXT][NH*HD] queries after RoPE
  void *kv;       // [L][2][NKV][max_seq][HD] (f32 or f16)
  float *attp;    // [MAXT][NH][nsplit_max][APS]
  unsigned *cnt;  // [MAXT][NH] finished splits of the current layer
  float *logits;  // [MAXT][V]
  float *amv;     // [MAXT][lm_tiles]
  int *ami;
  uint2 *amt;     // [2][lm_tiles][2] persistent decode: each lm_head tile's first maximum (value, row) as tagged pairs, by step parity
  uint2 *amtv;    // [MAXT][lm_tiles][2] persistent verify: each token's tile maxima as tagged pairs
  uint2 *attpt;   // [MAXT][NH][nsplit_max][APT] persistent kernels: attention split partials (m, l, acc) as tagged pairs
  int lm_rpt, lm_tiles, lm_grid;
  PassState *st;
  int *hist;      // [max_seq + 1]
};

// What a phase needs to know about the pass besides the parameters.
struct Step {
  int pos0;   // position of token 0
  bool done;  // a chained decode already emitted eos: issue the first loads, store nothing
  int tag;    // tag of layer 0's handoff values; layer li writes tag + li
};
constexpr int TAGL = 128;  // tags per step (layers < TAGL)

// ---------------------------------------------------------------- stage probe
// A library built with -DMLLM_STAGE_PROBE (microllm-lab_amd/stage_probe.py)
// records when each item of the chained decode kernel k_flow3 reaches fixed
// points: thread 0 reads the 100 MHz real-time counter into LDS, and an
// item's stamps go out to the device array g_probe (vector stores) when its
// workgroup takes its next item or ends.  mllm_probe_read copies the array
// out, mllm_probe_clear zeroes it.  Layout [pos & 15][slot][item][PK] of u64:
// slot = layer for the layer items (item = index within the layer), PROBE_LM
// for the lm_head share and PROBE_TOP for the step-top token resolve (item =
// workgroup).  Stamps in use, by item kind:
//   all     0 item start, 7 item end
//   QKV     1 inputs gathered, 2 norm records done, 3 chunk dots, 4 row sums
//   ATT     1 q/k/v rows in, 4 K/V assembled, 5 score/P.V loop done, 2 after
//           the store wait and barrier, 3 split merges done
//   MLP     1 inputs gathered, 2 norm records done, 3 gate/up dots, 4 activation records
//   QKV, MLP (thread 0's wave, in the norm) 5 norm scale known, 6 records staged
//   LM      1 last layer's flags seen, 2 final-norm records in, 3 tiles done;
//           workgroup 0 (the final norm) also 4 partials gathered, 7 residual
//           summed, 5 norm scale known, 6 records staged
// The default build compiles none of this.
#ifdef MLLM_STAGE_PROBE
constexpr int PNI = 256, PSLOTS = 34, PK = 8, PROBE_TOP = 32, PROBE_LM = 33;
__device__ unsigned long long g_probe[16 * PSLOTS * PNI * PK];
__shared__ int g_pctx;
__shared__ unsigned long long g_pl[PK];
__device__ __forceinline__ void probe_flush() {
  if (threadIdx.x == 0 && g_pctx >= 0)
    for (int k = 0; k < PK; ++k)
      coh_st8(g_probe, (uint32_t)(g_pctx + k) * 8u, make_uint2((uint32_t)g_pl[k], (uint32_t)(g_pl[k] >> 32)));
}
__device__ __forceinline__ void probe_init() {
  if (threadIdx.x == 0) g_pctx = -1;
}
__device__ __forceinline__ void probe_set(int pos, int slot, int item) {
  probe_flush();
  if (threadIdx.x == 0) {
    g_pctx = ((((pos & 15) * PSLOTS + min(slot, PSLOTS - 1)) * PNI + min(item, PNI - 1)) * PK);
    for (int k = 0; k < PK; ++k) g_pl[k] = 0;
  }
}
__device__ __forceinline__ void probe_stamp(int k) {
  if (threadIdx.x == 0) g_pl[k] = __builtin_amdgcn_s_memrealtime();
}
#define PROBE_INIT() probe_init()
#define PROBE_SET(pos, slot, item) probe_set(pos, slot, item)
#define PROBE(k) probe_stamp(k)
#define PROBE_END() probe_flush()
#else
#define PROBE_INIT() ((void)0)
#define PROBE_SET(pos, slot, item) ((void)0)
#define PROBE(k) ((void)0)
#define PROBE_END() ((void)0)
#endif

// The pass state is read and written with coherent access: inside the
// persistent kernel ARGMAX updates it for workgroups on other XCDs.
#define ST_OFF(field) ((uint32_t)offsetof(PassState, field))
__device__ __forceinline__ int st_ld(const DecParams &P, uint32_t off) { return coh_ldi(P.st, off); }
__device__ __forceinline__ void st_st(const DecParams &P, uint32_t off, int v) { coh_sti(P.st, off, v); }

// No wait: the kernel-per-phase modes order phases by kernel boundaries.
struct NoWait {
  __device__ bool operator()() const { return false; }
};

// ---------------------------------------------------------------- helpers

// LDS regions read or written as float4 start on a 16-byte boundary.
__host__ __device__ __forceinline__ size_t al4(size_t n) { return (n + 3) & ~(size_t)3; }

__device__ __forceinline__ size_t kv_index(const DecParams &P, int li, int which, int h, int pos) {
  return ((((size_t)li * 2 + which) * P.NKV + h) * P.max_seq + pos) * HD;
}

// ---------------------------------------------------------------- residual and norm
// A phase's serial per-token work (the residual sum, the norm, row sums,
// the RoPE and activation epilogues) runs on one wave: token t on wave
// t % NWV.  The other waves wait at the next barrier instead of running the
// same dependent chain four waves to a SIMD.  Loads and dot products use
// every wave.  Which wave runs a token does not change its arithmetic, so a
// row of a multi-token pass is bit-identical to the single-token step.
__device__ __forceinline__ int wave_id() { return tid() >> 6; }
__device__ __forceinline__ int lane_id() { return tid() & 63; }

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// The norm gains (LayerNorm: gamma || beta) and the residual's bias go to
// LDS, where the norm wave reads them: gl[0, 2D) gains, gl[2D, 3D) bias.
// Loaded into registers (three per thread, d_model <= 1024) with the item's
// other early loads, stored once they have arrived.
struct GainsReg {
  float g[3];
};
__device__ __forceinline__ void gains_load(const DecParams &P, const float *w, const float *bias, GainsReg &G) {
  const int n = P.arch == 1 ? 2 * P.D : P.D;
  const int tot = n + (bias ? P.D : 0);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int e = min(tid() + k * 1024, tot - 1);  // branch-free; lanes past tot unused
    G.g[k] = e < n ? w[e] : bias[e - n];
  }
}
__device__ __forceinline__ void gains_store(const DecParams &P, const float *bias, const GainsReg &G, float *gl) {
  const int n = P.arch == 1 ? 2 * P.D : P.D;
  const int tot = n + (bias ? P.D : 0);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int e = tid() + k * 1024;
    if (e < tot) gl[e < n ? e : 2 * P.D + (e - n)] = G.g[k];
  }
}

// The residual of one token:
//   x = base + (((B_0 + B_1) + ... + B_{nb-1}) + bias)
// where B_b sums parts[p] for p in [b*PB, min(np, (b+1)*PB)) in ascending p
// (from +0).  The order of every addition is fixed by np alone.
// The partials are rows of D tagged pairs.  The block sums use every thread
// of a 1024-thread workgroup: item it = b * (D / 2) + c (round it / 1024)
// forms B_b of two columns.  With W16 these are columns 2c and 2c + 1, read
// as one 16-byte load (two neighbouring pairs) per partial, so each load
// instruction of a wave reads 1 KB contiguous; without it, columns c and
// c + D / 2 by two 8-byte loads.  A workgroup's gather rate is bound by its
// load instructions (16-byte loads move a 110 KB gather in about half the
// time of 8-byte ones), and the gather of the down partials is the larger part
// of a handoff.  A round's
// loads all go out before its first add, so a round costs one memory
// latency; round 0 can be loaded ahead (resid_blocks_load) so its latency
// overlaps the weight loads.  With POLL (persistent kernels) a round is
// polled until every pair carries the tag `want`: POLL 1 loads the
// whole round again, POLL 2 only the pairs still missing.
// Branch-free: an item or partial past the end reads pair 0 of partial 0
// (valid memory) and is left out.
struct ResidReg {
  uint2 v[2 * PB];
};

// Spin bound of the data polls: as kSpinLimit for flags; on time-out (or
// once another workgroup failed) the error is recorded and the wait returns.
__device__ __forceinline__ bool poll_give_up(const DecParams &P, unsigned spins);

// With W16, pairs 2c and 2c + 1 of a partial come from one 16-byte load (1 KB
// contiguous per wave instruction, half the load instructions); without it,
// pairs c and c + D / 2 come from two 8-byte loads.
template <bool W16>
__device__ __forceinline__ void resid_pair2(const uint2 *pt, int D, int p, int c, bool ok, uint2 &lo, uint2 &hi) {
  if (W16) {
    const uint4 u = coh_ld16(pt, (ok ? (uint32_t)(p * D + 2 * c) : 0u) * 8u);
    lo = make_uint2(u.x, u.y);
    hi = make_uint2(u.z, u.w);
  } else {
    const uint32_t e = ok ? (uint32_t)(p * D + c) : 0u;
    lo = tag_ld(pt, e);
    hi = tag_ld(pt, e + (ok ? (uint32_t)(D >> 1) : 0u));
  }
}

template <int POLL, bool W16 = false>
__device__ __forceinline__ void resid_blocks_load(const DecParams &P, const uint2 *pt, int np, int round, int want,
                                                  ResidReg &R) {
  const int D = P.D, nc2 = D >> 1, nitems = nc2 * ((np + PB - 1) / PB);
  const int it = tid() + round * 1024;
  const int b = it / nc2, c = it - b * nc2;
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const int p = b * PB + k;
    resid_pair2<W16>(pt, D, p, c, it < nitems && p < np, R.v[2 * k], R.v[2 * k + 1]);
  }
  if (POLL) {
    for (unsigned spins = 1;; ++spins) {
      bool ready = true;
#pragma unroll
      for (int k = 0; k < PB; ++k)
        ready &= !(it < nitems && b * PB + k < np) || (pair_ok(R.v[2 * k], want) && pair_ok(R.v[2 * k + 1], want));
      if (ready || poll_give_up(P, spins)) break;
      poll_fence();
      if (POLL == 1) {
#pragma unroll
        for (int k = 0; k < PB; ++k) {
          const int p = b * PB + k;
          resid_pair2<W16>(pt, D, p, c, it < nitems && p < np, R.v[2 * k], R.v[2 * k + 1]);
        }
        continue;
      }
      // POLL 2: only the pairs whose tag is not there yet are loaded again:
      // once most producers are done, a round carries the few missing pairs
      // instead of the whole gather (a CU's outstanding coherent loads bound
      // its rate)
#pragma unroll
      for (int k = 0; k < PB; ++k) {
        const int p = b * PB + k;
        const bool ok = it < nitems && p < np;
        const bool miss = !(pair_ok(R.v[2 * k], want) && pair_ok(R.v[2 * k + 1], want));
        if (ok && miss) resid_pair2<W16>(pt, D, p, c, true, R.v[2 * k], R.v[2 * k + 1]);
      }
    }
  }
}

// The loaded registers are consumed on every lane (only the store is
// conditional): a load consumed inside a divergent branch leaves the
// compiler unsure it has completed, and it then waits for every load in
// flight before the register is reused.
template <bool W16 = false>
__device__ __forceinline__ void resid_blocks_add(int D, int np, int round, const ResidReg &R, float *blk) {
  const int nc2 = D >> 1, nitems = nc2 * ((np + PB - 1) / PB);
  const int it = tid() + round * 1024;
  const int b = it / nc2, c = it - b * nc2;
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < PB; ++k) {
    const bool use = b * PB + k < np;
    a0 = a0 + (use ? __uint_as_float(R.v[2 * k].x) : 0.f);
    a1 = a1 + (use ? __uint_as_float(R.v[2 * k + 1].x) : 0.f);
  }
  if (it < nitems) {
    if (W16) {
      *reinterpret_cast<float2 *>(blk + b * D + 2 * c) = make_float2(a0, a1);
    } else {
      blk[b * D + c] = a0;
      blk[b * D + c + nc2] = a1;
    }
  }
}

// Every round of the block sums, round 0 already loaded into R0.
template <int POLL, bool W16 = false>
__device__ __forceinline__ void resid_blocks_rest(const DecParams &P, const uint2 *pt, int np, int want,
                                                  const ResidReg &R0, float *blk) {
  const int D = P.D;
  resid_blocks_add<W16>(D, np, 0, R0, blk);
  const int nitems = (D >> 1) * ((np + PB - 1) / PB);
  for (int round = 1; round * 1024 < nitems; ++round) {
    ResidReg R1;
    resid_blocks_load<POLL, W16>(P, pt, np, round, want, R1);
    resid_blocks_add<W16>(D, np, round, R1, blk);
  }
}

template <int POLL, bool W16 = false>
__device__ __forceinline__ void resid_blocks(const DecParams &P, const uint2 *pt, int np, int want, float *blk) {
  ResidReg R0;
  resid_blocks_load<POLL, W16>(P, pt, np, 0, want, R0);
  resid_blocks_rest<POLL, W16>(P, pt, np, want, R0, blk);
}

// One token's residual and norm, one float4 column q < nq per thread
// (threads 0 .. nq-1, d_model <= 1024):
//   x = base + (((B_0 + B_1) + ... + B_{nb-1}) + bias)
// from the block sums in blk, then RMSNorm (infer.js:134-143,
// x * (1/sqrt(mean(x^2) + eps)) * w) or LayerNorm (infer.js:147-164,
// eps 1e-5): each wave sums its columns with DPP, the waves' sums are added
// in order.  1/sqrt is the hardware reciprocal square root.  The
// normalised row is staged as Q6 records at qx_t (when set).  The gains (LayerNorm:
// gamma || beta) and the bias are in gl[0, 2D) and gl[2D, 3D).  Every
// thread of the workgroup must call it (it holds barriers); red needs
// 2 x 16 floats.
struct ColOut {
  uint2 *x;  // the residual row (tagged coherent stores), or null
  int tag;   // its tag
  float *y;  // the normalised row (coherent store), or null
};

__device__ __forceinline__ float4 col_finish(const float *blk, int nq, int np, float4 base, const float *gl, int D,
                                             bool has_bias) {
  const int q = min(tid(), nq - 1), nb = (np + PB - 1) / PB;  // threads past the row: a valid column, unused
  const float4 *b4 = reinterpret_cast<const float4 *>(blk);
  float4 s = b4[q];
  for (int b = 1; b < nb; ++b) s = add4(s, b4[b * nq + q]);
  if (has_bias) s = add4(s, reinterpret_cast<const float4 *>(gl + 2 * D)[q]);
  return add4(base, s);
}

// Sum over the first nw waves of one value per thread, into every thread.
__device__ __forceinline__ float waves_sum(float v, int nw, float *red) {
  const int wv = wave_id();
  if (wv < nw) {
    const float w = wave_sum(v);
    if (lane_id() == 0) red[wv] = w;
  }
  __syncthreads();
  // the four slots read at once (red holds at least four floats; slots past
  // nw are not added), then added in wave order
  const float r0 = red[0], r1 = red[1], r2 = red[2], r3 = red[3];
  float t = r0;
  if (nw > 1) t += r1;
  if (nw > 2) t += r2;
  if (nw > 3) t += r3;
  return t;
}

__device__ __forceinline__ void col_norm(const DecParams &P, float4 x, const float *gl, float *red, uint32_t *qx_t,
                                         const ColOut &o) {
  const int D = P.D, nq = D >> 2, q = tid(), nw = (nq + 63) >> 6;
  const bool in = q < nq;
  if (!in) x = make_float4(0.f, 0.f, 0.f, 0.f);
  if (o.x && in) {  // element 4q + j at pair j * nq + q (col_base_load)
    tag_st(o.x, q, x.x, o.tag);
    tag_st(o.x, nq + q, x.y, o.tag);
    tag_st(o.x, 2 * nq + q, x.z, o.tag);
    tag_st(o.x, 3 * nq + q, x.w, o.tag);
  }
  const float inv_d = 1.0f / (float)D;
  const float4 *g4 = reinterpret_cast<const float4 *>(gl);
  const int qc = min(q, nq - 1);
  float4 y;
  if (P.arch == 1) {
    const float4 g = g4[qc], b = g4[(D >> 2) + qc];  // read before the reductions' barriers
    const float mean = waves_sum((x.x + x.y) + (x.z + x.w), nw, red) * inv_d;
    const float4 d = in ? make_float4(x.x - mean, x.y - mean, x.z - mean, x.w - mean) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float r =
        __builtin_amdgcn_rsqf(waves_sum((d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w), nw, red + 16) * inv_d + 1e-5f);
    y = make_float4(__builtin_fmaf(d.x * r, g.x, b.x), __builtin_fmaf(d.y * r, g.y, b.y),
                    __builtin_fmaf(d.z * r, g.z, b.z), __builtin_fmaf(d.w * r, g.w, b.w));
  } else {
    const float4 g = g4[qc];  // read before the reduction's barrier
    const float r = __builtin_amdgcn_rsqf(waves_sum((x.x * x.x + x.y * x.y) + (x.z * x.z + x.w * x.w), nw, red) * inv_d +
                                          P.eps);
    y = make_float4(x.x * r * g.x, x.y * r * g.y, x.z * r * g.z, x.w * r * g.w);
  }
  if (!in) y = make_float4(0.f, 0.f, 0.f, 0.f);
  PROBE(5);
  if (o.y && in) coh_st4(o.y, 16u * q, y);
  if (qx_t && wave_id() < nw) q6_stage_col(y, in, q, qx_t);
  PROBE(6);
}

// The base column of this thread from a tagged row (branch-free); with POLL,
// loaded again until its tags reach `want`.  A residual row of D pairs
// keeps element 4q + j at pair j * nq + q (nq = D / 4), so each of the four
// load instructions of a wave reads 64 consecutive pairs.
template <bool POLL>
__device__ __forceinline__ float4 col_base_load(const DecParams &P, const uint2 *base, int nq, int want) {
  const uint32_t b = (uint32_t)min(tid(), nq - 1), n = (uint32_t)nq;
  uint2 v0 = tag_ld(base, b), v1 = tag_ld(base, b + n), v2 = tag_ld(base, b + 2 * n), v3 = tag_ld(base, b + 3 * n);
  if (POLL && tid() < nq) {
    for (unsigned spins = 1; !(pair_ok(v0, want) && pair_ok(v1, want) && pair_ok(v2, want) && pair_ok(v3, want)) &&
                             !poll_give_up(P, spins);
         ++spins) {
      poll_fence();
      v0 = tag_ld(base, b);
      v1 = tag_ld(base, b + n);
      v2 = tag_ld(base, b + 2 * n);
      v3 = tag_ld(base, b + 3 * n);
    }
  }
  return make_float4(__uint_as_float(v0.x), __uint_as_float(v1.x), __uint_as_float(v2.x), __uint_as_float(v3.x));
}

// Per-chunk partials of a tile in registers for m staged tokens:
// part[t*nch + c] (the arithmetic of tile_compute); no barrier.
template <int C>
__device__ __forceinline__ void tile_partials(const TileRegs<C> &R, int ng, int nch, int m, const uint32_t *qx,
                                              float *part) {
  int gj[C];
  {
    int g = tid() % ng;
    const int gstep = 1024 % ng;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      gj[j] = g;
      g += gstep;
      if (g >= ng) g -= ng;
    }
  }
  for (int t = 0; t < m; ++t) {
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int c = tid() + j * 1024;
      if (c < nch) part[t * nch + c] = q4_dot6(R.w[j], qx + (t * ng + gj[j]) * Q6R, R.s[j]);
      // one chunk at a time: the activations of several chunks in flight at
      // once would not fit beside the registers the caller holds (the other
      // waves of the SIMD hide the LDS latency)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The same partials for one token, chunk c taken by thread c % S (S =
// fixed_stride(ng), chunks loaded by tile_load3): every chunk of a thread is
// of group tid % ng, so its activation record is read from LDS once.  The
// partials have the arithmetic of tile_partials (q4_dot6).
template <int C>
__device__ __forceinline__ void tile_partials_fixed(const TileRegs<C> &R, int ng, int nch, const uint32_t *qx,
                                                    float *part) {
  const int S = fixed_stride(ng);
  if ((int)tid() < S) {
    float o[C];
    q4_dot6_planes<C>(R.w, R.s, qx + (tid() % ng) * Q6R, o);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int c = tid() + j * S;
      if (c < nch) part[c] = o[j];
    }
  }
}

// A slice is two groups (64 columns, groups g0 and g0 + 1) of every row of
// W.  Wave-slot ws = wave + (NT / 64) k (register k) takes rows
// [RPW ws, RPW ws + RPW): lane L holds the chunk of row RPW ws + L / 2,
// group g0 + (L & 1).
constexpr int RPW = 32;
template <int C, int NT>
__device__ __forceinline__ void slice_load(const Q4Mat &W, int g0, int rows, TileRegs<C> &R) {
  const int ng = W.cols >> 5;
  const int L = lane_id(), wv = wave_id();
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const int ws = wv + k * (NT / 64);
    const int r = min(RPW * ws + (L >> 1), rows - 1);  // branch-free; rows past the end unused
    const size_t gc = (size_t)r * ng + g0 + (L & 1);
    R.w[k] = W.q[gc];
    R.s[k] = W.s[gc];
  }
}

// The slice against two staged groups (Q6 records v, v + Q6R):
// row r = part(group g0) + part(group g0 + 1), the row_sum order of two
// groups, stored as a tagged pair by the even lane of the row.  Every lane
// takes part in the shuffle.
// With zero (a block the debug knobs switch off) the partial is stored as 0.
template <int C, int NT>
__device__ __forceinline__ void slice_gemv(const TileRegs<C> &R, int rows, const uint32_t *v, uint2 *out, int tag,
                                           bool zero = false) {
  const int L = lane_id(), wv = wave_id();
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const int ws = wv + k * (NT / 64);
    const int r = RPW * ws + (L >> 1);
    float p = 0.f;
    if (r < rows) p = q4_dot6(R.w[k], v + (L & 1) * Q6R, R.s[k]);
    const float sum = p + lane_xor1(p);  // rows past the end are 0
    if ((L & 1) == 0 && r < rows) tag_st(out, (uint32_t)r, zero ? 0.f : sum, tag);
  }
}

// Three 64-row ranges r0, r1, r2 of one matrix as one tile (chunk c of row
// c / ng of the ranges in order).  Branch-free: chunks past the tile load its
// last chunk (unused).
template <int C>
__device__ __forceinline__ void tile_load3(const Q4Mat &W, int r0, int r1, int r2, int ng, TileRegs<C> &R) {
  const int per = HD * ng, nch = 3 * per, S = fixed_stride(ng);
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = min(min((int)tid(), S - 1) + j * S, nch - 1);
    const int k = c / per, cc = c - k * per;
    // arithmetic, not a select chain (which the compiler turns into a table
    // in scratch memory)
    const int rb = r0 + (k >= 1 ? r1 - r0 : 0) + (k >= 2 ? r2 - r1 : 0);
    const size_t gc = (size_t)rb * ng + cc;
    R.w[j] = W.q[gc];
    R.s[j] = W.s[gc];
  }
}

// Embedding column q = tid of one token (infer.js:360-420): the
// dequantised row of the tied lm_head; gpt2 divides it by scale_factors
// (when present) and adds the learned position.  Branch-free (the column is
// clamped for threads past the row).
__device__ __forceinline__ float4 embed_col(const DecParams &P, int tok, int pos) {
  const int D = P.D, ng = D >> 5, q = min(tid(), (D >> 2) - 1);
  const bool gpt2 = P.arch == 1;
  const uint8_t *row = reinterpret_cast<const uint8_t *>(P.lm.q) + (size_t)tok * (D >> 1);
  const unsigned short b2 = *reinterpret_cast<const unsigned short *>(row + 2 * q);
  const float s = (P.lm.s + (size_t)tok * ng)[q >> 3];
  float4 e = make_float4((float)((int)(b2 & 15) - 8) * s, (float)((int)((b2 >> 4) & 15) - 8) * s,
                         (float)((int)((b2 >> 8) & 15) - 8) * s, (float)((int)(b2 >> 12) - 8) * s);
  if (gpt2) {
    if (P.sf) {
      const float4 f = reinterpret_cast<const float4 *>(P.sf)[q];
      e = make_float4(e.x / f.x, e.y / f.y, e.z / f.z, e.w / f.w);
    }
    e = add4(e, reinterpret_cast<const float4 *>(P.wpe + (size_t)pos * D)[q]);
  }
  return e;
}

// ---------------------------------------------------------------- phases
// Every phase is written once for both ways of running it.
//   FLOW = 0 (one kernel per phase): the activations are loaded first, then
//     the weights; loads retire in issue order, so the prologue never waits
//     for the weights.
//   FLOW = 1 (the persistent kernel): the weights are loaded first, then
//     wait() blocks until the producers of this item's inputs have published
//     them (it returns true once the chained decode has ended), then the
//     activations are loaded.
// The arithmetic is the same in both, so both give the same bits.

// QKV item: one head's 64 rows of attn.qkv (query head, K head or V head),
// so the RoPE partners d and d + 32 are in the item.
struct QkvPre {
  TileRegs<QC> R;
  float c_own, s_own;  // llama: RoPE cos/sin of (token wave, dim lane); gpt2: bias of row lane
};

__device__ __forceinline__ void qkv_pre(const DecParams &P, const LayerW &Lw, int head, int pos0, QkvPre &Q) {
  const int ng = P.D >> 5;
  tile_load<QC, QT>(Lw.qkv, head * HD, HD, 0, ng, HD * ng, Q.R);
  const int d = lane_id();
  const size_t ri = (size_t)min(pos0 + wave_id(), P.max_seq - 1) * HD + d;  // positions clamped past m
  const float *pc = P.arch == 1 ? Lw.qkv_b + head * HD + d : P.rope_cos + ri;
  const float *ps = P.arch == 1 ? pc : P.rope_sin + ri;
  Q.c_own = *pc;
  Q.s_own = *ps;
}

template <bool FLOW, class W>
__device__ void phase_qkv(const DecParams &P, const LayerW &Lw, int m, int li, int head, const Step &st, float *smem,
                          W &&wait) {
  const int D = P.D, ng = D >> 5, nq = D >> 2;
  const int nch = HD * ng;
  const int pos0 = st.pos0;
  const bool gpt2 = P.arch == 1;
  const int nb = (P.nchunk + PB - 1) / PB;
  float *gl = smem, *part = gl + al4(3 * D) + m * ng * Q6R;
  uint32_t *qx = reinterpret_cast<uint32_t *>(gl + al4(3 * D));  // m x ng Q6 records
  float *blk = part + m * nch;  // 2 x nb * D (alternating tokens), then red
  const float *rbias = gpt2 && li > 0 ? Lw.prev_mproj_b : nullptr;
  QkvPre Q;
  GainsReg GR;
  if (FLOW) {
    qkv_pre(P, Lw, head, pos0, Q);
    gains_load(P, Lw.n1, rbias, GR);
    gains_store(P, rbias, GR, gl);
    if (wait()) return;
  }
  const int wv = wave_id(), lane = lane_id();
  float *red = blk + 2 * nb * D;  // 32
  ResidReg R0;
  float4 base = make_float4(0.f, 0.f, 0.f, 0.f);
  if (!FLOW) {
    // loads retire in issue order: everything the prologue reads goes out
    // before the weight tile, so the prologue never waits for the weights
    if (li > 0) {
      base = col_base_load<false>(P, P.xb, nq, 0);
      resid_blocks_load<false>(P, P.dpart, P.nchunk, 0, 0, R0);
    }
    gains_load(P, Lw.n1, rbias, GR);
    qkv_pre(P, Lw, head, pos0, Q);
    if (st.done) return;  // a chained decode that reached eos: loads only, no stores
    if (li > 0) resid_blocks_rest<false>(P, P.dpart, P.nchunk, 0, R0, blk);
    gains_store(P, rbias, GR, gl);
  }
  // stage every token: x, the norm, its Q6 records
  for (int t = 0; t < m; ++t) {
    float *bt = blk + (t & 1) * nb * D;
    if (li == 0) {
      const int tok = min(max(st_ld(P, ST_OFF(tok) + 4u * t), 0), P.V - 1);  // host and ARGMAX keep it in range
      base = embed_col(P, tok, min(pos0 + t, P.max_seq - 1));
    } else if (FLOW || t > 0) {
      base = col_base_load<FLOW>(P, P.xb + (size_t)t * D, nq, st.tag + li - 1);
      resid_blocks<FLOW>(P, P.dpart + (size_t)t * P.nchunk * D, P.nchunk, st.tag + li - 1, bt);
    }
    __syncthreads();
    const float4 x = li == 0 ? base : col_finish(bt, nq, P.nchunk, base, gl, D, rbias != nullptr);
    col_norm(P, x, gl, red, qx + t * ng * Q6R, ColOut{head == 0 ? P.xa + (size_t)t * D : nullptr, st.tag + li});
  }
  __syncthreads();
  tile_partials<QC>(Q.R, ng, nch, m, qx, part);
  __syncthreads();
  // the m x 64 row sums, four lanes each (the decode attention item's order)
  float *rs = red + 32;
  for (int base = 0; base < m * HD; base += 256) {
    const int r = base + (int)(tid() >> 2);
    const int rr = min(r, m * HD - 1), tr = rr / HD;
    const float a = row_sum4(part + tr * nch + (rr - tr * HD) * ng, ng, tid() & 3);
    if ((tid() & 3) == 0 && r < m * HD) rs[r] = a;
  }
  __syncthreads();
  // epilogue on the token's wave: lane d is head dimension d
  for (int t = wv; t < m; t += NWV) {
    const int d = lane;
    float v = rs[t * HD + d];
    const int pos = pos0 + t;
    const bool is_q = head < P.NH, is_k = !is_q && head < P.NH + P.NKV;
    if (gpt2) {
      v = v + Q.c_own;  // the bias
    } else if (is_q || is_k) {
      const float mate = __shfl_xor(v, 32);  // rotate-half partner d +- 32
      v = __builtin_fmaf(v, Q.c_own, (d < 32 ? -mate : mate) * Q.s_own);
    }
    if (is_q) {
      coh_stf(P.q, 4u * (t * P.NH * HD + head * HD + d), v);
    } else {
      const int kvh = is_k ? head - P.NH : head - P.NH - P.NKV;
      const size_t k = kv_index(P, li, is_k ? 0 : 1, kvh, pos) + d;
      if (P.kv_fp16)
        coh_sth(P.kv, 2u * (uint32_t)k, __half_as_ushort(__float2half_rn(v)));
      else
        coh_stf(P.kv, 4u * (uint32_t)k, v);
    }
  }
}

// ---------------------------------------------------------------- attention
// One (token, split, head) item, 1024 threads: wave w takes keys
// 16w .. 16w+15 of the split.  Every K/V load of the item is issued at once:
// the score of key p is formed by the four lanes 4p .. 4p+3 (16 dimensions
// each, joined with DPP), and lane d of wave w holds V[16w + k][d] for
// k < 16.  Each wave forms its keys' softmax statistics (max, sum of
// weights) and its P.V for the 64 dimensions by itself, with no exchange
// between waves; wave 0 merges the 16 wave partials in wave order (the
// flash-decoding merge).  The last split of (token, head) to finish --
// counted in P.cnt; a single split is its own last -- merges the splits the
// same way, in split order, and writes the head's partial of the attention
// output projection to P.opart.
constexpr int AW = AT / 64;  // waves of an attention item; 16 keys each (AW * 16 == ACH)
static_assert(AW * 16 == ACH, "one wave per 16 keys of a split");
struct AttnLds {
  float *qs;       // 64: the query
  float *wm, *wl;  // AW: each wave's score maximum and sum of weights
  float *wacc;     // AW x 64: each wave's P.V
  uint32_t *attq;  // 2 x Q6R: merged head output, staged for the W_o slice
  int *flag;
};
constexpr int ATT_LDS = HD + 2 * AW + AW * HD + 2 * Q6R + 4;  // floats

__device__ __forceinline__ AttnLds attn_lds(float *base) {
  AttnLds A;
  A.qs = base;
  A.wm = A.qs + HD;
  A.wl = A.wm + AW;
  A.wacc = A.wl + AW;
  A.attq = reinterpret_cast<uint32_t *>(A.wacc + AW * HD);
  A.flag = reinterpret_cast<int *>(A.attq + 2 * Q6R);
  return A;
}

// K rows of keys kp < nkeys (four lanes per key) and V rows (lane d of wave
// w: dimension d of keys 16w .. 16w+15) of the split starting at position s0.
// Keys at and past nkeys are not loaded (at short contexts most lanes have
// none; duplicated clamped loads measured slower here).
//
// These are ordinary (L2-cached) loads, not device-coherent ones: a cached
// row never changes once written, and it is first read -- on any XCD -- only
// after its writer's tagged output has been seen, which follows the row's
// completed stores (the item waits for them before it publishes).  The
// cache line (128 B; a row is 256 B in f32, 128 B in f16, line-aligned)
// therefore cannot be in a reader's L2 from before the write, except from an
// earlier launch, and the persistent kernel opens with an agent-scope acquire
// that drops such lines.  Each attention item runs on the same workgroup in
// every step, so from the second step on its rows come from its XCD's L2.
__device__ __forceinline__ float4 kv_ld4(const void *base, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), (int)off, 0, 0);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ uint4 kv_ld16(const void *base, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void attn_k_load(const DecParams &P, int li, int kvh, int s0, int nkeys, float4 (&kr)[4]) {
  const uint32_t kbase = (uint32_t)kv_index(P, li, 0, kvh, s0);
  const int kp = tid() >> 2, ku = tid() & 3;
  if (kp < nkeys) {
    if (P.kv_fp16) {
      const uint32_t off = 2u * (kbase + kp * HD + 16 * ku);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint4 u = kv_ld16(P.kv, off + 16u * j);
        const __half2 *hp = reinterpret_cast<const __half2 *>(&u);
        const float2 f0 = __half22float2(hp[0]), f1 = __half22float2(hp[1]);
        const float2 f2 = __half22float2(hp[2]), f3 = __half22float2(hp[3]);
        kr[2 * j] = make_float4(f0.x, f0.y, f1.x, f1.y);
        kr[2 * j + 1] = make_float4(f2.x, f2.y, f3.x, f3.y);
      }
    } else {
      const uint32_t off = 4u * (kbase + kp * HD + 16 * ku);
#pragma unroll
      for (int j = 0; j < 4; ++j) kr[j] = kv_ld4(P.kv, off + 16u * j);
    }
  }
}

__device__ __forceinline__ void attn_v_load(const DecParams &P, int li, int kvh, int s0, int nkeys, float (&vr)[16]) {
  const uint32_t vbase = (uint32_t)kv_index(P, li, 1, kvh, s0) + (uint32_t)lane_id();
  const int k0 = 16 * wave_id();
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    vr[k] = 0.f;
    if (k0 + k < nkeys) {
      const uint32_t e = vbase + (uint32_t)(k0 + k) * HD;
      if (P.kv_fp16)
        vr[k] = __half2float(__ushort_as_half(
            __builtin_amdgcn_raw_buffer_load_b16(coh_rsrc(P.kv), (int)(2u * e), 0, 0)));
      else
        vr[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(coh_rsrc(P.kv), (int)(4u * e), 0, 0));
    }
  }
}

// One wave's merge of a split's AW wave partials, every lane taking part:
// mx = max_w m_w, f_w = expf(m_w - mx) (0 for a wave with no key), and
// l = sum_w l_w f_w, own = sum_w acc_w[lane] f_w, each accumulated in
// ascending w by FMA from +0.  The weights go back to LDS in place of the
// maxima and return as broadcast reads, and every operand is loaded before
// the first FMA: the chain then waits for LDS once, not once per pair of
// waves, and needs no lane reads.  wm, wl: AW floats each (16-byte aligned);
// wacc: AW rows of HD floats.
__device__ __forceinline__ void split_merge(float *wm, const float *wl, const float *wacc, float &mx, float &l,
                                            float &own) {
  const int lane = lane_id();
  const float wmv = lane < AW ? wm[lane] : -INFINITY;
  mx = wave_max(wmv);
  const float f = lane < AW ? expf(wmv - mx) : 0.f;
  if (lane < AW) wm[lane] = f;  // the same wave reads it back: LDS operations of a wave complete in order
  float av[AW], fv[AW], lv[AW];
#pragma unroll
  for (int w = 0; w < AW; ++w) av[w] = wacc[w * HD + lane];
#pragma unroll
  for (int w = 0; w < AW; w += 4) {
    const float4 a = *reinterpret_cast<const float4 *>(wm + w);
    const float4 b = *reinterpret_cast<const float4 *>(wl + w);
    fv[w] = a.x;
    fv[w + 1] = a.y;
    fv[w + 2] = a.z;
    fv[w + 3] = a.w;
    lv[w] = b.x;
    lv[w + 1] = b.y;
    lv[w + 2] = b.z;
    lv[w + 3] = b.w;
  }
  l = 0.f;
  own = 0.f;
#pragma unroll
  for (int w = 0; w < AW; ++w) {
    l = __builtin_fmaf(lv[w], fv[w], l);
    own = __builtin_fmaf(av[w], fv[w], own);
  }
}

// Scores, softmax statistics, P.V, the merge and the head's W_o slice, with
// the query staged in A.qs and the keys in kr/vr; key knew of the split (when
// >= 0) is taken from LDS instead (kvn: K row then V row), selected where it
// is used so that no load of kr/vr is waited for early.  Ro holds the slice
// when ro_loaded; the merging split of a multi-split head loads it otherwise.
// Returns true in the workgroup that wrote the head's output.
template <int C>
__device__ bool attn_core(const DecParams &P, const LayerW &Lw, int t, int sp, int h, int ns, int cnt,
                          const float4 (&kr)[4], const float (&vr)[16], int knew, const float *kvn, TileRegs<C> &Ro,
                          bool ro_loaded, const AttnLds &A, int tag) {
  const int D = P.D;
  const bool solo = ns == 1;
  const int kp = tid() >> 2, ku = tid() & 3;
  const int lane = lane_id(), wv = wave_id();
  __syncthreads();
  // A wave whose 16 keys all lie past the split's end skips the arithmetic:
  // its maximum -inf, sum +0 and P.V +0 are what the arithmetic gives it (no
  // score, every weight 0), and it leaves the SIMDs to the waves with keys.
  float mw = -INFINITY, lw = 0.f, acc = 0.f;
  if (16 * wv < cnt) {
    float part = 0.f;
    if (kp < cnt) {
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
      const float *qq = A.qs + 16 * ku;
      const bool nk = kp == knew;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 kk = nk ? reinterpret_cast<const float4 *>(kvn)[4 * ku + j] : kr[j];
        a0 = __builtin_fmaf(qq[4 * j + 0], kk.x, a0);
        a1 = __builtin_fmaf(qq[4 * j + 1], kk.y, a1);
        a2 = __builtin_fmaf(qq[4 * j + 2], kk.z, a2);
        a3 = __builtin_fmaf(qq[4 * j + 3], kk.w, a3);
      }
      part = (a0 + a1) + (a2 + a3);
    }
    // the four quarters: (q0 + q1) + (q2 + q3) in every lane of the quad
    part = part + dpp_f<0xB1>(part);
    part = part + dpp_f<0x4E>(part);
    const float score = kp < cnt ? part * P.attn_scale : -INFINITY;
    // the wave's 16 keys: maximum, weights, their sum and P.V (lane = dimension)
    mw = wave_max(score);
    const float e = kp < cnt ? expf(score - mw) : 0.f;
    lw = wave_sum(ku == 0 ? e : 0.f);
    // branch-free: the new key's value is read from LDS once, and selected
    const float vnew = kvn[HD + lane];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int key = 16 * wv + k;
      const float ek = readlane_f(e, 4 * k);
      float vv = key == knew ? vnew : vr[k];
      vv = key < cnt ? vv : 0.f;
      acc = __builtin_fmaf(ek, vv, acc);
    }
  }
  A.wacc[wv * HD + lane] = acc;
  if (lane == 0) {
    A.wm[wv] = mw;
    A.wl[wv] = lw;
  }
  __syncthreads();
  // wave 0: the split's maximum, sum and P.V from the wave partials, added
  // in wave order (a wave with no key has m_w = -inf and weight 0; wave 0
  // always has key 0)
  float mx = 0.f, l = 0.f, own = 0.f;
  if (wv == 0) split_merge(A.wm, A.wl, A.wacc, mx, l, own);
  // split partials of (t, h): [nsplit_max][APS] floats (m, l, pad, pad, acc[64])
  const float *parts = P.attp + (size_t)(t * P.NH + h) * P.nsplit_max * APS;
  if (!solo) {
    // publish this split, then count it; the last one merges
    float *dst = P.attp + ((size_t)(t * P.NH + h) * P.nsplit_max + sp) * APS;
    if (wv == 0) {
      coh_stf(dst, 4u * (4 + lane), own);
      if (lane == 0) {
        coh_stf(dst, 0, mx);
        coh_stf(dst, 4, l);
      }
    }
    wait_stores();
    __syncthreads();
    if (tid() == 0) {
      unsigned *c = P.cnt + t * P.NH + h;
      const unsigned arrived = atomicAdd(c, 1u);
      A.flag[0] = arrived == (unsigned)(ns - 1);
      if (A.flag[0]) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!A.flag[0]) return false;
    if (!ro_loaded) slice_load<C, AT>(Lw.proj, 2 * h, D, Ro);
  }
  if (wv == 0) {
    const int d = lane;
    float v;
    if (solo) {
      v = own / l;  // the merge below with one split: weight expf(0) = 1
    } else {
      float M = sp == 0 ? mx : coh_ldf(parts, 0);
      for (int j = 1; j < ns; ++j) M = fmaxf(M, j == sp ? mx : coh_ldf(parts, 4u * (j * APS)));
      const float m0 = sp == 0 ? mx : coh_ldf(parts, 0), l0 = sp == 0 ? l : coh_ldf(parts, 4),
                  a0 = sp == 0 ? own : coh_ldf(parts, 4u * (4 + d));
      const float w0 = expf(m0 - M);
      float ls = __builtin_fmaf(l0, w0, 0.f), as = __builtin_fmaf(a0, w0, 0.f);
      for (int j = 1; j < ns; ++j) {
        const float mj = j == sp ? mx : coh_ldf(parts, 4u * (j * APS));
        const float lj = j == sp ? l : coh_ldf(parts, 4u * (j * APS + 1));
        const float aj = j == sp ? own : coh_ldf(parts, 4u * (j * APS + 4 + d));
        const float w = expf(mj - M);
        ls = __builtin_fmaf(lj, w, ls);
        as = __builtin_fmaf(aj, w, as);
      }
      v = as / ls;
    }
    q6_stage_lanes(v, A.attq);  // the head output: two groups, wave 0
  }
  // the item's earlier stores (its K/V cache row) complete before the head's
  // output becomes visible, so whoever sees the output also sees them
  wait_stores();
  __syncthreads();
  slice_gemv<C, AT>(Ro, D, A.attq, P.opart + (size_t)(t * P.NH + h) * D, tag, Lw.dbg & 1);
  return true;
}

// Multi-token passes: the item reads its query and the K/V rows that the
// QKV phase stored.
template <bool FLOW, class W>
__device__ bool phase_attn(const DecParams &P, const LayerW &Lw, int m, int li, int item, const Step &st,
                           float *smem, W &&wait) {
  const int per_tok = P.NH * P.nsplit_max;
  const int t = item / per_tok;
  const int rem = item - t * per_tok;
  const int sp = rem / P.NH, h = rem - sp * P.NH;
  if (t >= m || st.done) return false;
  const int pos = st.pos0 + t;
  const int s0 = sp * ACH;
  if (s0 > pos) return false;
  const int ns = pos / ACH + 1;
  TileRegs<SC> Ro;
  if (FLOW) {
    slice_load<SC, AT>(Lw.proj, 2 * h, P.D, Ro);  // W_o columns of this head
    if (wait()) return false;
  }
  const int cnt = min(ACH, pos + 1 - s0);
  const AttnLds A = attn_lds(smem);
  float4 kr[4];
  float vr[16];
  if (tid() < HD) A.qs[tid()] = coh_ldf(P.q, 4u * ((t * P.NH + h) * HD + tid()));
  attn_k_load(P, li, h / (P.NH / P.NKV), s0, cnt, kr);
  attn_v_load(P, li, h / (P.NH / P.NKV), s0, cnt, vr);
  const bool ro = FLOW || ns == 1;
  if (!FLOW && ns == 1) slice_load<SC, AT>(Lw.proj, 2 * h, P.D, Ro);  // behind the K/V loads
  return attn_core<SC>(P, Lw, t, sp, h, ns, cnt, kr, vr, -1, A.qs, Ro, ro, A, st.tag + li);  // no key from LDS
}

// Weights and other inputs of a fused decode attention item that do not
// depend on the previous phase: the q/k/v tile, the head's W_o slice, this
// thread's RoPE entries (gpt2: its row's bias) and the norm gains.
template <int AQC>
__device__ __forceinline__ void attn1_pre(const DecParams &P, const LayerW &Lw, int rq, int rk, int rv, int h, int pos,
                                          int row_own, const float *rbias, TileRegs<AQC> &Wt, TileRegs<SC> &Ro,
                                          float &c_own, float &s_own, GainsReg &GR) {
  const int ng = P.D >> 5;
  tile_load3<AQC>(Lw.qkv, rq, rk, rv, ng, Wt);
  slice_load<SC, AT>(Lw.proj, 2 * h, P.D, Ro);
  const size_t ri = (size_t)min(pos, P.max_seq - 1) * HD + lane_id();
  const float *pc = P.arch == 1 ? Lw.qkv_b + min(row_own, rv + HD - 1) : P.rope_cos + ri;
  const float *ps = P.arch == 1 ? pc : P.rope_sin + ri;
  c_own = *pc;
  s_own = *ps;
  gains_load(P, Lw.n1, rbias, GR);
}

// Deferred K/V-row stores of the persistent kernel.  Only later steps read
// a position's cached K/V row from memory (the query heads of the group form
// the row themselves, and the current position lies in the last split only),
// so the writer keeps the row's two stores -- one word per lane of waves 1
// (K) and 2 (V) -- in LDS slots of its own (byte offset, bits; offset ~0: none)
// and issues them when the workgroup starts its next attention item.  A slot
// with nothing pending points at a pad word past the end of the cache
// (kv_pad), so the store is issued unconditionally.  That
// item's output, and any later one, waits for the workgroup's stores before it
// becomes visible (attn_core), and every reader of the row in a later step
// depends through the data edges on the workgroup's next item of the same step
// (or, past the last layer, of the next step); the kernel issues what is left
// when it ends.  The writer therefore never waits for the acknowledgement of
// a row it has just stored, and the output it publishes does not wait either.
__device__ __forceinline__ uint2 *kv_slot(float *smem, int kvp) {
  return reinterpret_cast<uint2 *>(smem + kvp) + (tid() - 64);
}
// The persistent kernel's broadcast slots (LDS, past the deferred K/V slots):
// [0] the step's input token, [1] the chain is done, [2] workgroup 0's count
// of history tokens, [3] the eos id (-1: none), [4] chained decode, [5, 21)
// eight waves' (value, row) maxima (flow_tiles_argmax).
__device__ __forceinline__ int *flow_slots(float *smem, int kvp) { return reinterpret_cast<int *>(smem + kvp + 256); }

__device__ __forceinline__ uint2 kv_pad(const DecParams &P) {
  return make_uint2((uint32_t)kv_index(P, P.L, 0, 0, 0) * (P.kv_fp16 ? 2u : 4u), 0u);
}
__device__ __forceinline__ void kv_flush(const DecParams &P, float *smem, int kvp) {
  const int wv = wave_id();
  if (wv == 1 || wv == 2) {
    uint2 *slot = kv_slot(smem, kvp);
    const uint2 e = *slot;
    if (P.kv_fp16) coh_sth(P.kv, e.x, (unsigned short)e.y);
    else coh_sti(P.kv, e.x, (int)e.y);
    *slot = kv_pad(P);
  }
}

// Single-token attention item (split sp, head h) with the QKV projection
// fused in: the item forms its own query head and its K/V head's rows of
// attn.qkv from the residual (the K/V rows are formed again by every query
// head that shares them), then attends over its split.  The split holding
// the current position takes the new K/V row from LDS, rounded as the cache
// stores it; the first query head of the group writes it to the cache.
// Every row has the arithmetic of phase_qkv (same chunk partials, same row
// order), so the step matches a multi-token pass bit for bit.
template <bool FLOW, int AQC, class W>
__device__ bool phase_attn1(const DecParams &P, const LayerW &Lw, int li, int item, const Step &st, float *smem,
                            W &&wait, int kvp = 0) {
  const int sp = item / P.NH, h = item - sp * P.NH;
  if (st.done) return false;
  const int pos = st.pos0;
  const int s0 = sp * ACH;
  if (s0 > pos) return false;
  const int ns = pos / ACH + 1;
  const bool last = sp == ns - 1;
  const int rep = P.NH / P.NKV, kvh = h / rep;
  const bool writer = last && h % rep == 0;
  const int D = P.D, ng = D >> 5, nq = D >> 2;
  const int nch = 3 * HD * ng;
  const int cnt = min(ACH, pos + 1 - s0);
  const bool gpt2 = P.arch == 1;
  const float *rbias = gpt2 && li > 0 ? Lw.prev_mproj_b : nullptr;
  const int nb = (P.nchunk + PB - 1) / PB;
  float *gl = smem, *part = gl + al4(3 * D) + ng * Q6R;
  uint32_t *qx = reinterpret_cast<uint32_t *>(gl + al4(3 * D));  // ng Q6 records
  float *blk = part + nch, *red = blk + nb * D, *kvn = red + 32;  // kvn: the new K row (64) then V row (64)
  float *rs = kvn + 2 * HD;  // 3 x 64 row sums: q, k, v
  const AttnLds A = attn_lds(rs + 3 * HD);  // 16-byte aligned: every region before it is a multiple of 4 floats
  const int wv = wave_id(), lane = lane_id();
  // rows of the fused tile: [q head h | K head kvh | V head kvh], 64 each
  const int rq = h * HD, rk = (P.NH + kvh) * HD, rv = (P.NH + P.NKV + kvh) * HD;
  TileRegs<AQC> Wt;
  TileRegs<SC> Ro;
  GainsReg GR;
  float c_own = 0.f, s_own = 0.f;
  float4 kr[4];
  float vr[16];
  ResidReg R0;
  float4 base = make_float4(0.f, 0.f, 0.f, 0.f);
  // wave w < 3 forms row (w: q, k, v) lane d of the tile: its RoPE entries
  // at pos (q and k) or its bias (gpt2)
  const int row_own = rq + min(wv, 2) * (rk - rq) + (wv >= 2 ? rv - rk - (rk - rq) : 0) + lane;
  // The cached K rows are loaded once the residual's block sums are formed
  // (their registers are then free), the V rows once the q/k/v tile is
  // consumed; their latency overlaps the norm, the q/k/v rows and the scores.
  if (FLOW) {
    kv_flush(P, smem, kvp);  // the previous item's K/V row
    attn1_pre(P, Lw, rq, rk, rv, h, pos, row_own, rbias, Wt, Ro, c_own, s_own, GR);
    gains_store(P, rbias, GR, gl);
    if (wait()) return false;
    if (li > 0) {
      base = col_base_load<true>(P, P.xb, nq, st.tag + li - 1);
      resid_blocks<2, true>(P, P.dpart, P.nchunk, st.tag + li - 1, blk);
    }
  } else {
    // activations first, then the weights (loads retire in issue order)
    if (li > 0) {
      base = col_base_load<false>(P, P.xb, nq, 0);
      resid_blocks_load<false>(P, P.dpart, P.nchunk, 0, 0, R0);
    }
    attn1_pre(P, Lw, rq, rk, rv, h, pos, row_own, rbias, Wt, Ro, c_own, s_own, GR);
    if (li > 0) resid_blocks_rest<false>(P, P.dpart, P.nchunk, 0, R0, blk);
    gains_store(P, rbias, GR, gl);
  }
  // stage boundaries are fixed (sched_barrier) so that the tile, the K rows
  // and the V rows are not all held at once
  __builtin_amdgcn_sched_barrier(0);
  attn_k_load(P, li, kvh, s0, last ? cnt - 1 : cnt, kr);  // cached positions: written by earlier steps
  attn_v_load(P, li, kvh, s0, last ? cnt - 1 : cnt, vr);
  __builtin_amdgcn_sched_barrier(0);
  // the residual (layer 0: the embedding) and the norm
  if (li == 0) {
    // the persistent kernel takes the step's token from its slot
    const int tok = FLOW ? flow_slots(smem, kvp)[0] : min(max(st_ld(P, ST_OFF(tok)), 0), P.V - 1);
    base = embed_col(P, tok, min(pos, P.max_seq - 1));
  }
  __syncthreads();
  const float4 x = li == 0 ? base : col_finish(blk, nq, P.nchunk, base, gl, D, rbias != nullptr);
  col_norm(P, x, gl, red, qx, ColOut{item == 0 ? P.xa : nullptr, st.tag + li});
  __syncthreads();
  tile_partials_fixed<AQC>(Wt, ng, nch, qx, part);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  {
    // the 192 row sums, four lanes each
    const int r = tid() >> 2;
    const float a = row_sum4(part + min(r, 3 * HD - 1) * ng, ng, tid() & 3);
    if ((tid() & 3) == 0 && r < 3 * HD) rs[r] = a;
  }
  __syncthreads();
  // rows: wave 0 the query, wave 1 the key, wave 2 the value (lane d)
  if (wv < 3) {
    float v = rs[wv * HD + lane];
    if (gpt2) {
      v = v + c_own;  // the bias
    } else if (wv < 2) {
      const float mate = __shfl_xor(v, 32);  // rotate-half partner d +- 32
      v = __builtin_fmaf(v, c_own, (lane < 32 ? -mate : mate) * s_own);
    }
    if (wv == 0) {
      A.qs[lane] = v;
    } else {
      const size_t k = kv_index(P, li, wv - 1, kvh, pos) + lane;
      float r = v;
      // FLOW: the row's stores are issued by the workgroup's next attention item
      uint2 *slot = kv_slot(smem, kvp);
      if (P.kv_fp16) {
        const __half hv = __float2half_rn(v);
        r = __half2float(hv);
        if (writer && FLOW) *slot = make_uint2(2u * (uint32_t)k, __half_as_ushort(hv));
        else if (writer) coh_sth(P.kv, 2u * (uint32_t)k, __half_as_ushort(hv));
      } else if (writer && FLOW) {
        *slot = make_uint2(4u * (uint32_t)k, __float_as_uint(v));
      } else if (writer) {
        coh_stf(P.kv, 4u * (uint32_t)k, v);
      }
      kvn[(wv - 1) * HD + lane] = r;
    }
  }
  // the current position (key cnt - 1 of the last split) comes from LDS
  return attn_core<SC>(P, Lw, 0, sp, h, ns, cnt, kr, vr, last ? cnt - 1 : -1, kvn, Ro, true, A, st.tag + li);
}

// Hidden units [item*UNITS, (item+1)*UNITS): gate/up (or fc) rows, the
// activation, then the units' two-group slice of the down projection.
struct MlpPre {
  TileRegs<MC> Rg, Ru, Rd;
  float fcb;
};

__device__ __forceinline__ void mlp_pre_up(const DecParams &P, const LayerW &Lw, int item, MlpPre &M) {
  const int ng = P.D >> 5, r0 = item * UNITS;
  // gate/up chunk c = tid + j*S (S = (MT / ng) * ng): every chunk of a thread
  // is group tid % ng, so its activations are read from LDS once
  const int S = (MT / ng) * ng;
  tile_load_strided<MC>(Lw.w1, r0, UNITS, ng, S, M.Rg);
  if (P.arch != 1) tile_load_strided<MC>(Lw.w3, r0, UNITS, ng, S, M.Ru);
  // unconditional load (llama reads its norm gains instead and ignores it)
  M.fcb = (P.arch == 1 ? Lw.fc_b + r0 : Lw.n2)[lane_id()];
}

template <bool FLOW, class W>
__device__ void phase_mlp(const DecParams &P, const LayerW &Lw, int m, int li, int item, const Step &st, float *smem,
                          W &&wait) {
  const int D = P.D, ng = D >> 5, nq = D >> 2;
  const bool gpt2 = P.arch == 1;
  const int nch = UNITS * ng;
  const int S = (MT / ng) * ng;
  const int nb = (P.NH + PB - 1) / PB;
  float *gl = smem, *part = gl + al4(3 * D) + m * ng * Q6R;  // part: 2 x (gate || up)
  uint32_t *qx = reinterpret_cast<uint32_t *>(gl + al4(3 * D));  // m x ng Q6 records
  uint32_t *hq = reinterpret_cast<uint32_t *>(part + 4 * nch);   // m x 2 Q6 records of h
  float *blk = reinterpret_cast<float *>(hq + m * 2 * Q6R);     // 2 x nb * D, then red
  float *red = blk + 2 * nb * D;
  float *rsum = red + 32;  // 2 x (gate || up) row sums, by token parity
  const float *rbias = gpt2 ? Lw.proj_b : nullptr;
  MlpPre M;
  GainsReg GR;
  if (FLOW) {
    mlp_pre_up(P, Lw, item, M);
    slice_load<MC, MT>(Lw.w2, 2 * item, D, M.Rd);
    gains_load(P, Lw.n2, rbias, GR);
    gains_store(P, rbias, GR, gl);
    if (wait()) return;
  }
  const int wv = wave_id(), lane = lane_id();
  float4 base = make_float4(0.f, 0.f, 0.f, 0.f);
  const int want = st.tag + li;  // the attention block of this layer
  if (!FLOW) {
    base = col_base_load<false>(P, P.xa, nq, 0);
    ResidReg R0;
    resid_blocks_load<false>(P, P.opart, P.NH, 0, 0, R0);
    gains_load(P, Lw.n2, rbias, GR);
    mlp_pre_up(P, Lw, item, M);  // before the down slice (loads retire in issue order)
    if (st.done) return;
    resid_blocks_rest<false>(P, P.opart, P.NH, 0, R0, blk);
    gains_store(P, rbias, GR, gl);
  }
  for (int t = 0; t < m; ++t) {
    float *bt = blk + (t & 1) * nb * D;
    if (FLOW || t > 0) {
      base = col_base_load<FLOW>(P, P.xa + (size_t)t * D, nq, want);
      resid_blocks<FLOW ? 2 : 0, FLOW>(P, P.opart + (size_t)t * P.NH * D, P.NH, want, bt);
    }
    __syncthreads();
    col_norm(P, col_finish(bt, nq, P.NH, base, gl, D, rbias != nullptr), gl, red, qx + t * ng * Q6R,
             ColOut{item == 0 ? P.xb + (size_t)t * D : nullptr, want});
  }
  if (!FLOW) slice_load<MC, MT>(Lw.w2, 2 * item, D, M.Rd);  // needed last: behind everything the prologue reads
  __syncthreads();
  const int g = tid() % ng;
  static_assert(2 * UNITS * 8 == MT, "one 8-lane row sum per gate and up row");
  for (int t = 0; t < m; ++t) {
    // gate and up chunk partials of token t, then the row sums on every
    // wave (8 lanes per row), then the token's wave (unit r = lane) forms
    // the activation and the two group records of h
    float *pt = part + (t & 1) * 2 * nch;
    float *rt = rsum + (t & 1) * 2 * UNITS;
    {
      // gate chunks then up chunks against the thread's one group record
      uint4 w[2 * MC];
      float ws[2 * MC], o[2 * MC];
#pragma unroll
      for (int k = 0; k < MC; ++k) {
        w[k] = M.Rg.w[k];
        ws[k] = M.Rg.s[k];
        w[MC + k] = M.Ru.w[k];
        ws[MC + k] = M.Ru.s[k];
      }
      q4_dot6_planes<2 * MC>(w, ws, qx + (t * ng + g) * Q6R, o);
#pragma unroll
      for (int k = 0; k < MC; ++k) {
        const int c = tid() + k * S;
        if ((int)tid() < S && c < nch) {
          pt[c] = o[k];
          if (!gpt2) pt[nch + c] = o[MC + k];
        }
      }
    }
    __syncthreads();
    {
      // row r (gate rows, then up rows): lane s adds partials s, s + 8, ...
      // in order, then a fixed 8-lane tree
      const int r = tid() >> 3, s = tid() & 7;
      const int nrows = gpt2 ? UNITS : 2 * UNITS;
      const float *pr = pt + (r < UNITS ? 0 : nch) + (r & (UNITS - 1)) * ng;
      float a = 0.f;
      if (r < nrows)
        for (int k = s; k < ng; k += 8) a = a + pr[k];
      a = sum8f(a);
      if (s == 0 && r < nrows) rt[r] = a;
    }
    __syncthreads();
    if (wv == (t & (NWV - 1))) {
      const int r = lane;
      const float gv = rt[r];
      float h;
      if (gpt2) {
        const float v = gv + M.fcb;
        h = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
      } else {
        h = (gv / (1.0f + expf(-gv))) * rt[UNITS + r];
      }
      q6_stage_lanes(h, hq + t * 2 * Q6R);
    }
  }
  __syncthreads();
  for (int t = 0; t < m; ++t)
    slice_gemv<MC, MT>(M.Rd, D, hq + t * 2 * Q6R, P.dpart + ((size_t)t * P.nchunk + item) * D, want, Lw.dbg & 2);
}

// The last layer's residual and the final norm of token t: Q6 records (LDS)
// for the lm_head of the persistent kernel, or xn (coherent stores) for the
// lm_head kernel.  blk needs nb * D floats; the
// caller has staged the norm_f gains in gl.
template <int POLL>
__device__ __forceinline__ void final_row(const DecParams &P, int t, float *blk, const float *gl, uint32_t *qx,
                                          bool to_global, int want) {
  const int D = P.D, nq = D >> 2;
  const float4 base = col_base_load<(POLL != 0)>(P, P.xb + (size_t)t * D, nq, want);
  resid_blocks<POLL, POLL == 2>(P, P.dpart + (size_t)t * P.nchunk * D, P.nchunk, want, blk);
  __syncthreads();
  PROBE(4);
  const float4 x = col_finish(blk, nq, P.nchunk, base, gl, D, P.arch == 1 && P.last_mproj_b != nullptr);
  PROBE(7);
  col_norm(P, x, gl, blk + ((P.nchunk + PB - 1) / PB) * D, qx, ColOut{nullptr, 0, to_global ? P.xn + (size_t)t * D : nullptr});
}

// Kernel-per-phase mode: item t writes xn[t] (only the rows the
// lm_head reads).
__device__ void phase_final(const DecParams &P, int m, int item, const Step &st, float *smem) {
  const int lm_rows = st_ld(P, ST_OFF(lm_rows));
  if (lm_rows == 0 || st.done) return;
  const int tb = lm_rows == 1 ? m - 1 : 0;
  const int t = item;
  if (t < tb || t >= m) return;
  float *gl = smem, *blk = gl + al4(3 * P.D);
  const float *rbias = P.arch == 1 ? P.last_mproj_b : nullptr;
  GainsReg GR;
  gains_load(P, P.norm_f, rbias, GR);
  gains_store(P, rbias, GR, gl);
  final_row<false>(P, t, blk, gl, nullptr, true, 0);
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
  uint32_t *qx;  // the normed rows, Q6 records
  float *part, *out;
  int *lists;
};

// Row tiles of the tied lm_head: rpt rows each, ntiles tiles.  The
// kernel-per-phase mode uses 256-thread tiles of P.lm_rpt rows; the
// persistent kernel uses 1024-thread tiles.  Every row's arithmetic is the
// same (tile_compute), and the first maximum does not depend on the tiling.
struct LmGeom {
  int rpt, ntiles;
};

// One lm_head tile whose weights are in R: logits rows [r0, r0+nr) of the m
// tokens from tb, then the tile's first maximum per token (gpt2 chain: with
// the argmaxGpt2 adjustments).
// With amt, token t's tile maximum goes out as two tagged pairs (value, row)
// at amt[2 ((tb + t) ntiles + tile)] instead of to amv / ami.
template <int TCN, int NT>
__device__ __forceinline__ void lm_tile(const DecParams &P, const LmGeom &L, const TileRegs<TCN> &R, int tile, int tb,
                                        int m, const LmLds &s, bool penal, int nban, int nrec, uint2 *amt = nullptr,
                                        int amtag = 0) {
  const int ng = P.D >> 5, rpt = L.rpt;
  const int r0 = tile * rpt, nr = min(rpt, P.V - r0);
  tile_compute_q6<TCN, NT>(R, nr, ng, nr * ng, m, s.qx, tid() % ng, NT % ng, s.part, s.out, rpt);
  for (int e = tid(); e < m * nr; e += NT) {
    const int t = e / nr, r = e - t * nr;
    P.logits[(size_t)(tb + t) * P.V + r0 + r] = s.out[t * rpt + r];
  }
  for (int t = wave_id(); t < m; t += NT / 64) {  // token t on wave t % (NT / 64)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int r = lane_id(); r < nr; r += 64) {
      float v = s.out[t * rpt + r];
      if (penal) v = gpt2_adjust(v, r0 + r, s.lists + 34, nban, s.lists + 2, nrec);
      if (amax_better(v, r0 + r, bv, bi)) {
        bv = v;
        bi = r0 + r;
      }
    }
    wave_argmax(bv, bi);
    if (lane_id() == 0) {
      if (amt) {
        const uint2 pv = tag_pair(__float_as_uint(bv), amtag), pi = tag_pair((uint32_t)bi, amtag);
        coh_st16(amt, 16u * (uint32_t)((tb + t) * L.ntiles + tile), make_uint4(pv.x, pv.y, pi.x, pi.y));
      } else {
        coh_stf(P.amv, 4u * ((tb + t) * P.lm_tiles + tile), bv);
        coh_sti(P.ami, 4u * ((tb + t) * P.lm_tiles + tile), bi);
      }
    }
  }
  __syncthreads();
}

template <int TCN, int NT>
__device__ __forceinline__ void lm_load(const DecParams &P, const LmGeom &L, int tile, TileRegs<TCN> &R) {
  if (tile < L.ntiles) {
    const int ng = P.D >> 5, r0 = tile * L.rpt, nr = min(L.rpt, P.V - r0);
    tile_load<TCN, NT>(P.lm, r0, nr, 0, ng, nr * ng, R);
  }
}

// infer.js:252-287 over hist[0..n) (thread 0): banned = tokens that would
// repeat the last 3-gram, recent = the last 32 tokens.
__device__ __forceinline__ void gpt2_lists(const DecParams &P, int *lists) {
  const int n = st_ld(P, ST_OFF(n_hist));
  int nrec = 0, nban = 0;
  for (int h = max(0, n - 32); h < n; ++h) lists[2 + nrec++] = coh_ldi(P.hist, 4u * h);
  if (n >= 2) {
    const int t1 = coh_ldi(P.hist, 4u * (n - 2)), t2 = coh_ldi(P.hist, 4u * (n - 1));
    for (int h = 0; h < n - 2; ++h)
      if (coh_ldi(P.hist, 4u * h) == t1 && coh_ldi(P.hist, 4u * (h + 1)) == t2) lists[34 + nban++] = coh_ldi(P.hist, 4u * (h + 2));
  }
  lists[0] = nban;
  lists[1] = nrec;
}

// Kernel-per-phase lm_head: row tiles wg, wg + nwg, ...; the normed rows come
// from FINAL (xn) and are staged here as in the persistent kernel; the next
// tile's weights are
// loaded while the current one is computed (two register sets used in turn,
// each with constant indices so both stay in VGPRs).
__device__ void phase_lm(const DecParams &P, int m_all, int wg, int nwg, const Step &st, float *smem) {
  const LmGeom L{P.lm_rpt, P.lm_tiles};
  if (wg >= L.ntiles) return;
  const int lm_rows = st_ld(P, ST_OFF(lm_rows));
  if (lm_rows == 0 || st.done) return;
  const int tb = lm_rows == 1 ? m_all - 1 : 0;
  const int m = m_all - tb;
  const int D = P.D, ng = D >> 5, nq = D >> 2;
  TileRegs<TC> Ra, Rb;
  int tile = wg;
  // the normed rows first, then the weights (loads retire in issue order);
  // thread f of a round stages column f % nq of token f / nq (a token's row
  // is a multiple of 8 columns, so a group's columns are 8 neighbouring lanes)
  float4 xv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int f = min(tid() + k * LT, m * nq - 1);  // branch-free; extra lanes unused
    xv[k] = coh_ld4(P.xn + (size_t)tb * D, 16u * f);
  }
  lm_load<TC, LT>(P, L, tile, Ra);
  LmLds s;
  s.qx = reinterpret_cast<uint32_t *>(smem);
  s.part = smem + m * ng * Q6R;
  s.out = s.part + m * TC * LT;
  s.lists = reinterpret_cast<int *>(s.out + m * L.rpt);  // [0]: nban, [1]: nrec, [2..34): rec, then ban
  const bool penal = P.arch == 1 && st_ld(P, ST_OFF(chain)) != 0;
  if (penal && tid() == 0) gpt2_lists(P, s.lists);
  for (int base = 0; base < m * nq; base += 4 * LT) {
    if (base > 0)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int f = min(base + tid() + k * LT, m * nq - 1);
        xv[k] = coh_ld4(P.xn + (size_t)tb * D, 16u * f);
      }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int f = base + tid() + k * LT;
      const int fc = min(f, m * nq - 1), t = fc / nq;
      q6_stage_col(xv[k], f < m * nq, fc - t * nq, s.qx + t * ng * Q6R);
    }
  }
  __syncthreads();
  const int nban = penal ? s.lists[0] : 0, nrec = penal ? s.lists[1] : 0;
  while (tile < L.ntiles) {
    lm_load<TC, LT>(P, L, tile + nwg, Rb);
    lm_tile<TC, LT>(P, L, Ra, tile, tb, m, s, penal, nban, nrec);
    tile += nwg;
    if (tile >= L.ntiles) break;
    lm_load<TC, LT>(P, L, tile + nwg, Ra);
    lm_tile<TC, LT>(P, L, Rb, tile, tb, m, s, penal, nban, nrec);
    tile += nwg;
  }
}

// First maximum over the tiles' (value, index) pairs of each lm row; the
// chained decode feeds it back as the next input token.
template <int NT>
__device__ void phase_argmax(const DecParams &P, int ntiles, const Step &st, float *smem) {
  const int lm_rows = st_ld(P, ST_OFF(lm_rows));
  if (lm_rows == 0 || st.done) return;
  const int ntok = st_ld(P, ST_OFF(ntok));
  const int tb = lm_rows == 1 ? ntok - 1 : 0;
  constexpr int NW = NT / 64;
  float *rv = smem;
  int *ri = reinterpret_cast<int *>(smem + NW);
  int last = 0;
  for (int t = tb; t < ntok; ++t) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = 0; base < ntiles; base += 16 * NT) {
      float vv[16];
      int iv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {  // all loads of the batch before any compare
        const int k = min(base + (int)tid() + j * NT, ntiles - 1);
        vv[j] = coh_ldf(P.amv, 4u * (t * P.lm_tiles + k));
        iv[j] = coh_ldi(P.ami, 4u * (t * P.lm_tiles + k));
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int k = base + tid() + j * NT;
        if (k < ntiles && amax_better(vv[j], iv[j], bv, bi)) {
          bv = vv[j];
          bi = iv[j];
        }
      }
    }
    wave_argmax(bv, bi);
    __syncthreads();
    if ((tid() & 63) == 0) {
      rv[tid() >> 6] = bv;
      ri[tid() >> 6] = bi;
    }
    __syncthreads();
    if (tid() == 0) {
      float v = rv[0];
      int i = ri[0];
      for (int w = 1; w < NW; ++w)
        if (amax_better(rv[w], ri[w], v, i)) {
          v = rv[w];
          i = ri[w];
        }
      st_st(P, ST_OFF(res) + 4u * t, i);
      last = i;
    }
    __syncthreads();
  }
  if (tid() == 0 && st_ld(P, ST_OFF(chain))) {
    int tok = last;
    if (tok < 0 || tok >= P.V) {  // no finite maximum (non-finite logits)
      st_st(P, ST_OFF(bad_tok), 1);
      tok = 0;
    }
    const int n_hist = st_ld(P, ST_OFF(n_hist));
    coh_sti(P.hist, 4u * n_hist, tok);
    st_st(P, ST_OFF(n_hist), n_hist + 1);
    st_st(P, ST_OFF(tok), tok);
    st_st(P, ST_OFF(pos0), st.pos0 + 1);
    if (tok == st_ld(P, ST_OFF(eos))) st_st(P, ST_OFF(done), 1);
  }
}

__host__ __device__ __forceinline__ int phase_items(const DecParams &P, int ph, int m) {
  switch (ph) {
  case PH_QKV: return P.NH + 2 * P.NKV;
  case PH_ATTN: return m * P.NH * P.nsplit_max;
  case PH_MLP: return P.nchunk;
  case PH_FINAL: return m;
  case PH_LM: return P.lm_grid;
  default: return 1;
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
  float *smem = reinterpret_cast<float *>(smem4);
  const Step st{st_ld(P, ST_OFF(pos0)), st_ld(P, ST_OFF(done)) != 0, st_ld(P, ST_OFF(tag0))};
  const int mm = ONE ? 1 : m;
  const int item = blockIdx.x;
  switch (PH) {
  case PH_QKV: phase_qkv<false>(P, Lw, mm, li, item, st, smem, NoWait{}); break;
  case PH_ATTN: phase_attn<false>(P, Lw, mm, li, item, st, smem, NoWait{}); break;
  case PH_MLP: phase_mlp<false>(P, Lw, mm, li, item, st, smem, NoWait{}); break;
  case PH_FINAL: phase_final(P, mm, item, st, smem); break;
  case PH_LM: phase_lm(P, mm, item, gridDim.x, st, smem); break;
  default: phase_argmax<LT>(P, P.lm_tiles, st, smem); break;
  }
}

// The decode step's attention item (QKV fused in), one instance per tile size.
template <int AQC>
__global__ __launch_bounds__(AT) void k_attn1(DecParams P, LayerW Lw, int li, int m) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  const Step st{st_ld(P, ST_OFF(pos0)), st_ld(P, ST_OFF(done)) != 0, st_ld(P, ST_OFF(tag0))};
  (void)m;
  phase_attn1<false, AQC>(P, Lw, li, blockIdx.x, st, smem, NoWait{});
}

using PhaseKernel = void (*)(DecParams, LayerW, int, int);
static const PhaseKernel kAttn1Kernels[3] = {k_attn1<4>, k_attn1<5>, k_attn1<6>};
static const PhaseKernel kPhaseKernels[2][PH_COUNT] = {
    {k_phase<PH_QKV, 0>, k_phase<PH_ATTN, 0>, k_phase<PH_MLP, 0>, k_phase<PH_FINAL, 0>, k_phase<PH_LM, 0>,
     k_phase<PH_ARGMAX, 0>},
    {k_phase<PH_QKV, 1>, k_phase<PH_ATTN, 1>, k_phase<PH_MLP, 1>, k_phase<PH_FINAL, 1>, k_phase<PH_LM, 1>,
     k_phase<PH_ARGMAX, 1>}};
static const char *const kPhaseNames[PH_COUNT] = {"QKV", "ATTN", "MLP", "FINAL", "LM", "ARGMAX"};

// ---------------------------------------------------------------- persistent kernel
// Mode 3: the single-token decode of `steps` chained tokens in one
// cooperative launch of 1024-thread workgroups, one per CU.  Per layer the
// items are the attention (split, head) items, each with its QKV rows fused
// in, and the MLP chunks; workgroup w runs items w, w + G, ... of every layer in order, so a
// workgroup's next weights are loaded as soon as it has finished its previous
// item, while other workgroups still produce that item's inputs.  After its
// last layer item every workgroup loads its lm_head tile, waits for the last
// layer, forms the final norm itself (no separate FINAL step) and computes
// the tile; the last workgroup to finish its tile takes the argmax.
//
// Ordering is by tags carried in the data instead of kernel boundaries: an
// item stores its outputs as (value, tag) pairs, tag = step epoch * TAGL +
// layer, and a consumer polls exactly the values it reads until they carry
// the tag it needs (the residual, the per-head or per-chunk partials).
// Dependencies:
//   ATTN(l)     <- MLP(l-1), every chunk     (l = 0: the previous step's ARGMAX)
//   MLP(l)      <- ATTN(l), every head (written by the split that merged the head)
//   LM          <- MLP(L-1), every chunk;   ARGMAX: the last LM workgroup
// A buffer is rewritten only by items that depend, through these edges, on
// every reader of its previous contents.  Every item depends only on items
// earlier in the order (layer, stage) and every workgroup runs its items in
// that order, so with all workgroups resident (a cooperative launch) the
// grid always makes progress.  Epochs and tags grow across launches, so
// nothing is ever cleared; they are compared modulo 2^32.  The ARGMAX and
// lm_head counters still use flags (set after a completion wait).
struct FlowGeom {
  int *flags;             // [L][NH + nm] attention heads and MLP chunks, LM counter, ARGMAX
  int ep0, steps;         // epoch of the launch's first step; chained steps
  int m;                  // tokens of a verify step (k_flowm; the decode kernel takes 1)
  int tq, ta, mt;         // k_flowm: tokens per QKV, attention and MLP item (the items of a stage are x token group)
  int fuse;               // k_flowm: no norm items; the QKV, MLP and lm_head items form their tokens' norms
  int na, nm, ni;         // items per layer: attention (split, head) items, MLP chunks; ni = na + nm
  int lm_rpt, lm_tiles;   // lm_head tiles of the 1024-thread role (one per workgroup w < lm_tiles, then w + G ...)
  int kvp;                // k_flow: LDS float offset of the deferred K/V-row slots (kv_flush)
  int xcd;                // k_flow3: the attention items of a (split, KV head) group share an XCD
};

constexpr int FLT = 1024;               // threads per workgroup of the persistent kernel
constexpr unsigned kSpinLimit = 1u << 22;  // polls before a wait gives up (seconds)

__device__ __forceinline__ bool poll_give_up(const DecParams &P, unsigned spins) {
  if (spins > kSpinLimit) {
    st_st(P, ST_OFF(err), 1);
    return true;
  }
  return (spins & 255) == 0 && st_ld(P, ST_OFF(err)) != 0;
}

__device__ __forceinline__ int flag_ld(const int *f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_st(int *f, int v) {
  __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 polls up to three flag ranges until every flag holds >= e; the
// other waves wait at the barrier.  The poll is bounded: on time-out, or
// once another workgroup has failed, st->err is set and the wait returns
// (the host then reports the error; every later wait of the launch returns
// at once, so the grid drains).
// A nonzero `sleep` spaces the polls (s_sleep units of 64 clocks): waits
// that are known to be long poll slowly, so that the flags' memory channel
// is not flooded while other workgroups publish through it.
template <int SLEEP = 0>
__device__ void flow_wait(const DecParams &P, const int *f0, int n0, const int *f1, int n1, const int *f2, int n2,
                          int e) {
  if (tid() < 64) {
    const int lane = tid();
    unsigned spins = 0;
    bool failed = __builtin_amdgcn_readfirstlane(st_ld(P, ST_OFF(err))) != 0;
    while (!failed) {
      bool ok = true;
      for (int i = lane; i < n0; i += 64) ok &= tag_ok((uint32_t)flag_ld(f0 + i), e);
      for (int i = lane; i < n1; i += 64) ok &= tag_ok((uint32_t)flag_ld(f1 + i), e);
      for (int i = lane; i < n2; i += 64) ok &= tag_ok((uint32_t)flag_ld(f2 + i), e);
      if (__all(ok)) break;
      if (SLEEP) __builtin_amdgcn_s_sleep(SLEEP);
      ++spins;
      if ((spins & 15) == 0) failed = __builtin_amdgcn_readfirstlane(st_ld(P, ST_OFF(err))) != 0;
      if (spins > kSpinLimit) {
        if (lane == 0) st_st(P, ST_OFF(err), 1);
        failed = true;
      }
    }
  }
  __syncthreads();
}

// The item's outputs are complete (every thread waits for its own stores),
// then its flag is set.
__device__ __forceinline__ void flow_publish(int *f, int e) {
  wait_stores();
  __syncthreads();
  if (tid() == 0) flag_st(f, e);
}

// Step handoffs of the persistent decode kernel past the last layer.
//  - Workgroup 0 (attention item 0's) forms the last layer's residual and the
//    final norm once and publishes the normed row's Q6 records as tagged
//    pairs (tag st.tag + L) at P.rec; every lm_head workgroup loads those 2 KB
//    instead of gathering the last layer's 110 KB of down partials itself.
//  - Every lm_head tile stores its first maximum (value, row) as two tagged
//    pairs at P.amt (tag st.tag + TAGL - 2), without waiting for its stores.
//    The pairs alternate between two buffers by step parity: step s + 2's
//    tiles depend on every tile of step s + 1, and each of those was written
//    by a workgroup after it read step s's maxima, so no reader of a step's
//    maxima can find them overwritten.
//  - At its first wait of the next step, every workgroup takes the first
//    maximum over the tiles' pairs itself (the same total order, so the same
//    token everywhere): the token for the embedding, and whether the chain
//    emitted eos.  Workgroup 0 also records the step for the host (res,
//    tok, pos0, the history, done, bad_tok; infer.js argmax and the chain
//    rules of phase_argmax).  Its next attention output waits for all of its
//    stores (attn_core), and every later reader of the history (the gpt2
//    lm_head lists) depends on that output, so those stores need no wait of
//    their own.  The last step's maximum is taken by workgroup 0 at the end
//    of the launch.
constexpr int TAG_LM = TAGL - 2;  // st.tag + TAG_LM: the lm_head tiles' maxima


// Waves 0-7 (AMW): the first maximum over the ntiles tiles' tagged pairs of
// tag `want`; tile k is taken by wave (k / 64) % AMW, one 16-byte load per
// lane and round, polled (bounded) until both of its pairs carry the tag (one
// round up to 512 tiles).  Each wave leaves its (value, row) in slots
// [5 + 2 wv], [6 + 2 wv]; the caller combines them after a barrier.
constexpr int AMW = 8;
__device__ __forceinline__ uint2 *flow_amt(const DecParams &P, int e) {
  return P.amt + (size_t)(e & 1) * 2 * P.lm_tiles;
}
__device__ __forceinline__ void flow_tiles_argmax(const DecParams &P, const uint2 *amt, int ntiles, int want,
                                                  int *slots) {
  const int lane = lane_id(), wv = wave_id();
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = 64 * wv; b < ntiles; b += AMW * 64) {
    const uint32_t off = 16u * (uint32_t)min(b + lane, ntiles - 1);
    uint4 u = coh_ld16(amt, off);
    for (unsigned spins = 1; !__all(pair_ok(make_uint2(u.x, u.y), want) && pair_ok(make_uint2(u.z, u.w), want)) &&
                             !poll_give_up(P, spins);
         ++spins) {
      poll_fence();
      u = coh_ld16(amt, off);
    }
    const float v = __uint_as_float(u.x);
    const int i = (int)u.z;
    if (b + lane < ntiles && amax_better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  wave_argmax(bv, bi);
  if (lane == 0) {
    slots[5 + 2 * wv] = __float_as_int(bv);
    slots[6 + 2 * wv] = bi;
  }
}

// Thread 0: the first maximum's row from the AMW waves' slots.
__device__ __forceinline__ int flow_tiles_combine(const int *slots) {
  float v = __int_as_float(slots[5]);
  int i = slots[6];
  for (int k = 1; k < AMW; ++k)
    if (amax_better(__int_as_float(slots[5 + 2 * k]), slots[6 + 2 * k], v, i)) {
      v = __int_as_float(slots[5 + 2 * k]);
      i = slots[6 + 2 * k];
    }
  return i;
}

// Wave 0 of workgroup 0, lane 0: the host's record of a finished step whose
// first maximum is row i at position pos (phase_argmax's rules).
__device__ __forceinline__ void flow_record_step(const DecParams &P, int *slots, int i, int pos) {
  st_st(P, ST_OFF(res), i);
  if (slots[4]) {
    int tok = i;
    if (tok < 0 || tok >= P.V) {  // no finite maximum (non-finite logits)
      st_st(P, ST_OFF(bad_tok), 1);
      tok = 0;
    }
    const int n_hist = slots[2];
    coh_sti(P.hist, 4u * n_hist, tok);
    slots[2] = n_hist + 1;
    st_st(P, ST_OFF(n_hist), n_hist + 1);
    st_st(P, ST_OFF(tok), tok);
    st_st(P, ST_OFF(pos0), pos + 1);
    if (tok == slots[3]) st_st(P, ST_OFF(done), 1);
  }
}

// A workgroup's waits within one step.  resolve(), at the top of every step
// after the first, takes the previous step's token from the lm_head tiles'
// maxima (there no item holds registers, so the poll costs none of theirs).
struct FlowCtl {
  const DecParams &P;
  int *slots;
  int w, ntiles;
  int e, pos;     // the step's epoch and position
  bool pending;   // the previous step's token is still due
  bool done;
  __device__ void resolve() {
    if (pending) {
      PROBE_SET(pos, PROBE_TOP, w);
      PROBE(0);
      if (wave_id() < AMW)
        flow_tiles_argmax(P, flow_amt(P, e - 1), ntiles, (int)((uint32_t)(e - 1) * (uint32_t)TAGL) + TAG_LM, slots);
      __syncthreads();
      if (tid() == 0) {
        const int i = flow_tiles_combine(slots);
        const int tok = i < 0 || i >= P.V ? 0 : i;
        if (w == 0) flow_record_step(P, slots, i, pos - 1);
        slots[0] = tok;
        slots[1] = slots[4] && tok == slots[3];
      }
      __syncthreads();
      done = slots[1] != 0;
      __syncthreads();  // slot 1 is written again only at the next step's resolve
      PROBE(1);
      pending = false;
    }
  }
  template <int SLEEP = 0>
  __device__ bool wait(const int *f0, int n0, const int *f1 = nullptr, int n1 = 0, const int *f2 = nullptr,
                       int n2 = 0) {
    if (done) return true;
    if (n0 + n1 + n2) flow_wait<SLEEP>(P, f0, n0, f1, n1, f2, n2, e);
    return false;
  }
};

// The persistent kernel's lm_head share of one workgroup (tiles wg, wg + G,
// ...).  Workgroup 0 (pub) forms the final norm and publishes its records;
// the others load them.  Returns true when this workgroup computed at least
// one tile.
template <class W>
__device__ bool flow_lm(const DecParams &P, const LmGeom &L, int wg, int nwg, const Step &st, float *smem, bool pub,
                        W &&wait) {
  if (wg >= L.ntiles && !pub) return false;
  const int D = P.D, ng = D >> 5, nrec = ng * Q6R;
  const int ftag = st.tag + P.L;  // the final norm's records
  TileRegs<FTC> Ra, Rb;
  int tile = wg;
  lm_load<FTC, FLT>(P, L, tile, Ra);
  LmLds s;
  float *gl = smem;
  // every region 16-byte aligned (the block sums are read as float4s)
  s.qx = reinterpret_cast<uint32_t *>(gl + al4(3 * D));
  s.part = gl + al4(3 * D) + al4(ng * Q6R);
  s.out = s.part + FTC * FLT;
  s.lists = reinterpret_cast<int *>(s.out + al4(L.rpt));
  float *blk = reinterpret_cast<float *>(s.lists + al4(34 + P.max_seq));
  if (pub) {
    const float *rbias = P.arch == 1 ? P.last_mproj_b : nullptr;
    GainsReg GR;
    gains_load(P, P.norm_f, rbias, GR);
    gains_store(P, rbias, GR, gl);
  }
  PROBE_SET(st.pos0, PROBE_LM, wg);
  PROBE(0);
  if (wait()) return false;
  PROBE(1);
  const bool penal = P.arch == 1 && st_ld(P, ST_OFF(chain)) != 0;
  if (penal && tid() == 0) gpt2_lists(P, s.lists);
  if (pub) {
    final_row<2>(P, 0, blk, gl, s.qx, false, st.tag + P.L - 1);
    __syncthreads();
    for (int i = tid(); i < nrec; i += FLT) coh_st8(P.rec, (uint32_t)i * 8u, tag_pair(s.qx[i], ftag));
  } else {
    // the records, two tagged pairs per 16-byte load (nrec is even)
    const int i = min((int)tid(), (nrec >> 1) - 1);
    uint4 u = coh_ld16(P.rec, 16u * (uint32_t)i);
    if ((int)tid() < (nrec >> 1)) {
      for (unsigned spins = 1; !(pair_ok(make_uint2(u.x, u.y), ftag) && pair_ok(make_uint2(u.z, u.w), ftag)) &&
                               !poll_give_up(P, spins);
           ++spins) {
        poll_fence();
        u = coh_ld16(P.rec, 16u * (uint32_t)i);
      }
      s.qx[2 * i] = u.x;
      s.qx[2 * i + 1] = u.z;
    }
  }
  __syncthreads();
  PROBE(2);
  if (tile >= L.ntiles) return false;
  const int nban = penal ? s.lists[0] : 0, nrc = penal ? s.lists[1] : 0;
  const int amtag = st.tag + TAG_LM;
  uint2 *const amt = flow_amt(P, (int)((uint32_t)st.tag / TAGL));
  while (tile < L.ntiles) {
    lm_load<FTC, FLT>(P, L, tile + nwg, Rb);
    lm_tile<FTC, FLT>(P, L, Ra, tile, 0, 1, s, penal, nban, nrc, amt, amtag);
    tile += nwg;
    if (tile >= L.ntiles) break;
    lm_load<FTC, FLT>(P, L, tile + nwg, Ra);
    lm_tile<FTC, FLT>(P, L, Rb, tile, 0, 1, s, penal, nban, nrc, amt, amtag);
    tile += nwg;
  }
  PROBE(3);
  return true;
}

template <int AQC>
__global__ __launch_bounds__(FLT) void k_flow(DecParams P, FlowGeom F) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  // lines of the KV cache that an XCD's L2 may still hold from before the
  // launch are dropped before any ordinary load of the cache (kv_ld4)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const int w = blockIdx.x, G = gridDim.x;
  const int stride = P.NH + F.nm;
  const int nlm = min(G, F.lm_tiles);  // workgroups with lm_head tiles
  const LmGeom lg{F.lm_rpt, F.lm_tiles};
  const int pos_start = st_ld(P, ST_OFF(pos0));
  int *const slots = flow_slots(smem, F.kvp);
  if (wave_id() == 1 || wave_id() == 2) *kv_slot(smem, F.kvp) = kv_pad(P);  // no deferred K/V row yet
  if (tid() == 0) {
    slots[0] = min(max(st_ld(P, ST_OFF(tok)), 0), P.V - 1);  // the first step's input token
    slots[1] = 0;
    slots[2] = st_ld(P, ST_OFF(n_hist));
    slots[3] = st_ld(P, ST_OFF(eos));
    slots[4] = st_ld(P, ST_OFF(chain));
  }
  __syncthreads();
  if (w >= F.ni && w >= nlm && w != 0) return;  // no item and no lm_head tile in any step
  bool stopped = false;
  for (int step = 0; step < F.steps; ++step) {
    FlowCtl C{P, slots, w, F.lm_tiles, F.ep0 + step, pos_start + step, step > 0, false};
    C.resolve();
    if (C.done) {
      stopped = true;
      break;
    }
    const int e = C.e;
    const Step st{pos_start + step, false, (int)((uint32_t)e * (uint32_t)TAGL)};
    for (int lv = 0; lv < P.L && !C.done; ++lv) {
      // the layer and item indices are made opaque to the compiler: it would
      // otherwise hoist per-thread addresses out of the loops and keep them
      // live past the register budget of a 1024-thread workgroup
      int li = lv;
      asm volatile("" : "+s"(li));
      const LayerW &Lw = P.layers[li];  // fields loaded where they are used (scalar registers are scarce)
      int *const fl = F.flags + li * stride;
      for (int jv = w; jv < F.ni && !C.done; jv += G) {
        int j = jv;
        asm volatile("" : "+s"(j));
        // items poll their inputs' tags (the previous layer's residual and
        // down partials, or this layer's attention partials); the step's
        // token and `done` were taken at its top (resolve)
        if (j < F.na) {
          phase_attn1<true, AQC>(P, Lw, li, j, st, smem, [&] { return C.wait(nullptr, 0); }, F.kvp);
        } else {
          const int it = j - F.na;
          phase_mlp<true>(P, Lw, 1, li, it, st, smem, [&] { return C.wait(nullptr, 0); });
          // a hint for the lm_head's coarse waits, set without waiting for the
          // stores: the data itself carries the tags that decide
          if (!C.done && tid() == 0) flag_st(fl + P.NH + it, e);
        }
      }
    }
    if (!C.done && (w < nlm || w == 0)) {
      // the lm_head waits through the whole layer stack: first slowly on
      // earlier layers, then closely on the last one
      if (P.L > 4) {
        C.wait<127>(F.flags + (P.L - 4) * stride + P.NH, F.nm);
        C.wait<16>(F.flags + (P.L - 2) * stride + P.NH, F.nm);
      }
      const int *dep = F.flags + (P.L - 1) * stride + P.NH;
      // workgroup 0 polls the last layer's data itself; the others wait for
      // its flags, then for the published records
      flow_lm(P, lg, w, G, st, smem, w == 0, [&] { return C.wait(dep, w == 0 ? 0 : F.nm); });
    }
  }
  kv_flush(P, smem, F.kvp);
  if (!stopped && w == 0) {
    // the last step's token, for the host
    const uint32_t e = (uint32_t)(F.ep0 + F.steps - 1);
    if (wave_id() < AMW) flow_tiles_argmax(P, flow_amt(P, (int)e), F.lm_tiles, (int)(e * (uint32_t)TAGL) + TAG_LM, slots);
    __syncthreads();
    if (tid() == 0) flow_record_step(P, slots, flow_tiles_combine(slots), pos_start + F.steps - 1);
  }
}

// ---------------------------------------------------------------- verify step
// The persistent kernel's m-token verify step (k_flowm: speculation's k + 1
// rows, webgpu.js:568-685).  Each layer runs five stages of items; the token
// work of a stage is spread over its items and over the workgroup instead of
// being taken one token at a time:
//   NA(t)  token t's residual (layer 0: the embedding) and attention norm:
//          the residual row xa[t] and the normed row's Q6 records rec[0][t];
//   QKV    (row head, token group): 64 rows of attn.qkv for the group's
//          tokens, the q/k/v rows to P.qkvr, the K/V rows to the cache;
//   ATT    (split, head, token group): the group's scores and P.V over the
//          split, the merges, the W_o slice;
//   NM(t)  token t's residual after attention xb[t] and the MLP norm's
//          records rec[1][t];
//   MLP    (unit block, token group): gate/up rows, activation and the
//          down-projection slice of the group's tokens.
// After the last layer NA(t) forms the final norm's records for the lm_head
// tiles.  A residual is summed once per token rather than once per consumer
// item, so each partial row is read once per token and layer.  Every token's
// arithmetic is the single-token step's (the same functions in the same
// order), so each row of a verify step is, bit for bit, the decode step at
// that position.  The records are tagged pairs like every other handoff, with
// tag st.tag + layer (st.tag + L for the final norm).
constexpr int VQB = 4;  // tokens per batch of the attention item's q/k/v rows
constexpr int VMB = 4;  // tokens per batch of the MLP item's gate/up rows
constexpr int VLB = 4;  // tokens per pass over an lm_head tile

// The n dwords at LDS src as tagged pairs at dst.
__device__ __forceinline__ void rec_put(uint2 *dst, const uint32_t *src, int n, int tag) {
  for (int i = tid(); i < n; i += 1024) coh_st8(dst, (uint32_t)i * 8u, tag_pair(src[i], tag));
}

// n tagged dwords into LDS dst, loaded again until every tag reaches want:
// eight pairs per thread in flight.  Branch-free loads (lanes past n read the
// last pair).
__device__ __forceinline__ void rec_get(const DecParams &P, const uint2 *src, int n, int want, uint32_t *dst) {
  for (int b = 0; b < n; b += 8 * 1024) {
    uint2 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = tag_ld(src, (uint32_t)min(b + (int)tid() + k * 1024, n - 1));
    for (unsigned spins = 1;; ++spins) {
      bool ready = true;
#pragma unroll
      for (int k = 0; k < 8; ++k) ready &= pair_ok(v[k], want);
      if (ready || poll_give_up(P, spins)) break;
      poll_fence();
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = tag_ld(src, (uint32_t)min(b + (int)tid() + k * 1024, n - 1));
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = b + (int)tid() + k * 1024;
      if (i < n) dst[i] = v[k].x;
    }
  }
}

__device__ __forceinline__ uint2 *rec_row(const DecParams &P, int side, int t) {
  return P.rec + ((size_t)side * MAXT + t) * (P.D >> 5) * Q6R;
}

// Token t's residual and norm into the Q6 records at LDS qx.  side 0 at
// layer li < L: the attention norm (phase_attn1's residual and norm); li ==
// L: the final norm (final_row's); side 1: the MLP norm (phase_mlp's).  The
// residual row (xa[t], side 0, or xb[t], side 1; none for the final norm) is
// written when write_x.  scratch holds the gains, the block sums and the
// reduction (norm_scratch floats).  Every thread calls it (it holds
// barriers); the records are complete after the caller's next barrier.
__host__ __device__ inline size_t norm_scratch(size_t D, size_t nbd) { return al4(3 * D) + nbd * D + 32; }
__device__ __forceinline__ void resid_norm(const DecParams &P, int li, int t, int side, const Step &st, float *scratch,
                                           uint32_t *qx, bool write_x, int tok_in = -1) {
  const int D = P.D, nq = D >> 2;
  const bool gpt2 = P.arch == 1, fin = li == P.L;
  const LayerW &Lw = P.layers[min(li, P.L - 1)];
  const float *gain = side ? Lw.n2 : fin ? P.norm_f : Lw.n1;
  const float *rbias = !gpt2 ? nullptr : side ? Lw.proj_b : li == 0 ? nullptr : fin ? P.last_mproj_b : Lw.prev_mproj_b;
  const int np = side ? P.NH : P.nchunk;
  const int want = st.tag + li - (side ? 0 : 1);  // the inputs' tag
  float *gl = scratch;
  float *blk = gl + al4(3 * D), *red = blk + ((np + PB - 1) / PB) * D;
  GainsReg GR;
  gains_load(P, gain, rbias, GR);
  gains_store(P, rbias, GR, gl);
  float4 x;
  if (side == 0 && li == 0) {
    // tok_in: the chained kernel's token (taken at the step's top)
    const int tok = tok_in >= 0 ? tok_in : min(max(st_ld(P, ST_OFF(tok) + 4u * t), 0), P.V - 1);
    x = embed_col(P, tok, min(st.pos0 + t, P.max_seq - 1));
    __syncthreads();
  } else {
    const uint2 *brow = (side ? P.xa : P.xb) + (size_t)t * D;
    const uint2 *prow = side ? P.opart + (size_t)t * P.NH * D : P.dpart + (size_t)t * P.nchunk * D;
    const float4 base = col_base_load<true>(P, brow, nq, want);
    resid_blocks<1, true>(P, prow, np, want, blk);
    __syncthreads();
    PROBE(1);
    // the waves past the row's columns skip the block reads (col_norm leaves
    // their x out)
    x = wave_id() < ((nq + 63) >> 6) ? col_finish(blk, nq, np, base, gl, D, rbias != nullptr) : base;
  }
  uint2 *xo = write_x && !fin ? (side ? P.xb : P.xa) + (size_t)t * D : nullptr;
  col_norm(P, x, gl, red, qx, ColOut{xo, st.tag + li});
}

// Norm item t (the five-stage step): resid_norm, then the records to
// P.rec for the stage's consumers.
__device__ void flowm_norm(const DecParams &P, int li, int t, int side, const Step &st, float *smem) {
  const int ng = P.D >> 5;
  uint32_t *qx = reinterpret_cast<uint32_t *>(smem);  // ng Q6 records
  resid_norm(P, li, t, side, st, smem + al4(ng * Q6R), qx, true);
  __syncthreads();
  rec_put(rec_row(P, side, t), qx, ng * Q6R, st.tag + li);
}

// QKV item of the verify step: rows [rh*64, rh*64 + 64) of attn.qkv (query
// head rh, K head rh - NH or V head rh - NH - NKV) for tokens [t0, t0 + nt):
// phase_qkv's arithmetic (tile_partials, four-lane row sums, RoPE or the
// bias), which is the single-token step's.  The rows go to P.qkvr as tagged
// pairs (K and V rows rounded as the cache stores them), the K and V rows
// also to the cache.  nt <= VQT.
constexpr int VQT = 8;  // tokens per QKV item at most (its LDS)
// hf >= 0 takes half of the row head: dimensions 16 hf .. 16 hf + 15 and
// their RoPE partners 32 + 16 hf .. (32 rows; the per-row arithmetic is the
// full item's, so the rows carry the same bits).
__device__ void flowm_qkv(const DecParams &P, const LayerW &Lw, int li, int rh, int t0, int nt, const Step &st,
                          bool fused, float *smem, int tok_in = -1, int hf = -1) {
  const int D = P.D, ng = D >> 5, rpi = hf < 0 ? HD : HD / 2, nch = rpi * ng;  // rows per item and token
  const int nrow = (P.NH + 2 * P.NKV) * HD;
  const bool gpt2 = P.arch == 1;
  const bool is_q = rh < P.NH, is_k = !is_q && rh < P.NH + P.NKV;
  uint32_t *qx = reinterpret_cast<uint32_t *>(smem);  // nt x ng Q6 records
  float *part = smem + al4(nt * ng * Q6R);            // nt x nch chunk partials
  float *rs = part + nt * nch;                        // nt x 64 row sums
  float *rt = rs + nt * HD;                           // nt x (cos, sin) (gpt2: the bias)
  TileRegs<QC> R;
  if (hf < 0)
    tile_load<QC, QT>(Lw.qkv, rh * HD, HD, 0, ng, nch, R);
  else
    tile_load<QC, QT>(Lw.qkv, rh * HD + 16 * hf, 16, rh * HD + 32 + 16 * hf, ng, nch, R);
  if ((int)tid() < nt * HD) {
    const int tt = tid() / HD, d = tid() - tt * HD;
    if (gpt2) {
      rt[tt * 2 * HD + d] = Lw.qkv_b[rh * HD + d];
    } else {
      const size_t ri = (size_t)min(st.pos0 + t0 + tt, P.max_seq - 1) * HD + d;
      rt[tt * 2 * HD + d] = P.rope_cos[ri];
      rt[tt * 2 * HD + HD + d] = P.rope_sin[ri];
    }
  }
  if (fused) {
    // each token's residual and norm here (the row head 0 item writes xa)
    float *scratch = rt + al4(nt * 2 * HD);
    for (int tt = 0; tt < nt; ++tt)
      resid_norm(P, li, t0 + tt, 0, st, scratch, qx + tt * ng * Q6R, rh == 0 && hf <= 0, tok_in);
  } else {
    rec_get(P, rec_row(P, 0, t0), nt * ng * Q6R, st.tag + li, qx);
  }
  __syncthreads();
  PROBE(2);
  tile_partials<QC>(R, ng, nch, nt, qx, part);
  __syncthreads();
  PROBE(3);
  // the nt x rpi row sums, four lanes each (the decode attention item's
  // order), at their head dimension
  for (int base = 0; base < nt * rpi; base += 256) {
    const int r = base + (int)(tid() >> 2);
    const int rr = min(r, nt * rpi - 1), tr = rr / rpi, lr = rr - tr * rpi;
    const float a = row_sum4(part + tr * nch + lr * ng, ng, tid() & 3);
    const int dim = hf < 0 ? lr : (lr < 16 ? 16 * hf + lr : 16 + 16 * hf + lr);
    if ((tid() & 3) == 0 && r < nt * rpi) rs[tr * HD + dim] = a;
  }
  __syncthreads();
  PROBE(4);
  // token t0 + tt on wave tt, lane d = head dimension d
  for (int tt = wave_id(); tt < nt; tt += NWV) {
    const int d = lane_id(), t = t0 + tt, pos = st.pos0 + t;
    float v = rs[tt * HD + d];
    if (gpt2) {
      v = v + rt[tt * 2 * HD + d];  // the bias
    } else if (is_q || is_k) {
      const float mate = __shfl_xor(v, 32);  // rotate-half partner d +- 32
      v = __builtin_fmaf(v, rt[tt * 2 * HD + d], (d < 32 ? -mate : mate) * rt[tt * 2 * HD + HD + d]);
    }
    if (hf >= 0 && ((d >> 4) & 1) != hf) continue;  // a dimension of the other half
    float r = v;
    if (!is_q) {
      const int kvh = is_k ? rh - P.NH : rh - P.NH - P.NKV;
      const size_t k = kv_index(P, li, is_k ? 0 : 1, kvh, pos) + d;
      if (P.kv_fp16) {
        const __half hv = __float2half_rn(v);
        r = __half2float(hv);
        coh_sth(P.kv, 2u * (uint32_t)k, __half_as_ushort(hv));
      } else {
        coh_stf(P.kv, 4u * (uint32_t)k, v);
      }
    }
    tag_st(P.qkvr, (uint32_t)((li * MAXT + t) * nrow + rh * HD + d), r, st.tag + li);
  }
}

// The q rows of tokens [u0, u1) of head h and the K and V rows of tokens
// [0, u1) of KV head kvh from layer li's P.qkvr into LDS (qrows: row t; kvn:
// row t = K then V), each pair loaded again until its tag reaches want.  An
// attention item reads the K/V rows of earlier token groups, whose items may
// run a layer ahead: each layer keeps its own rows, so none is overwritten
// within the pass.
__device__ __forceinline__ void qkv_rows_get(const DecParams &P, int li, int want, int u0, int u1, int h, int kvh,
                                             float *qrows, float *kvn) {
  const int nrow = (P.NH + 2 * P.NKV) * HD;
  const int nqr = (u1 - u0) * HD, n = nqr + u1 * 2 * HD;  // <= 3 x 16 x 64
  uint32_t src[3];
  float *dst[3];
  uint2 v[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int i = min((int)tid() + k * 1024, n - 1);
    int t, col;
    if (i < nqr) {
      t = u0 + i / HD;
      col = h * HD + (i - (i / HD) * HD);
      dst[k] = qrows + t * HD + (col - h * HD);
    } else {
      const int j = i - nqr, tk = j / (2 * HD), e = j - tk * 2 * HD;  // e < 64: K, else V
      t = tk;
      col = (e < HD ? P.NH + kvh : P.NH + P.NKV + kvh) * HD + (e & (HD - 1));
      dst[k] = kvn + tk * 2 * HD + e;
    }
    src[k] = (uint32_t)((li * MAXT + t) * nrow + col);
    v[k] = tag_ld(P.qkvr, src[k]);
  }
  for (unsigned spins = 1;; ++spins) {
    bool ready = true;
#pragma unroll
    for (int k = 0; k < 3; ++k) ready &= pair_ok(v[k], want);
    if (ready || poll_give_up(P, spins)) break;
    poll_fence();
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = tag_ld(P.qkvr, src[k]);
  }
#pragma unroll
  for (int k = 0; k < 3; ++k)
    if ((int)tid() + k * 1024 < n) *dst[k] = __uint_as_float(v[k].x);
}

// Attention item (split sp, head h, tokens [u0, u1)) of the verify step: the
// scores, softmax statistics and P.V of every token of the range whose
// position reaches the split (attn_core's arithmetic), the merges (wave w
// takes tokens ta + w, ta + w + 16, ...) and the W_o slice of each token
// this item completes.  Cached keys (< pos0) come from the cache; the pass's
// own K/V rows come from the QKV items (rounded as the cache holds them).
template <bool MS = true>
__device__ void flowm_attn(const DecParams &P, const LayerW &Lw, int li, int item, int u0, int u1, const Step &st,
                           int m, float *smem) {
  const int sp = item / P.NH, h = item - sp * P.NH;
  const int pos0 = st.pos0, s0 = sp * ACH;
  if (s0 > pos0 + u1 - 1) return;  // no token of the range reaches this split
  const int rep = P.NH / P.NKV, kvh = h / rep;
  const int D = P.D;
  const int ta = max(u0, s0 - pos0);  // the first token of the range whose position reaches this split
  const int knew = pos0 - s0;         // keys from knew on are the pass's own rows (LDS row key - knew)
  const int ncached = min(max(knew, 0), ACH);
  const int wv = wave_id(), lane = lane_id();
  float *kvn = smem;                  // m x (K row, V row)
  float *qrows = kvn + m * 2 * HD;    // m x 64 queries
  float *wacc = qrows + m * HD, *wm = wacc + m * AW * HD, *wl = wm + m * AW;  // per token: AW x 64 P.V, AW maxima, sums
  uint32_t *attq = reinterpret_cast<uint32_t *>(wl + m * AW);  // m x 2 Q6 records: the head outputs
  // the W_o slice, loaded only by an item that completes some token's head
  // output (its only split, or the merging last split); at 2048 context the
  // other seven split items of a head would fetch 38 KB each and drop it
  bool need_o = !MS;
  if constexpr (MS)
    for (int t = ta; t < u1; ++t) {
      const int ns = (pos0 + t) / ACH + 1;
      need_o |= ns == 1 || sp == ns - 1;
    }
  TileRegs<SC> Ro;
  if (need_o) slice_load<SC, AT>(Lw.proj, 2 * h, D, Ro);
  float4 kr[4];
  float vr[16];
  attn_k_load(P, li, kvh, s0, ncached, kr);  // cached positions: written by earlier steps
  attn_v_load(P, li, kvh, s0, ncached, vr);
  qkv_rows_get(P, li, st.tag + li, u0, u1, h, kvh, qrows, kvn);
  __syncthreads();
  PROBE(1);
  // this thread's K quarter and V values of the split, cached or the pass's
  // own (row key - knew, clamped: keys past the range's last row are past
  // every count of the range)
  const int kp = tid() >> 2, ku = tid() & 3;
  float4 kk[4];
  float vs[16];
  if (16 * wv + 15 >= knew) {
    // a wave holding one of the pass's own keys (wave-uniform): LDS rows
    // where the key is new, the cache's otherwise
    const float4 *kn = reinterpret_cast<const float4 *>(kvn + 2 * HD * min(max(kp - knew, 0), u1 - 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) kk[j] = kp >= knew ? kn[4 * ku + j] : kr[j];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int key = 16 * wv + k;
      vs[k] = key >= knew ? kvn[2 * HD * min(max(key - knew, 0), u1 - 1) + HD + lane] : vr[k];
    }
  } else {
    // every key of the wave is cached: no LDS read (at decode all waves but
    // the newest key's; the reads of the others cost the LDS 0.5 us a layer)
#pragma unroll
    for (int j = 0; j < 4; ++j) kk[j] = kr[j];
#pragma unroll
    for (int k = 0; k < 16; ++k) vs[k] = vr[k];
  }
  PROBE(4);
  // every token's scores, wave statistics and P.V (attn_core's arithmetic;
  // keys past the count have weight 0 and finite values, which changes at
  // most the sign of a zero sum, and the Q6 staging of the output drops it)
  for (int t = ta; t < u1; ++t) {
    const int cnt = min(ACH, pos0 + t + 1 - s0);
    // a wave whose keys all lie past the count skips the arithmetic (as in
    // attn_core: -inf, +0 and +0 are what it would give)
    float mw = -INFINITY, lw = 0.f, acc = 0.f;
    if (16 * wv < cnt) {
      float pt = 0.f;
      if (kp < cnt) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        const float *qq = qrows + t * HD + 16 * ku;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          a0 = __builtin_fmaf(qq[4 * j + 0], kk[j].x, a0);
          a1 = __builtin_fmaf(qq[4 * j + 1], kk[j].y, a1);
          a2 = __builtin_fmaf(qq[4 * j + 2], kk[j].z, a2);
          a3 = __builtin_fmaf(qq[4 * j + 3], kk[j].w, a3);
        }
        pt = (a0 + a1) + (a2 + a3);
      }
      pt = pt + dpp_f<0xB1>(pt);
      pt = pt + dpp_f<0x4E>(pt);
      const float score = kp < cnt ? pt * P.attn_scale : -INFINITY;
      mw = wave_max(score);
      const float e = kp < cnt ? expf(score - mw) : 0.f;
      lw = wave_sum(ku == 0 ? e : 0.f);
#pragma unroll
      for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(readlane_f(e, 4 * k), vs[k], acc);
    }
    wacc[(t * AW + wv) * HD + lane] = acc;
    if (lane == 0) {
      wm[t * AW + wv] = mw;
      wl[t * AW + wv] = lw;
    }
  }
  PROBE(5);
  // the workgroup's earlier stores (a K/V cache row of an earlier item) are
  // complete before any output of this item becomes visible
  wait_stores();
  __syncthreads();
  PROBE(2);
  if constexpr (!MS) {
    // every token of the pass in one split (the launch's positions < ACH):
    // the split's statistics, its output, the W_o slice
    for (int t = ta + wv; t < u1; t += NWV) {
      float mx, l, own;
      split_merge(wm + t * AW, wl + t * AW, wacc + t * AW * HD, mx, l, own);
      q6_stage_lanes(own / l, attq + t * 2 * Q6R);
    }
    __syncthreads();
    PROBE(3);
    for (int t = ta; t < u1; ++t)
      slice_gemv<SC, AT>(Ro, D, attq + t * 2 * Q6R, P.opart + (size_t)(t * P.NH + h) * D, st.tag + li, Lw.dbg & 1);
    return;
  }
  // each token's split statistics from its wave partials, in wave order; a
  // solo split stages its output; of a multi-split token, the last split
  // (the fewest keys) merges and the others publish their partials as tagged
  // pairs (m, l, acc[64]): no completion wait and no counter on the chain.
  // A lower split of the head has a lower item index, so a merging item
  // never waits for an item that its own workgroup has yet to run.
  for (int t = ta + wv; t < u1; t += NWV) {
    const int ns = (pos0 + t) / ACH + 1;
    float mx, l, own;
    split_merge(wm + t * AW, wl + t * AW, wacc + t * AW * HD, mx, l, own);
    if (ns == 1) {
      q6_stage_lanes(own / l, attq + t * 2 * Q6R);
    } else if (sp == ns - 1) {
      // kept for the merge
      wacc[t * AW * HD + lane] = own;
      if (lane == 0) {
        wm[t * AW] = mx;
        wl[t * AW] = l;
      }
    } else {
      uint2 *dst = P.attpt + ((size_t)(t * P.NH + h) * P.nsplit_max + sp) * APT;
      tag_st(dst, 2u + lane, own, st.tag + li);
      if (lane == 0) {
        tag_st(dst, 0, mx, st.tag + li);
        tag_st(dst, 1, l, st.tag + li);
      }
    }
  }
  __syncthreads();
  // the merging tokens' other splits into LDS (wave partial slots 1 .. AW-1
  // of the token, free after the merge above), polled until every tag is
  // there, then the merges; nothing of this when the item merges no token
  int nt = 0;  // tokens of [ta, u1) this item merges: t with ns(t) - 1 == sp > 0
  for (int t = ta; t < u1; ++t) nt += (pos0 + t) / ACH == sp && sp > 0;
  {
    const int per = sp * APT;  // splits 0 .. sp-1
    for (int b = 0; b < nt * per; b += 1024) {
      const int i = min(b + (int)tid(), nt * per - 1);
      int k = i / per, t = ta;
      for (;; ++t)  // the k-th merging token
        if ((pos0 + t) / ACH == sp && k-- == 0) break;
      const int r = i - (i / per) * per, j = r / APT, e = r - j * APT;
      const uint2 *src = P.attpt + ((size_t)(t * P.NH + h) * P.nsplit_max + j) * APT;
      uint2 v = tag_ld(src, (uint32_t)e);
      for (unsigned spins = 1; !pair_ok(v, st.tag + li) && !poll_give_up(P, spins); ++spins) {
        poll_fence();
        v = tag_ld(src, (uint32_t)e);
      }
      if (b + (int)tid() < nt * per) wacc[t * AW * HD + HD + r] = __uint_as_float(v.x);
    }
    if (nt > 0) __syncthreads();  // uniform in the workgroup
    for (int t = ta + wv; t < u1; t += NWV) {
      const int ns = (pos0 + t) / ACH + 1;
      if (ns == 1 || sp != ns - 1) continue;
      // the splits of (t, h) in split order, this one's (the last) from its own slot
      const float *parts = wacc + t * AW * HD + HD;  // split j: m, l, acc[64] at j * APT
      const float mx = wm[t * AW], l = wl[t * AW], own = wacc[t * AW * HD + lane];
      const int d = lane;
      float M = parts[0];
      for (int j = 1; j < ns; ++j) M = fmaxf(M, j == sp ? mx : parts[j * APT]);
      const float m0 = parts[0], l0 = parts[1], a0 = parts[2 + d];
      const float w0 = expf(m0 - M);
      float ls = __builtin_fmaf(l0, w0, 0.f), as = __builtin_fmaf(a0, w0, 0.f);
      for (int j = 1; j < ns; ++j) {
        const float mj = j == sp ? mx : parts[j * APT];
        const float lj = j == sp ? l : parts[j * APT + 1];
        const float aj = j == sp ? own : parts[j * APT + 2 + d];
        const float w = expf(mj - M);
        ls = __builtin_fmaf(lj, w, ls);
        as = __builtin_fmaf(aj, w, as);
      }
      q6_stage_lanes(as / ls, attq + t * 2 * Q6R);
    }
    if (nt > 0) __syncthreads();
  }
  PROBE(3);
  for (int t = ta; t < u1; ++t) {
    const int ns = (pos0 + t) / ACH + 1;
    if (ns == 1 || sp == ns - 1)
      slice_gemv<SC, AT>(Ro, D, attq + t * 2 * Q6R, P.opart + (size_t)(t * P.NH + h) * D, st.tag + li, Lw.dbg & 1);
  }
}

// MLP item of the verify step: hidden units [item*UNITS, (item+1)*UNITS) of
// tokens [ta, ta + m) (phase_mlp's arithmetic), VMB tokens per batch, then
// the units' slice of the down projection for each of them.
__device__ void flowm_mlp(const DecParams &P, const LayerW &Lw, int li, int item, const Step &st, int ta, int m,
                          bool fused, float *smem) {
  const int D = P.D, ng = D >> 5, nch = UNITS * ng, S = (MT / ng) * ng;
  const bool gpt2 = P.arch == 1;
  uint32_t *qx = reinterpret_cast<uint32_t *>(smem);                   // m x ng Q6 records
  float *part = smem + al4(m * ng * Q6R);                              // VMB x (gate || up) chunk partials
  float *rsum = part + VMB * 2 * nch;                                  // VMB x (gate || up) row sums
  uint32_t *hq = reinterpret_cast<uint32_t *>(rsum + VMB * 2 * UNITS);  // m x 2 Q6 records of h
  MlpPre M;
  mlp_pre_up(P, Lw, item, M);
  slice_load<MC, MT>(Lw.w2, 2 * item, D, M.Rd);
  const int want = st.tag + li;
  if (fused) {
    // each token's residual and norm here (the unit block 0 item writes xb)
    float *scratch = reinterpret_cast<float *>(hq + al4(m * 2 * Q6R));  // 16-byte aligned: float4 gains and blocks
    for (int tt = 0; tt < m; ++tt) resid_norm(P, li, ta + tt, 1, st, scratch, qx + tt * ng * Q6R, item == 0);
  } else {
    rec_get(P, rec_row(P, 1, ta), m * ng * Q6R, want, qx);
  }
  __syncthreads();
  PROBE(2);
  const int wv = wave_id(), lane = lane_id(), g = tid() % ng;
  for (int t0 = 0; t0 < m; t0 += VMB) {
    const int nt = min(VMB, m - t0);
    for (int tt = 0; tt < nt; ++tt) {
      // gate chunks then up chunks against the thread's one group record
      float *pt = part + tt * 2 * nch;
      uint4 w[2 * MC];
      float ws[2 * MC], o[2 * MC];
#pragma unroll
      for (int k = 0; k < MC; ++k) {
        w[k] = M.Rg.w[k];
        ws[k] = M.Rg.s[k];
        w[MC + k] = M.Ru.w[k];
        ws[MC + k] = M.Ru.s[k];
      }
      q4_dot6_planes<2 * MC>(w, ws, qx + ((t0 + tt) * ng + g) * Q6R, o);
#pragma unroll
      for (int k = 0; k < MC; ++k) {
        const int c = tid() + k * S;
        if ((int)tid() < S && c < nch) {
          pt[c] = o[k];
          if (!gpt2) pt[nch + c] = o[MC + k];
        }
      }
    }
    __syncthreads();
    PROBE(3);
    for (int tt = 0; tt < nt; ++tt) {
      // row r (gate rows, then up rows): lane s adds partials s, s + 8, ...
      // in order, then a fixed 8-lane tree
      const float *pt = part + tt * 2 * nch;
      const int r = tid() >> 3, s = tid() & 7;
      const int nrows = gpt2 ? UNITS : 2 * UNITS;
      const float *pr = pt + (r < UNITS ? 0 : nch) + (r & (UNITS - 1)) * ng;
      float a = 0.f;
      if (r < nrows)
        for (int k = s; k < ng; k += 8) a = a + pr[k];
      a = sum8f(a);
      if (s == 0 && r < nrows) rsum[tt * 2 * UNITS + r] = a;
    }
    __syncthreads();
    // token t0 + tt's activation on wave tt (unit = lane); the next batch's
    // row sums overwrite rsum only after its partials' barrier
    for (int tt = wv; tt < nt; tt += NWV) {
      const float *rt = rsum + tt * 2 * UNITS;
      const float gv = rt[lane];
      float hv;
      if (gpt2) {
        const float v = gv + M.fcb;
        hv = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
      } else {
        hv = (gv / (1.0f + expf(-gv))) * rt[UNITS + lane];
      }
      q6_stage_lanes(hv, hq + (t0 + tt) * 2 * Q6R);
    }
  }
  __syncthreads();
  PROBE(4);
  for (int t = 0; t < m; ++t)
    slice_gemv<MC, MT>(M.Rd, D, hq + t * 2 * Q6R, P.dpart + ((size_t)(ta + t) * P.nchunk + item) * D, want,
                       Lw.dbg & 2);
}

// lm_head share of the verify step (tiles wg, wg + nwg, ...): every token's
// logits rows and tile maxima against the final norm's records, VLB tokens
// per pass over a tile (no penalties: a verify pass is greedy).  Returns
// true when this workgroup computed at least one tile.
__device__ bool flowm_lm(const DecParams &P, const LmGeom &L, int wg, int nwg, const Step &st, int m, bool fused,
                         float *smem, int amtag) {
  if (wg >= L.ntiles) return false;
  const int ng = P.D >> 5;
  TileRegs<FTC> R;
  int tile = wg;
  lm_load<FTC, FLT>(P, L, tile, R);
  LmLds s;
  s.qx = reinterpret_cast<uint32_t *>(smem);
  s.part = smem + al4(m * ng * Q6R);
  s.out = s.part + VLB * FTC * FLT;
  s.lists = nullptr;
  if (fused) {
    // each token's final norm here
    float *scratch = s.out + al4(VLB * L.rpt);  // 16-byte aligned
    for (int t = 0; t < m; ++t) resid_norm(P, P.L, t, 0, st, scratch, s.qx + t * ng * Q6R, false);
  } else {
    rec_get(P, rec_row(P, 0, 0), m * ng * Q6R, st.tag + P.L, s.qx);
  }
  __syncthreads();
  for (;;) {
    for (int t0 = 0; t0 < m; t0 += VLB) {
      LmLds u = s;
      u.qx = s.qx + t0 * ng * Q6R;
      lm_tile<FTC, FLT>(P, L, R, tile, t0, min(VLB, m - t0), u, false, 0, 0, P.amtv, amtag);
    }
    tile += nwg;
    if (tile >= L.ntiles) break;
    lm_load<FTC, FLT>(P, L, tile, R);
  }
  return true;
}

// Every row's first maximum over the tiles' tagged maxima (tag `want`), one
// wave per row, each lane's 16-byte loads polled (bounded) until both pairs
// carry the tag; the relation is a total order on (value, index), so the
// order of the comparisons does not change the result.
__device__ void flowm_argmax(const DecParams &P, int ntiles, int m, int want) {
  for (int t = wave_id(); t < m; t += NWV) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = 0; base < ntiles; base += 64) {
      const uint32_t off = 16u * (uint32_t)(t * ntiles + min(base + lane_id(), ntiles - 1));
      uint4 u = coh_ld16(P.amtv, off);
      for (unsigned spins = 1; !__all(pair_ok(make_uint2(u.x, u.y), want) && pair_ok(make_uint2(u.z, u.w), want)) &&
                               !poll_give_up(P, spins);
           ++spins) {
        poll_fence();
        u = coh_ld16(P.amtv, off);
      }
      const float v = __uint_as_float(u.x);
      const int i = (int)u.z;
      if (base + lane_id() < ntiles && amax_better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
    wave_argmax(bv, bi);
    if (lane_id() == 0) st_st(P, ST_OFF(res) + 4u * t, bi);
  }
}

// One verify step of m tokens in one launch (the stages above), then every
// row's argmax.  Items are numbered per layer [NA(t) | QKV (row head, token
// group of F.tq) | ATT (split, head, token group of F.ta) | NM(t) | MLP (unit
// block, token group of F.mt)] and item j runs on workgroup j % G, each
// workgroup taking its items layer by layer in order; an item waits only for
// items of earlier stages or layers, so every wait ends.  The step is not
// chained.
__global__ __launch_bounds__(FLT) void k_flowm(DecParams P, FlowGeom F) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // as in k_flow: no stale cache lines of the KV cache
  const int w = blockIdx.x, G = gridDim.x, m = F.m;
  const int stride = P.NH + F.nm;
  const int nlm = min(G, F.lm_tiles);
  const LmGeom lg{F.lm_rpt, F.lm_tiles};
  int *const red = reinterpret_cast<int *>(smem);
  const int e = F.ep0;
  const Step st{st_ld(P, ST_OFF(pos0)), false, (int)((uint32_t)e * (uint32_t)TAGL)};
  const int nrh = P.NH + 2 * P.NKV;
  const int ngq = (m + F.tq - 1) / F.tq, nga = (m + F.ta - 1) / F.ta, ngm = (m + F.mt - 1) / F.mt;  // token groups
  // norm items per stage; a fused step leaves them idle (its QKV, MLP and
  // lm_head items form their tokens' norms)
  const int iq = m, ia = iq + nrh * ngq, inm = ia + F.na * nga, im = inm + m, ni = im + F.nm * ngm;
  for (int lv = 0; lv < P.L; ++lv) {
    int li = lv;
    asm volatile("" : "+s"(li));
    const LayerW &Lw = P.layers[li];
    int *const fl = F.flags + li * stride;
    for (int jv = w; jv < ni; jv += G) {
      int j = jv;
      asm volatile("" : "+s"(j));
      __syncthreads();  // the previous item's LDS is free
      if (j < iq) {
        if (!F.fuse) flowm_norm(P, li, j, 0, st, smem);
      } else if (j < ia) {
        const int tg = (j - iq) / nrh, rh = (j - iq) - tg * nrh;
        flowm_qkv(P, Lw, li, rh, tg * F.tq, min(F.tq, m - tg * F.tq), st, F.fuse, smem);
      } else if (j < inm) {
        const int tg = (j - ia) / F.na, it = (j - ia) - tg * F.na;
        flowm_attn(P, Lw, li, it, tg * F.ta, min(m, (tg + 1) * F.ta), st, m, smem);
      } else if (j < im) {
        if (!F.fuse) flowm_norm(P, li, j - inm, 1, st, smem);
      } else {
        const int tg = (j - im) / F.nm, it = (j - im) - tg * F.nm;
        flowm_mlp(P, Lw, li, it, st, tg * F.mt, min(F.mt, m - tg * F.mt), F.fuse, smem);
        // a hint for the lm_head's coarse waits (the records carry the tags that decide)
        if (tid() == 0) flag_st(fl + P.NH + it, e);
      }
    }
  }
  if (!F.fuse && w < m) {
    __syncthreads();
    flowm_norm(P, P.L, w, 0, st, smem);  // the final norm of token w
  }
  if (w < nlm) {
    if (P.L > 4) {
      flow_wait<127>(P, F.flags + (P.L - 4) * stride + P.NH, F.nm, nullptr, 0, nullptr, 0, e);
      flow_wait<16>(P, F.flags + (P.L - 2) * stride + P.NH, F.nm, nullptr, 0, nullptr, 0, e);
    }
    __syncthreads();
    // each tile stores its tokens' maxima as tagged pairs, without waiting;
    // workgroup 0 then takes every row's argmax over them
    flowm_lm(P, lg, w, G, st, m, F.fuse, smem, st.tag + TAG_LM);
    if (w == 0) flowm_argmax(P, F.lm_tiles, m, st.tag + TAG_LM);
  }
}

// The attention item that stage slot a (workgroup ia + a, or ia + a - G
// ...) runs in k_flow3.  Workgroups go to the eight XCDs round-robin, each
// with its own L2; with F.xcd the rep items of a (split, KV head) group --
// the query heads that read the same K/V split -- sit on workgroups of one
// XCD, so the group's split is read from HBM once and from that L2 by the
// others.  Slot a is the k-th of its XCD's slots; XCD x runs groups
// x, x + 8, ... (g = split * NKV + kvh), rep items each.  (F.xcd is set
// when the stage's items and groups divide evenly over the eight XCDs.)
__device__ __forceinline__ int flow3_attn_item(const DecParams &P, const FlowGeom &F, int a, int ia) {
  if (!F.xcd) return a;
  const int x = (ia + a) & 7, first = (x - ia) & 7, k = (a - first) >> 3;
  const int rep = P.NH / P.NKV, kg = k / rep, r = k - kg * rep;
  const int g = x + 8 * kg, sp = g / P.NKV, kvh = g - sp * P.NKV;
  return sp * P.NH + kvh * rep + r;
}

// The chained decode step in three stages per layer (the verify step's fused
// items at one row): QKV items (half a row head: 32 rows of attn.qkv, the
// dimensions 16 hf .. 16 hf + 15 and their RoPE partners, each item forming
// the token's residual and norm; row head 0's first half writes the residual
// row; measured against whole row heads: 135M after a 512-token prompt 455 ->
// 450 us per token, 360M after 1536 tokens 674 -> 664, unchanged at short
// context),
// attention items (split, head) that read the q/k/v rows from P.qkvr, and
// the MLP items; then k_flow's lm_head share and step handoffs.  Every row
// head's rows are formed once, where k_flow's attention items each form
// their query head's and their K/V head's rows; that costs a handoff per
// layer and pays where the rows are many (d_model 960) or the splits are (a
// head's split items each form its rows).  Each QKV item first waits for
// its workgroup's earlier stores: the K/V cache row of the previous layer
// (or step) is then complete before the workgroup's next tagged output, on
// which every later reader of that row depends.  The arithmetic is the
// verify step's, so the rows are bit for bit k_flow's.
template <bool MS>
__global__ __launch_bounds__(FLT) void k_flow3(DecParams P, FlowGeom F) {
  extern __shared__ float4 smem4[];
  float *smem = reinterpret_cast<float *>(smem4);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // as in k_flow: no stale cache lines of the KV cache
  const int w = blockIdx.x, G = gridDim.x;
  const int stride = P.NH + F.nm;
  const int nlm = min(G, F.lm_tiles);
  const LmGeom lg{F.lm_rpt, F.lm_tiles};
  const int nrh = P.NH + 2 * P.NKV;
  const int ia = 2 * nrh, im = ia + F.na, ni = im + F.nm;  // items per layer: QKV halves | attention | MLP
  const int pos_start = st_ld(P, ST_OFF(pos0));
  int *const slots = flow_slots(smem, F.kvp);
  if (tid() == 0) {
    slots[0] = min(max(st_ld(P, ST_OFF(tok)), 0), P.V - 1);
    slots[1] = 0;
    slots[2] = st_ld(P, ST_OFF(n_hist));
    slots[3] = st_ld(P, ST_OFF(eos));
    slots[4] = st_ld(P, ST_OFF(chain));
  }
  __syncthreads();
  if (w >= ni && w >= nlm && w != 0) return;  // no item and no lm_head tile in any step
  PROBE_INIT();
  bool stopped = false;
  for (int step = 0; step < F.steps; ++step) {
    FlowCtl C{P, slots, w, F.lm_tiles, F.ep0 + step, pos_start + step, step > 0, false};
    C.resolve();
    if (C.done) {
      stopped = true;
      break;
    }
    const int e = C.e;
    const Step st{pos_start + step, false, (int)((uint32_t)e * (uint32_t)TAGL)};
    const int tok = slots[0];
    for (int lv = 0; lv < P.L; ++lv) {
      int li = lv;
      asm volatile("" : "+s"(li));
      const LayerW &Lw = P.layers[li];
      int *const fl = F.flags + li * stride;
      for (int jv = w; jv < ni; jv += G) {
        int j = jv;
        asm volatile("" : "+s"(j));
        __syncthreads();  // the previous item's LDS is free
        PROBE_SET(st.pos0, li, j);
        PROBE(0);
        if (j < ia) {
          wait_stores();
          flowm_qkv(P, Lw, li, j >> 1, 0, 1, st, true, smem, tok, j & 1);
        } else if (j < im) {
          flowm_attn<MS>(P, Lw, li, flow3_attn_item(P, F, j - ia, ia), 0, 1, st, 1, smem);
        } else {
          const int it = j - im;
          flowm_mlp(P, Lw, li, it, st, 0, 1, true, smem);
          if (tid() == 0) flag_st(fl + P.NH + it, e);  // the lm_head's coarse waits
        }
        PROBE(7);
      }
    }
    if (w < nlm || w == 0) {
      __syncthreads();  // the last item's LDS is free
      // no coarse, spaced waits on earlier layers' flags before this one:
      // measured without them, 135M 392.4 -> 391.2 us per token at a 32-token
      // prompt, 451.7 -> 447.5 us at 512, 360M 661.6 -> 656.5 us at 1536
      const int *dep = F.flags + (P.L - 1) * stride + P.NH;
      flow_lm(P, lg, w, G, st, smem, w == 0, [&] { return C.wait(dep, w == 0 ? 0 : F.nm); });
    }
    __syncthreads();  // the slots are read before the next step's resolve writes them
  }
  if (!stopped && w == 0) {
    const uint32_t e = (uint32_t)(F.ep0 + F.steps - 1);
    if (wave_id() < AMW) flow_tiles_argmax(P, flow_amt(P, (int)e), F.lm_tiles, (int)(e * (uint32_t)TAGL) + TAG_LM, slots);
    __syncthreads();
    if (tid() == 0) flow_record_step(P, slots, flow_tiles_combine(slots), pos_start + F.steps - 1);
  }
  PROBE_END();
}

using FlowKernel = void (*)(DecParams, FlowGeom);
static const FlowKernel kFlowKernels[3] = {k_flow<4>, k_flow<5>, k_flow<6>};



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
  std::vector<LayerW> layers_base;  // as created (the debug knobs edit layers)
  int dbg_max_layers = -1, dbg_no_attn = 0, dbg_no_mlp = 0, dbg_mlp_to = -1;
  bool dbg_on = false;              // some knob set: prompts take the pass path
  struct Named {
    std::string name;
    int storage, rows, cols, group;
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
  // persistent kernel (exec mode 3)
  FlowGeom flow{};
  int flow_grid = 0;      // 0: not available on this device
  int flowm_max = 0;      // most tokens of a verify step in the persistent kernel (0: verify uses the phase kernels)
  bool flow3_ok = false;  // k_flow3 is resident on the persistent grid
  int flow3_policy = 1;   // the decode step's kernel: 0 k_flow, 1 k_flow3, 2 by shape (MLLM_FLOW3)
  int verify_fuse = 9;    // verify steps of at most this many tokens run fused (MLLM_VERIFY_FUSE); faster at every M <= 9 measured
  size_t flowm_lds = 0;
  bool flow_default = false;  // mode 3 was chosen by default, not by mllm_set_exec_mode
  bool refuse_coop = false;   // test hook (MLLM_REFUSE_COOPERATIVE): cooperative launches act as refused
  std::vector<std::pair<void *, size_t>> tagged;  // every tagged buffer and flag array (cleared when the epochs restart)
  size_t flow_lds = 0;
  int flow_epoch = 0;     // epochs used so far (flags hold epochs; cleared only when the epochs restart)
  int aq_idx = 0;         // instance of the decode attention item / persistent kernel (tile size 4, 5, 6)
  hipEvent_t ev0 = nullptr, ev1 = nullptr;  // around the kernels of the last call
  std::vector<hipEvent_t> prof_ev;          // mllm_profile_decode
  float last_ms = 0.f;
  int last_tokens = 0;
  // batched prompt processing (mllm_prefill.hip): prompts of at least
  // pf_min tokens (0: never) run their first n - 1 tokens through it
  PfArgs pf{};
  std::vector<PfLayer> pf_layer;
  int pf_min = 0;
  int pf_tc_max = 0;  // tokens the work buffers hold
  hipEvent_t ev_pf = nullptr;
  std::vector<void *> allocs;
  // models the fused step does not take (a matrix other than Q4 group-32, or
  // a shape outside its limits) run the kind-generic step (mllm_generic.hip)
  bool generic = false;
  GArgs g{};
  std::vector<GLayer> g_layers, g_layers_base;
  int *d_ids = nullptr;              // a call's token ids
  GCursor *h_gcur = nullptr;         // pinned: the cursor a call starts from
  hipGraphExec_t g_graph[2] = {};    // one step without / with the lm_head (exec mode 1)
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
  const size_t nbo = (P.NH + PB - 1) / PB, nbd = (P.nchunk + PB - 1) / PB;
  switch (ph) {
  case PH_QKV: return al4(3 * D) + m * ngd * Q6R + (size_t)m * HD * ngd + 2 * nbd * D + 32 + (size_t)m * HD;
  case PH_ATTN:
    if (m == 1) return al4(3 * D) + ngd * Q6R + 3 * HD * ngd + nbd * D + 32 + 2 * HD + 3 * HD + ATT_LDS;
    return ATT_LDS;
  case PH_MLP:
    return al4(3 * D) + m * ngd * Q6R + 4 * UNITS * ngd + (size_t)m * 2 * Q6R + 2 * nbo * D + 32 + 4 * UNITS;
  case PH_FINAL: return al4(3 * D) + nbd * D + 32;
  case PH_LM: return m * ngd * Q6R + (size_t)m * TC * LT + (size_t)m * P.lm_rpt + 34 + P.max_seq;
  default: return 2 * (LT / 64);
  }
}

// The persistent kernel: every phase at m = 1, the lm_head and ARGMAX
// with 1024-thread workgroups.
size_t flow_lds_bytes(const DecParams &P, const FlowGeom &F) {
  const size_t ngd = P.D / 32;
  size_t f = 2 * (FLT / 64);
  for (int ph = PH_QKV; ph <= PH_FINAL; ++ph) f = std::max(f, lds_floats(P, ph, 1));
  const size_t nbd = (P.nchunk + PB - 1) / PB;
  f = std::max(f, al4(3 * (size_t)P.D) + al4(ngd * Q6R) + (size_t)FTC * FLT + al4((size_t)F.lm_rpt) +
                      al4(34 + (size_t)P.max_seq) + nbd * P.D + 32);
  return f * sizeof(float);
}

// The verify kernel for m tokens: the largest of its items' LDS (k_flowm),
// with the norm scratch the fused step's QKV, MLP and lm_head items add.
size_t flowm_lds_bytes(const DecParams &P, const FlowGeom &F, int m) {
  const size_t ngd = P.D / 32, D = P.D, mm = m, mq = std::min(m, VQT);
  const size_t nbd = (std::max(P.nchunk, P.NH) + PB - 1) / PB;
  const size_t rec = al4(mm * ngd * Q6R), ns = norm_scratch(D, nbd);
  size_t f = 2 * (FLT / 64);
  f = std::max(f, al4(ngd * Q6R) + ns);                                                 // norm items
  f = std::max(f, al4(mq * ngd * Q6R) + mq * (HD * ngd + HD) + al4(mq * 2 * HD) + ns);  // QKV items
  f = std::max(f, mm * (3 * HD + AW * HD + 2 * AW + 2 * Q6R) + al4(mm));               // attention items
  f = std::max(f, rec + VMB * (2 * UNITS * ngd + 2 * UNITS) + al4(mm * 2 * Q6R) + ns);  // MLP items
  f = std::max(f, rec + (size_t)VLB * FTC * FLT + al4((size_t)VLB * F.lm_rpt) + ns);    // lm_head share
  return f * sizeof(float);
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
  if (t->storage != MLLM_Q4 || t->group != 32)
    return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s: storage %d group %d unsupported by the fused step (q4 group 32 only)",
                     n.c_str(), t->storage, t->group);
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
  // kernel-per-phase passes tag their handoff values below every tag a later
  // persistent launch waits for (its epochs start at flow_epoch + 1)
  M->h_st->tag0 = (int)((uint32_t)M->flow_epoch * (uint32_t)TAGL);
  MLLM_HIP(hipMemcpyAsync(M->d_st, M->h_st, sizeof(PassState), hipMemcpyHostToDevice, M->stream));
  return 0;
}

// The kernel of phase ph in a pass of m tokens: the decode step (m = 1) runs
// the attention item with the QKV rows fused in.
PhaseKernel phase_kernel(const mllm_model *M, int ph, int m) {
  if (m == 1 && ph == PH_ATTN) return kAttn1Kernels[M->aq_idx];
  return kPhaseKernels[m == 1][ph];
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
    MLLM_HIP(hipExtLaunchKernel(reinterpret_cast<const void *>(phase_kernel(M, ph, m)), dim3(n),
                                dim3(phase_threads(ph)), args,
                                lds_for(M->P, m), M->stream, e0, e1, 0));
    return 0;
  }
  hipLaunchKernelGGL(phase_kernel(M, ph, m), dim3(n), dim3(phase_threads(ph)), lds_for(M->P, m), M->stream, M->P,
                     Lw, li, m);
  MLLM_HIP(hipGetLastError());
  return 0;
}

// One cooperative launch of the persistent kernel: `steps` single-token
// steps (chained when the pass state says so).  Returns kFlowFellBack when
// the runtime refuses the cooperative launch (e.g. another process holds
// the device's cooperative-launch resources) and mode 3 was only the
// default: the model then switches to mode 1 for good and the caller
// enqueues the phase kernels instead (same results, bit for bit).
constexpr int kFlowFellBack = -1;
int launch_flowm(mllm_model *M, int m, int pos0);

// A cooperative launch of a persistent kernel (decode chain or verify step).
// With refuse_coop set (MLLM_REFUSE_COOPERATIVE=1 at create, a test hook)
// the runtime's refusal is simulated without launching anything.  A refusal
// while mode 3 is only the default switches the model to mode 1 for good and
// returns kFlowFellBack: the caller enqueues the phase kernels instead (same
// results, bit for bit).  An explicit mllm_set_exec_mode(3) reports it.
int launch_coop(mllm_model *M, const void *kern, void **args, size_t lds, const char *what) {
  const hipError_t e = M->refuse_coop ? hipErrorCooperativeLaunchTooLarge
                                      : hipLaunchCooperativeKernel(kern, dim3(M->flow_grid), dim3(FLT), args, lds,
                                                                   M->stream);
  if (e == hipSuccess) return 0;
  if (M->flow_default && (e == hipErrorIllegalState || e == hipErrorNotSupported ||
                          e == hipErrorCooperativeLaunchTooLarge)) {
    (void)hipGetLastError();
    M->exec_mode = 1;
    M->flow_grid = 0;
    return kFlowFellBack;
  }
  return hip_fail(e, what, __FILE__, __LINE__);
}
// The decode step's kernel: k_flow3 (three stages per layer) whenever it is
// resident on the persistent grid, k_flow otherwise (or with MLLM_FLOW3=0).
// Measured chains, us per token, k_flow vs k_flow3: 135M after a 32-token
// prompt 413.2 vs 413.5, after 512 tokens 522.0 vs 486.6; 360M after 32
// tokens 733.3 vs 594.0, after 1536 tokens 1005.7 vs 809.3; GPT-2 124M after
// 16 tokens 258.1 vs 245.7.  With MLLM_FLOW3=2 the choice goes by shape:
// k_flow3 for d_model >= 960 or past the first attention split.
// Tags are epoch * TAGL + layer in 32 bits, so epochs must stay below
// 2^32 / TAGL.  Before a launch would pass that, the stream is drained, every
// tagged buffer and flag is cleared (tag 0: below every tag a launch waits
// for, since launches start at epoch 1) and the epochs start again from 0.
// This runs on the host between launches, never inside a graph.
constexpr int64_t kEpochEnd = int64_t(1) << 25;  // 2^32 / TAGL
int flow_epoch_room(mllm_model *M, int steps) {
  if ((int64_t)M->flow_epoch + steps < kEpochEnd) return 0;
  MLLM_HIP(hipStreamSynchronize(M->stream));
  for (const auto &b : M->tagged) MLLM_HIP(hipMemset(b.first, 0, b.second));
  MLLM_HIP(hipDeviceSynchronize());
  M->flow_epoch = 0;
  return 0;
}

bool use_flow3(const mllm_model *M, int pos) {
  if (!M->flow3_ok || M->flow3_policy == 0) return false;
  return M->flow3_policy == 1 || M->P.D >= 960 || pos >= ACH;
}

int launch_flow(mllm_model *M, int steps) {
  if (int rc = flow_epoch_room(M, steps)) return rc;
  FlowGeom F = M->flow;
  F.ep0 = M->flow_epoch + 1;
  F.steps = steps;
  F.m = 1;
  void *args[] = {&M->P, &F};
  // k_flow3<false> while every position of the chain lies in the first
  // attention split (no split merges), k_flow3<true> past it
  const FlowKernel kern = !use_flow3(M, M->h_st->pos0)               ? kFlowKernels[M->aq_idx]
                          : M->h_st->pos0 + steps - 1 < ACH ? k_flow3<false>
                                                                      : k_flow3<true>;
  if (M->exec_mode == 4) {
    // the same kernel and grid through an ordinary launch (profilers that do
    // not follow cooperative launches): every workgroup is resident only if
    // the device runs nothing else meanwhile; a wait that times out is
    // reported as an error, as in mode 3
    hipLaunchKernelGGL(kern, dim3(M->flow_grid), dim3(FLT), M->flow_lds, M->stream, M->P, F);
    MLLM_HIP(hipGetLastError());
    M->flow_epoch += steps;
    return 0;
  }
  const int rc = launch_coop(M, reinterpret_cast<const void *>(kern), args, M->flow_lds,
                             "hipLaunchCooperativeKernel(k_flow)");
  if (rc == 0) M->flow_epoch += steps;
  return rc;
}

// One verify step of m tokens at positions pos0 .. pos0+m-1 in the
// persistent kernel (k_flowm), launched as mode 3 (cooperative) or mode 4
// launches k_flow.  Only the attention splits that the pass reaches get
// items, and the stages' token groups are as small as the grid allows (every
// item of a layer on its own workgroup).
int launch_flowm(mllm_model *M, int m, int pos0) {
  if (int rc = flow_epoch_room(M, 1)) return rc;
  FlowGeom F = M->flow;
  F.ep0 = M->flow_epoch + 1;
  F.steps = 1;
  F.m = m;
  F.na = M->P.NH * ((pos0 + m - 1) / ACH + 1);
  const int nrh = M->P.NH + 2 * M->P.NKV;
  // up to verify_fuse tokens: three stages per layer, one token per item,
  // every item forming its token's norm; past that, five stages with norm
  // items and token groups as small as the grid allows
  F.fuse = m <= M->verify_fuse;
  for (int tpi = 1; tpi <= m; ++tpi) {
    F.ta = F.mt = tpi;
    F.tq = std::min(tpi, VQT);
    const auto groups = [m](int per) { return (m + per - 1) / per; };
    const int ni = 2 * m + nrh * groups(F.tq) + F.na * groups(F.ta) + F.nm * groups(F.mt);
    if (F.fuse || ni <= M->flow_grid) break;
  }
  if (M->exec_mode == 4) {
    hipLaunchKernelGGL(k_flowm, dim3(M->flow_grid), dim3(FLT), M->flowm_lds, M->stream, M->P, F);
    MLLM_HIP(hipGetLastError());
  } else {
    void *args[] = {&M->P, &F};
    // a refusal falls back like the decode step's: in spec decode the first
    // persistent launch is usually a verify step
    const int rc = launch_coop(M, reinterpret_cast<const void *>(k_flowm), args, M->flowm_lds,
                               "hipLaunchCooperativeKernel(k_flowm)");
    if (rc) return rc;
  }
  M->flow_epoch += 1;
  return 0;
}

// The phases of one pass in order: (phase, layer) pairs.
std::vector<std::pair<int, int>> pass_phases(const mllm_model *M, bool lm, int m) {
  std::vector<std::pair<int, int>> v;
  for (int li = 0; li < M->cfg.n_layers; ++li)
    for (int ph = m == 1 ? PH_ATTN : PH_QKV; ph <= PH_MLP; ++ph) v.emplace_back(ph, li);
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
  for (const auto &pl : pass_phases(M, true, 1)) {
    int ph = pl.first, li = pl.second;
    LayerW Lw = ph <= PH_MLP ? M->layers[li] : LayerW{};
    void *args[] = {&M->P, &Lw, &li, &m};
    hipKernelNodeParams kp;
    memset(&kp, 0, sizeof kp);
    kp.func = reinterpret_cast<void *>(phase_kernel(M, ph, 1));
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
  for (const auto &pl : pass_phases(M, lm, m))
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
  int rc = kFlowFellBack;
  // one row, with or without "every row's" logits, is the decode step
  if (M->exec_mode >= 3 && m == 1 && lm_rows != 0) rc = launch_flow(M, 1);
  else if (M->exec_mode >= 3 && m <= M->flowm_max && lm_rows == 2) rc = launch_flowm(M, m, pos0);
  if (rc == kFlowFellBack) rc = enqueue_pass_phases(M, m, lm_rows != 0);
  if (rc) return rc;
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

// Every layer matrix and the lm_head stored Q4 group-32 (the fused step's
// weights); missing tensors are reported by the path that reads them.
bool all_q4_g32(const mllm_model *M) {
  static const char *const llama[] = {"attn.qkv", "attn.proj", "mlp.w1", "mlp.w3", "mlp.w2"};
  static const char *const gpt2[] = {"attn.qkv", "attn.proj", "mlp.fc", "mlp.proj"};
  auto q4 = [&](const std::string &n) {
    const auto *t = find(M, n);
    return !t || (t->storage == MLLM_Q4 && t->group == 32);
  };
  if (!q4("lm_head")) return false;
  for (int i = 0; i < M->cfg.n_layers; ++i) {
    const std::string b = "blocks." + std::to_string(i) + ".";
    if (M->cfg.arch == 1) {
      for (const char *m : gpt2)
        if (!q4(b + m)) return false;
    } else {
      for (const char *m : llama)
        if (!q4(b + m)) return false;
    }
  }
  return true;
}

// A matrix for the kind-generic step: any storage it reads, rows x cols,
// 16-byte aligned data (chunks of 8 columns are read as one vector).
int get_gmat(mllm_model *M, const std::string &n, int rows, int cols, GMat *out) {
  const auto *t = find(M, n);
  if (!t) return set_error(MLLM_ERR_INVALID, "missing tensor %s", n.c_str());
  if (!g_kind_supported(t->storage, t->group))
    return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s: storage %d (group %d) unsupported", n.c_str(), t->storage,
                     t->group);
  if (t->rows != rows || t->cols != cols)
    return set_error(MLLM_ERR_INVALID, "tensor %s has shape [%d,%d], expected [%d,%d]", n.c_str(), t->rows, t->cols,
                     rows, cols);
  if (cols % 8 || ((t->storage == MLLM_Q4 || t->storage == MLLM_Q8G32) && cols % t->group))
    return set_error(MLLM_ERR_UNSUPPORTED, "tensor %s: %d columns do not divide into its groups", n.c_str(), cols);
  if (((uintptr_t)t->data & 15) != 0) return set_error(MLLM_ERR_INVALID, "tensor %s is not 16-byte aligned", n.c_str());
  *out = GMat{t->data, t->scale, t->storage, rows, cols, t->storage == MLLM_Q8G32 ? 32 : t->group};
  return 0;
}

// The kind-generic model: its matrices as stored, the f32 vectors, the
// RoPE tables, the KV cache and one token's work rows.
int generic_create(mllm_model *M) {
  const mllm_config &c = M->cfg;
  const int D = c.d_model, FF = c.d_ff, NH = c.n_heads, NKV = c.n_kv_heads, V = c.vocab_size, L = c.n_layers;
  const int kvd = NKV * HD;
  // the staged input row (k_g_gemv), the attention weights (k_g_attn) and
  // the history lists (k_g_argmax) live in LDS
  if (std::max(D, FF) > 15000)
    return set_error(MLLM_ERR_UNSUPPORTED, "rows of %d columns exceed the staged row", std::max(D, FF));
  if ((size_t)(HD + c.max_seq_len + 4 + 256 + 4) * sizeof(float) > 64 * 1024)
    return set_error(MLLM_ERR_UNSUPPORTED, "max_seq_len %d exceeds the attention workgroup's LDS", c.max_seq_len);
  GArgs &A = M->g;
  A.arch = c.arch;
  A.L = L;
  A.D = D;
  A.NH = NH;
  A.NKV = NKV;
  A.FF = FF;
  A.V = V;
  A.max_seq = c.max_seq_len;
  A.kv_fp16 = c.kv_fp16 ? 1 : 0;
  A.eps = c.norm_eps > 0 ? c.norm_eps : 1e-6f;
  A.attn_scale = (float)(1.0 / sqrt((double)HD));
  M->g_layers.assign(L, GLayer{});
  for (int i = 0; i < L; ++i) {
    GLayer &w = M->g_layers[i];
    const std::string b = "blocks." + std::to_string(i) + ".";
    int rc = get_gmat(M, b + "attn.qkv", D + 2 * kvd, D, &w.qkv);
    if (!rc) rc = get_gmat(M, b + "attn.proj", D, D, &w.proj);
    if (c.arch == 1) {
      if (!rc) rc = get_gmat(M, b + "mlp.fc", FF, D, &w.w1);
      if (!rc) rc = get_gmat(M, b + "mlp.proj", D, FF, &w.w2);
      if (!rc) rc = get_f32(M, b + "ln1", 2 * D, &w.n1);
      if (!rc) rc = get_f32(M, b + "ln2", 2 * D, &w.n2);
      if (!rc) rc = get_f32(M, b + "attn.qkv_bias", D + 2 * kvd, &w.qkv_b);
      if (!rc) rc = get_f32(M, b + "attn.proj_bias", D, &w.proj_b);
      if (!rc) rc = get_f32(M, b + "mlp.fc_bias", FF, &w.fc_b);
      if (!rc) rc = get_f32(M, b + "mlp.proj_bias", D, &w.mproj_b);
    } else {
      if (!rc) rc = get_gmat(M, b + "mlp.w1", FF, D, &w.w1);
      if (!rc) rc = get_gmat(M, b + "mlp.w3", FF, D, &w.w3);
      if (!rc) rc = get_gmat(M, b + "mlp.w2", D, FF, &w.w2);
      if (!rc) rc = get_f32(M, b + "norm1", D, &w.n1);
      if (!rc) rc = get_f32(M, b + "norm2", D, &w.n2);
    }
    if (rc) return rc;
  }
  M->g_layers_base = M->g_layers;
  A.layers = M->g_layers.data();
  if (int rc = get_gmat(M, "lm_head", V, D, &A.lm)) return rc;
  if (c.arch == 1) {
    int rc = get_f32(M, "ln_f", 2 * D, &A.norm_f);
    if (!rc) rc = get_f32(M, "wpe", (size_t)c.max_seq_len * D, &A.wpe);
    if (!rc) rc = get_f32(M, "scale_factors", D, &A.sf, false);
    if (rc) return rc;
  } else {
    if (int rc = get_f32(M, "norm_f", D, &A.norm_f)) return rc;
    int rd = 0;
    std::vector<float> cs = build_rope_table(c, HD, false, &rd), sn = build_rope_table(c, HD, true, &rd);
    if (int rc = dev_alloc(M, (void **)&M->d_rope_cos, cs.size() * 4)) return rc;
    if (int rc = dev_alloc(M, (void **)&M->d_rope_sin, sn.size() * 4)) return rc;
    MLLM_HIP(hipMemcpy(M->d_rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    MLLM_HIP(hipMemcpy(M->d_rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    A.rope_cos = M->d_rope_cos;
    A.rope_sin = M->d_rope_sin;
    A.rope_dim = rd;
  }
  const size_t kv_bytes = (size_t)L * 2 * NKV * c.max_seq_len * HD * (c.kv_fp16 ? 2 : 4);
  int rc = dev_alloc(M, &A.kv, kv_bytes);
  if (!rc) rc = dev_alloc(M, (void **)&A.x, sizeof(float) * D);
  if (!rc) rc = dev_alloc(M, (void **)&A.qkv, sizeof(float) * (D + 2 * kvd));
  if (!rc) rc = dev_alloc(M, (void **)&A.att, sizeof(float) * D);
  if (!rc) rc = dev_alloc(M, (void **)&A.h, sizeof(float) * FF);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_logits, sizeof(float) * MAXT * (size_t)V);
  if (!rc) rc = dev_alloc(M, (void **)&A.res, sizeof(int) * MAXT);
  if (!rc) rc = dev_alloc(M, (void **)&A.cur, sizeof(GCursor));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_ids, sizeof(int) * ((size_t)c.max_seq_len + 1));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_hist, sizeof(int) * ((size_t)c.max_seq_len + 1));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_x, sizeof(float) * std::max(FF, D) * 4);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_y, sizeof(float) * std::max((size_t)V, (size_t)std::max(FF, D + 2 * kvd)));
  if (rc) return rc;
  MLLM_HIP(hipMemset(A.kv, 0, kv_bytes));
  MLLM_HIP(hipMemset(A.cur, 0, sizeof(GCursor)));
  MLLM_HIP(hipHostMalloc((void **)&M->h_gcur, sizeof(GCursor), hipHostMallocDefault));
  A.logits = M->d_logits;
  A.ids = M->d_ids;
  A.hist = M->d_hist;
  M->generic = true;
  M->max_pass = MAXT;
  M->exec_mode = 1;
  return 0;
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
  // coherent loads and stores address the KV cache with 32-bit byte offsets
  MLLM_CHECK((uint64_t)c.n_layers * 2 * c.n_kv_heads * c.max_seq_len * HD * (c.kv_fp16 ? 2 : 4) < (1ull << 31),
             "KV cache of %d layers x %d positions exceeds 2 GiB", c.n_layers, c.max_seq_len);
  if (c.d_model / c.n_heads != HD)
    return set_error(MLLM_ERR_UNSUPPORTED, "head_dim %d unsupported (64 only)", c.d_model / c.n_heads);
  if (c.arch == 1 && c.n_kv_heads != c.n_heads) return set_error(MLLM_ERR_INVALID, "gpt2 needs n_kv_heads == n_heads");
  // the fused step's shape limits; other shapes take the kind-generic step
  const bool fused_shape = c.n_layers < TAGL && c.d_model % 32 == 0 && c.d_model <= 1024 && c.d_ff % UNITS == 0 &&
                           c.d_ff <= UNITS * PB * NBMAX && c.n_heads <= PB * NBMAX &&
                           (c.arch == 1 || (int)floor(HD * c.rope_pct) == HD);

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
  if (hipEventCreate(&M->ev0) != hipSuccess || hipEventCreate(&M->ev1) != hipSuccess ||
      hipEventCreate(&M->ev_pf) != hipSuccess)
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
    M->tensors.push_back({t.name, t.storage, t.rows, t.cols, t.group > 0 ? t.group : 32, M->d_payload + t.offset,
                          scaled ? reinterpret_cast<const float *>(M->d_payload + t.scale_offset) : nullptr});
  }

  if (!fused_shape || !all_q4_g32(M)) {
    if (int rc = generic_create(M)) return fail(rc);
    *out = M;
    clear_error();
    return 0;
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
  M->layers_base = M->layers;

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
  M->aq_idx = aqc_for(ngd) - 4;
  if (aqc_for(ngd) > 6 || HD * ngd > QC * QT || UNITS * ngd > MC * ((MT / ngd) * ngd) || D > RPW * (MT / 64) * MC ||
      D > RPW * (AT / 64) * SC ||
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
  const size_t tagged_bytes[4] = {sizeof(uint2) * MAXT * D, sizeof(uint2) * MAXT * D, sizeof(uint2) * MAXT * NH * D,
                                   sizeof(uint2) * MAXT * P.nchunk * D};
  int rc = dev_alloc(M, (void **)&P.xa, tagged_bytes[0]);
  if (!rc) rc = dev_alloc(M, (void **)&P.xb, tagged_bytes[1]);
  if (!rc) rc = dev_alloc(M, (void **)&P.opart, tagged_bytes[2]);
  if (!rc) rc = dev_alloc(M, (void **)&P.dpart, tagged_bytes[3]);
  if (!rc) rc = dev_alloc(M, (void **)&P.xn, sizeof(float) * MAXT * D);
  if (!rc) rc = dev_alloc(M, (void **)&P.rec, sizeof(uint2) * 2 * MAXT * ngd * Q6R);
  if (!rc) rc = dev_alloc(M, (void **)&P.qkvr, sizeof(uint2) * L * MAXT * (NH + 2 * NKV) * HD);
  if (!rc) rc = dev_alloc(M, (void **)&P.q, sizeof(float) * MAXT * NH * HD);
  // + a pad word that the persistent kernel's deferred K/V stores write when
  // nothing is pending
  if (!rc) rc = dev_alloc(M, &P.kv, kv_elems * (c.kv_fp16 ? 2 : 4) + 256);
  if (!rc) rc = dev_alloc(M, (void **)&P.attp, sizeof(float) * MAXT * NH * P.nsplit_max * APS);
  if (!rc) rc = dev_alloc(M, (void **)&P.attpt, sizeof(uint2) * MAXT * NH * P.nsplit_max * APT);
  if (!rc) rc = dev_alloc(M, (void **)&P.cnt, sizeof(unsigned) * MAXT * NH);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_logits, sizeof(float) * MAXT * (size_t)V);
  if (!rc) rc = dev_alloc(M, (void **)&P.amv, sizeof(float) * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&P.ami, sizeof(int) * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&P.amt, sizeof(uint2) * 4 * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&P.amtv, sizeof(uint2) * 2 * MAXT * P.lm_tiles);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_hist, sizeof(int) * (c.max_seq_len + 1));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_st, sizeof(PassState));
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_x, sizeof(float) * std::max(FF, D) * 4);
  if (!rc) rc = dev_alloc(M, (void **)&M->d_gemv_y, sizeof(float) * std::max((size_t)V, (size_t)std::max(FF, D + 2 * kvd)));
  if (rc) return fail(rc);
  if (hipHostMalloc((void **)&M->h_st, sizeof(PassState), hipHostMallocDefault) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "pinned state"));
  if (hipMemset(M->d_st, 0, sizeof(PassState)) != hipSuccess ||
      hipMemset(P.xa, 0, tagged_bytes[0]) != hipSuccess || hipMemset(P.xb, 0, tagged_bytes[1]) != hipSuccess ||
      hipMemset(P.opart, 0, tagged_bytes[2]) != hipSuccess || hipMemset(P.dpart, 0, tagged_bytes[3]) != hipSuccess ||
      hipMemset(P.cnt, 0, sizeof(unsigned) * MAXT * NH) != hipSuccess ||
      hipMemset(P.amt, 0, sizeof(uint2) * 4 * P.lm_tiles) != hipSuccess ||
      hipMemset(P.amtv, 0, sizeof(uint2) * 2 * MAXT * P.lm_tiles) != hipSuccess ||
      hipMemset(P.attpt, 0, sizeof(uint2) * MAXT * NH * P.nsplit_max * APT) != hipSuccess ||
      hipMemset(P.rec, 0, sizeof(uint2) * 2 * MAXT * ngd * Q6R) != hipSuccess ||
      hipMemset(P.qkvr, 0, sizeof(uint2) * L * MAXT * (NH + 2 * NKV) * HD) != hipSuccess ||
      hipMemset(P.kv, 0, kv_elems * (c.kv_fp16 ? 2 : 4)) != hipSuccess)
    return fail(set_error(MLLM_ERR_HIP, "memset"));
  P.logits = M->d_logits;
  P.hist = M->d_hist;
  P.st = M->d_st;
  M->tagged = {{P.xa, tagged_bytes[0]},
               {P.xb, tagged_bytes[1]},
               {P.opart, tagged_bytes[2]},
               {P.dpart, tagged_bytes[3]},
               {P.amt, sizeof(uint2) * 4 * P.lm_tiles},
               {P.amtv, sizeof(uint2) * 2 * MAXT * P.lm_tiles},
               {P.attpt, sizeof(uint2) * MAXT * NH * P.nsplit_max * APT},
               {P.rec, sizeof(uint2) * 2 * MAXT * ngd * Q6R},
               {P.qkvr, sizeof(uint2) * L * MAXT * (NH + 2 * NKV) * HD}};

  // batched prompt processing: the weights as PGW1 matrices, work buffers
  // for up to 2048 tokens per chunk
  {
    PfArgs &A = M->pf;
    auto mat = [](const Q4Mat &w) { return PfMat{reinterpret_cast<const uint8_t *>(w.q), w.s, w.rows, w.cols}; };
    A.arch = c.arch;
    A.L = L;
    A.D = D;
    A.NH = NH;
    A.NKV = NKV;
    A.FF = FF;
    A.max_seq = c.max_seq_len;
    A.kv_fp16 = P.kv_fp16;
    A.eps = P.eps;
    A.attn_scale = P.attn_scale;
    A.emb = mat(P.lm);
    A.wpe = P.wpe;
    A.sf = P.sf;
    A.rope_cos = P.rope_cos;
    A.rope_sin = P.rope_sin;
    A.kv = P.kv;
    A.norm_f = P.norm_f;
    A.logits = M->d_logits;
    A.res = &M->d_st->res[0];
    M->pf_layer.resize(L);
    for (int i = 0; i < L; ++i) {
      const LayerW &w = M->layers[i];
      PfLayer &f = M->pf_layer[i];
      f.qkv = mat(w.qkv);
      f.proj = mat(w.proj);
      f.w1 = mat(w.w1);
      f.w3 = mat(w.w3);
      f.w2 = mat(w.w2);
      f.n1 = w.n1;
      f.n2 = w.n2;
      f.qkv_b = w.qkv_b;
      f.proj_b = w.proj_b;
      f.fc_b = w.fc_b;
      f.mproj_b = w.mproj_b;
    }
    A.layers = M->pf_layer.data();
    if (pf_supported(A)) {
      const int tc = std::min(c.max_seq_len, 2048);
      void *buf = nullptr;
      if (int rc = dev_alloc(M, &buf, pf_buffer_bytes(A, tc))) return fail(rc);
      pf_carve(A, buf, tc);
      // the lm_head argmax's counter starts at zero (each launch leaves it so)
      if (hipMemset(A.amx, 0, gemv_q4_argmax_scratch(A.emb.rows, A.emb.cols)) != hipSuccess)
        return fail(set_error(MLLM_ERR_HIP, "memset"));
      // the layer matrices as tiled copies (about the payload's size again)
      size_t tiled = 0;
      for (PfLayer &f : M->pf_layer)
        for (PfMat *w : {&f.qkv, &f.proj, &f.w1, &f.w3, &f.w2})
          if (w->q) tiled += pf_tiled_bytes(*w);
      uint8_t *tb = nullptr;
      if (int rc = dev_alloc(M, (void **)&tb, tiled)) return fail(rc);
      for (PfLayer &f : M->pf_layer)
        for (PfMat *w : {&f.qkv, &f.proj, &f.w1, &f.w3, &f.w2})
          if (w->q) {
            const size_t b = pf_tiled_bytes(*w);
            if (int rc = pf_tile(*w, tb, w, M->stream)) return fail(rc);
            tb += b;
          }
      if (hipStreamSynchronize(M->stream) != hipSuccess) return fail(set_error(MLLM_ERR_HIP, "weight tiling"));
      M->pf_tc_max = tc;
      M->pf_min = 2;  // faster than the passes from 2 tokens on (one token: the decode step)
    }
  }

  // persistent kernel: geometry, LDS, one resident workgroup set, flags
  {
    FlowGeom &F = M->flow;
    F.na = phase_items(P, PH_ATTN, 1);
    F.nm = phase_items(P, PH_MLP, 1);
    F.ni = F.na + F.nm;
    F.lm_rpt = std::min(V, std::max(1, (FTC * FLT) / ngd));
    F.lm_tiles = (V + F.lm_rpt - 1) / F.lm_rpt;
    // one LDS layout for k_flow and k_flow3 (the verify step's items at one row)
    F.kvp = (int)al4(std::max(flow_lds_bytes(P, F), flowm_lds_bytes(P, F, 1)) / sizeof(float));
    M->flow_lds = ((size_t)F.kvp + 2 * 128 + 24) * sizeof(float);  // + the deferred K/V-row slots and flow_slots
    int per_cu = 0;
    const bool lds_ok = M->flow_lds <= lds_cap &&
                        (M->flow_lds <= 64 * 1024 ||
                         hipFuncSetAttribute(reinterpret_cast<const void *>(kFlowKernels[M->aq_idx]),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)M->flow_lds) == hipSuccess);
    int coop = 0;
    (void)hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, M->device);
    if (lds_ok && coop && F.lm_tiles <= P.lm_tiles &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kFlowKernels[M->aq_idx]), FLT,
                                                     M->flow_lds) == hipSuccess &&
        per_cu > 0) {
      const int G = per_cu * M->num_cus;
      const size_t nflags = (size_t)L * (NH + F.nm) + 2 + G;
      if (int rc = dev_alloc(M, (void **)&F.flags, sizeof(int) * nflags)) return fail(rc);
      if (hipMemset(F.flags, 0, sizeof(int) * nflags) != hipSuccess) return fail(set_error(MLLM_ERR_HIP, "memset"));
      M->tagged.emplace_back(F.flags, sizeof(int) * nflags);
      // test hook: start the epochs near their end (MLLM_FLOW_EPOCH0)
      if (const char *v = getenv("MLLM_FLOW_EPOCH0")) M->flow_epoch = (int)std::min<int64_t>(atoll(v), kEpochEnd - 1);
      M->flow_grid = G;
      M->exec_mode = 3;
      M->flow_default = true;
      // the lm_head tiles dealt evenly over the grid: k tiles per workgroup
      // (the fewest that cover the vocabulary at FTC chunk registers per
      // thread), each of ceil(V / (k G)) rows, so that no workgroup takes a
      // second tile while others are idle; kept only when the tile count
      // still fits the tile-maxima buffers (amt, amtv: P.lm_tiles tiles)
      {
        const int k = (F.lm_tiles + G - 1) / G;
        const int rpt = std::min(F.lm_rpt, (V + k * G - 1) / (k * G)), nt = (V + rpt - 1) / rpt;
        if (nt <= P.lm_tiles) {
          F.lm_rpt = rpt;
          F.lm_tiles = nt;
        }
      }
      // the attention items of a (split, KV head) group on one XCD when the
      // stage's items and groups divide over the eight (MLLM_ATTN_XCD=0: off)
      const char *ax = getenv("MLLM_ATTN_XCD");
      F.xcd = (!ax || atoi(ax) != 0) && G % 8 == 0 && F.na % 8 == 0 && (F.na / (NH / NKV)) % 8 == 0;
      // the three-stage chained kernel, when it is resident on the same grid
      const void *k3 = reinterpret_cast<const void *>(k_flow3<true>);
      const void *k3s = reinterpret_cast<const void *>(k_flow3<false>);
      int pc3 = 0, pc3s = 0;
      // (the merging split of an attention item gathers the other splits'
      // partials into its wave-partial slots: at most AW - 1 splits)
      M->flow3_ok = P.nsplit_max < AW &&
                    (M->flow_lds <= 64 * 1024 ||
                     hipFuncSetAttribute(k3, hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->flow_lds) ==
                         hipSuccess) &&
                    hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc3, k3, FLT, M->flow_lds) == hipSuccess &&
                    pc3 >= per_cu &&
                    (M->flow_lds <= 64 * 1024 ||
                     hipFuncSetAttribute(k3s, hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->flow_lds) ==
                         hipSuccess) &&
                    hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc3s, k3s, FLT, M->flow_lds) == hipSuccess &&
                    pc3s >= per_cu;
      if (const char *v = getenv("MLLM_FLOW3")) M->flow3_policy = atoi(v);
      if (const char *v = getenv("MLLM_REFUSE_COOPERATIVE")) M->refuse_coop = atoi(v) != 0;
      // the verify kernel: the most tokens whose LDS still lets the same grid
      // be resident (one workgroup per CU)
      if (const char *v = getenv("MLLM_VERIFY_FUSE")) M->verify_fuse = atoi(v);
      const void *km = reinterpret_cast<const void *>(k_flowm);
      for (int mm = std::min(MAXT, M->max_pass); P.nsplit_max < AW && mm >= 2; --mm) {
        const size_t b = flowm_lds_bytes(P, F, mm);
        int pc = 0;
        if (b <= lds_cap &&
            (b <= 64 * 1024 || hipFuncSetAttribute(km, hipFuncAttributeMaxDynamicSharedMemorySize, (int)b) ==
                                   hipSuccess) &&
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, km, FLT, b) == hipSuccess && pc * M->num_cus >= G) {
          M->flowm_max = mm;
          M->flowm_lds = b;
          break;
        }
      }
    }
    (void)hipGetLastError();
  }
  if (M->lds_max > 64 * 1024) {
    bool ok = true;
    for (int one = 0; one < 2; ++one)
      for (int ph = 0; ph < PH_COUNT; ++ph)
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void *>(kPhaseKernels[one][ph]),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)M->lds_max) == hipSuccess;
    ok = ok && hipFuncSetAttribute(reinterpret_cast<const void *>(kAttn1Kernels[M->aq_idx]),
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
  for (hipGraphExec_t &ge : M->g_graph)
    if (ge) hipGraphExecDestroy(ge);
  if (M->h_gcur) hipHostFree(M->h_gcur);
  for (void *p : M->allocs) hipFree(p);
  if (M->h_st) hipHostFree(M->h_st);
  for (hipEvent_t e : M->prof_ev) (void)hipEventDestroy(e);
  if (M->ev0) hipEventDestroy(M->ev0);
  if (M->ev1) hipEventDestroy(M->ev1);
  if (M->ev_pf) hipEventDestroy(M->ev_pf);
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
  MLLM_CHECK(mode >= 1 && mode <= 4,
             "exec mode %d (1: graph replay, 2: direct launches, 3: persistent kernel, 4: persistent kernel, "
             "ordinary launch)",
             mode);
  if (mode >= 3 && !M->flow_grid) return set_error(MLLM_ERR_UNSUPPORTED, "persistent kernel unavailable on this device");
  M->exec_mode = mode;
  M->flow_default = false;
  return 0;
}

extern "C" int mllm_get_exec_mode(const mllm_model *M) { return M ? M->exec_mode : -1; }

extern "C" const char *mllm_decode_kernel_name(const mllm_model *M) {
  static const char *const names[3] = {"k_flow<4>", "k_flow<5>", "k_flow<6>"};
  if (!M) return "";
  if (M->generic) return "generic kernels";
  if (M->exec_mode < 3) return "phase kernels";
  return use_flow3(M, M->cache_len) ? "k_flow3" : names[M->aq_idx];
}

// The GPU engine's layer-truncation knobs (webgpu-metal.js:1263-1279, set
// from the page's query string at app.js:1317-1325): only the first
// max_layers layers run (< 0: all), no_attn drops every attention block,
// no_mlp every MLP block, mlp_to < 0 keeps the MLP blocks of all layers,
// else those of layers < mlp_to.  A dropped block adds nothing to the
// residual: its output projection writes zero partials and (GPT-2) its bias
// is left out, in every execution mode; so the logits are those of the
// truncated network, as the reference's skipped dispatches give them.  Its
// q/k/v rows still go to the KV cache (the reference leaves the dropped
// layer's cache rows unwritten; no kept block reads them).  While a knob is
// set, prompts run through the decode passes, not the batched path.
extern "C" int mllm_set_debug(mllm_model *M, int max_layers, int no_attn, int no_mlp, int mlp_to) {
  MLLM_CHECK(M, "null model");
  const int L = M->cfg.n_layers;
  MLLM_HIP(hipStreamSynchronize(M->stream));
  bool on = false;
  if (M->generic) {
    // a dropped block's kernels are not launched (its bias goes with it)
    for (int li = 0; li < L; ++li) {
      int d = 0;
      if (max_layers >= 0 && li >= max_layers) d = 3;
      if (no_attn) d |= 1;
      if (no_mlp || (mlp_to >= 0 && li >= mlp_to)) d |= 2;
      M->g_layers[li] = M->g_layers_base[li];
      M->g_layers[li].dbg = d;
      on |= d != 0;
    }
    for (hipGraphExec_t &ge : M->g_graph)  // their launch sequence changed
      if (ge) {
        (void)hipGraphExecDestroy(ge);
        ge = nullptr;
      }
    M->dbg_max_layers = max_layers;
    M->dbg_no_attn = no_attn != 0;
    M->dbg_no_mlp = no_mlp != 0;
    M->dbg_mlp_to = mlp_to;
    M->dbg_on = on;
    return 0;
  }
  for (int li = 0; li < L; ++li) {
    LayerW w = M->layers_base[li];
    int d = 0;
    if (max_layers >= 0 && li >= max_layers) d = 3;
    if (no_attn) d |= 1;
    if (no_mlp || (mlp_to >= 0 && li >= mlp_to)) d |= 2;
    w.dbg = d;
    if (d & 1) w.proj_b = nullptr;  // GPT-2: the attention block's bias goes with it
    on |= d != 0;
    M->layers[li] = w;
  }
  // GPT-2: the MLP block's bias enters the next layer's residual (or the final one)
  for (int li = 1; li < L; ++li) M->layers[li].prev_mproj_b = (M->layers[li - 1].dbg & 2) ? nullptr : M->layers_base[li].prev_mproj_b;
  M->P.last_mproj_b = (M->layers[L - 1].dbg & 2) ? nullptr : M->layers_base[L - 1].mproj_b;
  MLLM_HIP(hipMemcpy(M->d_layers, M->layers.data(), sizeof(LayerW) * L, hipMemcpyHostToDevice));
  if (M->chain_graph) {  // its kernel nodes hold the layers by value
    (void)hipGraphExecDestroy(M->chain_graph);
    M->chain_graph = nullptr;
  }
  M->dbg_max_layers = max_layers;
  M->dbg_no_attn = no_attn != 0;
  M->dbg_no_mlp = no_mlp != 0;
  M->dbg_mlp_to = mlp_to;
  M->dbg_on = on;
  return 0;
}

extern "C" int mllm_flow_verify_tokens(const mllm_model *M) { return M && M->exec_mode >= 3 ? M->flowm_max : 0; }

extern "C" int mllm_set_prefill(mllm_model *M, int min_tokens, int chunk_tokens) {
  MLLM_CHECK(M, "null model");
  MLLM_CHECK(min_tokens >= 0, "prefill threshold %d", min_tokens);
  if (min_tokens > 0 && !M->pf_tc_max) return set_error(MLLM_ERR_UNSUPPORTED, "batched prompts unsupported for this model");
  MLLM_CHECK(chunk_tokens >= 0 && chunk_tokens <= M->pf_tc_max, "prefill chunk %d (at most %d)", chunk_tokens,
             M->pf_tc_max);
  M->pf_min = min_tokens;
  M->pf.tc = chunk_tokens ? chunk_tokens : M->pf_tc_max;
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

// The kind-generic step: a call writes the cursor it starts from, then
// enqueues one step per token -- replayed from a captured graph (exec mode
// 1) or launched directly (mode 2).
static int g_begin(mllm_model *M, const int32_t *ids, int n, int pos0, int chain, int rows, int first, int n_hist,
                   int eos) {
  GCursor &c = *M->h_gcur;
  memset(&c, 0, sizeof c);
  c.pos_next = pos0;
  c.chain = chain;
  c.rows = rows;
  c.tok = first;
  c.n_hist = n_hist;
  c.eos = eos;
  c.gpt2_rule = M->cfg.arch == 1;
  MLLM_HIP(hipMemcpyAsync(M->g.cur, &c, sizeof c, hipMemcpyHostToDevice, M->stream));
  if (ids) MLLM_HIP(hipMemcpyAsync(M->d_ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, M->stream));
  return 0;
}

static int g_enqueue(mllm_model *M, bool lm) {
  if (M->exec_mode == 2) return g_step(M->g, lm, M->stream);
  hipGraphExec_t &ge = M->g_graph[lm ? 1 : 0];
  if (!ge) {
    MLLM_HIP(hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal));
    const int rc = g_step(M->g, lm, M->stream);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(M->stream, &g);
    if (rc || e != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return rc ? rc : hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    }
    const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) {
      ge = nullptr;
      return hip_fail(ei, "hipGraphInstantiate", __FILE__, __LINE__);
    }
  }
  MLLM_HIP(hipGraphLaunch(ge, M->stream));
  return 0;
}

// ids[0..n) at positions pos0..: logits and argmax of every row (rows:
// verify) or of the last token only.
static int g_run(mllm_model *M, const int32_t *ids, int n, int pos0, bool rows, float *logits, int32_t *argmax) {
  if (int rc = g_begin(M, ids, n, pos0, 0, rows ? 1 : 0, 0, 0, -1)) return rc;
  MLLM_HIP(hipEventRecord(M->ev0, M->stream));
  for (int t = 0; t < n; ++t)
    if (int rc = g_enqueue(M, rows || t == n - 1)) return rc;
  MLLM_HIP(hipEventRecord(M->ev1, M->stream));
  MLLM_HIP(hipStreamSynchronize(M->stream));
  MLLM_HIP(hipEventElapsedTime(&M->last_ms, M->ev0, M->ev1));
  M->last_tokens = n;
  const int nr = rows ? n : 1;
  if (logits)
    MLLM_HIP(hipMemcpy(logits, M->d_logits, sizeof(float) * (size_t)nr * M->cfg.vocab_size, hipMemcpyDeviceToHost));
  if (argmax) MLLM_HIP(hipMemcpy(argmax, M->g.res, sizeof(int32_t) * nr, hipMemcpyDeviceToHost));
  return 0;
}

extern "C" int mllm_forward_prompt(mllm_model *M, const int32_t *ids, int n, float *logits, int32_t *argmax) {
  MLLM_CHECK(M && ids, "null argument");
  MLLM_CHECK(n > 0 && n <= M->cfg.max_seq_len, "prompt length %d out of range", n);
  if (int rc = check_ids(M, ids, n)) return rc;
  if (M->generic) {
    if (int rc = g_run(M, ids, n, 0, false, logits, argmax)) return rc;
    M->cache_len = n;
    return 0;
  }
  if (M->pf_min > 0 && n >= M->pf_min && !M->dbg_on) {
    // the prompt in chunks; the last one also forms the logits
    MLLM_HIP(hipEventRecord(M->ev_pf, M->stream));
    for (int p0 = 0; p0 < n; p0 += M->pf.tc) {
      const int m = std::min(M->pf.tc, n - p0);
      if (int rc = pf_layers(M->pf, ids + p0, m, p0, p0 + m == n, M->stream)) return rc;
    }
    MLLM_HIP(hipEventRecord(M->ev1, M->stream));
    MLLM_HIP(hipStreamSynchronize(M->stream));
    MLLM_HIP(hipEventElapsedTime(&M->last_ms, M->ev_pf, M->ev1));
    M->last_tokens = n;
    M->cache_len = n;
    return fetch_outputs(M, 0, 1, logits, argmax);
  }
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
  if (M->generic) {
    if (int rc = g_run(M, &id, 1, M->cache_len, false, logits, argmax)) return rc;
    M->cache_len += 1;
    return 0;
  }
  if (int rc = run_pass(M, &id, 1, M->cache_len, 1)) return rc;
  M->cache_len += 1;
  return fetch_outputs(M, 0, 1, logits, argmax);
}

extern "C" int mllm_forward_verify(mllm_model *M, const int32_t *ids, int n, int32_t *argmax, float *logits) {
  MLLM_CHECK(M && ids, "null argument");
  MLLM_CHECK(n > 0 && n <= M->max_pass, "verify length %d out of range [1, %d]", n, M->max_pass);
  MLLM_CHECK(M->cache_len + n <= M->cfg.max_seq_len, "verify pass exceeds the context");
  if (int rc = check_ids(M, ids, n)) return rc;
  if (M->generic) {
    if (int rc = g_run(M, ids, n, M->cache_len, true, logits, argmax)) return rc;
    M->cache_len += n;
    return 0;
  }
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
  if (M->generic) {
    // each step's argmax lands at d_hist[n_hist + i] and is step i + 1's
    // input; the steps after an EOS return at once
    if (int rc = g_begin(M, nullptr, 0, M->cache_len, 1, 0, first, n_hist, eos_id)) return rc;
    MLLM_HIP(hipEventRecord(M->ev0, M->stream));
    for (int i = 0; i < n_steps; ++i)
      if (int rc = g_enqueue(M, true)) return rc;
    MLLM_HIP(hipEventRecord(M->ev1, M->stream));
    MLLM_HIP(hipStreamSynchronize(M->stream));
    MLLM_HIP(hipEventElapsedTime(&M->last_ms, M->ev0, M->ev1));
    GCursor c;
    MLLM_HIP(hipMemcpy(&c, M->g.cur, sizeof c, hipMemcpyDeviceToHost));
    MLLM_CHECK(c.emitted >= 1 && c.emitted <= n_steps, "chain emitted %d ids of %d steps", c.emitted, n_steps);
    MLLM_HIP(hipMemcpy(out_ids, M->d_hist + n_hist, sizeof(int32_t) * c.emitted, hipMemcpyDeviceToHost));
    *n_out = c.emitted;
    M->last_tokens = c.emitted;
    M->cache_len += c.emitted;
    return 0;
  }
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
  int rc = M->exec_mode >= 3 ? launch_flow(M, n_steps) : kFlowFellBack;
  if (rc == kFlowFellBack) {
    rc = 0;
    if (M->exec_mode == 2) {
      for (int i = 0; i < n_steps && !rc; ++i) rc = enqueue_pass_phases(M, 1, true);
    } else {
      if (!M->chain_graph) rc = build_chain_graph(M);
      for (int i = 0; i < n_steps && !rc; ++i) MLLM_HIP(hipGraphLaunch(M->chain_graph, M->stream));
    }
  }
  if (rc) return rc;
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
  if (M->generic) return set_error(MLLM_ERR_UNSUPPORTED, "phase profile: the fused step's phases only");
  MLLM_CHECK(n_steps > 0, "n_steps %d", n_steps);
  MLLM_CHECK(M->cache_len + n_steps <= M->cfg.max_seq_len, "profile run exceeds the context");
  if (int rc = check_ids(M, &first, 1)) return rc;
  const auto phases = pass_phases(M, true, 1);
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

#ifdef MLLM_STAGE_PROBE
// The stage probe's stamps (a library built with MLLM_STAGE_PROBE only; not
// part of include/mllm.h): 16 x 34 x 256 x 8 u64 values.
extern "C" int mllm_probe_read(void *out) {
  MLLM_CHECK(out, "null argument");
  MLLM_HIP(hipDeviceSynchronize());
  MLLM_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(g_probe), sizeof(g_probe)));
  return 0;
}
extern "C" int mllm_probe_clear(void) {
  MLLM_HIP(hipDeviceSynchronize());
  static unsigned long long zero[16 * PSLOTS * PNI * PK];
  MLLM_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_probe), zero, sizeof(g_probe)));
  return 0;
}
#endif

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
    rc = t->group == 32 ? mllm_gemv_q4(t->rows, t->cols, (const uint8_t *)t->data, t->scale, 32, M->d_gemv_x,
                                       M->d_gemv_y, M->stream)
                        : g_gemv(GMat{t->data, t->scale, t->storage, t->rows, t->cols, t->group}, M->d_gemv_x,
                                 M->d_gemv_y, M->stream);
    break;
  case MLLM_F16:
  case MLLM_BF16:
    rc = g_gemv(GMat{t->data, nullptr, t->storage, t->rows, t->cols, 0}, M->d_gemv_x, M->d_gemv_y, M->stream);
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
