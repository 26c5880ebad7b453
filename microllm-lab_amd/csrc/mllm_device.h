// mllm_device.h -- device building blocks shared by the operator kernels and
// the decode engine (gfx950, wave64).
//
// Q4 group-32 weights at batch 1 are read as 16-byte "chunks" (the 32
// nibbles of one group of one row; scale[c] belongs to chunk c), so every
// 128-bit load of a wavefront covers 1 KiB of contiguous memory.  The
// activations are quantised per group to 24-bit integers (Q6 records, below)
// and dotted with the nibbles by the 4-bit dot instruction (no MFMA), in the
// decode engine and in the standalone GEMV alike.  Per-chunk partials are summed per row in a fixed order that does not
// depend on how rows or tokens are split across workgroups, so a row's value
// is the same in every launch shape (the verify pass relies on it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mllm {

constexpr int WG = 256;          // threads per workgroup

// The thread index as a value the compiler cannot move.  Inside the
// persistent decode kernel's loops it would otherwise hoist every
// thread-dependent address and lane mask of every phase out of the loops and
// keep them all live at once, past the register budget of a 1024-thread
// workgroup; recomputing them where they are used costs a few VALU ops.
__device__ __forceinline__ int tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ int lane_id64() { return tid() & 63; }

struct Q4Mat {
  const uint4 *q;  // packed nibbles, as 16-byte chunks
  const float *s;  // one scale per chunk
  int rows, cols;  // cols % 32 == 0
};

// ---------------------------------------------------------------- coherent access
// Values one workgroup hands to another (activations, partial sums, the KV
// cache, the pass state) are stored and loaded with device-scope (sc1) buffer
// instructions.  Each XCD of the chip has its own L2; an sc1 store writes
// through it and an sc1 load does not return a line that another XCD may
// have changed, so a handoff inside one launch needs no L2 write-back or
// invalidate (which a release/acquire fence at agent scope would issue).
// The buffer resource covers [base, base + 2 GiB); base must be uniform in
// the wave (kernel arguments and values derived from them), the per-lane
// part goes in the 32-bit byte offset.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
constexpr int CP_SC1 = 16;  // cache-policy operand: device scope

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float4 coh_ld4(const void *base, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), (int)off, 0, CP_SC1);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ uint4 coh_ld16(const void *base, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), (int)off, 0, CP_SC1);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 coh_ld8(const void *base, uint32_t off) {
  const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(coh_rsrc(base), (int)off, 0, CP_SC1);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float coh_ldf(const void *base, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(coh_rsrc(base), (int)off, 0, CP_SC1));
}
__device__ __forceinline__ int coh_ldi(const void *base, uint32_t off) {
  return (int)__builtin_amdgcn_raw_buffer_load_b32(coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_st4(void *base, uint32_t off, float4 v) {
  const u32x4_t u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
  __builtin_amdgcn_raw_buffer_store_b128(u, coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_stf(void *base, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_sti(void *base, uint32_t off, int v) {
  __builtin_amdgcn_raw_buffer_store_b32((unsigned)v, coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_sth(void *base, uint32_t off, unsigned short v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_st8(void *base, uint32_t off, uint2 v) {
  const u32x2_t u = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(u, coh_rsrc(base), (int)off, 0, CP_SC1);
}
__device__ __forceinline__ void coh_st16(void *base, uint32_t off, uint4 v) {
  const u32x4_t u = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(u, coh_rsrc(base), (int)off, 0, CP_SC1);
}
// Wait until this thread's stores (and loads) have completed: a workgroup
// barrier alone does not wait for them.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0) */ }

// Tagged values.  A value handed from one workgroup to another inside the
// persistent kernel travels with the tag of the (step, layer) that wrote it,
// as one naturally aligned 8-byte pair (x, y) = (v, v ^ tag) of float bits v,
// stored by one 8-byte device-scope (sc1) store.  Readers load pairs with
// sc1 loads of 8 or 16 bytes (two neighbouring pairs) and accept a pair only
// when x ^ y equals the tag they wait for exactly; the value is then x.
// The argument needs nothing wider than single-copy atomic dwords:
//  - a location is rewritten only after every reader of its previous version
//    is done (each buffer's writers depend, through the data edges, on all of
//    its readers), so a polling reader sees one of two versions of a pair:
//    the old (v0, v0 ^ t0) with t0 != want, or the new (v1, v1 ^ want);
//  - a read that returns both dwords of one version passes the check exactly
//    when that version is the new one;
//  - a read that mixes the versions' dwords passes only with a value that is
//    the new one's: (v1, v0 ^ t0) passes iff v1 ^ v0 ^ t0 == want, and then
//    x = v1; (v0, v1 ^ want) passes iff v0 == v1, and then x = v0 = v1.
// So a reader that sees the tag it waits for holds the value stored with it,
// whether or not the hardware moves a lane's 8 or 16 bytes in one piece, and
// polling the data replaces a completion wait plus a flag.  Every writer of
// these buffers (decode, verify and phase kernels) uses the encoding, so no
// stale pair can pass either.  Tags grow across launches (32-bit, wrapping
// after 2^25 steps); buffers start zeroed (tag 0, below every tag waited for).
__device__ __forceinline__ uint32_t pair_tag(uint2 p) { return p.x ^ p.y; }
__device__ __forceinline__ bool pair_ok(uint2 p, int want) { return (p.x ^ p.y) == (uint32_t)want; }
// Flags (single dwords) are compared modulo 2^32: at least e.
__device__ __forceinline__ bool tag_ok(uint32_t tag, int want) { return (int)(tag - (uint32_t)want) >= 0; }
// Element i of a row of pairs at a wave-uniform base.
__device__ __forceinline__ uint2 tag_ld(const uint2 *base, uint32_t i) { return coh_ld8(base, i * 8u); }
__device__ __forceinline__ uint2 tag_pair(uint32_t bits, int tag) { return make_uint2(bits, bits ^ (uint32_t)tag); }
__device__ __forceinline__ void tag_st(uint2 *base, uint32_t i, float v, int tag) {
  coh_st8(base, i * 8u, tag_pair(__float_as_uint(v), tag));
}
// A compiler barrier for polling loops: the loads after it are issued again
// on every iteration instead of being hoisted out of the loop.
__device__ __forceinline__ void poll_fence() { asm volatile("" ::: "memory"); }

// ---------------------------------------------------------------- integer group dots (Q6 records)
// Every Q4 GEMV of this library takes its activations as 24-bit integers
// per 32-element group (the Q4 group): xi = rint(x * Q6MAX / amax), with the
// group's scale sx = amax / Q6MAX (amax = max |x| of the group; 0 for an
// all-zero group).  Rounding x to 24 bits moves it by at most
// amax / (2 Q6MAX) = 6.4e-8 amax: the size of one float32 rounding of the
// group's largest element, so the products keep float32 accuracy.
//
// Each xi is held as six signed 4-bit digits, xi = sum_k 16^k d_k with
// d_k in [-8, 7].  Flipping bit 3 of a stored nibble q gives the signed
// nibble q - 8, so one v_dot8_i32_i4 per 8 weights and digit plane yields
//   dot = sum_k 16^k sum_e (q_e - 8) d_{k,e} = sum_e (q_e - 8) xi_e,
// exact in int32: |dot| <= 32 * 8 * Q6MAX < 2^31 (the Horner partial sums may
// wrap; the final value does not).  The group adds ((float)dot * sx) * w_scale
// to its row: 4 XOR, 24 dot8, 5 shifts, a convert and 2 multiplies per 32
// weights.
//
// Digits: with u = xi + Q6C (Q6C = 8 (16^6 - 1) / 15, so u >= 0), digit k of
// xi is hex digit k of u minus 8, i.e. its 4-bit pattern is bfe(u, 4k, 4) ^ 8.
//
// A group's record is Q6R dwords: plane k (k = 0 .. 5) is dwords 4k .. 4k+3,
// dword j of a plane holding the digits of elements 8j .. 8j+7 (element 8j+i
// in nibble i, the weights' own nibble order); dword 24 is sx; 25 .. 27 pad
// the record to 16-byte alignment.
constexpr int Q6R = 28;
constexpr int Q6C = 8947848;         // 8 * (16^6 - 1) / 15
constexpr float Q6MAX = 7829360.0f;  // below 7 * (16^6 - 1) / 15 = 7829367 by more than the rcp rounding

__device__ __forceinline__ float q6_inv(float amax) { return amax > 0.f ? Q6MAX * __builtin_amdgcn_rcpf(amax) : 0.f; }
__device__ __forceinline__ uint32_t q6_u(float v, float inv) { return (uint32_t)((int)__builtin_rintf(v * inv) + Q6C); }

// One 16-byte chunk (the 32 weights of one group of one row) against a
// group's digit planes xr[24], activation scale sx and weight scale ws.
__device__ __forceinline__ float q4_dot6(const uint4 w, const uint32_t (&xr)[24], float sx, float ws) {
  const int d[4] = {(int)(w.x ^ 0x88888888u), (int)(w.y ^ 0x88888888u), (int)(w.z ^ 0x88888888u),
                    (int)(w.w ^ 0x88888888u)};
  int acc = 0;
#pragma unroll
  for (int k = 5; k >= 0; --k) {
    if (k < 5) acc = (int)((uint32_t)acc << 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_sdot8(d[j], (int)xr[4 * k + j], acc, false);
  }
  return ((float)acc * sx) * ws;
}

// A group's record held in registers (e.g. a thread's one group of a tile).
struct Q6Rec {
  uint32_t d[24];
  float sx;
};
__device__ __forceinline__ Q6Rec q6_load(const uint32_t *__restrict__ rec) {
  Q6Rec r;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const uint4 v = *reinterpret_cast<const uint4 *>(rec + 4 * k);
    r.d[4 * k] = v.x;
    r.d[4 * k + 1] = v.y;
    r.d[4 * k + 2] = v.z;
    r.d[4 * k + 3] = v.w;
  }
  r.sx = __uint_as_float(rec[24]);
  return r;
}
__device__ __forceinline__ float q4_dot6(const uint4 w, const Q6Rec &r, float ws) { return q4_dot6(w, r.d, r.sx, ws); }

// C chunks of one group against that group's record in LDS, taken digit
// plane by digit plane, so that at most one plane of the record is held in
// registers beside the chunks: out[j] is q4_dot6 of chunk j, bit for bit
// (the same dot instructions in the same order).
template <int C>
__device__ __forceinline__ void q4_dot6_planes(const uint4 (&w)[C], const float (&ws)[C],
                                               const uint32_t *__restrict__ rec, float (&out)[C]) {
  int acc[C];
#pragma unroll
  for (int j = 0; j < C; ++j) acc[j] = 0;
#pragma unroll
  for (int k = 5; k >= 0; --k) {
    const uint4 v = *reinterpret_cast<const uint4 *>(rec + 4 * k);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      if (k < 5) acc[j] = (int)((uint32_t)acc[j] << 4);
      acc[j] = __builtin_amdgcn_sdot8((int)(w[j].x ^ 0x88888888u), (int)v.x, acc[j], false);
      acc[j] = __builtin_amdgcn_sdot8((int)(w[j].y ^ 0x88888888u), (int)v.y, acc[j], false);
      acc[j] = __builtin_amdgcn_sdot8((int)(w[j].z ^ 0x88888888u), (int)v.z, acc[j], false);
      acc[j] = __builtin_amdgcn_sdot8((int)(w[j].w ^ 0x88888888u), (int)v.w, acc[j], false);
    }
  }
  const float sx = __uint_as_float(rec[24]);
#pragma unroll
  for (int j = 0; j < C; ++j) out[j] = ((float)acc[j] * sx) * ws[j];
}

// One chunk against a record in LDS.
__device__ __forceinline__ float q4_dot6(const uint4 w, const uint32_t *__restrict__ rec, float ws) {
  const uint4 wa[1] = {w};
  const float sa[1] = {ws};
  float o[1];
  q4_dot6_planes<1>(wa, sa, rec, o);
  return o[0];
}

// Cross-lane moves through DPP (a VALU operand modifier) instead of
// ds_bpermute, which goes through the LDS crossbar and costs an LDS round
// trip per step.  Control codes (GFX9 DPP16): quad_perm(1,0,3,2) = 0xB1,
// quad_perm(2,3,0,1) = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
// Callers run them with all 64 lanes active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

// The partner of lane ^ 1 (quad_perm), e.g. the two groups of a row pair.
__device__ __forceinline__ float lane_xor1(float v) { return dpp_f<0xB1>(v); }

// Sum over each 16-lane row, left in every lane of the row: pairs (xor 1),
// quads (xor 2), half rows (mirror within 8), rows (mirror within 16).
// Every lane of a row ends with the same bits (each step adds the same two
// values).
__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp_f<0xB1>(v);
  v = v + dpp_f<0x4E>(v);
  v = v + dpp_f<0x141>(v);
  v = v + dpp_f<0x140>(v);
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave-wide sum / max, uniform in the wave: rows reduced with DPP, then the
// four row results read as scalars and combined as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Pairwise tree over N = 2^k values: (tree(lower half) + tree(upper half)).
template <int N>
__device__ __forceinline__ float tree_sum(const float *r) {
  if constexpr (N == 1) return r[0];
  else return tree_sum<N / 2>(r) + tree_sum<N / 2>(r + N / 2);
}
template <int N>
__device__ __forceinline__ float tree_max(const float *r) {
  if constexpr (N == 1) return r[0];
  else return fmaxf(tree_max<N / 2>(r), tree_max<N / 2>(r + N / 2));
}

// Deterministic block-wide sum for NT threads; red needs NT / 64 floats of LDS.
template <int NT = WG>
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int lane = tid() & 63, wv = tid() >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  const float r = tree_sum<NT / 64>(red);
  __syncthreads();
  return r;
}

template <int NT = WG>
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  const int lane = tid() & 63, wv = tid() >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  const float r = tree_max<NT / 64>(red);
  __syncthreads();
  return r;
}

// (value, index) "better" relation of infer.js argmax: larger value, then
// lower index (the first maximum).
__device__ __forceinline__ bool amax_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int CTRL>
__device__ __forceinline__ void amax_step(float &v, int &i) {
  const float ov = dpp_f<CTRL>(v);
  const int oi = dpp_i<CTRL>(i);
  if (amax_better(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

// Wave-wide first maximum (value, index), uniform in the wave.  The relation
// is a total order on (value, index) pairs, so the result does not depend on
// the combining order.
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
  amax_step<0xB1>(v, i);
  amax_step<0x4E>(v, i);
  amax_step<0x141>(v, i);
  amax_step<0x140>(v, i);
  float bv = readlane_f(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float rv = readlane_f(v, r);
    const int ri = __builtin_amdgcn_readlane(i, r);
    if (amax_better(rv, ri, bv, bi)) {
      bv = rv;
      bi = ri;
    }
  }
  v = bv;
  i = bi;
}

// Sum of a row's n group partials in a fixed order: eight interleaved
// accumulators (k mod 8) so the LDS reads overlap, then a fixed tree.
__device__ __forceinline__ float row_sum(const float *p, int n) {
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int k = 0;
  for (; k + 8 <= n; k += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] += p[k + j];
  }
  for (int j = 0; k < n; ++k, ++j) a[j] += p[k];
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// ---------------------------------------------------------------- activation staging (Q6 records)
// Max over the 8 lanes of each half-row (lanes 8k .. 8k+7).
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  return fmaxf(v, dpp_f<0x141>(v));
}
// The sum of a row's ng partials p[0 .. ng) on 4 lanes (s = lane & 3):
// lane s adds partials s, s + 4, ... in order (from +0), then a fixed 4-lane
// tree; the same bits in all 4 lanes.  Called with the whole quad active.
__device__ __forceinline__ float row_sum4(const float *p, int ng, int s) {
  float a = 0.f;
  for (int k = s; k < ng; k += 4) a = a + p[k];
  a = a + dpp_f<0xB1>(a);
  return a + dpp_f<0x4E>(a);
}

// Sum over the 8 lanes of each half-row, the same bits in all 8 lanes.
__device__ __forceinline__ float sum8f(float v) {
  v = v + dpp_f<0xB1>(v);
  v = v + dpp_f<0x4E>(v);
  return v + dpp_f<0x141>(v);
}

// A row staged by one thread per float4 column q (elements 4q .. 4q+3 of
// group q >> 3; a group's columns are 8 neighbouring lanes): the Q6 records
// of the row's groups at rec0.  Called by whole waves (DPP); `in` marks real
// columns (lanes past the row take part in the max with zeros).
__device__ __forceinline__ void q6_stage_col(float4 y, bool in, int q, uint32_t *rec0) {
  if (!in) y = make_float4(0.f, 0.f, 0.f, 0.f);
  const float a = max8(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  const float inv = q6_inv(a);
  const uint32_t u0 = q6_u(y.x, inv), u1 = q6_u(y.y, inv), u2 = q6_u(y.z, inv), u3 = q6_u(y.w, inv);
  if (!in) return;
  uint32_t *rec = rec0 + (q >> 3) * Q6R;
  uint8_t *rb = reinterpret_cast<uint8_t *>(rec);
  // column q holds elements 4(q & 7) .. +3: dword (q & 7) >> 1 of a plane, its
  // low or high 16 bits
  const int off = 4 * ((q & 7) >> 1) + 2 * (q & 1);
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    const uint32_t v = __builtin_amdgcn_ubfe(u0, 4 * k, 4) | (__builtin_amdgcn_ubfe(u1, 4 * k, 4) << 4) |
                       (__builtin_amdgcn_ubfe(u2, 4 * k, 4) << 8) | (__builtin_amdgcn_ubfe(u3, 4 * k, 4) << 12);
    *reinterpret_cast<unsigned short *>(rb + 16 * k + off) = (unsigned short)(v ^ 0x8888u);
  }
  if ((q & 7) == 0) rec[24] = __float_as_uint(a * (1.0f / Q6MAX));
}

// 64 values, one per lane of the calling wave (lane r: element r & 31 of
// group r >> 5): the two Q6 records at rec0.  Called by the whole wave.
__device__ __forceinline__ void q6_stage_lanes(float v, uint32_t *rec0) {
  const int r = lane_id64(), e = r & 31;
  const float m16 = row16_max(fabsf(v));
  const float a = r < 32 ? fmaxf(readlane_f(m16, 0), readlane_f(m16, 16))
                         : fmaxf(readlane_f(m16, 32), readlane_f(m16, 48));
  const uint32_t u = q6_u(v, q6_inv(a));
  const uint32_t uo = (uint32_t)dpp_i<0xB1>((int)u);  // the odd neighbour's (lane ^ 1)
  if ((e & 1) == 0) {
    // elements e, e + 1: byte (e & 7) >> 1 of dword e >> 3 of each plane
    uint8_t *rb = reinterpret_cast<uint8_t *>(rec0 + (r >> 5) * Q6R) + 4 * (e >> 3) + ((e & 7) >> 1);
#pragma unroll
    for (int k = 0; k < 6; ++k)
      rb[16 * k] = (uint8_t)((__builtin_amdgcn_ubfe(u, 4 * k, 4) | (__builtin_amdgcn_ubfe(uo, 4 * k, 4) << 4)) ^ 0x88u);
    if (e == 0) rec0[(r >> 5) * Q6R + 24] = __float_as_uint(a * (1.0f / Q6MAX));
  }
}

// ---------------------------------------------------------------- tiles
// A tile is up to two contiguous row ranges [r0a, r0a+na) and [r0b, r0b+nb)
// of one matrix (two ranges let a QKV tile hold both RoPE partners d and
// d+32 of a head).  Its chunks are loaded into registers first (tile_load),
// so the loads are in flight while the activations are staged, then
// consumed by tile_compute.  C = chunks per thread.
template <int C>
struct TileRegs {
  uint4 w[C];
  float s[C];
};

// Branch-free: chunks past nch load the tile's last chunk (ignored later).
template <int C, int NT = WG>
__device__ __forceinline__ void tile_load(const Q4Mat &W, int r0a, int na, int r0b, int ng, int nch,
                                          TileRegs<C> &R) {
  const int split = na * ng;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = min((int)tid() + j * NT, nch - 1);
    const size_t gc = c < split ? (size_t)r0a * ng + c : (size_t)r0b * ng + (c - split);
    R.w[j] = W.q[gc];
    R.s[j] = W.s[gc];
  }
}

// Rows [r0, r0 + nrows) of W, chunk c = tid + j*stride (stride a multiple of
// ng: all of a thread's chunks are one group, tid % ng).  Threads past the
// stride and chunks past nrows*ng load the tile's last chunk (unused).
template <int C>
__device__ __forceinline__ void tile_load_strided(const Q4Mat &W, int r0, int nrows, int ng, int stride,
                                                  TileRegs<C> &R) {
  const int nch = nrows * ng;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int c = min(min((int)tid(), stride - 1) + j * stride, nch - 1);
    const size_t gc = (size_t)r0 * ng + c;
    R.w[j] = W.q[gc];
    R.s[j] = W.s[gc];
  }
}

// A tile against activations staged as Q6 records (m tokens x ng groups):
// chunk partials to part, then the row sums in row_sum's order to out.
template <int C, int NT = WG>
__device__ __forceinline__ void tile_compute_q6(const TileRegs<C> &R, int nrows, int ng, int nch, int m,
                                                const uint32_t *qx, int gfirst, int gstep, float *part, float *out,
                                                int ostride) {
  int gj[C];
  {
    int g = gfirst;
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
      const int c = tid() + j * NT;
      if (c < nch) part[t * nch + c] = q4_dot6(R.w[j], qx + (t * ng + gj[j]) * Q6R, R.s[j]);
    }
  }
  __syncthreads();
  for (int i = tid(); i < nrows * m; i += NT) {
    const int t = i / nrows, r = i - t * nrows;
    out[t * ostride + r] = row_sum(part + t * nch + r * ng, ng);
  }
  __syncthreads();
}

}  // namespace mllm
