// mllm_device.h -- device building blocks shared by the operator kernels and
// the decode engine (gfx950, wave64).
//
// Q4 group-32 weights at batch 1 are read as 16-byte "chunks" (the 32
// nibbles of one group of one row; scale[c] belongs to chunk c), so every
// 128-bit load of a wavefront covers 1 KiB of contiguous memory.  The
// activations are quantised per group to integers and dotted with the
// nibbles by the byte/nibble dot instructions (no MFMA): the decode engine
// uses 16-bit records (QX, below), the standalone GEMV of mllm_ops.hip 24-bit
// ones.  Per-chunk partials are summed per row in a fixed order that does not
// depend on how rows or tokens are split across workgroups, so a row's value
// is the same in every launch shape (the verify pass relies on it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mllm {

constexpr int WG = 256;          // threads per workgroup
constexpr int XS = 36;           // LDS floats per staged 32-float group
constexpr int SUB_CH = WG * 4;   // chunks per sub-tile of the Q8 GEMV

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

__device__ __forceinline__ float ubyte(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xFFu); }

// 16 signed 8-bit weights against 16 floats: sum((u - 128) * x) with
// u = q ^ 0x80 converted by v_cvt_f32_ubyte; the -128 is folded by the caller.
__device__ __forceinline__ float q8_chunk_dot(const uint4 w, const float *__restrict__ xg) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  const uint32_t dw[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4 xa = *reinterpret_cast<const float4 *>(xg + 4 * j);
    a0 = __builtin_fmaf(ubyte(dw[j], 0), xa.x, a0);
    a1 = __builtin_fmaf(ubyte(dw[j], 1), xa.y, a1);
    a2 = __builtin_fmaf(ubyte(dw[j], 2), xa.z, a2);
    a3 = __builtin_fmaf(ubyte(dw[j], 3), xa.w, a3);
  }
  return (a0 + a1) + (a2 + a3);
}

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
// in the same naturally aligned access: a 64-bit (float bits, tag) pair, or a
// 16-byte quad of three floats and the tag (the residual partials).  Such an
// access reaches memory whole, so a reader that sees the tag it waits for also
// sees that writer's values, and polling the data replaces a completion wait
// plus a flag.  (For the quads this rests on the 16-byte stores and loads
// being observed whole on this device; torn quads were searched for and not
// seen.)  Tags grow across launches and are compared modulo 2^32.
__device__ __forceinline__ bool tag_ok(uint32_t tag, int want) { return (int)(tag - (uint32_t)want) >= 0; }
__device__ __forceinline__ uint2 tagged(float v, int tag) { return make_uint2(__float_as_uint(v), (uint32_t)tag); }
// A compiler barrier for polling loops: the loads after it are issued again
// on every iteration instead of being hoisted out of the loop.
__device__ __forceinline__ void poll_fence() { asm volatile("" ::: "memory"); }

// ---------------------------------------------------------------- integer group dots
// The decode engine's GEMVs take their activations quantised per 32-element
// group (the Q4 group) to int16: xi = rint(x * 32767 / amax), scale
// sx = amax / 32767 (amax = max |x| of the group; 0 for an all-zero group).
// Splitting xi = 256 * hi + lo (hi signed, lo unsigned bytes) turns the
// group's dot with the nibbles into byte dot products that are exact in
// int32:
//   sum_k (q_k - 8) * xi_k = 256 * sdot4(q, hi) + udot4(q, lo) - 8 * sum_k xi_k
// A packed dword of the weights holds elements 8j .. 8j+7 (byte b: element
// 8j+2b in the low nibble, 8j+2b+1 in the high one), so the activations are
// stored per group as a QX record of QXR dwords:
//   [0..3]  high bytes of the even elements 8j, 8j+2, 8j+4, 8j+6 (dword j)
//   [4..7]  high bytes of the odd elements
//   [8..11] low bytes of the even elements, [12..15] of the odd ones
//   [16] sx (float bits), [17] sum of xi, [18..19] padding
// The group's contribution to a row is then ((float)dot * sx) * w_scale:
// about 34 VALU operations per 32 weights instead of 80 for float
// dequantisation.  The only rounding is that of x to 16 bits (relative
// 1.5e-5 per element).
constexpr int QXR = 20;

__device__ __forceinline__ float q4_qx_part(const uint4 w, const uint32_t *__restrict__ rec, float ws) {
  const uint4 he = *reinterpret_cast<const uint4 *>(rec), ho = *reinterpret_cast<const uint4 *>(rec + 4);
  const uint4 le = *reinterpret_cast<const uint4 *>(rec + 8), lo = *reinterpret_cast<const uint4 *>(rec + 12);
  const uint2 sc = *reinterpret_cast<const uint2 *>(rec + 16);
  const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
  const uint32_t xhe[4] = {he.x, he.y, he.z, he.w}, xho[4] = {ho.x, ho.y, ho.z, ho.w};
  const uint32_t xle[4] = {le.x, le.y, le.z, le.w}, xlo[4] = {lo.x, lo.y, lo.z, lo.w};
  int h = 0;
  uint32_t l = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ev = dw[j] & 0x0F0F0F0Fu, od = (dw[j] >> 4) & 0x0F0F0F0Fu;
    h = __builtin_amdgcn_sdot4((int)ev, (int)xhe[j], h, false);
    h = __builtin_amdgcn_sdot4((int)od, (int)xho[j], h, false);
    l = __builtin_amdgcn_udot4(ev, xle[j], l, false);
    l = __builtin_amdgcn_udot4(od, xlo[j], l, false);
  }
  const int dot = h * 256 + (int)l - 8 * (int)sc.y;
  return ((float)dot * __uint_as_float(sc.x)) * ws;
}

// The same with the group's record held in registers (x16: dwords 0..15,
// sx, xs = sum of xi), e.g. for the gate and up rows of one unit.
struct QxRec {
  uint32_t d[16];
  float sx;
  int xs;
};
__device__ __forceinline__ QxRec qx_load(const uint32_t *__restrict__ rec) {
  QxRec r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4 v = *reinterpret_cast<const uint4 *>(rec + 4 * k);
    r.d[4 * k] = v.x;
    r.d[4 * k + 1] = v.y;
    r.d[4 * k + 2] = v.z;
    r.d[4 * k + 3] = v.w;
  }
  const uint2 sc = *reinterpret_cast<const uint2 *>(rec + 16);
  r.sx = __uint_as_float(sc.x);
  r.xs = (int)sc.y;
  return r;
}
__device__ __forceinline__ float q4_qx_part_reg(const uint4 w, const QxRec &r, float ws) {
  const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
  int h = 0;
  uint32_t l = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ev = dw[j] & 0x0F0F0F0Fu, od = (dw[j] >> 4) & 0x0F0F0F0Fu;
    h = __builtin_amdgcn_sdot4((int)ev, (int)r.d[j], h, false);
    h = __builtin_amdgcn_sdot4((int)od, (int)r.d[4 + j], h, false);
    l = __builtin_amdgcn_udot4(ev, r.d[8 + j], l, false);
    l = __builtin_amdgcn_udot4(od, r.d[12 + j], l, false);
  }
  const int dot = h * 256 + (int)l - 8 * r.xs;
  return ((float)dot * r.sx) * ws;
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

// Copy m rows x[t*ldx + i] (i < n, n % 32 == 0, 16-byte aligned rows) into
// the skewed layout.  Loads go out in batches of 4 float4 per thread before
// any LDS store, so a batch costs one memory latency, not one per element.
// stage_rows_load / stage_rows_store split one batch (float4 index base +
// tid + k*NT) so a caller can issue it ahead of other loads; stage_rows
// then copies the batches from `from` on.
// Loads here are branch-free: an out-of-range lane reads a valid element
// (its index clamped) and the value is ignored where it is used.  A load
// inside a divergent branch makes the compiler wait for it at the join,
// which would serialise loads meant to be in flight together.
template <int NT = WG>
__device__ __forceinline__ void stage_rows_load(const float *__restrict__ x, int ldx, int m, int n, int base,
                                                float4 (&v)[4]) {
  const int nq = n >> 2, total = m * nq;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int f = min(base + (int)tid() + k * NT, total - 1);
    const int t = f / nq, q = f - t * nq;
    v[k] = *reinterpret_cast<const float4 *>(x + (size_t)t * ldx + 4 * q);
  }
}

template <int NT = WG>
__device__ __forceinline__ void stage_rows_store(int m, int n, int base, const float4 (&v)[4], float *xs) {
  const int nq = n >> 2, total = m * nq, ng = n >> 5;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int f = base + tid() + k * NT;
    if (f < total) {
      const int t = f / nq, i = 4 * (f - t * nq);
      *reinterpret_cast<float4 *>(xs + (t * ng + (i >> 5)) * XS + (i & 31)) = v[k];
    }
  }
}

template <int NT = WG>
__device__ __forceinline__ void stage_rows(const float *__restrict__ x, int ldx, int m, int n, float *xs,
                                           int from = 0) {
  const int nq = n >> 2, total = m * nq;
  for (int base = from; base < total; base += 4 * NT) {
    float4 v[4];
    stage_rows_load<NT>(x, ldx, m, n, base, v);
    stage_rows_store<NT>(m, n, base, v, xs);
  }
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

// ---------------------------------------------------------------- activation staging (QX)
// Max / sum over the 8 lanes of each half-row (lanes 8k .. 8k+7).
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ int sum8i(int v) {
  v = v + dpp_i<0xB1>(v);
  v = v + dpp_i<0x4E>(v);
  return v + dpp_i<0x141>(v);
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
__device__ __forceinline__ float qx_inv(float amax) { return amax > 0.f ? 32767.0f / amax : 0.f; }
__device__ __forceinline__ int qx_round(float v, float inv) { return (int)__builtin_rintf(v * inv); }

// A row staged by one thread per float4 column q (elements 4q .. 4q+3, the
// group's columns on 8 neighbouring lanes): the QX records of the row's
// groups at qx.  Called by whole waves (DPP); `in` marks real columns.
__device__ __forceinline__ void qx_stage_col(float4 y, bool in, int q, uint32_t *qx) {
  if (!in) y = make_float4(0.f, 0.f, 0.f, 0.f);
  const float a = max8(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))));
  const float inv = qx_inv(a);
  const int x0 = qx_round(y.x, inv), x1 = qx_round(y.y, inv), x2 = qx_round(y.z, inv), x3 = qx_round(y.w, inv);
  const int s = sum8i((x0 + x1) + (x2 + x3));
  if (in) {
    uint32_t *rec = qx + (q >> 3) * QXR;
    uint8_t *rb = reinterpret_cast<uint8_t *>(rec);
    const int off = 4 * ((q & 7) >> 1) + 2 * (q & 1);  // even/odd element slots of this column
    *reinterpret_cast<unsigned short *>(rb + off) = (unsigned short)(((x0 >> 8) & 255) | (((x2 >> 8) & 255) << 8));
    *reinterpret_cast<unsigned short *>(rb + 16 + off) = (unsigned short)(((x1 >> 8) & 255) | (((x3 >> 8) & 255) << 8));
    *reinterpret_cast<unsigned short *>(rb + 32 + off) = (unsigned short)((x0 & 255) | ((x2 & 255) << 8));
    *reinterpret_cast<unsigned short *>(rb + 48 + off) = (unsigned short)((x1 & 255) | ((x3 & 255) << 8));
    if ((q & 7) == 0) {
      rec[16] = __float_as_uint(a / 32767.0f);
      rec[17] = (uint32_t)s;
    }
  }
}

// 64 values, one per lane of the calling wave (lane r: element r & 31 of
// group r >> 5): the two QX records at qx.  Called by the whole wave.
__device__ __forceinline__ void qx_stage_lanes(float v, uint32_t *qx) {
  const int r = lane_id64(), k = r & 31;
  const float m16 = row16_max(fabsf(v));
  const float a = r < 32 ? fmaxf(readlane_f(m16, 0), readlane_f(m16, 16))
                         : fmaxf(readlane_f(m16, 32), readlane_f(m16, 48));
  const int xi = qx_round(v, qx_inv(a));
  int s16 = xi;
  s16 = s16 + dpp_i<0xB1>(s16);
  s16 = s16 + dpp_i<0x4E>(s16);
  s16 = s16 + dpp_i<0x141>(s16);
  s16 = s16 + dpp_i<0x140>(s16);
  const int s = r < 32 ? __builtin_amdgcn_readlane(s16, 0) + __builtin_amdgcn_readlane(s16, 16)
                       : __builtin_amdgcn_readlane(s16, 32) + __builtin_amdgcn_readlane(s16, 48);
  uint32_t *rec = qx + (r >> 5) * QXR;
  uint8_t *rb = reinterpret_cast<uint8_t *>(rec);
  const int off = 16 * (k & 1) + 4 * (k >> 3) + ((k & 7) >> 1);
  rb[off] = (uint8_t)((xi >> 8) & 255);
  rb[32 + off] = (uint8_t)(xi & 255);
  if (k == 0) {
    rec[16] = __float_as_uint(a / 32767.0f);
    rec[17] = (uint32_t)s;
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

// tile_compute with the activations staged as QX records (m tokens x ng
// groups).
template <int C, int NT = WG>
__device__ __forceinline__ void tile_compute_qx(const TileRegs<C> &R, int nrows, int ng, int nch, int m,
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
      if (c < nch) part[t * nch + c] = q4_qx_part(R.w[j], qx + (t * ng + gj[j]) * QXR, R.s[j]);
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
