// mllm_generic.h -- the decode step for models whose matrices are not all
// Q4 group-32: infer.js:313-346 binds every matrix by its own storage (f32,
// f16, bf16, per-row Q8, Q4 of any group size; this library adds Q8
// group-32), and the reference's GPU engine packs Q8, f16 and bf16 models
// as they are (webgpu.js:902-973).  One token per step, a short chain of
// kernels per layer: norm + GEMV (QKV), RoPE + KV write, attention, GEMV +
// residual (O), norm + GEMV (gate/up + SwiGLU, or fc + GELU), GEMV +
// residual (down); then the final norm + lm_head GEMV and the argmax.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mllm {

// A matrix in the PGW1 payload: w [rows][cols] in its storage (kind = the
// MLLM_* storage code), s its scales (Q8: one per row; Q8 group-32 and Q4:
// one per row and group of `group` columns), null for unscaled kinds.
struct GMat {
  const void *w;
  const float *s;
  int kind, rows, cols, group;
};

struct GLayer {
  GMat qkv, proj, w1, w3, w2;                    // gpt2: w1 = mlp.fc, w2 = mlp.proj, no w3
  const float *n1, *n2;                          // RMS gains; gpt2: LayerNorm gamma || beta
  const float *qkv_b, *proj_b, *fc_b, *mproj_b;  // gpt2 biases (proj_b / mproj_b may be null)
  int dbg;  // debug knobs: bit 0 drops the attention block, bit 1 the MLP block
};

// Where a call stands, in device memory.  The host writes it before a call
// (pos_next = the first position, i_next = 0, the call's kind); each step's
// first kernel takes position and token index from it and advances them, so
// every step of a call launches the same kernels with the same arguments
// (and can be replayed from a graph).
struct GCursor {
  int pos_next, i_next;  // the next step's position and token index
  int pos, i;            // this step's
  int tok;               // chained calls: the next input token (the host sets the first)
  int chain;             // 1: chained decode (the input token is the previous argmax)
  int rows;              // 1: logits row i per step (verify); 0: row 0
  int n_hist, eos, gpt2_rule;  // chained calls: history length, EOS id, argmaxGpt2 (gpt2)
  int done, emitted;     // chained calls: an EOS was emitted; ids emitted so far
};

struct GArgs {
  int arch, L, D, NH, NKV, FF, V, max_seq, kv_fp16;
  int rope_dim;          // rotated components per head (llama; infer.js:185-206)
  float eps, attn_scale;
  const GLayer *layers;  // host array of L layers
  GMat lm;               // tied lm_head (and the embedding rows)
  const float *norm_f, *wpe, *sf, *rope_cos, *rope_sin;
  void *kv;                  // [L][2][NKV][max_seq][64], f32 or f16 (the engine's cache)
  float *x, *qkv, *att, *h;  // one token's rows: [D], [D + 2 NKV 64], [D], [FF]
  float *logits;             // [rows][V]
  int *res;                  // argmax per logits row
  GCursor *cur;
  const int *ids;            // a call's token ids (cursor index i)
  int *hist;                 // chained calls: the history, then the ids emitted
};

// Enqueue one token's step: embedding of the cursor's token at its
// position, every layer, and with lm the final norm, the lm_head (logits
// row: the cursor's i with rows set, else 0) and the argmax (res[row]; in
// chained calls the chain's bookkeeping).  In chained calls every kernel
// returns at once once an EOS has been emitted.
int g_step(const GArgs &A, bool lm, hipStream_t s);

// y[rows] = W . x[cols] (model.gemv for any storage).
int g_gemv(const GMat &W, const float *x, float *y, hipStream_t s);

// The storage kinds and group sizes g_step reads.
bool g_kind_supported(int kind, int group);

}  // namespace mllm
