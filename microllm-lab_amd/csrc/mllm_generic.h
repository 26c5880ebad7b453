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
  int *state;                // chained steps: [0] stop flag (EOS emitted), [1] ids emitted
};

// A chained step's argmax: appended at hist[n_hist + step]; gpt2_rule
// applies argmaxGpt2 (infer.js:252-287) over hist[0 .. n_hist + step).
struct GChain {
  int *hist;
  int n_hist, step, eos, gpt2_rule;
};

// One token (its id read on the device at tok) at position pos through
// every layer; with row >= 0, the final norm, the lm_head into logits row
// `row` and its argmax into res[row] (and, with chain, the chain's
// bookkeeping).  With chain, every kernel returns at once once state[0] is set.
int g_step(const GArgs &A, const int *tok, int pos, int row, const GChain *chain, hipStream_t s);

// y[rows] = W . x[cols] (model.gemv for any storage).
int g_gemv(const GMat &W, const float *x, float *y, hipStream_t s);

// The storage kinds and group sizes g_step reads.
bool g_kind_supported(int kind, int group);

}  // namespace mllm
