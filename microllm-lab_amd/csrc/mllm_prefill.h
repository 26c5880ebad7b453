// mllm_prefill.h -- batched prompt processing (infer.js:553-577 forwardPrompt):
// every layer of a chunk of prompt tokens as a few wide kernels (Q4 GEMMs and
// one causal attention kernel on the f16 matrix cores), writing the KV cache;
// the last chunk also forms the last token's logits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mllm {

// A Q4 group-32 matrix as stored in the PGW1 payload: packed nibbles
// [rows][cols / 2] (byte k/2 of a group holds element k in the low nibble,
// k + 1 in the high one) and scales [rows][cols / 32].
struct PfMat {
  const uint8_t *q;
  const float *s;
  int rows, cols;
};

// The layer matrices are tiled copies (pf_tile); the embedding is not.
struct PfLayer {
  PfMat qkv, proj, w1, w3, w2;             // gpt2: w1 = mlp.fc, w2 = mlp.proj, no w3
  const float *n1, *n2;                    // RMS gains; gpt2: LayerNorm gamma || beta
  const float *qkv_b, *proj_b, *fc_b, *mproj_b;  // gpt2 biases (proj_b / mproj_b may be null)
};

struct PfArgs {
  int arch, L, D, NH, NKV, FF, max_seq, kv_fp16;
  float eps, attn_scale;
  const PfLayer *layers;  // host array of L layers
  PfMat emb;              // tied lm_head: the embedding rows
  const float *wpe, *sf, *rope_cos, *rope_sin;
  const float *norm_f;    // final norm gains (gpt2: ln_f gamma || beta)
  void *kv;               // [L][2][NKV][max_seq][64], f32 or f16
  float *logits;          // [V] the last token's logits
  int *res;               // its argmax
  unsigned char *amx;     // the lm_head argmax launch's scratch (gemv_q4_argmax_scratch bytes, first word zero)
  // work buffers for up to tc tokens
  int tc;
  int32_t *ids;  // [tc]
  float *x;      // [tc][D] residual stream
  float *q;      // [tc][D] roped queries
  float *att;    // [tc][D] attention output
  float *h;      // [tc][FF] MLP activation
  uint8_t *px;   // per 32-token tile: [K / 32][3 pieces x 2 K halves][64 lanes][16 B] f16, then [32] int exponents
};

// The tiled copy of a Q4 matrix that the prefill GEMMs read (rows and cols
// multiples of 32): for row tile rt and group g, 64 lane operands of 8 bytes
// (lane 32 hh + j: bytes 8hh .. 8hh+7 of the group in row 32 rt + j), then the
// scales per (row tile, group) as 32 floats.  pf_tile enqueues the copy on
// `stream` into dst (pf_tiled_bytes(W) bytes) and describes it in *out.
size_t pf_tiled_bytes(const PfMat &W);
int pf_tile(const PfMat &W, void *dst, PfMat *out, hipStream_t stream);

// Shapes the kernels take: head_dim 64, at most 4 query heads per KV head,
// d_model and d_ff multiples of 64 up to 4096.
bool pf_supported(const PfArgs &A);

// Bytes of work buffers for tc tokens (one allocation, carved by pf_carve).
size_t pf_buffer_bytes(const PfArgs &A, int tc);
void pf_carve(PfArgs &A, void *base, int tc);

// Tokens ids[0 .. n) at positions pos0 .. pos0 + n (n <= tc, pos0 + n <=
// max_seq) through every layer: their K and V are written to the cache.
// With `last` (the chunk ends the prompt) the last token's logits and argmax
// are formed as well (the last layer's attention and MLP for its 32-token
// tile, the final norm, the lm_head); otherwise the last layer stops after
// its K and V.  Returns 0 or an MLLM_ERR_* code with the message set.
int pf_layers(const PfArgs &A, const int32_t *ids, int n, int pos0, bool last, hipStream_t stream);

}  // namespace mllm
