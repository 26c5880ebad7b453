/*
 * mllm_oracle.h -- CPU oracle for the fused Q4 decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product library (libmllm) never links,
 * loads or calls it.
 *
 * It is a plain-C restatement of the reference's CPU path:
 *   - engine/infer.js   (JS numbers: fp64 accumulation, Float32Array stores)
 *   - engine/kernels.rs (the wasm kernels: f32 accumulation)
 *   - engine/weights.js (PGW1 dequantisation)
 *   - tools/convert_hf_to_pgw.py quant_q4 (the converter's quantiser)
 *   - engine/webgpu.js  lookupDraft + speculative acceptance
 * Every function cites the reference lines it follows in mllm_oracle.c.
 *
 * Pinning status of each function is listed at the top of mllm_oracle.c.
 */
#ifndef MLLM_ORACLE_H
#define MLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage codes: 0..4 are the PGW1 dtype codes (weights.js:3).  5 is the
 * build-defined Q8 group-32 layout (i8 [m][n] + f32 [m][n/32]). */
enum {
  ORC_F32 = 0,
  ORC_F16 = 1,
  ORC_BF16 = 2,
  ORC_Q8 = 3,
  ORC_Q4 = 4,
  ORC_Q8G32 = 5
};

/* ---- quantisers ------------------------------------------------------- */
/* convert_hf_to_pgw.py:18-34 */
void orc_quant_q4(const float *mat, int rows, int cols, int group, uint8_t *packed, float *scales);
/* Build-defined Q8 group-32: sc = amax/127 (1 if amax==0), q = clip(rint(x/sc), -127, 127). */
void orc_quant_q8g32(const float *mat, int rows, int cols, int8_t *q, float *scales);
/* Build-defined per-row Q8 (the reference ships no Q8 quantiser): same rule over a whole row. */
void orc_quant_q8row(const float *mat, int rows, int cols, int8_t *q, float *scales);

/* ---- dequant ---------------------------------------------------------- */
/* weights.js:106-123 */
void orc_dequant_q4(const uint8_t *packed, const float *scales, int rows, int cols, int group, float *out);
/* weights.js:96-104 */
void orc_dequant_q8row(const int8_t *q, const float *scales, int rows, int cols, float *out);
void orc_dequant_q8g32(const int8_t *q, const float *scales, int rows, int cols, float *out);

/* ---- GEMV, infer.js semantics (fp64 accumulate, f32 store) ------------- */
void orc_gemv_q4_js(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y);
void orc_gemv_q8_js(int m, int n, const int8_t *q, const float *scale, const float *x, float *y);
void orc_gemv_q8g32_js(int m, int n, const int8_t *q, const float *scale, const float *x, float *y);
void orc_gemv_f32_js(int m, int n, const float *w, const float *x, float *y);

/* ---- GEMV + elementwise, kernels.rs semantics (f32 accumulate) ---------- */
void orc_gemv_q4_wasm(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y);
void orc_gemv_q8_wasm(int m, int n, const int8_t *q, const float *scale, const float *x, float *y);
void orc_gemv_f32_wasm(int m, int n, const float *w, const float *x, float *y);
void orc_rms_norm_wasm(int n, const float *x, const float *w, float *out, int tokens, float eps);
void orc_silu_mul_wasm(int n, float *a, const float *b);

/* ---- elementwise, infer.js semantics ------------------------------------ */
void orc_rms_norm_js(const float *x, const float *w, float *out, int dim, int tokens, double eps);
void orc_layer_norm_js(const float *x, const float *wb, float *out, int dim, int tokens, double eps);
void orc_silu_mul_js(float *a, const float *b, int n);
void orc_gelu_new_js(float *a, int n);
void orc_build_rope(int max_seq, int head_dim, double theta, double pct, float *cos_out, float *sin_out, int *rope_dim);
void orc_apply_rope_js(float *q, int n_heads, int t, int head_dim, const float *cos_t, const float *sin_t, int rope_dim,
                       int offset);
void orc_softmax_js(float *x, int n);

/* ---- argmax / draft ------------------------------------------------------ */
int orc_argmax(const float *logits, int n);
int orc_argmax_gpt2(const float *logits, int n, const int32_t *hist, int n_past, int no_repeat_ngram, double penalty);
int orc_lookup_draft(const int32_t *seq, int len, int k, int n, int32_t *draft);

/* ---- model ---------------------------------------------------------------- */
typedef struct orc_config {
  int32_t arch; /* 0 = llama, 1 = gpt2 (weights.js:15-16) */
  int32_t vocab_size, n_layers, d_model, n_heads, n_kv_heads, d_ff, max_seq_len;
  double rope_theta, rope_pct;
  double norm_eps; /* RMSNorm eps; infer.js:8 fixes 1e-6 */
} orc_config;

/* One entry of the PGW1 tensor table (convert_hf_to_pgw.py:44-69). */
typedef struct orc_tensor {
  const char *name;
  int32_t storage; /* ORC_* */
  int32_t rows, cols, group;
  uint64_t offset, nbytes, scale_offset, scale_nbytes;
} orc_tensor;

typedef struct orc_model orc_model;

orc_model *orc_model_create(const orc_config *cfg, const uint8_t *payload, const orc_tensor *tensors, int n_tensors);
void orc_model_destroy(orc_model *m);
void orc_reset_cache(orc_model *m);
/* webgpu-metal.js:1263-1279: the GPU engine's layer-truncation knobs */
void orc_set_debug(orc_model *m, int max_layers, int no_attn, int no_mlp, int mlp_to);
int orc_cache_len(const orc_model *m);
void orc_set_cache_len(orc_model *m, int len);
/* infer.js:553-577 -- returns a pointer to the model's logits scratch [V]. */
const float *orc_forward_prompt(orc_model *m, const int32_t *ids, int t);
/* infer.js:579-601 */
const float *orc_forward_decode(orc_model *m, int32_t id);
/* t tokens at positions cacheLen..cacheLen+t-1 with a causal mask, logits for every row
 * into logits_all [t][V] (the fused pass of webgpu.js:557-686 with logits_each, in
 * infer.js arithmetic).  cacheLen becomes cacheLen+t. */
void orc_forward_multi(orc_model *m, const int32_t *ids, int t, float *logits_all);
/* model.gemv(name, x, y) (infer.js:338-346) */
int orc_model_gemv(orc_model *m, const char *name, const float *x, float *y);
/* Greedy generate (infer.js:603-646) without timing: returns the number of ids written. */
int orc_generate(orc_model *m, const int32_t *ids, int n_ids, int max_new, int eos_id, int32_t *out, int *stop_reason);

#ifdef __cplusplus
}
#endif
#endif
