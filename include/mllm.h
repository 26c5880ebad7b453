/*
 * mllm.h -- C ABI of libmllm, the MI355X (gfx950) fused Q4 decode step.
 *
 * This is the drop-in boundary for microllm-lab's decode hot path.  Two levels:
 *
 *  1. Operator level: the kernels the reference exports from engine/kernels.rs
 *     (compiled to kernels.wasm and plugged into PetitGPT.gemv by
 *     engine/worker.js:20-31).  Same argument order and meaning; pointers are
 *     DEVICE pointers (the reference's are wasm linear-memory offsets); every
 *     call returns a status code instead of nothing.
 *
 *  2. Engine level: the PetitGPT model API of engine/infer.js:289-647
 *     (constructor, forwardPrompt, forwardDecode, resetCache, cacheLen, gemv)
 *     plus the GPU engine's multi-token pass (engine/webgpu.js:1120-1138 with
 *     logitsEach) and its chained decode (CHAIN_TOK, engine/webgpu-metal.js:22,
 *     609-610).  Host buffers in, host buffers out; weights, KV cache and
 *     scratch stay resident in HBM.
 *
 * Conventions:
 *   - Return value 0 (MLLM_OK) on success, otherwise an MLLM_ERR_* code; the
 *     message is available from mllm_last_error() (thread-local).
 *   - `stream` is a hipStream_t passed as void*; NULL means the default stream.
 *     Operator calls are asynchronous on that stream.
 *   - Engine calls are synchronous and not thread-safe per model (the
 *     reference serialises calls per engine the same way, app.js:58-63).
 *   - Arrays of group-32 Q4 weights use the PGW1 layout: packed [m][n/2] bytes
 *     (element 2k in the low nibble of byte k, 2k+1 in the high nibble) and
 *     scales [m][n/32] f32; w = (nibble - 8) * scale.
 */
#ifndef MLLM_H
#define MLLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLLM_OK 0
#define MLLM_ERR_INVALID 1     /* bad argument or shape */
#define MLLM_ERR_HIP 2         /* HIP runtime error */
#define MLLM_ERR_OOM 3         /* device allocation failed */
#define MLLM_ERR_UNSUPPORTED 4 /* shape/format this build does not handle */
#define MLLM_ERR_DEVICE 5      /* a kernel reported an error (e.g. barrier time-out) */

/* Thread-local message for the last non-zero return (never NULL). */
const char *mllm_last_error(void);

/* kernels.rs:133-136 kernel_version() -> 1.  This library reports 1 as well:
 * the operator semantics below are the reference's version-1 semantics. */
int mllm_kernel_version(void);

/* ========================================================================
 * Operator level (device pointers)
 * ====================================================================== */

/* kernels.rs:13-39 gemv_f32(m, n, w, x, y): y[m] = W[m][n] . x[n] */
int mllm_gemv_f32(int m, int n, const float *w, const float *x, float *y, void *stream);

/* kernels.rs:41-57 gemv_q8(m, n, q, scale, x, y): per-row Q8,
 * y[i] = scale[i] * sum_k q[i][k] * x[k]   (weights.js:96-104 layout) */
int mllm_gemv_q8(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, void *stream);

/* kernels.rs:59-97 gemv_q4(m, n, packed, scale, group, x, y) and
 * infer.js:88-116 gemvQ4: y[i] = sum_g scale[i][g] * sum_k (nib - 8) * x[g*32+k].
 * group must be 32; n % 32 == 0; packed and x 16-byte aligned. */
int mllm_gemv_q4(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y,
                 void *stream);

/* infer.js:597-600 (the lm_head GEMV of the last row) followed by argmax,
 * infer.js:240-250 (GPU: webgpu-metal.js:786-813): y = W x as mllm_gemv_q4
 * computes it (bit-identical), and *argmax = the first index of the maximum
 * of y (best = 0, bestV = y[0], then each later row strictly larger; NaN
 * rows never win).  argmax is a device pointer.  The per-workgroup maxima and
 * a completion counter live in a scratch buffer that the library allocates
 * per device on first use; calls on one device must not overlap. */
int mllm_gemv_q4_argmax(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y,
                        int32_t *argmax, void *stream);

/* No counterpart in the reference.  mllm_gemv_q4_argmax for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc): the same kernel and results, with its scratch in a
 * fixed 128 KiB device array (one per GPU, held until the process ends), so
 * the call allocates nothing.  At most 16376 workgroup tiles (the 49152-row
 * lm_head takes 1536); larger shapes return MLLM_ERR_UNSUPPORTED.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU race. */
int mllm_gemv_q4_argmax_noalloc(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x,
                                float *y, int32_t *argmax, void *stream);

/* No reference counterpart (BASELINE config 2 asks for it; the reference's Q8
 * is per-row only): Q8 group-32, q [m][n] i8 + scale [m][n/32] f32. */
int mllm_gemv_q8_g32(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, void *stream);

/* infer.js:118-132 gemmGeneric for a Q4 matrix: y[t][m] = W . x[t][n] for
 * t tokens, each row bit-identical to mllm_gemv_q4 on that token. */
int mllm_gemm_q4(int t, int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y,
                 void *stream);

/* No reference counterpart: one launch over `count` Q4 GEMVs of the same
 * shape (a layer stack), arrays of device pointers in device memory (every
 * packed and x pointer 16-byte aligned). */
int mllm_gemv_q4_batched(int count, int m, int n, const uint8_t *const *packed, const float *const *scale,
                         const float *const *x, float *const *y, void *stream);

/* No reference counterpart (BASELINE config 2 times the Q8 group-32 variant
 * of each layer shape stacked): one launch over `count` mllm_gemv_q8_g32
 * calls of the same shape, arrays of device pointers in device memory
 * (every q and x pointer 16-byte aligned); each matrix's rows are
 * bit-identical to a single mllm_gemv_q8_g32 call's. */
int mllm_gemv_q8_g32_batched(int count, int m, int n, const int8_t *const *q, const float *const *scale,
                             const float *const *x, float *const *y, void *stream);

/* kernels.rs:99-120 rms_norm(n, x, w, out, tokens) with eps as a parameter
 * (the reference hard-codes 1e-6: infer.js:8, kernels.rs:106). */
int mllm_rms_norm(int n, const float *x, const float *w, float *out, int tokens, float eps, void *stream);

/* kernels.rs:122-131 silu_mul(n, a, b): a[i] = silu(a[i]) * b[i] */
int mllm_silu_mul(int n, float *a, const float *b, void *stream);

/* weights.js:106-123 dequantizeToF32 (q4 branch): out[m][n], bit-exact. */
int mllm_dequant_q4(int m, int n, const uint8_t *packed, const float *scale, int group, float *out, void *stream);

/* ========================================================================
 * Engine level (infer.js PetitGPT)
 * ====================================================================== */

/* Model configuration: the PGW1 header fields (weights.js:17-29) plus the
 * two numeric choices the header does not carry. */
typedef struct mllm_config {
  int32_t arch; /* 0 = llama, 1 = gpt2 (weights.js:15-16) */
  int32_t vocab_size, n_layers, d_model, n_heads, n_kv_heads, d_ff, max_seq_len;
  double rope_theta, rope_pct;
  float norm_eps;  /* RMSNorm eps; the reference uses 1e-6 (infer.js:8) */
  int32_t kv_fp16; /* 0: f32 KV cache as the reference; 1: fp16 KV cache */
} mllm_config;

/* Storage codes: the PGW1 dtype codes (weights.js:3) plus 5 = Q8 group-32. */
#define MLLM_F32 0
#define MLLM_F16 1
#define MLLM_BF16 2
#define MLLM_Q8 3
#define MLLM_Q4 4
#define MLLM_Q8G32 5

/* One entry of the PGW1 JSON tensor table (convert_hf_to_pgw.py:44-69);
 * offsets are relative to the payload start. */
typedef struct mllm_tensor {
  const char *name;
  int32_t storage;
  int32_t rows, cols, group; /* 1-D tensors: rows = 1 */
  uint64_t offset, nbytes, scale_offset, scale_nbytes;
} mllm_tensor;

typedef struct mllm_model mllm_model;

/* new PetitGPT(bundle) (infer.js:290-311) + the device upload of
 * GpuPetitGPT.init (webgpu.js:892-1106): copies the payload to HBM once and
 * allocates the KV cache and scratch.  payload is host memory.  Tensor names
 * follow the converters (lm_head, blocks.{i}.attn.qkv, ...).  Matrices may be
 * stored in any kind infer.js:313-346 binds (f32, f16, bf16, per-row Q8, Q4
 * of a group size that is a multiple of 8) or as Q8 group-32, each 16-byte
 * aligned; norms, biases and positions are f32.  A model whose layer matrices
 * and lm_head are all Q4 group-32, at the fused step's shapes, runs the
 * fused decode step (mllm_decode_kernel_name: "k_flow3", "phase kernels",
 * ...); any other runs the kind-generic step ("generic kernels": a few
 * kernels per layer and token, exec modes 1 and 2 only, prompts token by
 * token). */
int mllm_model_create(const mllm_config *cfg, const void *payload, uint64_t payload_nbytes,
                      const mllm_tensor *tensors, int n_tensors, mllm_model **out);
/* GpuPetitGPT.destroy (webgpu.js:1284-1297); NULL is accepted. */
int mllm_model_destroy(mllm_model *model);

/* infer.js:348-358 resetCache; cacheLen getter/setter. */
int mllm_reset_cache(mllm_model *model);
int mllm_cache_len(const mllm_model *model);
int mllm_set_cache_len(mllm_model *model, int len);

/* infer.js:553-577 forwardPrompt(ids): positions 0..n-1, cacheLen = n.
 * logits (host, vocab floats) receives the last row; argmax (nullable) its
 * first-maximum index (infer.js:240-250). */
int mllm_forward_prompt(mllm_model *model, const int32_t *ids, int n, float *logits, int32_t *argmax);

/* infer.js:579-601 forwardDecode(id): one token at position cacheLen,
 * cacheLen += 1.  logits and argmax are nullable. */
int mllm_forward_decode(mllm_model *model, int32_t id, float *logits, int32_t *argmax);

/* The multi-token pass of webgpu.js:557-686 (logitsEach): ids[0..n) at
 * positions cacheLen..cacheLen+n-1 with a causal mask, one argmax per row
 * (argmax[n]); logits [n][vocab] optional.  Every row is bit-identical to the
 * forward_decode call that would have computed it.  Leaves cacheLen += n; the
 * caller rolls it back with mllm_set_cache_len after acceptance
 * (webgpu.js:1254,1263).  n <= mllm_max_pass_tokens(). */
int mllm_forward_verify(mllm_model *model, const int32_t *ids, int n, int32_t *argmax, float *logits);
int mllm_max_pass_tokens(const mllm_model *model);

/* Chained greedy decode on the device (CHAIN_TOK, webgpu-metal.js:609-610;
 * webgpu.js:1202-1226): starting from token `first` at position cacheLen,
 * run up to n_steps decode steps where each step's argmax feeds the next
 * step, without host round trips.  Stops after a step that emits eos_id
 * (eos_id < 0: never).  out_ids receives the emitted ids, *n_out their count;
 * cacheLen advances by *n_out.  For gpt2 the argmax applies argmaxGpt2's
 * 3-gram block and 1.15 penalty (infer.js:252-287) over hist[0..n_hist)
 * followed by the ids emitted here. */
int mllm_decode_chain(mllm_model *model, int32_t first, int n_steps, int32_t eos_id, const int32_t *hist, int n_hist,
                      int32_t *out_ids, int *n_out);

/* model.gemv(name, x, y) (infer.js:338-346): host x [cols] -> host y [rows]. */
int mllm_model_gemv(mllm_model *model, const char *name, const float *x, float *y);

/* Execution mode of the single-token decode step.  3 (the default where the
 * device can co-schedule one workgroup per CU) = one persistent cooperative
 * kernel per decode call or chain, its workgroups ordered by per-item epoch
 * flags instead of grid barriers; 1 (the default otherwise) = one kernel per
 * phase, a chained step replayed from a HIP graph; 2 = the phase kernels
 * launched directly (for profilers); 4 = mode 3's kernel and grid through an
 * ordinary (not cooperative) launch, for profilers that do not follow
 * cooperative launches -- every workgroup is resident only while the device
 * runs nothing else, so it is not a serving mode.  Multi-token passes
 * (prefill, verify) always use the phase kernels.  Results are bit-identical
 * across modes.  Returns MLLM_ERR_UNSUPPORTED for modes 3 and 4 where the
 * persistent kernel is unavailable. */
int mllm_set_exec_mode(mllm_model *model, int mode);

/* No reference counterpart: the execution mode the next decode call will use
 * (after a refused cooperative launch, a default mode 3 has fallen back to
 * 1); -1 for a null model. */
int mllm_get_exec_mode(const mllm_model *model);

/* No reference counterpart: the name of the kernel that runs the next decode
 * step ("k_flow3", "k_flow<4>" ... in exec modes 3 and 4, "phase kernels" in
 * modes 1 and 2), for reports; "" for a null model. */
const char *mllm_decode_kernel_name(const mllm_model *model);

/* No reference counterpart: the most tokens a verify pass (mllm_forward_verify)
 * runs as one step of the persistent kernel in exec modes 3 and 4; longer
 * passes, and every pass in modes 1 and 2, run the phase kernels (the same
 * results, bit for bit).  0 when the persistent kernel is not in use. */
int mllm_flow_verify_tokens(const mllm_model *model);

/* GpuPetitGPT's debug knobs debugMaxLayers / debugNoAttn / debugNoMlp /
 * debugMlpTo (webgpu-metal.js:1263-1279; set from the page's query string,
 * app.js:1317-1325): only the first max_layers layers run (< 0: all),
 * no_attn != 0 drops every attention block, no_mlp != 0 every MLP block,
 * mlp_to >= 0 keeps the MLP blocks of layers < mlp_to only (< 0: all).  A
 * dropped block adds nothing to the residual, in every execution mode and in
 * verify passes, so the logits are the truncated network's, as the
 * reference's skipped dispatches give them (its q/k/v rows are still written
 * to the KV cache, where the reference leaves them unwritten; no kept block
 * reads them).  While a knob is set, prompts run through the decode passes
 * instead of the batched path.  mllm_set_debug(m, -1, 0, 0, -1) restores the
 * full network. */
int mllm_set_debug(mllm_model *model, int max_layers, int no_attn, int no_mlp, int mlp_to);

/* Prompts of at least min_tokens tokens (default 2; 0 = never) are
 * processed in batches (no counterpart in the reference, whose GPU path runs
 * a prompt token by token, webgpu.js:1178-1187): the tokens go through every
 * layer as Q4 GEMMs and one causal attention kernel on the f16 matrix
 * cores, in chunks of up to 2048 tokens, and write the KV cache; the last
 * chunk runs its last layer's attention and MLP on its final 32-token tile
 * and forms the last token's logits (final norm, lm_head, argmax).  Shorter
 * prompts run in passes of mllm_max_pass_tokens() tokens through the decode
 * phases.  The GEMMs take each activation exactly (three f16 pieces of the
 * row scaled by a power of two), the decode GEMVs as 24-bit integers per
 * 32-element group; the two agree to 2e-5 of the logits' scale, not bit for
 * bit (different roundings and summation orders).
 * chunk_tokens (1 .. 2048 or max_seq_len if smaller; 0 = the largest) bounds
 * the tokens per chunk; later chunks read the earlier ones' keys from the
 * cache.  Models with more than 4 query heads per KV head, or d_model / d_ff
 * not multiples of 64, keep the pass path (min_tokens > 0 then returns
 * MLLM_ERR_UNSUPPORTED). */
int mllm_set_prefill(mllm_model *model, int min_tokens, int chunk_tokens);

/* GpuPetitGPT.lastTiming {n, gpuMs} (webgpu.js:1143-1160): the time between
 * HIP events recorded on the model's stream immediately before and after the
 * kernels of the last forward / chain call, and the tokens it produced. */
int mllm_last_timing(const mllm_model *model, float *gpu_ms, int *n_tokens);

/* Per-phase timing of the decode step, the per-kernel counterpart of
 * lastTiming (webgpu.js:1143-1160): runs n_steps chained steps from token
 * `first` at position cacheLen, launching each phase kernel directly on the
 * model's stream with HIP events that stamp the kernel's own begin and end
 * (hipExtLaunchKernel), and writes the mean microseconds per launch of each
 * phase to phase_us[0..MLLM_PHASES): QKV, ATTN, MLP, FINAL, LM, ARGMAX (names
 * from mllm_phase_name).  cacheLen advances by n_steps. */
#define MLLM_PHASES 6
int mllm_profile_decode(mllm_model *model, int32_t first, int n_steps, float *phase_us);
/* Name of decode phase `phase` (0 <= phase < MLLM_PHASES), else NULL. */
const char *mllm_phase_name(int phase);

/* Bytes of device memory the model holds (GpuPetitGPT.bytesAllocated). */
uint64_t mllm_model_device_bytes(const mllm_model *model);

#ifdef __cplusplus
}
#endif
#endif
