/*
 * mllm_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see mllm_oracle.h).
 *
 * A plain-C restatement of the reference's CPU decode path.  Numerics follow
 * the reference exactly where it is cheap to do so:
 *   - infer.js functions use C doubles where JS uses numbers and round to
 *     float exactly where infer.js stores into a Float32Array;
 *   - kernels.rs functions use float everywhere, in the same order;
 *   - compiled with -ffp-contract=off so no FMA is formed.
 *
 * Pinning (how each function is checked beyond restating it; tests/ files):
 *   orc_quant_q4        golden vectors written by the reference quant_q4
 *                       (tests/golden/quant_q4_vectors.npz) + brute-force cases
 *   orc_dequant_*       quant->dequant error bound and exact requantisation
 *   orc_gemv_*_js       numpy float64 matmul of the dequantised matrix
 *   orc_gemv_*_wasm     same, to f32 rounding bounds
 *   orc_rms_norm_*      torch float64 rms_norm
 *   orc_layer_norm_js   torch float64 layer_norm
 *   orc_silu_mul_*      torch float64 silu
 *   orc_gelu_new_js     torch float64 gelu(approximate="tanh")
 *   orc_build_rope /    complex-rotation closed form (x_d + i x_{d+half}) * e^{i p w}
 *   orc_apply_rope_js
 *   orc_softmax_js      torch float64 softmax
 *   orc_argmax*         brute force on tiny vocabularies
 *   orc_lookup_draft    hand-made sequences with known drafts
 *   orc_forward_*       HF transformers LlamaForCausalLM / GPT2LMHeadModel (float64)
 *                       built from the same dequantised weights; prefill/decode
 *                       consistency invariant
 *   orc_quant_q8*       the reference ships no Q8 quantiser (its Q8 format,
 *                       weights.js:96-104, is per-row), so the rule is this
 *                       build's: pinned by closed form and brute force (scale
 *                       exactly f32(amax/127), the largest element to +-127,
 *                       every element to the nearest of the 255 levels, ties
 *                       to even).
 */
#define _POSIX_C_SOURCE 200809L
#include "mllm_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* quantisers                                                                */
/* ------------------------------------------------------------------------ */

/* convert_hf_to_pgw.py:18-34 (identical in convert_gpt2_to_pgw.py:18-34).
 * amax = float(max|chunk|); sc = amax/8 (f64) or 1.0; scales stores f32(sc).
 * chunk / sc is a float32 array divided by a Python float: NumPy computes it in
 * float32 with sc cast to float32; np.rint rounds half to even; +8, clip to
 * [0, 15], then low nibble = even element, high nibble = odd element. */
void orc_quant_q4(const float *mat, int rows, int cols, int group, uint8_t *packed, float *scales) {
  const int ng = cols / group;
  for (int r = 0; r < rows; r++) {
    const float *row = mat + (size_t)r * cols;
    for (int g = 0; g < ng; g++) {
      const float *chunk = row + (size_t)g * group;
      float amaxf = 0.0f;
      for (int k = 0; k < group; k++) {
        float a = fabsf(chunk[k]);
        if (a > amaxf) amaxf = a;
      }
      double amax = (double)amaxf;
      double sc = amax > 0 ? amax / 8.0 : 1.0;
      float scf = (float)sc;
      scales[(size_t)r * ng + g] = scf;
      uint8_t *dst = packed + (size_t)r * (cols / 2) + (size_t)g * (group / 2);
      for (int k = 0; k < group; k += 2) {
        float q0 = rintf(chunk[k] / scf) + 8.0f;
        float q1 = rintf(chunk[k + 1] / scf) + 8.0f;
        q0 = q0 < 0.0f ? 0.0f : (q0 > 15.0f ? 15.0f : q0);
        q1 = q1 < 0.0f ? 0.0f : (q1 > 15.0f ? 15.0f : q1);
        dst[k / 2] = (uint8_t)((uint8_t)q0 | ((uint8_t)q1 << 4));
      }
    }
  }
}

static void quant_q8_span(const float *x, int n, int8_t *q, float *sc_out) {
  float amaxf = 0.0f;
  for (int k = 0; k < n; k++) {
    float a = fabsf(x[k]);
    if (a > amaxf) amaxf = a;
  }
  float sc = amaxf > 0 ? (float)((double)amaxf / 127.0) : 1.0f;
  *sc_out = sc;
  for (int k = 0; k < n; k++) {
    float v = rintf(x[k] / sc);
    v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
    q[k] = (int8_t)v;
  }
}

void orc_quant_q8g32(const float *mat, int rows, int cols, int8_t *q, float *scales) {
  const int ng = cols / 32;
  for (int r = 0; r < rows; r++)
    for (int g = 0; g < ng; g++)
      quant_q8_span(mat + (size_t)r * cols + g * 32, 32, q + (size_t)r * cols + g * 32, scales + (size_t)r * ng + g);
}

void orc_quant_q8row(const float *mat, int rows, int cols, int8_t *q, float *scales) {
  for (int r = 0; r < rows; r++) quant_q8_span(mat + (size_t)r * cols, cols, q + (size_t)r * cols, scales + r);
}

/* ------------------------------------------------------------------------ */
/* dequant                                                                   */
/* ------------------------------------------------------------------------ */

/* weights.js:106-123 (and infer.js:402-415 for one row): ((b & 15) - 8) * sc for
 * the even element, ((b >> 4) - 8) * sc for the odd one; one f32 rounding. */
void orc_dequant_q4(const uint8_t *packed, const float *scales, int rows, int cols, int group, float *out) {
  const int ng = cols / group;
  for (int r = 0; r < rows; r++)
    for (int g = 0; g < ng; g++) {
      const double sc = scales[(size_t)r * ng + g];
      const uint8_t *base = packed + (size_t)r * (cols / 2) + (size_t)g * (group / 2);
      float *dst = out + (size_t)r * cols + (size_t)g * group;
      for (int k = 0; k < group; k += 2) {
        const int b = base[k / 2];
        dst[k] = (float)((double)((b & 15) - 8) * sc);
        dst[k + 1] = (float)((double)((b >> 4) - 8) * sc);
      }
    }
}

/* weights.js:96-104 */
void orc_dequant_q8row(const int8_t *q, const float *scales, int rows, int cols, float *out) {
  for (int r = 0; r < rows; r++)
    for (int c = 0; c < cols; c++)
      out[(size_t)r * cols + c] = (float)((double)q[(size_t)r * cols + c] * (double)scales[r]);
}

void orc_dequant_q8g32(const int8_t *q, const float *scales, int rows, int cols, float *out) {
  const int ng = cols / 32;
  for (int r = 0; r < rows; r++)
    for (int c = 0; c < cols; c++)
      out[(size_t)r * cols + c] = (float)((double)q[(size_t)r * cols + c] * (double)scales[(size_t)r * ng + c / 32]);
}

/* ------------------------------------------------------------------------ */
/* GEMV, infer.js semantics                                                  */
/* ------------------------------------------------------------------------ */

/* infer.js:88-116.  Per group: s accumulates 8-term sums left to right in
 * fp64; acc += s * sc in fp64; y stores f32(acc). */
void orc_gemv_q4_js(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y) {
  const int ng = n / group, packed_row = n / 2, half = group / 2;
  for (int i = 0; i < m; i++) {
    double acc = 0;
    const uint8_t *row = packed + (size_t)i * packed_row;
    const float *so = scale + (size_t)i * ng;
    for (int g = 0; g < ng; g++) {
      const double sc = so[g];
      const uint8_t *base = row + (size_t)g * half;
      const float *xb = x + (size_t)g * group;
      double s = 0;
      for (int k = 0; k < half; k += 4) {
        const int b0 = base[k], b1 = base[k + 1], b2 = base[k + 2], b3 = base[k + 3];
        const float *xi = xb + k * 2;
        double e = (double)((b0 & 15) - 8) * xi[0];
        e += (double)((b0 >> 4) - 8) * xi[1];
        e += (double)((b1 & 15) - 8) * xi[2];
        e += (double)((b1 >> 4) - 8) * xi[3];
        e += (double)((b2 & 15) - 8) * xi[4];
        e += (double)((b2 >> 4) - 8) * xi[5];
        e += (double)((b3 & 15) - 8) * xi[6];
        e += (double)((b3 >> 4) - 8) * xi[7];
        s += e;
      }
      acc += s * sc;
    }
    y[i] = (float)acc;
  }
}

/* infer.js:79-86 */
void orc_gemv_q8_js(int m, int n, const int8_t *q, const float *scale, const float *x, float *y) {
  for (int i = 0; i < m; i++) {
    double s = 0;
    const int8_t *row = q + (size_t)i * n;
    for (int k = 0; k < n; k++) s += (double)row[k] * (double)x[k];
    y[i] = (float)(s * (double)scale[i]);
  }
}

/* Build-defined Q8 group-32, written in the style of infer.js:88-116. */
void orc_gemv_q8g32_js(int m, int n, const int8_t *q, const float *scale, const float *x, float *y) {
  const int ng = n / 32;
  for (int i = 0; i < m; i++) {
    double acc = 0;
    const int8_t *row = q + (size_t)i * n;
    for (int g = 0; g < ng; g++) {
      double s = 0;
      for (int k = 0; k < 32; k++) s += (double)row[g * 32 + k] * (double)x[g * 32 + k];
      acc += s * (double)scale[(size_t)i * ng + g];
    }
    y[i] = (float)acc;
  }
}

/* infer.js:10-29 (the 8-way unroll adds sequentially, so order is k = 0..n-1) */
void orc_gemv_f32_js(int m, int n, const float *w, const float *x, float *y) {
  for (int i = 0; i < m; i++) {
    double s = 0;
    const float *row = w + (size_t)i * n;
    for (int k = 0; k < n; k++) s += (double)row[k] * (double)x[k];
    y[i] = (float)s;
  }
}

/* ------------------------------------------------------------------------ */
/* kernels.rs semantics (f32)                                                */
/* ------------------------------------------------------------------------ */

/* kernels.rs:59-97 */
void orc_gemv_q4_wasm(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y) {
  const int ng = n / group, packed_row = n / 2;
  for (int i = 0; i < m; i++) {
    float acc = 0.0f;
    const uint8_t *row = packed + (size_t)i * packed_row;
    for (int g = 0; g < ng; g++) {
      const float sc = scale[(size_t)i * ng + g];
      const uint8_t *base = row + (size_t)g * (group / 2);
      float s = 0.0f;
      for (int k = 0; k < group; k += 2) {
        const int b = base[k / 2];
        s += (float)((b & 15) - 8) * x[g * group + k];
        s += (float)((b >> 4) - 8) * x[g * group + k + 1];
      }
      acc += s * sc;
    }
    y[i] = acc;
  }
}

/* kernels.rs:41-57 */
void orc_gemv_q8_wasm(int m, int n, const int8_t *q, const float *scale, const float *x, float *y) {
  for (int i = 0; i < m; i++) {
    float s = 0.0f;
    const int8_t *row = q + (size_t)i * n;
    for (int k = 0; k < n; k++) s += (float)row[k] * x[k];
    y[i] = s * scale[i];
  }
}

/* kernels.rs:13-39: four f32 lanes over 16-wide blocks, lane sum, scalar tail */
void orc_gemv_f32_wasm(int m, int n, const float *w, const float *x, float *y) {
  for (int i = 0; i < m; i++) {
    const float *row = w + (size_t)i * n;
    float a[4] = {0, 0, 0, 0};
    int k = 0;
    while (k + 16 <= n) {
      for (int u = 0; u < 4; u++) {
        for (int j = 0; j < 4; j++) a[j] = a[j] + row[k + j] * x[k + j];
        k += 4;
      }
    }
    float s = a[0] + a[1] + a[2] + a[3];
    while (k < n) {
      s += row[k] * x[k];
      k++;
    }
    y[i] = s;
  }
}

/* kernels.rs:99-120 (eps is fixed at 1e-6 there; a parameter here) */
void orc_rms_norm_wasm(int n, const float *x, const float *w, float *out, int tokens, float eps) {
  for (int t = 0; t < tokens; t++) {
    const float *xo = x + (size_t)t * n;
    float *oo = out + (size_t)t * n;
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += xo[i] * xo[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) oo[i] = xo[i] * inv * w[i];
  }
}

/* kernels.rs:122-131 */
void orc_silu_mul_wasm(int n, float *a, const float *b) {
  for (int i = 0; i < n; i++) {
    const float v = a[i];
    a[i] = (v / (1.0f + expf(-v))) * b[i];
  }
}

/* ------------------------------------------------------------------------ */
/* elementwise, infer.js semantics                                           */
/* ------------------------------------------------------------------------ */

/* infer.js:134-143 */
void orc_rms_norm_js(const float *x, const float *w, float *out, int dim, int tokens, double eps) {
  for (int t = 0; t < tokens; t++) {
    const float *xo = x + (size_t)t * dim;
    float *oo = out + (size_t)t * dim;
    double ss = 0;
    for (int i = 0; i < dim; i++) ss += (double)xo[i] * (double)xo[i];
    const double inv = 1.0 / sqrt(ss / dim + eps);
    for (int i = 0; i < dim; i++) oo[i] = (float)((double)xo[i] * inv * (double)w[i]);
  }
}

/* infer.js:147-164 (LN_EPS = 1e-5 at infer.js:145; wb = gamma || beta) */
void orc_layer_norm_js(const float *x, const float *wb, float *out, int dim, int tokens, double eps) {
  for (int t = 0; t < tokens; t++) {
    const float *xo = x + (size_t)t * dim;
    float *oo = out + (size_t)t * dim;
    double mean = 0;
    for (int i = 0; i < dim; i++) mean += xo[i];
    mean /= dim;
    double v = 0;
    for (int i = 0; i < dim; i++) {
      const double del = (double)xo[i] - mean;
      v += del * del;
    }
    const double inv = 1.0 / sqrt(v / dim + eps);
    for (int i = 0; i < dim; i++) oo[i] = (float)(((double)xo[i] - mean) * inv * (double)wb[i] + (double)wb[dim + i]);
  }
}

/* infer.js:178-183 */
void orc_silu_mul_js(float *a, const float *b, int n) {
  for (int i = 0; i < n; i++) {
    const double v = a[i];
    a[i] = (float)((v / (1.0 + exp(-v))) * (double)b[i]);
  }
}

/* infer.js:166-171 */
void orc_gelu_new_js(float *a, int n) {
  for (int i = 0; i < n; i++) {
    const double v = a[i];
    a[i] = (float)(0.5 * v * (1.0 + tanh(0.7978845608028654 * (v + 0.044715 * v * v * v))));
  }
}

/* infer.js:185-206: inv[i] is stored in a Float32Array; freq = t * inv[i] in
 * fp64; cos/sin tables are Float32Array in the cat(freqs, freqs) layout. */
void orc_build_rope(int max_seq, int head_dim, double theta, double pct, float *cos_out, float *sin_out, int *rope_dim) {
  int rd = (int)floor(head_dim * pct);
  rd -= rd % 2;
  const int half = rd / 2;
  float *inv = (float *)malloc(sizeof(float) * (half > 0 ? half : 1));
  for (int i = 0; i < half; i++) inv[i] = (float)(1.0 / pow(theta, (2.0 * i) / rd));
  for (int t = 0; t < max_seq; t++)
    for (int i = 0; i < half; i++) {
      const double freq = (double)t * (double)inv[i];
      const float c = (float)cos(freq), s = (float)sin(freq);
      cos_out[(size_t)t * rd + i] = c;
      cos_out[(size_t)t * rd + half + i] = c;
      sin_out[(size_t)t * rd + i] = s;
      sin_out[(size_t)t * rd + half + i] = s;
    }
  free(inv);
  *rope_dim = rd;
}

/* infer.js:208-225: q is [nHeads][t][headDim]; rotate_half on the first
 * ropeDim components at position offset + ti. */
void orc_apply_rope_js(float *q, int n_heads, int t, int head_dim, const float *cos_t, const float *sin_t, int rope_dim,
                       int offset) {
  const int half = rope_dim / 2;
  float rot[1024];
  for (int h = 0; h < n_heads; h++)
    for (int ti = 0; ti < t; ti++) {
      const int pos = offset + ti;
      float *base = q + ((size_t)h * t + ti) * head_dim;
      const float *c = cos_t + (size_t)pos * rope_dim;
      const float *s = sin_t + (size_t)pos * rope_dim;
      for (int i = 0; i < half; i++) rot[i] = -base[half + i];
      for (int i = 0; i < half; i++) rot[half + i] = base[i];
      for (int i = 0; i < rope_dim; i++)
        base[i] = (float)((double)base[i] * (double)c[i] + (double)rot[i] * (double)s[i]);
    }
}

/* infer.js:227-238: x[i] stores f32(e) but the sum uses the unrounded e. */
void orc_softmax_js(float *x, int n) {
  double mx = -INFINITY;
  for (int i = 0; i < n; i++)
    if (x[i] > mx) mx = x[i];
  double s = 0;
  for (int i = 0; i < n; i++) {
    const double e = exp((double)x[i] - mx);
    x[i] = (float)e;
    s += e;
  }
  const double inv = 1.0 / s;
  for (int i = 0; i < n; i++) x[i] = (float)((double)x[i] * inv);
}

/* ------------------------------------------------------------------------ */
/* argmax / draft                                                            */
/* ------------------------------------------------------------------------ */

/* infer.js:240-250: first index of the maximum */
int orc_argmax(const float *logits, int n) {
  int bi = 0;
  float bv = logits[0];
  for (int i = 1; i < n; i++)
    if (logits[i] > bv) {
      bv = logits[i];
      bi = i;
    }
  return bi;
}

/* infer.js:252-287 */
int orc_argmax_gpt2(const float *logits, int n, const int32_t *hist, int n_past, int no_repeat_ngram, double penalty) {
  int t1 = -1, t2 = -1;
  if (no_repeat_ngram == 3 && n_past >= 2) {
    t1 = hist[n_past - 2];
    t2 = hist[n_past - 1];
  }
  int best = 0;
  double best_v = -INFINITY;
  const int recent = n_past - 32 > 0 ? n_past - 32 : 0;
  for (int i = 0; i < n; i++) {
    double v = logits[i];
    if (no_repeat_ngram == 3 && n_past >= 2) {
      for (int h = 0; h < n_past - 2; h++)
        if (hist[h] == t1 && hist[h + 1] == t2 && hist[h + 2] == i) {
          v = -1e9;
          break;
        }
    }
    if (penalty > 1.0 && v > -1e8) {
      for (int h = recent; h < n_past; h++)
        if (hist[h] == i) {
          v = v > 0 ? v / penalty : v * penalty;
          break;
        }
    }
    if (v > best_v) {
      best_v = v;
      best = i;
    }
  }
  return best;
}

/* webgpu.js:846-865: the k tokens that followed the most recent earlier
 * occurrence of the last n tokens of seq (scan i = len-n-1 down to 0). */
int orc_lookup_draft(const int32_t *seq, int len, int k, int n, int32_t *draft) {
  if (len < n + 1) return 0;
  const int32_t *suf = seq + len - n;
  const int limit = len - n;
  for (int i = limit - 1; i >= 0; i--) {
    int ok = 1;
    for (int j = 0; j < n; j++)
      if (seq[i + j] != suf[j]) {
        ok = 0;
        break;
      }
    if (ok) {
      int d = 0;
      for (int t = 0; t < k && i + n + t < len; t++) draft[d++] = seq[i + n + t];
      return d;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* model: infer.js PetitGPT                                                  */
/* ------------------------------------------------------------------------ */

typedef struct {
  int storage, rows, cols, group;
  const void *data;
  const float *scale;
} omat;

typedef struct {
  const float *norm1, *norm2; /* gpt2: ln1 / ln2 (gamma || beta) */
  omat qkv, proj, w1, w3, w2; /* gpt2: w1 = mlp.fc, w2 = mlp.proj */
  const float *qkv_bias, *proj_bias, *fc_bias, *mproj_bias;
} olayer;

typedef struct {
  int t;
  float *x, *xn, *qkv, *q, *k, *v, *attn, *proj, *ff1, *ff3, *ff2, *scores, *yhead, *logits, *tmp;
} oscratch;

struct orc_model {
  orc_config cfg;
  int head_dim, kv_dim, rep, is_gpt2;
  float *rope_cos, *rope_sin;
  int rope_dim;
  const uint8_t *payload;
  orc_tensor *tensors;
  int n_tensors;
  omat lm_head;
  const float *norm_f, *wpe, *scale_factors;
  olayer *layers;
  float **kcache, **vcache;
  int cache_len;
  int *dbg; /* per layer: bit 0 no attention block, bit 1 no MLP block (orc_set_debug) */
  oscratch s;
};

static const orc_tensor *find_tensor(const orc_model *m, const char *name) {
  for (int i = 0; i < m->n_tensors; i++)
    if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
  return NULL;
}

static int get_mat(const orc_model *m, const char *name, omat *out) {
  const orc_tensor *t = find_tensor(m, name);
  if (!t) return -1;
  out->storage = t->storage;
  out->rows = t->rows;
  out->cols = t->cols;
  out->group = t->group ? t->group : 32;
  out->data = m->payload + t->offset;
  out->scale = (t->storage == ORC_Q4 || t->storage == ORC_Q8 || t->storage == ORC_Q8G32)
                   ? (const float *)(m->payload + t->scale_offset)
                   : NULL;
  return 0;
}

static const float *get_vec(const orc_model *m, const char *name) {
  const orc_tensor *t = find_tensor(m, name);
  if (!t || t->storage != ORC_F32) return NULL;
  return (const float *)(m->payload + t->offset);
}

/* weights.js:129-152 */
static float f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000) << 16;
  int e = (h >> 10) & 0x1f;
  uint32_t f = h & 0x3ff, bits;
  if (e == 0) {
    if (f == 0)
      bits = s;
    else {
      e = 1;
      while ((f & 0x400) == 0) {
        f <<= 1;
        e -= 1;
      }
      f &= 0x3ff;
      bits = s | ((uint32_t)(e + 127 - 15) << 23) | (f << 13);
    }
  } else if (e == 31)
    bits = s | 0x7f800000u | (f << 13);
  else
    bits = s | ((uint32_t)(e + 127 - 15) << 23) | (f << 13);
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static float bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* infer.js:338-346 */
static void mat_gemv(const omat *w, const float *x, float *y) {
  const int m = w->rows, n = w->cols;
  switch (w->storage) {
  case ORC_F32: orc_gemv_f32_js(m, n, (const float *)w->data, x, y); break;
  case ORC_Q8: orc_gemv_q8_js(m, n, (const int8_t *)w->data, w->scale, x, y); break;
  case ORC_Q8G32: orc_gemv_q8g32_js(m, n, (const int8_t *)w->data, w->scale, x, y); break;
  case ORC_Q4: orc_gemv_q4_js(m, n, (const uint8_t *)w->data, w->scale, w->group, x, y); break;
  case ORC_F16:
  case ORC_BF16: { /* infer.js:57-77 */
    const uint16_t *u = (const uint16_t *)w->data;
    for (int i = 0; i < m; i++) {
      double s = 0;
      for (int k = 0; k < n; k++) {
        const uint16_t h = u[(size_t)i * n + k];
        s += (double)(w->storage == ORC_F16 ? f16_to_f32(h) : bf16_to_f32(h)) * (double)x[k];
      }
      y[i] = (float)s;
    }
    break;
  }
  default: memset(y, 0, sizeof(float) * m);
  }
}

/* infer.js:118-132 */
static void gemm_generic(const omat *w, int t, const float *x, float *y) {
  for (int i = 0; i < t; i++) mat_gemv(w, x + (size_t)i * w->cols, y + (size_t)i * w->rows);
}

static void add_bias(float *y, const float *b, int n) {
  if (!b) return;
  for (int i = 0; i < n; i++) y[i] = (float)((double)y[i] + (double)b[i]);
}

static void free_scratch(oscratch *s) {
  float **p[] = {&s->x, &s->xn, &s->qkv, &s->q, &s->k, &s->v, &s->attn, &s->proj,
                 &s->ff1, &s->ff3, &s->ff2, &s->scores, &s->yhead, &s->logits, &s->tmp};
  for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) {
    free(*p[i]);
    *p[i] = NULL;
  }
  s->t = 0;
}

/* infer.js:529-551 */
static void ensure_scratch(orc_model *m, int t) {
  if (m->s.t >= t) return;
  free_scratch(&m->s);
  const orc_config *c = &m->cfg;
  const int hd = m->head_dim, kv = m->kv_dim;
  oscratch *s = &m->s;
  s->t = t;
  s->x = calloc((size_t)t * c->d_model, 4);
  s->xn = calloc((size_t)t * c->d_model, 4);
  s->qkv = calloc((size_t)t * (c->d_model + 2 * kv), 4);
  s->q = calloc((size_t)c->n_heads * t * hd, 4);
  s->k = calloc((size_t)c->n_kv_heads * t * hd, 4);
  s->v = calloc((size_t)c->n_kv_heads * t * hd, 4);
  s->attn = calloc((size_t)t * c->d_model, 4);
  s->proj = calloc((size_t)t * c->d_model, 4);
  s->ff1 = calloc((size_t)t * c->d_ff, 4);
  s->ff3 = calloc((size_t)t * c->d_ff, 4);
  s->ff2 = calloc((size_t)t * c->d_model, 4);
  s->scores = calloc((size_t)c->max_seq_len, 4);
  s->yhead = calloc((size_t)hd, 4);
  s->logits = calloc((size_t)c->vocab_size, 4);
  s->tmp = calloc((size_t)(c->d_model > c->d_ff ? c->d_model : c->d_ff) + 2 * kv + c->d_model, 4);
}

orc_model *orc_model_create(const orc_config *cfg, const uint8_t *payload, const orc_tensor *tensors, int n_tensors) {
  orc_model *m = calloc(1, sizeof(orc_model));
  m->cfg = *cfg;
  m->payload = payload;
  m->n_tensors = n_tensors;
  m->tensors = calloc((size_t)n_tensors, sizeof(orc_tensor));
  for (int i = 0; i < n_tensors; i++) {
    m->tensors[i] = tensors[i];
    m->tensors[i].name = strdup(tensors[i].name);
  }
  const orc_config *c = &m->cfg;
  m->head_dim = c->d_model / c->n_heads;
  m->kv_dim = c->n_kv_heads * m->head_dim;
  m->rep = c->n_heads / c->n_kv_heads;
  m->is_gpt2 = c->arch == 1;
  if (!m->is_gpt2) {
    m->rope_cos = malloc(sizeof(float) * (size_t)c->max_seq_len * m->head_dim);
    m->rope_sin = malloc(sizeof(float) * (size_t)c->max_seq_len * m->head_dim);
    orc_build_rope(c->max_seq_len, m->head_dim, c->rope_theta, c->rope_pct, m->rope_cos, m->rope_sin, &m->rope_dim);
  }
  int bad = get_mat(m, "lm_head", &m->lm_head);
  m->layers = calloc((size_t)c->n_layers, sizeof(olayer));
  char nm[128];
  for (int i = 0; i < c->n_layers && !bad; i++) {
    olayer *L = &m->layers[i];
#define MAT(field, suffix)                                   \
  snprintf(nm, sizeof nm, "blocks.%d.%s", i, suffix);       \
  bad |= get_mat(m, nm, &L->field);
#define VEC(field, suffix)                                   \
  snprintf(nm, sizeof nm, "blocks.%d.%s", i, suffix);       \
  L->field = get_vec(m, nm);
    MAT(qkv, "attn.qkv");
    MAT(proj, "attn.proj");
    if (m->is_gpt2) {
      VEC(norm1, "ln1");
      VEC(norm2, "ln2");
      MAT(w1, "mlp.fc");
      MAT(w2, "mlp.proj");
      VEC(qkv_bias, "attn.qkv_bias");
      VEC(proj_bias, "attn.proj_bias");
      VEC(fc_bias, "mlp.fc_bias");
      VEC(mproj_bias, "mlp.proj_bias");
    } else {
      VEC(norm1, "norm1");
      VEC(norm2, "norm2");
      MAT(w1, "mlp.w1");
      MAT(w3, "mlp.w3");
      MAT(w2, "mlp.w2");
    }
    if (!L->norm1 || !L->norm2) bad = 1;
#undef MAT
#undef VEC
  }
  if (m->is_gpt2) {
    m->norm_f = get_vec(m, "ln_f");
    m->wpe = get_vec(m, "wpe");
    m->scale_factors = get_vec(m, "scale_factors");
    if (!m->wpe) bad = 1;
  } else {
    m->norm_f = get_vec(m, "norm_f");
  }
  if (!m->norm_f) bad = 1;
  if (bad) {
    orc_model_destroy(m);
    return NULL;
  }
  m->kcache = calloc((size_t)c->n_layers, sizeof(float *));
  m->vcache = calloc((size_t)c->n_layers, sizeof(float *));
  for (int i = 0; i < c->n_layers; i++) {
    m->kcache[i] = calloc((size_t)c->n_kv_heads * c->max_seq_len * m->head_dim, 4);
    m->vcache[i] = calloc((size_t)c->n_kv_heads * c->max_seq_len * m->head_dim, 4);
  }
  ensure_scratch(m, 1);
  return m;
}

void orc_model_destroy(orc_model *m) {
  if (!m) return;
  for (int i = 0; i < m->n_tensors; i++) free((void *)m->tensors[i].name);
  free(m->tensors);
  if (m->kcache)
    for (int i = 0; i < m->cfg.n_layers; i++) {
      free(m->kcache[i]);
      free(m->vcache[i]);
    }
  free(m->kcache);
  free(m->vcache);
  free(m->layers);
  free(m->dbg);
  free(m->rope_cos);
  free(m->rope_sin);
  free_scratch(&m->s);
  free(m);
}

/* infer.js:348-358 */
/* The GPU engine's debug knobs (webgpu-metal.js:1263-1279; app.js:1317-1325):
 * layers >= max_layers run nothing (max_layers < 0: all run), no_attn skips
 * every attention block, no_mlp every MLP block, mlp_to >= 0 the MLP blocks
 * of layers >= mlp_to.  A skipped block leaves the residual as it is (and,
 * as in the reference, writes nothing to its KV cache). */
void orc_set_debug(orc_model *m, int max_layers, int no_attn, int no_mlp, int mlp_to) {
  if (!m->dbg) m->dbg = calloc((size_t)m->cfg.n_layers, sizeof(int));
  for (int li = 0; li < m->cfg.n_layers; li++) {
    int d = 0;
    if (max_layers >= 0 && li >= max_layers) d = 3;
    if (no_attn) d |= 1;
    if (no_mlp || (mlp_to >= 0 && li >= mlp_to)) d |= 2;
    m->dbg[li] = d;
  }
}

void orc_reset_cache(orc_model *m) {
  for (int i = 0; i < m->cfg.n_layers; i++) {
    memset(m->kcache[i], 0, sizeof(float) * (size_t)m->cfg.n_kv_heads * m->cfg.max_seq_len * m->head_dim);
    memset(m->vcache[i], 0, sizeof(float) * (size_t)m->cfg.n_kv_heads * m->cfg.max_seq_len * m->head_dim);
  }
  m->cache_len = 0;
}

int orc_cache_len(const orc_model *m) { return m->cache_len; }
void orc_set_cache_len(orc_model *m, int len) { m->cache_len = len; }

/* infer.js:395-420 */
static void embed_row_quant(const orc_model *m, int id, float *row) {
  const omat *w = &m->lm_head;
  const int n = m->cfg.d_model;
  if (w->storage == ORC_Q8) {
    const double sc = w->scale[id];
    for (int i = 0; i < n; i++) row[i] = (float)((double)((const int8_t *)w->data)[(size_t)id * n + i] * sc);
  } else if (w->storage == ORC_Q8G32) {
    orc_dequant_q8g32((const int8_t *)w->data + (size_t)id * n, w->scale + (size_t)id * (n / 32), 1, n, row);
  } else if (w->storage == ORC_Q4) {
    const int ng = n / w->group;
    orc_dequant_q4((const uint8_t *)w->data + (size_t)id * (n / 2), w->scale + (size_t)id * ng, 1, n, w->group, row);
  }
  if (m->is_gpt2 && m->scale_factors)
    for (int i = 0; i < n; i++) row[i] = (float)((double)row[i] / (double)m->scale_factors[i]);
}

/* infer.js:360-393 */
static void embed(const orc_model *m, const int32_t *ids, int t, float *out, int pos0) {
  const int D = m->cfg.d_model;
  const omat *w = &m->lm_head;
  for (int ti = 0; ti < t; ti++) {
    float *dst = out + (size_t)ti * D;
    const int id = ids[ti];
    if (w->storage == ORC_F32) {
      memcpy(dst, (const float *)w->data + (size_t)id * D, sizeof(float) * D);
    } else if (w->storage == ORC_F16 || w->storage == ORC_BF16) {
      const uint16_t *u = (const uint16_t *)w->data + (size_t)id * D;
      for (int i = 0; i < D; i++) dst[i] = w->storage == ORC_F16 ? f16_to_f32(u[i]) : bf16_to_f32(u[i]);
    } else {
      embed_row_quant(m, id, dst);
    }
  }
  if (m->is_gpt2) {
    const int max_seq = m->cfg.max_seq_len ? m->cfg.max_seq_len : 1024;
    for (int ti = 0; ti < t; ti++) {
      float *dst = out + (size_t)ti * D;
      const int pos = pos0 + ti < max_seq - 1 ? pos0 + ti : max_seq - 1;
      const float *src = m->wpe + (size_t)pos * D;
      for (int i = 0; i < D; i++) dst[i] = (float)((double)dst[i] + (double)src[i]);
    }
  }
}

/* infer.js:422-504 */
static const float *attention(orc_model *m, int layer, const float *x, int t, int past) {
  const orc_config *c = &m->cfg;
  const int D = c->d_model, hd = m->head_dim, kv = m->kv_dim, NH = c->n_heads, NKV = c->n_kv_heads;
  const int width = D + 2 * kv;
  oscratch *s = &m->s;
  const olayer *L = &m->layers[layer];
  gemm_generic(&L->qkv, t, x, s->qkv);
  if (m->is_gpt2)
    for (int ti = 0; ti < t; ti++) add_bias(s->qkv + (size_t)ti * width, L->qkv_bias, width);
  for (int ti = 0; ti < t; ti++) {
    const float *src = s->qkv + (size_t)ti * width;
    for (int h = 0; h < NH; h++)
      for (int d = 0; d < hd; d++) s->q[((size_t)h * t + ti) * hd + d] = src[h * hd + d];
    for (int h = 0; h < NKV; h++)
      for (int d = 0; d < hd; d++) {
        s->k[((size_t)h * t + ti) * hd + d] = src[D + h * hd + d];
        s->v[((size_t)h * t + ti) * hd + d] = src[D + kv + h * hd + d];
      }
  }
  if (!m->is_gpt2) {
    orc_apply_rope_js(s->q, NH, t, hd, m->rope_cos, m->rope_sin, m->rope_dim, past);
    orc_apply_rope_js(s->k, NKV, t, hd, m->rope_cos, m->rope_sin, m->rope_dim, past);
  }
  float *kC = m->kcache[layer], *vC = m->vcache[layer];
  const int seq = past + t;
  for (int h = 0; h < NKV; h++)
    for (int ti = 0; ti < t; ti++) {
      const size_t dst = ((size_t)h * c->max_seq_len + past + ti) * hd;
      const size_t src = ((size_t)h * t + ti) * hd;
      memcpy(kC + dst, s->k + src, sizeof(float) * hd);
      memcpy(vC + dst, s->v + src, sizeof(float) * hd);
    }
  const double scale = 1.0 / sqrt((double)hd);
  for (int h = 0; h < NH; h++) {
    const int kvh = h / m->rep;
    for (int qi = 0; qi < t; qi++) {
      const int qpos = past + qi;
      const float *qv = s->q + ((size_t)h * t + qi) * hd;
      for (int kj = 0; kj < seq; kj++) {
        if (kj > qpos) {
          s->scores[kj] = -1e9f;
          continue;
        }
        const float *kr = kC + ((size_t)kvh * c->max_seq_len + kj) * hd;
        double dot = 0;
        for (int d = 0; d < hd; d++) dot += (double)qv[d] * (double)kr[d];
        s->scores[kj] = (float)(dot * scale);
      }
      orc_softmax_js(s->scores, seq);
      for (int d = 0; d < hd; d++) s->yhead[d] = 0.0f;
      for (int kj = 0; kj < seq; kj++) {
        const double a = s->scores[kj];
        if (a == 0) continue;
        const float *vr = vC + ((size_t)kvh * c->max_seq_len + kj) * hd;
        for (int d = 0; d < hd; d++) s->yhead[d] = (float)((double)s->yhead[d] + a * (double)vr[d]);
      }
      memcpy(s->attn + ((size_t)qi * NH + h) * hd, s->yhead, sizeof(float) * hd);
    }
  }
  gemm_generic(&L->proj, t, s->attn, s->proj);
  if (m->is_gpt2)
    for (int ti = 0; ti < t; ti++) add_bias(s->proj + (size_t)ti * D, L->proj_bias, D);
  return s->proj;
}

/* infer.js:506-527 */
static const float *ffn(orc_model *m, int layer, const float *x, int t) {
  const orc_config *c = &m->cfg;
  oscratch *s = &m->s;
  const olayer *L = &m->layers[layer];
  const int n = t * c->d_ff;
  if (m->is_gpt2) {
    gemm_generic(&L->w1, t, x, s->ff1);
    for (int ti = 0; ti < t; ti++) add_bias(s->ff1 + (size_t)ti * c->d_ff, L->fc_bias, c->d_ff);
    orc_gelu_new_js(s->ff1, n);
    gemm_generic(&L->w2, t, s->ff1, s->ff2);
    for (int ti = 0; ti < t; ti++) add_bias(s->ff2 + (size_t)ti * c->d_model, L->mproj_bias, c->d_model);
    return s->ff2;
  }
  gemm_generic(&L->w1, t, x, s->ff1);
  gemm_generic(&L->w3, t, x, s->ff3);
  orc_silu_mul_js(s->ff1, s->ff3, n);
  gemm_generic(&L->w2, t, s->ff1, s->ff2);
  return s->ff2;
}

static void norm(const orc_model *m, const float *x, const float *w, float *out, int t) {
  if (m->is_gpt2)
    orc_layer_norm_js(x, w, out, m->cfg.d_model, t, 1e-5);
  else
    orc_rms_norm_js(x, w, out, m->cfg.d_model, t, m->cfg.norm_eps);
}

/* the shared body of infer.js:553-601: t tokens at positions past..past+t-1;
 * leaves the final-normed activations in s->xn. */
static void forward_body(orc_model *m, const int32_t *ids, int t, int past) {
  const orc_config *c = &m->cfg;
  ensure_scratch(m, t);
  oscratch *s = &m->s;
  const int D = c->d_model;
  embed(m, ids, t, s->x, past);
  for (int li = 0; li < c->n_layers; li++) {
    /* webgpu-metal.js:1263-1279: a dropped block's dispatches are skipped */
    const int dbg = m->dbg ? m->dbg[li] : 0;
    if (!(dbg & 1)) {
      norm(m, s->x, m->layers[li].norm1, s->xn, t);
      const float *att = attention(m, li, s->xn, t, past);
      for (int i = 0; i < t * D; i++) s->x[i] = (float)((double)s->x[i] + (double)att[i]);
    }
    if (!(dbg & 2)) {
      norm(m, s->x, m->layers[li].norm2, s->xn, t);
      const float *ff = ffn(m, li, s->xn, t);
      for (int i = 0; i < t * D; i++) s->x[i] = (float)((double)s->x[i] + (double)ff[i]);
    }
  }
  m->cache_len = past + t;
  norm(m, s->x, m->norm_f, s->xn, t);
}

/* infer.js:553-577 (pastLen = 0) */
const float *orc_forward_prompt(orc_model *m, const int32_t *ids, int t) {
  forward_body(m, ids, t, 0);
  mat_gemv(&m->lm_head, m->s.xn + (size_t)(t - 1) * m->cfg.d_model, m->s.logits);
  return m->s.logits;
}

/* infer.js:579-601 */
const float *orc_forward_decode(orc_model *m, int32_t id) {
  forward_body(m, &id, 1, m->cache_len);
  mat_gemv(&m->lm_head, m->s.xn, m->s.logits);
  return m->s.logits;
}

void orc_forward_multi(orc_model *m, const int32_t *ids, int t, float *logits_all) {
  forward_body(m, ids, t, m->cache_len);
  for (int i = 0; i < t; i++)
    mat_gemv(&m->lm_head, m->s.xn + (size_t)i * m->cfg.d_model, logits_all + (size_t)i * m->cfg.vocab_size);
}

int orc_model_gemv(orc_model *m, const char *name, const float *x, float *y) {
  omat w;
  if (get_mat(m, name, &w)) return -1;
  mat_gemv(&w, x, y);
  return 0;
}

/* infer.js:603-646 without the clocks.  stop_reason: 0 max_new_tokens, 1 eos. */
int orc_generate(orc_model *m, const int32_t *ids, int n_ids, int max_new, int eos_id, int32_t *out, int *stop_reason) {
  const int max_seq = m->cfg.max_seq_len ? m->cfg.max_seq_len : 2048;
  int max_prompt = max_seq - max_new - 1;
  if (max_prompt < 1) max_prompt = 1;
  if (n_ids > max_prompt) {
    ids += n_ids - max_prompt;
    n_ids = max_prompt;
  }
  orc_reset_cache(m);
  const float *logits = orc_forward_prompt(m, ids, n_ids);
  const int V = m->cfg.vocab_size;
  int n_out = 0;
  int next = m->is_gpt2 ? orc_argmax_gpt2(logits, V, out, 0, 3, 1.15) : orc_argmax(logits, V);
  out[n_out++] = next;
  *stop_reason = 0;
  if (next == eos_id) {
    *stop_reason = 1;
    return n_out;
  }
  for (int i = 1; i < max_new; i++) {
    if (n_ids + n_out >= m->cfg.max_seq_len) break;
    const float *st = orc_forward_decode(m, next);
    next = m->is_gpt2 ? orc_argmax_gpt2(st, V, out, n_out, 3, 1.15) : orc_argmax(st, V);
    out[n_out++] = next;
    if (next == eos_id) {
      *stop_reason = 1;
      return n_out;
    }
  }
  return n_out;
}
