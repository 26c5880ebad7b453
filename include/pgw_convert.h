/* pgw_convert.h -- C ABI of the PGW1 converter (libpgwconvert.so and the
 * pgw_convert command): a HuggingFace checkpoint (config.json + safetensors)
 * to the PGW1 Q4 file the engine loads, written the way the reference's
 * converters write it.
 *
 * Every function returns 0 or a nonzero code; pgwc_last_error() holds the
 * message of the calling thread's last failure. */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quant_q4 (tools/convert_hf_to_pgw.py:18-34, the same function in
 * tools/convert_gpt2_to_pgw.py): per group of 32 columns, amax = max |x|,
 * sc = amax / 8 (1 when amax is 0) stored as f32, q = clip(rint(x / sc) + 8,
 * 0, 15) in float32 with ties to even, element 2k in the low nibble.  mat is
 * [rows][cols] f32 (cols % 32 == 0); packed [rows][cols / 2], scales
 * [rows][cols / 32]. */
int pgwc_quant_q4(const float *mat, int64_t rows, int64_t cols, uint8_t *packed, float *scales);

/* convert() of tools/convert_hf_to_pgw.py:78-144 without the model download:
 * the Llama-style checkpoint in directory hf_dir (config.json; model.safetensors
 * or model.safetensors.index.json with its shards; F32, F16, BF16 or F64
 * tensors) to out_path, byte for byte the file the reference writes from the
 * same weights (tensor order :104-122, JSON table and 256-byte header
 * :124-141).  max_seq is the header's maxSeqLen (the reference's --max-seq,
 * default 2048).  The tokenizer files and card.json the reference also writes
 * are not produced. */
int pgwc_convert_llama(const char *hf_dir, const char *out_path, int max_seq);

/* convert() of tools/convert_gpt2_to_pgw.py:86-186 after its SmoothQuant
 * calibration: scale_factors [n_embd] f32 are the calibrated channel scales
 * (the reference computes them by running the model over its calibration
 * texts, :103-131; NULL = all ones; n_scale must then equal n_embd); the file written is the reference's
 * for those factors (lm_head scaled by them, ln_f divided by them, Conv1D
 * weights transposed, wpe cut to min(n_positions, max_seq) rows, header qGroup
 * 1).  max_seq: the reference's default is 1024. */
int pgwc_convert_gpt2(const char *hf_dir, const char *out_path, int max_seq, const float *scale_factors, int n_scale);

const char *pgwc_last_error(void);

#ifdef __cplusplus
}
#endif
