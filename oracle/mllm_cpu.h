/* mllm_cpu.h -- TEST INFRASTRUCTURE ONLY (part of the oracle, liboracle.so).
 *
 * The operator entry points of include/mllm.h with identical signatures, on
 * host pointers: the CPU restatement of the reference's native operator ABI
 * (the wasm exports of engine/kernels.rs:13-136, f32 arithmetic) behind the
 * names and argument checks the GPU library uses, so a test can call either
 * with the same argument list and compare.  The stream argument is ignored.
 * Return codes are those of mllm.h (MLLM_ERR_INVALID 1, MLLM_ERR_UNSUPPORTED
 * 4); mllm_cpu_last_error() holds the calling thread's last message.  No
 * product code links this. */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *mllm_cpu_last_error(void);
int mllm_cpu_kernel_version(void);
int mllm_cpu_gemv_f32(int m, int n, const float *w, const float *x, float *y, void *stream);
int mllm_cpu_gemv_q8(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, void *stream);
int mllm_cpu_gemv_q4(int m, int n, const uint8_t *packed, const float *scale, int group, const float *x, float *y,
                     void *stream);
int mllm_cpu_gemv_q8_g32(int m, int n, const int8_t *q, const float *scale, const float *x, float *y, void *stream);
int mllm_cpu_gemm_q4(int t, int m, int n, const uint8_t *packed, const float *scale, int group, const float *x,
                     float *y, void *stream);
int mllm_cpu_rms_norm(int n, const float *x, const float *w, float *out, int tokens, float eps, void *stream);
int mllm_cpu_silu_mul(int n, float *a, const float *b, void *stream);
int mllm_cpu_dequant_q4(int m, int n, const uint8_t *packed, const float *scale, int group, float *out, void *stream);

#ifdef __cplusplus
}
#endif
