// mllm_host.h -- host-side helpers shared by the libmllm translation units:
// the thread-local error message behind mllm_last_error() and HIP checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "mllm.h"

namespace mllm {

int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char *what, const char *file, int line);
void clear_error();

// y = W x for one token (the Q4 GEMV of mllm_gemv_q4, the same bits) and the
// first index of its maximum into *argmax, in one launch, with a scratch the
// caller owns: gemv_q4_argmax_scratch(m, n) bytes whose first word is zero
// before the first launch (every launch leaves it zero).  Launches that share
// a scratch must not overlap.
size_t gemv_q4_argmax_scratch(int m, int n);
int gemv_q4_argmax_into(int m, int n, const uint8_t *packed, const float *scale, const float *x, float *y,
                        int32_t *argmax, unsigned char *scratch, hipStream_t st);

}  // namespace mllm

#define MLLM_HIP(expr)                                                   \
  do {                                                                   \
    hipError_t e_ = (expr);                                              \
    if (e_ != hipSuccess) return mllm::hip_fail(e_, #expr, __FILE__, __LINE__); \
  } while (0)

#define MLLM_CHECK(cond, ...)                                    \
  do {                                                           \
    if (!(cond)) return mllm::set_error(MLLM_ERR_INVALID, __VA_ARGS__); \
  } while (0)
