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
