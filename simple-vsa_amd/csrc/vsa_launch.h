// Host-side helpers for the C ABI entry points: dtype dispatch and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/vsa_capi.h"

// Instantiate BODY with T bound to the element type named by `dtype`;
// returns VSA_ERR_DTYPE from the enclosing function for anything else.
#define VSA_DISPATCH_ALL(dtype, T, BODY)      \
  do {                                        \
    if ((dtype) == VSA_BF16) {                \
      typedef __bf16 T;                       \
      BODY;                                   \
    } else if ((dtype) == VSA_F16) {          \
      typedef _Float16 T;                     \
      BODY;                                   \
    } else if ((dtype) == VSA_F32) {          \
      typedef float T;                        \
      BODY;                                   \
    } else {                                  \
      return VSA_ERR_DTYPE;                   \
    }                                         \
  } while (0)

// Same, for the MFMA kernels (bf16 / fp16 only).
#define VSA_DISPATCH_MFMA(dtype, T, BODY)     \
  do {                                        \
    if ((dtype) == VSA_BF16) {                \
      typedef __bf16 T;                       \
      BODY;                                   \
    } else if ((dtype) == VSA_F16) {          \
      typedef _Float16 T;                     \
      BODY;                                   \
    } else {                                  \
      return VSA_ERR_DTYPE;                   \
    }                                         \
  } while (0)

static inline int vsa_check_launch() {
  return hipGetLastError() == hipSuccess ? VSA_OK : VSA_ERR_LAUNCH;
}
