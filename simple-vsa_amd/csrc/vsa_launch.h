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

// Alignment the kernels' accesses need (NULL, an absent optional buffer,
// passes): 16 bytes for rows of the element type and the fp32 score /
// probability rows, 8 for int64 index arrays, 4 for int32 arrays and
// lse / delta.
template <unsigned A, typename... P>
static inline bool vsa_aligned(P... p) {
  return ((((uintptr_t)(const void*)p) % A == 0) && ...);
}

static inline int vsa_check_launch() {
  return hipGetLastError() == hipSuccess ? VSA_OK : VSA_ERR_LAUNCH;
}

// CUs of the current device (cached per device; a racy first fill writes the
// same value)
static inline int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace vsa {
// out = T(out_c[block] * gate + fine) with an fp32 gate (common.hip); out may
// alias fine.  gate_mode is 1, 2 or 3 (without the VSA_GATE_F32 flag).
int combine_f32gate(const void* fine, const void* out_c, const void* gate, int gate_mode,
                    int gate_heads, void* out, int64_t bh, int64_t sq, int D, int be, int dtype,
                    hipStream_t s);
// The shape checks combine_f32gate makes, for callers that must reject a call
// before launching anything else.
bool combine_f32gate_shape_ok(int64_t bh, int64_t sq, int D, int be, int dtype);
// Scheduling counters (take_entry) of the persistent forward and dQ kernels for
// launches on stream s, from a file-scope device array (common.hip): one slot
// of zeroed counters per (device, stream), which every launch leaves zeroed.
// nullptr when the slots are all taken or s is not on the current device: the
// kernels then use a fixed stride over their XCD's range.
int32_t* sched_counters(hipStream_t s);
}  // namespace vsa
