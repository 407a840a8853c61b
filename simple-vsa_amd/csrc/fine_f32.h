// Host launchers of the fp32 fine kernels (fine_f32.hip); the C ABI entry
// points vsa_sparse_fwd / vsa_sparse_bwd_dq / vsa_sparse_bwd_dkdv dispatch
// fp32 inputs to them.  Arguments and results are those of the entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vsa {

int sparse_fwd_f32(const void* q, const void* k, const void* v, const int32_t* selected,
                   const int32_t* kv_vbs, void* out, void* fine, float* lse, const void* out_c,
                   const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq,
                   int64_t skv, int D, int be, int topk, float scale, hipStream_t s);

int sparse_dq_f32(const void* q, const void* k, const void* v, const void* dout,
                  const float* lse, const float* delta, const int32_t* selected,
                  const int32_t* kv_vbs, void* dq, const void* dqc, const int32_t* q_vbs,
                  int64_t bh, int64_t sq, int64_t skv, int D, int be, int topk, float scale,
                  hipStream_t s);

int sparse_dkdv_f32(const void* q, const void* k, const void* v, const void* dout,
                    const float* lse, const float* delta, const int32_t* counts,
                    const int32_t* offsets, const int32_t* inverse, const int32_t* kv_vbs,
                    void* dk, void* dv, const void* dkc, const void* dvc, int64_t bh, int64_t sq,
                    int64_t skv, int D, int be, int topk, float scale, hipStream_t s);

}  // namespace vsa
