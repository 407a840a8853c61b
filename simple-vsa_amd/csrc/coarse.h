// Host launchers of the MFMA coarse-attention kernels and the radix Top-K
// (coarse.hip); the C ABI entry points in common.hip dispatch to them for the
// shapes they cover.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vsa {

// bf16 / fp16 with head_dim 64 or 128
bool coarse_mfma_supported(int D, int dtype);

int coarse_fwd_mfma(const void* qc, const void* kc, const void* vc, float* scores, float* probs,
                    void* outc, int64_t bh, int qb, int kb, int D, float scale, int dtype,
                    hipStream_t s);

int topk_radix(const float* scores, int32_t* selected, int64_t rows, int kb, int topk,
               hipStream_t s);

int coarse_bwd_mfma(const void* qc, const void* kc, const void* vc, const float* probs,
                    const void* d_outc, float* ds, void* d_qc, void* d_kc, void* d_vc,
                    int64_t bh, int qb, int kb, int D, float scale, int dtype, hipStream_t s);

}  // namespace vsa
