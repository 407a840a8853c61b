// Sparse fine forward, dQ and dK/dV for fp32 inputs (the reference's GPU path
// accepts fp32: triton_impl.py:375-376).  gfx950 has no fast fp32 matrix
// instruction (the fp32 MFMA runs at 1/16 of bf16), so these kernels keep
// every product in fp32 on the vector ALU and are written for exactness of
// the fp32 arithmetic rather than speed: outputs, LSE (base 2), the fused
// combine, the pooled-gradient folds and the padding masks follow the bf16 /
// fp16 kernels of fine_fwd.hip and fine_bwd.hip with T = fp32 (no rounding).
//
// Layout: a workgroup owns 64 rows (queries, or keys for dK/dV), four lanes
// per row, each lane holding D/4 consecutive dims; a dot product is a lane
// partial plus two quad exchanges.  The other operand streams through LDS in
// chunks of 32 rows, single-buffered.
#include "fine_f32.h"
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

namespace {

constexpr int kRows = 64;   // rows per workgroup
constexpr int kChunk = 32;  // streamed rows per LDS chunk

__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

// Copy `rows` rows of D floats (row stride D) into LDS; rows past `valid`
// are zero (they are never used for a valid result, only kept finite).
template <int D>
__device__ __forceinline__ void stage_rows_f32(float* dst, const float* __restrict__ src,
                                               int rows, int valid) {
  constexpr int V4 = D / 4;  // float4 per row
  for (int x = threadIdx.x; x < rows * V4; x += 256) {
    const int r = x / V4, c = x % V4;
    f32x4 val = {0.f, 0.f, 0.f, 0.f};
    if (r < valid) val = *reinterpret_cast<const f32x4*>(src + (int64_t)r * D + 4 * c);
    *reinterpret_cast<f32x4*>(dst + r * D + 4 * c) = val;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward: out = softmax(q k^T scale) v over the selected blocks, LSE base 2,
// combine `out_c * gate` in the epilogue.  grid: bh * Sq / 64.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(256) void sparse_fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
    float* __restrict__ out, float* __restrict__ lse, const float* __restrict__ outc,
    const float* __restrict__ gate, int gate_mode, int gate_heads, int tiles_per_head, int sq,
    int skv, int qb, int kb, int topk, float c2) {
  constexpr int DS = D / 4;
  __shared__ __attribute__((aligned(16))) float ks[kChunk * D];
  __shared__ __attribute__((aligned(16))) float vs[kChunk * D];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int q0 = (blockIdx.x % tiles_per_head) * kRows;
  const int qblk = q0 / BE;
  const int row = threadIdx.x >> 2, sl = threadIdx.x & 3;
  const int myq = q0 + row;
  const int64_t tok = b * sq + myq;
  float qv[DS], o[DS];
#pragma unroll
  for (int i = 0; i < DS; i += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(q + tok * D + sl * DS + i);
    qv[i] = x[0]; qv[i + 1] = x[1]; qv[i + 2] = x[2]; qv[i + 3] = x[3];
  }
#pragma unroll
  for (int i = 0; i < DS; ++i) o[i] = 0.f;
  float m = -INFINITY, l = 0.f;
  const int32_t* sel = selected + (b * qb + qblk) * topk;
  const float* kbase = k + b * (int64_t)skv * D;
  const float* vbase = v + b * (int64_t)skv * D;
  for (int s = 0; s < topk; ++s) {
    const int kv = sel[s];
    if (kv < 0 || kv >= kb) continue;
    const int nvb = clamp_valid(kv_vbs[kv], BE);
    for (int c0 = 0; c0 < nvb; c0 += kChunk) {
      const int nk = min(kChunk, nvb - c0);
      __syncthreads();
      stage_rows_f32<D>(ks, kbase + ((int64_t)kv * BE + c0) * D, kChunk, nk);
      stage_rows_f32<D>(vs, vbase + ((int64_t)kv * BE + c0) * D, kChunk, nk);
      __syncthreads();
      // all kChunk scores are formed (staged rows past nk are zero) so the
      // array stays in registers; keys past nk are masked to -inf
      float sv[kChunk];
      float cmax = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < kChunk; ++kk) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < DS; ++i) d = fmaf(qv[i], ks[kk * D + sl * DS + i], d);
        sv[kk] = kk < nk ? quad_sum(d) * c2 : -INFINITY;
        cmax = fmaxf(cmax, sv[kk]);
      }
      const float mnew = fmaxf(m, cmax);
      const float alpha = exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < DS; ++i) o[i] *= alpha;
      m = mnew;
#pragma unroll
      for (int kk = 0; kk < kChunk; ++kk) {
        const float p = kk < nk ? exp2f(sv[kk] - m) : 0.f;
        l += p;
#pragma unroll
        for (int i = 0; i < DS; ++i) o[i] = fmaf(p, vs[kk * D + sl * DS + i], o[i]);
      }
    }
  }
  // epilogue: normalise, fused combine, LSE
  const float inv = 1.0f / l;
  if (lse != nullptr && sl == 0) lse[tok] = m + log2f(l);
  const float* ocrow = outc ? outc + (b * qb + qblk) * D + sl * DS : nullptr;
  const float* grow = nullptr;
  float gtok = 1.f;
  if (outc && gate_mode == 1) grow = gate + tok * D + sl * DS;
  if (outc && gate_mode == 2) gtok = gate[tok];
  if (outc && gate_mode == 3)
    grow = gate + (((b / gate_heads) * sq + myq) * gate_heads + b % gate_heads) * D + sl * DS;
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    float val = o[i] * inv;
    if (ocrow) val = fmaf(ocrow[i], grow ? grow[i] : gtok, val);
    out[tok * D + sl * DS + i] = val;
  }
}

// ---------------------------------------------------------------------------
// dQ (query-owned): P = exp2(S c2 - lse), dS = P (dP - delta), dQ = scale dS K,
// plus the pooled gradient d_q_c / count on the block's valid rows.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(256) void sparse_dq_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, const int32_t* __restrict__ selected,
    const int32_t* __restrict__ kv_vbs, float* __restrict__ dq, const float* __restrict__ dqc,
    const int32_t* __restrict__ q_vbs, int tiles_per_head, int sq, int skv, int qb, int kb,
    int topk, float c2, float scale) {
  constexpr int DS = D / 4;
  __shared__ __attribute__((aligned(16))) float ks[kChunk * D];
  __shared__ __attribute__((aligned(16))) float vs[kChunk * D];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int q0 = (blockIdx.x % tiles_per_head) * kRows;
  const int qblk = q0 / BE;
  const int row = threadIdx.x >> 2, sl = threadIdx.x & 3;
  const int myq = q0 + row;
  const int64_t tok = b * sq + myq;
  float qv[DS], dov[DS], acc[DS];
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    qv[i] = q[tok * D + sl * DS + i];
    dov[i] = dout[tok * D + sl * DS + i];
    acc[i] = 0.f;
  }
  const float my_lse = lse[tok], my_delta = delta[tok];
  const int32_t* sel = selected + (b * qb + qblk) * topk;
  const float* kbase = k + b * (int64_t)skv * D;
  const float* vbase = v + b * (int64_t)skv * D;
  for (int s = 0; s < topk; ++s) {
    const int kv = sel[s];
    if (kv < 0 || kv >= kb) continue;
    const int nvb = clamp_valid(kv_vbs[kv], BE);
    for (int c0 = 0; c0 < nvb; c0 += kChunk) {
      const int nk = min(kChunk, nvb - c0);
      __syncthreads();
      stage_rows_f32<D>(ks, kbase + ((int64_t)kv * BE + c0) * D, kChunk, nk);
      stage_rows_f32<D>(vs, vbase + ((int64_t)kv * BE + c0) * D, kChunk, nk);
      __syncthreads();
      for (int kk = 0; kk < nk; ++kk) {
        float ds = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < DS; ++i) {
          ds = fmaf(qv[i], ks[kk * D + sl * DS + i], ds);
          dp = fmaf(dov[i], vs[kk * D + sl * DS + i], dp);
        }
        const float p = exp2f(fmaf(quad_sum(ds), c2, -my_lse));
        const float dsv = p * (quad_sum(dp) - my_delta);
#pragma unroll
        for (int i = 0; i < DS; ++i) acc[i] = fmaf(dsv, ks[kk * D + sl * DS + i], acc[i]);
      }
    }
  }
  float cdiv = 1.f;
  bool cvalid = false;
  if (dqc) {
    const int32_t cnt = q_vbs[qblk];
    cvalid = myq - qblk * BE < clamp_valid(cnt, BE);
    cdiv = (float)(cnt > 1 ? cnt : 1);
  }
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    const float cv = cvalid ? dqc[(b * qb + qblk) * D + sl * DS + i] / cdiv : 0.f;
    dq[tok * D + sl * DS + i] = acc[i] * scale + cv;
  }
}

// ---------------------------------------------------------------------------
// dK / dV (key-owned over the CSR in-edges of the key block): for every row of
// every in-edge query block, dV += P dO, dK += dS Q; dK *= scale; pooled
// gradients folded on valid keys; padding keys get zero.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(256) void sparse_dkdv_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ inverse,
    const int32_t* __restrict__ kv_vbs, float* __restrict__ dk, float* __restrict__ dv,
    const float* __restrict__ dkc, const float* __restrict__ dvc, int tiles_per_head, int sq,
    int skv, int qb, int kb, int topk, float c2, float scale) {
  constexpr int DS = D / 4;
  __shared__ __attribute__((aligned(16))) float qs[kChunk * D];
  __shared__ __attribute__((aligned(16))) float ds_[kChunk * D];
  __shared__ float ls[kChunk], es[kChunk];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int k0 = (blockIdx.x % tiles_per_head) * kRows;
  const int kvblk = k0 / BE;
  const int row = threadIdx.x >> 2, sl = threadIdx.x & 3;
  const int mykey = k0 + row;
  const int64_t ktok = b * skv + mykey;
  const bool key_valid = mykey - kvblk * BE < clamp_valid(kv_vbs[kvblk], BE);
  float kvv[DS], vvv[DS], ak[DS], av[DS];
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    kvv[i] = k[ktok * D + sl * DS + i];
    vvv[i] = v[ktok * D + sl * DS + i];
    ak[i] = av[i] = 0.f;
  }
  const int64_t meta = b * kb + kvblk;
  const int nedge = counts[meta];
  const int32_t* seg = inverse + b * (int64_t)qb * topk + offsets[meta];
  const float* qbase = q + b * (int64_t)sq * D;
  const float* dbase = dout + b * (int64_t)sq * D;
  for (int e = 0; e < nedge; ++e) {
    const int qblock = seg[e];
    for (int c0 = 0; c0 < BE; c0 += kChunk) {
      const int qrow0 = qblock * BE + c0;
      __syncthreads();
      stage_rows_f32<D>(qs, qbase + (int64_t)qrow0 * D, kChunk, kChunk);
      stage_rows_f32<D>(ds_, dbase + (int64_t)qrow0 * D, kChunk, kChunk);
      if (threadIdx.x < kChunk) {
        ls[threadIdx.x] = lse[b * sq + qrow0 + threadIdx.x];
        es[threadIdx.x] = delta[b * sq + qrow0 + threadIdx.x];
      }
      __syncthreads();
      for (int qq = 0; qq < kChunk; ++qq) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < DS; ++i) {
          s = fmaf(qs[qq * D + sl * DS + i], kvv[i], s);
          dp = fmaf(ds_[qq * D + sl * DS + i], vvv[i], dp);
        }
        const float p = exp2f(fmaf(quad_sum(s), c2, -ls[qq]));
        const float dsv = p * (quad_sum(dp) - es[qq]);
#pragma unroll
        for (int i = 0; i < DS; ++i) {
          av[i] = fmaf(p, ds_[qq * D + sl * DS + i], av[i]);
          ak[i] = fmaf(dsv, qs[qq * D + sl * DS + i], ak[i]);
        }
      }
    }
  }
  const int32_t cnt = kv_vbs[kvblk];
  const float cdiv = (float)(cnt > 1 ? cnt : 1);
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    const int d = sl * DS + i;
    const float ck = (key_valid && dkc) ? dkc[meta * D + d] / cdiv : 0.f;
    const float cv = (key_valid && dvc) ? dvc[meta * D + d] / cdiv : 0.f;
    dk[ktok * D + d] = (key_valid ? ak[i] * scale : 0.f) + ck;
    dv[ktok * D + d] = (key_valid ? av[i] : 0.f) + cv;
  }
}

// ---------------------------------------------------------------------------
// Host launchers (the C ABI in fine_fwd.hip / fine_bwd.hip dispatches fp32
// here).  Shapes: head_dim 64 / 128 / 256, block volume 64 / 128 / 256 (the
// Python layer pads other shapes onto these, as for bf16).
// ---------------------------------------------------------------------------
// every kernel shape has 64 | block volume, so a workgroup's 64 rows lie in
// one block and sequence lengths (multiples of the volume) split evenly
static bool f32_shape(int D, int be) {
  return (D == 64 || D == 128 || D == 256) && (be == 64 || be == 128 || be == 256);
}

#define VSA_F32_SHAPES(X) \
  X(64, 64) X(64, 128) X(64, 256) X(128, 64) X(128, 128) X(128, 256) X(256, 64) X(256, 128) X(256, 256)

int sparse_fwd_f32(const void* q, const void* k, const void* v, const int32_t* selected,
                   const int32_t* kv_vbs, void* out, float* lse, const void* out_c,
                   const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq,
                   int64_t skv, int D, int be, int topk, float scale, hipStream_t s) {
  if (!f32_shape(D, be)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * (sq / kRows);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int tph = (int)(sq / kRows);
  const float c2 = scale * kLog2e;
#define VSA_F(DD, BB)                                                                        \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_fwd_f32_kernel<DD, BB>), dim3((unsigned)tiles), dim3(256), 0, \
                       s, (const float*)q, (const float*)k, (const float*)v, selected, kv_vbs, \
                       (float*)out, lse, (const float*)out_c, (const float*)gate, gate_mode,  \
                       gate_heads, tph, (int)sq, (int)skv, (int)(sq / BB), (int)(skv / BB),  \
                       topk, c2);                                                            \
    return vsa_check_launch();                                                               \
  }
  VSA_F32_SHAPES(VSA_F)
#undef VSA_F
  return VSA_ERR_UNSUPPORTED;
}

int sparse_dq_f32(const void* q, const void* k, const void* v, const void* dout,
                  const float* lse, const float* delta, const int32_t* selected,
                  const int32_t* kv_vbs, void* dq, const void* dqc, const int32_t* q_vbs,
                  int64_t bh, int64_t sq, int64_t skv, int D, int be, int topk, float scale,
                  hipStream_t s) {
  if (!f32_shape(D, be)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * (sq / kRows);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int tph = (int)(sq / kRows);
  const float c2 = scale * kLog2e;
#define VSA_F(DD, BB)                                                                        \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_dq_f32_kernel<DD, BB>), dim3((unsigned)tiles), dim3(256), 0,  \
                       s, (const float*)q, (const float*)k, (const float*)v,                 \
                       (const float*)dout, lse, delta, selected, kv_vbs, (float*)dq,         \
                       (const float*)dqc, q_vbs, tph, (int)sq, (int)skv, (int)(sq / BB),     \
                       (int)(skv / BB), topk, c2, scale);                                    \
    return vsa_check_launch();                                                               \
  }
  VSA_F32_SHAPES(VSA_F)
#undef VSA_F
  return VSA_ERR_UNSUPPORTED;
}

int sparse_dkdv_f32(const void* q, const void* k, const void* v, const void* dout,
                    const float* lse, const float* delta, const int32_t* counts,
                    const int32_t* offsets, const int32_t* inverse, const int32_t* kv_vbs,
                    void* dk, void* dv, const void* dkc, const void* dvc, int64_t bh, int64_t sq,
                    int64_t skv, int D, int be, int topk, float scale, hipStream_t s) {
  if (!f32_shape(D, be)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * (skv / kRows);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int tph = (int)(skv / kRows);
  const float c2 = scale * kLog2e;
#define VSA_F(DD, BB)                                                                        \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_dkdv_f32_kernel<DD, BB>), dim3((unsigned)tiles), dim3(256), 0, \
                       s, (const float*)q, (const float*)k, (const float*)v,                 \
                       (const float*)dout, lse, delta, counts, offsets, inverse, kv_vbs,     \
                       (float*)dk, (float*)dv, (const float*)dkc, (const float*)dvc, tph,    \
                       (int)sq, (int)skv, (int)(sq / BB), (int)(skv / BB), topk, c2, scale); \
    return vsa_check_launch();                                                               \
  }
  VSA_F32_SHAPES(VSA_F)
#undef VSA_F
  return VSA_ERR_UNSUPPORTED;
}

}  // namespace vsa
