// Sparse fine forward, dQ and dK/dV for fp32 inputs (the reference's GPU path
// accepts fp32: triton_impl.py:375-376).  Every product and sum stays fp32
// (no operand rounding): outputs, LSE (base 2), the fused combine, the
// pooled-gradient folds and the padding masks follow the bf16 / fp16 kernels
// of fine_fwd.hip and fine_bwd.hip with T = fp32.
//
// The products run on v_mfma_f32_32x32x2_f32 (the fp32 matrix core: 1/16 of
// the bf16 rate, twice the unpacked fp32 VALU rate).  Its operands are one
// float per lane:
//   A (32 x 2): lane (r, h) = row r, k = h;  B (2 x 32): lane (c, h) = column c, k = h;
//   C (32 x 32): element i of lane (c, h) = row 8(i/4) + 4h + i%4, column c.
// A dot product over D dims is D/2 MFMAs; k-step t pairs dim t (h = 0) with
// dim D/2 + t (h = 1), so each lane reads its row contiguously.  The C tile of
// one product is the B operand of the next with no data movement (element t of
// the accumulator is the k = h value of k-step t, rows 8(t/4) + 4h + t%4), and
// the other operand is read in that row order.
//
// Work decomposition as in the bf16 kernels: 32 rows (queries, or keys for
// dK/dV) per wave, two waves per workgroup; the streamed operand goes through
// LDS in 32-row chunks (rows padded by 4 floats so that the row reads of 32
// lanes hit distinct banks).  dK/dV at head_dim 256 (whose fragments and
// accumulators would exceed a wave's registers) keeps a vector-ALU kernel.
#include "fine_f32.h"
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

namespace {

constexpr int kRows = 64;   // rows per workgroup
constexpr int kChunk = 32;  // streamed rows per LDS chunk

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

// Copy 32 rows of D floats (global row stride D) into LDS with row stride LD;
// rows past `valid` are zero (never used for a valid result, only kept finite).
template <int D, int LD, int NT>
__device__ __forceinline__ void stage32(float* dst, const float* __restrict__ src, int valid) {
  constexpr int V4 = D / 4;  // float4 per row
#pragma unroll 4
  for (int x = threadIdx.x; x < kChunk * V4; x += NT) {
    const int r = x / V4, c = x % V4;
    f32x4 val = {0.f, 0.f, 0.f, 0.f};
    if (r < valid) val = *reinterpret_cast<const f32x4*>(src + (int64_t)r * D + 4 * c);
    *reinterpret_cast<f32x4*>(dst + r * LD + 4 * c) = val;
  }
}

// stage32 split in two: load() issues this thread's loads of a 32-row tile
// into registers, store() writes them to LDS, so the next chunk's loads are in
// flight while the current one is multiplied (for kernels at one wave per
// SIMD, where no other wave of the SIMD hides the copy).
template <int D, int LD, int NT>
struct Stage32 {
  static constexpr int V4 = D / 4;
  static constexpr int N = kChunk * V4 / NT;  // float4 per thread
  static_assert(kChunk * V4 % NT == 0, "tile must split evenly over the workgroup");
  f32x4 buf[N];
  __device__ __forceinline__ void load(const float* __restrict__ src, int valid) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int x = (int)threadIdx.x + i * NT, r = x / V4, c = x % V4;
      buf[i] = r < valid ? *reinterpret_cast<const f32x4*>(src + (int64_t)r * D + 4 * c)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __device__ __forceinline__ void store(float* dst) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int x = (int)threadIdx.x + i * NT, r = x / V4, c = x % V4;
      *reinterpret_cast<f32x4*>(dst + r * LD + 4 * c) = buf[i];
    }
  }
};

// Copy `rows` rows of D floats (row stride D) into LDS (row stride D) with 256
// threads; rows past `valid` are zero.
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

// this lane's row fragment: x[row][h * D/2 + t], t < D/2
template <int D>
__device__ __forceinline__ void load_frag(float (&f)[D / 2], const float* __restrict__ row, int h) {
#pragma unroll
  for (int t = 0; t < D / 2; t += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + h * (D / 2) + t);
    f[t] = x[0]; f[t + 1] = x[1]; f[t + 2] = x[2]; f[t + 3] = x[3];
  }
}

// acc += rows(lds, 32 x D, stride LD) . frag^T: A = LDS row r (lane r), B = frag
template <int D, int LD>
__device__ __forceinline__ void mma_rows(f32x16& acc, const float* lds, const float (&f)[D / 2],
                                         int r, int h) {
  const float* row = lds + r * LD + h * (D / 2);
#pragma unroll
  for (int t = 0; t < D / 2; t += 4) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(row + t);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = mfma_f32(a[e], f[t + e], acc);
  }
}

// acc[mt] += (LDS rows)^T . B, B = the C tile `bop` (rows 8(t/4) + 4h + t%4 of
// the LDS tile paired with k-step t): A = LDS[row(t, h)][32 mt + r]
template <int D, int LD>
__device__ __forceinline__ void mma_cols(f32x16 (&acc)[D / 32], const float* lds, const f32x16& bop,
                                         int r, int h) {
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const float* row = lds + (8 * (t >> 2) + 4 * h + (t & 3)) * LD + r;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt) acc[mt] = mfma_f32(row[32 * mt], bop[t], acc[mt]);
  }
}

}  // namespace

template <int D>
struct F32Cfg {
  static constexpr int LD = D + 4;                 // LDS row stride (floats)
  static constexpr int NT = 128;                   // two waves
  // waves per SIMD the registers are sized for: forward and dQ hold two D/2
  // fragments or accumulators of D/32 tiles, dK/dV four
  static constexpr int WPE_FWD = D <= 128 ? 2 : 1;
  static constexpr int WPE_DQ = D <= 64 ? 2 : 1;
  static constexpr int WPE_KV = D <= 64 ? 2 : 1;
};

// ---------------------------------------------------------------------------
// Forward: out = softmax(q k^T scale) v over the selected blocks, LSE base 2,
// combine `out_c * gate` in the epilogue.  Per wave and 32-key chunk:
//   S^T = K Q^T (D/2 MFMAs), online softmax per lane-query (lane halves hold
//   16 keys each, joined by a permlane swap), O^T += V^T P^T (16 D/32 MFMAs).
// grid: bh * Sq / 64.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(F32Cfg<D>::WPE_FWD))) void
sparse_fwd_f32m_kernel(const float* __restrict__ q, const float* __restrict__ k,
                       const float* __restrict__ v, const int32_t* __restrict__ selected,
                       const int32_t* __restrict__ kv_vbs, float* __restrict__ out,
                       float* __restrict__ fine, float* __restrict__ lse,
                       const float* __restrict__ outc, const float* __restrict__ gate,
                       int gate_mode, int gate_heads, int tiles_per_head, int sq, int skv, int qb,
                       int kb, int topk, float c2) {
  using C = F32Cfg<D>;
  constexpr int LD = C::LD;
  __shared__ __attribute__((aligned(16))) float ks[kChunk * LD];
  __shared__ __attribute__((aligned(16))) float vs[kChunk * LD];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int q0 = (blockIdx.x % tiles_per_head) * kRows;
  const int qblk = q0 / BE;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int myq = q0 + wave * 32 + r;
  const int64_t tok = b * sq + myq;
  float qf[D / 2];
  load_frag<D>(qf, q + tok * D, h);
  f32x16 o[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) o[mt] = f32x16{};
  float m = -INFINITY, l = 0.f;  // running max (log2 units), this half's partial sum
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
      stage32<D, LD, C::NT>(ks, kbase + ((int64_t)kv * BE + c0) * D, nk);
      stage32<D, LD, C::NT>(vs, vbase + ((int64_t)kv * BE + c0) * D, nk);
      __syncthreads();
      f32x16 sacc = f32x16{};
      mma_rows<D, LD>(sacc, ks, qf, r, h);
      float cmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = 8 * (i >> 2) + 4 * h + (i & 3);
        sacc[i] = key < nk ? sacc[i] * c2 : -INFINITY;
        cmax = fmaxf(cmax, sacc[i]);
      }
      const float mnew = fmaxf(m, pair_max32(cmax));
      const float alpha = exp2f(m - mnew);
      m = mnew;
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sacc[i] = exp2f(sacc[i] - m);
        psum += sacc[i];
      }
      l = l * alpha + psum;
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) o[mt] *= alpha;
      mma_cols<D, LD>(o, vs, sacc, r, h);
    }
  }
  // epilogue: normalise, fused combine, LSE
  const float ltot = pair_sum32(l);
  const float inv = 1.0f / ltot;
  if (lse != nullptr && h == 0) lse[tok] = m + log2f(ltot);
  const float* ocrow = outc ? outc + (b * qb + qblk) * D : nullptr;
  const float* grow = nullptr;
  float gtok = 1.f;
  if (outc && gate_mode == 1) grow = gate + tok * D;
  if (outc && gate_mode == 2) gtok = gate[tok];
  if (outc && gate_mode == 3)
    grow = gate + (((b / gate_heads) * sq + myq) * gate_heads + b % gate_heads) * D;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      f32x4 val;
#pragma unroll
      for (int e = 0; e < 4; ++e) val[e] = o[mt][4 * g + e] * inv;
      if (ocrow && fine) *reinterpret_cast<f32x4*>(fine + tok * D + d0) = val;
      if (ocrow) {
        const f32x4 oc = *reinterpret_cast<const f32x4*>(ocrow + d0);
        const f32x4 gv = grow ? *reinterpret_cast<const f32x4*>(grow + d0)
                              : f32x4{gtok, gtok, gtok, gtok};
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = fmaf(oc[e], gv[e], val[e]);
      }
      *reinterpret_cast<f32x4*>(out + tok * D + d0) = val;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ (query-owned): per wave and 32-key chunk S^T = K Q^T, dP^T = V dO^T,
// P^T = exp2(S^T c2 - lse), dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T;
// dQ = scale dQ plus the pooled gradient d_q_c / count on the block's valid
// rows.  grid: bh * Sq / 64.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(F32Cfg<D>::WPE_DQ))) void
sparse_dq_f32m_kernel(const float* __restrict__ q, const float* __restrict__ k,
                      const float* __restrict__ v, const float* __restrict__ dout,
                      const float* __restrict__ lse, const float* __restrict__ delta,
                      const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
                      float* __restrict__ dq, const float* __restrict__ dqc,
                      const int32_t* __restrict__ q_vbs, int tiles_per_head, int sq, int skv,
                      int qb, int kb, int topk, float c2, float scale) {
  using C = F32Cfg<D>;
  constexpr int LD = C::LD;
  __shared__ __attribute__((aligned(16))) float ks[kChunk * LD];
  __shared__ __attribute__((aligned(16))) float vs[kChunk * LD];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int q0 = (blockIdx.x % tiles_per_head) * kRows;
  const int qblk = q0 / BE;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int myq = q0 + wave * 32 + r;
  const int64_t tok = b * sq + myq;
  float qf[D / 2], df[D / 2];
  load_frag<D>(qf, q + tok * D, h);
  load_frag<D>(df, dout + tok * D, h);
  const float my_lse = lse[tok], my_delta = delta[tok];
  f32x16 acc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) acc[mt] = f32x16{};
  const int32_t* sel = selected + (b * qb + qblk) * topk;
  const float* kbase = k + b * (int64_t)skv * D;
  const float* vbase = v + b * (int64_t)skv * D;
  // chunk cursor over the route: slot s, key block kv with nvb valid keys, first key c0
  auto advance = [&](int& s, int& kv, int& nvb, int& c0) {
    c0 += kChunk;
    while (c0 >= nvb) {
      if (++s >= topk) return false;
      kv = sel[s];
      nvb = (kv >= 0 && kv < kb) ? clamp_valid(kv_vbs[kv], BE) : 0;
      c0 = 0;
    }
    return true;
  };
  // head_dim <= 128: the next chunk's loads stay in flight under this chunk's
  // products (64 more registers); head_dim 256 has no registers to spare
  constexpr bool kPrefetch = D <= 128;
  Stage32<D, LD, C::NT> kst, vst;
  auto load_chunk = [&](int kv_, int nvb_, int c0_) {
    if constexpr (kPrefetch) {
      kst.load(kbase + ((int64_t)kv_ * BE + c0_) * D, min(kChunk, nvb_ - c0_));
      vst.load(vbase + ((int64_t)kv_ * BE + c0_) * D, min(kChunk, nvb_ - c0_));
    }
  };
  int s = -1, kv = 0, nvb = 0, c0 = 0;
  bool have = advance(s, kv, nvb, c0);
  if (have) load_chunk(kv, nvb, c0);
  while (have) {
    const int nk = min(kChunk, nvb - c0);
    __syncthreads();
    if constexpr (kPrefetch) {
      kst.store(ks);
      vst.store(vs);
    } else {
      stage32<D, LD, C::NT>(ks, kbase + ((int64_t)kv * BE + c0) * D, nk);
      stage32<D, LD, C::NT>(vs, vbase + ((int64_t)kv * BE + c0) * D, nk);
    }
    const bool have2 = advance(s, kv, nvb, c0);
    if (have2) load_chunk(kv, nvb, c0);
    __syncthreads();
    f32x16 sacc = f32x16{}, pacc = f32x16{};
    mma_rows<D, LD>(sacc, ks, qf, r, h);
    mma_rows<D, LD>(pacc, vs, df, r, h);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = 8 * (i >> 2) + 4 * h + (i & 3);
      const float p = key < nk ? exp2f(fmaf(sacc[i], c2, -my_lse)) : 0.f;
      sacc[i] = p * (pacc[i] - my_delta);
    }
    mma_cols<D, LD>(acc, ks, sacc, r, h);
    have = have2;
  }
  float cdiv = 1.f;
  bool cvalid = false;
  if (dqc) {
    const int32_t cnt = q_vbs[qblk];
    cvalid = myq - qblk * BE < clamp_valid(cnt, BE);
    cdiv = (float)(cnt > 1 ? cnt : 1);
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      f32x4 cv = {0.f, 0.f, 0.f, 0.f};
      if (cvalid) cv = *reinterpret_cast<const f32x4*>(dqc + (b * qb + qblk) * D + d0);
      f32x4 val;
#pragma unroll
      for (int e = 0; e < 4; ++e) val[e] = acc[mt][4 * g + e] * scale + cv[e] / cdiv;
      *reinterpret_cast<f32x4*>(dq + tok * D + d0) = val;
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV (key-owned over the CSR in-edges of the key block), head_dim 64 /
// 128: per wave (32 keys) and 32-query item S = Q K^T, dP = dO V^T,
// P = exp2(S c2 - lse), dS = P (dP - delta), dV^T += dO^T P, dK^T += Q^T dS;
// dK *= scale; pooled gradients folded on valid keys; padding keys get zero.
// grid: bh * Skv / 64.
// ---------------------------------------------------------------------------
template <int D, int BE>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(F32Cfg<D>::WPE_KV))) void
sparse_dkdv_f32m_kernel(const float* __restrict__ q, const float* __restrict__ k,
                        const float* __restrict__ v, const float* __restrict__ dout,
                        const float* __restrict__ lse, const float* __restrict__ delta,
                        const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                        const int32_t* __restrict__ inverse, const int32_t* __restrict__ kv_vbs,
                        float* __restrict__ dk, float* __restrict__ dv,
                        const float* __restrict__ dkc, const float* __restrict__ dvc,
                        int tiles_per_head, int sq, int skv, int qb, int kb, int topk, float c2,
                        float scale) {
  using C = F32Cfg<D>;
  constexpr int LD = C::LD;
  __shared__ __attribute__((aligned(16))) float qs[kChunk * LD];
  __shared__ __attribute__((aligned(16))) float os[kChunk * LD];
  __shared__ __attribute__((aligned(16))) float ls[kChunk], es[kChunk];
  const int64_t b = blockIdx.x / tiles_per_head;
  const int k0 = (blockIdx.x % tiles_per_head) * kRows;
  const int kvblk = k0 / BE;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int mykey = k0 + wave * 32 + r;
  const int64_t ktok = b * skv + mykey;
  const bool key_valid = mykey - kvblk * BE < clamp_valid(kv_vbs[kvblk], BE);
  float kf[D / 2], vf[D / 2];
  load_frag<D>(kf, k + ktok * D, h);
  load_frag<D>(vf, v + ktok * D, h);
  f32x16 dka[D / 32], dva[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) dka[mt] = dva[mt] = f32x16{};
  const int64_t meta = b * kb + kvblk;
  const int nedge = counts[meta];
  const int32_t* seg = inverse + b * (int64_t)qb * topk + offsets[meta];
  const float* qbase = q + b * (int64_t)sq * D;
  const float* dbase = dout + b * (int64_t)sq * D;
  // item it: 32 queries (rows (it % (BE/32)) * 32 ..) of in-edge query block it / (BE/32);
  // head_dim 128: the next item's Q / dO / statistics loads stay in flight
  // under this item's products (64 more registers; 64 has no headroom at two
  // waves per SIMD)
  constexpr int SUBS = BE / kChunk;
  constexpr bool kPrefetch = D == 128;
  const int items = nedge * SUBS;
  Stage32<D, LD, C::NT> qst, ost;
  float stv = 0.f;  // lse (threads < 32) or delta (32 .. 63) of the staged item
  auto load_item = [&](int it) {
    const int qrow0 = seg[it / SUBS] * BE + (it % SUBS) * kChunk;
    qst.load(qbase + (int64_t)qrow0 * D, kChunk);
    ost.load(dbase + (int64_t)qrow0 * D, kChunk);
    if (threadIdx.x < 2 * kChunk)
      stv = threadIdx.x < kChunk ? lse[b * sq + qrow0 + threadIdx.x]
                                 : delta[b * sq + qrow0 + threadIdx.x - kChunk];
  };
  if (kPrefetch && items > 0) load_item(0);
  for (int it = 0; it < items; ++it) {
    {
      __syncthreads();
      if (!kPrefetch) load_item(it);
      qst.store(qs);
      ost.store(os);
      if (threadIdx.x < kChunk) ls[threadIdx.x] = stv;
      else if (threadIdx.x < 2 * kChunk) es[threadIdx.x - kChunk] = stv;
      if (kPrefetch && it + 1 < items) load_item(it + 1);
      __syncthreads();
      f32x16 sacc = f32x16{}, pacc = f32x16{};
      mma_rows<D, LD>(sacc, qs, kf, r, h);   // S  (queries x keys), lane column = key r
      mma_rows<D, LD>(pacc, os, vf, r, h);   // dP
      f32x16 ds;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(ls + 8 * g + 4 * h);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(es + 8 * g + 4 * h);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 4 * g + j;
          sacc[i] = exp2f(fmaf(sacc[i], c2, -l4[j]));
          ds[i] = sacc[i] * (pacc[i] - d4[j]);
        }
      }
      mma_cols<D, LD>(dva, os, sacc, r, h);  // dV^T += dO^T P
      mma_cols<D, LD>(dka, qs, ds, r, h);    // dK^T += Q^T dS
    }
  }
  const int32_t cnt = kv_vbs[kvblk];
  const float cdiv = (float)(cnt > 1 ? cnt : 1);
  // pooled-gradient rows loaded before the first store (a load issued after a
  // store also waits for that store)
  f32x4 ckr[D / 32][4], cvr[D / 32][4];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ckr[mt][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      cvr[mt][g] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (key_valid && dkc) {
        const int d0 = 32 * mt + 8 * g + 4 * h;
        ckr[mt][g] = *reinterpret_cast<const f32x4*>(dkc + meta * D + d0);
        cvr[mt][g] = *reinterpret_cast<const f32x4*>(dvc + meta * D + d0);
      }
    }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      const f32x4 ck = ckr[mt][g], cv = cvr[mt][g];
      f32x4 kk, vv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kk[e] = (key_valid ? dka[mt][4 * g + e] * scale : 0.f) + ck[e] / cdiv;
        vv[e] = (key_valid ? dva[mt][4 * g + e] : 0.f) + cv[e] / cdiv;
      }
      *reinterpret_cast<f32x4*>(dk + ktok * D + d0) = kk;
      *reinterpret_cast<f32x4*>(dv + ktok * D + d0) = vv;
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV at head_dim 256 on the vector ALU (key-owned over the CSR in-edges
// of the key block): four lanes per key, each holding 64 dims; for every row of
// every in-edge query block dV += P dO, dK += dS Q; dK *= scale; pooled
// gradients folded on valid keys; padding keys get zero.  grid: bh * Skv / 64.
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
                   const int32_t* kv_vbs, void* out, void* fine, float* lse, const void* out_c,
                   const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq,
                   int64_t skv, int D, int be, int topk, float scale, hipStream_t s) {
  if (!f32_shape(D, be)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * (sq / kRows);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int tph = (int)(sq / kRows);
  const float c2 = scale * kLog2e;
#define VSA_F(DD, BB)                                                                        \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_fwd_f32m_kernel<DD, BB>), dim3((unsigned)tiles), dim3(128), 0, \
                       s, (const float*)q, (const float*)k, (const float*)v, selected, kv_vbs, \
                       (float*)out, (float*)fine, lse, (const float*)out_c,                \
                       (const float*)gate, gate_mode, gate_heads, tph, (int)sq, (int)skv,     \
                       (int)(sq / BB), (int)(skv / BB), topk, c2);                           \
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
    hipLaunchKernelGGL((sparse_dq_f32m_kernel<DD, BB>), dim3((unsigned)tiles), dim3(128), 0, \
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
  // head_dim 64 / 128 on the matrix core, 256 on the vector ALU
#define VSA_F(DD, BB)                                                                        \
  if constexpr (DD <= 128) {                                                                 \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_dkdv_f32m_kernel<DD, BB>), dim3((unsigned)tiles), dim3(128), 0, \
                       s, (const float*)q, (const float*)k, (const float*)v,                 \
                       (const float*)dout, lse, delta, counts, offsets, inverse, kv_vbs,     \
                       (float*)dk, (float*)dv, (const float*)dkc, (const float*)dvc, tph,    \
                       (int)sq, (int)skv, (int)(sq / BB), (int)(skv / BB), topk, c2, scale); \
    return vsa_check_launch();                                                               \
  }                                                                                          \
  } else {                                                                                   \
  if (D == DD && be == BB) {                                                                 \
    hipLaunchKernelGGL((sparse_dkdv_f32_kernel<DD, BB>), dim3((unsigned)tiles), dim3(256), 0, \
                       s, (const float*)q, (const float*)k, (const float*)v,                 \
                       (const float*)dout, lse, delta, counts, offsets, inverse, kv_vbs,     \
                       (float*)dk, (float*)dv, (const float*)dkc, (const float*)dvc, tph,    \
                       (int)sq, (int)skv, (int)(sq / BB), (int)(skv / BB), topk, c2, scale); \
    return vsa_check_launch();                                                               \
  }                                                                                          \
  }
  VSA_F32_SHAPES(VSA_F)
#undef VSA_F
  return VSA_ERR_UNSUPPORTED;
}

}  // namespace vsa
