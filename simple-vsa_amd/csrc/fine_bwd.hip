// Split sparse backward on gfx950 MFMA: a query-owned dQ kernel and a
// KV-owned dK/dV kernel walking the CSR inverse route.  Neither uses float
// atomics, so both are deterministic.
//
// Reference contract: _triton_sparse_attention_backward (triton_impl.py:1321-1527)
// with the dQ kernels (703-969) and dK/dV kernels (972-1318).  The pooled
// (coarse) gradients are folded into the epilogues: the reference applies them
// in a separate block-mean backward (fused_common.py:62-103) and autograd adds
// the two gradients afterwards.
//
// dQ, per wave (32 queries) and 64-key chunk, P recomputed from the saved LSE:
//   S^T  = K Q^T,  dP^T = V dO^T,  dS^T = P^T (dP^T - delta),  dQ^T += K^T dS^T
// dK/dV, per wave (32 keys) and 32-query sub-tile of an in-edge query block:
//   S = Q K^T,  dP = dO V^T,  dS = P (dP - delta),  dV^T += dO^T P,  dK^T += Q^T dS
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

// ===========================================================================
// dQ
// ===========================================================================
template <int D, int BE>
struct DqCfg {
  static constexpr int QT = BE >= 128 ? 128 : BE;
  static constexpr int NW = QT / 32;
  static constexpr int NT = NW * 64;
  static constexpr int KC = 64;
  static constexpr int TILE = KC * D;            // one K (or V) chunk, swizzled row-major
  static constexpr int STAGE = 2 * TILE;
};

template <int BE>
__device__ __forceinline__ bool next_valid_chunk_b(const int32_t* __restrict__ sel,
                                                   const int32_t* __restrict__ vbs, int topk,
                                                   int kb, int& s, int& c, int& kv, int& nvb) {
  // Uniform indices keep these reads on the scalar path: a vector load here
  // would need vmcnt(0) and so wait for every K/V copy still in flight.
  while (s < topk) {
    kv = __builtin_amdgcn_readfirstlane(sel[__builtin_amdgcn_readfirstlane(s)]);
    if (kv >= 0 && kv < kb) {
      nvb = __builtin_amdgcn_readfirstlane(clamp_valid(vbs[kv], BE));
      if (c * 64 < nvb) return true;
    }
    ++s;
    c = 0;
  }
  return false;
}

template <typename T, int D, int BE>
__global__ __launch_bounds__((DqCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(2))) void
sparse_dq_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                 const T* __restrict__ dout, const float* __restrict__ lse,
                 const float* __restrict__ delta, const int32_t* __restrict__ selected,
                 const int32_t* __restrict__ kv_vbs, T* __restrict__ dq,
                 const T* __restrict__ dqc, const int32_t* __restrict__ q_vbs, int num_tiles,
                 int tiles_per_head, int sq, int skv, int qb, int kb, int topk, float c2,
                 uint32_t qsign, float scale) {
  using C = DqCfg<D, BE>;
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) T smem[2 * C::STAGE];

  const int tile = xcd_tile(blockIdx.x, num_tiles);
  if (tile >= num_tiles) return;
  const int64_t b = tile / tiles_per_head;
  const int q0 = (tile % tiles_per_head) * C::QT;
  const int qblk = q0 / BE;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  const int myq = q0 + wave * 32 + r;
  const int64_t tok = (int64_t)b * sq + myq;

  V8 qf[D / 16], df[D / 16];
  {
    const T* qrow = q + tok * D + 8 * h;
    const T* drow = dout + tok * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + 16 * ks);
      raw ^= qsign;
      qf[ks] = as_vec8<T>(raw);
      df[ks] = as_vec8<T>(*reinterpret_cast<const u32x4*>(drow + 16 * ks));
    }
  }
  const float my_lse = lse[tok];
  const float my_delta = delta[tok];

  const int32_t* sel = selected + ((int64_t)b * qb + qblk) * topk;
  const T* kbase = k + (int64_t)b * skv * D;
  const T* vbase = v + (int64_t)b * skv * D;

  auto dma = [&](int kvb, int ch, int stg) {
    const int64_t off = ((int64_t)kvb * BE + ch * C::KC) * D;
    T* Ks = smem + stg * C::STAGE;
    dma_tile<T, D, C::KC, C::NT>(Ks, kbase + off);
    dma_tile<T, D, C::KC, C::NT>(Ks + C::TILE, vbase + off);
  };

  f32x16 dqacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) dqacc[mt] = f32x16{};

  int s = 0, ch = 0, kv = 0, nvb = 0;
  bool have = next_valid_chunk_b<BE>(sel, kv_vbs, topk, kb, s, ch, kv, nvb);
  if (have) dma(kv, ch, 0);
  dma_wait();
  __syncthreads();
  int stage = 0;
  while (have) {
    const int nv = min(nvb - ch * 64, 64);
    int s2 = s, ch2 = ch + 1, kv2 = kv, nvb2 = nvb;
    const bool have2 = next_valid_chunk_b<BE>(sel, kv_vbs, topk, kb, s2, ch2, kv2, nvb2);
    if (have2) dma(kv2, ch2, stage ^ 1);
    const T* Ks = smem + stage * C::STAGE;
    const T* Vs = Ks + C::TILE;

    f32x16 sacc[2] = {f32x16{}, f32x16{}};
    f32x16 pacc[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int smt = 0; smt < 2; ++smt) {
        sacc[smt] = E::mfma32(row_a8<T, D>(Ks, smt * 32 + r, ks, h), qf[ks], sacc[smt]);
        pacc[smt] = E::mfma32(row_a8<T, D>(Vs, smt * 32 + r, ks, h), df[ks], pacc[smt]);
      }
    }
    // dS^T = P^T (dP^T - delta), consumed 8 keys at a time as the B operand
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      float dsv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * (kk & 1) + e;
        const float p = fast_exp2(fmaf(sacc[kk >> 1][i], c2, -my_lse));
        dsv[e] = p * (pacc[kk >> 1][i] - my_delta);
        if (nv < 64) {
          const int key = (kk >> 1) * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key >= nv) dsv[e] = 0.f;
        }
      }
      const V8 bop = pack8<T>(dsv);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        dqacc[mt] = E::mfma32(tr_a8<T, D>(Ks, mt * 32, 16 * kk, 16 * kk + 8), bop, dqacc[mt]);
    }
    dma_wait();
    __syncthreads();
    stage ^= 1;
    s = s2; ch = ch2; kv = kv2; nvb = nvb2; have = have2;
  }

  // ---- epilogue: scale, fold the pooled gradient, store ------------------
  const int qpos = myq - qblk * BE;
  float cdiv = 1.f;
  bool cvalid = false;
  const T* crow = nullptr;
  if (dqc) {
    const int32_t cnt = q_vbs[qblk];
    cvalid = qpos < clamp_valid(cnt, BE);
    cdiv = (float)(cnt > 1 ? cnt : 1);
    crow = dqc + ((int64_t)b * qb + qblk) * D;
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = mt * 32 + 8 * g + 4 * h;
      float cval[4] = {0.f, 0.f, 0.f, 0.f};
      if (cvalid) {
        u32x2 cr = *reinterpret_cast<const u32x2*>(crow + d0);
        const T* cc = reinterpret_cast<const T*>(&cr);
#pragma unroll
        for (int e = 0; e < 4; ++e) cval[e] = round_t<T>(E::to_f(cc[e]) / cdiv);
      }
      T o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float val = round_t<T>(dqacc[mt][4 * g + e] * scale);
        o4[e] = E::from_f(val + cval[e]);
      }
      *reinterpret_cast<u32x2*>(dq + tok * D + d0) = *reinterpret_cast<const u32x2*>(o4);
    }
  }
}

// ===========================================================================
// dK / dV
// ===========================================================================
template <int D, int BE>
struct DkvCfg {
  static constexpr int KT = BE >= 128 ? 128 : BE;  // keys per workgroup
  static constexpr int NW = KT / 32;
  static constexpr int NT = NW * 64;
  static constexpr int QS = 32;                    // queries per LDS stage
  static constexpr int TILE = QS * D;              // one Q (or dO) sub-tile, swizzled
  static constexpr int STAGE = 2 * TILE;
  static constexpr int SUBS = BE / QS;             // sub-tiles per query block
};

template <typename T, int D, int BE>
__global__ __launch_bounds__((DkvCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(2))) void sparse_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ inverse, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ dk, T* __restrict__ dv, const T* __restrict__ dkc,
    const T* __restrict__ dvc, int num_tiles, int tiles_per_head, int sq, int skv, int qb,
    int kb, int topk, float c2, uint32_t ksign, float scale) {
  using C = DkvCfg<D, BE>;
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) T smem[2 * C::STAGE];
  __shared__ __attribute__((aligned(16))) float sstat[2][2][C::QS];  // [stage][lse, delta][query]

  const int tile = xcd_tile(blockIdx.x, num_tiles);
  if (tile >= num_tiles) return;
  const int64_t b = tile / tiles_per_head;
  const int k0 = (tile % tiles_per_head) * C::KT;  // first key (within head)
  const int kvblk = k0 / BE;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  const int mykey = k0 + wave * 32 + r;
  const int64_t ktok = (int64_t)b * skv + mykey;
  const int nvb = clamp_valid(kv_vbs[kvblk], BE);
  const bool key_valid = (mykey - kvblk * BE) < nvb;

  // K^T, V^T fragments (B operands): lane (r, h) holds key r, dims 16ks + 8h ..
  V8 kf[D / 16], vf[D / 16];
  {
    const T* krow = k + ktok * D + 8 * h;
    const T* vrow = v + ktok * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(krow + 16 * ks);
      raw ^= ksign;
      kf[ks] = as_vec8<T>(raw);
      vf[ks] = as_vec8<T>(*reinterpret_cast<const u32x4*>(vrow + 16 * ks));
    }
  }

  const int64_t meta = (int64_t)b * kb + kvblk;
  const int nedge = counts[meta];
  const int32_t* seg = inverse + (int64_t)b * qb * topk + offsets[meta];
  const int items = nedge * C::SUBS;
  const T* qbase = q + (int64_t)b * sq * D;
  const T* dbase = dout + (int64_t)b * sq * D;
  const float* lbase = lse + (int64_t)b * sq;
  const float* ebase = delta + (int64_t)b * sq;

  // Q / dO sub-tile -> two swizzled LDS tiles; lse / delta (32 + 32 floats)
  // -> sstat[stg] through one dword-wide direct load by wave 0.
  auto dma = [&](int item, int stg) {
    const int qblock = seg[item / C::SUBS];
    const int qrow0 = qblock * BE + (item % C::SUBS) * C::QS;
    T* base = smem + stg * C::STAGE;
    dma_tile<T, D, C::QS, C::NT>(base, qbase + (int64_t)qrow0 * D);
    dma_tile<T, D, C::QS, C::NT>(base + C::TILE, dbase + (int64_t)qrow0 * D);
    if (tid < 64) {
      const float* src = tid < C::QS ? lbase + qrow0 + tid : ebase + qrow0 + (tid - C::QS);
      dma4(src, __builtin_amdgcn_readfirstlane(lds_addr(&sstat[stg][0][0])));
    }
  };

  f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
    dkacc[mt] = f32x16{};
    dvacc[mt] = f32x16{};
  }

  if (items > 0) dma(0, 0);
  dma_wait();
  __syncthreads();
  int stage = 0;
  for (int it = 0; it < items; ++it) {
    const bool more = it + 1 < items;
    if (more) dma(it + 1, stage ^ 1);
    const T* Qs = smem + stage * C::STAGE;
    const T* Ds = Qs + C::TILE;

    // S = Q K^T and dP = dO V^T: 32 queries x 32 keys
    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      sacc = E::mfma32(row_a8<T, D>(Qs, r, ks, h), kf[ks], sacc);
      pacc = E::mfma32(row_a8<T, D>(Ds, r, ks, h), vf[ks], pacc);
    }
    // rows of this lane: queries 8g + 4h + e; consumed 8 queries (g = 2j, 2j+1)
    // at a time: dV^T += dO^T P ; dK^T += Q^T dS
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float pv[8], dsv[8];
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g = 2 * j + gg;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&sstat[stage][0][8 * g + 4 * h]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sstat[stage][1][8 * g + 4 * h]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = key_valid ? fast_exp2(fmaf(sacc[4 * g + e], c2, -l4[e])) : 0.f;
          pv[4 * gg + e] = p;
          dsv[4 * gg + e] = p * (pacc[4 * g + e] - d4[e]);
        }
      }
      const V8 bp = pack8<T>(pv);
      const V8 bs = pack8<T>(dsv);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) {
        dvacc[mt] = E::mfma32(tr_a8<T, D>(Ds, mt * 32, 16 * j, 16 * j + 8), bp, dvacc[mt]);
        dkacc[mt] = E::mfma32(tr_a8<T, D>(Qs, mt * 32, 16 * j, 16 * j + 8), bs, dkacc[mt]);
      }
    }
    dma_wait();
    __syncthreads();
    stage ^= 1;
  }

  // ---- epilogue ------------------------------------------------------------
  const int32_t cnt = kv_vbs[kvblk];
  const float cdiv = (float)(cnt > 1 ? cnt : 1);
  const T* kcrow = dkc ? dkc + ((int64_t)b * kb + kvblk) * D : nullptr;
  const T* vcrow = dvc ? dvc + ((int64_t)b * kb + kvblk) * D : nullptr;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = mt * 32 + 8 * g + 4 * h;
      float ck[4] = {0.f, 0.f, 0.f, 0.f}, cv[4] = {0.f, 0.f, 0.f, 0.f};
      if (key_valid && kcrow) {
        u32x2 a = *reinterpret_cast<const u32x2*>(kcrow + d0);
        u32x2 bb = *reinterpret_cast<const u32x2*>(vcrow + d0);
        const T* ka = reinterpret_cast<const T*>(&a);
        const T* va = reinterpret_cast<const T*>(&bb);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ck[e] = round_t<T>(E::to_f(ka[e]) / cdiv);
          cv[e] = round_t<T>(E::to_f(va[e]) / cdiv);
        }
      }
      T k4[4], v4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        k4[e] = E::from_f(round_t<T>(dkacc[mt][4 * g + e] * scale) + ck[e]);
        v4[e] = E::from_f(round_t<T>(dvacc[mt][4 * g + e]) + cv[e]);
      }
      *reinterpret_cast<u32x2*>(dk + ktok * D + d0) = *reinterpret_cast<const u32x2*>(k4);
      *reinterpret_cast<u32x2*>(dv + ktok * D + d0) = *reinterpret_cast<const u32x2*>(v4);
    }
  }
}

template <typename T, int D, int BE>
static int launch_dq(const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, const float* delta, const int32_t* selected,
                     const int32_t* kv_vbs, void* dq, const void* dqc, const int32_t* q_vbs,
                     int64_t bh, int64_t sq, int64_t skv, int topk, float scale,
                     hipStream_t stream) {
  using C = DqCfg<D, BE>;
  const int tph = (int)(sq / C::QT);
  const int64_t tiles = bh * tph;
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int grid = (int)(((tiles + 7) / 8) * 8);
  hipLaunchKernelGGL((sparse_dq_kernel<T, D, BE>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, selected,
                     kv_vbs, (T*)dq, (const T*)dqc, q_vbs, (int)tiles, tph, (int)sq, (int)skv,
                     (int)(sq / BE), (int)(skv / BE), topk, fabsf(scale) * kLog2e,
                     scale < 0.f ? 0x80008000u : 0u, scale);
  return vsa_check_launch();
}

template <typename T, int D, int BE>
static int launch_dkdv(const void* q, const void* k, const void* v, const void* dout,
                       const float* lse, const float* delta, const int32_t* counts,
                       const int32_t* offsets, const int32_t* inverse, const int32_t* kv_vbs,
                       void* dk, void* dv, const void* dkc, const void* dvc, int64_t bh,
                       int64_t sq, int64_t skv, int topk, float scale, hipStream_t stream) {
  using C = DkvCfg<D, BE>;
  const int tph = (int)(skv / C::KT);
  const int64_t tiles = bh * tph;
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int grid = (int)(((tiles + 7) / 8) * 8);
  hipLaunchKernelGGL((sparse_dkdv_kernel<T, D, BE>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, counts,
                     offsets, inverse, kv_vbs, (T*)dk, (T*)dv, (const T*)dkc, (const T*)dvc,
                     (int)tiles, tph, (int)sq, (int)skv, (int)(sq / BE), (int)(skv / BE), topk,
                     fabsf(scale) * kLog2e, scale < 0.f ? 0x80008000u : 0u, scale);
  return vsa_check_launch();
}

}  // namespace vsa

using namespace vsa;

#define VSA_BWD_SHAPES(X) X(128, 256) X(128, 128) X(128, 64) X(64, 256) X(64, 128) X(64, 64)

extern "C" int vsa_sparse_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                                 const float* lse, const float* delta, const int32_t* selected,
                                 const int32_t* kv_vbs, void* dq, const void* d_q_c,
                                 const int32_t* q_vbs, int64_t bh, int64_t sq, int64_t skv,
                                 int32_t D, int32_t be, int32_t topk, float scale, int32_t dtype,
                                 void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !selected || !kv_vbs || !dq) return VSA_ERR_NULL;
  if (d_q_c && !q_vbs) return VSA_ERR_NULL;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
#define VSA_DQ_CASE(DD, BB)                                                                  \
  if (D == DD && be == BB)                                                                   \
    return launch_dq<T, DD, BB>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c, q_vbs, \
                                bh, sq, skv, topk, scale, s);
  VSA_DISPATCH_MFMA(dtype, T, { VSA_BWD_SHAPES(VSA_DQ_CASE) });
#undef VSA_DQ_CASE
  return VSA_ERR_UNSUPPORTED;
}

extern "C" int vsa_sparse_bwd_dkdv(const void* q, const void* k, const void* v,
                                   const void* dout, const float* lse, const float* delta,
                                   const int32_t* counts, const int32_t* offsets,
                                   const int32_t* inverse, const int32_t* kv_vbs, void* dk,
                                   void* dv, const void* d_k_c, const void* d_v_c, int64_t bh,
                                   int64_t sq, int64_t skv, int32_t D, int32_t be, int32_t topk,
                                   float scale, int32_t dtype, void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !counts || !offsets || !inverse || !kv_vbs ||
      !dk || !dv)
    return VSA_ERR_NULL;
  if ((d_k_c == nullptr) != (d_v_c == nullptr)) return VSA_ERR_NULL;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
#define VSA_DKDV_CASE(DD, BB)                                                                \
  if (D == DD && be == BB)                                                                   \
    return launch_dkdv<T, DD, BB>(q, k, v, dout, lse, delta, counts, offsets, inverse,       \
                                  kv_vbs, dk, dv, d_k_c, d_v_c, bh, sq, skv, topk, scale, s);
  VSA_DISPATCH_MFMA(dtype, T, { VSA_BWD_SHAPES(VSA_DKDV_CASE) });
#undef VSA_DKDV_CASE
  return VSA_ERR_UNSUPPORTED;
}
