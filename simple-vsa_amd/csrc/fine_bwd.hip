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
  static constexpr int KP = D + 8;   // natural row pitch
  static constexpr int TP = KC + 8;  // transposed row pitch
  static constexpr int KS = KC * KP;
  static constexpr int KT = D * TP;
  static constexpr int STAGE = 2 * KS + KT;  // K, V natural + K transposed
  static constexpr int UNITS = (KC / 4) * (D / 8);  // 4 keys x 8 dims
  static constexpr int U_PER_T = (UNITS + NT - 1) / NT;
};

template <int BE>
__device__ __forceinline__ bool next_valid_chunk_b(const int32_t* __restrict__ sel,
                                                   const int32_t* __restrict__ vbs, int topk,
                                                   int kb, int& s, int& c, int& kv, int& nvb) {
  while (s < topk) {
    kv = sel[s];
    if (kv >= 0 && kv < kb) {
      nvb = clamp_valid(vbs[kv], BE);
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
  __shared__ __attribute__((aligned(16))) T smem[C::STAGE];
  T* Ks = smem;
  T* Vs = Ks + C::KS;
  T* Kt = Vs + C::KS;

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

  u32x4 kreg[C::U_PER_T][4], vreg[C::U_PER_T][4];
  auto gload = [&](int kvb, int ch) {
    const int64_t off = ((int64_t)kvb * BE + ch * C::KC) * D;
#pragma unroll
    for (int i = 0; i < C::U_PER_T; ++i) {
      const int u = tid + i * C::NT;
      if (C::UNITS % C::NT == 0 || u < C::UNITS) {
        const int kg = u & 15, dg = u >> 4;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int64_t o = off + (kg * 4 + rr) * D + dg * 8;
          kreg[i][rr] = *reinterpret_cast<const u32x4*>(kbase + o);
          vreg[i][rr] = *reinterpret_cast<const u32x4*>(vbase + o);
        }
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < C::U_PER_T; ++i) {
      const int u = tid + i * C::NT;
      if (C::UNITS % C::NT == 0 || u < C::UNITS) {
        const int kg = u & 15, dg = u >> 4;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          *reinterpret_cast<u32x4*>(Ks + (kg * 4 + rr) * C::KP + dg * 8) = kreg[i][rr];
          *reinterpret_cast<u32x4*>(Vs + (kg * 4 + rr) * C::KP + dg * 8) = vreg[i][rr];
        }
        u32x2 cols[8];
        transpose4x8_b16(kreg[i], cols);
        const int pos = (kg >> 2) * 16 + group4_pos(kg & 3) * 4;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<u32x2*>(Kt + (dg * 8 + j) * C::TP + pos) = cols[j];
      }
    }
  };

  f32x16 dqacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) dqacc[mt] = f32x16{};

  int s = 0, ch = 0, kv = 0, nvb = 0;
  bool have = next_valid_chunk_b<BE>(sel, kv_vbs, topk, kb, s, ch, kv, nvb);
  if (have) gload(kv, ch);
  while (have) {
    const int nv = min(nvb - ch * 64, 64);
    __syncthreads();  // previous chunk fully consumed
    lstore();
    __syncthreads();
    int s2 = s, ch2 = ch + 1, kv2 = kv, nvb2 = nvb;
    const bool have2 = next_valid_chunk_b<BE>(sel, kv_vbs, topk, kb, s2, ch2, kv2, nvb2);
    if (have2) gload(kv2, ch2);

    f32x16 sacc[2] = {f32x16{}, f32x16{}};
    f32x16 pacc[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int smt = 0; smt < 2; ++smt) {
        const int row = (smt * 32 + r) * C::KP + ks * 16 + h * 8;
        const V8 ak = as_vec8<T>(*reinterpret_cast<const u32x4*>(Ks + row));
        const V8 av = as_vec8<T>(*reinterpret_cast<const u32x4*>(Vs + row));
        sacc[smt] = E::mfma32(ak, qf[ks], sacc[smt]);
        pacc[smt] = E::mfma32(av, df[ks], pacc[smt]);
      }
    }
    float dsv[2][16];
#pragma unroll
    for (int smt = 0; smt < 2; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = exp2f(fmaf(sacc[smt][i], c2, -my_lse));
        dsv[smt][i] = p * (pacc[smt][i] - my_delta);
      }
    if (nv < 64) {
#pragma unroll
      for (int smt = 0; smt < 2; ++smt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key >= nv) dsv[smt][i] = 0.f;
        }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const V8 bop = pack8<T>(&dsv[kk >> 1][8 * (kk & 1)]);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) {
        const V8 a = as_vec8<T>(
            *reinterpret_cast<const u32x4*>(Kt + (mt * 32 + r) * C::TP + kk * 16 + h * 8));
        dqacc[mt] = E::mfma32(a, bop, dqacc[mt]);
      }
    }
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
  static constexpr int QS = 32;      // queries per LDS stage
  static constexpr int NP = D + 8;   // natural row pitch
  static constexpr int TP = QS + 8;  // transposed row pitch
  static constexpr int NS = QS * NP;
  static constexpr int TS = D * TP;
  static constexpr int STAGE = 2 * NS + 2 * TS;  // Q, dO natural + transposed
  static constexpr int UNITS = 2 * (QS / 4) * (D / 8);  // both tensors
  static constexpr int U_PER_T = (UNITS + NT - 1) / NT;
  static constexpr int SUBS = BE / QS;  // sub-tiles per query block
};

template <typename T, int D, int BE>
__global__ __launch_bounds__((DkvCfg<D, BE>::NT)) void sparse_dkdv_kernel(
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

  u32x4 reg[C::U_PER_T][4];
  float stat_reg = 0.f;
  auto gload = [&](int item) {
    const int qblock = seg[item / C::SUBS];
    const int qrow0 = qblock * BE + (item % C::SUBS) * C::QS;
#pragma unroll
    for (int i = 0; i < C::U_PER_T; ++i) {
      const int u = tid + i * C::NT;
      if (C::UNITS % C::NT == 0 || u < C::UNITS) {
        const int tsel = u / (C::UNITS / 2);  // 0: q, 1: dout
        const int uu = u % (C::UNITS / 2);
        const int qg = uu & 7, dg = uu >> 3;
        const T* src = (tsel ? dbase : qbase) + (int64_t)(qrow0 + qg * 4) * D + dg * 8;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) reg[i][rr] = *reinterpret_cast<const u32x4*>(src + rr * D);
      }
    }
    if (tid < 2 * C::QS) {
      const int qq = tid % C::QS;
      stat_reg = tid < C::QS ? lbase[qrow0 + qq] : ebase[qrow0 + qq];
    }
  };
  auto lstore = [&](int stage) {
    T* base = smem + stage * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::U_PER_T; ++i) {
      const int u = tid + i * C::NT;
      if (C::UNITS % C::NT == 0 || u < C::UNITS) {
        const int tsel = u / (C::UNITS / 2);
        const int uu = u % (C::UNITS / 2);
        const int qg = uu & 7, dg = uu >> 3;
        T* nat = base + tsel * C::NS;
        T* tr = base + 2 * C::NS + tsel * C::TS;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *reinterpret_cast<u32x4*>(nat + (qg * 4 + rr) * C::NP + dg * 8) = reg[i][rr];
        u32x2 cols[8];
        transpose4x8_b16(reg[i], cols);
        const int pos = (qg >> 2) * 16 + group4_pos(qg & 3) * 4;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<u32x2*>(tr + (dg * 8 + j) * C::TP + pos) = cols[j];
      }
    }
    if (tid < 2 * C::QS) sstat[stage][tid / C::QS][tid % C::QS] = stat_reg;
  };

  f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
    dkacc[mt] = f32x16{};
    dvacc[mt] = f32x16{};
  }

  if (items > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  int stage = 0;
  for (int it = 0; it < items; ++it) {
    const bool more = it + 1 < items;
    if (more) gload(it + 1);
    const T* base = smem + stage * C::STAGE;
    const T* Qs = base;
    const T* Ds = base + C::NS;
    const T* Qt = base + 2 * C::NS;
    const T* Dt = Qt + C::TS;

    // S = Q K^T and dP = dO V^T: 32 queries x 32 keys
    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const int row = r * C::NP + ks * 16 + h * 8;
      const V8 aq = as_vec8<T>(*reinterpret_cast<const u32x4*>(Qs + row));
      const V8 ad = as_vec8<T>(*reinterpret_cast<const u32x4*>(Ds + row));
      sacc = E::mfma32(aq, kf[ks], sacc);
      pacc = E::mfma32(ad, vf[ks], pacc);
    }
    // rows of this lane: queries 8g + 4h + e
    float pv[16], dsv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(&sstat[stage][0][8 * g + 4 * h]);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sstat[stage][1][8 * g + 4 * h]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * g + e;
        const float p = key_valid ? exp2f(fmaf(sacc[i], c2, -l4[e])) : 0.f;
        pv[i] = p;
        dsv[i] = p * (pacc[i] - d4[e]);
      }
    }
    // dV^T += dO^T P ; dK^T += Q^T dS   (reduce over the 32 queries)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const V8 bp = pack8<T>(&pv[8 * j]);
      const V8 bs = pack8<T>(&dsv[8 * j]);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) {
        const int trow = (mt * 32 + r) * C::TP + j * 16 + h * 8;
        const V8 ad = as_vec8<T>(*reinterpret_cast<const u32x4*>(Dt + trow));
        const V8 aq = as_vec8<T>(*reinterpret_cast<const u32x4*>(Qt + trow));
        dvacc[mt] = E::mfma32(ad, bp, dvacc[mt]);
        dkacc[mt] = E::mfma32(aq, bs, dkacc[mt]);
      }
    }
    if (more) lstore(stage ^ 1);
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
