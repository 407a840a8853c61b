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
// dQ, per wave (32 queries) and KC-key chunk, P recomputed from the saved LSE:
//   S^T  = K Q^T,  dP^T = V dO^T,  dS^T = P^T (dP^T - delta),  dQ^T += K^T dS^T
// dK/dV, per wave (32 keys) and 32-query sub-tile of an in-edge query block:
//   S = Q K^T,  dP = dO V^T,  dS = P (dP - delta),  dV^T += dO^T P,  dK^T += Q^T dS
#include <mutex>
#include <type_traits>

#include "dkdv_cfg.h"
#include "fine_f32.h"
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
  // keys per chunk: 32 at block 64, so that a 2-wave workgroup's double buffer
  // is 32 KiB at head_dim 128 (four workgroups share a CU) and 16 KiB at 64
  // (twice the resident waves of 64-key chunks: c5 forward 0.88 -> 0.78 ms,
  // dQ 0.93 -> 0.89 ms)
  static constexpr int KC = BE == 64 ? 32 : 64;
  static constexpr int NSM = KC / 32;            // 32-key sub-tiles per chunk
  static constexpr int WPE = D == 256 ? 1 : 2;    // waves per SIMD the registers are sized for
  static constexpr int TILE = KC * D;            // one K (or V) chunk, swizzled row-major
  static constexpr int STAGE = 2 * TILE;
};

// dQ epilogue: scale, fold the pooled gradient of the query block
// (`d_q_c / count`, valid rows only), store.  One lane = one query row,
// holding dQ^T column r.  With RASTER, dq is a raster-order sequence of s_out
// tokens: slot myq goes to raster row orows[myq], a padding slot (< 0) nowhere.
template <typename T, int D, int BE, bool RASTER = false>
__device__ __forceinline__ void dq_epilogue(const f32x16 (&dqacc)[D / 32], int64_t b, int myq,
                                            int qblk, int h, int sq, int qb, T* __restrict__ dq,
                                            const T* __restrict__ dqc,
                                            const int32_t* __restrict__ q_vbs, float scale,
                                            const int32_t* __restrict__ orows = nullptr,
                                            int64_t s_out = 0, int heads = 0) {
  using E = Elem<T>;
  int64_t tok = (int64_t)b * sq + myq;
  if constexpr (RASTER) {
    const int r = orows[myq];
    if (r < 0 || r >= s_out) return;
    tok = raster_row(b, r, s_out, heads);
  }
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
  const float rcp = 1.0f / cdiv;
  // the row regrouped for 16-byte accesses: w[mt][p][i] is dim
  // mt*32 + 8(2p + h) + i (both lanes of a swapped pair hold this query, so
  // they return above together)
  float w[D / 32][2][8];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) swap_rows16(dqacc[mt], scale, w[mt]);
  u32x4 cr[D / 32][2];  // loaded together, so their latency is paid once
  if (cvalid) {
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        cr[mt][p] = *reinterpret_cast<const u32x4*>(crow + mt * 32 + 16 * p + 8 * h);
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d0 = mt * 32 + 16 * p + 8 * h;
      float cval[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (cvalid) {
        const T* cc = reinterpret_cast<const T*>(&cr[mt][p]);
#pragma unroll
        for (int e = 0; e < 8; ++e) cval[e] = round_t<T>(div_by_count(E::to_f(cc[e]), cdiv, rcp));
      }
      T o8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o8[e] = E::from_f(round_t<T>(w[mt][p][e]) + cval[e]);
      *reinterpret_cast<u32x4*>(dq + tok * D + d0) = *reinterpret_cast<const u32x4*>(o8);
    }
  }
}

template <typename T, int D, int BE, bool RASTER>
__global__ __launch_bounds__((DqCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(DqCfg<D, BE>::WPE))) void
sparse_dq_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                 const T* __restrict__ dout, const float* __restrict__ lse,
                 const float* __restrict__ delta, const int32_t* __restrict__ selected,
                 const int32_t* __restrict__ kv_vbs, T* __restrict__ dq,
                 const T* __restrict__ dqc, const int32_t* __restrict__ q_vbs, int num_tiles,
                 int tiles_per_head, int sq, int skv, int qb, int kb, int topk, float c2,
                 uint32_t qsign, float scale, const int32_t* __restrict__ orows, int64_t s_out, int heads) {
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

  TileDma<T, D, C::KC, C::NT> tdma;
  tdma.init();
  auto dma = [&](int kvb, int ch, int stg) {
    const int64_t off = ((int64_t)kvb * BE + ch * C::KC) * D;
    T* Ks = smem + stg * C::STAGE;
    tdma.copy(Ks, kbase + off);
    tdma.copy(Ks + C::TILE, vbase + off);
  };

  f32x16 dqacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) dqacc[mt] = f32x16{};

  // Per-lane LDS byte offsets inside a tile, set once (the offsets row_a8 /
  // tr_a8 compute: the swizzle repeats every 16 rows, so rows 32*smt + r sit
  // at row_off[ks] + 32*smt*D*2 and the transposed pieces of keys 16*kk + ..
  // at tr_off[mt][hi] + 16*kk*D*2; left to the compiler, that arithmetic was
  // redone for every chunk).  At head dim 256 the 32 offsets, held across the
  // chunk loop next to the 512 registers of fragments and accumulators, made
  // the kernel spill inside the loop (dQ 8.1 -> 10.5 ms at 20 heads x 40 960
  // tokens): there the offsets are formed per read and the loop keeps one body.
  constexpr bool LANE_OFFSETS = D <= 128;
  uint32_t row_off[D / 16], tr_off[D / 32][2];
  if constexpr (LANE_OFFSETS) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) row_off[ks] = opaque((uint32_t)(swz<D>(r, 2 * ks + h) * sizeof(T)));
    const int grp = lane >> 4, jl = lane & 15, qq = grp & 1, hh = grp >> 1;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        tr_off[mt][hi] = opaque((uint32_t)(
            swz_elem<D>(8 * hi + 4 * hh + (jl >> 2), mt * 32 + 16 * qq + 4 * (jl & 3)) * sizeof(T)));
  }
  const char* smem_c = reinterpret_cast<const char*>(smem);
  auto t_row = [&](int stg, int tilesel, int ks, int smt) {  // K (tilesel 0) or V rows 32*smt + r
    if constexpr (!LANE_OFFSETS)
      return row_a8<T, D>(smem + stg * C::STAGE + tilesel * C::TILE, smt * 32 + r, ks, h);
    else
      return as_vec8<T>(*reinterpret_cast<const u32x4*>(
          smem_c + (stg * C::STAGE + tilesel * C::TILE + smt * 32 * D) * (int)sizeof(T) + row_off[ks]));
  };
  auto k_tr = [&](int stg, int mt, int kk) {  // K^T pieces, keys 16kk ..
    if constexpr (!LANE_OFFSETS) {
      return tr_a8<T, D>(smem + stg * C::STAGE, mt * 32, 16 * kk, 16 * kk + 8);
    } else {
      const char* base = smem_c + (stg * C::STAGE + kk * 16 * D) * (int)sizeof(T);
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][0]));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][1]));
      u32x4 rr;
      rr[0] = __builtin_bit_cast(u32x2, lo)[0];
      rr[1] = __builtin_bit_cast(u32x2, lo)[1];
      rr[2] = __builtin_bit_cast(u32x2, hi)[0];
      rr[3] = __builtin_bit_cast(u32x2, hi)[1];
      return as_vec8<T>(rr);
    }
  };

  RouteRegs<BE, C::KC> route{sel, kv_vbs, topk, kb};
  route.load(0);
  int s = 0, ch = 0, kv = 0, nvb = 0;
  bool have = route.next(s, ch, kv, nvb);
  if (have) dma(kv, ch, 0);
  dma_wait();
  __syncthreads();
  // one chunk on stage stage_c (with lane offsets the loop below is unrolled
  // by the two stages, so that every LDS address is a lane offset plus an
  // immediate)
  auto chunk = [&](auto stage_c) {
    const int stage = stage_c;
    const int nv = min(nvb - ch * C::KC, C::KC);
    int s2 = s, ch2 = ch + 1, kv2 = kv, nvb2 = nvb;
    const bool have2 = route.next(s2, ch2, kv2, nvb2);
    if (have2) dma(kv2, ch2, stage ^ 1);

    f32x16 sacc[C::NSM], pacc[C::NSM];
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt) sacc[smt] = pacc[smt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int smt = 0; smt < C::NSM; ++smt) {
        sacc[smt] = E::mfma32(t_row(stage, 0, ks, smt), qf[ks], sacc[smt]);
        pacc[smt] = E::mfma32(t_row(stage, 1, ks, smt), df[ks], pacc[smt]);
      }
    }
    // dS^T = P^T (dP^T - delta), consumed 8 keys at a time as the B operand
#pragma unroll
    for (int kk = 0; kk < 2 * C::NSM; ++kk) {
      float dsv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * (kk & 1) + e;
        const float p = fast_exp2(fmaf(sacc[kk >> 1][i], c2, -my_lse));
        dsv[e] = p * (pacc[kk >> 1][i] - my_delta);
      }
      if (nv < C::KC) {
        // key (kk >> 1)*32 + 8(i >> 2) + (i & 3) + 4h >= nv, compared as 4h >=
        // nv - (its constant part) on a count re-read inside the branch (no
        // comparison hoisted out of the branch into every chunk)
        const int nvl = uniform_here(nv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * (kk & 1) + e;
          if (4 * h >= nvl - ((kk >> 1) * 32 + 8 * (i >> 2) + (i & 3))) dsv[e] = 0.f;
        }
      }
      const V8 bop = pack8<T>(dsv);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        dqacc[mt] = E::mfma32(k_tr(stage, mt, kk), bop, dqacc[mt]);
    }
    dma_wait();
    __syncthreads();
    s = s2; ch = ch2; kv = kv2; nvb = nvb2; have = have2;
  };
  // one exit: a break between the two chunks let the two bodies keep the
  // accumulators in different registers, with a copy of every accumulator
  // between them
  if constexpr (LANE_OFFSETS) {
    while (have) {
      chunk(std::integral_constant<int, 0>{});
      if (have) chunk(std::integral_constant<int, 1>{});
    }
  } else {
    for (int stage = 0; have; stage ^= 1) chunk(stage);
  }

  dq_epilogue<T, D, BE, RASTER>(dqacc, b, myq, qblk, h, sq, qb, dq, dqc, q_vbs, scale, orows,
                                s_out, heads);
}

// ===========================================================================
// dK / dV: one workgroup per KV tile of KT keys (wave w owns keys KW w ..
// KW w + KW - 1 as KTL 32-key MFMA tiles, K^T/V^T fragments in VGPRs),
// looping over the 32-query sub-tiles ("items") of the tile's CSR in-edges.
// Per item i the wave computes
//   A(i): S = Q_i K^T, dP = dO_i V^T             (MFMA, rows of the LDS tiles)
//   B(i): P = exp2(S c2 - lse), dS = P (dP - delta)          (VALU)
//   C(i): dV^T += dO_i^T P, dK^T += Q_i^T dS      (MFMA, transposed LDS reads)
// software-pipelined so that A(i+1) is issued between the VALU work of B(i)
// (an MFMA only overlaps VALU work of its own wave on CDNA4).  One wave per
// SIMD: the accumulators live in AGPRs, and latency is covered inside the
// wave by an LDS read stream L operands deep and an NS-stage LDS ring of
// items filled by direct global->LDS loads spread over each step.  Every LDS
// operand read feeds KTL MFMAs (one per key tile of the wave).
// ===========================================================================
// DkvCfg (shape, stage protocol) and DkvShared (LDS layout): dkdv_cfg.h

// One key tile (tile_s < num_tiles) of sparse_dkdv_kernel, start to finish.
// On return every wave's direct loads may still be in flight (the last steps
// re-copy the last item): the caller drains them before the LDS is reused.
template <typename T, int D, int BE, bool RASTER>
__device__ __forceinline__ void dkdv_tile(
    DkvShared<T, D, BE>& sh, int tile_s,
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ inverse, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ dk, T* __restrict__ dv, const T* __restrict__ dkc,
    const T* __restrict__ dvc, int tiles_per_head, int sq, int skv, int qb,
    int kb, int topk, float c2, uint32_t ksign, float scale,
    const int32_t* __restrict__ orows, int64_t s_out, int heads) {
  using C = DkvCfg<D, BE>;
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  constexpr int NS = C::NS, NA = C::NA, NC = C::NC, L = C::L, TP = C::TP, KTL = C::KTL;
  constexpr int NV = C::NV;
  auto& smem = sh.smem;
  auto& sstat = sh.sstat;
  auto& sseg = sh.sseg;

  const int tile = tile_s / C::NSPLIT;
  const int d_off = (tile_s % C::NSPLIT) * C::DH;  // first dK/dV dim of this workgroup
  const int64_t b = tile / tiles_per_head;
  const int k0 = (tile % tiles_per_head) * C::KT;  // first key (within head)
  const int kvblk = k0 / BE;
  // the wave index is uniform: every direct-load LDS base derived from it stays
  // on the scalar unit (no per-copy read-back of a vector register)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  // this lane's key in key tile t: mykey0 + 32 t
  const int mykey0 = k0 + wave * C::KW + r;
  const int32_t cnt = kv_vbs[kvblk];  // read once: the epilogue's pooled division needs it too
  const int nvb = clamp_valid(cnt, BE);

  // K^T, V^T fragments (B operands): lane (r, h) of key tile t holds key
  // mykey0 + 32 t, dims 16ks + 8h ..
  V8 kf[KTL][D / 16], vf[KTL][D / 16];
#pragma unroll
  for (int t = 0; t < KTL; ++t) {
    const int64_t ktok = (int64_t)b * skv + mykey0 + 32 * t;
    const T* krow = k + ktok * D + 8 * h;
    const T* vrow = v + ktok * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(krow + 16 * ks);
      raw ^= ksign;
      kf[t][ks] = as_vec8<T>(raw);
      vf[t][ks] = as_vec8<T>(*reinterpret_cast<const u32x4*>(vrow + 16 * ks));
    }
  }

  const int64_t meta = (int64_t)b * kb + kvblk;
  const int nedge = counts[meta];
  const int32_t* seg = inverse + (int64_t)b * qb * topk + offsets[meta];
  const int items = nedge * C::SUBS;
  // The pooled-gradient rows are one per key block: their dims are divided by
  // the count and rounded to T here, once per workgroup and dim, into LDS (in
  // the epilogue every lane would repeat them for its own key: about half of
  // the epilogue's VALU work).
  constexpr int NPOOL = (2 * C::DH + C::NT - 1) / C::NT;   // pooled dims per thread
  float pool_raw[NPOOL];
  // the thread index passes through an asm that reads the tile, so that the
  // lane addresses below are formed per tile: hoisted out of the persistent
  // loop they would stay live (spilled) across every tile
  int ptid = tid;
  asm volatile("" : "+v"(ptid) : "s"(tile_s));
  if (dkc) {
    const int64_t prow = ((int64_t)b * kb + kvblk) * D + d_off;
#pragma unroll
    for (int i = 0; i < NPOOL; ++i) {
      const int x = ptid + i * C::NT;
      pool_raw[i] = x < 2 * C::DH ? E::to_f((x < C::DH ? dkc : dvc)[prow + x % C::DH]) : 0.f;
    }
  }
  // The first NT entries of the CSR segment are loaded here too, under the
  // fragment loads' wait, instead of after it in the first refill (one memory
  // round trip and a barrier less per tile).
  const int seg0 = ptid < nedge ? seg[ptid] : 0;
  // Retire the fragment loads before the ring starts: the compiler's own vmcnt
  // bookkeeping does not see the direct loads, and a wait it placed in the
  // loop for these registers would also drain the in-flight stages.
  dma_wait();
  if (dkc) {
    const float cdiv = (float)(cnt > 1 ? cnt : 1), rcp = 1.0f / cdiv;
#pragma unroll
    for (int i = 0; i < NPOOL; ++i) {
      const int x = ptid + i * C::NT;
      if (x < 2 * C::DH)
        sh.spool[x / C::DH][x % C::DH] = E::from_f(div_by_count(pool_raw[i], cdiv, rcp));
    }
  }
  if (ptid < nedge) sseg[ptid] = seg0;
  __syncthreads();  // publishes spool and the first CSR entries
  const T* qbase = q + (int64_t)b * sq * D;
  const T* dbase = dout + (int64_t)b * sq * D;
  const float* lbase = lse + (int64_t)b * sq;
  const float* ebase = delta + (int64_t)b * sq;

  // ---- per-lane LDS / global offsets (bytes), fixed for the whole loop ----
  uint32_t row_off[D / 16];  // A rows: lane (r, h), dims 16ks + 8h .. +7
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) row_off[ks] = opaque((uint32_t)(swz<D>(r, 2 * ks + h) * 2));
  uint32_t tr_off[C::DH / 32][2];  // C operands: rows 8hi + 4h + e, dims d_off + 32mt + 16q + 4g
  {
    const int grp = lane >> 4, jl = lane & 15;
    const int qq = grp & 1, hh = grp >> 1;
#pragma unroll
    for (int mt = 0; mt < C::DH / 32; ++mt)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        tr_off[mt][hi] = opaque((uint32_t)(
            swz_elem<D>(8 * hi + 4 * hh + (jl >> 2), d_off + mt * 32 + 16 * qq + 4 * (jl & 3)) * 2));
  }
  const uint32_t st_off = opaque((uint32_t)(4 * h * 4));
  uint32_t cp_goff[TP], cp_loff[TP];  // direct-load pieces: global offset, LDS block
#pragma unroll
  for (int i = 0; i < TP; ++i) {
    const int blk = C::piece_block(i, wave);
    int c;
    const int row = unswz_row_chunk<D>(blk * 64 + lane, c);
    cp_goff[i] = opaque((uint32_t)((row * D + c * 8) * 2));
    cp_loff[i] = (uint32_t)(blk * 1024);
  }
  const uint32_t smem_lds = lds_addr(&smem[0][0]);
  const uint32_t sstat_lds = lds_addr(&sstat[0][0][0]);
  const char* smem_c = reinterpret_cast<const char*>(&smem[0][0]);
  const char* sstat_c = reinterpret_cast<const char*>(&sstat[0][0][0]);

  // CSR segment staged in LDS, SEGMAX entries at a time (a scalar load per
  // item would put scalar-memory latency in front of every copy, a vector
  // load would need vmcnt(0) and drain the ring).  The refill runs where every
  // wave has finished with the previous entries (all waves call qblock_of at
  // the same program point, between two barriers).  Entries [0, NT) were
  // staged before the ring started.
  int seg_lo = 0, seg_hi = C::NT;
  auto qblock_of = [&](int item) {
    const int e = item / C::SUBS;
    if (e >= seg_hi) {
      __syncthreads();
      seg_lo = e;
      seg_hi = e + C::SEGMAX;
      for (int i = tid; i < C::SEGMAX && seg_lo + i < nedge; i += C::NT) sseg[i] = seg[seg_lo + i];
      __syncthreads();
    }
    return __builtin_amdgcn_readfirstlane(sseg[e - seg_lo]);
  };
  struct Copy {
    const char* qsrc;
    const char* dsrc;
    const float* ssrc;  // per lane: lse (lanes < 32) or delta
  };
  auto copy_of = [&](int item) {
    Copy cp;
    const int qrow0 = qblock_of(item) * BE + (item % C::SUBS) * C::QS;
    cp.qsrc = reinterpret_cast<const char*>(qbase + (int64_t)qrow0 * D);
    cp.dsrc = reinterpret_cast<const char*>(dbase + (int64_t)qrow0 * D);
    cp.ssrc = lane < C::QS ? lbase + qrow0 + lane : ebase + qrow0 + (lane - C::QS);
    return cp;
  };
  // piece p of an item's copy into stage stg (p < TP: Q, < 2TP: dO, else stats)
  auto copy_piece = [&](const Copy& cp, int stg, int p) {
    if (p < 2 * TP) {
      const int i = p % TP;
      const uint32_t lds = smem_lds + (uint32_t)((stg * 2 * C::TILE + (p < TP ? 0 : C::TILE)) * 2) + cp_loff[i];
      dma16_s(cp_goff[i], p < TP ? cp.qsrc : cp.dsrc, __builtin_amdgcn_readfirstlane(lds));
    } else {
      dma4(cp.ssrc, __builtin_amdgcn_readfirstlane(sstat_lds + (uint32_t)(stg * 2 * C::QS * 4)));
    }
  };

  // Each accumulator leaves its zero through an asm of its own: without it the
  // compiler shares one zero register between them and the S / dP tiles and
  // then moves two dK/dV accumulators aside every step to make room for S/dP
  // (about 16 extra accumulator moves per step, and a spill at head_dim 256).
  // At two waves per SIMD a wave has 256 registers and every product keeps its
  // accumulator in VGPRs (no AGPR is pinned).
  f32x16 dkacc[C::DH / 32][KTL], dvacc[C::DH / 32][KTL];
#pragma unroll
  for (int mt = 0; mt < C::DH / 32; ++mt)
#pragma unroll
    for (int t = 0; t < KTL; ++t) {
      dkacc[mt][t] = f32x16{};
      dvacc[mt][t] = f32x16{};
      if constexpr (C::WPE == 1) asm volatile("" : "+a"(dkacc[mt][t]), "+a"(dvacc[mt][t]));
    }

  auto row_read = [&](int stg, int tilesel, int ks) {
    return as_vec8<T>(*reinterpret_cast<const u32x4*>(
        smem_c + row_off[ks] + (stg * 2 * C::TILE + tilesel * C::TILE) * 2));
  };
  auto tr_read = [&](int stg, int tilesel, int mt, int j) {
    const char* base = smem_c + (stg * 2 * C::TILE + tilesel * C::TILE + 16 * j * D) * 2;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][0]));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][1]));
    u32x4 rr;
    rr[0] = __builtin_bit_cast(u32x2, lo)[0];
    rr[1] = __builtin_bit_cast(u32x2, lo)[1];
    rr[2] = __builtin_bit_cast(u32x2, hi)[0];
    rr[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_vec8<T>(rr);
  };
  auto read_stats = [&](int stg, f32x4 (&l4)[4], f32x4 (&d4)[4], int g) {
    const char* st = sstat_c + st_off + stg * 2 * C::QS * 4;
    l4[g] = *reinterpret_cast<const f32x4*>(st + 8 * g * 4);
    d4[g] = *reinterpret_cast<const f32x4*>(st + (C::QS + 8 * g) * 4);
  };

  // Every step copies exactly one item (past the last item it re-copies the
  // last one into the free stage).
  //
  // Stage protocol (NS = 4 stages, one item each).  Step i runs A(i+1) on the
  // rows of item i+1 and C(i) on the transposed tiles of item i, and copies
  // item i+3 into the stage of item i-1.
  //  * EARLY_BARRIER: the step's workgroup barrier sits inside C(i), KB dV / dK
  //    products before its end.  Every copy piece of item i+3 is issued before
  //    it, so waiting until at most PER loads are in flight means item i+2 has
  //    landed in this wave; the barrier then publishes item i+2 to every wave
  //    and retires every wave's reads of item i (all issued, and waited for by
  //    the barrier's lgkmcnt, before it), whose stage step i+1 copies into.
  //    Right after it the first L operand reads of step i+1 (rows of item
  //    i+2) are issued, so the last KB products of C(i) cover their LDS
  //    latency and step i+1 opens with an MFMA (c3 dK/dV 1.5 %, c2 4.6 % less
  //    time than the barrier at the step's top, bit-identical).
  //  * otherwise the barrier opens step i: at most PER loads in flight means
  //    item i+1 has landed, the barrier publishes it and retires the reads of
  //    item i-1, and the step's first operand reads follow it.
  constexpr bool EB = C::EARLY_BARRIER;
  constexpr int VB = C::VB;   // the early barrier follows C iteration VB
  if constexpr (C::WPE > 1) {
    // Two waves per SIMD: step i runs item i start to finish (S and dP, P and
    // dS, dV and dK) on stage i % NS.  It waits until at most (NS - 2) items
    // of copies are in flight (item i, copied three steps ahead, has landed),
    // the barrier publishes item i and retires every wave's reads of item i-1,
    // and the step copies item i+3 into that stage.
    if (items > 0) {
#pragma unroll
      for (int i = 0; i < NS - 1; ++i) {
        const Copy cp = copy_of(i < items ? i : items - 1);
#pragma unroll
        for (int p = 0; p < C::PER; ++p) copy_piece(cp, i, p);
      }
      Copy cpn = copy_of(NS - 1 < items ? NS - 1 : items - 1);
      auto sstep = [&](auto stage_c, int it) {
        constexpr int S = decltype(stage_c)::value, SP = C::copy_stage(S);
        wait_vmcnt<C::SIMPLE_WAIT>();
        __syncthreads();
        const Copy cp = cpn;
        f32x4 l4[4], d4[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) read_stats(S, l4, d4, g);
        f32x16 sacc[KTL], pacc[KTL];
#pragma unroll
        for (int t = 0; t < KTL; ++t) {
          sacc[t] = f32x16{};
          pacc[t] = f32x16{};
        }
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          const V8 qa = row_read(S, 0, ks), da = row_read(S, 1, ks);
#pragma unroll
          for (int t = 0; t < KTL; ++t) {
            sacc[t] = E::mfma32(qa, kf[t][ks], sacc[t]);
            pacc[t] = E::mfma32(da, vf[t][ks], pacc[t]);
          }
        }
        // the copy of item it+NS-1, issued while the S / dP products run
#pragma unroll
        for (int p = 0; p < C::PER; ++p) copy_piece(cp, SP, p);
        V8 bp[KTL][2], bs[KTL][2];
#pragma unroll
        for (int t = 0; t < KTL; ++t) {
          float pv[16], dsv[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            pv[e] = fast_exp2(fmaf(sacc[t][e], c2, -l4[e >> 2][e & 3]));
            dsv[e] = pv[e] * (pacc[t][e] - d4[e >> 2][e & 3]);
          }
          bp[t][0] = pack8<T>(pv);
          bp[t][1] = pack8<T>(pv + 8);
          bs[t][0] = pack8<T>(dsv);
          bs[t][1] = pack8<T>(dsv + 8);
        }
#pragma unroll
        for (int vv = 0; vv < NC; ++vv) {
          const int j = vv / (2 * (C::DH / 32)), mt = (vv >> 1) % (C::DH / 32);
          const V8 a = tr_read(S, (vv & 1) ? 0 : 1, mt, j);
#pragma unroll
          for (int t = 0; t < KTL; ++t) {
            if (vv & 1)
              dkacc[mt][t] = E::mfma32(a, bs[t][j], dkacc[mt][t]);
            else
              dvacc[mt][t] = E::mfma32(a, bp[t][j], dvacc[mt][t]);
          }
        }
        const int nn = it + NS;
        cpn = copy_of(nn < items ? nn : items - 1);
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      static_assert(NS == 4, "the step sequence below is unrolled for NS = 4");
      int it = 0;
      for (; it + 4 <= items; it += 4) {
        sstep(I0{}, it);
        sstep(I1{}, it + 1);
        sstep(I2{}, it + 2);
        sstep(I3{}, it + 3);
      }
      if (it < items) sstep(I0{}, it);
      if (it + 1 < items) sstep(I1{}, it + 1);
      if (it + 2 < items) sstep(I2{}, it + 2);
    }
  } else {
  f32x16 sA[KTL], pA[KTL], sB[KTL], pB[KTL];
  f32x4 lA[4], dA[4], lB[4], dB[4];
  V8 preA[L], preB[L];
  Copy cpn;
  if (items <= 0) goto epilogue;
  {
#pragma unroll
    for (int i = 0; i < NS - 1; ++i) {
      const Copy cp = copy_of(i < items ? i : items - 1);
#pragma unroll
      for (int p = 0; p < C::PER; ++p) copy_piece(cp, i, p);
    }
    cpn = copy_of(NS - 1 < items ? NS - 1 : items - 1);
    wait_vmcnt<(NS - 2) * C::PER>();   // item 0 landed
    __syncthreads();
#pragma unroll
    for (int t = 0; t < KTL; ++t) {
      sA[t] = f32x16{};
      pA[t] = f32x16{};
    }
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const V8 qa = row_read(0, 0, ks), da = row_read(0, 1, ks);
#pragma unroll
      for (int t = 0; t < KTL; ++t) {
        sA[t] = E::mfma32(qa, kf[t][ks], sA[t]);
        pA[t] = E::mfma32(da, vf[t][ks], pA[t]);
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) read_stats(0, lA, dA, g);
    if constexpr (EB) {
      wait_vmcnt<(NS - 3) * C::PER>();   // item 1 landed
      __syncthreads();
#pragma unroll
      for (int x = 0; x < L; ++x) preA[x] = row_read(1, x & 1, x >> 1);
    }
  }

  {
    // One pipeline step on item i (stage S = i % NS): B(i) between the MFMAs
    // of A(i+1), then C(i).  LDS operands stream with a lookahead of L: rows
    // of item i+1 for A (the first L of them read by the previous step, in
    // opc), then transposed tiles of item i for C, then the statistics of
    // item i+1; after the barrier, the first L rows of item i+2 into opn.
    // The copy of item i+NS-1 goes to stage S-1.
    auto step = [&](auto stage_c, int it, f32x16 (&sc)[KTL], f32x16 (&pc)[KTL],
                    f32x16 (&sn)[KTL], f32x16 (&pn)[KTL], f32x4 (&lc)[4], f32x4 (&dc)[4],
                    f32x4 (&ln)[4], f32x4 (&dn)[4], V8 (&opc)[L], V8 (&opn)[L]) {
      constexpr int S = C::c_stage(decltype(stage_c)::value);
      constexpr int SN = C::a_stage(S), SNN = C::pre_stage(S), SP = C::copy_stage(S);
      if constexpr (!EB) {
        wait_vmcnt<C::STEP_WAIT>();
        // publishes item it+1 to every wave and retires every wave's reads of
        // item it-1, whose stage the copy below reuses
        __syncthreads();
      }
      const Copy cp = cpn;
      V8 op[NA + NC];
      auto issue = [&](int x) {
        if (x < NA) {
          op[x] = row_read(SN, x & 1, x >> 1);
        } else if (x < NA + NC) {
          const int vv = x - NA;
          const int j = vv / (2 * (C::DH / 32)), mt = (vv >> 1) % (C::DH / 32);
          op[x] = tr_read(S, (vv & 1) ? 0 : 1, mt, j);
        } else if (x < NA + NC + 4) {
          read_stats(SN, ln, dn, x - NA - NC);
        }
      };
#pragma unroll
      for (int x = 0; x < L; ++x) {
        if constexpr (EB)
          op[x] = opc[x];
        else
          issue(x);
      }
#pragma unroll
      for (int t = 0; t < KTL; ++t) {
        sn[t] = f32x16{};
        pn[t] = f32x16{};
      }
      // B(i) is spread over the NA reads of A(i+1) and the first NC/2 of C(i):
      // value x at stream position x * (NA + NC/2) / NV, so that about four
      // VALU operations sit under each MFMA.  Value x is element e of key tile
      // t, in the order the halves of C consume them (rows 0-7 of every key
      // tile, then rows 8-15); the first half is done inside A; dS trails P
      // by one value (exp latency).
      float pv[KTL][16], dsv[KTL][16];
      auto b_slot = [&](int pos) {
#pragma unroll
        for (int x = 0; x < NV; ++x)
          if (x * (NA + NC / 2) / NV == pos) {
            const int t = (x / 8) % KTL, e = 8 * (x / (8 * KTL)) + x % 8;
            pv[t][e] = fast_exp2(fmaf(sc[t][e], c2, -lc[e >> 2][e & 3]));
            if (x >= 1) {
              const int y = x - 1;
              const int ty = (y / 8) % KTL, ey = 8 * (y / (8 * KTL)) + y % 8;
              dsv[ty][ey] = pv[ty][ey] * (pc[ty][ey] - dc[ey >> 2][ey & 3]);
            }
            if (x == NV - 1) dsv[t][e] = pv[t][e] * (pc[t][e] - dc[e >> 2][e & 3]);
          }
      };
      static_assert(8 * KTL * (NA + NC / 2) / NV < NA, "the first half of dS must be done inside A");
#pragma unroll
      for (int u = 0; u < NA; ++u) {
        issue(u + L);
#pragma unroll
        for (int t = 0; t < KTL; ++t) {
          if (u & 1)
            pn[t] = E::mfma32(op[u], vf[t][u >> 1], pn[t]);
          else
            sn[t] = E::mfma32(op[u], kf[t][u >> 1], sn[t]);
        }
        b_slot(u);
        __builtin_amdgcn_sched_barrier(0);
      }
      V8 bp[KTL][2], bs[KTL][2];
#pragma unroll
      for (int t = 0; t < KTL; ++t) {
        bp[t][0] = pack8<T>(pv[t]);
        bs[t][0] = pack8<T>(dsv[t]);
      }
#pragma unroll
      for (int vv = 0; vv < NC; ++vv) {
        issue(NA + vv + L);
        const int j = vv / (2 * (C::DH / 32)), mt = (vv >> 1) % (C::DH / 32);
#pragma unroll
        for (int t = 0; t < KTL; ++t) {
          if (vv & 1)
            dkacc[mt][t] = E::mfma32(op[NA + vv], bs[t][j], dkacc[mt][t]);
          else
            dvacc[mt][t] = E::mfma32(op[NA + vv], bp[t][j], dvacc[mt][t]);
        }
        // the copy of item it+NS-1, spread over C iterations CP0..CP1 (before
        // an early barrier): a copy stalls its wave on the address unit, and
        // there it overlaps MFMAs and little P / dS arithmetic (2 % less step
        // time than over the S / dP MFMAs)
#pragma unroll
        for (int p = 0; p < C::PER; ++p)
          if (C::piece_iter(p) == vv) copy_piece(cp, SP, p);
        if (vv < NC / 2) b_slot(NA + vv);
        if (vv == NC / 2 - 1) {
#pragma unroll
          for (int t = 0; t < KTL; ++t) {
            bp[t][1] = pack8<T>(pv[t] + 8);
            bs[t][1] = pack8<T>(dsv[t] + 8);
          }
        }
        if (EB && vv == VB) {
          // see the stage protocol above: publishes item it+2, retires the
          // reads of item it; then the next step's first operand reads
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<C::STEP_WAIT>();
          __syncthreads();
#pragma unroll
          for (int x = 0; x < L; ++x) opn[x] = row_read(SNN, x & 1, x >> 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int x = NA + NC + L; x < NA + NC + 4; ++x) issue(x);
      // descriptor of the copy issued by the next step (its CSR entry is an
      // LDS read, kept off the next step's critical path).  It comes after
      // both MFMA phases: the CSR refill branch inside it splits the code, and
      // placed between the phases it let the compiler sink B(i) (used only by
      // C(i)) past the branch, out from under the MFMAs of A(i+1).
      const int nn = it + NS;
      cpn = copy_of(nn < items ? nn : items - 1);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    static_assert(NS == 4, "the step sequence below is unrolled for NS = 4");
    int it = 0;
    for (; it + 4 <= items; it += 4) {
      step(I0{}, it, sA, pA, sB, pB, lA, dA, lB, dB, preA, preB);
      step(I1{}, it + 1, sB, pB, sA, pA, lB, dB, lA, dA, preB, preA);
      step(I2{}, it + 2, sA, pA, sB, pB, lA, dA, lB, dB, preA, preB);
      step(I3{}, it + 3, sB, pB, sA, pA, lB, dB, lA, dA, preB, preA);
    }
    if (it < items) step(I0{}, it, sA, pA, sB, pB, lA, dA, lB, dB, preA, preB);
    if (it + 1 < items) step(I1{}, it + 1, sB, pB, sA, pA, lB, dB, lA, dA, preB, preA);
    if (it + 2 < items) step(I2{}, it + 2, sA, pA, sB, pB, lA, dA, lB, dB, preA, preB);
  }
  }

epilogue:
  // ---- epilogue ------------------------------------------------------------
  // every key of the wave is in one key block: one pooled row for all of them
  const bool any_valid = mykey0 - kvblk * BE < nvb;
  // rows regrouped for 16-byte accesses (swap_rows16): w[p][i] is dim
  // d_off + mt*32 + 8(2p + h) + i of this lane's key; both lanes of a swapped
  // pair hold the same key
  u32x4 kcv[C::DH / 32][2], vcv[C::DH / 32][2];
  if (any_valid && dkc) {
#pragma unroll
    for (int mt = 0; mt < C::DH / 32; ++mt)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int d0 = mt * 32 + 16 * p + 8 * h;   // within this workgroup's dims
        kcv[mt][p] = *reinterpret_cast<const u32x4*>(&sh.spool[0][d0]);
        vcv[mt][p] = *reinterpret_cast<const u32x4*>(&sh.spool[1][d0]);
      }
  }
#pragma unroll
  for (int t = 0; t < KTL; ++t) {
    const int mykey = mykey0 + 32 * t;
    const bool key_valid = (mykey - kvblk * BE) < nvb;
    // dK / dV row: this key's slot, or with RASTER its raster row orows[mykey]
    // in a sequence of s_out tokens (a padding slot, < 0, has none)
    int64_t otok = (int64_t)b * skv + mykey;
    if constexpr (RASTER) {
      const int r = orows[mykey];
      otok = (r >= 0 && r < s_out) ? raster_row(b, r, s_out, heads) : -1;
    }
    const bool ostore = !RASTER || otok >= 0;
#pragma unroll
    for (int mt = 0; mt < C::DH / 32; ++mt) {
      float wk[2][8], wv[2][8];
      swap_rows16(dkacc[mt][t], scale, wk);
      swap_rows16(dvacc[mt][t], 1.0f, wv);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int d0 = d_off + mt * 32 + 16 * p + 8 * h;
        float ck[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float cv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (key_valid && dkc) {
          const T* ka = reinterpret_cast<const T*>(&kcv[mt][p]);
          const T* va = reinterpret_cast<const T*>(&vcv[mt][p]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            ck[e] = E::to_f(ka[e]);
            cv[e] = E::to_f(va[e]);
          }
        }
        // A padding key gets no gradient; its lane's accumulators (which only
        // ever hold that key) are dropped here instead of masking every score.
        T k8[8], v8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float fk = key_valid ? round_t<T>(wk[p][e]) : 0.f;
          const float fv = key_valid ? round_t<T>(wv[p][e]) : 0.f;
          k8[e] = E::from_f(fk + ck[e]);
          v8[e] = E::from_f(fv + cv[e]);
        }
        if (ostore) {
          *reinterpret_cast<u32x4*>(dk + otok * D + d0) = *reinterpret_cast<const u32x4*>(k8);
          *reinterpret_cast<u32x4*>(dv + otok * D + d0) = *reinterpret_cast<const u32x4*>(v8);
        }
      }
    }
  }
}

// Persistent dK/dV: as many workgroups as the CUs hold at once, each looping
// over key tiles (a workgroup per tile left every CU idle between one tile's
// end and the next one's start, about 5 % of the kernel, plus an uneven tail).
// Workgroup i runs on XCD i % 8 and takes tiles from that XCD's contiguous
// range: with a tile_order workspace (vsa_dkdv_tile_order) the next entry of
// the range's order comes from the XCD's counter (so early finishers take more
// tiles); once its own range is drained, a workgroup of an index-order range
// takes the remaining tiles of the other XCDs' ranges (XCD x+1, x+2, ... in
// turn), since the XCDs do not run equally fast (at c3 some took 3-4 % longer
// per item than others on the same tile counts: 2.7 % less kernel time with
// the stealing).  Longest-first ranges (entries tagged kLongestFirst) do not
// steal: at c5 that cost 1.8 %.  The last workgroup to finish zeroes the
// counters for the next launch.  Without a workspace, a fixed stride over the
// range in index order.  Head dim 256 keeps one workgroup per tile
// (tile_order[i] or the XCD order).
constexpr int kLongestFirst = 1 << 30;  // tag of the entries of a longest-first range

template <typename T, int D, int BE, bool RASTER>
__global__ __launch_bounds__((DkvCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(DkvCfg<D, BE>::WPE, DkvCfg<D, BE>::WPE))) void sparse_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ inverse, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ dk, T* __restrict__ dv, const T* __restrict__ dkc,
    const T* __restrict__ dvc, int num_tiles, int tiles_per_head, int sq, int skv, int qb,
    int kb, int topk, float c2, uint32_t ksign, float scale, int32_t* __restrict__ tile_order,
    const int32_t* __restrict__ orows, int64_t s_out, int heads) {
  __shared__ DkvShared<T, D, BE> sh;
  if constexpr (DkvCfg<D, BE>::NSPLIT > 1) {
    // head_dim 256: one tile per workgroup (the loop's state would push the
    // fragments and accumulators, which fill the register file, into scratch)
    const int tile_s = tile_order ? tile_order[blockIdx.x] & (kLongestFirst - 1)
                                  : xcd_tile(blockIdx.x, num_tiles);
    if (tile_s < num_tiles)
      dkdv_tile<T, D, BE, RASTER>(sh, tile_s, q, k, v, dout, lse, delta, counts, offsets,
                                  inverse, kv_vbs, dk, dv, dkc, dvc, tiles_per_head, sq, skv, qb,
                                  kb, topk, c2, ksign, scale, orows, s_out, heads);
    return;
  }
  __shared__ int s_next;
  const int xcd = blockIdx.x & 7;
  const int per = (num_tiles + 7) >> 3;       // tiles per XCD range
  const int stride = (int)(gridDim.x >> 3);   // workgroups per XCD
  int32_t* ctr = tile_order ? tile_order + 8 * per : nullptr;  // [8 ranges][done]
  // (thread 0) the ranges this workgroup may take tiles from: its own, and
  // with last = 8 the others (take_entry)
  int from = 0, last = 1;
  for (int round = 0;; ++round) {
    int j;
    if (ctr) {
      if (threadIdx.x == 0) s_next = take_entry(ctr, xcd, per, from, last);  // the order entry
      __syncthreads();
      j = s_next;
      if (j < 0) break;
      // an entry of its own index-order range lets the workgroup steal later
      if (threadIdx.x == 0 && from == 0 && !(tile_order[j] & kLongestFirst)) last = 8;
    } else {
      j = (int)(blockIdx.x >> 3) + round * stride;
      if (j >= per) break;
      j = 8 * j + xcd;
    }
    const int tile_s = ctr ? tile_order[j] & (kLongestFirst - 1) : xcd * per + (j >> 3);
    if (tile_s < num_tiles)
      dkdv_tile<T, D, BE, RASTER>(sh, tile_s, q, k, v, dout, lse, delta, counts, offsets,
                                  inverse, kv_vbs, dk, dv, dkc, dvc, tiles_per_head, sq, skv, qb,
                                  kb, topk, c2, ksign, scale, orows, s_out, heads);
    dma_wait();       // this wave's trailing copies land before the LDS is reused
    __syncthreads();  // and every wave is done with it (and with s_next)
  }
  if (ctr && threadIdx.x == 0) finish_entries(ctr);
}

// ---------------------------------------------------------------------------
// Ping-pong dQ for 256-token blocks: the schedule of the 8-wave forward.
// One workgroup of 8 waves owns a query block; group 0 (waves 0-3) and group 1
// (waves 4-7) share a SIMD pairwise and run one phase apart:
//   MFMA phase of chunk j:  dQ^T += K_{j-1}^T dS_{j-1}^T, then
//                           S_j = K_j Q^T and dP_j = V_j dO^T
//   VALU phase of chunk j:  P = exp2(S c2 - lse), dS = P (dP - delta), packed.
// K_j is read as rows in chunk j's phase and transposed in chunk j+1's, V_j
// only in chunk j's.  Per query row the arithmetic and its order are those of
// sparse_dq_kernel.
// ---------------------------------------------------------------------------
template <int D>
struct DqPPCfg {
  static constexpr int NT = 512;
  static constexpr int KC = 64;
  static constexpr int TILE = KC * D;
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NS = 4;
};

// One query block (tile < bh * Sq / 256) of sparse_dq_pp_kernel.
template <typename T, int D, bool RASTER>
__device__ __forceinline__ void dq_pp_tile(
    T* smem, int tile, const T* __restrict__ q, const T* __restrict__ k,
    const T* __restrict__ v, const T* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, const int32_t* __restrict__ selected,
    const int32_t* __restrict__ kv_vbs, T* __restrict__ dq, const T* __restrict__ dqc,
    const int32_t* __restrict__ q_vbs, int sq, int skv, int qb, int kb, int topk, float c2,
    uint32_t qsign, float scale, const int32_t* __restrict__ orows, int64_t s_out, int heads) {
  constexpr int BE = 256;
  using C = DqPPCfg<D>;
  using E = Elem<T>;
  typedef typename E::vec8 V8;

  const int64_t b = tile / qb;
  const int qblk = tile % qb;
  // the lane index passes through an asm that reads the tile, so the lane
  // offsets derived from it are recomputed per tile in the persistent loop
  // instead of being hoisted out of it and kept (spilled) across the tile
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid) : "s"(tile));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const bool grp1 = wave >= 4;
  const int myq = qblk * BE + wave * 32 + r;
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
  RouteRegs<BE, C::KC> route{sel, kv_vbs, topk, kb};
  route.load(0);
  TileDma<T, D, C::KC, C::NT> tdma;
  tdma.init();
  int ps = 0, pc = 0, pkv = 0, pnvb = 0;
  bool pvalid = route.next(ps, pc, pkv, pnvb);
  auto issue = [&](int stg) {  // copy the cursor's chunk; its valid keys (0: none)
    int nv = 0;
    if (pvalid) {
      const int64_t off = ((int64_t)pkv * BE + pc * C::KC) * D;
      T* Ks = smem + stg * C::STAGE;
      tdma.copy(Ks, kbase + off, wave);
      tdma.copy(Ks + C::TILE, vbase + off, wave);
      nv = min(pnvb - pc * C::KC, C::KC);
      ++pc;
      pvalid = route.next(ps, pc, pkv, pnvb);
    }
    return nv;
  };

  // per-lane LDS byte offsets (the swizzle repeats every 16 rows)
  uint32_t row_off[D / 16], tr_off[D / 32][2];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    row_off[ks] = opaque((uint32_t)(swz<D>(r, 2 * ks + h) * sizeof(T)));
  {
    const int grp = lane >> 4, jl = lane & 15, qq = grp & 1, hh = grp >> 1;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        tr_off[mt][hi] = opaque((uint32_t)(
            swz_elem<D>(8 * hi + 4 * hh + (jl >> 2), mt * 32 + 16 * qq + 4 * (jl & 3)) *
            sizeof(T)));
  }
  const char* smem_c = reinterpret_cast<const char*>(smem);
  auto t_row = [&](const char* base, int ks, int smt) {  // K or V rows 32*smt + r
    return as_vec8<T>(*reinterpret_cast<const u32x4*>(base + row_off[ks] +
                                                       smt * 32 * D * (int)sizeof(T)));
  };
  auto t_tr = [&](const char* base, int mt, int kk) {  // K^T pieces, keys 16kk ..
    const char* bb = base + kk * 16 * D * (int)sizeof(T);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bb + tr_off[mt][0]));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(bb + tr_off[mt][1]));
    u32x4 rr;
    rr[0] = __builtin_bit_cast(u32x2, lo)[0];
    rr[1] = __builtin_bit_cast(u32x2, lo)[1];
    rr[2] = __builtin_bit_cast(u32x2, hi)[0];
    rr[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_vec8<T>(rr);
  };

  f32x16 sacc[2], pacc[2], dqacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) dqacc[mt] = f32x16{};
  V8 bs[4];  // dS of the last VALU phase as B operands, 16 keys each

  // MFMA phase: when with_dq, dQ += K_{j-1}^T dS_{j-1}^T first (16 MFMAs, K^T
  // of stage sp; the packed dS dies before S and dP are written), then S_j and
  // dP_j (32 MFMAs, K and V rows of stage sj); every LDS operand is read L
  // MFMAs ahead of its use (head_dim 128: 2, the most that does not spill
  // inside the chunk loop).
  constexpr int NSP = 4 * (D / 16), NDQ = 4 * (D / 32), L = D == 128 ? 2 : 8;
  // Deeper stream while the dQ products run: the S / dP accumulators are not
  // live yet, so their registers hold operands instead.
  constexpr int LD = 8;
  // The first L operands of a phase with the dQ products (K^T pieces of chunk
  // j-1, in LDS since long before) are read at the end of the preceding VALU
  // phase, so the MFMA phase does not open with an LDS round trip.
  static_assert(L <= NDQ, "the prefetched operands are K^T pieces");
  V8 pre[L];
  auto prefetch = [&](int sp) {
    const char* Kp = smem_c + sp * C::STAGE * (int)sizeof(T);
    __builtin_amdgcn_sched_barrier(0);  // after the VALU phase's arithmetic
#pragma unroll
    for (int u = 0; u < L; ++u) pre[u] = t_tr(Kp, u % (D / 32), u / (D / 32));
  };
  auto mma_x = [&](int sj, int sp, auto with_dq) {
    constexpr int N0 = decltype(with_dq)::value ? NDQ : 0;  // dQ products first
    constexpr int NX = N0 + NSP;
    const char* Kb = smem_c + sj * C::STAGE * (int)sizeof(T);
    const char* Vb = Kb + C::TILE * (int)sizeof(T);
    const char* Kp = smem_c + sp * C::STAGE * (int)sizeof(T);
    V8 op[NX];
    // u < N0: y = u (kk = y / (D/32), mt = y % (D/32)); then x = (u - N0) >> 1
    // (ks = x >> 1, smt = x & 1), even: K row (S), odd: V row (dP)
    auto load = [&](int u) {
      if (u >= NX) return;
      if (u < N0) {
        op[u] = t_tr(Kp, u % (D / 32), u / (D / 32));
      } else {
        const int x = (u - N0) >> 1;
        op[u] = t_row(((u - N0) & 1) ? Vb : Kb, x >> 1, x & 1);
      }
    };
#pragma unroll
    for (int u = 0; u < L; ++u) {
      if (N0 > 0)
        op[u] = pre[u];
      else
        load(u);
    }
    // last operand index loaded by the time MFMA u issues: u + LD during the
    // dQ products, u + L after them (never less than already loaded)
    auto hi = [](int u) {
      if (u < 0) return L - 1;
      if (u < N0) return u + LD;
      return (N0 > 0 && N0 - 1 + LD > u + L) ? N0 - 1 + LD : u + L;
    };
#pragma unroll
    for (int u = 0; u < NX; ++u) {
#pragma unroll
      for (int x = hi(u - 1) + 1; x <= hi(u); ++x) load(x);
      if (u == N0) {
#pragma unroll
        for (int smt = 0; smt < 2; ++smt) sacc[smt] = pacc[smt] = f32x16{};
      }
      if (u < N0) {
        dqacc[u % (D / 32)] = E::mfma32(op[u], bs[u / (D / 32)], dqacc[u % (D / 32)]);
      } else {
        const int x = (u - N0) >> 1;
        if ((u - N0) & 1)
          pacc[x & 1] = E::mfma32(op[u], df[x >> 1], pacc[x & 1]);
        else
          sacc[x & 1] = E::mfma32(op[u], qf[x >> 1], sacc[x & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // VALU phase of chunk j: dS^T, packed 16 keys at a time
  auto valu = [&](int nv) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      float dsv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * (kk & 1) + e;
        const float p = fast_exp2(fmaf(sacc[kk >> 1][i], c2, -my_lse));
        dsv[e] = p * (pacc[kk >> 1][i] - my_delta);
      }
      if (nv < C::KC) {
        // key (kk >> 1)*32 + 8(i >> 2) + (i & 3) + 4h >= nv, compared as 4h >=
        // nv - (its constant part) on a count re-read inside the branch (no
        // comparison hoisted out of the branch into every chunk)
        const int nvl = uniform_here(nv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 8 * (kk & 1) + e;
          if (4 * h >= nvl - ((kk >> 1) * 32 + 8 * (i >> 2) + (i & 3))) dsv[e] = 0.f;
        }
      }
      bs[kk] = pack8<T>(dsv);
    }
  };
  auto phase_barrier = []() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  using NoDq = std::integral_constant<bool, false>;
  using WithDq = std::integral_constant<bool, true>;

  // The sequence and the ring protocol of sparse_fwd_pp_kernel: chunk j+1 is
  // published by the second barrier of group 0's iteration j; the stage of
  // chunk j+2 last held chunk j-2, whose last reader (group 1's MFMA phase of
  // chunk j-1, the K^T of the dQ product) finished before the first barrier
  // of iteration j.
  int nvm1 = 0;
  int nv0 = issue(0);
  int nv1 = issue(1);
  if (nv1 > 0)
    wait_vmcnt<2 * TileDma<T, D, C::KC, C::NT>::N>();
  else
    dma_wait();
  if (grp1) phase_barrier();
  if (nv0 > 0) {
    phase_barrier();
    mfma_priority_up();
    mma_x(0, 0, NoDq{});
    mfma_priority_down();
    dma_wait();  // this wave's copies of chunk 1
    phase_barrier();
    int nv2 = issue(2);
    int fin = nv0;  // valid keys of the chunk whose VALU phase is pending
    nvm1 = nv0;
    nv0 = nv1;
    nv1 = nv2;
    // chunks 1 .. n; at j = n (no chunk j) S and dP run on a stage no copy is
    // writing and their results are not used.  An iteration opens with the
    // VALU phase of chunk j-1, so the operands prefetched at its end stay
    // inside one iteration.
    for (int j = 1; nvm1 > 0; ++j) {
      if (fin > 0) valu(fin);
      prefetch((j - 1) % C::NS);
      phase_barrier();
      mfma_priority_up();
      mma_x(j % C::NS, (j - 1) % C::NS, WithDq{});
      mfma_priority_down();
      dma_wait();  // this wave's copies of chunk j+1
      phase_barrier();
      nv2 = issue((j + 2) % C::NS);
      fin = nv0;
      nvm1 = nv0;
      nv0 = nv1;
      nv1 = nv2;
    }
  }
  if (!grp1) phase_barrier();
  dq_epilogue<T, D, BE, RASTER>(dqacc, b, myq, qblk, h, sq, qb, dq, dqc, q_vbs, scale, orows,
                                s_out, heads);
}

// Persistent, with the query-block walk of sparse_fwd_pp_kernel.
template <typename T, int D, bool RASTER>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sparse_dq_pp_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    const T* __restrict__ dout, const float* __restrict__ lse,
                    const float* __restrict__ delta, const int32_t* __restrict__ selected,
                    const int32_t* __restrict__ kv_vbs, T* __restrict__ dq,
                    const T* __restrict__ dqc, const int32_t* __restrict__ q_vbs, int num_tiles,
                    int sq, int skv, int qb, int kb, int topk, float c2, uint32_t qsign,
                    float scale, const int32_t* __restrict__ orows, int64_t s_out, int heads,
                    int32_t* __restrict__ ctr) {
  using C = DqPPCfg<D>;
  __shared__ __attribute__((aligned(16))) T smem[C::NS * C::STAGE];
  __shared__ int s_next;
  const int xcd = blockIdx.x & 7, per = (num_tiles + 7) >> 3, stride = (int)(gridDim.x >> 3);
  int from = 0;
  for (int round = 0;; ++round) {
    int tile;
    if (ctr) {  // as in sparse_fwd_pp_kernel
      if (threadIdx.x == 0) s_next = take_entry(ctr, xcd, per, from, 8);
      __syncthreads();
      const int e = s_next;
      if (e < 0) break;
      tile = (e & 7) * per + (e >> 3);
    } else {
      const int j = (int)(blockIdx.x >> 3) + round * stride;
      if (j >= per) break;
      tile = xcd * per + j;
    }
    if (tile < num_tiles)
      dq_pp_tile<T, D, RASTER>(smem, tile, q, k, v, dout, lse, delta, selected, kv_vbs, dq, dqc,
                               q_vbs, sq, skv, qb, kb, topk, c2, qsign, scale, orows, s_out, heads);
    // No copy is in flight here (each chunk's copies are waited for before it
    // is read, and past the route's end nothing is copied): only the
    // epilogue's stores are outstanding, and they drain under the next tile's
    // first loads.
    __syncthreads();  // every wave is done with the LDS ring (and s_next) before the next tile
  }
  if (ctr && threadIdx.x == 0) finish_entries(ctr);
}

template <typename T, int D, bool RASTER = false>
static int launch_dq_pp(const void* q, const void* k, const void* v, const void* dout,
                        const float* lse, const float* delta, const int32_t* selected,
                        const int32_t* kv_vbs, void* dq, const void* dqc, const int32_t* q_vbs,
                        int64_t bh, int64_t sq, int64_t skv, int topk, float scale,
                        hipStream_t stream, const int32_t* orows = nullptr, int64_t s_out = 0, int heads = 0) {
  const int64_t tiles = bh * (sq / 256);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int64_t want = ((tiles + 7) / 8) * 8;
  const int resident = (cu_count() / 8) * 8;  // one 8-wave workgroup per CU
  const int grid = (int)(want < resident ? want : resident);
  hipLaunchKernelGGL((sparse_dq_pp_kernel<T, D, RASTER>), dim3(grid), dim3(512), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, selected,
                     kv_vbs, (T*)dq, (const T*)dqc, q_vbs, (int)tiles, (int)sq, (int)skv,
                     (int)(sq / 256), (int)(skv / 256), topk, fabsf(scale) * kLog2e,
                     scale < 0.f ? 0x80008000u : 0u, scale, orows, s_out, heads,
                     sched_counters(stream));
  return vsa_check_launch();
}

template <typename T, int D, int BE, bool RASTER = false>
static int launch_dq(const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, const float* delta, const int32_t* selected,
                     const int32_t* kv_vbs, void* dq, const void* dqc, const int32_t* q_vbs,
                     int64_t bh, int64_t sq, int64_t skv, int topk, float scale,
                     hipStream_t stream, const int32_t* orows = nullptr, int64_t s_out = 0, int heads = 0) {
  using C = DqCfg<D, BE>;
  const int tph = (int)(sq / C::QT);
  const int64_t tiles = bh * tph;
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int grid = (int)(((tiles + 7) / 8) * 8);
  hipLaunchKernelGGL((sparse_dq_kernel<T, D, BE, RASTER>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, selected,
                     kv_vbs, (T*)dq, (const T*)dqc, q_vbs, (int)tiles, tph, (int)sq, (int)skv,
                     (int)(sq / BE), (int)(skv / BE), topk, fabsf(scale) * kLog2e,
                     scale < 0.f ? 0x80008000u : 0u, scale, orows, s_out, heads);
  return vsa_check_launch();
}

template <typename T, int D, int BE, bool RASTER = false>
static int launch_dkdv(const void* q, const void* k, const void* v, const void* dout,
                       const float* lse, const float* delta, const int32_t* counts,
                       const int32_t* offsets, const int32_t* inverse, const int32_t* kv_vbs,
                       void* dk, void* dv, const void* dkc, const void* dvc, int64_t bh,
                       int64_t sq, int64_t skv, int topk, float scale, int32_t* tile_order,
                       hipStream_t stream, const int32_t* orows = nullptr, int64_t s_out = 0, int heads = 0) {
  using C = DkvCfg<D, BE>;
  const int tph = (int)(skv / C::KT);
  const int64_t tiles = bh * tph * C::NSPLIT;
  if (tiles >= kLongestFirst) return VSA_ERR_SHAPE;  // entries keep the tag bit free
  // persistent: the workgroups the CUs hold at once (WPE waves per SIMD), at
  // most one per tile, a multiple of 8 (the XCD count)
  const int resident = cu_count() * C::WG_PER_CU;
  const int64_t want = ((tiles + 7) / 8) * 8;
  const int grid = C::NSPLIT > 1 || want < resident ? (int)want : (resident / 8) * 8;
  hipLaunchKernelGGL((sparse_dkdv_kernel<T, D, BE, RASTER>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, counts,
                     offsets, inverse, kv_vbs, (T*)dk, (T*)dv, (const T*)dkc, (const T*)dvc,
                     (int)tiles, tph, (int)sq, (int)skv, (int)(sq / BE), (int)(skv / BE), topk,
                     fabsf(scale) * kLog2e, scale < 0.f ? 0x80008000u : 0u, scale, tile_order,
                     orows, s_out, heads);
  return vsa_check_launch();
}

// ---------------------------------------------------------------------------
// dK/dV tile order.  A dK/dV workgroup's work is proportional to the CSR
// in-edge count of its key block.  One workgroup per XCD range (the tiles
// xcd_tile gives XCD x) lists the range for the persistent workgroups:
//  * skewed routes (its largest tile exceeds a quarter of what each concurrent
//    workgroup slot of the XCD gets on average): longest-first, by a counting
//    sort on the edge count, so that the hot key blocks start first instead of
//    setting the kernel's end; these entries carry the kLongestFirst tag;
//  * otherwise in index order (the two 128-key tiles of a 256-key block, and a
//    head's neighbouring blocks, which share most query blocks, run together
//    and meet their Q / dO rows in L2), except that the range's smallest tiles
//    (at most kTailSlots per workgroup slot) are moved to the end, still in
//    index order: the last tiles a workgroup takes are then short, and the
//    workgroups of the XCD finish close together.
// Workgroup i of the dK/dV grid then takes tile_order[i].  Only the dispatch
// order changes: every tile computes the same values, so the order inside a
// count bin (set by LDS atomics) does not reach the results.
// ---------------------------------------------------------------------------
constexpr int kOrderBins = 1024;  // edge counts >= 1023 share the top bin
constexpr int kTailSlots = 4;

// block-wide exclusive prefix sum of one int per thread (1024 threads); the
// block total is returned in total
__device__ __forceinline__ int block_exclusive_sum(int v, int* wtot, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = 0;
  total = 0;
  for (int w = 0; w < 16; ++w) {
    if (w < wave) base += wtot[w];
    total += wtot[w];
  }
  __syncthreads();  // wtot may be reused by the next call
  return base + incl - v;
}

__global__ __launch_bounds__(1024) void dkdv_order_kernel(const int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ order,
                                                          int num_tiles, int per, int tph,
                                                          int tpb, int nsplit, int kb,
                                                          int slots) {
  __shared__ int bin[kOrderBins];
  __shared__ long long rsum[16];
  __shared__ int rmax[16];
  __shared__ int wtot[16];
  __shared__ int s_cut;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int x = blockIdx.x;
  const int lo = x * per, n = max(0, min(per, num_tiles - lo));
  // the scheduling counters sparse_dkdv_kernel advances: one per range, then
  // the finished-workgroup count
  if (tid == 0) order[8 * per + x] = 0;
  if (tid == 0 && x == 0) order[8 * per + 8] = 0;
  auto nedge_raw = [&](int j) {
    const int tile = (lo + j) / nsplit;
    return counts[(int64_t)(tile / tph) * kb + (tile % tph) / tpb];
  };
  auto nedge_of = [&](int j) { return min(nedge_raw(j), kOrderBins - 1); };  // its bin
  long long sum = 0;
  int mx = 0;
  for (int j = tid; j < n; j += 1024) {
    const int e = nedge_raw(j);
    sum += e;
    mx = max(mx, e);
  }
  for (int o = 32; o > 0; o >>= 1) {
    sum += __shfl_xor(sum, o, 64);
    mx = max(mx, __shfl_xor(mx, o, 64));
  }
  if (lane == 0) {
    rsum[wave] = sum;
    rmax[wave] = mx;
  }
  bin[tid] = 0;
  if (tid == 0) s_cut = -1;
  __syncthreads();
  sum = 0;
  mx = 0;
  for (int w = 0; w < 16; ++w) {
    sum += rsum[w];
    mx = max(mx, rmax[w]);
  }
  const bool skewed = (long long)mx * slots * 4 > sum;
  for (int j = tid; j < n; j += 1024) atomicAdd(&bin[nedge_of(j)], 1);
  __syncthreads();
  // bin[b] becomes the number of tiles with a larger edge count (the start of
  // bin b in descending order); thread t holds bin K-1-t
  {
    const int c = bin[kOrderBins - 1 - tid];
    int total;
    const int before = block_exclusive_sum(c, wtot, total);
    bin[kOrderBins - 1 - tid] = before;
  }
  __syncthreads();
  if (skewed) {
    for (int j = tid; j < n; j += 1024) {
      const int pos = atomicAdd(&bin[nedge_of(j)], 1);
      order[x + 8 * pos] = (lo + j) | kLongestFirst;
    }
  } else {
    // the cut: the largest edge count c with at most kTailSlots * slots tiles
    // of count <= c (-1: none, the whole range stays in index order)
    const int tail_max = kTailSlots * slots;
    {
      const int b = tid;
      const int le = n - bin[b];                                   // tiles with count <= b
      const int le_next = b + 1 < kOrderBins ? n - bin[b + 1] : n + tail_max + 1;
      if (le <= tail_max && le_next > tail_max) s_cut = b;
    }
    __syncthreads();
    const int cut = s_cut;
    const int nbulk = cut < 0 ? n : bin[cut];   // tiles with count > cut
    int carry = 0;                              // bulk tiles before this chunk
    for (int j0 = 0; j0 < n; j0 += 1024) {
      const int j = j0 + tid;
      const int f = (j < n && nedge_of(j) > cut) ? 1 : 0;
      int total;
      const int pre = carry + block_exclusive_sum(f, wtot, total);
      if (j < n) order[x + 8 * (f ? pre : nbulk + (j - pre))] = lo + j;
      carry += total;
    }
  }
  for (int j = n + tid; j < per; j += 1024) order[x + 8 * j] = num_tiles | (skewed ? kLongestFirst : 0);
}

// dK/dV grid geometry of the MFMA kernels for (head_dim, block volume): tiles
// per (b, h) and per key block, the head-dim split and the workgroups one CU
// runs at a time
struct DkvGeometry {
  int tph, tpb, nsplit, wg_per_cu;
};
template <int D, int BE>
static void dkdv_geometry_of(int64_t skv, DkvGeometry& g) {
  using C = DkvCfg<D, BE>;
  g.tph = (int)(skv / C::KT);
  g.tpb = BE / C::KT;
  g.nsplit = C::NSPLIT;
  g.wg_per_cu = C::WG_PER_CU;
}
static bool dkdv_geometry(int D, int be, int64_t skv, DkvGeometry& g) {
#define VSA_GEO_CASE(DD, BB)            \
  if (D == DD && be == BB) {            \
    dkdv_geometry_of<DD, BB>(skv, g);   \
    return true;                        \
  }
  VSA_GEO_CASE(64, 64) VSA_GEO_CASE(64, 128) VSA_GEO_CASE(64, 256)
  VSA_GEO_CASE(128, 64) VSA_GEO_CASE(128, 128) VSA_GEO_CASE(128, 256)
  VSA_GEO_CASE(256, 64) VSA_GEO_CASE(256, 128) VSA_GEO_CASE(256, 256)
#undef VSA_GEO_CASE
  return false;
}

}  // namespace vsa

using namespace vsa;

#define VSA_BWD_SHAPES(X) \
  X(128, 256) X(128, 128) X(128, 64) X(64, 256) X(64, 128) X(64, 64) X(256, 256) X(256, 128) X(256, 64)

extern "C" int vsa_sparse_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                                 const float* lse, const float* delta, const int32_t* selected,
                                 const int32_t* kv_vbs, void* dq, const void* d_q_c,
                                 const int32_t* q_vbs, int64_t bh, int64_t sq, int64_t skv,
                                 int32_t D, int32_t be, int32_t topk, float scale, int32_t dtype,
                                 void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !selected || !kv_vbs || !dq) return VSA_ERR_NULL;
  if (d_q_c && !q_vbs) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, dout, dq, d_q_c) || !vsa_aligned<4>(lse, delta, selected, kv_vbs, q_vbs))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VSA_F32)
    return sparse_dq_f32(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c, q_vbs, bh, sq,
                         skv, D, be, topk, scale, s);
#ifndef VSA_DQ_NO_PP
  // one 8-wave workgroup per query block once every CU gets one, at head dim
  // 128; at head dim 64 the 4-wave kernel is faster (block 256, 40 960 tokens,
  // 24 heads: 1.98 against 2.03 ms at topk 20, 1.02 against 1.08 at topk 10;
  // at head dim 128 the 8-wave kernel leads, 4.92 against 5.85 ms)
  if (be == 256 && bh * (sq / 256) >= 256 && D == 128 &&
      (dtype == VSA_BF16 || dtype == VSA_F16)) {
    if (dtype == VSA_BF16)
      return launch_dq_pp<__bf16, 128>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c,
                                        q_vbs, bh, sq, skv, topk, scale, s);
    return launch_dq_pp<_Float16, 128>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c,
                                        q_vbs, bh, sq, skv, topk, scale, s);
  }
#endif
#define VSA_DQ_CASE(DD, BB)                                                                  \
  if (D == DD && be == BB)                                                                   \
    return launch_dq<T, DD, BB>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c, q_vbs, \
                                bh, sq, skv, topk, scale, s);
  VSA_DISPATCH_MFMA(dtype, T, { VSA_BWD_SHAPES(VSA_DQ_CASE) });
#undef VSA_DQ_CASE
  return VSA_ERR_UNSUPPORTED;
}

extern "C" int vsa_dkdv_tile_order(const int32_t* counts, int32_t* tile_order,
                                   int64_t order_len, int64_t bh, int64_t skv, int32_t D,
                                   int32_t be, void* stream) {
  if (!counts || !tile_order) return VSA_ERR_NULL;
  if (!vsa_aligned<4>(counts, tile_order)) return VSA_ERR_ALIGN;
  DkvGeometry g;
  if (bh <= 0 || skv <= 0 || be <= 0 || skv % be) return VSA_ERR_SHAPE;
  if (!dkdv_geometry(D, be, skv, g)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * g.tph * g.nsplit;
  const int64_t per = (tiles + 7) / 8;
  if (tiles >= kLongestFirst || order_len < 8 * per + 16) return VSA_ERR_SHAPE;
  hipLaunchKernelGGL(dkdv_order_kernel, dim3(8), dim3(1024), 0, (hipStream_t)stream, counts,
                     tile_order, (int)tiles, (int)per, g.tph, g.tpb, g.nsplit,
                     (int)(skv / be), 32 * g.wg_per_cu);
  return vsa_check_launch();
}

extern "C" int vsa_sparse_bwd_dkdv(const void* q, const void* k, const void* v,
                                   const void* dout, const float* lse, const float* delta,
                                   const int32_t* counts, const int32_t* offsets,
                                   const int32_t* inverse, const int32_t* kv_vbs, void* dk,
                                   void* dv, const void* d_k_c, const void* d_v_c, int64_t bh,
                                   int64_t sq, int64_t skv, int32_t D, int32_t be, int32_t topk,
                                   float scale, int32_t* tile_order, int32_t dtype,
                                   void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !counts || !offsets || !inverse || !kv_vbs ||
      !dk || !dv)
    return VSA_ERR_NULL;
  if ((d_k_c == nullptr) != (d_v_c == nullptr)) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, dout, dk, dv, d_k_c, d_v_c) ||
      !vsa_aligned<4>(lse, delta, counts, offsets, inverse, kv_vbs, tile_order))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VSA_F32)
    return sparse_dkdv_f32(q, k, v, dout, lse, delta, counts, offsets, inverse, kv_vbs, dk, dv,
                           d_k_c, d_v_c, bh, sq, skv, D, be, topk, scale, s);
#define VSA_DKDV_CASE(DD, BB)                                                                \
  if (D == DD && be == BB)                                                                   \
    return launch_dkdv<T, DD, BB>(q, k, v, dout, lse, delta, counts, offsets, inverse,       \
                                  kv_vbs, dk, dv, d_k_c, d_v_c, bh, sq, skv, topk, scale, \
                                  tile_order, s);
  VSA_DISPATCH_MFMA(dtype, T, { VSA_BWD_SHAPES(VSA_DKDV_CASE) });
#undef VSA_DKDV_CASE
  return VSA_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// dK/dV without a caller workspace.  The tile order and scheduling counters
// live in a file-scope device array: one copy per GPU, held until the process
// ends.  Host code never passes the array's name to a kernel (on the host it
// is only a stand-in for the symbol): each device's address comes from
// hipGetSymbolAddress, resolved once per device with that device current.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchInts = 1 << 18;  // 1 MiB of int32
static __device__ __align__(256) int32_t scratch[kNoAllocScratchInts];

namespace {
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[64] = {nullptr};

// The current device's copy of `scratch` (nullptr if it cannot be resolved).
int32_t* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return nullptr;
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int vsa_sparse_bwd_dkdv_noalloc(const void* q, const void* k, const void* v,
                                           const void* dout, const float* lse,
                                           const float* delta, const int32_t* counts,
                                           const int32_t* offsets, const int32_t* inverse,
                                           const int32_t* kv_vbs, void* dk, void* dv,
                                           const void* d_k_c, const void* d_v_c, int64_t bh,
                                           int64_t sq, int64_t skv, int32_t D, int32_t be,
                                           int32_t topk, float scale, int32_t dtype,
                                           void* stream) {
  if (dtype == VSA_F32)  // the fp32 kernels use no scheduling workspace
    return vsa_sparse_bwd_dkdv(q, k, v, dout, lse, delta, counts, offsets, inverse, kv_vbs, dk,
                               dv, d_k_c, d_v_c, bh, sq, skv, D, be, topk, scale, nullptr, dtype,
                               stream);
  if (dtype != VSA_BF16 && dtype != VSA_F16) return VSA_ERR_DTYPE;
  // the checks of vsa_sparse_bwd_dkdv, made before the order kernel launches
  if (!q || !k || !v || !dout || !lse || !delta || !counts || !offsets || !inverse || !kv_vbs ||
      !dk || !dv)
    return VSA_ERR_NULL;
  if ((d_k_c == nullptr) != (d_v_c == nullptr)) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, dout, dk, dv, d_k_c, d_v_c) ||
      !vsa_aligned<4>(lse, delta, counts, offsets, inverse, kv_vbs))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  DkvGeometry g;
  if (!dkdv_geometry(D, be, skv, g)) return VSA_ERR_UNSUPPORTED;
  const int64_t tiles = bh * g.tph * g.nsplit;
  const int64_t order_len = 8 * ((tiles + 7) / 8) + 16;
  if (tiles >= kLongestFirst || order_len > kNoAllocScratchInts) return VSA_ERR_TOO_LARGE;
  // the scratch is the current device's: the stream must launch there too
  if (stream != nullptr) {
    int dev = 0;
    hipDevice_t sdev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess)
      return VSA_ERR_LAUNCH;
    if (sdev != dev) return VSA_ERR_DEVICE;
  }
  int32_t* order = device_scratch();
  if (order == nullptr) return VSA_ERR_LAUNCH;
  // the order call rewrites every entry the dK/dV kernel reads and zeroes its
  // counters, so the previous call's contents do not matter
  int rc = vsa_dkdv_tile_order(counts, order, order_len, bh, skv, D, be, stream);
  if (rc != VSA_OK) return rc;
  return vsa_sparse_bwd_dkdv(q, k, v, dout, lse, delta, counts, offsets, inverse, kv_vbs, dk,
                             dv, d_k_c, d_v_c, bh, sq, skv, D, be, topk, scale, order, dtype,
                             stream);
}

// ---------------------------------------------------------------------------
// Tiled-sequence variants: q, k, v, dout in the padded tile layout (as the
// forward's tile pass wrote them), dq / dk / dv written straight to a
// raster-order sequence of s_out tokens through slot_rows (tiled slot ->
// raster row, -1 for a padding slot), which is what untile() of the tiled
// gradients would produce for the real tokens.  bf16 / fp16, head dims 64 and
// 128, blocks of 64, 128 and 256 tokens.
// ---------------------------------------------------------------------------
#define VSA_TILED_SHAPES(X) X(128, 256) X(128, 128) X(128, 64) X(64, 256) X(64, 128) X(64, 64)

extern "C" int vsa_sparse_bwd_dq_tiled(const void* q, const void* k, const void* v,
                                       const void* dout, const float* lse, const float* delta,
                                       const int32_t* selected, const int32_t* kv_vbs, void* dq,
                                       const void* d_q_c, const int32_t* q_vbs,
                                       const int32_t* slot_rows, int64_t s_out, int32_t heads, int64_t bh,
                                       int64_t sq, int64_t skv, int32_t D, int32_t be,
                                       int32_t topk, float scale, int32_t dtype, void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !selected || !kv_vbs || !dq || !slot_rows)
    return VSA_ERR_NULL;
  if (d_q_c && !q_vbs) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, dout, dq, d_q_c) ||
      !vsa_aligned<4>(lse, delta, selected, kv_vbs, q_vbs, slot_rows))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      s_out <= 0 || s_out > sq || sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  if (heads < 0 || (heads > 0 && bh % heads)) return VSA_ERR_SHAPE;
  if (dtype != VSA_BF16 && dtype != VSA_F16) return dtype == VSA_F32 ? VSA_ERR_UNSUPPORTED : VSA_ERR_DTYPE;
  hipStream_t s = (hipStream_t)stream;
#define VSA_DQ_TILED_CASE(DD, BB)                                                            \
  if (D == DD && be == BB) {                                                                 \
    if (BB == 256 && DD == 128 && bh * (sq / 256) >= 256)                                    \
      return launch_dq_pp<T, DD, true>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c, \
                                       q_vbs, bh, sq, skv, topk, scale, s, slot_rows, s_out, heads); \
    return launch_dq<T, DD, BB, true>(q, k, v, dout, lse, delta, selected, kv_vbs, dq, d_q_c, \
                                      q_vbs, bh, sq, skv, topk, scale, s, slot_rows, s_out, heads);  \
  }
  VSA_DISPATCH_MFMA(dtype, T, { VSA_TILED_SHAPES(VSA_DQ_TILED_CASE) });
#undef VSA_DQ_TILED_CASE
  return VSA_ERR_UNSUPPORTED;
}

extern "C" int vsa_sparse_bwd_dkdv_tiled(const void* q, const void* k, const void* v,
                                         const void* dout, const float* lse, const float* delta,
                                         const int32_t* counts, const int32_t* offsets,
                                         const int32_t* inverse, const int32_t* kv_vbs, void* dk,
                                         void* dv, const void* d_k_c, const void* d_v_c,
                                         const int32_t* slot_rows, int64_t s_out, int32_t heads, int64_t bh,
                                         int64_t sq, int64_t skv, int32_t D, int32_t be,
                                         int32_t topk, float scale, int32_t* tile_order,
                                         int32_t dtype, void* stream) {
  if (!q || !k || !v || !dout || !lse || !delta || !counts || !offsets || !inverse || !kv_vbs ||
      !dk || !dv || !slot_rows)
    return VSA_ERR_NULL;
  if ((d_k_c == nullptr) != (d_v_c == nullptr)) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, dout, dk, dv, d_k_c, d_v_c) ||
      !vsa_aligned<4>(lse, delta, counts, offsets, inverse, kv_vbs, slot_rows, tile_order))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      s_out <= 0 || s_out > skv || sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  if (heads < 0 || (heads > 0 && bh % heads)) return VSA_ERR_SHAPE;
  if (dtype != VSA_BF16 && dtype != VSA_F16) return dtype == VSA_F32 ? VSA_ERR_UNSUPPORTED : VSA_ERR_DTYPE;
  hipStream_t s = (hipStream_t)stream;
#define VSA_DKDV_TILED_CASE(DD, BB)                                                          \
  if (D == DD && be == BB)                                                                   \
    return launch_dkdv<T, DD, BB, true>(q, k, v, dout, lse, delta, counts, offsets, inverse, \
                                        kv_vbs, dk, dv, d_k_c, d_v_c, bh, sq, skv, topk,     \
                                        scale, tile_order, s, slot_rows, s_out, heads);
  VSA_DISPATCH_MFMA(dtype, T, { VSA_TILED_SHAPES(VSA_DKDV_TILED_CASE) });
#undef VSA_DKDV_TILED_CASE
  return VSA_ERR_UNSUPPORTED;
}
