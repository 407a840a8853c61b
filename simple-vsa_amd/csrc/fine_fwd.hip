// Sparse fine forward on gfx950 MFMA, with the combine fused into the epilogue.
//
// Reference contract: _triton_sparse_attention_forward (triton_impl.py:358-473)
// and its kernels (39-355); combine: fused_common.py:175-199.
//
// Work decomposition: one workgroup owns QT query rows of one (b, h) (QT = 128
// for block volume >= 128, else the block), one wave owns 32 of them.  The
// workgroup walks the selected KV blocks of its query block in KC-key chunks
// (64 keys; 32 for head_dim 128 with 64-token blocks);
// every chunk is copied once into LDS (direct global->LDS loads) as two
// swizzled row-major tiles (K and V) shared by all waves; the next chunk's
// copy is in flight while the current chunk is multiplied (double-buffered
// LDS, one barrier per chunk).
//
// Per wave and chunk:
//   S^T (KC x 32)  = K (KC x D) . Q^T (D x 32)           A = K from LDS, B = Q in VGPRs
//   online softmax per query (each lane owns one query: column r of S^T)
//   O^T (D x 32)  += V^T (D x KC) . P^T (KC x 32)        A = V^T by transpose reads, B = P
// Holding S and O transposed keeps the softmax statistics and the O rescale
// lane-local; only the row max crosses the two lane halves.  The running max
// is only moved when a chunk exceeds it by more than 2^kRescaleSlack (the
// exponentials stay <= 2^8, exact in fp32 and within bf16 range), so the O
// rescale runs on a few chunks instead of most.
#include <type_traits>

#include "fine_f32.h"
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

template <int D, int BE>
struct FwdCfg {
  static constexpr int QT = BE >= 128 ? 128 : BE;  // queries per workgroup
  static constexpr int NW = QT / 32;               // waves per workgroup
  static constexpr int NT = NW * 64;
  // keys per chunk: 32 at block 64, so that a 2-wave workgroup's double buffer
  // is 32 KiB at head_dim 128 (four workgroups share a CU) and 16 KiB at 64
  // (twice the resident waves of 64-key chunks: c5 forward 0.88 -> 0.78 ms,
  // dQ 0.93 -> 0.89 ms)
  static constexpr int KC = BE == 64 ? 32 : 64;
  static constexpr int NSM = KC / 32;              // 32-key sub-tiles per chunk
  // waves per SIMD the registers are sized for: head_dim 256 (Q fragments and
  // O accumulators alone take 192 registers) runs one wave per SIMD
  static constexpr int WPE = D == 256 ? 1 : 2;
  static constexpr int TILE = KC * D;              // elements of one K (or V) chunk
  static constexpr int STAGE = 2 * TILE;           // K and V
};

constexpr float kRescaleSlack = 8.0f;  // log2 units

// Normalise, fused combine, store, LSE (one lane = one query row, holding
// O^T column r and a partial row sum).  With RASTER the combined output and
// the gate are rows of a raster-order sequence of s_out tokens: slot myq of
// the tiled layout is raster row orows[myq] (< 0 for a padding slot, which
// has no output row); the fine output and the LSE stay in the tiled layout.
template <typename T, int D, bool RASTER = false>
__device__ __forceinline__ void fwd_epilogue(const f32x16 (&oacc)[D / 32], float lsum, float m,
                                             int64_t b, int myq, int qblk, int h, int sq, int qb,
                                             T* __restrict__ out, T* __restrict__ fine, float* __restrict__ lse,
                                             const T* __restrict__ outc,
                                             const T* __restrict__ gate, int gate_mode,
                                             int gate_heads, const int32_t* __restrict__ orows = nullptr,
                                             int64_t s_out = 0, int heads = 0) {
  using E = Elem<T>;
  const float ltot = pair_sum32(lsum);
  const float inv = 1.0f / ltot;
  const int64_t tok = (int64_t)b * sq + myq;
  int64_t otok = tok;  // row of the combined output and of the gate
  if constexpr (RASTER) {
    const int r = orows[myq];
    otok = (r >= 0 && r < s_out) ? raster_row(b, r, s_out, heads) : -1;
  }
  const bool ostore = !RASTER || otok >= 0;
  const T* ocrow = outc ? outc + ((int64_t)b * qb + qblk) * D : nullptr;
  float gtok = 1.f;
  if (outc && gate_mode == 2 && ostore) gtok = E::to_f(gate[otok]);
  // gate row of this token: [BH, Sq, D] (mode 1) or token-major [B, Sq, H, D] (mode 3)
  const T* grow = nullptr;
  if (gate_mode == 1 && ostore) grow = gate + otok * D;
  if (!RASTER && gate_mode == 3)
    grow = gate + (((int64_t)(b / gate_heads) * sq + myq) * gate_heads + b % gate_heads) * D;
  // The row regrouped so that every global access below is 16 bytes wide (half
  // the memory instructions of the accumulator's 8-byte pieces): after
  // swap_rows16, w[p][i] is dim mt*32 + 8(2p + h) + i.  The combine operands
  // are loaded first, together, so their latency is paid once.
  u32x4 ocr[D / 32][2], gr[D / 32][2];
  if (ocrow) {
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        ocr[mt][p] = *reinterpret_cast<const u32x4*>(ocrow + mt * 32 + 16 * p + 8 * h);
  }
  if (grow) {
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        gr[mt][p] = *reinterpret_cast<const u32x4*>(grow + mt * 32 + 16 * p + 8 * h);
  }
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
    float w[2][8];
    swap_rows16(oacc[mt], inv, w);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d0 = mt * 32 + 16 * p + 8 * h;
      float val[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) val[e] = w[p][e];
      if (ocrow) {
        const T* oc = reinterpret_cast<const T*>(&ocr[mt][p]);
        float gv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[e] = gtok;
        if (grow) {
          const T* gg = reinterpret_cast<const T*>(&gr[mt][p]);
#pragma unroll
          for (int e = 0; e < 8; ++e) gv[e] = E::to_f(gg[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) val[e] = fmaf(E::to_f(oc[e]), gv[e], val[e]);
      }
      T o8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o8[e] = E::from_f(val[e]);
      if (ostore) *reinterpret_cast<u32x4*>(out + otok * D + d0) = *reinterpret_cast<const u32x4*>(o8);
      if (ocrow && fine) {  // the fine output as stored in T, for the backward's delta
        T f8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f8[e] = E::from_f(w[p][e]);
        *reinterpret_cast<u32x4*>(fine + tok * D + d0) = *reinterpret_cast<const u32x4*>(f8);
      }
    }
  }
  // stored last: a load issued after a store also waits for that store
  if (lse != nullptr && h == 0) lse[tok] = m + log2f(ltot);
}

template <typename T, int D, int BE, bool RASTER>
__global__ __launch_bounds__((FwdCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(FwdCfg<D, BE>::WPE))) void sparse_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ out, T* __restrict__ fine, float* __restrict__ lse, const T* __restrict__ outc,
    const T* __restrict__ gate, int gate_mode, int gate_heads, int num_tiles, int tiles_per_head, int sq,
    int skv, int qb, int kb, int topk, float c2, uint32_t qsign, const int32_t* __restrict__ orows,
    int64_t s_out, int heads) {
  using C = FwdCfg<D, BE>;
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

  // Q^T fragments: lane (r, h) holds query r, dims 16*ks + 8h .. +7.
  V8 qf[D / 16];
  {
    const T* qrow = q + ((int64_t)b * sq + myq) * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + 16 * ks);
      raw ^= qsign;  // negative softmax scale folded into q
      qf[ks] = as_vec8<T>(raw);
    }
  }

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

  float m = -INFINITY;  // running max in log2 units (scaled)
  float lsum = 0.f;     // per-lane partial row sum
  f32x16 oacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) oacc[mt] = f32x16{};

  // Per-lane LDS byte offsets inside a tile, set once: the swizzle repeats
  // every 16 rows, so the K rows of key 32*smt + r sit at row_off[ks] +
  // 32*smt*D*2 and the transposed V pieces of keys 16*kk + .. at
  // tr_off[mt][hi] + 16*kk*D*2 (the offsets row_a8 / tr_a8 compute; left to
  // the compiler, that swizzle arithmetic was redone for every chunk).
  uint32_t row_off[D / 16], tr_off[D / 32][2];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) row_off[ks] = opaque((uint32_t)(swz<D>(r, 2 * ks + h) * sizeof(T)));
  {
    const int grp = lane >> 4, jl = lane & 15, qq = grp & 1, hh = grp >> 1;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi)
        tr_off[mt][hi] = opaque((uint32_t)(
            swz_elem<D>(8 * hi + 4 * hh + (jl >> 2), mt * 32 + 16 * qq + 4 * (jl & 3)) * sizeof(T)));
  }
  const char* smem_c = reinterpret_cast<const char*>(smem);
  auto k_row = [&](int stg, int ks, int smt) {
    return as_vec8<T>(*reinterpret_cast<const u32x4*>(smem_c + (stg * C::STAGE + smt * 32 * D) * (int)sizeof(T) +
                                                       row_off[ks]));
  };
  auto v_tr = [&](int stg, int mt, int kk) {
    const char* base = smem_c + (stg * C::STAGE + C::TILE + kk * 16 * D) * (int)sizeof(T);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][0]));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][1]));
    u32x4 rr;
    rr[0] = __builtin_bit_cast(u32x2, lo)[0];
    rr[1] = __builtin_bit_cast(u32x2, lo)[1];
    rr[2] = __builtin_bit_cast(u32x2, hi)[0];
    rr[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_vec8<T>(rr);
  };

  RouteRegs<BE, C::KC> route{sel, kv_vbs, topk, kb};
  route.load(0);
  int s = 0, ch = 0, kv = 0, nvb = 0;
  bool have = route.next(s, ch, kv, nvb);
  if (have) dma(kv, ch, 0);
  dma_wait();
  __syncthreads();
  // one chunk on stage stg (the loop below is unrolled by the two stages, so
  // that every LDS address is a lane offset plus an immediate)
  auto chunk = [&](auto stage_c) {
    constexpr int stage = decltype(stage_c)::value;
    const int nv = min(nvb - ch * C::KC, C::KC);
    int s2 = s, ch2 = ch + 1, kv2 = kv, nvb2 = nvb;
    const bool have2 = route.next(s2, ch2, kv2, nvb2);
    if (have2) dma(kv2, ch2, stage ^ 1);  // lands while this chunk is multiplied

    // ---- S^T = K Q^T -------------------------------------------------------
    f32x16 sacc[C::NSM];
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt) sacc[smt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int smt = 0; smt < C::NSM; ++smt)
        sacc[smt] = E::mfma32(k_row(stage, ks, smt), qf[ks], sacc[smt]);
    }
    // ---- online softmax (base 2, lazily rescaled) ---------------------------
    // Keys past nv get the score -inf.  At head_dim 64 the comparison is 4h >=
    // nv - (the key's constant part) on a count re-read inside the branch, so
    // it stays in the (rarely taken) branch: c5 forward -3.6 %.  At head dims
    // 128 / 256 the compiler hoists the comparisons of the plain form in
    // front of the branch, under the S products, and that form measured
    // faster there (t444 forward 7 % faster than with the branch-local one).
    if (nv < C::KC) {
      if constexpr (D == 64) {
        const int nvl = uniform_here(nv);
#pragma unroll
        for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (4 * h >= nvl - (smt * 32 + 8 * (i >> 2) + (i & 3))) sacc[smt][i] = -INFINITY;
      } else {
        keep_branch();
#pragma unroll
        for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3) >= nv) sacc[smt][i] = -INFINITY;
      }
    }
    float m4[4] = {sacc[0][0], sacc[0][1], sacc[0][2], sacc[0][3]};  // short chains
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) m4[i & 3] = vmax(m4[i & 3], sacc[smt][i]);
    float smax = vmax(vmax(m4[0], m4[1]), vmax(m4[2], m4[3]));
    smax = pair_max32(smax) * c2;
    // Only the lanes whose own chunk max passed the slack move their max (the
    // branch is wave-uniform, the update is not): a row's values then never
    // depend on the other rows of its wave, padding rows included.  A lane
    // that keeps m scales by exp2(0), exactly 1 (m is finite after the first
    // chunk, where every lane moves).
    const bool grow = smax > m + kRescaleSlack;
    if (__any(grow)) {
      const float mnew = grow ? smax : m;
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) oacc[mt] *= alpha;
      m = mnew;
    }
    float p[C::NSM][16];
    const float negm = -m;
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) p[smt][i] = fast_exp2(fmaf(sacc[smt][i], c2, negm));
    if (nv < C::KC) {  // as for the scores above
      if constexpr (D == 64) {
        const int nvl = uniform_here(nv);
#pragma unroll
        for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (4 * h >= nvl - (smt * 32 + 8 * (i >> 2) + (i & 3))) p[smt][i] = 0.f;
      } else {
        keep_branch();
#pragma unroll
        for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3) >= nv) p[smt][i] = 0.f;
      }
    }
    float l4[4] = {p[0][0], p[0][1], p[0][2], p[0][3]};  // chunk row sum in four short chains
#pragma unroll
    for (int x = 4; x < 16 * C::NSM; ++x) l4[x & 3] += p[x >> 4][x & 15];
    lsum += (l4[0] + l4[1]) + (l4[2] + l4[3]);
    // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
    for (int kk = 0; kk < 2 * C::NSM; ++kk) {
      const V8 bop = pack8<T>(&p[kk >> 1][8 * (kk & 1)]);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        oacc[mt] = E::mfma32(v_tr(stage, mt, kk), bop, oacc[mt]);
    }

    dma_wait();
    __syncthreads();
    s = s2; ch = ch2; kv = kv2; nvb = nvb2; have = have2;
  };
  while (have) {
    chunk(std::integral_constant<int, 0>{});
    if (!have) break;
    chunk(std::integral_constant<int, 1>{});
  }

  fwd_epilogue<T, D, RASTER>(oacc, lsum, m, b, myq, qblk, h, sq, qb, out, fine, lse, outc, gate,
                             gate_mode, gate_heads, orows, s_out, heads);
}

// ---------------------------------------------------------------------------
// Ping-pong forward for 256-token blocks.  One workgroup of 8 waves owns a whole
// query block; waves w and w+4 run on the same SIMD.  Group 0 (waves 0-3, rows
// 0-127) and group 1 (waves 4-7, rows 128-255) do the same per-chunk work half
// a phase apart, separated by workgroup barriers: while group 0 issues the
// MFMAs of chunk j (S_j, and O += V_{j-1} P_{j-1}), group 1 runs the softmax of
// chunk j-1; then group 0 runs the softmax of chunk j while group 1 issues the
// MFMAs of chunk j.
// On every SIMD one wave keeps the matrix core busy while the other uses the
// VALU (an MFMA and VALU work of another wave overlap on CDNA4).  Both groups
// read the same K/V chunks from a 4-stage LDS ring.
// Per query row the arithmetic and its order are those of sparse_fwd_kernel:
// the online-softmax rescale of chunk j follows the PV product of chunk j-1.
// ---------------------------------------------------------------------------
template <int D>
struct FwdPPCfg {
  static constexpr int NT = 512;
  static constexpr int KC = 64;
  static constexpr int TILE = KC * D;
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NS = 4;
  static constexpr int PER = 2 * (KC * D / 8 / NT);  // direct loads per wave per chunk
  // LDS ring: the NS K tiles first, then the NS V tiles.  With the chunk loop
  // unrolled by NS every operand read is a lane offset (one register, set up
  // once) plus an immediate below 64 KiB: the K tiles span 64 KiB from 0, and
  // the V region's start is folded into the transposed-read lane offsets.
  static constexpr int k_off(int stg) { return stg * TILE; }
  static constexpr int v_off(int stg) { return (NS + stg) * TILE; }
  static_assert(D > 128 || NS * TILE * 2 <= 65536, "K tiles addressed by 16-bit offsets");
};

// One query block (tile < bh * Sq / 256) of sparse_fwd_pp_kernel.
template <typename T, int D, bool RASTER>
__device__ __forceinline__ void fwd_pp_tile(
    T* smem, int tile, const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ out, T* __restrict__ fine, float* __restrict__ lse, const T* __restrict__ outc,
    const T* __restrict__ gate, int gate_mode, int gate_heads, int sq, int skv, int qb, int kb,
    int topk, float c2, uint32_t qsign, const int32_t* __restrict__ orows, int64_t s_out, int heads) {
  constexpr int BE = 256;
  using C = FwdPPCfg<D>;
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: group branches are scalar
  const int r = lane & 31, h = lane >> 5;
  const bool grp1 = wave >= 4;
  const int myq = qblk * BE + wave * 32 + r;

  V8 qf[D / 16];
  {
    const T* qrow = q + ((int64_t)b * sq + myq) * D + 8 * h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + 16 * ks);
      raw ^= qsign;
      qf[ks] = as_vec8<T>(raw);
    }
  }
  const int32_t* sel = selected + ((int64_t)b * qb + qblk) * topk;
  const T* kbase = k + (int64_t)b * skv * D;
  const T* vbase = v + (int64_t)b * skv * D;
  RouteRegs<BE, C::KC> route{sel, kv_vbs, topk, kb};
  route.load(0);
  TileDma<T, D, C::KC, C::NT> tdma;
  tdma.init();
  int ps = 0, pc = 0, pkv = 0, pnvb = 0;
  bool pvalid = route.next(ps, pc, pkv, pnvb);
  // Copy the cursor's chunk into stage stg; returns its valid keys (0: the
  // route is exhausted and nothing is copied).
  // the ring's LDS base, converted once (an address-space conversion inside
  // the loop also costs a null check per copy)
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  auto issue = [&](int stg) {
    int nv = 0;
    if (pvalid) {
      const int64_t off = ((int64_t)pkv * BE + pc * C::KC) * D;
      tdma.copy_lds(ring_lds + (uint32_t)(C::k_off(stg) * (int)sizeof(T)), kbase + off, wave);
      tdma.copy_lds(ring_lds + (uint32_t)(C::v_off(stg) * (int)sizeof(T)), vbase + off, wave);
      nv = min(pnvb - pc * C::KC, C::KC);
      ++pc;
      pvalid = route.next(ps, pc, pkv, pnvb);
    }
    return nv;
  };

  float m = -INFINITY, lsum = 0.f;
  f32x16 oacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) oacc[mt] = f32x16{};
  f32x16 sacc[2];
  V8 pk[4];  // P of the last softmax as B operands, 16 keys each

  // Per-lane LDS byte offsets inside a tile, fixed for the whole kernel.  The
  // swizzle repeats every 16 rows, so the other rows a lane reads differ from
  // these by constants (instruction offsets): K rows of key 32*smt + r at
  // row_off[ks] + 32*smt*D*2, transposed V pieces of keys 16*kk + .. at
  // tr_off[mt][hi] + 16*kk*D*2.  tr_off also holds the V region's start, so
  // the V tile of stage s is read at tr_off + k_off(s)*2 + those constants.
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
            (C::v_off(0) + swz_elem<D>(8 * hi + 4 * hh + (jl >> 2), mt * 32 + 16 * qq + 4 * (jl & 3))) *
            sizeof(T)));
  }
  const char* smem_c = reinterpret_cast<const char*>(smem);
  auto k_row = [&](const char* ks_base, int ks, int smt) {
    return as_vec8<T>(*reinterpret_cast<const u32x4*>(ks_base + row_off[ks] +
                                                       smt * 32 * D * (int)sizeof(T)));
  };
  auto v_tr = [&](const char* vs_base, int mt, int kk) {
    const char* base = vs_base + kk * 16 * D * (int)sizeof(T);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][0]));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + tr_off[mt][1]));
    u32x4 rr;
    rr[0] = __builtin_bit_cast(u32x2, lo)[0];
    rr[1] = __builtin_bit_cast(u32x2, lo)[1];
    rr[2] = __builtin_bit_cast(u32x2, hi)[0];
    rr[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_vec8<T>(rr);
  };
  auto mma_s = [&](int stg) {  // S^T = K Q^T
    const char* Kb = smem_c + C::k_off(stg) * (int)sizeof(T);
    sacc[0] = f32x16{};
    sacc[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
      for (int smt = 0; smt < 2; ++smt) sacc[smt] = E::mfma32(k_row(Kb, ks, smt), qf[ks], sacc[smt]);
  };
  // The online softmax of a chunk is split between the two phases of its wave.
  // prep (MFMA phase, under the O products): padding keys to -inf, row max,
  // the lazy-rescale decision and the exponent arguments t = s*c2 - m, in
  // place in sacc.  finish (softmax phase): the rescale of O and the row sum,
  // p = exp2(t), the chunk row sum and the packed P.  The values and their
  // order are those of sparse_fwd_kernel's softmax.
  bool resc = false;   // this chunk moved the running max (wave-uniform)
  float alpha = 1.f;   // exp2(m_old - m_new) when resc
  float m4[4];
  float tv[32];        // the chunk's scores, then its exponent arguments
  auto prep_step = [&](int st, int nv) {  // st in [0, 8): one slice of prep
    if (st == 0) {
#pragma unroll
      for (int x = 0; x < 32; ++x) tv[x] = sacc[x >> 4][x & 15];
      if (nv < C::KC) {
        const int nvl = uniform_here(nv);
#pragma unroll
        for (int x = 0; x < 32; ++x) {
          const int key = (x >> 4) * 32 + 8 * ((x & 15) >> 2) + 4 * h + (x & 3);
          if (key >= nvl) tv[x] = -INFINITY;
        }
      }
    }
    if (st == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) m4[i] = tv[i];
#pragma unroll
      for (int i = 4; i < 16; ++i) m4[i & 3] = vmax(m4[i & 3], tv[i]);
    }
    if (st == 2) {
#pragma unroll
      for (int i = 16; i < 32; ++i) m4[i & 3] = vmax(m4[i & 3], tv[i]);
    }
    if (st == 3) {
      float smax = vmax(vmax(m4[0], m4[1]), vmax(m4[2], m4[3]));
      smax = pair_max32(smax) * c2;
      // per-lane update under a wave-uniform branch, as in sparse_fwd_kernel
      const bool grow = smax > m + kRescaleSlack;
      resc = __any(grow);
      const float mnew = grow ? smax : m;
      alpha = fast_exp2(m - mnew);  // used only when resc (1 where m stays)
      m = mnew;
    }
    if (st >= 4) {
      const float negm = -m;
#pragma unroll
      for (int i = 0; i < 8; ++i) tv[(st - 4) * 8 + i] = here(fmaf(tv[(st - 4) * 8 + i], c2, negm));
    }
  };
  auto finish = [&](int nv) {
    if (resc) {
      lsum *= alpha;
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) oacc[mt] *= alpha;
    }
    float p[2][16];
#pragma unroll
    for (int smt = 0; smt < 2; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) p[smt][i] = fast_exp2(tv[smt * 16 + i]);
    if (nv < C::KC) {
      const int nvl = uniform_here(nv);
#pragma unroll
      for (int smt = 0; smt < 2; ++smt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key >= nvl) p[smt][i] = 0.f;
        }
    }
    float l4[4] = {p[0][0], p[0][1], p[0][2], p[0][3]};  // chunk row sum in four short chains
#pragma unroll
    for (int x = 4; x < 32; ++x) l4[x & 3] += p[x >> 4][x & 15];
    lsum += (l4[0] + l4[1]) + (l4[2] + l4[3]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) pk[kk] = pack8<T>(&p[kk >> 1][8 * (kk & 1)]);
  };
  // MFMA phase of chunk j: S_j, then O += V_{j-1} P_{j-1} with prep of chunk j
  // under it (the S results land while the first O products issue).  Every
  // LDS operand is read L MFMAs ahead of its use: this wave is the only MFMA
  // issuer of its SIMD during the phase, so nothing else covers the latency.
  // L is as deep as the registers allow without spills inside the chunk loop
  // (head_dim 128: 6, 2 % faster than 4; 7 spills there).
  constexpr int NSX = 2 * (D / 16), NOX = 4 * (D / 32), NX = NSX + NOX, L = D == 128 ? 6 : 8;
  // The first L operands of an MFMA phase (K rows of its chunk, published by
  // the barrier that opens the previous softmax phase) are read at the end of
  // that softmax phase, so the phase does not open with an LDS round trip.
  constexpr int NP = L;  // prefetched operands
  V8 pre[NP];
  auto prefetch = [&](int sj) {
    const char* Kb = smem_c + C::k_off(sj) * (int)sizeof(T);
    __builtin_amdgcn_sched_barrier(0);  // after the softmax phase's arithmetic
#pragma unroll
    for (int u = 0; u < NP; ++u) pre[u] = k_row(Kb, u >> 1, u & 1);
  };
  static_assert(L <= NSX, "the prefetched operands are K rows");
  auto mma_so = [&](int sj, int sp, int nv) {
    const char* Kb = smem_c + C::k_off(sj) * (int)sizeof(T);
    const char* Vb = smem_c + C::k_off(sp) * (int)sizeof(T);  // + tr_off: the V tile
    V8 op[NX];
    auto load = [&](int u) {  // u < NSX: K row (ks = u >> 1, smt = u & 1); else V^T piece
      if (u >= NX) return;
      if (u < NSX) {
        op[u] = k_row(Kb, u >> 1, u & 1);
      } else {
        const int x = u - NSX;  // kk = x / (D/32), mt = x % (D/32)
        op[u] = v_tr(Vb, x % (D / 32), x / (D / 32));
      }
    };
    sacc[0] = f32x16{};
    sacc[1] = f32x16{};
#pragma unroll
    for (int u = 0; u < L; ++u) {
      if (u < NP)
        op[u] = pre[u];
      else
        load(u);
    }
#pragma unroll
    for (int u = 0; u < NX; ++u) {
      load(u + L);
      if (u < NSX) {
        sacc[u & 1] = E::mfma32(op[u], qf[u >> 1], sacc[u & 1]);
      } else {
        const int x = u - NSX;
        oacc[x % (D / 32)] = E::mfma32(op[u], pk[x / (D / 32)], oacc[x % (D / 32)]);
        // prep slice st after O product x (from the third on: S has landed).
        // With nv = 0 (the stream's S half on a stale stage) prep masks every
        // key, so the running max is left as it is.
        if (x >= 2) {
          const int st_lo = (x - 2) * 8 / (NOX - 2), st_hi = (x - 1) * 8 / (NOX - 2);
#pragma unroll
          for (int st = 0; st < 8; ++st)
            if (st >= st_lo && st < st_hi) prep_step(st, nv);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto prep_all = [&](int nv) {
#pragma unroll
    for (int st = 0; st < 8; ++st) prep_step(st, nv);
  };

  int nvm1 = 0;        // valid keys of chunk j-1 (0: no such chunk)
  int nv0 = issue(0);  // chunk j
  int nv1 = issue(1);  // chunk j+1
  if (nv1 > 0)
    wait_vmcnt<C::PER>();
  else
    dma_wait();
  // A phase boundary: the barrier, with the instruction scheduler kept from
  // moving MFMA or VALU work across it (s_barrier only orders memory, so the
  // compiler would otherwise let one phase's arithmetic drift into the next).
  auto phase_barrier = []() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  if (grp1) {
    phase_barrier();
    // group 1's copies of chunk 1 land before the barrier after which group 0
    // reads chunk 1 (its operand prefetch opens its next softmax phase)
    dma_wait();
  }
  if (nv0 > 0) {
    // chunk 0: no chunk -1, so its MFMA phase is S_0 alone
    phase_barrier();
    mfma_priority_up();
    mma_s(0);
    prep_all(nv0);
    mfma_priority_down();
    dma_wait();  // this wave's copies of chunk 1
    phase_barrier();
    int nv2 = issue(2);
    int fin = nv0;  // valid keys of the chunk whose softmax phase is pending
    nvm1 = nv0;
    nv0 = nv1;
    nv1 = nv2;
    // chunks 1 .. n; at j = n (no chunk j) the S half of the stream runs on a
    // stage no copy is writing and its result is not used.  An iteration opens
    // with the softmax phase of chunk j-1, so the operands prefetched at its
    // end stay inside one iteration.  Chunk j+1 is complete in LDS at the
    // barrier that ends group 0's MFMA phase of chunk j (and opens group 1's):
    // group 0 waits for its copies of it before that barrier, group 1, whose
    // copies were issued at the start of the softmax phase just ending, at the
    // end of that phase.  Group 0 prefetches from chunk j+1 right after it.
    // The loop is unrolled by NS so that every stage index is a constant.
    auto iteration = [&](auto jc) {  // chunk j, j % NS == jc
      constexpr int sj = decltype(jc)::value;
      if (fin > 0) finish(fin);
      if (grp1) dma_wait();  // this wave's copies of chunk j+1
      prefetch(sj);
      phase_barrier();
      mfma_priority_up();
      mma_so(sj, (sj + C::NS - 1) % C::NS, nv0);
      mfma_priority_down();
      if (!grp1) dma_wait();  // this wave's copies of chunk j+1
      phase_barrier();
      // the stage of chunk j+2 last held chunk j-2, read for the last time in
      // group 1's MFMA phase of chunk j-1, which ended before this iteration's
      // first barrier
      nv2 = issue((sj + 2) % C::NS);
      fin = nv0;
      nvm1 = nv0;
      nv0 = nv1;
      nv1 = nv2;
    };
    static_assert(C::NS == 4, "the unrolled loop below walks four stages");
    while (nvm1 > 0) {
      iteration(std::integral_constant<int, 1>{});
      if (nvm1 <= 0) break;
      iteration(std::integral_constant<int, 2>{});
      if (nvm1 <= 0) break;
      iteration(std::integral_constant<int, 3>{});
      if (nvm1 <= 0) break;
      iteration(std::integral_constant<int, 0>{});
    }
  }
  if (!grp1) phase_barrier();
  fwd_epilogue<T, D, RASTER>(oacc, lsum, m, b, myq, qblk, h, sq, qb, out, fine, lse, outc, gate,
                             gate_mode, gate_heads, orows, s_out, heads);
}

// Persistent: as many workgroups as the CUs hold (one each).  Workgroup i runs
// on XCD i % 8 and takes the query blocks of that XCD's contiguous range (the
// xcd_tile order), so one head's K/V stay in one XCD's L2: with scheduling
// counters (sched_counters) the next block of the range, then the blocks left
// in the other XCDs' ranges (take_entry; every block has the same topk chunks,
// but the XCDs do not run equally fast: 0.6 % less time at c3 and 4.5 % at c4,
// where 56.25 blocks per workgroup also left a fixed stride uneven); without,
// a fixed stride over the range.
template <typename T, int D, bool RASTER>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sparse_fwd_pp_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                     const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
                     T* __restrict__ out, T* __restrict__ fine, float* __restrict__ lse, const T* __restrict__ outc,
                     const T* __restrict__ gate, int gate_mode, int gate_heads, int num_tiles,
                     int sq, int skv, int qb, int kb, int topk, float c2, uint32_t qsign,
                     const int32_t* __restrict__ orows, int64_t s_out, int heads,
                     int32_t* __restrict__ ctr) {
  using C = FwdPPCfg<D>;
  __shared__ __attribute__((aligned(16))) T smem[C::NS * C::STAGE];
  __shared__ int s_next;
  const int xcd = blockIdx.x & 7, per = (num_tiles + 7) >> 3, stride = (int)(gridDim.x >> 3);
  int from = 0;
  for (int round = 0;; ++round) {
    int tile;
    if (ctr) {
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
      fwd_pp_tile<T, D, RASTER>(smem, tile, q, k, v, selected, kv_vbs, out, fine, lse, outc, gate,
                                gate_mode, gate_heads, sq, skv, qb, kb, topk, c2, qsign, orows,
                                s_out, heads);
    // No copy is in flight here (every chunk's copy is waited for before the
    // chunk is read, and past the route's end nothing is copied), so only the
    // epilogue's stores are outstanding: they drain under the next tile's
    // first loads instead of in front of them.
    __syncthreads();  // every wave is done with the LDS ring (and s_next) before the next tile
  }
  if (ctr && threadIdx.x == 0) finish_entries(ctr);
}

template <typename T, int D, bool RASTER = false>
static int launch_fwd_pp(const void* q, const void* k, const void* v, const int32_t* selected,
                         const int32_t* kv_vbs, void* out, void* fine, float* lse, const void* outc,
                         const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq,
                         int64_t skv, int topk, float scale, hipStream_t stream,
                         const int32_t* orows = nullptr, int64_t s_out = 0, int heads = 0) {
  const int64_t tiles = bh * (sq / 256);
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int64_t want = ((tiles + 7) / 8) * 8;
  const int resident = (cu_count() / 8) * 8;  // one 8-wave workgroup per CU
  const int grid = (int)(want < resident ? want : resident);
  const float c2 = fabsf(scale) * kLog2e;
  const uint32_t qsign = scale < 0.f ? 0x80008000u : 0u;
  hipLaunchKernelGGL((sparse_fwd_pp_kernel<T, D, RASTER>), dim3(grid), dim3(512), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, selected, kv_vbs, (T*)out, (T*)fine, lse,
                     (const T*)outc, (const T*)gate, gate_mode, gate_heads, (int)tiles, (int)sq,
                     (int)skv, (int)(sq / 256), (int)(skv / 256), topk, c2, qsign, orows, s_out, heads,
                     sched_counters(stream));
  return vsa_check_launch();
}

template <typename T, int D, int BE, bool RASTER = false>
static int launch_fwd(const void* q, const void* k, const void* v, const int32_t* selected,
                      const int32_t* kv_vbs, void* out, void* fine, float* lse, const void* outc,
                      const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq, int64_t skv,
                      int topk, float scale, hipStream_t stream, const int32_t* orows = nullptr,
                      int64_t s_out = 0, int heads = 0) {
  using C = FwdCfg<D, BE>;
  const int tph = (int)(sq / C::QT);
  const int64_t tiles = bh * tph;
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int grid = (int)(((tiles + 7) / 8) * 8);
  const float c2 = fabsf(scale) * kLog2e;
  const uint32_t qsign = scale < 0.f ? 0x80008000u : 0u;
  hipLaunchKernelGGL((sparse_fwd_kernel<T, D, BE, RASTER>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, selected, kv_vbs, (T*)out, (T*)fine, lse,
                     (const T*)outc, (const T*)gate, gate_mode, gate_heads, (int)tiles, tph, (int)sq,
                     (int)skv, (int)(sq / BE), (int)(skv / BE), topk, c2, qsign, orows, s_out, heads);
  return vsa_check_launch();
}

}  // namespace vsa

using namespace vsa;

#ifndef VSA_FWD_NO_PP
// one 8-wave workgroup per query block: used at head dim 128 once there are
// enough blocks to give every CU one (smaller grids run better as 4-wave
// half-block workgroups).  At head dim 64 the 4-wave kernel is faster at every
// grid (block 256, 40 960 tokens, 24 heads: 1.53 against 1.87 ms at topk 20,
// 0.81 against 1.03 at topk 10; at head dim 128 the 8-wave kernel leads, 4.07
// against 4.40 ms at 40 heads, topk 20).
#define VSA_FWD_PP_CASE(DD)                                                                    \
  if (D == DD && be == 256 && bh * (sq / 256) >= 256)                                          \
    return launch_fwd_pp<T, DD>(q, k, v, selected, kv_vbs, out, fine_out, lse, out_c, gate, gate_mode,   \
                                gate_heads, bh, sq, skv, topk, scale, s);
#else
#define VSA_FWD_PP_CASE(DD)
#endif

#define VSA_FWD_CASE(DD, BB)                                                                   \
  if (D == DD && be == BB)                                                                     \
    return launch_fwd<T, DD, BB>(q, k, v, selected, kv_vbs, out, fine_out, lse, out_c, gate, gate_mode, gate_heads, \
                                 bh, sq, skv, topk, scale, s);

extern "C" int vsa_sparse_fwd(const void* q, const void* k, const void* v,
                              const int32_t* selected, const int32_t* kv_vbs, void* out,
                              void* fine_out, float* lse, const void* out_c, const void* gate, int32_t gate_mode,
                              int32_t gate_heads, int64_t bh, int64_t sq, int64_t skv, int32_t D,
                              int32_t be, int32_t topk, float scale, int32_t dtype, void* stream) {
  if (!q || !k || !v || !selected || !kv_vbs || !out) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, out, fine_out, out_c, gate) ||
      !vsa_aligned<4>(selected, kv_vbs, lse))
    return VSA_ERR_ALIGN;
  if (out_c && (gate_mode & VSA_GATE_F32) && dtype != VSA_F32) {
    // fp32 gate beside T inputs: fine output in T (into fine_out, or into out
    // when no backward needs it), then the combine as a second pass
    const int gm = gate_mode & ~VSA_GATE_F32;
    if (gm < 1 || gm > 3 || !gate) return gm == 0 ? VSA_ERR_SHAPE : VSA_ERR_NULL;
    if (gm == 3 && (gate_heads <= 0 || bh % gate_heads)) return VSA_ERR_SHAPE;
    // the combine's limits, checked before the fine pass writes anything
    if (!vsa::combine_f32gate_shape_ok(bh, sq, D, be, dtype)) return VSA_ERR_SHAPE;
    void* fine = fine_out ? fine_out : out;
    int rc = vsa_sparse_fwd(q, k, v, selected, kv_vbs, fine, nullptr, lse, nullptr, nullptr, 0,
                            gate_heads, bh, sq, skv, D, be, topk, scale, dtype, stream);
    if (rc != VSA_OK) return rc;
    return combine_f32gate(fine, out_c, gate, gm, gate_heads, out, bh, sq, D, be, dtype,
                           (hipStream_t)stream);
  }
  gate_mode &= ~VSA_GATE_F32;  // an fp32 gate beside fp32 inputs is the plain case
  if (gate_mode < 0 || gate_mode > 3) return VSA_ERR_SHAPE;
  if (out_c && gate_mode == 3 && (gate_heads <= 0 || bh % gate_heads)) return VSA_ERR_SHAPE;
  if (out_c && gate_mode != 0 && !gate) return VSA_ERR_NULL;
  if (!out_c) {  // without the combine, out is the fine output
    gate_mode = 0;
    fine_out = nullptr;
  }
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == VSA_F32)
    return sparse_fwd_f32(q, k, v, selected, kv_vbs, out, fine_out, lse, out_c, gate, gate_mode,
                          gate_heads, bh, sq, skv, D, be, topk, scale, s);
  VSA_DISPATCH_MFMA(dtype, T, {
    VSA_FWD_PP_CASE(128)
    VSA_FWD_CASE(128, 256)
    VSA_FWD_CASE(128, 128)
    VSA_FWD_CASE(128, 64)
    VSA_FWD_CASE(256, 256)
    VSA_FWD_CASE(256, 128)
    VSA_FWD_CASE(256, 64)
    VSA_FWD_CASE(64, 256)
    VSA_FWD_CASE(64, 128)
    VSA_FWD_CASE(64, 64)
  });
  return VSA_ERR_UNSUPPORTED;
}

#define VSA_FWD_TILED_CASE(DD, BB)                                                             \
  if (D == DD && be == BB) {                                                                   \
    if (BB == 256 && DD == 128 && bh * (sq / 256) >= 256)                                      \
      return launch_fwd_pp<T, DD, true>(q, k, v, selected, kv_vbs, out, fine_out, lse, out_c,  \
                                        gate, gate_mode, 0, bh, sq, skv, topk, scale, s,       \
                                        slot_rows, s_out, heads);                                     \
    return launch_fwd<T, DD, BB, true>(q, k, v, selected, kv_vbs, out, fine_out, lse, out_c,   \
                                       gate, gate_mode, 0, bh, sq, skv, topk, scale, s,        \
                                       slot_rows, s_out, heads);                                      \
  }

extern "C" int vsa_sparse_fwd_tiled(const void* q, const void* k, const void* v,
                                    const int32_t* selected, const int32_t* kv_vbs, void* out,
                                    void* fine_out, float* lse, const void* out_c,
                                    const void* gate, int32_t gate_mode,
                                    const int32_t* slot_rows, int64_t s_out, int32_t heads, int64_t bh,
                                    int64_t sq, int64_t skv, int32_t D, int32_t be, int32_t topk,
                                    float scale, int32_t dtype, void* stream) {
  if (!q || !k || !v || !selected || !kv_vbs || !out || !slot_rows) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, out, fine_out, out_c, gate) ||
      !vsa_aligned<4>(selected, kv_vbs, lse, slot_rows))
    return VSA_ERR_ALIGN;
  if (gate_mode < 0 || gate_mode > 2) return VSA_ERR_SHAPE;  // no token-major / fp32 gate here
  if (out_c && gate_mode != 0 && !gate) return VSA_ERR_NULL;
  if (!out_c) {
    gate_mode = 0;
    fine_out = nullptr;
  }
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      s_out <= 0 || s_out > sq || sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  if (heads < 0 || (heads > 0 && bh % heads)) return VSA_ERR_SHAPE;
  if (dtype == VSA_F32) return VSA_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  VSA_DISPATCH_MFMA(dtype, T, {
    VSA_FWD_TILED_CASE(128, 256)
    VSA_FWD_TILED_CASE(128, 128)
    VSA_FWD_TILED_CASE(128, 64)
    VSA_FWD_TILED_CASE(64, 256)
    VSA_FWD_TILED_CASE(64, 128)
    VSA_FWD_TILED_CASE(64, 64)
  });
  return VSA_ERR_UNSUPPORTED;
}
