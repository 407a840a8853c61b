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
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

template <int D, int BE>
struct FwdCfg {
  static constexpr int QT = BE >= 128 ? 128 : BE;  // queries per workgroup
  static constexpr int NW = QT / 32;               // waves per workgroup
  static constexpr int NT = NW * 64;
  // keys per chunk: 32 for (D 128, block 64) so that a 2-wave workgroup's
  // double buffer is 32 KiB and four workgroups share a CU
  static constexpr int KC = (D == 128 && BE == 64) ? 32 : 64;
  static constexpr int NSM = KC / 32;              // 32-key sub-tiles per chunk
  static constexpr int TILE = KC * D;              // elements of one K (or V) chunk
  static constexpr int STAGE = 2 * TILE;           // K and V
};

constexpr float kRescaleSlack = 8.0f;  // log2 units

// Advance (slot, chunk) to the next chunk that holds at least one valid key.
template <int BE, int KC>
__device__ __forceinline__ bool next_valid_chunk(const int32_t* __restrict__ sel,
                                                 const int32_t* __restrict__ vbs, int topk,
                                                 int kb, int& s, int& c, int& kv, int& nvb) {
  // Uniform indices keep these reads on the scalar path: a vector load here
  // would need vmcnt(0) and so wait for every K/V copy still in flight.
  while (s < topk) {
    kv = __builtin_amdgcn_readfirstlane(sel[__builtin_amdgcn_readfirstlane(s)]);
    if (kv >= 0 && kv < kb) {
      nvb = __builtin_amdgcn_readfirstlane(clamp_valid(vbs[kv], BE));
      if (c * KC < nvb) return true;
    }
    ++s;
    c = 0;
  }
  return false;
}

template <typename T, int D, int BE>
__global__ __launch_bounds__((FwdCfg<D, BE>::NT)) __attribute__((amdgpu_waves_per_eu(2))) void sparse_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ selected, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ out, float* __restrict__ lse, const T* __restrict__ outc,
    const T* __restrict__ gate, int gate_mode, int gate_heads, int num_tiles, int tiles_per_head, int sq,
    int skv, int qb, int kb, int topk, float c2, uint32_t qsign) {
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

  int s = 0, ch = 0, kv = 0, nvb = 0;
  bool have = next_valid_chunk<BE, C::KC>(sel, kv_vbs, topk, kb, s, ch, kv, nvb);
  if (have) dma(kv, ch, 0);
  dma_wait();
  __syncthreads();
  int stage = 0;
  while (have) {
    const int nv = min(nvb - ch * C::KC, C::KC);
    int s2 = s, ch2 = ch + 1, kv2 = kv, nvb2 = nvb;
    const bool have2 = next_valid_chunk<BE, C::KC>(sel, kv_vbs, topk, kb, s2, ch2, kv2, nvb2);
    if (have2) dma(kv2, ch2, stage ^ 1);  // lands while this chunk is multiplied

    const T* Ks = smem + stage * C::STAGE;
    const T* Vs = Ks + C::TILE;
    // ---- S^T = K Q^T -------------------------------------------------------
    f32x16 sacc[C::NSM];
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt) sacc[smt] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int smt = 0; smt < C::NSM; ++smt)
        sacc[smt] = E::mfma32(row_a8<T, D>(Ks, smt * 32 + r, ks, h), qf[ks], sacc[smt]);
    }
    // ---- online softmax (base 2, lazily rescaled) ---------------------------
    if (nv < C::KC) {
#pragma unroll
      for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key >= nv) sacc[smt][i] = -INFINITY;
        }
    }
    float smax = sacc[0][0];
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) smax = fmaxf(smax, sacc[smt][i]);
    smax = fmaxf(smax, __shfl_xor(smax, 32, 64)) * c2;
    if (__any(smax > m + kRescaleSlack)) {
      const float mnew = fmaxf(m, smax);
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
    if (nv < C::KC) {
#pragma unroll
      for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = smt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if (key >= nv) p[smt][i] = 0.f;
        }
    }
#pragma unroll
    for (int smt = 0; smt < C::NSM; ++smt)
#pragma unroll
      for (int i = 0; i < 16; ++i) lsum += p[smt][i];
    // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
    for (int kk = 0; kk < 2 * C::NSM; ++kk) {
      const V8 bop = pack8<T>(&p[kk >> 1][8 * (kk & 1)]);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        oacc[mt] = E::mfma32(tr_a8<T, D>(Vs, mt * 32, 16 * kk, 16 * kk + 8), bop, oacc[mt]);
    }

    dma_wait();
    __syncthreads();
    stage ^= 1;
    s = s2; ch = ch2; kv = kv2; nvb = nvb2; have = have2;
  }

  // ---- epilogue: normalise, fused combine, LSE ----------------------------
  const float ltot = lsum + __shfl_xor(lsum, 32, 64);
  const float inv = 1.0f / ltot;
  const int64_t tok = (int64_t)b * sq + myq;
  if (lse != nullptr && h == 0) lse[tok] = m + log2f(ltot);
  const T* ocrow = outc ? outc + ((int64_t)b * qb + qblk) * D : nullptr;
  float gtok = 1.f;
  if (outc && gate_mode == 2) gtok = E::to_f(gate[tok]);
  // gate row of this token: [BH, Sq, D] (mode 1) or token-major [B, Sq, H, D] (mode 3)
  const T* grow = nullptr;
  if (gate_mode == 1) grow = gate + tok * D;
  if (gate_mode == 3)
    grow = gate + (((int64_t)(b / gate_heads) * sq + myq) * gate_heads + b % gate_heads) * D;
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = mt * 32 + 8 * g + 4 * h;
      float val[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) val[e] = oacc[mt][4 * g + e] * inv;
      if (ocrow) {
        u32x2 ocr = *reinterpret_cast<const u32x2*>(ocrow + d0);
        const T* oc = reinterpret_cast<const T*>(&ocr);
        float gv[4] = {gtok, gtok, gtok, gtok};
        if (grow) {
          u32x2 gr = *reinterpret_cast<const u32x2*>(grow + d0);
          const T* gg = reinterpret_cast<const T*>(&gr);
#pragma unroll
          for (int e = 0; e < 4; ++e) gv[e] = E::to_f(gg[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = fmaf(E::to_f(oc[e]), gv[e], val[e]);
      }
      T o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = E::from_f(val[e]);
      *reinterpret_cast<u32x2*>(out + tok * D + d0) = *reinterpret_cast<const u32x2*>(o4);
    }
  }
}

template <typename T, int D, int BE>
static int launch_fwd(const void* q, const void* k, const void* v, const int32_t* selected,
                      const int32_t* kv_vbs, void* out, float* lse, const void* outc,
                      const void* gate, int gate_mode, int gate_heads, int64_t bh, int64_t sq, int64_t skv,
                      int topk, float scale, hipStream_t stream) {
  using C = FwdCfg<D, BE>;
  const int tph = (int)(sq / C::QT);
  const int64_t tiles = bh * tph;
  if (tiles > (1LL << 30)) return VSA_ERR_SHAPE;
  const int grid = (int)(((tiles + 7) / 8) * 8);
  const float c2 = fabsf(scale) * kLog2e;
  const uint32_t qsign = scale < 0.f ? 0x80008000u : 0u;
  hipLaunchKernelGGL((sparse_fwd_kernel<T, D, BE>), dim3(grid), dim3(C::NT), 0, stream,
                     (const T*)q, (const T*)k, (const T*)v, selected, kv_vbs, (T*)out, lse,
                     (const T*)outc, (const T*)gate, gate_mode, gate_heads, (int)tiles, tph, (int)sq,
                     (int)skv, (int)(sq / BE), (int)(skv / BE), topk, c2, qsign);
  return vsa_check_launch();
}

}  // namespace vsa

using namespace vsa;

#define VSA_FWD_CASE(DD, BB)                                                                   \
  if (D == DD && be == BB)                                                                     \
    return launch_fwd<T, DD, BB>(q, k, v, selected, kv_vbs, out, lse, out_c, gate, gate_mode, gate_heads, \
                                 bh, sq, skv, topk, scale, s);

extern "C" int vsa_sparse_fwd(const void* q, const void* k, const void* v,
                              const int32_t* selected, const int32_t* kv_vbs, void* out,
                              float* lse, const void* out_c, const void* gate, int32_t gate_mode,
                              int32_t gate_heads, int64_t bh, int64_t sq, int64_t skv, int32_t D,
                              int32_t be, int32_t topk, float scale, int32_t dtype, void* stream) {
  if (!q || !k || !v || !selected || !kv_vbs || !out) return VSA_ERR_NULL;
  if (gate_mode < 0 || gate_mode > 3) return VSA_ERR_SHAPE;
  if (out_c && gate_mode == 3 && (gate_heads <= 0 || bh % gate_heads)) return VSA_ERR_SHAPE;
  if (out_c && gate_mode != 0 && !gate) return VSA_ERR_NULL;
  if (!out_c) gate_mode = 0;
  if (bh <= 0 || sq <= 0 || skv <= 0 || be <= 0 || sq % be || skv % be || topk < 1 ||
      sq > (1LL << 31) / 256 || skv > (1LL << 31) / 256)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  VSA_DISPATCH_MFMA(dtype, T, {
    VSA_FWD_CASE(128, 256)
    VSA_FWD_CASE(128, 128)
    VSA_FWD_CASE(128, 64)
    VSA_FWD_CASE(64, 256)
    VSA_FWD_CASE(64, 128)
    VSA_FWD_CASE(64, 64)
  });
  return VSA_ERR_UNSUPPORTED;
}
