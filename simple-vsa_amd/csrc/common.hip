// Bandwidth- and latency-bound kernels of the VSA common path on gfx950:
// padded block mean, coarse block attention + Top-K routing, CSR inverse
// routing, backward preprocessing (delta + combine gradients) and the coarse
// branch backward.  The MFMA fine kernels live in fine_fwd.hip / fine_bwd.hip.
#include <mutex>
#include <type_traits>
#include <unordered_map>

#include "coarse.h"
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

// ---------------------------------------------------------------------------
// Padded block mean (fused_common.py:20-59): one workgroup per (tensor, bh,
// block); 16-byte coalesced loads over the valid rows only; fp32 sums reduced
// across row groups in LDS; result rounded to T.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void pool_qkv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ q_vbs, const int32_t* __restrict__ kv_vbs,
    T* __restrict__ qc, T* __restrict__ kc, T* __restrict__ vc,
    int64_t bh, int qb, int kb, int D, int be) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float part[256 * VEC];
  int64_t id = blockIdx.x;
  const int64_t nq = bh * qb, nk = bh * kb;
  const T* x;
  const int32_t* vbs;
  T* out;
  int nb;
  if (id < nq) {
    x = q; vbs = q_vbs; out = qc; nb = qb;
  } else if (id < nq + nk) {
    id -= nq; x = k; vbs = kv_vbs; out = kc; nb = kb;
  } else {
    id -= nq + nk; x = v; vbs = kv_vbs; out = vc; nb = kb;
  }
  const int n = (int)(id % nb);
  const int32_t cnt = vbs[n];
  const int valid = clamp_valid(cnt, be);
  const float div = (float)(cnt > 1 ? cnt : 1);
  const T* base = x + id * (int64_t)be * D;  // block id*: rows [n*be, n*be+be) of head id/nb
  const int tpr = D / VEC, rpi = 256 / tpr;
  const int col = threadIdx.x % tpr, row0 = threadIdx.x / tpr;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  // eight rows' loads in flight per thread before their sums (a load per
  // iteration leaves too few bytes in flight to cover HBM latency)
  constexpr int UR = 8;
  int t = row0;
  for (; t + (UR - 1) * rpi < valid; t += UR * rpi) {
    u32x4 raw[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u)
      raw[u] = ld_stream(reinterpret_cast<const u32x4*>(base + (int64_t)(t + u * rpi) * D + col * VEC));
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const T* vals = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += Elem<T>::to_f(vals[e]);
    }
  }
  for (; t < valid; t += rpi) {
    u32x4 raw = ld_stream(reinterpret_cast<const u32x4*>(base + (int64_t)t * D + col * VEC));
    const T* vals = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += Elem<T>::to_f(vals[e]);
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) part[row0 * D + col * VEC + e] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    float s = 0.f;
    for (int r = 0; r < rpi; ++r) s += part[r * D + d];
    out[id * D + d] = Elem<T>::from_f(s / div);
  }
}

// ---------------------------------------------------------------------------
// tile() and the padded block mean in one pass: x (q, k or v) is a
// raster-order sequence of s_out tokens per head (head-major, or token-major
// [B, s_out, heads, D] when heads > 0); the tiled copy xt gets row
// t of block n from raster row rows[n*be + t] (zero at a padding slot, < 0),
// and the block mean sums the valid rows of that copy in the order
// pool_qkv_kernel does, so both equal tile() followed by the pooling pass.
// One workgroup per (tensor, bh, block).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void tile_pool_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ rows, const int32_t* __restrict__ q_vbs,
    const int32_t* __restrict__ kv_vbs, T* __restrict__ qt,
    T* __restrict__ kt, T* __restrict__ vt, T* __restrict__ qc, T* __restrict__ kc,
    T* __restrict__ vc, int64_t bh, int nb, int D, int be, int64_t s_out, int heads) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float part[256 * VEC];
  int64_t id = blockIdx.x;
  const int64_t per = bh * nb;
  const T* x = q;
  T* xt = qt;
  T* out = qc;
  const int32_t* vbs = q_vbs;
  if (id >= 2 * per) {
    id -= 2 * per; x = v; xt = vt; out = vc; vbs = kv_vbs;
  } else if (id >= per) {
    id -= per; x = k; xt = kt; out = kc; vbs = kv_vbs;
  }
  const int n = (int)(id % nb);
  const int64_t head = id / nb;
  const int32_t cnt = vbs[n];
  const int valid = clamp_valid(cnt, be);
  const float div = (float)(cnt > 1 ? cnt : 1);

  T* dst = xt + id * (int64_t)be * D;
  const int32_t* brows = rows + (int64_t)n * be;
  const int tpr = D / VEC, rpi = 256 / tpr;
  const int col = threadIdx.x % tpr, row0 = threadIdx.x / tpr;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  constexpr int UR = 8;
  for (int t0 = row0; t0 < be; t0 += UR * rpi) {
    u32x4 raw[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int t = t0 + u * rpi;
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (t < be) {
        const int r = brows[t];
        if (r >= 0 && r < s_out)
          raw[u] = ld_stream(reinterpret_cast<const u32x4*>(
              x + raster_row(head, r, s_out, heads) * D + col * VEC));
      }
    }
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int t = t0 + u * rpi;
      if (t >= be) break;
      st_stream(reinterpret_cast<u32x4*>(dst + (int64_t)t * D + col * VEC), raw[u]);
      if (t < valid) {
        const T* vals = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += Elem<T>::to_f(vals[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) part[row0 * D + col * VEC + e] = acc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256) {
    float s = 0.f;
    for (int r = 0; r < rpi; ++r) s += part[r * D + d];
    out[id * D + d] = Elem<T>::from_f(s / div);
  }
}

// Key blocks per sequence: the generic coarse kernels keep [2 Kb + D] fp32 rows
// in LDS; the MFMA coarse kernels stream key tiles, and the Top-K keeps one
// row of Kb keys in LDS (64 KiB with its histogram).
constexpr int kMaxCoarseBlocks = 4096;
constexpr int kMaxRouteBlocks = 16000;
// batch * heads: the per-(batch, head) passes put it in the grid's y dimension
constexpr int64_t kMaxGridY = 65535;
static int max_coarse_blocks(int D, int dtype) {
  return coarse_mfma_supported(D, dtype) ? kMaxRouteBlocks : kMaxCoarseBlocks;
}

// Generic coarse forward (fp32, or head dims the MFMA kernels do not take):
// one workgroup per (bh, query block); scores in T, softmax in T, out_c in T
// (common.py:159-166).  The Top-K route runs afterwards (topk_radix).
template <typename T>
__global__ __launch_bounds__(256) void coarse_fwd_kernel(
    const T* __restrict__ qc, const T* __restrict__ kc, const T* __restrict__ vc,
    float* __restrict__ scores, float* __restrict__ probs, T* __restrict__ outc, int qb, int kb,
    int D, float scale) {
  extern __shared__ float smem[];
  float* qrow = smem;            // D
  float* srow = qrow + D;        // kb
  float* prow = srow + kb;       // kb
  float* red = prow + kb;        // 4
  const int64_t b = blockIdx.y;
  const int i = blockIdx.x;
  const T* qsrc = qc + (b * qb + i) * D;
  for (int d = threadIdx.x; d < D; d += 256) qrow[d] = Elem<T>::to_f(qsrc[d]);
  __syncthreads();
  const T* kbase = kc + b * kb * (int64_t)D;
  float lmax = -INFINITY;
  for (int j = threadIdx.x; j < kb; j += 256) {
    const T* kr = kbase + (int64_t)j * D;
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot = fmaf(qrow[d], Elem<T>::to_f(kr[d]), dot);
    const float s = round_t<T>(round_t<T>(dot) * scale);
    srow[j] = s;
    lmax = fmaxf(lmax, s);
  }
  const float mx = block_reduce<true>(lmax, red);
  float lsum = 0.f;
  for (int j = threadIdx.x; j < kb; j += 256) {
    const float e = expf(srow[j] - mx);
    prow[j] = e;
    lsum += e;
  }
  const float sum = block_reduce<false>(lsum, red);
  const int64_t rowoff = (b * qb + i) * (int64_t)kb;
  for (int j = threadIdx.x; j < kb; j += 256) {
    const float p = round_t<T>(prow[j] / sum);
    prow[j] = p;
    scores[rowoff + j] = srow[j];
    probs[rowoff + j] = p;
  }
  __syncthreads();
  const T* vbase = vc + b * kb * (int64_t)D;
  for (int d = threadIdx.x; d < D; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < kb; ++j) acc = fmaf(prow[j], Elem<T>::to_f(vbase[(int64_t)j * D + d]), acc);
    outc[(b * qb + i) * D + d] = Elem<T>::from_f(acc);
  }
}

// ---------------------------------------------------------------------------
// CSR inverse routing (triton_impl.py:476-595), in one pass without global
// atomics.  One workgroup per (range of kv_per key blocks, batch-head) marks in
// LDS which query blocks chose each of its key blocks (bit q of column kv), and
// counts on the way the edges whose key block lies below its range, which is
// the range's offset.  A wave per column then counts the column's bits and
// writes its query-block ids in ascending order, so the layout is
// deterministic.  (One workgroup per batch-head with LDS-atomic cursors left
// 24 workgroups at c5, serialised on the hot key blocks' counters.)  A route
// that chooses one key block twice sets one bit twice: the workgroup notices
// and lists that range by an ordered scan of the edges instead, so a repeated
// edge appears as often as it occurs.
// ---------------------------------------------------------------------------
constexpr int kCsrNT = 512;
constexpr int kCsrMaxCols = 256;      // key blocks per workgroup
constexpr int kCsrBitWords = 14336;   // 56 KiB of column bits

// wave-wide inclusive prefix sum
__device__ __forceinline__ int wave_incl_sum(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(v, o, 64);
    if (lane >= o) v += y;
  }
  return v;
}

__global__ __launch_bounds__(kCsrNT) void csr_cols_kernel(const int32_t* __restrict__ selected,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ inverse, int qb,
                                                          int kb, int topk, int kv_per) {
  extern __shared__ uint32_t cbits[];  // [nk][qw]
  __shared__ int ccount[kCsrMaxCols];
  __shared__ int wpart[kCsrNT / 64];
  __shared__ int s_dup;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NW = kCsrNT / 64;
  const int qw = (qb + 31) >> 5;
  const int64_t b = blockIdx.y;
  const int kv0 = (int)blockIdx.x * kv_per;
  const int nk = min(kb - kv0, kv_per);
  const int edges = qb * topk;
  const int32_t* sel = selected + b * edges;
  int32_t* inv = inverse + b * edges;
  for (int i = tid; i < nk * qw; i += kCsrNT) cbits[i] = 0;
  for (int i = tid; i < nk; i += kCsrNT) ccount[i] = 0;
  if (tid == 0) s_dup = 0;
  __syncthreads();
  int below = 0, dup = 0;
  for (int e = tid; e < edges; e += kCsrNT) {
    const int kv = sel[e];
    if (kv < 0 || kv >= kb) continue;  // ids outside [0, kb) contribute nothing
    if (kv < kv0) {
      ++below;
    } else if (kv < kv0 + nk) {
      const int q = e / topk;
      const uint32_t bit = 1u << (q & 31);
      if (atomicOr(&cbits[(kv - kv0) * qw + (q >> 5)], bit) & bit) dup = 1;
    }
  }
  below = wave_incl_sum(below);
  if (lane == 63) wpart[wave] = below;
  if (dup) s_dup = 1;
  __syncthreads();
  int base = 0;  // edges of this batch-head whose key block is below the range
#pragma unroll
  for (int w = 0; w < NW; ++w) base += wpart[w];
  const bool dups = s_dup != 0;
  // column counts
  if (!dups) {
    for (int c = wave; c < nk; c += NW) {
      int n = 0;
      for (int w = lane; w < qw; w += 64) n += __popc(cbits[c * qw + w]);
      n = wave_incl_sum(n);
      if (lane == 63) ccount[c] = n;
    }
  } else {
    for (int e = tid; e < edges; e += kCsrNT) {
      const int kv = sel[e];
      if (kv >= kv0 && kv < kv0 + nk) atomicAdd(&ccount[kv - kv0], 1);
    }
  }
  __syncthreads();
  // exclusive scan of the column counts (nk <= kCsrMaxCols <= kCsrNT), then
  // counts and offsets out; ccount becomes each column's first slot
  {
    const int c = tid < nk ? ccount[tid] : 0;
    const int incl = wave_incl_sum(c);
    __syncthreads();  // every count read before wpart and ccount are reused
    if (lane == 63) wpart[wave] = incl;
    __syncthreads();
    int pre = 0;
    for (int w = 0; w < wave; ++w) pre += wpart[w];
    if (tid < nk) {
      const int first = base + pre + incl - c;
      counts[b * kb + kv0 + tid] = c;
      offsets[b * kb + kv0 + tid] = first;
      ccount[tid] = first;
    }
  }
  __syncthreads();
  // the segments: a wave per column, ascending query block
  for (int c = wave; c < nk; c += NW) {
    int at = ccount[c];
    if (!dups) {
      for (int w0 = 0; w0 < qw; w0 += 64) {
        const int w = w0 + lane;
        uint32_t word = w < qw ? cbits[c * qw + w] : 0u;
        const int n = __popc(word);
        const int incl = wave_incl_sum(n);
        int pos = at + incl - n;
        while (word) {
          const int bit = __builtin_ctz(word);
          inv[pos++] = w * 32 + bit;
          word &= word - 1;
        }
        at += __shfl(incl, 63, 64);
      }
    } else {
      // ordered scan of the edges: edge e belongs to query block e / topk
      const int kv = kv0 + c;
      for (int e0 = 0; e0 < edges; e0 += 64) {
        const int e = e0 + lane;
        const bool hit = e < edges && sel[e] == kv;
        const uint64_t m = __ballot(hit);
        if (hit) inv[at + __popcll(m & ((1ull << lane) - 1))] = e / topk;
        at += __popcll(m);
      }
    }
  }
}

// Columns per workgroup of csr_cols_kernel: as many as 56 KiB of bits hold, and
// few enough that the grid has at least about 256 workgroups.
static int csr_cols_per_wg(int64_t bh, int qb, int kb) {
  const int qw = (qb + 31) / 32;
  int per = kCsrBitWords / qw;
  if (per > kCsrMaxCols) per = kCsrMaxCols;
  const int64_t splits = (256 + bh - 1) / bh;
  const int spread = (int)((kb + splits - 1) / splits);
  if (per > spread) per = spread;
  return per < 1 ? 1 : per;
}

// VEC consecutive gate values of element type G as fp32 (16-byte loads), and
// the matching store of VEC values of G.
template <typename G, int VEC>
__device__ __forceinline__ void load_gate(const G* __restrict__ p, float* out) {
  constexpr int N = VEC * (int)sizeof(G) / 16;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    u32x4 r = *reinterpret_cast<const u32x4*>(p + i * (16 / sizeof(G)));
    const G* g = reinterpret_cast<const G*>(&r);
#pragma unroll
    for (int e = 0; e < 16 / (int)sizeof(G); ++e) out[i * (16 / sizeof(G)) + e] = Elem<G>::to_f(g[e]);
  }
}

// The same VEC values kept as the raw 16-byte chunks, for a caller that issues
// the loads of several rows before converting any of them (a conversion right
// after each load would make every row wait for its own load).
template <typename G, int VEC>
struct GateRaw {
  static constexpr int N = VEC * (int)sizeof(G) / 16;
  u32x4 c[N];
  __device__ __forceinline__ void load(const G* __restrict__ p) {
#pragma unroll
    for (int i = 0; i < N; ++i) c[i] = *reinterpret_cast<const u32x4*>(p + i * (16 / sizeof(G)));
  }
  __device__ __forceinline__ float at(int e) const {
    return Elem<G>::to_f(reinterpret_cast<const G*>(c)[e]);
  }
};

// One gate value's bits, zero-extended to 32 (a 16-bit value loaded into half
// of a register shared with other data would be merged, and waited for, at
// once), and its value as fp32.
template <typename G>
__device__ __forceinline__ uint32_t load_bits(const G* p) {
  if constexpr (sizeof(G) == 2)
    return *reinterpret_cast<const uint16_t*>(p);
  else
    return *reinterpret_cast<const uint32_t*>(p);
}
template <typename G>
__device__ __forceinline__ float bits_to_f(uint32_t b) {
  G g;
  if constexpr (sizeof(G) == 2) {
    const uint16_t h = (uint16_t)b;
    __builtin_memcpy(&g, &h, 2);
  } else {
    __builtin_memcpy(&g, &b, 4);
  }
  return Elem<G>::to_f(g);
}

template <typename G, int VEC>
__device__ __forceinline__ void store_gate(G* __restrict__ p, const float* v) {
  constexpr int PER = 16 / (int)sizeof(G);
#pragma unroll
  for (int i = 0; i < VEC / PER; ++i) {
    G g[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) g[e] = Elem<G>::from_f(v[i * PER + e]);
    *reinterpret_cast<u32x4*>(p + i * PER) = *reinterpret_cast<const u32x4*>(g);
  }
}

// ---------------------------------------------------------------------------
// Backward preprocessing: one workgroup per (bh, query block).  delta is the
// row sum of the fine output as the forward stored it in T times dout (the
// reference's delta over its stored sparse output, triton_impl.py:598-700),
// never a difference recovered from the rounded combined output.  The gate
// has element type G: T, or fp32 for an fp32 gate beside T inputs (its
// gradient is then stored in fp32, as the reference stores it in the gate's
// dtype, fused_common.py:202-221).
// With RASTER, dout, the gate and d_gate are raster-order sequences of s_out
// tokens (head-major, or token-major [B, s_out, heads, ...] when heads > 0): tiled slot n*be + t of a head is raster row rows[n*be + t] (< 0 for a
// padding slot, whose dout and gate read as zero and which has no d_gate
// row), and the pass also writes dout in the tiled layout (dout_t, zero rows
// at the padding slots) for the fine backward kernels.  Every value is then
// what the tiled pass computes after tile() of dout and of the gate.
// ---------------------------------------------------------------------------
// GM is the gate mode, fixed at compile time so that each row's loads and
// arithmetic are straight-line code: -1 no coarse output (delta only), 0
// coarse output without a gate, 1 full gate [.., S, D], 2 per-token gate
// [.., S], 3 full gate in the token-major layout [B, S, H, D].
template <typename T, typename G, int GM, bool RASTER>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RASTER ? 3 : 4))) void bwd_prep_kernel(
    const T* __restrict__ fine, const T* __restrict__ dout, const T* __restrict__ outc,
    const G* __restrict__ gate, int gate_heads, float* __restrict__ delta,
    T* __restrict__ d_outc, G* __restrict__ d_gate, int qb, int D, int be,
    const int32_t* __restrict__ rows, int64_t s_out, int heads, T* __restrict__ dout_t) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr bool OC = GM >= 0;                  // coarse output present
  constexpr bool FULL = GM == 1 || GM == 3;     // a gate value per element
  __shared__ float part[OC ? 256 * VEC : 1];
  const int64_t blk = blockIdx.x + (int64_t)blockIdx.y * qb;  // bh*qb + n
  const int tpr = D / VEC, rpi = 256 / tpr;
  const int col = threadIdx.x % tpr, row0 = threadIdx.x / tpr;
  const int c0 = col * VEC;
  float oc[VEC], dacc[VEC];
  if constexpr (OC) {
    // one 16-byte load (element-wise loads would each wait for the previous)
    const u32x4 ocr = *reinterpret_cast<const u32x4*>(outc + blk * D + c0);
    const T* ocv = reinterpret_cast<const T*>(&ocr);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      oc[e] = Elem<T>::to_f(ocv[e]);
      dacc[e] = 0.f;
    }
  }
  // token-major gate [B, Sq, H, D]: element (bh = b*H + h, s, d) at ((b*Sq + s)*H + h)*D + d
  const int64_t bh = blockIdx.y;
  const int64_t sq = (int64_t)qb * be;
  const int64_t gbase =
      GM == 3 ? ((bh / gate_heads) * sq * gate_heads + bh % gate_heads) * D + c0 : 0;
  // UR rows per pass: their loads are issued together and their row
  // reductions run as UR independent chains (one row per pass left a single
  // load and a serial shuffle chain per iteration)
  constexpr int UR = 4;
  for (int t0 = row0; t0 < be; t0 += UR * rpi) {
    u32x4 ro[UR], rd[UR];
    GateRaw<G, VEC> graw[UR];  // full gate chunks as loaded
    uint32_t gtok[UR];         // per-token gate value's bits as loaded
    // RASTER: whether slot t holds a token, and the raster token its dout and
    // gate rows are read from (token 0 of the head for a padding slot, whose
    // values are then replaced by zeros)
    bool real[UR];
    int64_t rtok[UR];
    if constexpr (RASTER) {
      int r[UR];
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int t = t0 + u * rpi;
        if (t >= be) break;
        r[u] = rows[(int64_t)blockIdx.x * be + t];
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        if (t0 + u * rpi >= be) break;
        real[u] = r[u] >= 0 && r[u] < s_out;
        rtok[u] = raster_row(bh, real[u] ? r[u] : 0, s_out, heads);
      }
    }
    // every row's loads are issued before any of them is used (a value used
    // right after its load would make each row wait for its own)
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int t = t0 + u * rpi;
      if (t >= be) break;
      const int64_t tok = blk * be + t;
      ro[u] = ld_stream(reinterpret_cast<const u32x4*>(fine + tok * D + c0));
      const int64_t src = RASTER ? rtok[u] : tok;   // dout / gate token
      rd[u] = ld_stream(reinterpret_cast<const u32x4*>(dout + src * D + c0));
      if constexpr (GM == 1) graw[u].load(gate + src * D + c0);
      if constexpr (GM == 3)
        graw[u].load(gate + gbase + ((int64_t)blockIdx.x * be + t) * gate_heads * D);
      if constexpr (GM == 2) gtok[u] = load_bits(gate + src);
    }
    float dl[UR], dg[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u) dl[u] = dg[u] = 0.f;
#pragma unroll
    for (int u = 0; u < UR; ++u) {
      const int t = t0 + u * rpi;
      if (t >= be) break;
      const bool pad = RASTER && !real[u];   // a padding slot: dout and gate read as zero
      if constexpr (RASTER) {
        if (pad) rd[u] = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(dout_t + (blk * be + t) * D + c0) = rd[u];
      }
      const T* o = reinterpret_cast<const T*>(&ro[u]);
      const T* g = reinterpret_cast<const T*>(&rd[u]);
      float dgv[VEC];  // this chunk of d_gate (full gate), stored with 16-byte writes
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float dov = Elem<T>::to_f(g[e]);
        dl[u] = fmaf(Elem<T>::to_f(o[e]), dov, dl[u]);
        if constexpr (GM == 0) dacc[e] += dov;
        if constexpr (FULL) {
          dgv[e] = dov * oc[e];
          dacc[e] += round_t<T>(dov * (pad ? 0.f : graw[u].at(e)));
        }
        if constexpr (GM == 2) {
          dacc[e] += round_t<T>(dov * (pad ? 0.f : bits_to_f<G>(gtok[u])));
          dg[u] = fmaf(dov, oc[e], dg[u]);
        }
      }
      if constexpr (FULL) {
        if constexpr (RASTER) {
          if (real[u]) store_gate<G, VEC>(d_gate + rtok[u] * D + c0, dgv);
        } else {
          const int64_t goff = GM == 3 ? gbase + ((int64_t)blockIdx.x * be + t) * gate_heads * D
                                       : (blk * be + t) * D + c0;
          store_gate<G, VEC>(d_gate + goff, dgv);
        }
      }
    }
    // reduce over the tpr lanes of each row (contiguous lanes)
    for (int o2 = tpr >> 1; o2 > 0; o2 >>= 1) {
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        dl[u] += __shfl_xor(dl[u], o2, 64);
        if constexpr (GM == 2) dg[u] += __shfl_xor(dg[u], o2, 64);
      }
    }
    if (col == 0) {
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int t = t0 + u * rpi;
        if (t >= be) break;
        const int64_t tok = blk * be + t;
        delta[tok] = dl[u];
        if constexpr (GM == 2) {
          if (!RASTER) d_gate[tok] = Elem<G>::from_f(dg[u]);
          else if (real[u]) d_gate[rtok[u]] = Elem<G>::from_f(dg[u]);
        }
      }
    }
  }
  if constexpr (OC) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) part[row0 * D + c0 + e] = dacc[e];
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += 256) {
      float s = 0.f;
      for (int r = 0; r < rpi; ++r) s += part[r * D + d];
      d_outc[blk * D + d] = Elem<T>::from_f(s);
    }
  }
}

// Launches the bwd_prep_kernel instance of gate mode gm (-1..3; 3 only in the
// tiled layout, -1 and 0 only with G == T); false when there is none.
template <typename T, typename G, bool RASTER>
static bool launch_bwd_prep(int gm, dim3 grid, hipStream_t s, const T* fine, const T* dout,
                            const T* outc, const G* gate, int gate_heads, float* delta,
                            T* d_outc, G* d_gate, int qb, int D, int be, const int32_t* rows,
                            int64_t s_out, int heads, T* dout_t) {
  auto go = [&](auto mode) {
    constexpr int GM = decltype(mode)::value;
    hipLaunchKernelGGL((bwd_prep_kernel<T, G, GM, RASTER>), grid, dim3(256), 0, s, fine, dout,
                       outc, gate, gate_heads, delta, d_outc, d_gate, qb, D, be, rows, s_out,
                       heads, dout_t);
  };
  if constexpr (std::is_same<G, T>::value) {
    if (gm == -1) return go(std::integral_constant<int, -1>{}), true;
    if (gm == 0) return go(std::integral_constant<int, 0>{}), true;
  }
  if (gm == 1) return go(std::integral_constant<int, 1>{}), true;
  if (gm == 2) return go(std::integral_constant<int, 2>{}), true;
  if constexpr (!RASTER) {
    if (gm == 3) return go(std::integral_constant<int, 3>{}), true;
  }
  return false;
}

// ---------------------------------------------------------------------------
// Stand-alone combine for an fp32 gate beside T inputs (the fused epilogue of
// the fine forward reads the gate in T):
//   out[tok] = T(out_c[block] * gate[tok] + fine[tok]),
// the reference's fused combine over its T-rounded sparse output
// (fused_common.py:175-199).  out may alias fine.  One workgroup per
// (bh, query block), 16-byte chunks.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void combine_f32gate_kernel(
    const T* fine, const T* __restrict__ outc, const float* __restrict__ gate, int gate_mode,
    int gate_heads, T* out, int qb, int D, int be) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t blk = blockIdx.x + (int64_t)blockIdx.y * qb;
  const int tpr = D / VEC, rpi = 256 / tpr;
  const int col = threadIdx.x % tpr, row0 = threadIdx.x / tpr;
  const int c0 = col * VEC;
  float oc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) oc[e] = Elem<T>::to_f(outc[blk * D + c0 + e]);
  const int64_t bh = blockIdx.y;
  const int64_t sq = (int64_t)qb * be;
  const int64_t gbase = gate_mode == 3
                            ? ((bh / gate_heads) * sq * gate_heads + bh % gate_heads) * D + c0
                            : 0;
  for (int t = row0; t < be; t += rpi) {
    const int64_t tok = blk * be + t;
    const int64_t off = tok * D + c0;
    const int64_t goff = gate_mode == 3
                             ? gbase + ((int64_t)blockIdx.x * be + t) * gate_heads * D
                             : off;
    float gv[VEC];
    if (gate_mode == 1 || gate_mode == 3) {
      load_gate<float, VEC>(gate + goff, gv);
    } else {
      const float gs = gate_mode == 2 ? gate[tok] : 1.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) gv[e] = gs;
    }
    u32x4 rf = ld_stream(reinterpret_cast<const u32x4*>(fine + off));
    const T* f = reinterpret_cast<const T*>(&rf);
    T o[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = Elem<T>::from_f(fmaf(oc[e], gv[e], Elem<T>::to_f(f[e])));
    *reinterpret_cast<u32x4*>(out + off) = *reinterpret_cast<const u32x4*>(o);
  }
}

// ---------------------------------------------------------------------------
// Coarse backward.  Pass A (one workgroup per (bh, q row)): dP, softmax
// backward, scale, d_q_c.  Pass B (one workgroup per (bh, kv row)): d_k_c, d_v_c.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void coarse_bwd_rows_kernel(
    const T* __restrict__ kc, const T* __restrict__ vc, const float* __restrict__ probs,
    const T* __restrict__ d_outc, float* __restrict__ ds, T* __restrict__ d_qc, int qb, int kb,
    int D, float scale) {
  extern __shared__ float smem[];
  float* grow = smem;        // D
  float* dsrow = grow + D;   // kb
  float* red = dsrow + kb;   // 4
  const int64_t b = blockIdx.y;
  const int i = blockIdx.x;
  const int64_t rowq = b * qb + i;
  for (int d = threadIdx.x; d < D; d += 256) grow[d] = Elem<T>::to_f(d_outc[rowq * D + d]);
  __syncthreads();
  const T* vbase = vc + b * kb * (int64_t)D;
  const float* prow = probs + rowq * kb;
  float lsum = 0.f;
  for (int j = threadIdx.x; j < kb; j += 256) {
    const T* vr = vbase + (int64_t)j * D;
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot = fmaf(grow[d], Elem<T>::to_f(vr[d]), dot);
    const float dp = round_t<T>(dot);
    dsrow[j] = dp;
    lsum = fmaf(prow[j], dp, lsum);
  }
  const float sum = block_reduce<false>(lsum, red);
  for (int j = threadIdx.x; j < kb; j += 256) {
    const float p = prow[j];
    const float dsv = round_t<T>(round_t<T>(p * (dsrow[j] - sum)) * scale);
    dsrow[j] = dsv;
    ds[rowq * kb + j] = dsv;
  }
  __syncthreads();
  const T* kbase = kc + b * kb * (int64_t)D;
  for (int d = threadIdx.x; d < D; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < kb; ++j) acc = fmaf(dsrow[j], Elem<T>::to_f(kbase[(int64_t)j * D + d]), acc);
    d_qc[rowq * D + d] = Elem<T>::from_f(acc);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void coarse_bwd_cols_kernel(
    const T* __restrict__ qc, const float* __restrict__ probs, const T* __restrict__ d_outc,
    const float* __restrict__ ds, T* __restrict__ d_kc, T* __restrict__ d_vc, int qb, int kb,
    int D) {
  const int64_t b = blockIdx.y;
  const int j = blockIdx.x;
  const T* qbase = qc + b * qb * (int64_t)D;
  const T* gbase = d_outc + b * qb * (int64_t)D;
  const float* dsb = ds + b * qb * (int64_t)kb;
  const float* pb = probs + b * qb * (int64_t)kb;
  for (int d = threadIdx.x; d < D; d += 256) {
    float ak = 0.f, av = 0.f;
    for (int i = 0; i < qb; ++i) {
      ak = fmaf(dsb[(int64_t)i * kb + j], Elem<T>::to_f(qbase[(int64_t)i * D + d]), ak);
      av = fmaf(pb[(int64_t)i * kb + j], Elem<T>::to_f(gbase[(int64_t)i * D + d]), av);
    }
    d_kc[(b * kb + j) * D + d] = Elem<T>::from_f(ak);
    d_vc[(b * kb + j) * D + d] = Elem<T>::from_f(av);
  }
}

// ---------------------------------------------------------------------------
// Scheduling counters of the persistent forward and dQ kernels.  Launches on
// one stream run one after another, so they can share one slot of counters
// (each launch's last workgroup zeroes them for the next); launches on
// different streams may overlap and get different slots.  The array is one
// copy per GPU, held until the process ends; host code reaches it only
// through the address hipGetSymbolAddress gives for the current device.
// ---------------------------------------------------------------------------
constexpr int kSchedSlots = 256;     // streams per device with a slot of their own
constexpr int kSchedSlotInts = 32;   // 9 counters, one 128-byte line per slot
static __device__ __align__(256) int32_t sched_ctr[kSchedSlots * kSchedSlotInts];

namespace {
std::mutex g_sched_mu;
int32_t* g_sched_base[64] = {nullptr};
std::unordered_map<hipStream_t, int> g_sched_slot[64];
}  // namespace

int32_t* sched_counters(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (s != nullptr) {  // the array used is the current device's
    hipDevice_t sdev = 0;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev) return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_sched_mu);
  if (g_sched_base[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(sched_ctr)) != hipSuccess || p == nullptr)
      return nullptr;
    g_sched_base[dev] = static_cast<int32_t*>(p);
  }
  auto& slots = g_sched_slot[dev];
  auto it = slots.find(s);
  int slot;
  if (it != slots.end()) {
    slot = it->second;
  } else {
    if ((int)slots.size() >= kSchedSlots) return nullptr;
    slot = (int)slots.size();
    slots.emplace(s, slot);
  }
  return g_sched_base[dev] + (size_t)slot * kSchedSlotInts;
}

}  // namespace vsa

// ===========================================================================
// C ABI
// ===========================================================================
using namespace vsa;

extern "C" const char* vsa_status_string(int status) {
  switch (status) {
    case VSA_OK: return "ok";
    case VSA_ERR_NULL: return "a required pointer is NULL";
    case VSA_ERR_SHAPE: return "sizes are inconsistent or out of range";
    case VSA_ERR_DTYPE: return "dtype not supported by this entry point";
    case VSA_ERR_UNSUPPORTED: return "no kernel for this (block_elements, head_dim) pair";
    case VSA_ERR_LAUNCH: return "HIP kernel launch failed";
    case VSA_ERR_TOO_LARGE:
      return "the sizes need more than the library's static scratch (no-allocation entry point)";
    case VSA_ERR_ALIGN:
      return "a pointer is misaligned (16 bytes for element-type and score tensors, 4 for int32 "
             "arrays and lse / delta)";
    case VSA_ERR_DEVICE: return "the stream belongs to another GPU than the current device";
    default: return "unknown status";
  }
}

extern "C" const char* vsa_version(void) { return "mi355x-vsa 0.1 (gfx950)"; }

static bool vec_dim_ok(int D, int dtype) {
  const int vec = dtype == VSA_F32 ? 4 : 8;
  if (D <= 0 || D % vec) return false;
  const int tpr = D / vec;
  return tpr <= 256 && (256 % tpr) == 0;
}

extern "C" int vsa_pool_qkv(const void* q, const void* k, const void* v, const int32_t* q_vbs,
                            const int32_t* kv_vbs, void* q_c, void* k_c, void* v_c, int64_t bh,
                            int64_t sq, int64_t skv, int32_t D, int32_t be, int32_t dtype,
                            void* stream) {
  if (!q || !k || !v || !q_vbs || !kv_vbs || !q_c || !k_c || !v_c) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, q_c, k_c, v_c) || !vsa_aligned<4>(q_vbs, kv_vbs))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || be <= 0 || sq <= 0 || skv <= 0 || sq % be || skv % be || !vec_dim_ok(D, dtype))
    return VSA_ERR_SHAPE;
  const int qb = (int)(sq / be), kb = (int)(skv / be);
  const int64_t grid = bh * (qb + 2 * (int64_t)kb);
  hipStream_t s = (hipStream_t)stream;
  VSA_DISPATCH_ALL(dtype, T, {
    hipLaunchKernelGGL(pool_qkv_kernel<T>, dim3((unsigned)grid), dim3(256), 0, s, (const T*)q,
                       (const T*)k, (const T*)v, q_vbs, kv_vbs, (T*)q_c, (T*)k_c, (T*)v_c, bh, qb,
                       kb, D, be);
  });
  return vsa_check_launch();
}

extern "C" int vsa_tile_pool_qkv(const void* q, const void* k, const void* v,
                                 const int32_t* slot_rows, const int32_t* q_vbs,
                                 const int32_t* kv_vbs, void* q_t,
                                 void* k_t, void* v_t, void* q_c, void* k_c, void* v_c,
                                 int64_t bh, int64_t s_out, int32_t heads, int32_t nb, int32_t D,
                                 int32_t be, int32_t dtype, void* stream) {
  if (!q || !k || !v || !slot_rows || !q_vbs || !kv_vbs || !q_t || !k_t || !v_t || !q_c ||
      !k_c || !v_c)
    return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q, k, v, q_t, k_t, v_t, q_c, k_c, v_c) ||
      !vsa_aligned<4>(slot_rows, q_vbs, kv_vbs))
    return VSA_ERR_ALIGN;
  if (heads < 0 || (heads > 0 && bh % heads)) return VSA_ERR_SHAPE;
  if (bh <= 0 || nb <= 0 || be <= 0 || be > 256 || s_out <= 0 || s_out > (int64_t)nb * be ||
      !vec_dim_ok(D, dtype))
    return VSA_ERR_SHAPE;
  const int64_t grid = 3 * bh * nb;
  if (grid > (1LL << 31) - 1) return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  VSA_DISPATCH_ALL(dtype, T, {
    hipLaunchKernelGGL(tile_pool_kernel<T>, dim3((unsigned)grid), dim3(256), 0, s, (const T*)q,
                       (const T*)k, (const T*)v, slot_rows, q_vbs, kv_vbs, (T*)q_t, (T*)k_t,
                       (T*)v_t,
                       (T*)q_c, (T*)k_c, (T*)v_c, bh, nb, D, be, s_out, heads);
  });
  return vsa_check_launch();
}

extern "C" int vsa_coarse_fwd(const void* q_c, const void* k_c, const void* v_c, float* scores,
                              float* probs, void* out_c, int32_t* selected, int64_t bh,
                              int32_t qb, int32_t kb, int32_t D, int32_t topk, float scale,
                              int32_t dtype, void* stream) {
  if (!q_c || !k_c || !v_c || !scores || !probs || !out_c) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q_c, k_c, v_c, scores, probs, out_c) || !vsa_aligned<4>(selected))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || bh > kMaxGridY || qb <= 0 || kb <= 0 || kb > max_coarse_blocks(D, dtype) ||
      D <= 0 || D > 1024)
    return VSA_ERR_SHAPE;
  if (selected && (topk < 1 || topk > kb)) return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (coarse_mfma_supported(D, dtype)) {
    const int rc = coarse_fwd_mfma(q_c, k_c, v_c, scores, probs, out_c, bh, qb, kb, D, scale,
                                   dtype, s);
    if (rc || !selected) return rc;
    return topk_radix(scores, selected, bh * qb, kb, topk, s);
  }
  const size_t shm = (size_t)(D + 2 * kb + 4) * sizeof(float);
  VSA_DISPATCH_ALL(dtype, T, {
    hipLaunchKernelGGL(coarse_fwd_kernel<T>, dim3(qb, (unsigned)bh), dim3(256), shm, s,
                       (const T*)q_c, (const T*)k_c, (const T*)v_c, scores, probs, (T*)out_c, qb,
                       kb, D, scale);
  });
  const int rc = vsa_check_launch();
  if (rc || !selected) return rc;
  return topk_radix(scores, selected, bh * qb, kb, topk, s);
}

extern "C" int vsa_topk(const float* scores, int32_t* selected, int64_t rows, int32_t kb,
                        int32_t topk, void* stream) {
  if (!scores || !selected) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(scores) || !vsa_aligned<4>(selected)) return VSA_ERR_ALIGN;
  if (rows <= 0 || kb <= 0 || kb > kMaxRouteBlocks || topk < 1 || topk > kb) return VSA_ERR_SHAPE;
  return topk_radix(scores, selected, rows, kb, topk, (hipStream_t)stream);
}

constexpr int kMaxCsrBlocks = 16000;  // Qb: a column of 500 words, 28 columns per workgroup

extern "C" int vsa_csr_build(const int32_t* selected, int32_t* counts, int32_t* offsets,
                             int32_t* inverse, int64_t bh, int32_t qb, int32_t kb, int32_t topk,
                             void* stream) {
  if (!selected || !counts || !offsets || !inverse) return VSA_ERR_NULL;
  if (!vsa_aligned<4>(selected, counts, offsets, inverse)) return VSA_ERR_ALIGN;
  if (bh <= 0 || bh > kMaxGridY || qb <= 0 || kb <= 0 || topk <= 0 || kb > kMaxCsrBlocks ||
      qb > kMaxCsrBlocks ||
      (int64_t)qb * topk > (1 << 30))
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int per = csr_cols_per_wg(bh, qb, kb);
  const int qw = (qb + 31) / 32;
  hipLaunchKernelGGL(csr_cols_kernel, dim3((unsigned)((kb + per - 1) / per), (unsigned)bh),
                     dim3(kCsrNT), (size_t)per * qw * sizeof(uint32_t), s, selected, counts,
                     offsets, inverse, qb, kb, topk, per);
  return vsa_check_launch();
}

extern "C" int vsa_bwd_prep(const void* fine_out, const void* dout, const void* out_c,
                            const void* gate, int32_t gate_mode, int32_t gate_heads,
                            float* delta, void* d_out_c, void* d_gate, int64_t bh, int64_t sq,
                            int32_t D, int32_t be, int32_t dtype, void* stream) {
  if (!fine_out || !dout || !delta) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(fine_out, dout, out_c, gate, d_out_c, d_gate) || !vsa_aligned<4>(delta))
    return VSA_ERR_ALIGN;
  const bool gate_f32 = (gate_mode & VSA_GATE_F32) != 0;
  gate_mode &= ~VSA_GATE_F32;
  if (gate_mode < 0 || gate_mode > 3 || (gate_f32 && gate_mode == 0)) return VSA_ERR_SHAPE;
  if (out_c && gate_mode == 3 && (gate_heads <= 0 || bh % gate_heads)) return VSA_ERR_SHAPE;
  if (out_c && !d_out_c) return VSA_ERR_NULL;
  if (out_c && gate_mode != 0 && (!gate || !d_gate)) return VSA_ERR_NULL;
  if (!out_c) gate_mode = 0;
  if (bh <= 0 || bh > kMaxGridY || be <= 0 || sq <= 0 || sq % be || !vec_dim_ok(D, dtype))
    return VSA_ERR_SHAPE;
  const int qb = (int)(sq / be);
  hipStream_t s = (hipStream_t)stream;
  const int gm = out_c ? gate_mode : -1;
  const dim3 grid(qb, (unsigned)bh);
  bool launched = false;
  VSA_DISPATCH_ALL(dtype, T, {
    if (gate_f32 && gm > 0)
      launched = (launch_bwd_prep<T, float, false>)(
          gm, grid, s, (const T*)fine_out, (const T*)dout, (const T*)out_c, (const float*)gate,
          gate_heads, delta, (T*)d_out_c, (float*)d_gate, qb, D, be, nullptr, 0, 0, nullptr);
    else
      launched = (launch_bwd_prep<T, T, false>)(
          gm, grid, s, (const T*)fine_out, (const T*)dout, (const T*)out_c, (const T*)gate,
          gate_heads, delta, (T*)d_out_c, (T*)d_gate, qb, D, be, nullptr, 0, 0, nullptr);
  });
  if (!launched) return VSA_ERR_SHAPE;
  return vsa_check_launch();
}

extern "C" int vsa_bwd_prep_tiled(const void* fine_out, const void* dout, const void* out_c,
                                  const void* gate, int32_t gate_mode, const int32_t* slot_rows,
                                  int64_t s_out, int32_t heads, float* delta, void* d_out_c,
                                  void* d_gate, void* dout_t, int64_t bh, int64_t sq, int32_t D,
                                  int32_t be, int32_t dtype, void* stream) {
  if (!fine_out || !dout || !delta || !slot_rows || !dout_t) return VSA_ERR_NULL;
  if (!vsa_aligned<16>(fine_out, dout, out_c, gate, d_out_c, d_gate, dout_t) ||
      !vsa_aligned<4>(delta, slot_rows))
    return VSA_ERR_ALIGN;
  if (heads < 0 || (heads > 0 && bh % heads)) return VSA_ERR_SHAPE;
  if (gate_mode < 0 || gate_mode > 2) return VSA_ERR_SHAPE;  // no token-major / fp32 gate here
  if (out_c && !d_out_c) return VSA_ERR_NULL;
  if (out_c && gate_mode != 0 && (!gate || !d_gate)) return VSA_ERR_NULL;
  if (!out_c) gate_mode = 0;
  if (bh <= 0 || bh > kMaxGridY || be <= 0 || sq <= 0 || sq % be || s_out <= 0 || s_out > sq ||
      !vec_dim_ok(D, dtype))
    return VSA_ERR_SHAPE;
  const int qb = (int)(sq / be);
  hipStream_t s = (hipStream_t)stream;
  const int gm = out_c ? gate_mode : -1;
  bool launched = false;
  VSA_DISPATCH_ALL(dtype, T, {
    launched = (launch_bwd_prep<T, T, true>)(
        gm, dim3(qb, (unsigned)bh), s, (const T*)fine_out, (const T*)dout, (const T*)out_c,
        (const T*)gate, 1, delta, (T*)d_out_c, (T*)d_gate, qb, D, be, slot_rows, s_out, heads,
        (T*)dout_t);
  });
  if (!launched) return VSA_ERR_SHAPE;
  return vsa_check_launch();
}

namespace vsa {
bool combine_f32gate_shape_ok(int64_t bh, int64_t sq, int D, int be, int dtype) {
  return bh > 0 && bh <= kMaxGridY && be > 0 && sq > 0 && sq % be == 0 && vec_dim_ok(D, dtype);
}

int combine_f32gate(const void* fine, const void* out_c, const void* gate, int gate_mode,
                    int gate_heads, void* out, int64_t bh, int64_t sq, int D, int be, int dtype,
                    hipStream_t s) {
  if (!combine_f32gate_shape_ok(bh, sq, D, be, dtype)) return VSA_ERR_SHAPE;
  const int qb = (int)(sq / be);
  VSA_DISPATCH_ALL(dtype, T, {
    hipLaunchKernelGGL((combine_f32gate_kernel<T>), dim3(qb, (unsigned)bh), dim3(256), 0, s,
                       (const T*)fine, (const T*)out_c, (const float*)gate, gate_mode,
                       gate_heads, (T*)out, qb, D, be);
  });
  return vsa_check_launch();
}
}  // namespace vsa

extern "C" int vsa_coarse_bwd(const void* q_c, const void* k_c, const void* v_c,
                              const float* probs, const void* d_out_c, float* ds, void* d_q_c,
                              void* d_k_c, void* d_v_c, int64_t bh, int32_t qb, int32_t kb,
                              int32_t D, float scale, int32_t dtype, void* stream) {
  if (!q_c || !k_c || !v_c || !probs || !d_out_c || !ds || !d_q_c || !d_k_c || !d_v_c)
    return VSA_ERR_NULL;
  if (!vsa_aligned<16>(q_c, k_c, v_c, probs, d_out_c, ds, d_q_c, d_k_c, d_v_c))
    return VSA_ERR_ALIGN;
  if (bh <= 0 || bh > kMaxGridY || qb <= 0 || kb <= 0 || kb > max_coarse_blocks(D, dtype) ||
      D <= 0 || D > 1024)
    return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (coarse_mfma_supported(D, dtype))
    return coarse_bwd_mfma(q_c, k_c, v_c, probs, d_out_c, ds, d_q_c, d_k_c, d_v_c, bh, qb, kb, D,
                           scale, dtype, s);
  const size_t shm = (size_t)(D + kb + 4) * sizeof(float);
  int rc = 0;
  VSA_DISPATCH_ALL(dtype, T, {
    hipLaunchKernelGGL(coarse_bwd_rows_kernel<T>, dim3(qb, (unsigned)bh), dim3(256), shm, s,
                       (const T*)k_c, (const T*)v_c, probs, (const T*)d_out_c, ds, (T*)d_q_c, qb,
                       kb, D, scale);
    rc = vsa_check_launch();
    if (rc == 0)
      hipLaunchKernelGGL(coarse_bwd_cols_kernel<T>, dim3(kb, (unsigned)bh), dim3(256), 0, s,
                         (const T*)q_c, probs, (const T*)d_out_c, ds, (T*)d_k_c, (T*)d_v_c, qb,
                         kb, D);
  });
  if (rc) return rc;
  return vsa_check_launch();
}
