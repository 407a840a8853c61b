// Coarse (pooled-token) attention on gfx950 MFMA, its backward, and the Top-K
// route: the T-dtype softmax attention of common.py:159-166 over the block
// means, the per-row top-k of triton_impl.py:1710, and the autograd of the
// coarse branch.  These replace the one-row-per-workgroup kernels of
// common.hip for bf16 / fp16 with head_dim 64 or 128 (the shapes the fine
// kernels run); other dtypes / widths keep the generic kernels.
//
// Layout of the tiles: a workgroup owns 32 rows (query blocks, or key blocks
// in the column pass) and its 4 waves stride over 32-wide tiles of the other
// side.  Products are taken transposed (S^T = K Q^T, dP^T = V G^T) so that a
// lane owns one row and holds 16 of its columns: row statistics are a lane
// reduction plus one xor-32 exchange.  Results that sum over the strided
// tiles are reduced across the 4 waves in LDS in fixed wave order, so every
// output is deterministic.
//
// Rounding points follow the reference in T: scores T(T(q_c k_c) * scale),
// probabilities T(softmax), out_c T(P v_c); backward dP = T(G v_c^T),
// dS = T(T(P (dP - rowsum(P dP))) * scale), d_q_c = T(dS k_c),
// d_k_c = T(dS^T q_c), d_v_c = T(P^T G).
#include "coarse.h"

#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

namespace {

constexpr int kRows = 32;  // rows per workgroup
constexpr int kWaves = 4;

// B-operand fragments of 32 rows of a [rows, D] matrix: lane (r, h) holds
// row base + r (clamped to the last row), dims 16 ks + 8h .. +7.
template <typename T, int D>
__device__ __forceinline__ void load_rows_b(const T* __restrict__ m, int base, int rows,
                                            typename Elem<T>::vec8 (&f)[D / 16]) {
  const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int row = min(base + r, rows - 1);
  const T* p = m + (int64_t)row * D + 8 * h;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    f[ks] = as_vec8<T>(*reinterpret_cast<const u32x4*>(p + 16 * ks));
}

// Copy 32 rows of a [rows, D] matrix (rows past the end repeat the last row)
// into this wave's swizzled LDS tile, for transpose reads.  Every load is
// issued before the first LDS store: stored as it arrived, each chunk waited
// for its own load (one memory round trip per chunk).
template <typename T, int D>
__device__ __forceinline__ void stage_rows(T* tile, const T* __restrict__ m, int base, int rows) {
  const int lane = threadIdx.x & 63;
  constexpr int CH = 32 * D / 8;  // 16-byte chunks
  constexpr int N = CH / 64;      // per lane
  static_assert(CH % 64 == 0, "whole 16-byte chunks per lane");
  u32x4 v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int c = lane + 64 * i;
    const int row = c / (D / 8), ch = c % (D / 8);
    const int src = min(base + row, rows - 1);
    v[i] = *reinterpret_cast<const u32x4*>(m + (int64_t)src * D + ch * 8);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int c = lane + 64 * i;
    *reinterpret_cast<u32x4*>(tile + swz<D>(c / (D / 8), c % (D / 8))) = v[i];
  }
}

// key (or row) index of accumulator element i in a lane with half h
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// Sum a wave's [32 x D] transposed accumulators (lane (r, h) holds column r,
// rows mt*32 + acc_row) across the 4 waves in wave order into red[32][D].
template <int D>
__device__ __forceinline__ void reduce_waves(const f32x16 (&acc)[D / 32], float* red) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  __syncthreads();  // `red` may alias the waves' operand tiles
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float* dst = &red[r * D + mt * 32 + acc_row(i, h)];
          *dst = (w == 0 ? 0.f : *dst) + acc[mt][i];
        }
    }
    __syncthreads();
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward: scores, probabilities, out_c.  grid (ceil(Qb/32), BH), 256 threads.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void coarse_fwd_mfma_kernel(
    const T* __restrict__ qc, const T* __restrict__ kc, const T* __restrict__ vc,
    float* __restrict__ scores, float* __restrict__ probs, T* __restrict__ outc, int qb, int kb,
    float scale) {
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) T vtile[kWaves][32 * D];
  __shared__ float stat[kWaves][2][32];
  float* red = reinterpret_cast<float*>(&vtile[0][0]);  // after the tile loop
  const int64_t b = blockIdx.y;
  const int q0 = blockIdx.x * kRows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int myq = q0 + r;
  const bool qvalid = myq < qb;
  const T* qb_ = qc + b * qb * (int64_t)D;
  const T* kb_ = kc + b * kb * (int64_t)D;
  const T* vb_ = vc + b * kb * (int64_t)D;
  float* srow = scores + (b * qb + myq) * (int64_t)kb;
  float* prow = probs + (b * qb + myq) * (int64_t)kb;
  const int ntile = (kb + 31) / 32;
  const bool vec4 = (kb & 3) == 0;  // rows of the [.., Kb] fp32 buffers are 16-byte aligned

  V8 qf[D / 16];
  load_rows_b<T, D>(qb_, q0, qb, qf);

  // S^T tile (keys x queries) for key tile kt, rounded as the reference does
  auto scores_tile = [&](int kt, float (&s)[16]) {
    V8 kf[D / 16];
    load_rows_b<T, D>(kb_, kt * 32, kb, kf);  // A rows: key kt*32 + r
    f32x16 acc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) acc = E::mfma32(kf[ks], qf[ks], acc);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kt * 32 + acc_row(i, h);
      s[i] = key < kb ? round_t<T>(round_t<T>(acc[i]) * scale) : -INFINITY;
    }
  };

  // pass 1: scores out, running max / sum per query (lane-partial sums)
  float m = -INFINITY, l = 0.f;
  for (int kt = wave; kt < ntile; kt += kWaves) {
    float s[16];
    scores_tile(kt, s);
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mn = fmaxf(m, tmax);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) part += expf(s[i] - mn);
    l = l * expf(m - mn) + part;
    m = mn;
    if (qvalid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int key0 = kt * 32 + 8 * g + 4 * h;
        if (vec4 && key0 + 3 < kb) {
          f32x4 v4 = {s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]};
          *reinterpret_cast<f32x4*>(srow + key0) = v4;
        } else {
          for (int e = 0; e < 4; ++e)
            if (key0 + e < kb) srow[key0 + e] = s[4 * g + e];
        }
      }
    }
  }
  l += __shfl_xor(l, 32, 64);
  if (h == 0) {
    stat[wave][0][r] = m;
    stat[wave][1][r] = l;
  }
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, stat[w][0][r]);
  float L = 0.f;
  for (int w = 0; w < kWaves; ++w) {
    const float mw = stat[w][0][r];
    if (mw != -INFINITY) L += stat[w][1][r] * expf(mw - M);
  }

  // pass 2: probabilities out, out_c^T += V^T P^T
  f32x16 oacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) oacc[mt] = f32x16{};
  T* vt = &vtile[wave][0];
  for (int kt = wave; kt < ntile; kt += kWaves) {
    float s[16];
    scores_tile(kt, s);
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = round_t<T>(expf(s[i] - M) / L);  // 0 for padding keys
    if (qvalid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int key0 = kt * 32 + 8 * g + 4 * h;
        if (vec4 && key0 + 3 < kb) {
          f32x4 v4 = {p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]};
          *reinterpret_cast<f32x4*>(prow + key0) = v4;
        } else {
          for (int e = 0; e < 4; ++e)
            if (key0 + e < kb) prow[key0 + e] = p[4 * g + e];
        }
      }
    }
    stage_rows<T, D>(vt, vb_, kt * 32, kb);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const V8 bp = pack8<T>(p + 8 * kk);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        oacc[mt] = E::mfma32(tr_a8<T, D>(vt, mt * 32, 16 * kk, 16 * kk + 8), bp, oacc[mt]);
    }
  }
  reduce_waves<D>(oacc, red);
  for (int x = threadIdx.x; x < 32 * D; x += 256) {
    const int row = x / D, d = x % D;
    if (q0 + row < qb) outc[(b * qb + q0 + row) * (int64_t)D + d] = E::from_f(red[x]);
  }
}

// ---------------------------------------------------------------------------
// Top-K by radix select on the total-order score key (one workgroup per row):
// the k-th largest key T is found digit by digit (4 x 8 bits); every key above
// T is taken, and keys equal to T are taken by ascending id until topk ids are
// chosen -- the rule "larger score, then smaller id".  Ids are written in
// ascending order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void topk_radix_kernel(const float* __restrict__ scores,
                                                         int32_t* __restrict__ selected, int kb,
                                                         int topk) {
  extern __shared__ uint32_t keys[];  // kb
  __shared__ int hist[256];
  __shared__ int wsum[4][2];
  __shared__ int digit_sel[2];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int j = tid; j < kb; j += 256)
    keys[j] = (uint32_t)order_key(scores[row * kb + j]) ^ 0x80000000u;  // unsigned order
  __syncthreads();
  uint32_t prefix = 0, mask = 0;
  int remaining = topk;  // how many of the keys matching `prefix` are still to be taken
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int j = tid; j < kb; j += 256) {
      const uint32_t u = keys[j];
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    // suffix sums: hist[d] <- number of matching keys with digit >= d
    for (int o = 1; o < 256; o <<= 1) {
      const int add = tid + o < 256 ? hist[tid + o] : 0;
      __syncthreads();
      hist[tid] += add;
      __syncthreads();
    }
    const int above = tid < 255 ? hist[tid + 1] : 0;  // digit > tid
    if (hist[tid] >= remaining && above < remaining) {
      digit_sel[0] = tid;
      digit_sel[1] = above;
    }
    __syncthreads();
    const int d = digit_sel[0];
    remaining -= digit_sel[1];
    prefix |= (uint32_t)d << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  // prefix = T (k-th largest); `remaining` keys equal to T are taken, by id
  const uint32_t kth = prefix;
  int taken = 0, eq_seen = 0;
  int32_t* dst = selected + row * topk;
  for (int j0 = 0; j0 < kb; j0 += 256) {
    const int j = j0 + tid;
    const uint32_t u = j < kb ? keys[j] : 0u;
    const bool eq = j < kb && u == kth;
    const uint64_t beq = __ballot(eq);
    const int eq_before = __popcll(beq & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[wave][0] = __popcll(beq);
    __syncthreads();
    int eq_off = eq_seen;
    for (int w = 0; w < wave; ++w) eq_off += wsum[w][0];
    const bool sel = j < kb && (u > kth || (eq && eq_off + eq_before < remaining));
    const uint64_t bsel = __ballot(sel);
    const int sel_before = __popcll(bsel & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[wave][1] = __popcll(bsel);
    __syncthreads();
    int sel_off = taken;
    for (int w = 0; w < wave; ++w) sel_off += wsum[w][1];
    if (sel && sel_off + sel_before < topk) dst[sel_off + sel_before] = j;
    for (int w = 0; w < 4; ++w) {
      eq_seen += wsum[w][0];
      taken += wsum[w][1];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Backward, rows: dP, softmax backward, dS out, d_q_c.  grid (ceil(Qb/32), BH).
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void coarse_bwd_rows_mfma_kernel(
    const T* __restrict__ kc, const T* __restrict__ vc, const float* __restrict__ probs,
    const T* __restrict__ d_outc, float* __restrict__ ds, T* __restrict__ d_qc, int qb, int kb,
    float scale) {
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) T ktile[kWaves][32 * D];
  __shared__ float stat[kWaves][32];
  float* red = reinterpret_cast<float*>(&ktile[0][0]);  // after the tile loop
  const int64_t b = blockIdx.y;
  const int q0 = blockIdx.x * kRows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int myq = q0 + r;
  const bool qvalid = myq < qb;
  const int qrow = min(myq, qb - 1);
  const T* kb_ = kc + b * kb * (int64_t)D;
  const T* vb_ = vc + b * kb * (int64_t)D;
  const float* prow = probs + (b * qb + qrow) * (int64_t)kb;
  float* dsrow = ds + (b * qb + myq) * (int64_t)kb;
  const int ntile = (kb + 31) / 32;
  const bool vec4 = (kb & 3) == 0;  // rows of the [.., Kb] fp32 buffers are 16-byte aligned

  V8 gf[D / 16];
  load_rows_b<T, D>(d_outc + b * qb * (int64_t)D, q0, qb, gf);

  // dP^T tile (keys x queries), rounded to T; probabilities of the same entries
  auto dp_tile = [&](int kt, float (&dp)[16], float (&p)[16]) {
    V8 vf[D / 16];
    load_rows_b<T, D>(vb_, kt * 32, kb, vf);
    f32x16 acc = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) acc = E::mfma32(vf[ks], gf[ks], acc);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int key0 = kt * 32 + 8 * g + 4 * h;
      if (vec4 && key0 + 3 < kb) {
        const f32x4 p4 = *reinterpret_cast<const f32x4*>(prow + key0);
#pragma unroll
        for (int e = 0; e < 4; ++e) p[4 * g + e] = p4[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) p[4 * g + e] = key0 + e < kb ? prow[key0 + e] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) dp[i] = round_t<T>(acc[i]);
  };

  float part = 0.f;
  for (int kt = wave; kt < ntile; kt += kWaves) {
    float dp[16], p[16];
    dp_tile(kt, dp, p);
#pragma unroll
    for (int i = 0; i < 16; ++i) part = fmaf(p[i], dp[i], part);
  }
  part += __shfl_xor(part, 32, 64);
  if (h == 0) stat[wave][r] = part;
  __syncthreads();
  float rsum = 0.f;
  for (int w = 0; w < kWaves; ++w) rsum += stat[w][r];

  f32x16 qacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) qacc[mt] = f32x16{};
  T* kt_ = &ktile[wave][0];
  for (int kt = wave; kt < ntile; kt += kWaves) {
    float dp[16], p[16];
    dp_tile(kt, dp, p);
    float dsv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) dsv[i] = round_t<T>(round_t<T>(p[i] * (dp[i] - rsum)) * scale);
    if (qvalid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int key0 = kt * 32 + 8 * g + 4 * h;
        if (vec4 && key0 + 3 < kb) {
          f32x4 v4 = {dsv[4 * g], dsv[4 * g + 1], dsv[4 * g + 2], dsv[4 * g + 3]};
          *reinterpret_cast<f32x4*>(dsrow + key0) = v4;
        } else {
          for (int e = 0; e < 4; ++e)
            if (key0 + e < kb) dsrow[key0 + e] = dsv[4 * g + e];
        }
      }
    }
    stage_rows<T, D>(kt_, kb_, kt * 32, kb);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const V8 bs = pack8<T>(dsv + 8 * kk);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt)
        qacc[mt] = E::mfma32(tr_a8<T, D>(kt_, mt * 32, 16 * kk, 16 * kk + 8), bs, qacc[mt]);
    }
  }
  reduce_waves<D>(qacc, red);
  for (int x = threadIdx.x; x < 32 * D; x += 256) {
    const int row = x / D, d = x % D;
    if (q0 + row < qb) d_qc[(b * qb + q0 + row) * (int64_t)D + d] = E::from_f(red[x]);
  }
}

// ---------------------------------------------------------------------------
// Backward, columns: d_k_c = T(dS^T q_c), d_v_c = T(P^T d_out_c).
// grid (ceil(Kb/32), BH); waves stride over 32-query tiles.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void coarse_bwd_cols_mfma_kernel(
    const T* __restrict__ qc, const float* __restrict__ probs, const T* __restrict__ d_outc,
    const float* __restrict__ ds, T* __restrict__ d_kc, T* __restrict__ d_vc, int qb, int kb) {
  using E = Elem<T>;
  typedef typename E::vec8 V8;
  __shared__ __attribute__((aligned(16))) T qtile[kWaves][32 * D];
  __shared__ __attribute__((aligned(16))) T gtile[kWaves][32 * D];
  float* red = reinterpret_cast<float*>(&qtile[0][0]);  // after the tile loop
  const int64_t b = blockIdx.y;
  const int k0 = blockIdx.x * kRows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int mykey = min(k0 + r, kb - 1);
  const T* qb_ = qc + b * qb * (int64_t)D;
  const T* gb_ = d_outc + b * qb * (int64_t)D;
  const float* dsb = ds + b * qb * (int64_t)kb;
  const float* pb = probs + b * qb * (int64_t)kb;
  const int ntile = (qb + 31) / 32;

  f32x16 kacc[D / 32], vacc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt) {
    kacc[mt] = f32x16{};
    vacc[mt] = f32x16{};
  }
  T* qt = &qtile[wave][0];
  T* gt = &gtile[wave][0];
  for (int t = wave; t < ntile; t += kWaves) {
    stage_rows<T, D>(qt, qb_, t * 32, qb);
    stage_rows<T, D>(gt, gb_, t * 32, qb);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      // B operands: dS[q][key r], P[q][key r] for the 8 queries this lane feeds
      float dsv[8], pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int q = t * 32 + 16 * kk + 8 * (e >> 2) + 4 * h + (e & 3);
        const bool ok = q < qb;
        // clamped row, loaded unconditionally (a load under the condition
        // became a branch and a wait per value), zeroed after
        const int64_t at = (int64_t)min(q, qb - 1) * kb + mykey;
        const float dl = dsb[at], pl = pb[at];
        dsv[e] = ok ? dl : 0.f;
        pv[e] = ok ? pl : 0.f;
      }
      const V8 bs = pack8<T>(dsv);
      const V8 bp = pack8<T>(pv);
#pragma unroll
      for (int mt = 0; mt < D / 32; ++mt) {
        kacc[mt] = E::mfma32(tr_a8<T, D>(qt, mt * 32, 16 * kk, 16 * kk + 8), bs, kacc[mt]);
        vacc[mt] = E::mfma32(tr_a8<T, D>(gt, mt * 32, 16 * kk, 16 * kk + 8), bp, vacc[mt]);
      }
    }
  }
  reduce_waves<D>(kacc, red);
  for (int x = threadIdx.x; x < 32 * D; x += 256) {
    const int row = x / D, d = x % D;
    if (k0 + row < kb) d_kc[(b * kb + k0 + row) * (int64_t)D + d] = E::from_f(red[x]);
  }
  __syncthreads();
  reduce_waves<D>(vacc, red);
  for (int x = threadIdx.x; x < 32 * D; x += 256) {
    const int row = x / D, d = x % D;
    if (k0 + row < kb) d_vc[(b * kb + k0 + row) * (int64_t)D + d] = E::from_f(red[x]);
  }
}

// ---------------------------------------------------------------------------
// Host launchers (called by the C ABI in common.hip)
// ---------------------------------------------------------------------------
bool coarse_mfma_supported(int D, int dtype) {
  return (dtype == VSA_BF16 || dtype == VSA_F16) && (D == 64 || D == 128);
}

int coarse_fwd_mfma(const void* qc, const void* kc, const void* vc, float* scores, float* probs,
                    void* outc, int64_t bh, int qb, int kb, int D, float scale, int dtype,
                    hipStream_t s) {
  if (bh > 65535) return VSA_ERR_SHAPE;
  const dim3 grid((qb + kRows - 1) / kRows, (unsigned)bh);
#define VSA_CF(DD)                                                                              \
  if (D == DD) {                                                                                \
    hipLaunchKernelGGL((coarse_fwd_mfma_kernel<T, DD>), grid, dim3(256), 0, s, (const T*)qc,   \
                       (const T*)kc, (const T*)vc, scores, probs, (T*)outc, qb, kb, scale);   \
    return vsa_check_launch();                                                                  \
  }
  VSA_DISPATCH_MFMA(dtype, T, { VSA_CF(64) VSA_CF(128) });
#undef VSA_CF
  return VSA_ERR_UNSUPPORTED;
}

int topk_radix(const float* scores, int32_t* selected, int64_t rows, int kb, int topk,
               hipStream_t s) {
  if (rows > 0x7fffffffLL) return VSA_ERR_SHAPE;
  hipLaunchKernelGGL(topk_radix_kernel, dim3((unsigned)rows), dim3(256),
                     (size_t)kb * sizeof(uint32_t), s, scores, selected, kb, topk);
  return vsa_check_launch();
}

int coarse_bwd_mfma(const void* qc, const void* kc, const void* vc, const float* probs,
                    const void* d_outc, float* ds, void* d_qc, void* d_kc, void* d_vc,
                    int64_t bh, int qb, int kb, int D, float scale, int dtype, hipStream_t s) {
  if (bh > 65535) return VSA_ERR_SHAPE;
  const dim3 grows((qb + kRows - 1) / kRows, (unsigned)bh);
  const dim3 gcols((kb + kRows - 1) / kRows, (unsigned)bh);
#define VSA_CB(DD)                                                                               \
  if (D == DD) {                                                                                 \
    hipLaunchKernelGGL((coarse_bwd_rows_mfma_kernel<T, DD>), grows, dim3(256), 0, s,            \
                       (const T*)kc, (const T*)vc, probs, (const T*)d_outc, ds, (T*)d_qc, qb,   \
                       kb, scale);                                                               \
    int rc = vsa_check_launch();                                                                 \
    if (rc) return rc;                                                                           \
    hipLaunchKernelGGL((coarse_bwd_cols_mfma_kernel<T, DD>), gcols, dim3(256), 0, s,            \
                       (const T*)qc, probs, (const T*)d_outc, ds, (T*)d_kc, (T*)d_vc, qb, kb);  \
    return vsa_check_launch();                                                                   \
  }
  VSA_DISPATCH_MFMA(dtype, T, { VSA_CB(64) VSA_CB(128) });
#undef VSA_CB
  return VSA_ERR_UNSUPPORTED;
}

}  // namespace vsa
