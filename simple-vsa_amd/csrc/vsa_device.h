// Device-side helpers shared by the gfx950 VSA kernels.
//
// Conventions used by every kernel in this directory:
//  * tensors are dense row-major [B*H, S, D] (the reference's BHSD layout made
//    contiguous, triton_impl.py:1593-1595);
//  * fp32 accumulation everywhere, stores rounded to the element type T with
//    round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950);
//  * MFMA tiles are CDNA4's v_mfma_f32_32x32x16_{bf16,f16}.  For a wave with
//    lane = 32*h + r (r in 0..31, h in 0..1):
//       A (32 x 16, M x K): lane holds row r, k = 8h .. 8h+7
//       B (16 x 32, K x N): lane holds col r, k = 8h .. 8h+7
//       C (32 x 32, M x N): acc[i] is row 8*(i/4) + 4h + (i%4), col r
//    Because a C tile's per-lane rows are {16j + 4h + 0..3, 16j + 8 + 4h + 0..3}
//    for acc[8j .. 8j+7], a C tile converted to T can be fed straight back as
//    the B (or A) operand of a product that reduces over the C tile's rows,
//    provided the other operand enumerates those rows in the same order:
//    tr_a8 below reads a row-major LDS tile "down a column" in exactly that
//    order with ds_read_b64_tr_b16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vsa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Element traits
// ---------------------------------------------------------------------------
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_f(__bf16 x) { return (float)x; }
  static __device__ __forceinline__ __bf16 from_f(float x) { return (__bf16)x; }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Elem<_Float16> {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
  static __device__ __forceinline__ _Float16 from_f(float x) { return (_Float16)x; }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Elem<float> {
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
};

// Round an fp32 value through T and back (the reference's "computed in fp32,
// stored in T" points).
template <typename T>
__device__ __forceinline__ float round_t(float x) {
  return Elem<T>::to_f(Elem<T>::from_f(x));
}

// Pack 8 fp32 values (two groups of 4) into an MFMA operand of T.
template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 pack8(const float* v) {
  typename Elem<T>::vec8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = Elem<T>::from_f(v[e]);
  return r;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::vec8 as_vec8(u32x4 x) {
  return __builtin_bit_cast(typename Elem<T>::vec8, x);
}

// Token r of head bh in a raster-order sequence of s_out tokens: head-major
// [B*H, s_out, ...] rows when heads == 0, token-major [B, s_out, H, ...] rows
// (the layout a projection writes) when heads == H.
__device__ __forceinline__ int64_t raster_row(int64_t bh, int r, int64_t s_out, int heads) {
  if (heads == 0) return bh * s_out + r;
  const int b = (int)bh;  // batch*heads < 2^31 (the entry points check it)
  return ((int64_t)(b / heads) * s_out + r) * heads + b % heads;
}

// Streaming global accesses for data a pass touches once: non-temporal loads
// of the token rows in the block means, the backward preprocessing and the
// fp32-gate combine, loads and 16-byte stores of the row moves (8-12 % faster
// there).  The fine kernels' 8-byte epilogue stores and the gate's loads and
// stores measured slower with them (up to 8 %), so those stay plain.
template <typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
  return __builtin_nontemporal_load(p);
}
template <typename V>
__device__ __forceinline__ void st_stream(V* p, V v) {
  __builtin_nontemporal_store(v, p);
}

// Total-order integer key of a score: larger score -> larger key; -0 == +0;
// NaN above +inf (torch.topk's ranking).
__device__ __forceinline__ int order_key(float x) {
  uint32_t u = __float_as_uint(x + 0.0f);  // folds -0 into +0
  if (x != x) u = 0x7fffffffu;             // NaN: larger than +inf
  return (int)u >= 0 ? (int)u : (int)(u ^ 0x7fffffffu);
}

// ---------------------------------------------------------------------------
// Swizzled row-major LDS tiles.
//
// A tile X[s][d] (s = sequence row, d = head dim, D elements per row) is kept
// unpadded; its 16-byte chunk c of row r lives at chunk position c ^ f(r).
// The XOR keeps three access patterns free of bank conflicts on the 64-bank
// gfx950 LDS:
//   * MFMA row reads: 16 lanes read chunk c of 16 consecutive rows;
//   * stores: 16 lanes write the 16 chunks of one row (D = 128) or two rows
//     (D = 64);
//   * transpose reads (ds_read_b64_tr_b16): 32 lanes read 8 bytes each from 4
//     consecutive rows x 64 contiguous bytes.
// For D = 64 two rows form one 256-byte super-row and the XOR acts on it.
// Returns the element offset of the first element of the chunk.
// ---------------------------------------------------------------------------
template <int D>
__host__ __device__ __forceinline__ int swz(int r, int c);

template <>
__host__ __device__ __forceinline__ int swz<128>(int r, int c) {
  return r * 128 + ((c ^ (((r & 3) << 2) | ((r >> 2) & 3))) << 3);
}

// D = 256: a row is two 128-element halves (256 bytes each, one pass over the
// 64 banks), each swizzled as a D = 128 row.
template <>
__host__ __device__ __forceinline__ int swz<256>(int r, int c) {
  return r * 256 + ((c >> 4) << 7) + (((c & 15) ^ (((r & 3) << 2) | ((r >> 2) & 3))) << 3);
}

template <>
__host__ __device__ __forceinline__ int swz<64>(int r, int c) {
  const int R = r >> 1, C = ((r & 1) << 3) | c;
  return R * 128 + ((C ^ (((R & 1) << 2) | ((R >> 1) & 3))) << 3);
}

// Element offset of X[r][d] for d a multiple of 4 (8-byte aligned pieces).
template <int D>
__host__ __device__ __forceinline__ int swz_elem(int r, int d) {
  return swz<D>(r, d >> 3) + (d & 7);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// A operand (32 x 16, rows m = d0 .. d0+31, k = 8 sequence rows) of a
// 32x32x16 MFMA that reduces over the sequence, read from a swizzled
// row-major tile X[s][d] with two ds_read_b64_tr_b16.  Lane (r, h) receives
// X[sA(h) + 0..3][d0 + r] followed by X[sB(h) + 0..3][d0 + r], where
// sA(h) = sa + 4h and sB(h) = sb + 4h.
//
// ds_read_b64_tr_b16 (gfx950): inside each 16-lane group, lane i receives
// element i%4 of the 8-byte pieces addressed by lanes i/4, 4+i/4, 8+i/4 and
// 12+i/4 of that group.  Lane j = 4e + g of group (q, h) therefore addresses
// row s + e, dims d0 + 16q + 4g .. +3.
template <typename T, int D>
__device__ __forceinline__ typename Elem<T>::vec8 tr_a8(const T* X, int d0, int sa, int sb) {
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 4, j = lane & 15;
  const int q = grp & 1, h = grp >> 1;
  const int d = d0 + 16 * q + 4 * (j & 3);
  const int e = j >> 2;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(X + swz_elem<D>(sa + 4 * h + e, d)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(X + swz_elem<D>(sb + 4 * h + e, d)));
  u32x4 r;
  r[0] = __builtin_bit_cast(u32x2, lo)[0];
  r[1] = __builtin_bit_cast(u32x2, lo)[1];
  r[2] = __builtin_bit_cast(u32x2, hi)[0];
  r[3] = __builtin_bit_cast(u32x2, hi)[1];
  return as_vec8<T>(r);
}

// Row read for an MFMA operand: lane (r, h) gets X[row][16*ks + 8h .. +7].
template <typename T, int D>
__device__ __forceinline__ typename Elem<T>::vec8 row_a8(const T* X, int row, int ks, int h) {
  return as_vec8<T>(*reinterpret_cast<const u32x4*>(X + swz<D>(row, 2 * ks + h)));
}

// ---------------------------------------------------------------------------
// Direct global -> LDS copies (global_load_lds_dwordx4: lane i of a wave
// writes 16 bytes at LDS base + 16*i).  Each lane fetches the global chunk
// that the swizzle places at its LDS slot, so a row-major global tile lands
// in the swizzled layout without passing through VGPRs.  Completion is
// tracked by vmcnt: call dma_wait() before the barrier that publishes it.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

template <int D>
__host__ __device__ __forceinline__ int unswz_row_chunk(int P, int& c);  // P: LDS chunk index

template <>
__host__ __device__ __forceinline__ int unswz_row_chunk<128>(int P, int& c) {
  const int row = P >> 4;
  c = (P & 15) ^ (((row & 3) << 2) | ((row >> 2) & 3));
  return row;
}

template <>
__host__ __device__ __forceinline__ int unswz_row_chunk<256>(int P, int& c) {
  const int row = P >> 5, q = P & 31;
  c = (q & 16) | ((q & 15) ^ (((row & 3) << 2) | ((row >> 2) & 3)));
  return row;
}

template <>
__host__ __device__ __forceinline__ int unswz_row_chunk<64>(int P, int& c) {
  const int R = P >> 4;
  const int C = (P & 15) ^ (((R & 1) << 2) | ((R >> 1) & 3));
  c = C & 7;
  return 2 * R + (C >> 3);
}

// One global_load_lds_dwordx4 for this wave: lane i copies 16 bytes from `g`
// to LDS byte address lds + 16*i (`lds` wave-uniform, passed through M0).
// Issued as inline asm on purpose: when the compiler sees an LDS DMA in
// flight it puts vmcnt(0) in front of later LDS reads it cannot disambiguate
// (the transpose reads), which would drain the prefetch.  Every consumer of
// the copied tile waits on vmcnt explicitly (dma_wait) before its barrier.
// An LDS DMA that follows an SALU write of M0 needs one wait state (GFX9
// hazard; the compiler inserts it for the copies it issues itself, not inside
// an asm statement), hence the s_nop 0.  M0 is reserved to the compiler, which
// sets it before each of its own uses, so it is not listed as clobbered.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
               "s"(lds)
               : "memory");
}

// Same with 4 bytes per lane (LDS byte address lds + 4*i).
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds)
               : "memory");
}

// Same as dma16 with a scalar 64-bit base and a 32-bit per-lane byte offset
// (saddr form: no per-lane 64-bit address arithmetic).
__device__ __forceinline__ void dma16_s(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff),
               "s"(sbase), "s"(lds)
               : "memory");
}

// An empty side effect that keeps a uniform branch a branch: where the guard is
// implied by the guarded per-lane conditions (a partial-chunk mask), the
// compiler would otherwise drop it and run the selects on every iteration.
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

// A wave-uniform value redefined at this point: comparisons derived from it
// inside a rarely taken branch stay in the branch instead of being hoisted
// (and run on every iteration) in front of it.
__device__ __forceinline__ int uniform_here(int x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Keep a lane-dependent value in a register: the compiler would otherwise
// rematerialise address arithmetic at every use inside a loop.
template <typename X>
__device__ __forceinline__ X opaque(X x) {
  asm volatile("" : "+v"(x));
  return x;
}

// x / c for an integer-valued c >= 1, correctly rounded, given r = RN(1/c):
// q = x * r is within an ulp of x / c, and one FMA residual step rounds it
// correctly (Markstein's theorem) -- three operations instead of a full
// division.  Bit-identical to the division for every finite bf16 x, every
// finite fp16 x and every c in [1, 1024] (checked exhaustively on the host).
__device__ __forceinline__ float div_by_count(float x, float c, float r) {
  const float q0 = x * r;
  return fmaf(fmaf(-q0, c, x), r, q0);
}

// Compute a value at this program point: the compiler sinks arithmetic whose
// only use sits in a later conditional block into that block, which would
// move work scheduled under one phase's MFMAs into the next phase.
__device__ __forceinline__ float here(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Copy a NROWS x D row-major global tile into the swizzled LDS tile `dst`.
// All NT threads of the workgroup call it.
template <typename T, int D, int NROWS, int NT>
__device__ __forceinline__ void dma_tile(T* dst, const T* __restrict__ src) {
  constexpr int CHUNKS = NROWS * D / 8;
  static_assert(CHUNKS % NT == 0, "tile must split evenly over the workgroup");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < CHUNKS / NT; ++i) {
    const int blk = i * (NT / 64) + wave;  // 1 KiB block written by this wave
    int c;
    const int row = unswz_row_chunk<D>(blk * 64 + lane, c);
    dma16(src + row * D + c * 8,
          __builtin_amdgcn_readfirstlane(lds_addr(dst + blk * (1024 / (int)sizeof(T)))));
  }
}

// dma_tile with the scalar-base form: the lane offsets of a NROWS x D tile are
// computed once (they do not depend on which tile is copied) and every copy
// passes only the wave-uniform global base, so no 64-bit per-lane addresses
// stay live across a loop.
template <typename T, int D, int NROWS, int NT>
struct TileDma {
  static constexpr int N = NROWS * D / 8 / NT;
  static_assert(NROWS * D / 8 % NT == 0, "tile must split evenly over the workgroup");
  uint32_t voff[N];  // byte offset of this lane's source chunk within the tile

  __device__ __forceinline__ void init() {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      int c;
      const int row = unswz_row_chunk<D>((i * (NT / 64) + wave) * 64 + lane, c);
      voff[i] = opaque((uint32_t)((row * D + c * 8) * sizeof(T)));
    }
  }
  // piece i of copy(): `src` and `dst` are wave-uniform
  __device__ __forceinline__ void piece(int i, T* dst, const T* src) const {
    const uint32_t base =
        __builtin_amdgcn_readfirstlane(lds_addr(dst) + (uint32_t)(threadIdx.x >> 6) * 1024u);
    dma16_s(voff[i], src, base + (uint32_t)i * (NT / 64) * 1024u);
  }
  // `src` and `dst` are wave-uniform
  __device__ __forceinline__ void copy(T* dst, const T* src) const {
    const uint32_t base =
        __builtin_amdgcn_readfirstlane(lds_addr(dst) + (uint32_t)(threadIdx.x >> 6) * 1024u);
#pragma unroll
    for (int i = 0; i < N; ++i) dma16_s(voff[i], src, base + (uint32_t)i * (NT / 64) * 1024u);
  }
  // copy() with the caller's wave index held in a scalar register (no vector
  // temporary of the thread index stays live across the caller's loop)
  __device__ __forceinline__ void copy(T* dst, const T* src, int wave) const {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(dst)) + (uint32_t)wave * 1024u;
#pragma unroll
    for (int i = 0; i < N; ++i) dma16_s(voff[i], src, base + (uint32_t)i * (NT / 64) * 1024u);
  }
  // copy() to the tile at LDS byte address `dst` (wave-uniform), for callers
  // that convert their LDS base once outside the loop
  __device__ __forceinline__ void copy_lds(uint32_t dst, const T* src, int wave) const {
    const uint32_t base = dst + (uint32_t)wave * 1024u;
#pragma unroll
    for (int i = 0; i < N; ++i) dma16_s(voff[i], src, base + (uint32_t)i * (NT / 64) * 1024u);
  }
};

// Wait until at most N of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait for this wave's outstanding vector-memory loads (vmcnt = 0).
__device__ __forceinline__ void dma_wait() { wait_vmcnt<0>(); }

// Issue priority of this wave over the other wave of its SIMD (s_setprio), for
// the ping-pong kernels: raised for an MFMA phase, so that its MFMAs and LDS
// operand reads win issue arbitration over the other wave's VALU phase, and
// lowered after it.  The scheduler keeps the phase's work between the two.
__device__ __forceinline__ void mfma_priority_up() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void mfma_priority_down() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_sched_barrier(0);
}

// exp2 on the transcendental unit without the libm range fix-ups
// (results below 2^-126 flush to zero, which softmax weights tolerate).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum of two floats for the softmax row max: IEEE 754-2019 maximum (a NaN
// operand gives NaN, -0 < +0), which gfx950 runs as v_maximum3_f32, three
// operands per instruction.  fmaxf must quiet a signalling NaN, so the compiler
// puts a v_max_f32 x, x in front of each operand it cannot prove canonical
// (every MFMA result): 15 instructions for a 16-value max against 9 here.  On
// non-NaN values both return the larger operand, so the softmax is unchanged.
__device__ __forceinline__ float vmax(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// Max / sum of the lane pair (i, i ^ 32), in both lanes, with v_permlane32_swap
// (no LDS round trip, unlike a generic shuffle).  Both are symmetric, so the
// two swapped halves combine without a select.
__device__ __forceinline__ float pair_max32(float x) {
  const auto r =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One 32x32 MFMA accumulator tile whose rows are 32 dims of the rows (query or
// key) r = lane & 31: lane (r, h = lane >> 5) holds element 4g + e = dim
// 8g + 4h + e, g < 4, e < 4.  Regrouped for 16-byte accesses: one
// v_permlane32_swap per value of the pairs g = (2p, 2p + 1) leaves lane h with
// the eight consecutive dims 8(2p + h) + i in w[p][i] (each value times mul).
// Both lanes of a pair must be active.
__device__ __forceinline__ void swap_rows16(const f32x16& acc, float mul, float (&w)[2][8]) {
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[8 * p + e] * mul),
                                                       __float_as_uint(acc[8 * p + 4 + e] * mul),
                                                       false, false);
      w[p][e] = __uint_as_float(sw[0]);
      w[p][4 + e] = __uint_as_float(sw[1]);
    }
}

// ---------------------------------------------------------------------------
// Wave / block reductions (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide reduction through LDS; `red` must hold blockDim.x/64 floats.
template <bool kMax>
__device__ __forceinline__ float block_reduce(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  v = kMax ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < nw; ++w) r = kMax ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__device__ __forceinline__ int clamp_valid(int32_t vbs, int be) {
  return vbs < 0 ? 0 : (vbs > be ? be : (int)vbs);
}

// The route of one query block (its selected key blocks), held in VGPRs 64
// slots at a time: lane j keeps the key block of slot base + j and its valid
// token count (0 for an id outside [0, kb)).  Stepping to the next chunk is then
// a v_readlane with a scalar index instead of two dependent scalar loads from
// global memory (selected id, then its block size) in front of every copy.
// load() uses vector loads, so it is only called where no direct-to-LDS copy
// is in flight (the compiler's vmcnt wait would include them).
template <int BE, int KC>
struct RouteRegs {
  const int32_t* sel;
  const int32_t* vbs;
  int topk, kb;
  int base;  // first slot held (wave-uniform)
  int rkv, rnv;

  __device__ __forceinline__ void load(int b0) {
    base = b0;
    const int j = b0 + (int)(threadIdx.x & 63);
    const int kv = j < topk ? sel[j] : -1;
    rkv = kv;
    rnv = (kv >= 0 && kv < kb) ? clamp_valid(vbs[kv], BE) : 0;
  }
  // Advance (s, c) to the next chunk of KC keys that holds a valid key.
  __device__ __forceinline__ bool next(int& s, int& c, int& kv, int& nvb) {
    while (s < topk) {
      if (s - base >= 64) load(s);
      const int nv = __builtin_amdgcn_readlane(rnv, s - base);
      if (c * KC < nv) {
        kv = __builtin_amdgcn_readlane(rkv, s - base);
        nvb = nv;
        return true;
      }
      ++s;
      c = 0;
    }
    return false;
  }
};

// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs
// of an MI355X, so linear id i runs on XCD i % 8.  Give XCD x the contiguous
// tile range [x*per, (x+1)*per) so the tiles of one head stay on one XCD's L2.
__device__ __forceinline__ int xcd_tile(int linear_id, int num_tiles) {
  const int per = (num_tiles + 7) >> 3;
  return (linear_id & 7) * per + (linear_id >> 3);
}

// Scheduling counters of a persistent kernel's workgroups: ctr[x] hands out
// the entries 0 .. per-1 of XCD x's range, ctr[8] counts the workgroups that
// have finished.  Thread 0 of a workgroup on XCD `xcd` takes the next entry of
// its own range and, once that is drained, of ranges xcd+1 .. xcd+last-1
// (mod 8): the XCDs do not run equally fast, so the ones that finish first
// take over the others' remaining tiles.  `from` (kept by the caller from one
// call to the next, starting at 0) skips the ranges known to be drained.
// Returns 8 * entry + range, or -1 once every range it may take from is drained.
__device__ __forceinline__ int take_entry(int32_t* ctr, int xcd, int per, int& from, int last) {
  while (from < last) {
    const int x = (xcd + from) & 7;
    // another range's counter is read before it is advanced: at the end every
    // workgroup passes over every drained range, and read-modify-writes of one
    // address from all of them would queue up behind each other
    if (from == 0 ||
        __hip_atomic_load(ctr + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < per) {
      const int e = atomicAdd(ctr + x, 1);
      if (e < per) return 8 * e + x;
    }
    ++from;
  }
  return -1;
}

// Thread 0 of a workgroup that has taken its last entry: the last workgroup to
// finish zeroes the counters for the next launch.
__device__ __forceinline__ void finish_entries(int32_t* ctr) {
  __threadfence();
  if (atomicAdd(ctr + 8, 1) == (int)gridDim.x - 1) {
#pragma unroll
    for (int x = 0; x < 9; ++x) ctr[x] = 0;
  }
}

}  // namespace vsa
