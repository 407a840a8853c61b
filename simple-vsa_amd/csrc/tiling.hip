// 3-D tile layout of video tokens on gfx950: metadata and row movement.
//
// Reference contract: vsa/fastvideo_tiling.py of simple-vsa.  The reference
// builds the index tensors with a Python loop over tiles plus torch.cat /
// argsort (fastvideo_tiling.py:22-88) and moves tokens with advanced indexing
// (tile 130-140, untile 143-145).  Here the metadata comes from the closed
// form of the raster <-> tile mapping in one pass, and tile / untile (and their
// gradients) are index-driven row moves that are pure HBM streams.
//
// Closed form: raster token r = (t*H + h)*W + w lies in tile (nt, nh, nw) =
// (t/ts, h/hs, w/ws), tile id n = (nt*NH + nh)*NW + nw.  The tile's extents are
// (et, eh, ew) = (min(ts, T - nt*ts), ...), its members are ordered row-major
// over (t, h, w) inside the box, so the token's slot is
//   p = ((t - nt*ts)*eh + (h - nh*hs))*ew + (w - nw*ws),
// and the tiles before it hold
//   start(n) = nt*ts*H*W + et*(nh*hs)*W + et*eh*(nw*ws)
// tokens (whole t-slabs, then whole h-rows of this slab, then this row).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vsa_capi.h"
#include "vsa_device.h"
#include "vsa_launch.h"

namespace vsa {

__global__ void tile_metadata_kernel(int T, int H, int W, int ts, int hs, int ws, int NH, int NW,
                                     int be, int64_t S, int64_t nb, int64_t* __restrict__ tpi,
                                     int64_t* __restrict__ rev, int64_t* __restrict__ npi,
                                     int64_t* __restrict__ vbs) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g < S) {
    const int w = (int)(g % W);
    const int64_t th = g / W;
    const int h = (int)(th % H);
    const int t = (int)(th / H);
    const int nt = t / ts, nh = h / hs, nw = w / ws;
    const int et = min(ts, T - nt * ts), eh = min(hs, H - nh * hs), ew = min(ws, W - nw * ws);
    const int64_t n = ((int64_t)nt * NH + nh) * NW + nw;
    const int64_t p = ((int64_t)(t - nt * ts) * eh + (h - nh * hs)) * ew + (w - nw * ws);
    const int64_t start = (int64_t)nt * ts * H * W + (int64_t)et * nh * hs * W +
                          (int64_t)et * eh * nw * ws;
    const int64_t pos = start + p;
    tpi[pos] = g;
    rev[g] = pos;
    npi[pos] = n * be + p;
  }
  if (g < nb) {
    const int nw = (int)(g % NW);
    const int64_t r = g / NW;
    const int nh = (int)(r % NH);
    const int nt = (int)(r / NH);
    const int64_t et = min(ts, T - nt * ts), eh = min(hs, H - nh * hs), ew = min(ws, W - nw * ws);
    vbs[g] = et * eh * ew;
  }
}

// Inverse map for the fused tiled op: slot p of tile n (padded layout, tile
// volume be) holds raster token
//   r = ((nt*ts + dt)*H + nh*hs + dh)*W + nw*ws + dw,
// (dt, dh, dw) = (p / (eh*ew), (p / ew) % eh, p % ew), for p < et*eh*ew, and
// nothing (-1) after that.
__global__ void tile_slot_rows_kernel(int T, int H, int W, int ts, int hs, int ws, int NH, int NW,
                                      int be, int64_t slots, int32_t* __restrict__ rows) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= slots) return;
  const int64_t n = g / be;
  const int p = (int)(g - n * be);
  const int nw = (int)(n % NW);
  const int64_t rest = n / NW;
  const int nh = (int)(rest % NH);
  const int nt = (int)(rest / NH);
  const int et = min(ts, T - nt * ts), eh = min(hs, H - nh * hs), ew = min(ws, W - nw * ws);
  const int hw = eh * ew;
  if (p >= et * hw) {
    rows[g] = -1;
    return;
  }
  const int dt = p / hw, dh = (p - dt * hw) / ew, dw = p - dt * hw - dh * ew;
  rows[g] = (int32_t)(((int64_t)(nt * ts + dt) * H + nh * hs + dh) * W + nw * ws + dw);
}

// index of item i through an optional second level: outer ? a[outer[i]] : (a ? a[i] : i);
// -1 when a lookup would leave its table
__device__ __forceinline__ int64_t lookup(const int64_t* __restrict__ a, int64_t a_len,
                                          const int64_t* __restrict__ outer, int64_t i) {
  if (!a) return i;
  int64_t j = i;
  if (outer) {
    j = outer[i];
    if (j < 0 || j >= a_len) return -1;
  }
  return a[j];
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int VB> struct Vec;
template <> struct Vec<16> { typedef u32x4_t t; };
template <> struct Vec<8> { typedef u32x2_t t; };
template <> struct Vec<4> { typedef uint32_t t; };
template <> struct Vec<2> { typedef uint16_t t; };
template <> struct Vec<1> { typedef uint8_t t; };

// Row moves, TPR threads per row (power of two), 256 threads per workgroup;
// blockIdx.y walks the batch.  Rows are counted in VB-byte chunks: x rows are
// xc chunks long, out rows oc, the first cc chunks are copied and chunks
// [cc, oc) of the destination row are zeroed.
template <int VB>
__global__ __launch_bounds__(256) void rows_move_kernel(
    const char* __restrict__ x, int64_t x_rows, int64_t xc, char* __restrict__ out,
    int64_t out_rows, int64_t oc, int64_t cc, int64_t batch, int tpr_log2,
    const int64_t* __restrict__ src, int64_t src_len, const int64_t* __restrict__ src_outer,
    const int64_t* __restrict__ dst, int64_t dst_len, const int64_t* __restrict__ dst_outer,
    int64_t n) {
  typedef typename Vec<VB>::t V;
  const int tpr = 1 << tpr_log2;
  const int64_t i = (int64_t)blockIdx.x * (256 >> tpr_log2) + (threadIdx.x >> tpr_log2);
  if (i >= n) return;
  const int lane = threadIdx.x & (tpr - 1);
  const int64_t s = lookup(src, src_len, src_outer, i);
  const int64_t d = lookup(dst, dst_len, dst_outer, i);
  if (s < 0 || s >= x_rows || d < 0 || d >= out_rows) return;
  for (int64_t b = blockIdx.y; b < batch; b += gridDim.y) {
    const V* sp = reinterpret_cast<const V*>(x + (b * x_rows + s) * xc * VB);
    V* dp = reinterpret_cast<V*>(out + (b * out_rows + d) * oc * VB);
    for (int64_t c = lane; c < oc; c += tpr) st_stream(dp + c, c < cc ? ld_stream(sp + c) : V{});
  }
}

__global__ void mark_clear_kernel(uint8_t* __restrict__ mark, int64_t rows) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g < rows) mark[g] = 0;
}

__global__ void mark_set_kernel(uint8_t* __restrict__ mark, int64_t rows,
                                const int64_t* __restrict__ idx, int64_t n) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g < n) {
    const int64_t j = idx[g];
    if (j >= 0 && j < rows) mark[j] = 1;
  }
}

template <int VB>
__global__ __launch_bounds__(256) void rows_zero_kernel(char* __restrict__ out, int64_t out_rows,
                                                        int64_t batch, int64_t cpr, int tpr_log2,
                                                        const uint8_t* __restrict__ mark) {
  typedef typename Vec<VB>::t V;
  const int tpr = 1 << tpr_log2;
  const int64_t j = (int64_t)blockIdx.x * (256 >> tpr_log2) + (threadIdx.x >> tpr_log2);
  if (j >= out_rows || mark[j]) return;
  const int lane = threadIdx.x & (tpr - 1);
  for (int64_t b = blockIdx.y; b < batch; b += gridDim.y) {
    V* dp = reinterpret_cast<V*>(out + (b * out_rows + j) * cpr * VB);
    for (int64_t c = lane; c < cpr; c += tpr) st_stream(dp + c, V{});
  }
}

// Widest vector that divides every row length and keeps every row start aligned.
static int vec_bytes(int64_t a_bytes, int64_t b_bytes, int64_t c_bytes, const void* a,
                     const void* b) {
  const uintptr_t al = (uintptr_t)a | (uintptr_t)b;
  for (int vb = 16; vb > 1; vb >>= 1)
    if (a_bytes % vb == 0 && b_bytes % vb == 0 && c_bytes % vb == 0 && al % vb == 0) return vb;
  return 1;
}

// threads per row: the power of two >= chunks per row, capped at 256
static int tpr_log2_for(int64_t cpr) {
  int l = 0;
  while (l < 8 && ((int64_t)1 << l) < cpr) ++l;
  return l;
}

// grid.x covers the rows (256 / TPR rows per workgroup), grid.y the batch;
// false when the rows need more workgroups than one launch allows
static bool row_grid(int64_t rows, int tpr_log2, int64_t batch, dim3& grid) {
  const int64_t rpw = 256 >> tpr_log2;
  const int64_t gx = (rows + rpw - 1) / rpw;
  if (gx <= 0 || gx > 0x7fffffffLL) return false;
  grid = dim3((unsigned)gx, (unsigned)(batch < 65535 ? batch : 65535), 1);
  return true;
}

}  // namespace vsa

using namespace vsa;

extern "C" int vsa_tile_metadata(int32_t T, int32_t H, int32_t W, int32_t ts, int32_t hs,
                                 int32_t ws, int64_t* tile_partition_indices,
                                 int64_t* reverse_indices, int64_t* non_pad_index,
                                 int64_t* variable_block_sizes, void* stream) {
  if (!tile_partition_indices || !reverse_indices || !non_pad_index || !variable_block_sizes)
    return VSA_ERR_NULL;
  if (!vsa_aligned<8>(tile_partition_indices, reverse_indices, non_pad_index,
                      variable_block_sizes))
    return VSA_ERR_ALIGN;
  if (T <= 0 || H <= 0 || W <= 0 || ts <= 0 || hs <= 0 || ws <= 0) return VSA_ERR_SHAPE;
  const int64_t S = (int64_t)T * H * W;
  const int NT = (T + ts - 1) / ts, NH = (H + hs - 1) / hs, NW = (W + ws - 1) / ws;
  const int64_t nb = (int64_t)NT * NH * NW;
  const int64_t be = (int64_t)ts * hs * ws;
  if (S > (1LL << 40) || be > (1LL << 30) || nb * be > (1LL << 40)) return VSA_ERR_SHAPE;
  const int64_t work = S > nb ? S : nb;
  if ((work + 255) / 256 > 0x7fffffffLL) return VSA_ERR_SHAPE;
  hipLaunchKernelGGL(tile_metadata_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, T, H, W, ts, hs, ws, NH, NW, (int)be, S, nb,
                     tile_partition_indices, reverse_indices, non_pad_index,
                     variable_block_sizes);
  return vsa_check_launch();
}

extern "C" int vsa_tile_slot_rows(int32_t T, int32_t H, int32_t W, int32_t ts, int32_t hs,
                                  int32_t ws, int32_t* slot_rows, void* stream) {
  if (!slot_rows) return VSA_ERR_NULL;
  if (!vsa_aligned<4>(slot_rows)) return VSA_ERR_ALIGN;
  if (T <= 0 || H <= 0 || W <= 0 || ts <= 0 || hs <= 0 || ws <= 0) return VSA_ERR_SHAPE;
  const int64_t S = (int64_t)T * H * W;
  const int NT = (T + ts - 1) / ts, NH = (H + hs - 1) / hs, NW = (W + ws - 1) / ws;
  const int64_t be = (int64_t)ts * hs * ws;
  const int64_t slots = (int64_t)NT * NH * NW * be;
  if (S >= (1LL << 31) || be > (1LL << 20) || slots > (1LL << 40) ||
      (slots + 255) / 256 > 0x7fffffffLL)
    return VSA_ERR_SHAPE;
  hipLaunchKernelGGL(tile_slot_rows_kernel, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, T, H, W, ts, hs, ws, NH, NW, (int)be, slots, slot_rows);
  return vsa_check_launch();
}

extern "C" int vsa_rows_move(const void* x, int64_t x_rows, int64_t x_row_bytes, void* out,
                             int64_t out_rows, int64_t out_row_bytes, int64_t copy_bytes,
                             int64_t batch, const int64_t* src, int64_t src_len,
                             const int64_t* src_outer, const int64_t* dst, int64_t dst_len,
                             const int64_t* dst_outer, int64_t n, void* stream) {
  if (!x || !out) return VSA_ERR_NULL;
  if ((src_outer && !src) || (dst_outer && !dst)) return VSA_ERR_NULL;
  if (!vsa_aligned<8>(src, src_outer, dst, dst_outer)) return VSA_ERR_ALIGN;
  if (x_rows < 0 || out_rows < 0 || batch < 0 || n < 0 || copy_bytes <= 0 ||
      copy_bytes > x_row_bytes || copy_bytes > out_row_bytes)
    return VSA_ERR_SHAPE;
  if (n == 0 || batch == 0) return VSA_OK;
  const int vb = vec_bytes(x_row_bytes, out_row_bytes, copy_bytes, x, out);
  const int64_t xc = x_row_bytes / vb, oc = out_row_bytes / vb, cc = copy_bytes / vb;
  const int tl = tpr_log2_for(oc);
  dim3 grid;
  if (!row_grid(n, tl, batch, grid)) return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
#define VSA_MOVE(VB)                                                                          \
  hipLaunchKernelGGL(rows_move_kernel<VB>, grid, dim3(256), 0, s, (const char*)x, x_rows, xc, \
                     (char*)out, out_rows, oc, cc, batch, tl, src, src_len, src_outer, dst,   \
                     dst_len, dst_outer, n)
  switch (vb) {
    case 16: VSA_MOVE(16); break;
    case 8: VSA_MOVE(8); break;
    case 4: VSA_MOVE(4); break;
    case 2: VSA_MOVE(2); break;
    default: VSA_MOVE(1);
  }
#undef VSA_MOVE
  return vsa_check_launch();
}

extern "C" int vsa_rows_zero_unmarked(void* out, int64_t out_rows, int64_t batch,
                                      int64_t row_bytes, const int64_t* marked, int64_t n_marked,
                                      uint8_t* mark_workspace, void* stream) {
  if (!out || !mark_workspace || (n_marked > 0 && !marked)) return VSA_ERR_NULL;
  if (!vsa_aligned<8>(marked)) return VSA_ERR_ALIGN;
  if (out_rows < 0 || batch < 0 || row_bytes <= 0 || n_marked < 0) return VSA_ERR_SHAPE;
  if (out_rows == 0 || batch == 0) return VSA_OK;
  if (out_rows > (1LL << 38) || n_marked > (1LL << 38)) return VSA_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(mark_clear_kernel, dim3((unsigned)((out_rows + 255) / 256)), dim3(256), 0, s,
                     mark_workspace, out_rows);
  if (n_marked > 0)
    hipLaunchKernelGGL(mark_set_kernel, dim3((unsigned)((n_marked + 255) / 256)), dim3(256), 0,
                       s, mark_workspace, out_rows, marked, n_marked);
  const int vb = vec_bytes(row_bytes, row_bytes, row_bytes, out, out);
  const int64_t cpr = row_bytes / vb;
  const int tl = tpr_log2_for(cpr);
  dim3 grid;
  if (!row_grid(out_rows, tl, batch, grid)) return VSA_ERR_SHAPE;
#define VSA_ZERO(VB)                                                                           \
  hipLaunchKernelGGL(rows_zero_kernel<VB>, grid, dim3(256), 0, s, (char*)out, out_rows, batch, \
                     cpr, tl, mark_workspace)
  switch (vb) {
    case 16: VSA_ZERO(16); break;
    case 8: VSA_ZERO(8); break;
    case 4: VSA_ZERO(4); break;
    case 2: VSA_ZERO(2); break;
    default: VSA_ZERO(1);
  }
#undef VSA_ZERO
  return vsa_check_launch();
}
