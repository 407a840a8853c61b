/*
 * vsa_capi.h -- C ABI of the MI355X (gfx950) Video Sparse Attention kernels.
 *
 * This is the drop-in boundary under the reference's Python operator API
 * (ita9naiwa/simple-vsa): the host layer binds these symbols with ctypes and
 * keeps the reference's `*_vsa(q, k, v, variable_block_sizes,
 * q_variable_block_sizes, topk, block_size, compress_attn_weight)` and
 * `*_sparse_attention(q, k, v, selected, variable_block_sizes, *, block_size,
 * sm_scale)` signatures above them.
 *
 * Rules shared by every entry point:
 *  - plain device pointers, element counts and a hipStream_t passed as void*;
 *    no framework types cross this boundary;
 *  - tensors are contiguous row-major; q-like tensors are [BH, Sq, D], k/v-like
 *    [BH, Skv, D], block vectors [BH, nblocks, D], where BH = batch * heads;
 *    tensors of the element type (rows are read and written with 16-byte
 *    accesses) and the fp32 coarse score / probability buffers start 16-byte
 *    aligned, int64 index arrays 8-byte, int32 arrays and the per-row fp32
 *    vectors (lse, delta) 4-byte aligned (the row-move entry points take
 *    their rows at any alignment); an entry point returns VSA_ERR_ALIGN
 *    before any launch otherwise;
 *  - dtype: VSA_BF16, VSA_F16 or VSA_F32 for every kernel (the fine kernels
 *    run bf16 / fp16 on MFMA and fp32 on fp32 kernels, same results contract);
 *  - nothing here allocates or frees device memory: every output and every
 *    workspace buffer is owned by the caller (the library's own device memory
 *    is two file-scope arrays per GPU, held until the process ends: the
 *    scheduling counters below and vsa_sparse_bwd_dkdv_noalloc's workspace);
 *  - launches are asynchronous on `stream`; no host synchronisation;
 *  - the persistent forward and dQ kernels (bf16 / fp16, head dim 128, block
 *    256, at least 256 query blocks) take their query blocks from scheduling
 *    counters in a slot of a file-scope device array (256 slots of 128 bytes
 *    per GPU, one per stream that launches them; each launch leaves its slot
 *    zeroed for the next; a stream that finds every slot taken, or that is
 *    not on the current device, runs them with a fixed schedule instead, with
 *    the same results).  Launches on one stream share its slot, which stream
 *    order keeps apart; a HIP graph captured on stream S holds S's slot, so
 *    it must not be replayed while launches issued on S itself still run;
 *  - return 0 on success, a negative VSA_ERR_* code otherwise (no exceptions
 *    cross the ABI); vsa_status_string() turns a code into text;
 *  - BH <= 65535 (the per-(batch, head) passes put it in the grid's y
 *    dimension);
 *  - route ids outside [0, Kb) contribute nothing; block sizes are clamped to
 *    [0, block_elements] for token masking.
 */
#ifndef VSA_CAPI_H
#define VSA_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vsa_dtype { VSA_BF16 = 0, VSA_F16 = 1, VSA_F32 = 2 };

/*
 * How compress_attn_weight is laid out: absent, [BH, Sq, D], [BH, Sq, 1], or
 * token-major [B, Sq, H, D] -- the gate producer's Linear output before its
 * per-head transpose (common.py:326-328), read and written in place; H is the
 * `gate_heads` argument and bh = b*H + h.  The gate has the inputs' dtype,
 * unless VSA_GATE_F32 is OR-ed into the mode: then it is fp32 beside bf16 /
 * fp16 inputs (the reference promotes the gate with .float(), torch_impl.py:110,
 * and keeps its gradient in the gate's dtype, fused_common.py:202-221).
 */
enum vsa_gate_mode {
  VSA_GATE_NONE = 0,
  VSA_GATE_FULL = 1,
  VSA_GATE_PER_TOKEN = 2,
  VSA_GATE_TOKEN_MAJOR = 3,
  VSA_GATE_F32 = 4          /* flag: the gate (and d_gate) are fp32 */
};

enum vsa_status {
  VSA_OK = 0,
  VSA_ERR_NULL = -1,        /* a required pointer is NULL */
  VSA_ERR_SHAPE = -2,       /* sizes inconsistent or out of range */
  VSA_ERR_DTYPE = -3,       /* dtype not supported by this entry point */
  VSA_ERR_UNSUPPORTED = -4, /* (block_elements, head_dim) pair has no kernel */
  VSA_ERR_LAUNCH = -5,      /* the HIP launch itself failed */
  VSA_ERR_TOO_LARGE = -6,   /* beyond the static scratch of a no-allocation entry point */
  VSA_ERR_ALIGN = -7,       /* a pointer is not aligned as the shared rules require */
  VSA_ERR_DEVICE = -8       /* the stream belongs to another GPU than the current one */
};

/* Text for a status code (static storage). */
const char* vsa_status_string(int status);

/* Library version string (static storage). */
const char* vsa_version(void);

/*
 * Padded block mean of q, k and v in one launch.
 * Replaces fused_block_mean x3 (fused_common.py:20-59, 106-144, 340-347;
 * called from common.py:155-157).  out[bh, n, :] = T(sum_{t < vbs[n]}
 * x[bh, n*be + t, :] / max(vbs[n], 1)), fp32 sum.
 */
int vsa_pool_qkv(const void* q, const void* k, const void* v,
                 const int32_t* q_vbs, const int32_t* kv_vbs,
                 void* q_c, void* k_c, void* v_c,
                 int64_t bh, int64_t sq, int64_t skv, int32_t head_dim,
                 int32_t block_elements, int32_t dtype, void* stream);

/*
 * Coarse block attention on the pooled tokens plus Top-K routing.
 * Replaces coarse_branch_compact's matmul/softmax/matmul (common.py:159-166)
 * and scores.topk (triton_impl.py:1710; torch_impl.py:85).
 *   scores[bh, i, j] = T(T(q_c[i] . k_c[j]) * scale)      (stored as fp32)
 *   probs[bh, i, j]  = T(softmax_j(scores[bh, i, :]))      (stored as fp32)
 *   out_c[bh, i, :]  = T(sum_j probs[i, j] * v_c[j, :])
 *   selected[bh, i, :] = the `topk` key blocks with the largest scores; ties go
 *   to the smaller block id; written in ascending block-id order (int32).
 * `selected` may be NULL (no routing).  Kb <= 16000 for bf16 / fp16 at head
 * dims 64 and 128 (MFMA kernels streaming key tiles; the Top-K keeps one row
 * of Kb keys in LDS), Kb <= 4096 otherwise (generic kernels, two rows in LDS).
 */
int vsa_coarse_fwd(const void* q_c, const void* k_c, const void* v_c,
                   float* scores, float* probs, void* out_c, int32_t* selected,
                   int64_t bh, int32_t q_blocks, int32_t kv_blocks, int32_t head_dim,
                   int32_t topk, float scale, int32_t dtype, void* stream);

/*
 * Stand-alone Top-K over fp32 scores [rows, kv_blocks] -> int32 [rows, topk]
 * with the same tie rule and output order as vsa_coarse_fwd.
 * Replaces scores.topk(topk, dim=-1) (triton_impl.py:1710).  kv_blocks <= 16000.
 */
int vsa_topk(const float* scores, int32_t* selected, int64_t rows,
             int32_t kv_blocks, int32_t topk, void* stream);

/*
 * Compact KV-block -> query-block CSR per (batch, head).
 * Replaces _invert_indices (triton_impl.py:544-595): counts [BH, Kb],
 * offsets [BH, Kb] (exclusive prefix of counts), inverse [BH, Qb*topk].
 * Unlike the reference's atomic cursor, every segment is written in ascending
 * query-block order, so the result is deterministic (a query block that
 * chose one key block several times is listed that many times).  q_blocks,
 * kv_blocks <= 16000 (a bit per query block for each of a workgroup's key
 * blocks, in LDS).
 */
int vsa_csr_build(const int32_t* selected, int32_t* counts, int32_t* offsets,
                  int32_t* inverse, int64_t bh, int32_t q_blocks, int32_t kv_blocks,
                  int32_t topk, void* stream);

/*
 * Sparse fine forward over the selected KV blocks (bf16/fp16 MFMA, online
 * softmax in base 2), optionally fused with the combine.
 * Replaces _triton_sparse_attention_forward (triton_impl.py:358-473: T6/T7
 * kernels 39-355) and, when out_c != NULL, _FusedCombine.forward
 * (fused_common.py:175-199, 261-295):
 *   out = T(out_c[block] * gate + attn)   (gate = 1 when gate_mode == NONE)
 *   out = T(attn)                          when out_c == NULL
 *   fine_out = T(attn)   when out_c != NULL and fine_out != NULL: the fine
 *                        output the reference's fused path keeps as its own
 *                        tensor (triton_impl.py:408); vsa_bwd_prep takes it
 * With VSA_GATE_F32 the combine runs as a second pass over the T-rounded fine
 * output, out = T(out_c[block] * gate + T(attn)), as the reference's fused
 * combine does (fused_common.py:175-199).
 *   lse[bh, q] = log2(sum_j exp2(scale*log2(e) * q.k_j))   (may be NULL)
 * block_elements in {64, 128, 256}; head_dim in {64, 128, 256}.
 */
int vsa_sparse_fwd(const void* q, const void* k, const void* v,
                   const int32_t* selected, const int32_t* kv_vbs,
                   void* out, void* fine_out, float* lse, const void* out_c, const void* gate,
                   int32_t gate_mode, int32_t gate_heads, int64_t bh, int64_t sq, int64_t skv,
                   int32_t head_dim, int32_t block_elements, int32_t topk,
                   float scale, int32_t dtype, void* stream);

/*
 * Backward preprocessing over dout: the softmax delta plus the combine
 * gradients.  Replaces _delta_kernel/_delta_256_kernel (triton_impl.py:598-700)
 * and _FusedCombine.backward (fused_common.py:202-256, 298-337).
 * fine_out is the fine output as stored in T: vsa_sparse_fwd's fine_out when
 * the combine was fused (out_c != NULL), its out otherwise.
 *   delta[bh, q]   = sum_d fine_out * dout                           (fp32)
 *   d_out_c[bh, n] = T(sum_{t < be} T(dout * gate))     (if out_c != NULL)
 *   d_gate         = T(dout * out_c[block])  (per token: summed over d),
 * d_gate in the gate's own layout (token-major included) and dtype (fp32 with
 * VSA_GATE_F32).
 */
int vsa_bwd_prep(const void* fine_out, const void* dout, const void* out_c, const void* gate,
                 int32_t gate_mode, int32_t gate_heads, float* delta, void* d_out_c, void* d_gate,
                 int64_t bh, int64_t sq, int32_t head_dim, int32_t block_elements,
                 int32_t dtype, void* stream);

/*
 * Backward of the coarse branch (autograd of common.py:164-166 in T):
 *   dP = T(d_out_c v_c^T); d_v_c = T(P^T d_out_c);
 *   dS = T(scale * T(P * (dP - rowsum(P * dP))));
 *   d_q_c = T(dS k_c); d_k_c = T(dS^T q_c).
 * `ds` is fp32 workspace [BH, Qb, Kb].  Kb limits as for vsa_coarse_fwd.
 */
int vsa_coarse_bwd(const void* q_c, const void* k_c, const void* v_c, const float* probs,
                   const void* d_out_c, float* ds, void* d_q_c, void* d_k_c, void* d_v_c,
                   int64_t bh, int32_t q_blocks, int32_t kv_blocks, int32_t head_dim,
                   float scale, int32_t dtype, void* stream);

/*
 * Query-owned dQ over the selected KV blocks.  Replaces _vsa_dq_256_kernel /
 * _vsa_dq_kernel (triton_impl.py:703-969).  When d_q_c != NULL the pooled
 * gradient is folded in: dq[t] += T(d_q_c[block] / max(q_vbs[block], 1)) for
 * t < q_vbs[block] (block_mean backward, fused_common.py:62-103).
 */
int vsa_sparse_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                      const float* lse, const float* delta, const int32_t* selected,
                      const int32_t* kv_vbs, void* dq, const void* d_q_c,
                      const int32_t* q_vbs, int64_t bh, int64_t sq, int64_t skv,
                      int32_t head_dim, int32_t block_elements, int32_t topk,
                      float scale, int32_t dtype, void* stream);

/*
 * Scheduling workspace for vsa_sparse_bwd_dkdv's bf16 / fp16 kernel, from the
 * CSR counts of vsa_csr_build.  No reference counterpart: the reference's
 * dK/dV launch walks key blocks in index order (triton_impl.py:1394-1440), and
 * a hot key block (in-edges from most query blocks, as with skewed routes)
 * then serialises the end of the kernel.  The kernel's persistent workgroups
 * take the tiles of their XCD's range in the order written here, and then
 * the tiles left in the other XCDs' ranges: longest-first when the range's
 * largest tile exceeds a quarter of an average workgroup slot's share, else
 * index order with the range's smallest tiles (at most 4 per workgroup slot)
 * moved to the end.  tile_order holds order_len >= 8 * per + 16 int32 entries,
 * per = ceil(tiles / 8), tiles = bh * skv / min(block_elements, head_dim == 64
 * ? 256 : 128) * (head_dim > 128 ? 2 : 1), below 2^30: the order (entries of
 * a longest-first range carry bit 30 on top of the tile index; its workgroups
 * do not take other ranges' tiles), then 9 counters this call zeroes
 * and the dK/dV kernel advances (and leaves zeroed when it ends), so one
 * workspace serves one dK/dV launch at a time.  Results do not depend on the
 * order.
 */
int vsa_dkdv_tile_order(const int32_t* counts, int32_t* tile_order, int64_t order_len,
                        int64_t bh, int64_t skv, int32_t head_dim, int32_t block_elements,
                        void* stream);

/*
 * KV-owned dK/dV driven by the CSR from vsa_csr_build.  Replaces
 * _vsa_dkdv_256_kernel / _vsa_dkdv_kernel (triton_impl.py:972-1318).  When
 * d_k_c / d_v_c != NULL the pooled gradients are folded in as in
 * vsa_sparse_bwd_dq (using kv_vbs).  tile_order (nullable) is the workspace
 * from vsa_dkdv_tile_order for the same sizes (bf16 / fp16; ignored for
 * fp32); without it the persistent workgroups stride over the tiles in index
 * order.
 */
int vsa_sparse_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout,
                        const float* lse, const float* delta, const int32_t* counts,
                        const int32_t* offsets, const int32_t* inverse,
                        const int32_t* kv_vbs, void* dk, void* dv,
                        const void* d_k_c, const void* d_v_c,
                        int64_t bh, int64_t sq, int64_t skv, int32_t head_dim,
                        int32_t block_elements, int32_t topk, float scale,
                        int32_t* tile_order, int32_t dtype, void* stream);

/*
 * vsa_sparse_bwd_dkdv without a caller workspace: same arguments and results,
 * minus tile_order.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The tile order and scheduling
 * counters that vsa_dkdv_tile_order would write into a caller buffer live in
 * a file-scope device array of 1 MiB (262,144 int32) per GPU, held until the
 * process ends; the call writes the order there and then runs the dK/dV
 * kernel, allocating nothing.  Sizes whose order needs more than the array
 * (8 * ceil(tiles / 8) + 16 > 262,144 entries, tiles as in
 * vsa_dkdv_tile_order) return VSA_ERR_TOO_LARGE.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, or two host
 * threads) race and must be serialised by the caller.  The array used is the
 * current device's, so a non-NULL stream must belong to the current device
 * (else VSA_ERR_DEVICE, before any launch).  fp32 inputs need no workspace and
 * run as vsa_sparse_bwd_dkdv with tile_order = NULL.
 */
int vsa_sparse_bwd_dkdv_noalloc(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, const int32_t* counts,
                                const int32_t* offsets, const int32_t* inverse,
                                const int32_t* kv_vbs, void* dk, void* dv,
                                const void* d_k_c, const void* d_v_c,
                                int64_t bh, int64_t sq, int64_t skv, int32_t head_dim,
                                int32_t block_elements, int32_t topk, float scale,
                                int32_t dtype, void* stream);

/*
 * Tile-layout metadata for a (T, H, W) latent grid and (ts, hs, ws) tiles, in
 * one pass from the closed form of the raster <-> tile mapping.  Replaces
 * build_vsa_metadata's index tensors (fastvideo_tiling.py:22-88, 91-127):
 *   tile_partition_indices[S]  raster token ids in tile-contiguous order
 *                              (get_tile_partition_indices, 22-42);
 *   reverse_indices[S]         its inverse permutation (45-52);
 *   non_pad_index[S]           padded slot n*ts*hs*ws + p of each of them (81-88);
 *   variable_block_sizes[nb]   real tokens per tile (55-78),
 * with S = T*H*W and nb = ceil(T/ts)*ceil(H/hs)*ceil(W/ws); all int64.
 */
int vsa_tile_metadata(int32_t T, int32_t H, int32_t W, int32_t ts, int32_t hs, int32_t ws,
                      int64_t* tile_partition_indices, int64_t* reverse_indices,
                      int64_t* non_pad_index, int64_t* variable_block_sizes, void* stream);

/*
 * Indexed row move along dim 1 of x [batch, x_rows, x_row_bytes] -> out
 * [batch, out_rows, out_row_bytes] (any element type):
 *   for i < n:  s = src_outer ? src[src_outer[i]] : (src ? src[i] : i)
 *               d = dst_outer ? dst[dst_outer[i]] : (dst ? dst[i] : i)
 *               out[b, d, :copy_bytes] = x[b, s, :copy_bytes]
 *               out[b, d, copy_bytes:] = 0
 * (copy_bytes <= both row lengths; unequal row lengths pad or crop the last
 * dimension).  Index values outside their table / the row range are skipped.  With
 * vsa_rows_zero_unmarked it replaces tile's `buf[:, non_pad_index] =
 * x[:, tile_partition_indices]` (fastvideo_tiling.py:137-139), untile's
 * `x[:, non_pad_index][:, reverse]` (145) and the gradients autograd takes
 * through them.  Duplicate destinations race (the indices of a tiling never
 * repeat).
 */
int vsa_rows_move(const void* x, int64_t x_rows, int64_t x_row_bytes, void* out,
                  int64_t out_rows, int64_t out_row_bytes, int64_t copy_bytes, int64_t batch,
                  const int64_t* src, int64_t src_len, const int64_t* src_outer,
                  const int64_t* dst, int64_t dst_len, const int64_t* dst_outer, int64_t n,
                  void* stream);

/*
 * Zero every row of out [batch, out_rows, row] whose index is not listed in
 * marked[n_marked]: the zero padding of tile's `torch.zeros` buffer
 * (fastvideo_tiling.py:137-138) without writing the rows the move fills.
 * mark_workspace: caller-owned, out_rows bytes.
 */
int vsa_rows_zero_unmarked(void* out, int64_t out_rows, int64_t batch, int64_t row_bytes,
                           const int64_t* marked, int64_t n_marked, uint8_t* mark_workspace,
                           void* stream);

/*
 * ---- Tiled sequences: tile() / untile() fused into the op -------------------
 *
 * The reference tiles a raster-order video sequence before the op and untiles
 * the output after it as separate passes (tile: fastvideo_tiling.py:130-140,
 * untile: 143-145).  The entry points below run the op on raster-order
 * q, k, v, gate and dout and return raster-order out, dq, dk, dv and d_gate
 * directly: the passes that read the data anyway (block mean, backward
 * preprocessing) also write the tiled copies the fine kernels consume, and
 * the fine kernels' epilogues store their results at raster rows.  Every
 * value equals the unfused composition tile -> op -> untile bit for bit.
 * slot_rows[nb*be] (int32) maps a tiled slot n*be + p to its raster token,
 * -1 for a padding slot; it is shared by every batch and head.  s_out is the
 * raster length T*H*W, sq = skv = nb*be the tiled length.  The raster tensors
 * are head-major [bh, s_out, D] when heads == 0, or token-major
 * [bh / heads, s_out, heads, D] (a projection's [B, S, H, D] output, tile()'s
 * own [batch, seq, ...] layout) when heads > 0; the tiled tensors are always
 * [bh, sq, D].  bf16 / fp16, head
 * dims 64 and 128, tiles of 64, 128 or 256 tokens; gate_mode 0, 1 or 2 in the
 * input dtype (callers fall back to the composition otherwise).
 */

/*
 * slot_rows for a (T, H, W) latent in (ts, hs, ws) tiles (ceil(T/ts) *
 * ceil(H/hs) * ceil(W/ws) * ts*hs*ws entries), from the closed form of the
 * layout build_vsa_metadata describes (fastvideo_tiling.py:22-88): the
 * inverse of tile_partition_indices / non_pad_index.
 */
int vsa_tile_slot_rows(int32_t T, int32_t H, int32_t W, int32_t ts, int32_t hs, int32_t ws,
                       int32_t* slot_rows, void* stream);

/*
 * tile() of q, k, v [bh, s_out, D] into q_t, k_t, v_t [bh, nb*be, D] (zero rows
 * at padding slots) and the padded block mean of the tiled copies into
 * q_c, k_c, v_c [bh, nb, D], in one pass: vsa_pool_qkv after tile()
 * (fused_block_mean, fused_common.py:20-59, on tile's output), q's means
 * over q_variable_block_sizes, k's and v's over kv_variable_block_sizes.
 * With slot_rows[s] = s (tokens already in block order, s_out = nb*be) this
 * is vsa_pool_qkv reading token-major q, k, v in place.
 */
int vsa_tile_pool_qkv(const void* q, const void* k, const void* v, const int32_t* slot_rows,
                      const int32_t* q_variable_block_sizes,
                      const int32_t* kv_variable_block_sizes, void* q_t, void* k_t, void* v_t,
                      void* q_c, void* k_c, void* v_c, int64_t bh, int64_t s_out, int32_t heads,
                      int32_t nb, int32_t head_dim, int32_t block_elements, int32_t dtype,
                      void* stream);

/*
 * vsa_sparse_fwd on tiled q, k, v with out (and a gate_mode 1 / 2 gate) in
 * raster order [bh, s_out, ...]; fine_out and lse stay tiled.  Padding slots
 * produce no out row.
 */
int vsa_sparse_fwd_tiled(const void* q, const void* k, const void* v, const int32_t* selected,
                         const int32_t* kv_variable_block_sizes, void* out, void* fine_out,
                         float* lse, const void* out_c, const void* gate, int32_t gate_mode,
                         const int32_t* slot_rows, int64_t s_out, int32_t heads, int64_t bh,
                         int64_t sq, int64_t skv, int32_t head_dim, int32_t block_elements,
                         int32_t topk, float scale, int32_t dtype, void* stream);

/*
 * vsa_bwd_prep with dout and the gate in raster order and d_gate written in
 * raster order; fine_out, delta tiled.  Also writes dout_t [bh, sq, D], dout in
 * the tiled layout with zero rows at padding slots (untile's gradient,
 * fastvideo_tiling.py:143-145), for vsa_sparse_bwd_dq_tiled / _dkdv_tiled.
 */
int vsa_bwd_prep_tiled(const void* fine_out, const void* dout, const void* out_c,
                       const void* gate, int32_t gate_mode, const int32_t* slot_rows,
                       int64_t s_out, int32_t heads, float* delta, void* d_out_c, void* d_gate,
                       void* dout_t, int64_t bh, int64_t sq, int32_t head_dim,
                       int32_t block_elements, int32_t dtype, void* stream);

/*
 * vsa_sparse_bwd_dq on tiled inputs (dout = dout_t) with dq written in raster
 * order [bh, s_out, D]: tile()'s gradient (fastvideo_tiling.py:130-140) fused
 * into the dQ epilogue.
 */
int vsa_sparse_bwd_dq_tiled(const void* q, const void* k, const void* v, const void* dout,
                            const float* lse, const float* delta, const int32_t* selected,
                            const int32_t* kv_variable_block_sizes, void* dq, const void* d_q_c,
                            const int32_t* q_variable_block_sizes, const int32_t* slot_rows,
                            int64_t s_out, int32_t heads, int64_t bh, int64_t sq, int64_t skv,
                            int32_t head_dim, int32_t block_elements, int32_t topk, float scale,
                            int32_t dtype, void* stream);

/*
 * vsa_sparse_bwd_dkdv on tiled inputs with dk, dv written in raster order
 * [bh, s_out, D] (tile()'s gradient fused into the dK/dV epilogue).
 */
int vsa_sparse_bwd_dkdv_tiled(const void* q, const void* k, const void* v, const void* dout,
                              const float* lse, const float* delta, const int32_t* counts,
                              const int32_t* offsets, const int32_t* inverse,
                              const int32_t* kv_variable_block_sizes, void* dk, void* dv,
                              const void* d_k_c, const void* d_v_c, const int32_t* slot_rows,
                              int64_t s_out, int32_t heads, int64_t bh, int64_t sq, int64_t skv,
                              int32_t head_dim, int32_t block_elements, int32_t topk, float scale,
                              int32_t* tile_order, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VSA_CAPI_H */
