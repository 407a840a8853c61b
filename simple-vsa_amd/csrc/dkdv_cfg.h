// Shape, LDS layout and stage protocol of the dK/dV kernel (fine_bwd.hip),
// kept apart so that a host program can check them: every value here is a
// compile-time constant or a host-and-device function, and the kernel takes
// its stage indices, copy placement and barrier position from these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vsa {

template <int D, int BE>
struct DkvCfg {
  // waves per SIMD: two at head_dim 64 with block 64 (32 keys each, one item
  // per step: the other wave of the SIMD covers a wave's P / dS arithmetic,
  // which at head_dim 64 is as long as its MFMAs), else one
  static constexpr int WPE = (D == 64 && BE == 64) ? 2 : 1;
  // keys per wave: 64 at head_dim 64 (one wave per SIMD), where the fragments
  // and accumulators of two key tiles fit one wave's 512 registers and each
  // Q / dO operand read from LDS then feeds two MFMAs; 32 otherwise
  static constexpr int KW = (D == 64 && WPE == 1) ? 64 : 32;
  static constexpr int KTL = KW / 32;              // 32-key MFMA tiles per wave
  static constexpr int KT = BE < 4 * KW ? BE : 4 * KW;  // keys per workgroup
  static constexpr int NW = KT / KW;
  static constexpr int NT = NW * 64;
  static constexpr int QS = 32;                    // queries per LDS stage
  static constexpr int TILE = QS * D;              // one Q (or dO) sub-tile, swizzled
  static constexpr int SUBS = BE / QS;             // sub-tiles per query block
  static constexpr int NS = 4;                     // LDS ring depth (loop unrolled by NS)
  static constexpr int TP = TILE / 8 / NT;         // direct loads per thread per tile
  static constexpr int PER = 2 * TP + 1;           // direct loads per thread per item
  // Direct-load piece i (< TP) of a Q or dO tile: lane l of wave w copies the
  // 16-byte chunk that the swizzle places at byte 1024 * piece_block(i, w) +
  // 16 l of the tile (unswz_row_chunk gives its row and chunk).
  static __host__ __device__ constexpr int piece_block(int i, int w) { return i * NW + w; }
  // CSR entries staged in LDS (1024 where several workgroups share a CU)
  static constexpr int SEGMAX = (NW == 1 || WPE > 1) ? 1024 : 2048;
  // dK/dV dims accumulated per workgroup: all of them up to 128; for head_dim
  // 256 two workgroups share a key tile, each computing S and dP over all 256
  // dims and accumulating one 128-dim half of dK and dV (the full accumulators
  // would not fit next to the K and V fragments)
  static constexpr int DH = D > 128 ? 128 : D;
  static constexpr int NSPLIT = D / DH;
  static constexpr int NA = 2 * (D / 16);          // LDS reads of A (Q and dO rows interleaved)
  static constexpr int NC = 4 * (DH / 32);         // LDS reads of C (dO^T and Q^T tiles)
  static constexpr int NV = 16 * KTL;              // P (and dS) values per lane and item
  static constexpr int L = D > 128 ? 6 : KTL > 1 ? 6 : 12;  // LDS operand lookahead (reads)
  // Step barrier inside the previous step's dV / dK phase (see dkdv_tile); at
  // block 64 the operands it keeps live across the step boundary do not fit
  // the register file, and those kernels keep the barrier at the step's top.
  static constexpr bool EARLY_BARRIER = BE >= 128 && WPE == 1;
  // LDS of a workgroup (DkvShared with 2-byte elements, plus the persistent
  // loop's tile index) and the workgroups a CU holds at once: WPE waves per
  // SIMD, within the CU's 160 KiB of LDS
  static constexpr int LDS_BYTES = NS * 2 * TILE * 2 + NS * 2 * QS * 4 + SEGMAX * 4 + 2 * DH * 2 + 4;
  static constexpr int WG_BY_WAVES = 4 * WPE / NW;
  static constexpr int WG_BY_LDS = 160 * 1024 / LDS_BYTES;
  static constexpr int WG_PER_CU = WG_BY_WAVES < WG_BY_LDS ? WG_BY_WAVES : WG_BY_LDS;
  static_assert(WG_PER_CU >= 1, "a workgroup must fit a CU");

  // ---- stage protocol of the pipelined step (WPE == 1) ----
  // Step i reads item i+1's rows (A) from stage a_stage(i), item i's
  // transposed tiles (C) from c_stage(i), item i+1's statistics from
  // a_stage(i), and copies item i+NS-1 into copy_stage(i); with the early
  // barrier the next step's first L rows (item i+2) are read from pre_stage(i)
  // right after it.
  static constexpr int c_stage(int s) { return s % NS; }
  static constexpr int a_stage(int s) { return (s + 1) % NS; }
  static constexpr int pre_stage(int s) { return (s + 2) % NS; }
  static constexpr int copy_stage(int s) { return (s + NS - 1) % NS; }
  // C iterations after the early barrier, the C iteration it follows (NC: no
  // early barrier), and the C iterations the copy pieces are spread over
  static constexpr int KB = KTL > 1 ? 2 : 4;
  static constexpr int VB = EARLY_BARRIER ? NC - 1 - KB : NC;
  static constexpr int CP0 = EARLY_BARRIER ? NC / 4 : NC / 2;
  static constexpr int CP1 = EARLY_BARRIER ? VB : NC - 1;
  // C iteration that issues copy piece p (p < PER)
  static constexpr int piece_iter(int p) { return CP0 + (p * (CP1 - CP0 + 1)) / PER; }
  // loads in flight allowed at a step's wait: the items copied after the one
  // the wait is for (PER pieces each)
  static constexpr int STEP_WAIT = (NS - 3) * PER;
  static_assert(!EARLY_BARRIER || (VB >= CP0 && L <= NA), "barrier placement");

  // ---- one item per step (WPE > 1) ----
  // step i reads item i from stage i % NS and copies item i+NS-1 into the
  // stage of item i-1; its wait leaves the two younger items in flight
  static constexpr int SIMPLE_WAIT = (NS - 2) * PER;
};

template <typename T, int D, int BE>
struct DkvShared {
  using C = DkvCfg<D, BE>;
  __attribute__((aligned(16))) T smem[C::NS][2 * C::TILE];
  __attribute__((aligned(16))) float sstat[C::NS][2][C::QS];  // [stage][lse, delta][query]
  int32_t sseg[C::SEGMAX];
  // the key block's pooled dK and dV rows (this workgroup's DH dims), divided
  // by the block's token count and rounded to T: the same for every key
  __attribute__((aligned(16))) T spool[2][C::DH];
};

}  // namespace vsa
