// Host-side check of the dK/dV kernel's LDS map and stage protocol, for every
// (head_dim, block) instantiation.  It uses the kernel's own configuration
// (simple-vsa_amd/csrc/dkdv_cfg.h) and swizzle functions (vsa_device.h):
//  1. the shared-memory regions fit the CU's LDS at the workgroups per CU the
//     launch assumes, and the stage bases are 16-byte aligned;
//  2. the direct-load pieces of a Q / dO tile write every 16-byte chunk of the
//     stage tile exactly once, at the byte where the swizzled reads look for
//     that (row, chunk), from inside the 32-row source tile;
//  3. every row an item copies lies inside the sequence;
//  4. a replay of the step schedule (copies, waits, barriers, reads) for 1..24
//     items: every stage is read only after the barrier that publishes its
//     item (the wait before it leaves only younger copies in flight), and no
//     copy into a stage is issued before every read of the stage's previous
//     item has been retired by a barrier.
// Prints one line per instantiation and "ALL OK"; exits non-zero on a failure.
// Built with one of the PLANT_* macros it replays a protocol with a planted
// mistake, which must fail (tests/test_dkdv_layout.py builds both).
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "dkdv_cfg.h"
#include "vsa_device.h"

using namespace vsa;

static int failures = 0;
#define CHECK(cond, ...)                            \
  do {                                              \
    if (!(cond)) {                                  \
      std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
      std::printf(__VA_ARGS__);                     \
      std::printf("\n");                            \
      ++failures;                                   \
    }                                               \
  } while (0)

// --------------------------------------------------------------------------
// Schedule replay.  Intervals are the stretches between consecutive barriers
// (every wave passes the same barriers).  A read in interval k is retired by
// the barrier that ends k (the barrier waits for LDS reads).  A copy piece is
// an in-order vector load; a wait for at most N loads in flight means every
// load issued before the N most recent has landed.
// --------------------------------------------------------------------------
struct Replay {
  int interval = 0;                    // current interval
  long pieces = 0;                     // copy pieces issued so far (in order)
  std::vector<long> last_piece;        // item -> index of its last piece
  std::vector<int> copy_interval;      // item -> interval its copy was issued in
  std::vector<int> stage_of;           // item -> stage
  std::vector<int> published;          // item -> first interval it is readable in (-1: not yet)
  std::vector<int> last_read;          // item -> last interval a read of it happened in (-1: none)
  std::vector<int> occupant;           // stage -> item currently copied there (-1: none)
  int ns, per;
  const char* name;
  explicit Replay(int ns_, int per_, int items, const char* n)
      : last_piece(items, -1), copy_interval(items, -1), stage_of(items, -1), published(items, -1),
        last_read(items, -1), occupant(ns_, -1), ns(ns_), per(per_), name(n) {}

  void copy(int item, int stage) {
    const int prev = occupant[stage];
    if (prev >= 0)
      CHECK(last_read[prev] < interval, "%s: item %d copied into stage %d in interval %d while item %d "
            "was read there in interval %d", name, item, stage, interval, prev, last_read[prev]);
    occupant[stage] = item;
    stage_of[item] = stage;
    copy_interval[item] = interval;
    pieces += per;
    last_piece[item] = pieces - 1;
  }
  // wait for at most n loads in flight, then a barrier
  void wait_barrier(int n) {
    for (size_t j = 0; j < last_piece.size(); ++j)
      if (last_piece[j] >= 0 && published[j] < 0 && last_piece[j] <= pieces - 1 - n)
        published[j] = interval + 1;
    ++interval;
  }
  void read(int item, int stage) {
    CHECK(stage_of[item] == stage, "%s: item %d read from stage %d, copied to %d", name, item, stage,
          stage_of[item]);
    CHECK(published[item] >= 0 && published[item] <= interval,
          "%s: item %d read in interval %d, published in %d", name, item, interval, published[item]);
    if (interval > last_read[item]) last_read[item] = interval;
  }
};

template <int D, int BE>
static void check_schedule(int items) {
  using C = DkvCfg<D, BE>;
  constexpr int NS = C::NS;
#ifdef PLANT_SHORT_WAIT          // waits that leave one more item in flight
  constexpr int STEP_WAIT = C::STEP_WAIT + C::PER, SIMPLE_WAIT = C::SIMPLE_WAIT + C::PER;
#else
  constexpr int STEP_WAIT = C::STEP_WAIT, SIMPLE_WAIT = C::SIMPLE_WAIT;
#endif
#ifdef PLANT_COPY_INTO_READ_STAGE  // copies into the stage the step's C phase reads
  auto copy_stage = [](int s) { return C::c_stage(s); };
#else
  auto copy_stage = [](int s) { return C::copy_stage(s); };
#endif
#ifdef PLANT_LATE_COPY           // the early barrier before the step's copy pieces
  constexpr int VB = C::CP0 > 0 ? C::CP0 - 1 : 0;
#else
  constexpr int VB = C::VB;
#endif
  const int slots = items + NS + 2;     // items past the end are re-copies of the last one
  char name[64];
  std::snprintf(name, sizeof name, "D%d/BE%d/%d items", D, BE, items);
  Replay r(NS, C::PER, slots, name);
  if (C::WPE > 1) {
    // one item per step: step i waits for item i and copies item i+NS-1
    for (int i = 0; i < NS - 1; ++i) r.copy(i, i % NS);
    for (int it = 0; it < items; ++it) {
      r.wait_barrier(SIMPLE_WAIT);
      const int s = it % NS;
      r.read(it, s);   // rows, statistics, transposed tiles
      r.copy(it + NS - 1, copy_stage(s));
    }
    return;
  }
  // pipelined step: the prologue copies items 0..NS-2, publishes item 0 and runs
  // A(0); with the early barrier it also publishes item 1 and reads its first rows
  for (int i = 0; i < NS - 1; ++i) r.copy(i, i);
  r.wait_barrier((NS - 2) * C::PER);
  r.read(0, 0);
  if (C::EARLY_BARRIER) {
    r.wait_barrier(STEP_WAIT);
    r.read(1, C::a_stage(0));
  }
  for (int it = 0; it < items; ++it) {
    const int s = C::c_stage(it % NS);
    if (!C::EARLY_BARRIER) r.wait_barrier(STEP_WAIT);
    r.read(it + 1, C::a_stage(s));        // A(i+1): rows of item i+1
    r.read(it, s);                         // C(i): transposed tiles of item i
    bool copied = false;
    for (int vv = 0; vv < C::NC; ++vv) {
      // statistics of item i+1 at stream position NA + NC + g, read L ahead
      for (int g = 0; g < 4; ++g)
        if (C::NC + g - C::L == vv || (vv == 0 && C::NC + g - C::L < 0)) r.read(it + 1, C::a_stage(s));
      for (int p = 0; p < C::PER; ++p)
        if (C::piece_iter(p) == vv && !copied) {
          r.copy(it + NS - 1, copy_stage(s));   // all PER pieces of the item
          copied = true;
        }
      if (C::EARLY_BARRIER && vv == VB) {
        CHECK(copied, "%s: barrier before the step's copy", name);
        r.wait_barrier(STEP_WAIT);
        r.read(it + 2, C::pre_stage(s));     // the next step's first rows
      }
    }
    CHECK(copied, "%s: step %d copied nothing", name, it);
  }
}

template <int D, int BE>
static void check_one() {
  using C = DkvCfg<D, BE>;
  using Sh = DkvShared<__bf16, D, BE>;
  const int before = failures;
  // 1. LDS budget and alignment
  const size_t lds = sizeof(Sh) + sizeof(int);   // + the persistent loop's tile index
  CHECK(lds == (size_t)C::LDS_BYTES, "D%d/BE%d: %zu B of LDS, the launch assumes %d", D, BE, lds,
        C::LDS_BYTES);
  CHECK(lds * C::WG_PER_CU <= 160 * 1024 && C::WG_PER_CU >= 1 && C::WG_PER_CU * C::NW <= 4 * C::WPE,
        "D%d/BE%d: %zu B of LDS x %d workgroups per CU", D, BE, lds, C::WG_PER_CU);
  CHECK(offsetof(Sh, smem) % 16 == 0 && offsetof(Sh, sstat) % 16 == 0, "D%d/BE%d: alignment", D, BE);
  CHECK(offsetof(Sh, sstat) == sizeof(__bf16) * C::NS * 2 * C::TILE, "D%d/BE%d: sstat offset", D, BE);
  CHECK(offsetof(Sh, sseg) == offsetof(Sh, sstat) + sizeof(float) * C::NS * 2 * C::QS, "D%d/BE%d: sseg",
        D, BE);
  CHECK(C::NW * 64 == C::NT && C::NW * C::KW == C::KT && C::TP * C::NT * 8 == C::TILE,
        "D%d/BE%d: shape", D, BE);
  // 2. copy pieces of one tile
  std::vector<int> hit(C::QS * (D / 8), 0);
  for (int i = 0; i < C::TP; ++i)
    for (int w = 0; w < C::NW; ++w)
      for (int l = 0; l < 64; ++l) {
        const int blk = C::piece_block(i, w);
        int c = -1;
        const int row = unswz_row_chunk<D>(blk * 64 + l, c);
#ifdef PLANT_SWIZZLE                 // a piece written one chunk over
        const int byte = blk * 1024 + 16 * ((l + 1) & 63);
#else
        const int byte = blk * 1024 + 16 * l;
#endif
        CHECK(row >= 0 && row < C::QS && c >= 0 && c < D / 8, "D%d/BE%d: piece (%d,%d,%d) row %d chunk %d",
              D, BE, i, w, l, row, c);
        if (row < 0 || row >= C::QS || c < 0 || c >= D / 8) continue;
        CHECK(byte + 16 <= C::TILE * 2, "D%d/BE%d: piece byte %d outside the tile", D, BE, byte);
        CHECK(swz<D>(row, c) * 2 == byte, "D%d/BE%d: chunk (%d,%d) written at %d, read at %d", D, BE, row, c,
              byte, swz<D>(row, c) * 2);
        ++hit[row * (D / 8) + c];
      }
  for (size_t x = 0; x < hit.size(); ++x)
    CHECK(hit[x] == 1, "D%d/BE%d: chunk %zu copied %d times", D, BE, x, hit[x]);
  // statistics: lane l copies 4 bytes to byte 4 l of the stage's [2][QS] floats
  CHECK(64 * 4 == (int)sizeof(float) * 2 * C::QS, "D%d/BE%d: statistics copy", D, BE);
  // 3. rows of an item: sub-tile `sub` of query block q is rows q*BE + sub*QS + [0, QS)
  for (int q = 0; q < 4; ++q)
    for (int sub = 0; sub < C::SUBS; ++sub)
      CHECK(q * BE + sub * C::QS + C::QS <= (q + 1) * BE, "D%d/BE%d: rows outside the block", D, BE);
  // 4. schedule replay
  for (int items = 1; items <= 24; ++items) check_schedule<D, BE>(items);
  std::printf("D%d/BE%d: WPE %d, %d keys x %d waves, early barrier %d, LDS %zu B x %d WG/CU: %s\n", D, BE,
              C::WPE, C::KW, C::NW, (int)C::EARLY_BARRIER, lds, C::WG_PER_CU,
              failures == before ? "ok" : "FAILED");
}

int main() {
  check_one<64, 64>();
  check_one<64, 128>();
  check_one<64, 256>();
  check_one<128, 64>();
  check_one<128, 128>();
  check_one<128, 256>();
  check_one<256, 64>();
  check_one<256, 128>();
  check_one<256, 256>();
  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  std::printf("ALL OK\n");
  return 0;
}
