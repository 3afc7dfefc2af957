// mxs_pick.h -- layout, scratch records and launch arguments of the
// single-kernel token pick behind mxs_sample (mx_sample.hip).
//
// One launch handles a whole batch.  Each logit row is split into C
// balanced chunks of at most CHMAX tokens; a 1024-thread workgroup streams
// one chunk into registers (10 four-token quads per thread), applies logit
// bias, penalties, the grammar mask and the finite check, reduces the
// chunk's statistics and writes its candidate tokens.  The last workgroup
// of a row to arrive (an agent-scope release / acquire on the row's
// counter) then decides the row: greedy argmax, top-k -> top-p -> min-p and
// the inverse-CDF draw.
#pragma once
#include <stdint.h>

#include "../../include/mx_sampler.h"

namespace mxs {
namespace pk {

constexpr int PT = 1024;                        // threads per workgroup
constexpr int PW = PT / 64;                     // waves per workgroup
constexpr int QMAX = 10;                        // quads (4 tokens) per thread per chunk
constexpr uint32_t CHMAX = (uint32_t)PT * QMAX * 4u;  // 40960 tokens per chunk at most
constexpr uint32_t MAXCH = 64;                  // chunks per row at most
constexpr uint32_t VMAX = MAXCH * CHMAX;        // largest vocabulary (2,621,440)
constexpr int NSEG = QMAX * PW;                 // 256-token segments per chunk (one per wave and quad round)
constexpr uint32_t HTAB_MAX = 32767;            // longest history the 15-bit LDS counts take
constexpr uint32_t BCAP = PT;                   // bias entries staged in LDS
constexpr int NBB = 12;                         // log2 of the selection passes' histogram bins
constexpr int NB = 1 << NBB;                    // 4096 bins, four per thread
static_assert(NB == 4 * PT, "four histogram bins per thread");
constexpr uint32_t SYNC = 32;                   // u32 words per row of the row-sync array (one 128-byte line)
constexpr uint32_t NONE = 0xffffffffu;

// Balanced chunk layout of a row of V tokens: C chunks of CH tokens (a
// multiple of 32, so each chunk's mask words start on a word), `per`
// quad rounds of PT threads.
struct Layout {
  uint32_t C, CH, per;
};
inline Layout layout(uint32_t V) {
  uint32_t C = (V + CHMAX - 1u) / CHMAX;
  if (C < 1u) C = 1u;
  uint32_t ch = (V + C - 1u) / C;
  ch = (ch + 31u) & ~31u;
  return {C, ch, (ch / 4u + (uint32_t)PT - 1u) / (uint32_t)PT};
}

// Chunk flags.
enum : uint32_t { F_NONFINITE = 1u, F_BADHIST = 2u, F_BADBIAS = 4u, F_UNIFORM = 8u };

// One chunk's statistics, read by the row's finisher.
struct alignas(16) Stat {
  uint32_t maxkey;    // total-order key of the largest legal adjusted logit; 0 when the chunk has none
  uint32_t gkey;      // greedy: key of the IEEE maximum with -0 merged into +0 (0: none)
  uint32_t gid;       // greedy: lowest token id holding that maximum
  uint32_t nlegal;    // legal tokens in the chunk
  uint32_t ncand;     // candidates written
  uint32_t flags;
  float thr;          // every legal token with adjusted value >= thr is a candidate
  uint32_t minkey;    // total-order key of the smallest legal adjusted logit (NONE: none)
  double mass;        // sum over legal tokens of exp((l - chunk max) / T), when computed
  double mass_err;    // bound on |mass - exact sum|
};
static_assert(sizeof(Stat) == 48, "Stat layout");

// One 256-token segment's mass relative to its own maximum (keep-all rows).
struct alignas(16) Seg {
  float ref;          // the segment's largest legal logit (-inf: none)
  uint32_t pad;
  double mass;        // sum of exp((l - ref) / T) over its legal tokens
};

// Device scratch of mxs_sample, sized for the context's limits.
struct Scratch {
  // [max_rows * SYNC]: per row, word 0 counts the chunks done and word 1
  // holds the largest chunk-maximum key published so far; the row's
  // finisher resets both.  Rows sit on separate cache lines, so the
  // atomics of different rows do not queue on one line.
  uint32_t* sync;
  Stat* stat;         // [max_rows * cm]
  uint2* cand;        // [max_rows * cand_stride] (value bits, token id)
  Seg* seg;           // [max_rows * cm * NSEG]
  uint32_t* gtab;     // [max_rows * gtab_stride] u32 history counts for histories longer than HTAB_MAX
  uint32_t cm;        // chunk records per row
  uint64_t cand_stride, gtab_stride;
};

struct Args {
  const void* logits;
  uint64_t stride;            // elements between rows
  uint32_t rows, V, C, CH, per;
  uint32_t masked, tv, nodraw;
  uint64_t mstride;
  const double* T;
  const uint32_t* topk;
  const double* topp;
  const double* minp;
  const float* rep;
  const float* pres;
  const float* freq;
  const double* u;
  const uint32_t* hoff;
  const uint32_t* hids;
  const uint32_t* boff;
  const uint32_t* bids;
  const float* bvals;
  const uint32_t* mask;
  int32_t* token;
  double* lp;
  int32_t* status;
  uint32_t* kept_count;
  float* adjusted;
  uint32_t* kept_bits;
  Scratch s;
  uint64_t* timing;
};

}  // namespace pk
}  // namespace mxs
