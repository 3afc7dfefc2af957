// mx_sample.hip -- mxs_sample: the single-kernel token pick for MI355X (gfx950).
//
// One launch per call.  A row of V logits is split into C balanced chunks of
// at most 20480 tokens; one 512-thread workgroup streams a chunk into
// registers (16-byte quads, ten per thread, every load issued up front),
// while the row's history ids, which are issued first, build an LDS count
// table.  As each quad lands it gets logit bias and penalties, the grammar
// mask, the finite check and the running maximum.  The chunk then publishes
// its maximum, picks a candidate threshold that is a proven lower bound of
// every token the row's decision can need, writes its candidates in token-ID
// order, and arrives on the row's counter.  The last chunk of the row to
// arrive (agent-scope release/acquire) decides the row: greedy argmax, or
// top-k -> top-p -> min-p -> inverse-CDF draw over the candidates.
//
// Reference semantics (arclabs561/metallix):
//   nucleus_mask        crates/app/cli/src/qwen_forward.rs:474-549
//   sample_categorical  crates/core/engine/src/sampling.rs:56-158
//   greedy_token        crates/app/cli/src/chat_generation.rs:2213-2231
//   masked_argmax       crates/core/engine/src/constraint.rs:895-932
//   fill_legal_mask     crates/core/engine/src/constraint.rs:793-806
// plus the penalty, bias, min-p and mask-with-nucleus stages this sampler
// defines (the oracle's orc_sample_row states them executably).
//
// Exactness.  The reference sums f64 weights sequentially; this kernel sums
// them in parallel.  Every comparison against such a sum (the top-p cut, the
// draw) is taken only when its margin exceeds a rigorous bound on the
// difference of the two computations (both summation orders, 1 ulp of
// exp on each side, the f64 rounding of the shifted logit).  A decision
// inside its bound leaves the row with status 1 (uncertified) and the
// device's best decision.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_math.h"
#include "mxs_pick.h"

namespace mxs {
namespace pk {

constexpr double U53 = 1.1102230246251565e-16;   // 2^-53
constexpr float U24 = 5.9604644775390625e-08f;   // 2^-24
constexpr double LOG2E = 1.4426950408889634;

// Workgroup barrier for LDS traffic only (outstanding global loads keep
// streaming across it).
__device__ __forceinline__ void bar() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t popc(uint32_t x) { return (uint32_t)__builtin_popcount(x); }
__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
__device__ __forceinline__ float fmax_(float a, float b) { return vmax(a, b); }
__device__ __forceinline__ double rd_lane(double v, uint32_t l) {
  return __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, v), l));
}

// ---------------------------------------------------------------------------
// LDS: one static pool, carved per phase.
constexpr uint32_t NCL = 6144;       // candidates the finisher keeps in LDS
struct alignas(16) Mem {             // one gathered member of a histogram bin
  uint32_t key, id;
  double w;
};
struct alignas(16) Lds {
  union {
    struct {
      uint32_t ctab[CHMAX / 2];      // per token a u16: history count (15 bits) | bias flag (bit 15)
      uint32_t mask[CHMAX / 32];     // the chunk's grammar-mask words
      uint32_t bid[BCAP];            // the row's bias list (when it has at most BCAP entries)
      float bval[BCAP];
    } c;
    uint32_t hist[NB];               // chunk top-k threshold histogram (after the quad loop)
    struct {
      float cl[NCL];                 // the finisher's working candidate list (token-ID order)
      uint32_t cid[NCL];
      double cw[NCL];                // each entry's weight exp((l - M) / T) (0 below the threshold)
      double bm[NB];                 // per-bin f64 mass
      uint32_t bc[NB];               // per-bin count
      Mem mem[64];                   // gathered members of one bin
      Mem dmem[64];                  // the register finisher's survivors in token order
      uint32_t mix[64];              // their token-order indices
      uint32_t dkf[64];              // kept flags in token order
      uint32_t nmem;
      uint32_t segtab[256];          // the draw segment's history counts (keep-all rows)
    } f;
  } u;
  uint32_t wcnt[QMAX * PW];          // candidates per (quad round, wave)
  uint32_t woff[QMAX * PW];
  uint32_t wr[4 * PW];               // per-wave chunk reductions (max key, flags, legal count, min key)
  unsigned long long wg[PW];         // per-wave greedy keys
  uint32_t coff[MAXCH + 1];          // candidate offsets of the row's chunks
  uint32_t bc[8];                    // broadcast words
  double bd[4];
  // one-barrier block reductions: two slot sets, used alternately
  uint32_t xu[2][4 * PW];
  double xd[2][2 * PW];
  unsigned long long xq[2][PW];
};

// ---------------------------------------------------------------------------
// Block reductions and scans for PT-thread workgroups, one barrier each.
// Every thread makes the same sequence of calls; successive calls alternate
// between two LDS slot sets (Blk::p), so a set is rewritten only after a
// later call's barrier has passed every reader of its previous contents.
__device__ __forceinline__ uint32_t lane_() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_() { return threadIdx.x >> 6; }
struct Blk {
  uint32_t p = 0u;
};
// The finisher's width: a row whose candidate list is short is finished by
// one wave (the others end once the list is in LDS), with no cross-wave
// reductions; a long list keeps every wave.  nb histogram bins (nbb bits),
// bpt per thread.
struct Fw {
  uint32_t nt, nw, nb, nbb, bpt;
};
constexpr uint32_t BPT_MAX = 8;
constexpr uint32_t SHORT_LIST = 512;   // lists up to this length take one wave
__device__ __forceinline__ uint32_t red_sum_u32(uint32_t v, Lds& S, Blk& B, uint32_t nw) {
  v = wave_sum_u32(v);
  if (lane_() == 0u) S.xu[B.p][wave_()] = v;
  bar();
  uint32_t s = 0u;
  for (uint32_t i = 0; i < nw; ++i) s += S.xu[B.p][i];
  B.p ^= 1u;
  return s;
}
__device__ __forceinline__ uint32_t red_or_u32(uint32_t v, Lds& S, Blk& B, uint32_t nw) {
  v = wave_or_u32(v);
  if (lane_() == 0u) S.xu[B.p][wave_()] = v;
  bar();
  uint32_t s = 0u;
  for (uint32_t i = 0; i < nw; ++i) s |= S.xu[B.p][i];
  B.p ^= 1u;
  return s;
}
__device__ __forceinline__ uint32_t red_min_u32(uint32_t v, Lds& S, Blk& B, uint32_t nw) {
  v = ~wave_max_u32(~v);
  if (lane_() == 0u) S.xu[B.p][wave_()] = v;
  bar();
  uint32_t s = NONE;
  for (uint32_t i = 0; i < nw; ++i) s = min(s, S.xu[B.p][i]);
  B.p ^= 1u;
  return s;
}
__device__ __forceinline__ double red_sum_f64(double v, Lds& S, Blk& B, uint32_t nw) {
  v = wave_sum_f64(v);
  if (lane_() == 0u) S.xd[B.p][wave_()] = v;
  bar();
  double s = 0.0;
  for (uint32_t i = 0; i < nw; ++i) s += S.xd[B.p][i];
  B.p ^= 1u;
  return s;
}
// The block sum of `sum` and the minimum of nonnegative `mn` (f64 bit
// patterns of nonnegative values order as u64), in one barrier.
__device__ __forceinline__ void red_sum_minpos_f64(double sum, double mn, Lds& S, Blk& B, double* osum, double* omin,
                                                   uint32_t nw) {
  sum = wave_sum_f64(sum);
  const unsigned long long m = ~wave_max_u64(~__builtin_bit_cast(unsigned long long, mn));
  if (lane_() == 0u) {
    S.xd[B.p][wave_()] = sum;
    S.xq[B.p][wave_()] = m;
  }
  bar();
  double s = 0.0;
  unsigned long long r = ~0ull;
  for (uint32_t i = 0; i < nw; ++i) {
    s += S.xd[B.p][i];
    r = min(r, S.xq[B.p][i]);
  }
  B.p ^= 1u;
  *osum = s;
  *omin = __builtin_bit_cast(double, r);
}
// Inclusive scans in thread order (f64: the lane tree, then the waves in
// order); *total receives the block total.
__device__ __forceinline__ uint32_t scan_u32(uint32_t v, Lds& S, Blk& B, uint32_t* total, uint32_t nw) {
  const uint32_t inc = wave_scan_u32(v);
  if (lane_() == 63u) S.xu[B.p][wave_()] = inc;
  bar();
  uint32_t before = 0u, all = 0u;
  for (uint32_t i = 0; i < nw; ++i) {
    const uint32_t r = S.xu[B.p][i];
    before += i < wave_() ? r : 0u;
    all += r;
  }
  B.p ^= 1u;
  *total = all;
  return before + inc;
}
__device__ __forceinline__ double scan_f64(double v, Lds& S, Blk& B, double* total, uint32_t nw) {
  const double inc = wave_scan_f64(v);
  if (lane_() == 63u) S.xd[B.p][wave_()] = inc;
  bar();
  double before = 0.0, all = 0.0;
  for (uint32_t i = 0; i < nw; ++i) {
    const double r = S.xd[B.p][i];
    if (i < wave_()) before += r;
    all += r;
  }
  B.p ^= 1u;
  *total = all;
  return before + inc;
}

// ---------------------------------------------------------------------------
// Row parameters.  Parameter errors in the oracle's precedence: temperature,
// top_p, min_p, penalties (decided before any data), then history ids, bias
// ids and the uniform (carried as chunk flags).
struct Cfg {
  double T, top_p, min_p, u, inv_rep, invT;
  double L_mp;    // ln(min_p) (-inf when min_p = 0)
  double L_nuc;   // ln((1 - top_p) / (2 V)), the nucleus bound's offset (-inf: no bound)
  uint32_t k, h0, hlen, b0, blen;
  float rep, pres, freq;
  int32_t err;
  bool greedy, uerr;
};
// Row-uniform values moved to scalar registers.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ float uni(float v) { return __uint_as_float(uni(__float_as_uint(v))); }
__device__ __forceinline__ double uni(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  return __builtin_bit_cast(double, ((unsigned long long)uni((uint32_t)(b >> 32)) << 32) | uni((uint32_t)b));
}
__device__ __forceinline__ Cfg load_cfg(const Args& A, uint32_t row) {
  Cfg c;
  c.T = uni(A.T[row]);
  c.k = uni(A.topk[row]);
  c.top_p = uni(A.topp[row]);
  c.min_p = uni(A.minp[row]);
  c.rep = uni(A.rep[row]);
  c.pres = uni(A.pres[row]);
  c.freq = uni(A.freq[row]);
  c.u = uni(A.u[row]);
  c.h0 = uni(A.hoff[row]);
  c.hlen = uni(A.hoff[row + 1]) - c.h0;
  c.b0 = uni(A.boff[row]);
  c.blen = uni(A.boff[row + 1]) - c.b0;
  c.greedy = c.T == 0.0;
  int32_t e = 0;
  if (!(c.T >= 0.0) || !isfinite(c.T)) e = MXS_ROW_INVALID_TEMPERATURE;
  else if (!c.greedy && !(c.top_p > 0.0 && c.top_p <= 1.0)) e = MXS_ROW_INVALID_TOP_P;
  else if (!c.greedy && !(c.min_p >= 0.0 && c.min_p <= 1.0)) e = MXS_ROW_INVALID_MIN_P;
  else if (!(isfinite(c.rep) && c.rep > 0.0f) || !isfinite(c.pres) || !isfinite(c.freq)) e = MXS_ROW_INVALID_PENALTY;
  c.err = e;
  c.uerr = !c.greedy && !(isfinite(c.u) && c.u >= 0.0 && c.u < 1.0);
  c.inv_rep = uni(1.0 / (double)c.rep);
  c.invT = uni(c.greedy ? 0.0 : 1.0 / c.T);
  c.L_mp = -INFINITY;
  c.L_nuc = -INFINITY;
  return c;
}

__device__ __forceinline__ void stamp(const Args& A, uint32_t row, uint32_t slot, uint32_t k) {
  if (A.timing) A.timing[((uint64_t)row * MXS_DEBUG_TIMING_SLOTS + slot) * 8u + k] = wall_clock64();
}

// The bias value of token `tok` (which has an entry): binary search in the
// row's sorted list, in LDS when it has at most BCAP entries.
__device__ __forceinline__ float bias_of(const Args& A, const Cfg& cf, const Lds& S, uint32_t tok) {
  uint32_t lo = 0, hi = cf.blen;
  if (cf.blen <= BCAP) {
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (S.u.c.bid[mid] < tok) lo = mid + 1u; else hi = mid;
    }
    return S.u.c.bval[min(lo, cf.blen - 1u)];
  }
  const uint32_t* ids = A.bids + cf.b0;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (ids[mid] < tok) lo = mid + 1u; else hi = mid;
  }
  return A.bvals[cf.b0 + min(lo, cf.blen - 1u)];
}

// The keep-all rows' f64 segment mass: exp((l - ref) / T) with the shift
// multiplied by 1/T (an extra rounding the draw's error bound covers).
__device__ __forceinline__ double seg_w(float l, float ref, double invT) {
  return exp_neg(((double)l - (double)ref) * invT);
}

// ===========================================================================
// The row finisher.  Runs on the last-arriving chunk workgroup of the row.
// ===========================================================================

// The row's working candidate list (token-ID order): in LDS when it fits,
// with each entry's weight, else read in place from the chunks' global lists.
struct Work {
  uint32_t n;
  bool lds;
  float thr;   // entries below thr are not candidates (the lists hold some)
};

__device__ __forceinline__ void wget(const Args& A, const Lds& S, uint32_t row, const Work& W, uint32_t i, float* l,
                                     uint32_t* id) {
  if (W.lds) {
    *l = S.u.f.cl[i];
    *id = S.u.f.cid[i];
    return;
  }
  uint32_t lo = 0, hi = A.C;   // the last chunk c with coff[c] <= i
  while (hi - lo > 1u) {
    const uint32_t mid = (lo + hi) >> 1;
    if (S.coff[mid] <= i) lo = mid; else hi = mid;
  }
  const uint2 e = A.s.cand[(uint64_t)row * A.s.cand_stride + (uint64_t)lo * A.CH + (i - S.coff[lo])];
  *l = __uint_as_float(e.x);
  *id = e.y;
}
// entry i's weight exp((l - M) / T): cached in LDS, else evaluated
__device__ __forceinline__ double wgt(const Lds& S, const Work& W, uint32_t i, float l, double Md, double invT) {
  return W.lds ? S.u.f.cw[i] : exp_neg(((double)l - Md) * invT);
}

// Passes over the working list.  For an LDS list every thread's entries are
// loaded together first (at most RMAX per thread), so a pass costs one LDS
// round trip rather than one per entry; a global list is walked in place.
// each(): entries t, t + nt, ...; each_range(): the contiguous [i0, i1).
// fn(i, l, id, w) receives the entry and its weight (cached in LDS, else
// evaluated only when `need_w`).
constexpr uint32_t RMAX = 8;    // 8 x 64 >= SHORT_LIST and 8 x PT >= NCL
constexpr uint32_t RBATCH = 4;  // entries loaded together (register budget)
template <bool need_w, typename Fn>
__device__ __forceinline__ void each(const Args& A, const Lds& S, uint32_t row, const Work& W, const Fw& F, double Md,
                                     double invT, Fn fn) {
  const uint32_t t = threadIdx.x;
  if (W.lds) {
#pragma unroll
    for (uint32_t r0 = 0; r0 < RMAX; r0 += RBATCH) {
      if (t + r0 * F.nt >= W.n) break;
      float l[RBATCH];
      uint32_t id[RBATCH];
      double wv[RBATCH];
#pragma unroll
      for (uint32_t r = 0; r < RBATCH; ++r) {
        const uint32_t i = t + (r0 + r) * F.nt;
        l[r] = 0.0f;
        id[r] = 0u;
        wv[r] = 0.0;
        if (i < W.n) {
          l[r] = S.u.f.cl[i];
          id[r] = S.u.f.cid[i];
          if (need_w) wv[r] = S.u.f.cw[i];
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < RBATCH; ++r) {
        const uint32_t i = t + (r0 + r) * F.nt;
        if (i < W.n) fn(i, l[r], id[r], wv[r]);
      }
    }
  } else {
    for (uint32_t i = t; i < W.n; i += F.nt) {
      float l;
      uint32_t id;
      wget(A, S, row, W, i, &l, &id);
      fn(i, l, id, need_w ? exp_neg(((double)l - Md) * invT) : 0.0);
    }
  }
}
template <bool need_w, typename Fn>
__device__ __forceinline__ void each_range(const Args& A, const Lds& S, uint32_t row, const Work& W, uint32_t i0,
                                           uint32_t i1, double Md, double invT, Fn fn) {
  if (W.lds) {
#pragma unroll
    for (uint32_t r0 = 0; r0 < RMAX; r0 += RBATCH) {
      if (i0 + r0 >= i1) break;
      float l[RBATCH];
      uint32_t id[RBATCH];
      double wv[RBATCH];
#pragma unroll
      for (uint32_t r = 0; r < RBATCH; ++r) {
        const uint32_t i = i0 + r0 + r;
        l[r] = 0.0f;
        id[r] = 0u;
        wv[r] = 0.0;
        if (i < i1) {
          l[r] = S.u.f.cl[i];
          id[r] = S.u.f.cid[i];
          if (need_w) wv[r] = S.u.f.cw[i];
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < RBATCH; ++r) {
        const uint32_t i = i0 + r0 + r;
        if (i < i1) fn(i, l[r], id[r], wv[r]);
      }
    }
  } else {
    for (uint32_t i = i0; i < i1; ++i) {
      float l;
      uint32_t id;
      wget(A, S, row, W, i, &l, &id);
      fn(i, l, id, need_w ? exp_neg(((double)l - Md) * invT) : 0.0);
    }
  }
}

// Copies the entries of the chunks' global lists that satisfy keep(l, id)
// into LDS with their weights, in token-ID order (each thread a contiguous
// range, then a block scan).  Returns the count; the caller checks it fits.
template <typename Keep>
__device__ __forceinline__ uint32_t compact(const Args& A, Lds& S, Blk& B, const Fw& F, uint32_t row, uint32_t N, Keep keep,
                                            double Md, double invT) {
  const uint32_t t = threadIdx.x;
  const Work G{N, false, -INFINITY};
  const uint32_t R = (N + F.nt - 1u) / F.nt, i0 = min(N, t * R), i1 = min(N, i0 + R);
  uint32_t mine = 0u;
  for (uint32_t i = i0; i < i1; ++i) {
    float l;
    uint32_t id;
    wget(A, S, row, G, i, &l, &id);
    mine += keep(l, id) ? 1u : 0u;
  }
  uint32_t tot;
  uint32_t p = scan_u32(mine, S, B, &tot, F.nw) - mine;
  for (uint32_t i = i0; i < i1; ++i) {
    float l;
    uint32_t id;
    wget(A, S, row, G, i, &l, &id);
    if (keep(l, id) && p < NCL) {
      S.u.f.cl[p] = l;
      S.u.f.cid[p] = id;
      S.u.f.cw[p] = exp_neg(((double)l - Md) * invT);
      ++p;
    }
  }
  bar();
  return tot;
}

// Keeps the LDS working list's entries with keep(l, id), in order, in place:
// every thread reads its contiguous share into registers before any write.
// Full width only (F.nt = PT).
template <typename Keep>
__device__ __forceinline__ uint32_t compact_lds(Lds& S, Blk& B, const Fw& F, const Work& W, Keep keep) {
  const uint32_t t = threadIdx.x;
  constexpr uint32_t RM = (NCL + PT - 1u) / PT;
  const uint32_t R = (W.n + F.nt - 1u) / F.nt, i0 = min(W.n, t * R);
  float l[RM];
  uint32_t id[RM];
  double wv[RM];
  uint32_t km = 0u, mine = 0u;
#pragma unroll
  for (uint32_t r = 0; r < RM; ++r) {
    const uint32_t i = i0 + r;
    l[r] = -INFINITY;
    id[r] = 0u;
    wv[r] = 0.0;
    if (r < R && i < W.n) {
      l[r] = S.u.f.cl[i];
      id[r] = S.u.f.cid[i];
      wv[r] = S.u.f.cw[i];
      if (l[r] >= W.thr && keep(l[r], id[r])) {
        km |= 1u << r;
        ++mine;
      }
    }
  }
  uint32_t tot;
  uint32_t p = scan_u32(mine, S, B, &tot, F.nw) - mine;   // (its barrier also ends every read)
#pragma unroll
  for (uint32_t r = 0; r < RM; ++r) {
    if ((km >> r) & 1u) {
      S.u.f.cl[p] = l[r];
      S.u.f.cid[p] = id[r];
      S.u.f.cw[p] = wv[r];
      ++p;
    }
  }
  bar();
  return tot;
}

// Error bound for comparing an f64 sum of n weights (each at most 1, total
// S) formed here with the reference's sequential sum of the same weights:
// 1 ulp of exp on each side, the shift rounded once more here, both sides'
// summation errors, and the weights' own absolute rounding.
__device__ __forceinline__ double sum_err(double S, double n) { return (S * (2.0 * n + 40.0) + n) * U53; }

// The reference's descending comparator: total order of the value, then
// ascending id.  better(a, b): a sorts before b.
__device__ __forceinline__ bool better(uint32_t ka, uint32_t ia, uint32_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// In the descending order (key desc, id asc) over the working list's members
// (member(l, id)), finds the first member at which the running measure
// reaches `need`.  The measure is 1 per member (MASS = false: the need-th
// member) or its weight exp((l - M) / T) (MASS = true: the first member whose
// inclusive running mass is >= need).  Bins of d = Mkey - key, refined F.nbb
// bits at a time; a bin of at most 64 members is finished on one wave; equal
// keys are taken in ID order.  Outputs the member's key and id, the running
// measure before it (*before) and its own (*wself).  *found = false when the
// members' total stays below `need` (*before then holds that total).
template <bool MASS, typename Memb>
__device__ __forceinline__ void crossing(const Args& A, Lds& S, Blk& B, const Fw& F, uint32_t row, const Work& W,
                                         Memb member,
                                         uint32_t Mkey, double Md, double invT, uint32_t dmax, double need,
                                         bool* found, uint32_t* kout, uint32_t* iout, double* before,
                                         double* wself) {
  const uint32_t t = threadIdx.x;
  uint32_t lo = 0;
  int sh = 32 - __builtin_clz(dmax | 1u) - (int)F.nbb;
  if (sh < 0) sh = 0;
  double cum = 0.0;   // measure of the members before the current range
  for (;;) {
    for (uint32_t b = t; b < F.nb; b += F.nt) {
      S.u.f.bc[b] = 0u;
      if (MASS) S.u.f.bm[b] = 0.0;
    }
    if (t == 0) {
      S.u.f.nmem = 0u;
      S.bc[0] = NONE;
    }
    bar();
    const uint32_t span = sh >= 32 - (int)F.nbb ? 0xffffffffu : ((F.nb << sh) - 1u);
    each<MASS>(A, S, row, W, F, Md, invT, [&](uint32_t, float l, uint32_t id, double wv) {
      if (!(l >= W.thr) || !member(l, id)) return;
      const uint32_t d = Mkey - okey(l);
      if (d < lo || d - lo > span) return;
      const uint32_t b = (d - lo) >> sh;
      atomicAdd(&S.u.f.bc[b], 1u);
      if (MASS) atomicAdd(&S.u.f.bm[b], wv);
    });
    bar();
    // thread t owns bins bpt t .. bpt t + bpt - 1 (descending value order)
    uint32_t c4[BPT_MAX], csum = 0u;
    double m4[BPT_MAX], msum = 0.0;
#pragma unroll
    for (int q = 0; q < (int)BPT_MAX; ++q) {
      c4[q] = 0u;
      m4[q] = 0.0;
      if (q < (int)F.bpt) {
        c4[q] = S.u.f.bc[F.bpt * t + (uint32_t)q];
        m4[q] = MASS ? S.u.f.bm[F.bpt * t + (uint32_t)q] : (double)c4[q];
      }
      csum += c4[q];
      msum += m4[q];
    }
    double incl, tot;
    if (MASS) {
      incl = scan_f64(msum, S, B, &tot, F.nw);
    } else {
      uint32_t tu;
      incl = (double)scan_u32(csum, S, B, &tu, F.nw);
      tot = (double)tu;
    }
    const double tb = cum + (incl - msum);
    if (tb < need && cum + incl >= need) {
      double r = tb;
      bool done = false;
#pragma unroll
      for (int q = 0; q < (int)BPT_MAX; ++q) {
        if (!done && q < (int)F.bpt && r + m4[q] >= need) {
          S.bc[0] = F.bpt * t + (uint32_t)q;
          S.bc[1] = c4[q];
          S.bd[0] = r;
          done = true;
        }
        r += m4[q];
      }
    }
    bar();
    const uint32_t bstar = S.bc[0];
    if (bstar == NONE) {
      *found = false;
      *before = cum + tot;
      *wself = 0.0;
      return;
    }
    const uint32_t bcnt = S.bc[1];
    cum = S.bd[0];
    lo += bstar << sh;
    if (bcnt <= 64u) {
      const uint32_t bspan = sh >= 32 ? 0xffffffffu : ((1u << sh) - 1u);
      each<MASS>(A, S, row, W, F, Md, invT, [&](uint32_t, float l, uint32_t id, double wv) {
        if (!(l >= W.thr) || !member(l, id)) return;
        const uint32_t d = Mkey - okey(l);
        if (d < lo || d - lo > bspan) return;
        const uint32_t p = atomicAdd(&S.u.f.nmem, 1u);
        if (p < 64u) {
          Mem e;
          e.key = okey(l);
          e.id = id;
          e.w = MASS ? wv : 1.0;
          S.u.f.mem[p] = e;
        }
      });
      bar();
      if (t < 64u) {
        const uint32_t n = min(S.u.f.nmem, 64u);
        Mem me;
        me.key = 0u;
        me.id = NONE;
        me.w = 0.0;
        if (t < n) me = S.u.f.mem[t];
        // the measure of the bin's members before this one
        double bef = 0.0;
        for (uint32_t j = 0; j < n; ++j) {
          const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)j);
          const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)j);
          const double wj = rd_lane(me.w, j);
          if (better(kj, ij, me.key, me.id)) bef += wj;
        }
        const uint64_t hm = ballot(t < n && cum + bef < need && cum + bef + me.w >= need);
        if (hm) {
          if (t == (uint32_t)__builtin_ctzll(hm)) {
            S.bc[2] = me.key;
            S.bc[3] = me.id;
            S.bd[1] = cum + bef;
            S.bd[2] = me.w;
            S.bc[4] = 1u;
          }
        } else {
          const double all = cum + wave_sum_f64(t < n ? me.w : 0.0);
          if (t == 0u) {
            S.bc[4] = 0u;
            S.bd[1] = all;
            S.bd[2] = 0.0;
          }
        }
      }
      bar();
      *found = S.bc[4] != 0u;
      *kout = S.bc[2];
      *iout = S.bc[3];
      *before = S.bd[1];
      *wself = S.bd[2];
      return;
    }
    if (sh == 0) break;
    sh = sh > (int)F.nbb ? sh - (int)F.nbb : 0;
  }
  // equal keys (Mkey - lo) in ID order: contiguous ranges and a block scan
  const uint32_t kk = Mkey - lo;
  const uint32_t R = (W.n + F.nt - 1u) / F.nt, i0 = min(W.n, t * R), i1 = min(W.n, i0 + R);
  double mine = 0.0;
  each_range<MASS>(A, S, row, W, i0, i1, Md, invT, [&](uint32_t, float l, uint32_t id, double wv) {
    if (l >= W.thr && member(l, id) && okey(l) == kk) mine += MASS ? wv : 1.0;
  });
  double tot;
  const double incl = scan_f64(mine, S, B, &tot, F.nw);
  double r = cum + incl - mine;
  uint32_t best = NONE;
  double bb = 0.0, bw = 0.0;
  each_range<MASS>(A, S, row, W, i0, i1, Md, invT, [&](uint32_t, float l, uint32_t id, double wv) {
    if (best != NONE || !(l >= W.thr) || !member(l, id) || okey(l) != kk) return;
    const double m = MASS ? wv : 1.0;
    if (r < need && r + m >= need) { best = id; bb = r; bw = m; }
    r += m;
  });
  const uint32_t win = red_min_u32(best, S, B, F.nw);
  if (win != NONE && best == win) {
    S.bd[1] = bb;
    S.bd[2] = bw;
  }
  bar();
  *found = win != NONE;
  *kout = kk;
  *iout = win;
  *before = win != NONE ? S.bd[1] : cum + tot;
  *wself = win != NONE ? S.bd[2] : 0.0;
}

// Writes one row's outputs.
__device__ __forceinline__ void put_row(const Args& A, uint32_t row, int32_t status, int32_t token, double lp,
                                        uint32_t kept) {
  A.token[row] = token;
  A.status[row] = status;
  if (A.lp) A.lp[row] = lp;
  if (A.kept_count) A.kept_count[row] = kept;
}

// The inverse-CDF draw over the working list's kept entries (kept(l, id, w)),
// token-ID order, and the row's outputs.  `unc` carries an earlier
// uncertain decision; closep(l, id) marks an entry whose min-p decision could
// fall either way (status 1 as well).
template <typename Kept, typename Close>
__device__ __forceinline__ void draw_row(const Args& A, Lds& S, Blk& B, const Fw& F, const Cfg& cf, uint32_t row,
                                         const Work& W,
                                         Kept kept, Close closep, double Md, bool unc) {
  const uint32_t t = threadIdx.x, w = wave_(), L = lane_();
  const uint32_t R = (W.n + F.nt - 1u) / F.nt, i0 = min(W.n, t * R), i1 = min(W.n, i0 + R);
  const uint32_t kwords = (A.V + 31u) / 32u;
  uint32_t nk = 0u, n1 = 0u, mink = NONE, close = 0u;
  double mass = 0.0;
  each_range<true>(A, S, row, W, i0, i1, Md, cf.invT, [&](uint32_t, float l, uint32_t id, double wv) {
    if (!(l >= W.thr)) return;
    if (closep(l, id)) close = 1u;
    if (!kept(l, id, wv)) return;
    ++nk;
    n1 += (double)l == Md ? 1u : 0u;
    mink = min(mink, okey(l));
    mass += wv;
    if (A.kept_bits) atomicOr(A.kept_bits + (uint64_t)row * kwords + (id >> 5), 1u << (id & 31u));
  });
  // counts, smallest kept key, the close flag and the mass scan: one barrier
  const uint32_t P = B.p;
  {
    const uint32_t a = wave_sum_u32(nk), b = wave_sum_u32(n1);
    const uint32_t m = ~wave_max_u32(~mink), o = wave_or_u32(close);
    const double inc = wave_scan_f64(mass);
    if (L == 63u) {
      S.xu[P][w] = a;
      S.xu[P][PW + w] = b;
      S.xu[P][2 * PW + w] = m;
      S.xu[P][3 * PW + w] = o;
      S.xd[P][w] = inc;
    }
    if (t == 0) {
      S.bc[5] = NONE;
      S.bc[6] = 0u;
    }
    bar();
    uint32_t nkept = 0u, nones = 0u, mk = NONE, cl = 0u;
    double before = 0.0, Ssum = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < F.nw; ++i) {
      nkept += S.xu[P][i];
      nones += S.xu[P][PW + i];
      mk = min(mk, S.xu[P][2 * PW + i]);
      cl |= S.xu[P][3 * PW + i];
      const double r = S.xd[P][i];
      if (i < w) before += r;
      Ssum += r;
    }
    B.p ^= 1u;
    if (cl) unc = true;
    // sample_categorical's shifted_logit check over the kept set: the
    // smallest kept value has the largest shift
    if (nkept && !isfinite(((double)okey_value(mk) - Md) / cf.T)) {
      if (t == 0) put_row(A, row, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
      return;
    }
    if (A.nodraw) {
      if (t == 0) put_row(A, row, unc ? MXS_ROW_UNCERTIFIED : MXS_ROW_OK, -1, 0.0, nkept);
      return;
    }
    const double target = cf.u * Ssum;
    // every kept weight exactly 1 (ties at the maximum): the sums are small
    // integers on both sides and target is the same product, so the
    // comparisons are exact
    const double E = nones == nkept ? 0.0 : 2.0 * sum_err(Ssum, (double)nkept) + U53 * target;
    double r = before + inc - mass;
    uint32_t hit = NONE, last = NONE, hid = NONE, lid = NONE;
    double hb = 0.0, ha = 0.0;
    float hl = 0.0f, ll = 0.0f;
    each_range<true>(A, S, row, W, i0, i1, Md, cf.invT, [&](uint32_t i, float l, uint32_t id, double wv) {
      if (!(l >= W.thr) || !kept(l, id, wv)) return;
      if (hit == NONE && target < r + wv) { hit = i; hb = r; ha = r + wv; hl = l; hid = id; }
      if (wv > 0.0) { last = i; ll = l; lid = id; }
      r += wv;
    });
    if (hit != NONE) atomicMin(&S.bc[5], hit);
    if (last != NONE) atomicMax(&S.bc[6], last + 1u);
    bar();
    const uint32_t win = S.bc[5], lwin = S.bc[6];
    // the winning entry's thread writes the row; past every running mass
    // (rounding) the last positive-weight entry is taken, uncertified
    if (win != NONE) {
      if (hit == win) {
        const bool cert = target - hb >= E && ha - target > E;
        put_row(A, row, (cert && !unc) ? MXS_ROW_OK : MXS_ROW_UNCERTIFIED, (int32_t)hid,
                ((double)hl - Md) / cf.T - log(Ssum), nkept);
      }
    } else if (lwin != 0u) {
      if (last == lwin - 1u) put_row(A, row, MXS_ROW_UNCERTIFIED, (int32_t)lid, ((double)ll - Md) / cf.T - log(Ssum), nkept);
    } else if (t == 0) {
      put_row(A, row, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u);
    }
  }
}

// Keep-all rows: the draw walks the row's 256-token segment masses, then
// re-derives the crossing segment's weights exactly.
template <typename In>
__device__ __forceinline__ void keepall_segments(const Args& A, Lds& S, Blk& B, const Fw& F, const Cfg& cf, uint32_t row,
                                                 uint32_t Mkey, uint32_t nl) {
  const uint32_t t = threadIdx.x, L = lane_();
  const double Md = (double)okey_value(Mkey);
  const uint32_t nseg = A.C * (uint32_t)NSEG;
  const Seg* sg = A.s.seg + (uint64_t)row * A.s.cm * NSEG;
  // segment s = c NSEG + j PW + w covers chunk c's tokens [4 (j PT + w 64), + 256);
  // thread t sums segments [t R, t R + R)
  const uint32_t R = (nseg + F.nt - 1u) / F.nt, s0 = min(nseg, t * R), s1 = min(nseg, s0 + R);
  auto segmass = [&](uint32_t s) {
    const uint32_t c = s / NSEG, j = (s - c * NSEG) / PW;
    if (j >= A.per) return 0.0;
    const Seg e = sg[s];
    return e.mass > 0.0 ? e.mass * exp_neg(((double)e.ref - Md) * cf.invT) : 0.0;
  };
  double mine = 0.0;
  for (uint32_t s = s0; s < s1; ++s) mine += segmass(s);
  if (t == 0) {
    S.bc[5] = NONE;
    S.bc[6] = 0u;
  }
  double Ssum;
  const double incl = scan_f64(mine, S, B, &Ssum, F.nw);
  const double target = cf.u * Ssum;
  // each weight differs from the reference's by a few ulp (two exp
  // evaluations, two extra roundings); both sides' summation orders
  const double E = (Ssum * (4.0 * (double)nl + 64.0) + 4.0 * (double)nl) * U53 + U53 * target;
  double r = incl - mine;
  uint32_t hs = NONE, ls = NONE;
  double hb = 0.0, lb = 0.0;
  for (uint32_t s = s0; s < s1; ++s) {
    const double m = segmass(s);
    if (hs == NONE && target < r + m) { hs = s; hb = r; }
    if (m > 0.0) { ls = s; lb = r; }
    r += m;
  }
  if (hs != NONE) atomicMin(&S.bc[5], hs);
  if (ls != NONE) atomicMax(&S.bc[6], ls + 1u);
  if (t < 256u) S.u.f.segtab[t] = 0u;
  bar();
  const bool fallback = S.bc[5] == NONE;
  const uint32_t seg = fallback ? S.bc[6] - 1u : S.bc[5];
  if ((!fallback && hs == seg) || (fallback && ls == seg)) S.bd[0] = fallback ? lb : hb;
  bar();
  const double sbefore = S.bd[0];
  const uint32_t c = seg / NSEG, rr = seg - c * NSEG, j = rr / PW, wv = rr - j * PW;
  const uint32_t c0 = c * A.CH, cend = min(c0 + A.CH, A.V);
  const uint32_t sbase = c0 + 4u * (j * PT + wv * 64u);
  for (uint32_t i = t; i < cf.hlen; i += F.nt) {
    const uint32_t id = A.hids[cf.h0 + i];
    if (id - sbase < 256u) atomicAdd(&S.u.f.segtab[id - sbase], 1u);
  }
  bar();
  if (t >= 64u) return;
  const uint32_t g0 = sbase + 4u * L;
  float x[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  uint32_t leg = 0u;
  if (g0 < cend) {
    const In* lrow = (const In*)A.logits + (uint64_t)row * A.stride;
    Quad<In>::unpack(Quad<In>::load(lrow + g0), x);
    const uint32_t tvl = A.masked ? min(A.tv, A.V) : A.V;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t tok = g0 + (uint32_t)i;
      if (tok >= cend) continue;
      const uint32_t cnt = S.u.f.segtab[tok - sbase];
      bool hb2 = false;
      float bv = 0.0f;
      if (cf.blen) {
        uint32_t lo = 0, hi = cf.blen;
        const uint32_t* ids = A.bids + cf.b0;
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (ids[mid] < tok) lo = mid + 1u; else hi = mid;
        }
        if (lo < cf.blen && ids[lo] == tok) { hb2 = true; bv = A.bvals[cf.b0 + lo]; }
      }
      if (cnt || hb2)
        x[i] = bias_and_penalize(x[i], ((hb2 ? 1u : 0u) << 31) | cnt, bv, cf.rep, cf.inv_rep, cf.freq, cf.pres);
      bool lg = tok < tvl;
      if (A.masked) lg = lg && ((A.mask[(uint64_t)row * A.mstride + (tok >> 5)] >> (tok & 31u)) & 1u);
      if (lg) leg |= 1u << i;
    }
  }
  double wq[4], lsum = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wq[i] = ((leg >> i) & 1u) ? exp_neg(((double)x[i] - Md) / cf.T) : 0.0;
    lsum += wq[i];
  }
  double r2 = sbefore + wave_scan_f64(lsum) - lsum;
  uint32_t hit = NONE, lastp = NONE;
  double hb3 = 0.0, ha3 = 0.0;
  float hl = 0.0f, lastl = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if ((leg >> i) & 1u) {
      if (hit == NONE && target < r2 + wq[i]) { hit = g0 + (uint32_t)i; hb3 = r2; ha3 = r2 + wq[i]; hl = x[i]; }
      if (wq[i] > 0.0) { lastp = g0 + (uint32_t)i; lastl = x[i]; }
      r2 += wq[i];
    }
  }
  const uint64_t hm = ballot(hit != NONE), lm = ballot(lastp != NONE);
  uint32_t src = NONE;
  bool fb = fallback;
  if (!fallback && hm) src = (uint32_t)__builtin_ctzll(hm);
  else if (lm) { src = 63u - (uint32_t)__builtin_clzll(lm); fb = true; }
  if (L == src) {
    const uint32_t tok = fb ? lastp : hit;
    const double sft = ((double)(fb ? lastl : hl) - Md) / cf.T;
    // the fallback (target past every running mass) only happens by rounding
    const bool cert = !fb && target - hb3 >= E && ha3 - target > E;
    put_row(A, row, cert ? MXS_ROW_OK : MXS_ROW_UNCERTIFIED, (int32_t)tok, sft - log(Ssum), nl);
  }
  if (src == NONE && L == 0u) put_row(A, row, MXS_ROW_UNCERTIFIED, -1, 0.0, nl);
}

// Rows with a min-p cut: every kept token is a member at or above the cut
// (a prefix of the descending order), so past the top-k mass the decision
// only involves those survivors.  With at most 64 of them, one wave finishes
// the row: lane j holds survivor j (token order), the running mass before
// each in descending order comes from the other lanes, the top-p crossing is
// the lane where it reaches `target` (E = Ea, plus Eb unless the crossing
// sits on the maximum's plateau), and the draw scans the kept lanes.  A
// crossing past every survivor keeps them all.  Returns false (nothing
// written) when there are more than 64 survivors.
template <typename Memb, typename Ok, typename Near>
__device__ __forceinline__ bool minp_tail(const Args& A, Lds& S, Blk& B, const Fw& F, const Cfg& cf, uint32_t row,
                                          const Work& W, Memb member, Ok ok, Near nearp, uint32_t Mkey, double Md,
                                          double target, double Ea, double Eb) {
  const uint32_t t = threadIdx.x, L = lane_();
  const uint32_t R = (W.n + F.nt - 1u) / F.nt, i0 = min(W.n, t * R), i1 = min(W.n, i0 + R);
  uint32_t mine = 0u, near = 0u;
  each_range<false>(A, S, row, W, i0, i1, Md, cf.invT, [&](uint32_t, float l, uint32_t id, double) {
    if (!(l >= W.thr) || !member(l, id)) return;
    if (nearp(l)) near = 1u;
    if (ok(l)) ++mine;
  });
  // survivors (low 16 bits) and near-cut members (high bits) in one scan
  uint32_t tot;
  const uint32_t v = mine | (near << 16);
  const uint32_t p0 = (scan_u32(v, S, B, &tot, F.nw) - v) & 0xffffu;
  const uint32_t n = tot & 0xffffu;
  if (n > 64u) return false;
  uint32_t p = p0;
  each_range<true>(A, S, row, W, i0, i1, Md, cf.invT, [&](uint32_t, float l, uint32_t id, double wv) {
    if (!(l >= W.thr) || !member(l, id) || !ok(l)) return;
    Mem e;
    e.key = okey(l);
    e.id = id;
    e.w = wv;
    S.u.f.mem[p++] = e;
  });
  bar();
  if (t >= 64u) return true;
  Mem me;
  me.key = 0u;
  me.id = NONE;
  me.w = 0.0;
  if (L < n) me = S.u.f.mem[L];
  // the survivors' mass before this one in the reference's descending order
  double bef = 0.0;
  for (uint32_t j = 0; j < n; ++j) {
    const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)j);
    const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)j);
    const double wj = rd_lane(me.w, j);
    if (better(kj, ij, me.key, me.id)) bef += wj;
  }
  bool unc = (tot >> 16) != 0u;
  bool kept;
  const uint64_t hm = ballot(L < n && bef < target && bef + me.w >= target);
  if (hm) {
    const uint32_t c = (uint32_t)__builtin_ctzll(hm);
    const uint32_t ck = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)c);
    const uint32_t ci = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)c);
    const double b2 = rd_lane(bef, c), w2 = rd_lane(me.w, c);
    const double E = Ea + (ck == Mkey ? 0.0 : Eb);
    if (!(target - b2 > E && b2 + w2 - target >= E)) unc = true;
    kept = L < n && !better(ck, ci, me.key, me.id);
  } else {
    // the crossing lies past every survivor: all of them are kept
    const double covered = wave_sum_f64(L < n ? me.w : 0.0);
    if (!(covered < target - (Ea + Eb))) unc = true;
    kept = L < n;
  }
  const float lv = okey_value(me.key);
  const uint64_t km = ballot(kept);
  const uint32_t nkept = (uint32_t)__builtin_popcountll(km);
  const uint32_t nones = (uint32_t)__builtin_popcountll(ballot(kept && (double)lv == Md));
  // sample_categorical's shifted_logit check: the smallest kept value
  const uint32_t mk = ~wave_max_u32(kept ? ~me.key : 0u);
  if (nkept && !isfinite(((double)okey_value(mk) - Md) / cf.T)) {
    if (L == 0u) put_row(A, row, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
    return true;
  }
  if (kept && A.kept_bits) {
    const uint32_t kwords = (A.V + 31u) / 32u;
    atomicOr(A.kept_bits + (uint64_t)row * kwords + (me.id >> 5), 1u << (me.id & 31u));
  }
  if (A.nodraw) {
    if (L == 0u) put_row(A, row, unc ? MXS_ROW_UNCERTIFIED : MXS_ROW_OK, -1, 0.0, nkept);
    return true;
  }
  // the inverse-CDF draw over the kept lanes, token order
  const double wk = kept ? me.w : 0.0;
  const double incl = wave_scan_f64(wk);
  const double Ssum = rd_lane(incl, 63u);
  const double td = cf.u * Ssum;
  const double Ed = nones == nkept ? 0.0 : 2.0 * sum_err(Ssum, (double)nkept) + U53 * td;
  const uint64_t hh = ballot(kept && td < incl);
  if (hh) {
    if (L == (uint32_t)__builtin_ctzll(hh)) {
      const double hb = incl - wk;
      const bool cert = td - hb >= Ed && incl - td > Ed;
      put_row(A, row, (cert && !unc) ? MXS_ROW_OK : MXS_ROW_UNCERTIFIED, (int32_t)me.id,
              ((double)lv - Md) / cf.T - log(Ssum), nkept);
    }
  } else {
    // past every running mass (rounding): the last positive-weight kept lane
    const uint64_t pm = ballot(kept && wk > 0.0);
    if (pm) {
      if (L == 63u - (uint32_t)__builtin_clzll(pm))
        put_row(A, row, MXS_ROW_UNCERTIFIED, (int32_t)me.id, ((double)lv - Md) / cf.T - log(Ssum), nkept);
    } else if (L == 0u) {
      put_row(A, row, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u);
    }
  }
  return true;
}

constexpr uint32_t PD = 4;   // candidate entries each finisher thread prefetches

// The register finisher, for a row with a min-p cut whose candidates all sit
// in the threads' prefetched registers (entry q of thread t: chunk mc, slot
// mo + q SPC).  Top-k rows first find the k-th candidate in the reference's
// descending order (histogram rounds over d = Mkey - key on the entries in
// registers, the final bin of at most 64 ranked on one wave) and the top-k
// mass; then the survivors of the min-p cut (at most 64) go to one wave,
// which takes the top-p crossing among them, the kept set and the draw in
// token order, with the same certification as the general path.  Returns
// false, having written nothing, when a bin of more than 64 equal keys or
// more than 64 survivors needs the general path.
__device__ __forceinline__ bool finish_regs(const Args& A, Lds& S, Blk& B, const Cfg& cf, uint32_t row,
                                            const uint2 (&pre)[PD], uint32_t ev, uint32_t mc, uint32_t mo,
                                            uint32_t SPC, uint32_t myoff, bool kact, uint32_t Mkey, double Md,
                                            float thr, uint32_t N, uint32_t nl, bool complete, double total0,
                                            double terr0) {
  const uint32_t t = threadIdx.x, w = wave_(), L = lane_();
  (void)mc;
  float el[PD];
  uint32_t ek[PD], eid[PD];
  double ew[PD];
  uint32_t cand = 0u;   // bit q: entry q is a candidate (exists and >= thr)
#pragma unroll
  for (uint32_t q = 0; q < PD; ++q) {
    el[q] = __uint_as_float(pre[q].x);
    eid[q] = pre[q].y;
    ek[q] = okey(el[q]);
    ew[q] = 0.0;
    if (((ev >> q) & 1u) && el[q] >= thr) cand |= 1u << q;
  }
  // min-p, as the general path decides it
  const double L_mp = cf.L_mp;
  const double mp_p = L_mp * cf.T;
  const double mp_m = fabs(mp_p) * 0x1p-49 + 1e-300;
  const double mp_c = fabs(mp_p) * 0x1p-47 + 1e-300;
  auto minp_ok = [&](float l) {
    const double y = (double)l - Md;
    if (y >= mp_p + mp_m) return true;
    if (y <= mp_p - mp_m) return false;
    return y / cf.T >= L_mp;
  };
  auto minp_close = [&](float l) {
    if (cf.min_p >= 1.0) return false;
    const double y = (double)l - Md;
    if (fabs(y - mp_p) > mp_c) return false;
    return fabs(y / cf.T - L_mp) <= 4.0 * U53 * fabs(L_mp);
  };
  uint32_t memb = cand;     // the decision's members: the top-k for a top-k row
  bool weighed = false;     // ew[] holds the members' weights
  double target = INFINITY, Ea = 0.0, Eb = 0.0;
  if (kact) {
    // ---- the k-th candidate: histogram rounds, 12 bits of d at a time
    uint32_t need = cf.k, lo = 0u;
    const uint32_t dmax = Mkey - okey(thr);
    int sh = 32 - __builtin_clz(dmax | 1u) - NBB;
    if (sh < 0) sh = 0;
    uint32_t kk = 0u, ki = NONE;
    for (;;) {
#pragma unroll
      for (uint32_t b = 0; b < 4u; ++b) S.u.f.bc[4u * t + b] = 0u;
      if (t == 0) S.bc[0] = NONE;
      bar();
      const uint32_t span = sh >= 32 - NBB ? 0xffffffffu : (((uint32_t)NB << sh) - 1u);
#pragma unroll
      for (uint32_t q = 0; q < PD; ++q) {
        const uint32_t d = Mkey - ek[q];
        if (((cand >> q) & 1u) && d >= lo && d - lo <= span) atomicAdd(&S.u.f.bc[(d - lo) >> sh], 1u);
      }
      bar();
      uint32_t c4[4], csum = 0u;
#pragma unroll
      for (uint32_t b = 0; b < 4u; ++b) {
        c4[b] = S.u.f.bc[4u * t + b];
        csum += c4[b];
      }
      uint32_t tot;
      const uint32_t incl = scan_u32(csum, S, B, &tot, PW);
      if (incl - csum < need && incl >= need) {
        uint32_t r = incl - csum;
#pragma unroll
        for (uint32_t b = 0; b < 4u; ++b) {
          if (r < need && r + c4[b] >= need) {
            S.bc[0] = 4u * t + b;
            S.bc[1] = c4[b];
            S.bc[2] = r;
          }
          r += c4[b];
        }
      }
      bar();
      const uint32_t bstar = S.bc[0];
      if (bstar == NONE) {   // fewer candidates than k: the candidate bound failed
        if (t == 0) put_row(A, row, MXS_ROW_UNCERTIFIED, -1, 0.0, 0u);
        return true;
      }
      const uint32_t bcnt = S.bc[1];
      need -= S.bc[2];
      lo += bstar << sh;
      if (bcnt <= 64u || sh == 0) {
        if (bcnt > 64u) return false;   // more than 64 equal keys
        const uint32_t bspan = sh >= 32 ? 0xffffffffu : ((1u << sh) - 1u);
        uint32_t inb = 0u, nm = 0u;
#pragma unroll
        for (uint32_t q = 0; q < PD; ++q) {
          const uint32_t d = Mkey - ek[q];
          if (((cand >> q) & 1u) && d >= lo && d - lo <= bspan) {
            inb |= 1u << q;
            ++nm;
          }
        }
        uint32_t tot2;
        uint32_t p = scan_u32(nm, S, B, &tot2, PW) - nm;
#pragma unroll
        for (uint32_t q = 0; q < PD; ++q) {
          if ((inb >> q) & 1u) {
            Mem e;
            e.key = ek[q];
            e.id = eid[q];
            e.w = 0.0;
            S.u.f.mem[p++] = e;
          }
        }
        bar();
        if (w == 0u) {
          Mem me;
          me.key = 0u;
          me.id = NONE;
          me.w = 0.0;
          if (L < tot2) me = S.u.f.mem[L];
          uint32_t rank = 0u;
          for (uint32_t j = 0; j < tot2; ++j) {
            const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)j);
            const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)j);
            rank += better(kj, ij, me.key, me.id) ? 1u : 0u;
          }
          if (L < tot2 && rank == need - 1u) {
            S.bc[3] = me.key;
            S.bc[4] = me.id;
          }
        }
        bar();
        kk = S.bc[3];
        ki = S.bc[4];
        break;
      }
      sh = sh > NBB ? sh - NBB : 0;
    }
    // ---- the top-k members and their mass
    memb = 0u;
    double km = 0.0, wmin = 1.0;
#pragma unroll
    for (uint32_t q = 0; q < PD; ++q) {
      if (((cand >> q) & 1u) && (ek[q] > kk || (ek[q] == kk && eid[q] <= ki))) {
        memb |= 1u << q;
        ew[q] = exp_neg(((double)el[q] - Md) * cf.invT);
        km += ew[q];
        wmin = fmin(wmin, ew[q]);
      }
    }
    weighed = true;
    double kept;
    red_sum_minpos_f64(km, wmin, S, B, &kept, &wmin, PW);
    // every top-k token tied at the maximum: kept is exactly k on both sides
    const bool kones = kk == Mkey;
    const double Ekept = kones ? 0.0 : sum_err(kept, (double)cf.k);
    target = cf.top_p * kept;
    Ea = cf.top_p * Ekept + (kones ? 0.0 : U53 * target);
    Eb = Ekept;
  } else if (cf.top_p < 1.0) {
    double total = total0, terr = terr0;
    bool tones = false;
    if (complete) {
      // every legal token is a candidate: the total from the candidates
      double tm = 0.0;
      uint32_t n1 = 0u;
#pragma unroll
      for (uint32_t q = 0; q < PD; ++q) {
        if ((cand >> q) & 1u) {
          ew[q] = exp_neg(((double)el[q] - Md) * cf.invT);
          tm += ew[q];
          n1 += (double)el[q] == Md ? 1u : 0u;
        }
      }
      weighed = true;
      total = red_sum_f64(tm, S, B, PW);
      terr = sum_err(total, (double)nl);
      tones = red_sum_u32(n1, S, B, PW) == nl;   // every weight 1: the total is exactly nl
    }
    target = cf.top_p * total;
    Ea = tones ? 0.0 : cf.top_p * terr + U53 * target;
    Eb = sum_err(total, (double)N);
  }
  // ---- the survivors of the min-p cut, and members within its rounding band
  uint32_t surv = 0u, ns = 0u, near = 0u;
#pragma unroll
  for (uint32_t q = 0; q < PD; ++q) {
    if ((memb >> q) & 1u) {
      if (minp_close(el[q])) near = 1u;
      if (minp_ok(el[q])) {
        surv |= 1u << q;
        ++ns;
        if (!weighed) ew[q] = exp_neg(((double)el[q] - Md) * cf.invT);
      }
    }
  }
  uint32_t tot;
  const uint32_t v = ns | (near << 16);
  uint32_t p = (scan_u32(v, S, B, &tot, PW) - v) & 0xffffu;
  const uint32_t n = tot & 0xffffu;
  if (n > 64u) return false;
#pragma unroll
  for (uint32_t q = 0; q < PD; ++q) {
    if ((surv >> q) & 1u) {
      Mem e;
      e.key = ek[q];
      e.id = eid[q];
      e.w = ew[q];
      S.u.f.mem[p] = e;
      S.u.f.mix[p] = myoff + mo + q * SPC;
      ++p;
    }
  }
  bar();
  if (w != 0u) return true;
  // ---- one wave: lane j holds survivor j
  Mem me;
  me.key = 0u;
  me.id = NONE;
  me.w = 0.0;
  uint32_t mix = NONE;
  if (L < n) {
    me = S.u.f.mem[L];
    mix = S.u.f.mix[L];
  }
  // the mass before each survivor in the descending order, and its place in
  // token order
  double bef = 0.0;
  uint32_t trank = 0u;
  for (uint32_t j = 0; j < n; ++j) {
    const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)j);
    const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)j);
    const uint32_t xj = (uint32_t)__builtin_amdgcn_readlane((int)mix, (int)j);
    const double wj = rd_lane(me.w, j);
    if (better(kj, ij, me.key, me.id)) bef += wj;
    trank += xj < mix ? 1u : 0u;
  }
  bool unc = (tot >> 16) != 0u;
  bool kept;
  const uint64_t hm = ballot(L < n && bef < target && bef + me.w >= target);
  if (hm) {
    const uint32_t c = (uint32_t)__builtin_ctzll(hm);
    const uint32_t ck = (uint32_t)__builtin_amdgcn_readlane((int)me.key, (int)c);
    const uint32_t ci = (uint32_t)__builtin_amdgcn_readlane((int)me.id, (int)c);
    const double b2 = rd_lane(bef, c), w2 = rd_lane(me.w, c);
    const double E = Ea + (ck == Mkey ? 0.0 : Eb);
    if (!(target - b2 > E && b2 + w2 - target >= E)) unc = true;
    kept = L < n && !better(ck, ci, me.key, me.id);
  } else {
    // the crossing lies past every survivor (or there is no top-p): all kept
    const double covered = wave_sum_f64(L < n ? me.w : 0.0);
    if (!(covered < target - (Ea + Eb))) unc = true;
    kept = L < n;
  }
  // to token order
  if (L < n) {
    S.u.f.dmem[trank] = me;
    S.u.f.dkf[trank] = kept ? 1u : 0u;
  }
  bar();   // (this wave alone is left)
  Mem d;
  d.key = 0u;
  d.id = NONE;
  d.w = 0.0;
  bool dk = false;
  if (L < n) {
    d = S.u.f.dmem[L];
    dk = S.u.f.dkf[L] != 0u;
  }
  const float lv = okey_value(d.key);
  const uint32_t nkept = (uint32_t)__builtin_popcountll(ballot(dk));
  const uint32_t nones = (uint32_t)__builtin_popcountll(ballot(dk && (double)lv == Md));
  // sample_categorical's shifted_logit check: the smallest kept value
  const uint32_t mk = ~wave_max_u32(dk ? ~d.key : 0u);
  if (nkept && !isfinite(((double)okey_value(mk) - Md) / cf.T)) {
    if (L == 0u) put_row(A, row, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
    return true;
  }
  if (dk && A.kept_bits) {
    const uint32_t kwords = (A.V + 31u) / 32u;
    atomicOr(A.kept_bits + (uint64_t)row * kwords + (d.id >> 5), 1u << (d.id & 31u));
  }
  if (A.nodraw) {
    if (L == 0u) put_row(A, row, unc ? MXS_ROW_UNCERTIFIED : MXS_ROW_OK, -1, 0.0, nkept);
    return true;
  }
  // the inverse-CDF draw over the kept lanes, token order
  const double wk = dk ? d.w : 0.0;
  const double incl = wave_scan_f64(wk);
  const double Ssum = rd_lane(incl, 63u);
  const double td = cf.u * Ssum;
  const double Ed = nones == nkept ? 0.0 : 2.0 * sum_err(Ssum, (double)nkept) + U53 * td;
  const uint64_t hh = ballot(dk && td < incl);
  if (hh) {
    if (L == (uint32_t)__builtin_ctzll(hh)) {
      const double hb = incl - wk;
      const bool cert = td - hb >= Ed && incl - td > Ed;
      put_row(A, row, (cert && !unc) ? MXS_ROW_OK : MXS_ROW_UNCERTIFIED, (int32_t)d.id,
              ((double)lv - Md) / cf.T - log(Ssum), nkept);
    }
  } else {
    // past every running mass (rounding): the last positive-weight kept lane
    const uint64_t pm = ballot(dk && wk > 0.0);
    if (pm) {
      if (L == 63u - (uint32_t)__builtin_clzll(pm))
        put_row(A, row, MXS_ROW_UNCERTIFIED, (int32_t)d.id, ((double)lv - Md) / cf.T - log(Ssum), nkept);
    } else if (L == 0u) {
      put_row(A, row, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u);
    }
  }
  return true;
}

template <typename In>
__device__ __forceinline__ void finish_row(const Args& A, Lds& S, const Cfg& cf, uint32_t row) {
  const uint32_t t = threadIdx.x, w = wave_(), L = lane_();
  const uint32_t C = A.C;
  Blk B;
  stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 0u);
  // ---- one round trip: each wave's lane c reads chunk c's statistics, and
  // each thread the first entry of its share of a chunk's candidate list
  // (SPC threads per chunk; entries past the chunk's count are ignored)
  Stat s{};
  s.thr = -INFINITY;
  s.minkey = NONE;
  if (L < C) s = A.s.stat[(uint64_t)row * A.s.cm + L];
  // thread t reads chunk mc's entries mo, mo + SPC, ... (PD of them; never
  // past the chunk's CH slots)
  const uint32_t SPC = PT / C;
  const uint32_t mc = t / SPC, mo = t - mc * SPC;
  uint2 pre[PD];
#pragma unroll
  for (uint32_t q = 0; q < PD; ++q) {
    const uint32_t o = mo + q * SPC;
    pre[q] = make_uint2(0u, 0u);
    if (mc < C && o < A.CH) pre[q] = A.s.cand[(uint64_t)row * A.s.cand_stride + (uint64_t)mc * A.CH + o];
  }
  // ---- the header, on every wave
  const uint32_t Mkey = wave_max_u32(s.maxkey);
  const uint32_t mink = ~wave_max_u32(~s.minkey);
  const uint32_t fl = wave_or_u32(s.flags);
  const uint32_t nl = wave_sum_u32(s.nlegal);
  const unsigned long long gk =
      wave_max_u64(s.gkey ? (((unsigned long long)s.gkey << 32) | (unsigned long long)(~s.gid)) : 0ull);
  const uint32_t nc = s.ncand;
  const uint32_t inc = wave_scan_u32(nc);
  const uint32_t coffL = inc - nc;
  const uint32_t N = bcast63(inc);
  const uint32_t thrkey = wave_max_u32(L < C ? okey(s.thr) : 0u);
  const bool complete = wave_or_u32(L < C && s.ncand != s.nlegal ? 1u : 0u) == 0u;
  const double Md = (double)okey_value(Mkey);
  double rm = 0.0, re = 0.0;
  if (L < C && s.maxkey && s.mass > 0.0) {
    // chunk masses rescaled to the row maximum
    const double f = exp_neg(((double)okey_value(s.maxkey) - Md) * cf.invT);
    rm = s.mass * f;
    re = s.mass_err * f + rm * 8.0 * U53;
  }
  const double total0 = wave_sum_f64(rm);
  const double terr0 = wave_sum_f64(re) + total0 * 80.0 * U53;
  const float thr = okey_value(thrkey);
  if (w == 0u) {
    if (L < C) S.coff[L] = coffL;
    if (L == 0u) S.coff[C] = N;
  }
  if (t == 0) {
    A.s.sync[(uint64_t)row * SYNC] = 0u;
    A.s.sync[(uint64_t)row * SYNC + 1u] = 0u;
  }
  int32_t status = MXS_ROW_OK;
  if (fl & F_BADHIST) status = MXS_ROW_INVALID_HISTORY;
  else if (fl & F_BADBIAS) status = MXS_ROW_INVALID_BIAS;
  else if (fl & F_UNIFORM) status = MXS_ROW_INVALID_UNIFORM;
  else if (fl & F_NONFINITE) status = MXS_ROW_NON_FINITE_LOGIT;
  else if (nl == 0u) status = MXS_ROW_EMPTY_SUPPORT;
  if (status != MXS_ROW_OK) {
    if (t == 0) put_row(A, row, status, -1, 0.0, 0u);
    return;
  }
  const uint32_t kwords = (A.V + 31u) / 32u;
  if (cf.greedy) {
    if (t == 0) {
      const uint32_t id = gk ? ~(uint32_t)gk : NONE;
      put_row(A, row, MXS_ROW_OK, (int32_t)id, 0.0, 1u);
      if (A.kept_bits) atomicOr(A.kept_bits + (uint64_t)row * kwords + (id >> 5), 1u << (id & 31u));
    }
    return;
  }
  const bool kact = cf.k > 0u && cf.k < nl;
  // the finisher's width: one wave for a short candidate list
  const Fw Ffull{(uint32_t)PT, (uint32_t)PW, (uint32_t)NB, (uint32_t)NBB, 4u};
  const Fw F = N <= SHORT_LIST ? Fw{64u, 1u, 512u, 9u, 8u} : Ffull;
  if (!kact && cf.top_p >= 1.0 && cf.min_p == 0.0 && !complete) {
    // keep-all without a complete candidate list
    if (A.nodraw) {
      if (t == 0) put_row(A, row, MXS_ROW_OK, -1, 0.0, nl);
      return;
    }
    // the reference's legal_shifted_sum checks every legal token's shifted
    // logit; the smallest overflows first
    if (mink != NONE && !isfinite(((double)okey_value(mink) - Md) / cf.T)) {
      if (t == 0) put_row(A, row, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
      return;
    }
    bar();   // S.coff is written
    keepall_segments<In>(A, S, B, Ffull, cf, row, Mkey, nl);
    return;
  }
  // ---- this thread's prefetched entries: value, id, index in token order
  const uint32_t myn = (uint32_t)__shfl((int)nc, (int)(mc < C ? mc : 0u), 64);
  const uint32_t myoff = (uint32_t)__shfl((int)coffL, (int)(mc < C ? mc : 0u), 64);
  uint32_t ev = 0u;   // bit q: prefetched entry q exists
#pragma unroll
  for (uint32_t q = 0; q < PD; ++q)
    if (mc < C && mo + q * SPC < myn) ev |= 1u << q;
  // every entry of every chunk is in some thread's registers
  const bool all_pre = wave_or_u32(L < C && nc > PD * SPC ? 1u : 0u) == 0u;
  if (all_pre && cf.min_p > 0.0 && (cf.top_p < 1.0 || !kact) &&
      finish_regs(A, S, B, cf, row, pre, ev, mc, mo, SPC, myoff, kact, Mkey, Md, thr, N, nl, complete, total0, terr0))
    return;
  // ---- the working candidate list: in LDS with its weights when it fits
  Work W{N, false, thr};
  uint32_t dmax = Mkey - okey(thr);
  if (N <= NCL) {
    // this thread's chunk offset (lane mc of the wave's scan)
    const uint32_t off = (uint32_t)__shfl((int)coffL, (int)(mc < C ? mc : 0u), 64);
    const uint32_t cnt = (uint32_t)__shfl((int)nc, (int)(mc < C ? mc : 0u), 64);
    // weights now for rows without a top-k; top-k rows weigh their members later
    auto place = [&](uint32_t p, uint2 e) {
      const float l = __uint_as_float(e.x);
      S.u.f.cl[p] = l;
      S.u.f.cid[p] = e.y;
      if (!kact) S.u.f.cw[p] = l >= thr ? exp_neg(((double)l - Md) * cf.invT) : 0.0;
    };
#pragma unroll
    for (uint32_t q = 0; q < PD; ++q)
      if ((ev >> q) & 1u) place(off + mo + q * SPC, pre[q]);
    // entries past each chunk's first PD SPC: every load in flight, then placed
    if (!all_pre) {
      bar();   // S.coff is written
      constexpr uint32_t RMAX = (NCL + PT - 1u) / PT;
      uint2 e[RMAX];
      uint32_t at[RMAX];
#pragma unroll
      for (uint32_t r = 0; r < RMAX; ++r) {
        const uint32_t i = t + r * PT;
        at[r] = NONE;
        e[r] = make_uint2(0u, 0u);
        if (i < N) {
          uint32_t lo = 0, hi = C;   // the last chunk c with coff[c] <= i
          while (hi - lo > 1u) {
            const uint32_t mid = (lo + hi) >> 1;
            if (S.coff[mid] <= i) lo = mid; else hi = mid;
          }
          const uint32_t o = i - S.coff[lo];
          if (o >= PD * SPC) {
            at[r] = i;
            e[r] = A.s.cand[(uint64_t)row * A.s.cand_stride + (uint64_t)lo * A.CH + o];
          }
        }
      }
#pragma unroll
      for (uint32_t r = 0; r < RMAX; ++r)
        if (at[r] != NONE) place(at[r], e[r]);
    }
    bar();
    W = Work{N, true, thr};
    if (w >= F.nw) return;   // the finisher's waves go on alone
  } else {
    bar();   // S.coff is written
    if (w >= F.nw) return;
    if (kact) {
      // stream the global lists once: the bin holding the k-th member bounds it
      int sh = 32 - __builtin_clz(dmax | 1u) - (int)F.nbb;
      if (sh < 0) sh = 0;
      for (uint32_t b = t; b < F.nb; b += F.nt) S.u.f.bc[b] = 0u;
      if (t == 0) S.bc[0] = NONE;
      bar();
      for (uint32_t i = t; i < N; i += F.nt) {
        float l;
        uint32_t id;
        wget(A, S, row, W, i, &l, &id);
        if (l >= thr) atomicAdd(&S.u.f.bc[(Mkey - okey(l)) >> sh], 1u);
      }
      bar();
      uint32_t c4[BPT_MAX], cs = 0u;
#pragma unroll
      for (int q = 0; q < (int)F.bpt; ++q) {
        c4[q] = S.u.f.bc[F.bpt * t + (uint32_t)q];
        cs += c4[q];
      }
      uint32_t tot;
      const uint32_t incs = scan_u32(cs, S, B, &tot, F.nw);
      if (incs - cs < cf.k && incs >= cf.k) {
        uint32_t r = incs - cs;
#pragma unroll
        for (int q = 0; q < (int)F.bpt; ++q) {
          if (r < cf.k && r + c4[q] >= cf.k) { S.bc[0] = F.bpt * t + (uint32_t)q; S.bc[1] = r + c4[q]; }
          r += c4[q];
        }
      }
      bar();
      if (S.bc[0] != NONE && S.bc[1] <= NCL) {
        const uint32_t dlim = ((S.bc[0] + 1u) << sh) - 1u;
        const uint32_t n = compact(A, S, B, F, row, N, [&](float l, uint32_t) { return l >= thr && Mkey - okey(l) <= dlim; },
                                   Md, cf.invT);
        W = Work{n, true, thr};
        dmax = dlim;
      }
    }
  }
  stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 3u);
  bool unc = false;
  const double L_mp = cf.L_mp;
  // min-p: the reference keeps l when (l - M) / T >= ln(min_p) (f64).  The
  // division is taken only within a relative 2^-49 of the boundary
  // y = ln(min_p) T: further out the rounded quotient cannot reach across.
  const double mp_p = L_mp * cf.T;
  const double mp_m = fabs(mp_p) * 0x1p-49 + 1e-300;
  auto minp_ok = [&](float l) {
    if (cf.min_p <= 0.0) return true;
    const double y = (double)l - Md;
    if (y >= mp_p + mp_m) return true;
    if (y <= mp_p - mp_m) return false;
    return y / cf.T >= L_mp;
  };
  // a shifted logit within an ulp of ln(min_p) could fall on either side of
  // the reference's logarithm (only possible within 2^-47 of the boundary)
  const double mp_c = fabs(mp_p) * 0x1p-47 + 1e-300;
  auto minp_close = [&](float l) {
    if (cf.min_p <= 0.0 || cf.min_p >= 1.0) return false;
    const double y = (double)l - Md;
    if (fabs(y - mp_p) > mp_c) return false;
    return fabs(y / cf.T - L_mp) <= 4.0 * U53 * fabs(L_mp);
  };
  if (kact) {
    // ---- top-k: the k-th member, the kept mass, the nucleus cut
    bool f1;
    uint32_t kk, ki;
    double bef, wsf;
    auto all = [&](float, uint32_t) { return true; };
    crossing<false>(A, S, B, F, row, W, all, Mkey, Md, cf.invT, dmax, (double)cf.k, &f1, &kk, &ki, &bef, &wsf);
    stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 4u);
    if (!f1) {   // fewer candidates than k: the candidate bound failed
      if (t == 0) put_row(A, row, MXS_ROW_UNCERTIFIED, -1, 0.0, 0u);
      return;
    }
    auto inK = [&](float l, uint32_t id) {
      const uint32_t key = okey(l);
      return key > kk || (key == kk && id <= ki);
    };
    // a long list shrinks to the top-k members before the passes below
    if (W.lds && F.nt == (uint32_t)PT && W.n > 2u * cf.k && W.n > SHORT_LIST) {
      W.n = compact_lds(S, B, F, W, inK);
      dmax = Mkey - kk;
    }
    // the top-k members' weights (an LDS list caches them for the passes below)
    double km = 0.0, wmin = 1.0;
    each<false>(A, S, row, W, F, Md, cf.invT, [&](uint32_t i, float l, uint32_t id, double) {
      if (l >= W.thr && inK(l, id)) {
        const double wv = exp_neg(((double)l - Md) * cf.invT);
        if (W.lds) S.u.f.cw[i] = wv;
        km += wv;
        wmin = fmin(wmin, wv);
      }
    });
    double kept;
    red_sum_minpos_f64(km, wmin, S, B, &kept, &wmin, F.nw);
    stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 5u);
    // every top-k token tied at the maximum: kept is exactly k on both sides
    const bool kones = kk == Mkey;
    const double Ekept = kones ? 0.0 : sum_err(kept, (double)cf.k);
    if (cf.min_p > 0.0 && cf.top_p < 1.0 && W.lds) {
      const double target = cf.top_p * kept;
      if (minp_tail(A, S, B, F, cf, row, W, inK, minp_ok, minp_close, Mkey, Md, target,
                    cf.top_p * Ekept + (kones ? 0.0 : U53 * target), Ekept))
        return;
    }
    uint32_t ck = kk, ci = ki;
    double habs = -1.0, hlo = 0.0, hhi = 0.0;   // top_p = 1: weights at or below habs are absorbed
    if (cf.top_p < 1.0) {
      const double target = cf.top_p * kept;
      bool f2;
      double b2, w2;
      crossing<true>(A, S, B, F, row, W, inK, Mkey, Md, cf.invT, dmax, target, &f2, &ck, &ci, &b2, &w2);
      stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 6u);
      // running masses inside the maximum's plateau are exact integers
      const double Ec = ck == Mkey ? 0.0 : Ekept;
      const double E = cf.top_p * Ekept + Ec + (kones ? 0.0 : U53 * target);
      if (!f2) {
        // covered never reaches the target: every top-k token is kept
        ck = kk;
        ci = ki;
        if (!(b2 < target - E)) unc = true;
      } else if (!(target - b2 > E && b2 + w2 - target >= E)) {
        unc = true;
      }
    } else {
      // top_p = 1: the reference stops at the first running mass equal to
      // kept, i.e. before the first weight that adding to kept no longer
      // changes (at or below half an ulp of kept; weights descend)
      int e2;
      (void)frexp(kept, &e2);                 // kept in [2^(e2-1), 2^e2)
      const double h = ldexp(1.0, e2 - 54);   // half an ulp of kept
      // the reference's kept may sit in the neighbouring binade when ours is
      // within its error of a power of two: its half ulp is then h/2 or 2h
      hlo = kept - ldexp(1.0, e2 - 1) <= Ekept ? 0.5 * h : h;
      hhi = ldexp(1.0, e2) - kept <= Ekept ? 2.0 * h : h;
      if (!(wmin > hhi * (1.0 + 4.0 * U53))) habs = h;
    }
    auto keptf = [&](float l, uint32_t id, double wv) {
      const uint32_t key = okey(l);
      if (!(key > ck || (key == ck && id <= ci))) return false;
      if (habs >= 0.0 && !(wv > habs)) return false;
      return minp_ok(l);
    };
    if (habs >= 0.0) {
      // a weight within its rounding of habs could fall on either side
      uint32_t close = 0u;
      each<true>(A, S, row, W, F, Md, cf.invT, [&](uint32_t, float l, uint32_t id, double wv) {
        if (l >= W.thr && inK(l, id) && wv >= hlo * (1.0 - 4.0 * U53) && wv <= hhi * (1.0 + 4.0 * U53)) close = 1u;
      });
      if (red_or_u32(close, S, B, F.nw)) unc = true;
    }
    stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 7u);
    draw_row(A, S, B, F, cf, row, W, keptf, [&](float l, uint32_t id) { return inK(l, id) && minp_close(l); }, Md, unc);
    return;
  }
  // ---- no top-k: nucleus (top_p < 1), min-p only, or keep-all (complete list)
  auto all = [&](float, uint32_t) { return true; };
  bool reached = true;
  uint32_t ck = 0u, ci = NONE;
  if (cf.top_p < 1.0) {
    double total = total0, terr = terr0;
    bool tones = false;
    if (complete) {
      // every legal token is a candidate: the total from the candidates
      double tm = 0.0;
      uint32_t n1 = 0u;
      each<true>(A, S, row, W, F, Md, cf.invT, [&](uint32_t, float l, uint32_t, double wv) {
        if (l >= W.thr) {
          tm += wv;
          n1 += (double)l == Md ? 1u : 0u;
        }
      });
      total = red_sum_f64(tm, S, B, F.nw);
      terr = sum_err(total, (double)nl);
      tones = red_sum_u32(n1, S, B, F.nw) == nl;   // every weight 1: the total is exactly nl
    }
    const double target = cf.top_p * total;
    if (cf.min_p > 0.0 && W.lds &&
        minp_tail(A, S, B, F, cf, row, W, all, minp_ok, minp_close, Mkey, Md, target,
                  tones ? 0.0 : cf.top_p * terr + U53 * target, sum_err(total, (double)N)))
      return;
    bool f2;
    double b2, w2;
    stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 5u);
    crossing<true>(A, S, B, F, row, W, all, Mkey, Md, cf.invT, dmax, target, &f2, &ck, &ci, &b2, &w2);
    stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 6u);
    // running masses inside the maximum's plateau are exact integers; a
    // complete list tied at the maximum has an exact total
    const double E = (tones ? 0.0 : cf.top_p * terr + U53 * target) + (ck == Mkey ? 0.0 : sum_err(total, (double)N));
    if (!f2) {
      // the candidates' whole mass stays below the target: the kept set is
      // the min-p set (or, for a complete list, every token)
      reached = false;
      if (!(b2 < target - E)) unc = true;
      if (!complete && cf.min_p <= 0.0) unc = true;
    } else if (!(target - b2 > E && b2 + w2 - target >= E)) {
      unc = true;
    }
  }
  if (cf.top_p >= 1.0 && cf.min_p > 0.0 && W.lds &&
      minp_tail(A, S, B, F, cf, row, W, all, minp_ok, minp_close, Mkey, Md, INFINITY, 0.0, 0.0))
    return;
  const bool cut = cf.top_p < 1.0 && reached;
  auto keptf = [&](float l, uint32_t id, double) {
    if (cut) {
      const uint32_t key = okey(l);
      if (!(key > ck || (key == ck && id <= ci))) return false;
    }
    return minp_ok(l);
  };
  stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 7u);
  draw_row(A, S, B, F, cf, row, W, keptf, [&](float l, uint32_t) { return minp_close(l); }, Md, unc);
}

// ===========================================================================
// The chunk pass.
// ===========================================================================
// What the quad loop accumulates besides the maximum: the two largest
// values (top-k rows with 128 < k <= 1024) or the online f32 mass (top-p
// rows without a top-k).
enum : int { M_PLAIN = 0, M_TOP2 = 1, M_MASS = 2 };

__device__ __forceinline__ float vmin(float a, float b) {
  float r;
  __asm__("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

template <typename In>
__global__ __launch_bounds__(PT) void pick_kernel(Args A) {
  __shared__ Lds S;
  using Q = Quad<In>;
  Blk Bc;
  const uint32_t t = threadIdx.x, w = wave_(), L = lane_();
  // XCD-aware mapping: workgroup g runs on XCD g mod 8; a row's chunks share
  // one XCD (and its L2), rows r = 8 ri + ((x - ri) mod 8)
  const uint32_t g = blockIdx.x, xcd = g & 7u, slot = g >> 3;
  const uint32_t ri = slot / A.C, c = slot - ri * A.C;
  const uint32_t row = 8u * ri + ((xcd - ri) & 7u);
  if (row >= A.rows) return;
  const uint32_t V = A.V, c0 = c * A.CH;
  const uint32_t ntok = min(A.CH, V - c0);
  const uint32_t nq = (ntok + 3u) / 4u;

  // ---- loads.  The side inputs (history ids, the bias list, mask words)
  // go out first, so they land ahead of the chunk's stream and the LDS
  // tables are ready while most of the stream is still in flight; then
  // every quad round of the logits.
  const uint32_t h0 = A.hoff[row], hlen = A.hoff[row + 1] - h0;
  const uint32_t b0 = A.boff[row], blen = A.boff[row + 1] - b0;
  constexpr uint32_t HR = 2;
  uint32_t hreg[HR];
  const uint32_t hfirst = min(hlen, HR * (uint32_t)PT);
#pragma unroll
  for (uint32_t r = 0; r < HR; ++r) {
    const uint32_t i = t + r * PT;
    hreg[r] = i < hfirst ? A.hids[h0 + i] : 0u;
  }
  uint32_t bid0 = 0u, bprev = 0u;
  float bval0 = 0.0f;
  if (blen > 0u && blen <= BCAP && t < blen) {
    bid0 = A.bids[b0 + t];
    bval0 = A.bvals[b0 + t];
    if (t > 0) bprev = A.bids[b0 + t - 1u];
  }
  const uint32_t nmw = (ntok + 31u) / 32u;
  uint32_t mw0 = 0xffffffffu, mw1 = 0xffffffffu;
  if (A.masked) {
    const uint32_t* mrow = A.mask + (uint64_t)row * A.mstride + (c0 >> 5);
    if (t < nmw) mw0 = mrow[t];
    if (t + PT < nmw) mw1 = mrow[t + PT];
  }
  __asm__ volatile("" ::: "memory");
  typename Q::Raw raw[QMAX];
  const In* lrow = (const In*)A.logits + (uint64_t)row * A.stride + c0;
#pragma unroll
  for (int j = 0; j < QMAX; ++j) {
    const uint32_t q = (uint32_t)j * PT + t;
    if (j < (int)A.per && q < nq) raw[j] = Q::load(lrow + 4u * q);
    else raw[j] = typename Q::Raw{};
  }
  __asm__ volatile("" ::: "memory");
  Cfg cf = load_cfg(A, row);
  stamp(A, row, c, 0u);
  if (cf.err) {
    if (c == 0 && t == 0) put_row(A, row, cf.err, -1, 0.0, 0u);
    return;
  }
  const bool greedy = cf.greedy;
  const uint32_t k = cf.k;
  const bool kknown = !greedy && !A.masked && k > 0u && k < V;
  const bool kmaybe = !greedy && A.masked && k > 0u;
  const bool keepall_possible = !greedy && !kknown && cf.top_p >= 1.0 && cf.min_p == 0.0;
  const bool need_seg = keepall_possible && !A.nodraw && !kmaybe;
  const bool need_mass = !greedy && !kknown && cf.top_p < 1.0;
  // top-k bound from each thread's largest value (k <= 128), two largest
  // (k <= 1024) or every value
  const uint32_t topr = (kknown || kmaybe) ? (k <= 128u ? 1u : (k <= 1024u ? 2u : 40u)) : 0u;
  const int mode = need_mass ? M_MASS : (topr == 2u ? M_TOP2 : M_PLAIN);
  const bool has_hist = hlen > 0u, has_bias = blen > 0u;
  const bool long_hist = hlen > HTAB_MAX;
  const bool use_tab = has_hist || has_bias;

  // ---- LDS: count table, mask words, bias list
  if (use_tab)
    for (uint32_t q = t; q < nq; q += PT) *reinterpret_cast<uint2*>(&S.u.c.ctab[2u * q]) = make_uint2(0u, 0u);
  uint32_t* gt = A.s.gtab + (uint64_t)row * A.s.gtab_stride + c0;
  if (long_hist) {
    // counts past 15 bits: u32 counts in global scratch, LDS marks presence
    for (uint32_t q = t; q < nq; q += PT) *reinterpret_cast<uint4*>(gt + 4u * q) = make_uint4(0u, 0u, 0u, 0u);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // the logarithms the thresholds and the finisher use
  cf.L_mp = uni(cf.min_p > 0.0 ? log(cf.min_p) : -INFINITY);
  cf.L_nuc = uni((cf.top_p < 1.0 && 1.0 - cf.top_p > 8.0 * (double)V * U53)
                     ? log((1.0 - cf.top_p) / (2.0 * (double)V))
                     : -INFINITY);
  bar();
  if (A.masked) {
    if (t < nmw) S.u.c.mask[t] = mw0;
    if (t + PT < nmw) S.u.c.mask[t + PT] = mw1;
  }
  if (has_bias && blen <= BCAP && t < blen) {
    S.u.c.bid[t] = bid0;
    S.u.c.bval[t] = bval0;
  }
  uint32_t flags = cf.uerr ? F_UNIFORM : 0u;
  const uint32_t span = nq * 4u;
  auto scat = [&](uint32_t id) {
    if (id >= V) { flags |= F_BADHIST; return; }
    const uint32_t r = id - c0;
    if (r < span) {
      if (long_hist) {
        atomicOr(&S.u.c.ctab[r >> 1], 1u << (16u * (r & 1u)));
        atomicAdd(gt + r, 1u);
      } else {
        atomicAdd(&S.u.c.ctab[r >> 1], 1u << (16u * (r & 1u)));
      }
    }
  };
  if (has_hist) {
#pragma unroll
    for (uint32_t r = 0; r < HR; ++r)
      if (t + r * PT < hfirst) scat(hreg[r]);
    for (uint32_t i = HR * PT + t; i < hlen; i += PT) scat(A.hids[h0 + i]);
  }
  if (has_bias) {
    auto mark = [&](uint32_t id, float v, bool bad) {
      if (bad || id >= V || !isfinite(v)) { flags |= F_BADBIAS; return; }
      const uint32_t r = id - c0;
      if (r < span) atomicOr(&S.u.c.ctab[r >> 1], 0x8000u << (16u * (r & 1u)));
    };
    if (blen <= BCAP) {
      if (t < blen) mark(bid0, bval0, t > 0 && bprev >= bid0);
    } else {
      for (uint32_t i = t; i < blen; i += PT) {
        const uint32_t id = A.bids[b0 + i];
        mark(id, A.bvals[b0 + i], i > 0 && A.bids[b0 + i - 1u] >= id);
      }
    }
  }
  if (long_hist) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  }
  bar();
  stamp(A, row, c, 1u);

  // ---- the quad loop, as the stream lands: bias and penalties for the
  // listed tokens, the grammar mask, the finite check, the maximum and (by
  // mode) the two largest values or the online f32 mass
  const uint32_t tvl = A.masked ? min(A.tv, V) : V;
  // x: the adjusted values (for f32, the loaded registers themselves).  After
  // the loop, a token outside the chunk, past V or illegal under the mask
  // holds -inf, so later passes read x alone.
  float x[QMAX][4];
  uint32_t lg0 = 0u, lg1 = 0u, nleg = 0u;
  float tmax = -INFINITY, t1 = -INFINITY;
  float nfa = 0.0f;   // sum of x * 0 over the in-range values: NaN iff one is not finite
  const float c32 = need_mass ? (float)(LOG2E * cf.invT) : 0.0f;
  float ms = 0.0f, meb = 0.0f, mex = 0.0f, mref = -INFINITY;
  uint32_t mn = 0u;
  const uint32_t kwords = (V + 31u) / 32u;
  // tokens of quad round j this thread holds that lie in the chunk and below V
  auto in_range = [&](int j) -> uint32_t {
    const uint32_t q = (uint32_t)j * PT + t;
    const uint32_t g0 = c0 + 4u * q;
    if (q >= nq) return 0u;
    return g0 + 4u <= V ? 0xfu : ((1u << (V - g0)) - 1u);
  };
  // bias and penalties of listed token `tok` (table entry f != 0)
  auto adjust = [&](float v, uint32_t f, uint32_t tok) {
    uint32_t cnt = f & 0x7fffu;
    if (long_hist && cnt) cnt = __hip_atomic_load(gt + (tok - c0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t hb = f >> 15;
    float bv = 0.0f;
    if (hb) bv = bias_of(A, cf, S, tok);
    return bias_and_penalize(v, (hb << 31) | cnt, bv, cf.rep, cf.inv_rep, cf.freq, cf.pres);
  };
  // the online f32 mass of one quad's legal values (leg), whose maximum is qm
  auto mass_quad = [&](int j, float qm, uint32_t leg) {
    if (qm > mref) {
      if (mref > -INFINITY) {
        // rescale to the new reference; its own error joins the bound
        const float y = (mref - qm) * c32;
        const float f = __builtin_amdgcn_exp2f(y);
        mex = mex * f + ms * f * (-2.1f * y * U24 + 6.0f * U24);
        ms *= f;
        meb *= f;
      }
      mref = qm;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if ((leg >> i) & 1u) {
        const float y = (x[j][i] - mref) * c32;
        const float ev = __builtin_amdgcn_exp2f(y);
        ms += ev;
        meb = fmaf(ev, -y, meb);
        ++mn;
      }
    }
  };
  // the penalties alone (no bias entry, count in 15 bits): bias_and_penalize
  // for that case
  auto penalize = [&](float v, uint32_t cnt) {
    const float r = v < 0.0f ? v * cf.rep : div_by_recip(v, cf.inv_rep);
    const float fq = (float)cnt * cf.freq;
    return (r - fq) - cf.pres;
  };
  // the listed tokens of a quad in any case: one slot per pass, every pass
  // running the whole bias-and-penalty stage (the lanes of a wave rarely
  // hold more than one listed token of a round)
  auto adjust_quad = [&](int j, uint2 e, uint32_t rng, uint32_t g0) {
    uint32_t pend = (((e.x & 0xffffu) != 0u) ? 1u : 0u) | (((e.x >> 16) != 0u) ? 2u : 0u) |
                    (((e.y & 0xffffu) != 0u) ? 4u : 0u) | (((e.y >> 16) != 0u) ? 8u : 0u);
    pend &= rng;
    while (pend) {
      const uint32_t i = (uint32_t)__builtin_ctz(pend);
      pend &= pend - 1u;
      const uint32_t f = (((i & 2u) ? e.y : e.x) >> (16u * (i & 1u))) & 0xffffu;
      const float v = (i & 2u) ? ((i & 1u) ? x[j][3] : x[j][2]) : ((i & 1u) ? x[j][1] : x[j][0]);
      const float nv = adjust(v, f, g0 + i);
      x[j][0] = i == 0u ? nv : x[j][0];
      x[j][1] = i == 1u ? nv : x[j][1];
      x[j][2] = i == 2u ? nv : x[j][2];
      x[j][3] = i == 3u ? nv : x[j][3];
    }
  };
  // rows without a grammar mask whose listed tokens are history entries
  // only, counted in LDS
  const bool fast = !A.masked && blen == 0u && !long_hist;
  // full rounds: every lane's quad complete and below V
  const uint32_t nfull = (ntok / 4u) / (uint32_t)PT;
#pragma unroll
  for (int j = 0; j < QMAX; ++j) {
    Q::unpack(raw[j], x[j]);
    if (j < (int)A.per) {
      const uint32_t q = (uint32_t)j * PT + t;
      const uint32_t g0 = c0 + 4u * q;
      if (fast && (uint32_t)j < nfull) {
        // a full round without a grammar mask or bias list: every token in
        // range and legal
        if (use_tab) {
          const uint2 e = *reinterpret_cast<const uint2*>(&S.u.c.ctab[2u * q]);
          if (ballot((e.x | e.y) != 0u)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t f = ((i < 2 ? e.x : e.y) >> (16 * (i & 1))) & 0xffffu;
              if (ballot(f != 0u) && f) x[j][i] = penalize(x[j][i], f);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) nfa = fmaf(x[j][i], 0.0f, nfa);
        nleg += 4u;
        if (mode == M_TOP2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float b = vmin(tmax, x[j][i]);
            tmax = vmax(tmax, x[j][i]);
            t1 = vmax(t1, b);
          }
        } else if (mode == M_MASS) {
          const float qm = vmax3(x[j][0], x[j][1], vmax(x[j][2], x[j][3]));
          tmax = vmax(tmax, qm);
          mass_quad(j, qm, 0xfu);
        } else {
          tmax = vmax3(tmax, x[j][0], x[j][1]);
          tmax = vmax3(tmax, x[j][2], x[j][3]);
        }
      } else {
        // the chunk's last partial round, a grammar-masked row, or a row
        // with a bias list or a long history
        const uint32_t rng = in_range(j);
        if (use_tab) {
          const uint2 e = rng ? *reinterpret_cast<const uint2*>(&S.u.c.ctab[2u * q]) : make_uint2(0u, 0u);
          if (ballot((e.x | e.y) != 0u)) adjust_quad(j, e, rng, g0);
        }
        uint32_t leg = rng;
        if (A.masked) {
          leg &= (S.u.c.mask[q >> 3] >> ((q & 7u) * 4u)) & 0xfu;
          if (g0 + 4u > tvl) leg &= g0 >= tvl ? 0u : ((1u << (tvl - g0)) - 1u);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if ((rng >> i) & 1u) nfa = fmaf(x[j][i], 0.0f, nfa);
        if (j < 8) lg0 |= leg << (4 * j); else lg1 |= leg << (4 * (j - 8));
        nleg += popc(leg);
        float v4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = ((leg >> i) & 1u) ? x[j][i] : -INFINITY;
        const float qm = vmax3(v4[0], v4[1], vmax(v4[2], v4[3]));
        if (mode == M_TOP2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float b = vmin(tmax, v4[i]);
            tmax = vmax(tmax, v4[i]);
            t1 = vmax(t1, b);
          }
        } else {
          tmax = vmax(tmax, qm);
        }
        if (mode == M_MASS && qm > -INFINITY) mass_quad(j, qm, leg);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const uint32_t nfin = nfa == 0.0f ? 0u : 1u;
  stamp(A, row, c, 2u);

  // the adjusted logits (debug output), from the registers
  if (A.adjusted) {
#pragma unroll
    for (int j = 0; j < QMAX; ++j) {
      if (j < (int)A.per) {
        const uint32_t rng = in_range(j);
        float* ap = A.adjusted + (uint64_t)row * V + c0 + 4u * ((uint32_t)j * PT + t);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if ((rng >> i) & 1u) ap[i] = x[j][i];
      }
    }
  }
  // from here on x alone tells legality: every other slot becomes -inf
#pragma unroll
  for (int j = 0; j < QMAX; ++j) {
    if (j < (int)A.per && (A.masked || (uint32_t)j >= nfull)) {
      const uint32_t leg = ((j < 8 ? lg0 : lg1) >> (4 * (j & 7))) & 0xfu;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[j][i] = ((leg >> i) & 1u) ? x[j][i] : -INFINITY;
    } else if (j >= (int)A.per) {
#pragma unroll
      for (int i = 0; i < 4; ++i) x[j][i] = -INFINITY;
    }
  }
  // greedy: IEEE argmax, lowest id on ties (-0 ties +0)
  float gv = -INFINITY;
  uint32_t gi = NONE;
  if (greedy) {
#pragma unroll
    for (int j = 0; j < QMAX; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (x[j][i] > gv) {
          gv = x[j][i];
          gi = c0 + 4u * ((uint32_t)j * PT + t) + (uint32_t)i;
        }
  }
  // keep-all rows: f64 mass of each 256-token segment (wave w, round j)
  float tmin = INFINITY;
  if (need_seg) {
    Seg* segp = A.s.seg + ((uint64_t)row * A.s.cm + c) * NSEG;
#pragma unroll
    for (int j = 0; j < QMAX; ++j) {
      if (j < (int)A.per) {
        const float qm = vmax3(x[j][0], x[j][1], vmax(x[j][2], x[j][3]));
        const uint32_t wk = wave_max_u32(qm > -INFINITY ? okey(qm) : 0u);
        double sm = 0.0;
        float ref = -INFINITY;
        if (wk) {
          ref = okey_value(wk);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (x[j][i] > -INFINITY) {
              sm += seg_w(x[j][i], ref, cf.invT);
              tmin = fminf(tmin, x[j][i]);
            }
        }
        sm = wave_sum_f64(sm);
        if (L == 0u) {
          Seg e;
          e.ref = ref;
          e.pad = 0u;
          e.mass = wk ? sm : 0.0;
          segp[(uint32_t)j * PW + w] = e;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // kept bits: keep-all rows (the legal set, unless a top-k may apply) write
  // the chunk's legal words; every other row clears them for the finisher
  if (A.kept_bits) {
    uint32_t* kb = A.kept_bits + (uint64_t)row * kwords + (c0 >> 5);
    const bool legal_bits = keepall_possible && !kmaybe;
    for (uint32_t i = t; i < nmw; i += PT) {
      uint32_t bits = 0u;
      if (legal_bits) {
        const uint32_t tok0 = c0 + 32u * i;
        bits = A.masked ? S.u.c.mask[i] : 0xffffffffu;
        if (tok0 + 32u > tvl) bits &= tok0 >= tvl ? 0u : ((1u << (tvl - tok0)) - 1u);
      }
      kb[i] = bits;
    }
  }
  stamp(A, row, c, 4u);

  // ---- chunk reductions
  {
    const uint32_t wk = wave_max_u32(tmax > -INFINITY ? okey(tmax) : 0u);
    const uint32_t wmin = ~wave_max_u32(tmin < INFINITY ? ~okey(tmin) : 0u);
    const uint32_t wf = wave_or_u32(flags | (nfin ? F_NONFINITE : 0u));
    const uint32_t wl = wave_sum_u32(nleg);
    if (L == 0u) {
      S.wr[w] = wk;
      S.wr[PW + w] = wf;
      S.wr[2 * PW + w] = wl;
      S.wr[3 * PW + w] = wmin;
    }
    if (greedy) {
      const unsigned long long gk = wave_max_u64(
          gi != NONE ? (((unsigned long long)okey(gv == 0.0f ? 0.0f : gv) << 32) | (unsigned long long)(~gi)) : 0ull);
      if (L == 0u) S.wg[w] = gk;
    }
  }
  bar();   // (also: every wave is done with the count table, whose LDS the histogram reuses)
  // the chunk maximum and legal count now; flags, minimum and greedy key
  // only where the statistics are written
  uint32_t Mkey = 0u, nl_c = 0u;
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    Mkey = max(Mkey, S.wr[i]);
    nl_c += S.wr[2 * PW + i];
  }
  Mkey = uni(Mkey);
  nl_c = uni(nl_c);
  const float Mc = okey_value(Mkey);
  const bool want_hist = topr > 0u && topr <= 40u;
  const bool k_here = kknown || (kmaybe && nl_c > k);
  const bool hist_now = want_hist && k_here && Mkey;
  // rows whose threshold rests on the row maximum publish the chunk's and
  // read back the best seen so far
  const bool need_rowmax = !greedy && Mkey && !k_here && !kmaybe && !keepall_possible &&
                           !(A.masked && nl_c <= 4096u) && (cf.min_p > 0.0 || cf.L_nuc > -INFINITY);
  if (hist_now)
    for (uint32_t b = t; b < (uint32_t)NB; b += PT) S.u.hist[b] = 0u;
  if (need_rowmax && t == 0)
    S.bc[0] = max(__hip_atomic_fetch_max(A.s.sync + (uint64_t)row * SYNC + 1u, Mkey, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT),
                  Mkey);
  bar();
  // top-k bound: a value grid of 1/64 logit below the chunk maximum
  uint32_t bstar = NONE;
  if (hist_now) {
    auto add = [&](float y) {
      const float d = (Mc - y) * 64.0f;
      if (d < (float)NB) atomicAdd(&S.u.hist[(uint32_t)d], 1u);
    };
    if (topr == 1u) {
      if (tmax > -INFINITY) add(tmax);
    } else if (topr == 2u) {
      if (tmax > -INFINITY) add(tmax);
      if (t1 > -INFINITY) add(t1);
    } else {
#pragma unroll
      for (int j = 0; j < QMAX; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (x[j][i] > -INFINITY) add(x[j][i]);
    }
    bar();
    uint32_t h4[4];
    uint32_t hs = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      h4[q] = S.u.hist[4u * t + (uint32_t)q];
      hs += h4[q];
    }
    uint32_t tot;
    const uint32_t inc = scan_u32(hs, S, Bc, &tot, PW);
    if (inc - hs < k && inc >= k) {
      uint32_t r = inc - hs;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (r < k && r + h4[q] >= k) S.bc[1] = 4u * t + (uint32_t)q;
        r += h4[q];
      }
    } else if (t == PT - 1u && inc < k) {
      S.bc[1] = NONE;   // fewer than k values on the grid
    }
    bar();
    bstar = S.bc[1];
  }
  // ---- the candidate threshold: a proven lower bound of every token the
  // row's decision can need
  float thr = greedy ? INFINITY : -INFINITY;   // a chunk without legal tokens bounds nothing
  if (!greedy && Mkey) {
    if (k_here) {
      thr = -INFINITY;
      if (bstar != NONE) {
        const float lim = Mc - (float)(bstar + 1u) * (1.0f / 64.0f);
        thr = lim - (fabsf(Mc) + 32.0f) * 4.0f * U24;
      }
    } else if (kmaybe || (A.masked && nl_c <= 4096u && !keepall_possible)) {
      // at most k legal tokens here (or few under a grammar mask): all of
      // them, so the finisher sees the complete legal set
      thr = -INFINITY;
    } else if (keepall_possible) {
      thr = INFINITY;      // keep-all: segment masses, no candidates
    } else if (need_rowmax) {
      const float Mb = okey_value(S.bc[0]);   // best row maximum seen (>= Mc)
      double lim = -INFINITY;
      if (cf.min_p > 0.0) lim = fmax(lim, (double)Mb + cf.T * cf.L_mp);
      if (cf.L_nuc > -INFINITY) lim = fmax(lim, (double)Mb + cf.T * cf.L_nuc);
      const float lf = (float)lim;
      thr = lf - (fabsf(lf) + fabsf(Mb)) * 1e-6f - 1e-37f;
      if (!(thr > -INFINITY)) thr = -INFINITY;
    }
  }
  stamp(A, row, c, 5u);

  // ---- candidate emission in token-ID order: (quad round, wave, lane,
  // token).  Candidates are the values >= thr (-inf excluded); the four
  // slots' wave masks give each (round, wave) segment's count, then each
  // lane's place in it.
  uint32_t ncand = 0u;
  if (thr < INFINITY) {
    const float te = fmaxf(thr, -3.402823466e38f);
#pragma unroll
    for (int j = 0; j < QMAX; ++j) {
      if (j < (int)A.per) {
        const uint64_t m0 = ballot(x[j][0] >= te), m1 = ballot(x[j][1] >= te);
        const uint64_t m2 = ballot(x[j][2] >= te), m3 = ballot(x[j][3] >= te);
        const uint32_t cnt = (uint32_t)(__builtin_popcountll(m0) + __builtin_popcountll(m1) +
                                        __builtin_popcountll(m2) + __builtin_popcountll(m3));
        if (L == 0u) S.wcnt[(uint32_t)j * PW + w] = cnt;
      }
    }
    bar();
    if (w == 0u) {
      // (quad round, wave) counts in order, QMAX * PW of them over 64 lanes
      const uint32_t ne = A.per * (uint32_t)PW;
      constexpr uint32_t PER_LANE = (QMAX * PW + 63) / 64;
      uint32_t a[PER_LANE], sum = 0u;
#pragma unroll
      for (uint32_t r = 0; r < PER_LANE; ++r) {
        const uint32_t i = PER_LANE * L + r;
        a[r] = i < ne ? S.wcnt[i] : 0u;
        sum += a[r];
      }
      const uint32_t inc = wave_scan_u32(sum);
      uint32_t off = inc - sum;
#pragma unroll
      for (uint32_t r = 0; r < PER_LANE; ++r) {
        const uint32_t i = PER_LANE * L + r;
        if (i < ne) S.woff[i] = off;
        off += a[r];
      }
      if (L == 63u) S.bc[2] = inc;
    }
    bar();
    ncand = S.bc[2];
    uint2* cb = A.s.cand + (uint64_t)row * A.s.cand_stride + (uint64_t)c * A.CH;
#pragma unroll
    for (int j = 0; j < QMAX; ++j) {
      if (j < (int)A.per) {
        const uint64_t m0 = ballot(x[j][0] >= te), m1 = ballot(x[j][1] >= te);
        const uint64_t m2 = ballot(x[j][2] >= te), m3 = ballot(x[j][3] >= te);
        if (m0 | m1 | m2 | m3) {
          const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m0, 0u)) +
                                 __builtin_amdgcn_mbcnt_hi((uint32_t)(m1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m1, 0u)) +
                                 __builtin_amdgcn_mbcnt_hi((uint32_t)(m2 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m2, 0u)) +
                                 __builtin_amdgcn_mbcnt_hi((uint32_t)(m3 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m3, 0u));
          uint32_t p = S.woff[(uint32_t)j * PW + w] + below;
          const uint32_t g0 = c0 + 4u * ((uint32_t)j * PT + t);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (x[j][i] >= te) {
              cb[p] = make_uint2(__float_as_uint(x[j][i]), g0 + (uint32_t)i);
              ++p;
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  stamp(A, row, c, 6u);

  // chunk mass for the top-p total: each thread's online f32 sum scaled to
  // the chunk maximum in f64, with a rigorous bound.  Per term: |y| ln2 3u
  // (y rounded thrice) + 4u (v_exp_f32); f32 additions n u; results below
  // 2^-126 absolute; rescales (mex) as accumulated in the loop.
  double cmass = 0.0, cerr = 0.0;
  if (need_mass && Mkey) {
    double sm = 0.0, b = 0.0;
    if (mref > -INFINITY) {
      const double gsc = exp_neg(((double)mref - (double)Mc) * cf.invT);
      sm = (double)ms * gsc;
      b = ((double)meb * 2.1 * (double)U24 + (double)ms * (4.0 + (double)mn) * 1.01 * (double)U24 + (double)mex +
           (double)mn * 1.1754943508222875e-38) * gsc * 1.001 + sm * 4.0 * U53;
    }
    cmass = red_sum_f64(sm, S, Bc, PW);
    cerr = red_sum_f64(b, S, Bc, PW) + cmass * 16.0 * U53;
  }

  // ---- statistics, then arrive
  if (t == 0) {
    uint32_t cfl = 0u, minkey = NONE;
    unsigned long long gbest = 0ull;
    for (int i = 0; i < PW; ++i) {
      cfl |= S.wr[PW + i];
      minkey = min(minkey, S.wr[3 * PW + i]);
      if (greedy) gbest = max(gbest, S.wg[i]);
    }
    Stat st;
    st.maxkey = Mkey;
    st.gkey = (uint32_t)(gbest >> 32);
    st.gid = gbest ? ~(uint32_t)gbest : NONE;
    st.nlegal = nl_c;
    st.ncand = ncand;
    st.flags = cfl;
    st.thr = thr;
    st.minkey = minkey;
    st.mass = cmass;
    st.mass_err = cerr;
    A.s.stat[(uint64_t)row * A.s.cm + c] = st;
  }
  // Every thread's candidate, segment, statistics and kept-bit stores happen
  // before the workgroup barrier, which happens before thread 0's release
  // on the row counter; the last arriver's acquire fence then makes all of
  // them visible to its workgroup.
  __syncthreads();
  if (t == 0)
    S.bc[3] = __hip_atomic_fetch_add(A.s.sync + (uint64_t)row * SYNC, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (S.bc[3] != A.C - 1u) return;
  if (t == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  finish_row<In>(A, S, cf, row);
  stamp(A, row, MXS_DEBUG_TIMING_SLOTS - 1u, 1u);
}

}  // namespace pk

// mxs_sample's launch (also the kept-set pass of mxs_sample_race, with
// `nodraw`: no inverse-CDF draw, token -1, status certifies the kept set).
int pick_launch(mxs_ctx* ctx, const mxs_batch* b, const mxs_out* o, bool nodraw) {
  if (!ctx || !b || !o) return MXS_EINVAL;
  if (b->rows == 0) return MXS_OK;
  if (!b->logits || !b->temperature || !o->token || !o->status)
    return fail(ctx, MXS_EINVAL, "logits, temperature, token and status are required");
  if (b->rows > ctx->max_rows || b->vocab > ctx->max_vocab)
    return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  if (b->vocab == 0) return fail(ctx, MXS_EINVAL, "vocab must be positive");
  if (b->vocab > pk::VMAX) return fail(ctx, MXS_EINVAL, "vocab exceeds 2621440");
  if (b->dtype != MXS_F32 && b->dtype != MXS_BF16) return fail(ctx, MXS_EINVAL, "dtype must be MXS_F32 or MXS_BF16");
  if (b->row_stride < b->vocab || (b->row_stride & 3u))
    return fail(ctx, MXS_EINVAL, "row_stride must be >= vocab and a multiple of 4");
  const size_t align = b->dtype == MXS_F32 ? 16 : 8;
  if (((uintptr_t)b->logits) % align) return fail(ctx, MXS_EINVAL, "logits must be 16-byte (f32) or 8-byte (bf16) aligned");
  if (b->mask_words && b->mask_stride < (b->vocab + 31u) / 32u)
    return fail(ctx, MXS_EINVAL, "mask_stride must be >= ceil(vocab / 32)");
  if ((b->history_offsets == nullptr) != (b->history_ids == nullptr))
    return fail(ctx, MXS_EINVAL, "history offsets and ids go together");
  if ((b->bias_offsets == nullptr) != (b->bias_ids == nullptr) || (b->bias_offsets && !b->bias_values))
    return fail(ctx, MXS_EINVAL, "bias offsets, ids and values go together");
  const pk::Layout Ly = pk::layout(b->vocab);
  if (Ly.C > ctx->pick.cm || Ly.per > (uint32_t)pk::QMAX || Ly.C > pk::MAXCH)
    return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  pk::Args A{};
  A.logits = b->logits;
  A.stride = b->row_stride;
  A.rows = b->rows;
  A.V = b->vocab;
  A.C = Ly.C;
  A.CH = Ly.CH;
  A.per = Ly.per;
  A.masked = b->mask_words != nullptr;
  A.tv = A.masked ? b->tokenizer_vocab : b->vocab;
  A.nodraw = nodraw ? 1u : 0u;
  A.mstride = b->mask_stride;
  A.T = b->temperature;
  A.topk = b->top_k ? b->top_k : ctx->d_zero_u32;
  A.topp = b->top_p ? b->top_p : ctx->d_one_f64;
  A.minp = b->min_p ? b->min_p : ctx->d_zero_f64;
  A.rep = b->repetition ? b->repetition : ctx->d_one_f32;
  A.pres = b->presence ? b->presence : ctx->d_zero_f32;
  A.freq = b->frequency ? b->frequency : ctx->d_zero_f32;
  A.u = b->uniform ? b->uniform : ctx->d_zero_f64;
  A.hoff = b->history_offsets ? b->history_offsets : ctx->d_zero_u32;
  A.hids = b->history_ids ? b->history_ids : ctx->d_zero_u32;
  A.boff = b->bias_offsets ? b->bias_offsets : ctx->d_zero_u32;
  A.bids = b->bias_ids ? b->bias_ids : ctx->d_zero_u32;
  A.bvals = b->bias_values ? b->bias_values : ctx->d_zero_f32;
  A.mask = b->mask_words ? b->mask_words : ctx->d_mask_ones;
  A.token = o->token;
  A.lp = o->sampling_logprob;
  A.status = o->status;
  A.kept_count = o->kept_count;
  A.adjusted = o->adjusted;
  A.kept_bits = o->kept_bits;
  A.s = ctx->pick;
  A.timing = ctx->timing;
  const uint32_t groups = (b->rows + 7u) / 8u;
  const dim3 grid(8u * Ly.C * groups);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  if (b->dtype == MXS_F32)
    hipLaunchKernelGGL(pk::pick_kernel<float>, grid, dim3(pk::PT), 0, ctx->stream, A);
  else
    hipLaunchKernelGGL(pk::pick_kernel<uint16_t>, grid, dim3(pk::PT), 0, ctx->stream, A);
  if (ctx->split_event) hipEventRecord(ctx->split_event, ctx->stream);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "pick_kernel launch");
  return MXS_OK;
}

}  // namespace mxs
