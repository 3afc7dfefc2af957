// mx_logprob.hip -- full-vocabulary log-softmax with the top-N tokens
// (mxs_logsoftmax_topn of include/mx_sampler.h).
//
// Reference semantics (arclabs561/metallix): token_logprob
// (crates/app/cli/src/chat_turn.rs:506-563): maximum = max over f64(logit)
// (NaN ignored), log_normalizer = ln(sum of exp(f64(l) - maximum)), the
// `top` IDs by (total_cmp descending, ID ascending) and each one's
// f64(l) - maximum - log_normalizer.  The caller over-selects top + 8 and
// filters unspellable IDs, as the reference does.
//
// Two launches.  The chunk pass: each row is split into C chunks of TCH tokens, one 256-thread
// workgroup per chunk (small register and LDS footprints, so several
// workgroups share a CU and their streams overlap).  A chunk streams its
// logits once and reduces its maximum and the f64 sum of exp(l - chunk
// maximum) over weights each within 2^-22 of exact (a corrected f32 exp2;
// the returned log probabilities stay within 2^-22 relative, see below).  For its top n it takes a threshold that at least n of its
// tokens reach: each wave's n-th largest lane maximum (n lanes each hold a
// token at least that large), the largest over the waves.  The tokens at or
// above it (about n to 2n of 8192 on ordinary rows) are ranked exactly by
// counting, in (total_cmp descending, ID ascending) order.  A chunk whose
// threshold admits more than TWCAP tokens in one wave (near-ties) takes an
// exact radix select instead.  The merge, one workgroup per row, merges the C sorted lists (the entries at or above the largest last
// entry of a full list, ranked by counting) and the C (maximum, sum) pairs;
// the launch boundary orders the chunk pass's stores before the merge's
// loads, so the chunk workgroups exit without waiting on an arrival counter.

#include <hip/hip_runtime.h>

#include <float.h>
#include <math.h>
#include <string.h>

#include <mutex>
#include <string>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_math.h"

namespace mxs {

constexpr uint32_t TOPN_MAX = 64;         // largest n served
constexpr int TNT = 256;                  // threads per workgroup
constexpr int TNW = TNT / 64;             // waves per workgroup
constexpr int TQ = 8;                     // quads per thread per chunk
constexpr uint32_t TSL = TNT * 4;         // tokens per slice (one quad per thread)
constexpr uint32_t TCH = TSL * TQ;        // tokens per chunk (8192)
constexpr int TMAXC = 320;                // chunks per row (vocab <= 320 * 8192)
constexpr uint32_t TWCAP = 256;           // candidate slots per wave

struct TopnStat {
  float maxv;          // chunk maximum (NaN ignored)
  uint32_t flags;      // 1: a non-finite logit
  uint32_t count;      // entries in the chunk's list
  uint32_t pad;
  double sum;          // sum of exp(f64(l) - maxv) over the chunk
};

struct TopnArgs {
  const void* logits;
  uint64_t stride;
  uint32_t rows, V, n, C;
  int32_t* ids;
  double* logprobs;
  double* maximum;              // nullptr: not written
  double* lognorm;              // nullptr: not written
  int32_t* status;
  TopnStat* stat;               // [rows * C]
  unsigned long long* list;     // [rows * C * n], (okey << 32) | ~id, descending
  // Step receipts (mxs_step): rows whose want entry is MXS_RECEIPT_NONE
  // are skipped; the bias CSR's -inf entries are the suppressed tokens,
  // read as f32::MIN (ChatFormat::suppress,
  // crates/core/chat-format/src/lib.rs:771-780); token_lp[row] is the
  // picked token's log probability.  All nullptr for mxs_logsoftmax_topn.
  const uint32_t* want;
  const uint32_t* sup_off;
  const uint32_t* sup_ids;
  const float* sup_vals;
  const int32_t* token;
  double* token_lp;
  uint32_t bf16;                // logits are bf16 (the merge's token read)
};

struct alignas(16) TopnSmem {
  union {
    alignas(16) uint32_t hist[NBR];                  // exact select (one radix pass at a time)
    unsigned long long cand[TNW * TWCAP];            // threshold candidates, per-wave regions
  } u;
  unsigned long long top[TOPN_MAX];                  // the exact select's list
  double etab[128];                                  // 2^(j/64) and its low parts (exp_neg_t)
  uint32_t supw[TCH / 32];                           // the chunk's suppressed tokens (one bit each)
  uint32_t wcnt[TQ * TNW];
  uint32_t wkept[TNW];
  uint32_t red_u[3][TNW];
  float red_f[TNW];
  double red_d[TNW];
  uint32_t s_cnt;
};

__device__ __forceinline__ unsigned long long entry_key(uint32_t k, uint32_t id) {
  return ((unsigned long long)k << 32) | (unsigned long long)(~id);
}

template <typename In>
__device__ __noinline__ void exact_list(unsigned long long* list, TopnSmem& S, const In* src, uint32_t c0, uint32_t c1,
                                        uint32_t take, bool sup) {
  const uint32_t tid = threadIdx.x;
  if (tid == 0) S.s_cnt = 0u;
  uint32_t keys[TQ * 4];
  uint64_t act = 0;
  for (int q = 0; q < TQ; ++q) {
    const uint32_t e0 = c0 + (uint32_t)q * TSL + tid * 4u;
    float v[4];
    Quad<In>::unpack(Quad<In>::load(src + (e0 < c1 ? e0 : c0)), v);
    const uint32_t sb = sup ? (S.supw[(uint32_t)q * (TSL / 32u) + (tid >> 3)] >> ((tid & 7u) * 4u)) : 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if ((sb >> e) & 1u) v[e] = -FLT_MAX;
      keys[q * 4 + e] = okey(v[e]);
      if (e0 + (uint32_t)e < c1) act |= 1ull << (q * 4 + e);
    }
  }
  lds_barrier();
  uint32_t above = 0;
  const uint32_t kth = block_kth_largest<TQ * 4>(keys, act, take, S.u.hist, &above);
  // keys above kth go straight in; ties at kth in token-ID order
  const uint32_t need_t = take - above;
  for (int j = 0; j < TQ * 4; ++j) {
    if (((act >> j) & 1ull) && keys[j] > kth) {
      const uint32_t at = atomicAdd(&S.s_cnt, 1u);
      S.top[at] = entry_key(keys[j], c0 + (uint32_t)(j >> 2) * TSL + tid * 4u + (uint32_t)(j & 3));
    }
  }
  // tie counts per (slice, wave) in token-ID order, then ranks
  for (int q = 0; q < TQ; ++q) {
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      cnt += (uint32_t)__builtin_popcountll(
          __builtin_amdgcn_ballot_w64(((act >> (q * 4 + e)) & 1ull) && keys[q * 4 + e] == kth));
    if (lane() == 0) S.wcnt[q * TNW + wave()] = cnt;
  }
  lds_barrier();
  static_assert(TQ * TNW <= 64, "one tie count per lane");
  const uint32_t v0 = lane() < (uint32_t)(TQ * TNW) ? S.wcnt[lane()] : 0u;
  const uint32_t x0 = wave_scan_u32(v0) - v0;
  for (int q = 0; q < TQ; ++q) {
    const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)x0, q * TNW + (int)wave());
    if (base >= need_t) continue;
    uint32_t before_me = 0;
    bool tie[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tie[e] = ((act >> (q * 4 + e)) & 1ull) && keys[q * 4 + e] == kth;
      before_me += lanes_below(__builtin_amdgcn_ballot_w64(tie[e]));
    }
    uint32_t r = base + before_me;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (tie[e]) {
        if (r < need_t) {
          const uint32_t at = atomicAdd(&S.s_cnt, 1u);
          S.top[at] = entry_key(kth, c0 + (uint32_t)q * TSL + tid * 4u + (uint32_t)e);
        }
        ++r;
      }
    }
  }
  lds_barrier();
  // sort the list (take entries) by rank counting in wave 0
  if (wave() == 0) {
    const unsigned long long mine = lane() < take ? S.top[lane()] : 0ull;
    uint32_t rank = 0;
    for (uint32_t j = 0; j < take; ++j) rank += S.top[j] > mine ? 1u : 0u;
    if (lane() < take) st_dev(&list[rank], mine);
  }
}

template <typename In>
__global__ __launch_bounds__(TNT, 6) void topn_kernel(TopnArgs A) {
  __shared__ TopnSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  if (A.want && A.want[row] == MXS_RECEIPT_NONE) return;   // a step row without a receipt
  const uint32_t V = A.V;
  const uint32_t c0 = chunk * TCH;
  const uint32_t c1 = min(V, c0 + TCH);
  const In* src = reinterpret_cast<const In*>(A.logits) + (uint64_t)row * A.stride;

  // Token (q, e) of this thread is c0 + q TSL + 4 tid + e: one base register
  // and immediate offsets.  Out-of-range tokens (the row's last chunk) read
  // as -inf; a row with a real -inf is non-finite and takes no list.
  const uint32_t len = c1 - c0;
  const uint32_t tb = c0 + tid * 4u;
  const double tab = tid < 128u ? (tid < 64u ? kExp2Tab[tid] : kExp2TabLo[tid - 64u]) : 0.0;
  typename Quad<In>::Raw raw[TQ];
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    const uint32_t off = (uint32_t)q * TSL + tid * 4u;
    raw[q] = Quad<In>::load(src + c0 + (off < len ? off : 0u));
  }

  if (tid < 128u) S.etab[tid] = tab;

  // The row's suppressed tokens in this chunk, as a bitmap (bit b of word w:
  // token c0 + 32 w + b); a block-uniform branch.
  bool sup = false;
  if (A.sup_off) {
    const uint32_t s0 = A.sup_off[row], s1 = A.sup_off[row + 1];
    if (s1 > s0) {
      sup = true;
      static_assert(TCH / 32 == TNT, "one bitmap word per thread");
      S.supw[tid] = 0u;
      lds_barrier();
      for (uint32_t j = s0 + tid; j < s1; j += TNT) {
        const uint32_t d = A.sup_ids[j] - c0;
        if (d < len && A.sup_vals[j] == -INFINITY) atomicOr(&S.supw[d >> 5], 1u << (d & 31u));
      }
      lds_barrier();
    }
  }

  // ---- pass 1: maximum, finite check, lane maxima ---------------------------
  float x[TQ][4];
  float t1 = -INFINITY;
  bool nf = false;
  if (sup) {
    // suppressed tokens read as f32::MIN; out-of-range ones as -inf
    const int rem = (int)len - (int)(tid * 4u);
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
      float v[4];
      Quad<In>::unpack(raw[q], v);
      const uint32_t sb = S.supw[(uint32_t)q * (TSL / 32u) + (tid >> 3)] >> ((tid & 7u) * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool inr = q * (int)TSL + e < rem;
        x[q][e] = !inr ? -INFINITY : ((sb >> e) & 1u) ? -FLT_MAX : v[e];
        nf |= inr && !__builtin_isfinite(x[q][e]);
        t1 = fmaxf(t1, x[q][e]);
      }
    }
  } else if (len == TCH) {
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
      Quad<In>::unpack(raw[q], x[q]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nf |= !__builtin_isfinite(x[q][e]);
        t1 = fmaxf(t1, x[q][e]);
      }
    }
  } else {
    const int rem = (int)len - (int)(tid * 4u);   // tokens of the chunk from this thread's first on
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
      float v[4];
      Quad<In>::unpack(raw[q], v);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool inr = q * (int)TSL + e < rem;
        x[q][e] = inr ? v[e] : -INFINITY;
        nf |= inr && !__builtin_isfinite(v[e]);
        t1 = fmaxf(t1, x[q][e]);
      }
    }
  }
  const uint32_t n = A.n;
  const uint32_t take = min(n, len);
  // This wave's take-th largest lane maximum: `take` lanes hold a token at
  // least that large, so the chunk's take-th largest token is too (0 when
  // fewer than `take` lanes hold a token: every token qualifies then).
  const uint64_t actl = __builtin_amdgcn_ballot_w64(t1 > -INFINITY);
  const uint32_t lk = okey(t1);
  uint32_t wthr = 0u;
  if (take > 0u && (uint32_t)__builtin_popcountll(actl) >= take) {
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = wthr | (1u << bit);
      const uint64_t ge = __builtin_amdgcn_ballot_w64(t1 > -INFINITY && lk >= cand);
      if ((uint32_t)__builtin_popcountll(ge) >= take) wthr = cand;
    }
  }
  // The wave's tokens at or above its threshold go to its LDS region (the
  // block threshold, the largest of the waves', is applied when ranking);
  // then the f64 sum of exp(l - t1) relative to this thread's maximum.
  uint32_t woff = 0u;   // this wave's candidates (uniform)
  double part = 0.0;
  if (take > 0u) {
    unsigned long long* wc = S.u.cand + wave() * TWCAP;
    // (a float compare: a superset of key >= wthr, never an out-of-range
    // -inf; the ranking filters by key)
    const float fthr = okey_value(max(wthr, okey(-INFINITY) + 1u));
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool c = x[q][e] >= fthr;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(c);
        if (bal) {
          const uint32_t at = woff + lanes_below(bal);
          if (c && at < TWCAP) wc[at] = entry_key(okey(x[q][e]), tb + (uint32_t)(q * TSL + e));
          woff += (uint32_t)__builtin_popcountll(bal);
        }
      }
    }
  }
  lds_barrier();   // the exp tables
  if (t1 > -INFINITY) {
    // Each weight 2^y, y = (l - t1) log2(e) <= 0, from the f32 exp2 of y's
    // f32 head corrected by its tail (y - head, below 2^-24 |y|): within
    // 2^-22 of exp(l - t1), with no error on the thread maximum's weight 1;
    // summed in f64.  Every weight but the row maximum's carries at most
    // that relative error, so the sum S is within 2^-22 (S - 1) and
    // ln S within 2^-22 (S - 1) / S <= 2^-22 of the exact values, and a
    // log probability (l - M) - ln S, of magnitude at least (S - 1) / S,
    // within 2^-22 relative.  y is clamped at -1000 (2^-1000 is 0 in f32):
    // out-of-range tokens (-inf) and suppressed ones (f32::MIN) weigh 0.
    const double tm = (double)t1;
#pragma unroll
    for (int q = 0; q < TQ; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double y = fmax(((double)x[q][e] - tm) * 1.4426950408889634, -1000.0);
        const float yh = (float)y;
        const float yl = (float)(y - (double)yh);
        const float eh = __builtin_amdgcn_exp2f(yh);
        part += (double)__builtin_fmaf(eh, yl * 0.69314718f, eh);
      }
  }
  {
    const uint32_t kmax = wave_max_u32(lk);
    const uint64_t anynf = __builtin_amdgcn_ballot_w64(nf);
    if (lane() == 0) {
      S.red_u[0][wave()] = kmax;
      S.red_u[1][wave()] = anynf ? 1u : 0u;
      S.red_u[2][wave()] = wthr;
      S.wcnt[wave()] = woff;
    }
  }
  lds_barrier();
  uint32_t kmax = 0u, flags = 0u, lthr = 0u, ncand = 0u, over = 0u;
  uint32_t wb[TNW];
#pragma unroll
  for (int w = 0; w < TNW; ++w) {
    kmax = max(kmax, S.red_u[0][w]);
    flags |= S.red_u[1][w];
    lthr = max(lthr, S.red_u[2][w]);
    wb[w] = ncand;
    ncand += S.wcnt[w];
    over |= S.wcnt[w] > TWCAP ? 1u : 0u;
  }
  const float m = okey_value(kmax);
  double sum = 0.0;
  uint32_t listed = 0;
  if (!flags && len > 0) {
    // the thread's sum rescaled to the chunk maximum
    if (t1 > -INFINITY) part *= exp_neg_t((double)t1 - (double)m, S.etab, S.etab + 64);
    part = wave_sum_f64(part);
    if (lane() == 0) S.red_d[wave()] = part;
    if (take > 0u && !over) {
      // ---- the candidates at or above the block threshold: each wave
      // compacts its own region in place, then they are ranked by counting
      // (keys are distinct).
      {
        const uint32_t wn = S.wcnt[wave()];
        unsigned long long* wc = S.u.cand + wave() * TWCAP;
        unsigned long long ev[TWCAP / 64];
        bool keep[TWCAP / 64];
#pragma unroll
        for (int i = 0; i < (int)(TWCAP / 64); ++i) {
          const uint32_t k = lane() + 64u * (uint32_t)i;
          ev[i] = k < wn ? wc[k] : 0ull;
          keep[i] = k < wn && (uint32_t)(ev[i] >> 32) >= lthr;
        }
        uint32_t mk = 0;
#pragma unroll
        for (int i = 0; i < (int)(TWCAP / 64); ++i) {
          const uint64_t b = __builtin_amdgcn_ballot_w64(keep[i]);
          if (keep[i]) wc[mk + lanes_below(b)] = ev[i];
          mk += (uint32_t)__builtin_popcountll(b);
        }
        if (lane() == 0) S.wkept[wave()] = mk;
      }
      lds_barrier();
      uint32_t kb[TNW + 1];
      kb[0] = 0;
#pragma unroll
      for (int w = 0; w < TNW; ++w) kb[w + 1] = kb[w] + S.wkept[w];
      for (uint32_t j = tid; j < kb[TNW]; j += TNT) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 1; i < TNW; ++i) w += j >= kb[i] ? 1u : 0u;
        const unsigned long long mine = S.u.cand[w * TWCAP + (j - kb[w])];
        uint32_t rank = 0;
#pragma unroll
        for (int v = 0; v < TNW; ++v) {
          const unsigned long long* cw = S.u.cand + v * TWCAP;
          const uint32_t cn = kb[v + 1] - kb[v];
          for (uint32_t i = 0; i < cn; ++i) rank += cw[i] > mine ? 1u : 0u;
        }
        if (rank < take) st_dev(&A.list[((uint64_t)row * A.C + chunk) * n + rank], mine);
      }
      listed = take;
    } else if (take > 0u) {
      __syncthreads();   // the histograms overlay the candidate slots
      exact_list<In>(A.list + ((uint64_t)row * A.C + chunk) * n, S, src, c0, c1, take, sup);
      listed = take;
    }
    lds_barrier();
#pragma unroll
    for (int w = 0; w < TNW; ++w) sum += S.red_d[w];
  }
  if (tid == 0) {
    TopnStat* st = &A.stat[(uint64_t)row * A.C + chunk];
    st_dev(&st->maxv, m);
    st_dev(&st->flags, flags);
    st_dev(&st->count, listed);
    st_dev(&st->sum, sum);
  }
}

// ---------------------------------------------------------------------------
// The merge: one workgroup per row, after the chunk pass (the launch boundary
// orders the chunks' stores before its loads).  Every chunk of a row without
// non-finite logits lists min(n, its length) entries, sorted.  A list of n
// entries has n at or above its last, so entries below the largest such
// last entry (thr) cannot rank below n.  The entries at or above thr (about
// n to 2n on ordinary rows) are collected, in rounds of at most MGRP lists
// with the running top n, and ranked by counting.
constexpr uint32_t MDCAP = 2048;                  // collected entries a round selects from
struct alignas(16) MergeSmem {
  unsigned long long dense[MDCAP];
  unsigned long long tie[MDCAP];
  alignas(16) uint32_t hist[NBR];
  unsigned long long sel[TOPN_MAX];
  unsigned long long top[TOPN_MAX];
  uint32_t red_u[2][TNW];
  double red_d[TNW];
  unsigned long long red64[TNW];
  uint32_t s_m, s_sel, s_tie;
};

// The `want` largest of S.dense[0, m) (distinct keys, want <= m, want <=
// TOPN_MAX) into S.top[0, want), sorted descending: a radix select of the
// want-th largest high word (the f32 key), the entries above it, and the
// ties at it by counting on the full key.
__device__ __forceinline__ void top_of_dense(MergeSmem& S, uint32_t m, uint32_t want) {
  const uint32_t tid = threadIdx.x;
  constexpr int RM = (int)(MDCAP / TNT);
  if (tid == 0) { S.s_sel = 0u; S.s_tie = 0u; }
  if (want < m) {
    uint32_t keys[RM];
    uint64_t act = 0;
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const uint32_t j = tid + (uint32_t)i * TNT;
      keys[i] = j < m ? (uint32_t)(S.dense[j] >> 32) : 0u;
      if (j < m) act |= 1ull << i;
    }
    uint32_t above = 0;
    const uint32_t kth = block_kth_largest<RM>(keys, act, want, S.hist, &above);
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      if (!((act >> i) & 1ull)) continue;
      const unsigned long long e = S.dense[tid + (uint32_t)i * TNT];
      if (keys[i] > kth) S.sel[atomicAdd(&S.s_sel, 1u)] = e;
      else if (keys[i] == kth) S.tie[atomicAdd(&S.s_tie, 1u)] = e;
    }
    __syncthreads();
    const uint32_t need = want - above, t = S.s_tie;
    for (uint32_t j = tid; j < t; j += TNT) {
      const unsigned long long e = S.tie[j];
      uint32_t r = 0;
      if (t > need)
        for (uint32_t i = 0; i < t; ++i) r += S.tie[i] > e ? 1u : 0u;
      if (r < need) S.sel[above + (t > need ? r : j)] = e;
    }
  } else {
    for (uint32_t j = tid; j < m; j += TNT) S.sel[j] = S.dense[j];
  }
  __syncthreads();
  if (wave() == 0) {   // sort the selection by counting
    const unsigned long long e = lane() < want ? S.sel[lane()] : 0ull;
    uint32_t r = 0;
    for (uint32_t i = 0; i < want; ++i) r += S.sel[i] > e ? 1u : 0u;
    if (lane() < want) S.top[r] = e;
  }
  __syncthreads();
}

__global__ __launch_bounds__(TNT) void topn_merge_kernel(TopnArgs A) {
  __shared__ MergeSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t row = blockIdx.x;
  if (A.want && A.want[row] == MXS_RECEIPT_NONE) return;   // a step row without a receipt
  const uint32_t V = A.V, n = A.n;
  const uint32_t C = A.C;
  const unsigned long long* lists = A.list + (uint64_t)row * C * n;
  auto cnt_of = [&](uint32_t q) { return min(n, min(TCH, V - q * TCH)); };
  // chunk statistics and the last entry of each full list (chunks tid, tid + TNT)
  float cm[2];
  double cs[2];
  uint32_t fl = 0;
  float mx = -INFINITY;
  unsigned long long tl = 0ull;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t q = tid + (uint32_t)i * TNT;
    cm[i] = -INFINITY;
    cs[i] = 0.0;
    if (q < C) {
      const TopnStat* st = &A.stat[(uint64_t)row * C + q];
      cm[i] = ld_dev(&st->maxv);
      cs[i] = ld_dev(&st->sum);
      fl |= ld_dev(&st->flags);
      mx = fmaxf(mx, cm[i]);
      if (n > 0 && cnt_of(q) == n)
        tl = max(tl, __builtin_bit_cast(unsigned long long,
                                        ld_dev(reinterpret_cast<const double*>(&lists[(uint64_t)q * n + n - 1u]))));
    }
  }
  {
    const uint32_t wf = wave_or_u32(fl);
    const uint32_t wm = wave_max_u32(okey(mx));
    tl = wave_max_u64(tl);
    if (lane() == 0) { S.red_u[0][wave()] = wf; S.red_u[1][wave()] = wm; S.red64[wave()] = tl; }
  }
  __syncthreads();
  uint32_t rflags = 0, mkey = 0;
  unsigned long long thr = 0ull;
#pragma unroll
  for (int w = 0; w < TNW; ++w) {
    rflags |= S.red_u[0][w];
    mkey = max(mkey, S.red_u[1][w]);
    thr = max(thr, S.red64[w]);
  }
  if (rflags) {   // a non-finite logit (the chunks wrote no lists)
    for (uint32_t j = tid; j < n; j += TNT) {
      A.ids[(uint64_t)row * n + j] = -1;
      A.logprobs[(uint64_t)row * n + j] = __builtin_nan("");
    }
    if (tid == 0) {
      A.status[row] = MXS_ROW_NON_FINITE_LOGIT;
      if (A.maximum) A.maximum[row] = __builtin_nan("");
      if (A.lognorm) A.lognorm[row] = __builtin_nan("");
      if (A.token_lp) A.token_lp[row] = __builtin_nan("");
    }
    return;
  }
  const double M = (double)okey_value(mkey);
  double rpart = 0.0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (cs[i] > 0.0) rpart += cs[i] * exp_neg_p((double)cm[i] - M);
  rpart = wave_sum_f64(rpart);
  if (lane() == 0) S.red_d[wave()] = rpart;
  uint32_t nrun = 0;
  if (n > 0) {
    const uint32_t grp = (MDCAP - TOPN_MAX) / n;          // lists per round
    const uint32_t mg = ((1u << 20) + n - 1u) / n;        // j / n == (j * mg) >> 20 for j < 2^14
    for (uint32_t q0 = 0; q0 < C; q0 += grp) {
      const uint32_t q1 = min(C, q0 + grp);
      if (tid == 0) S.s_m = 0u;
      __syncthreads();
      // the running top n (all at or above thr are kept) and this round's
      // entries at or above thr
      for (uint32_t j = tid; j < nrun; j += TNT) {
        const unsigned long long e = S.top[j];
        if (e >= thr) S.dense[atomicAdd(&S.s_m, 1u)] = e;
      }
      const uint32_t span = (q1 - q0) * n;
      for (uint32_t j = tid; j < span; j += TNT) {
        const uint32_t l = (j * mg) >> 20;
        const uint32_t pos = j - l * n;
        if (pos >= cnt_of(q0 + l)) continue;
        const unsigned long long e = __builtin_bit_cast(
            unsigned long long, ld_dev(reinterpret_cast<const double*>(&lists[(uint64_t)(q0 + l) * n + pos])));
        if (e >= thr) S.dense[atomicAdd(&S.s_m, 1u)] = e;
      }
      __syncthreads();
      const uint32_t m = S.s_m;
      nrun = min(n, m);
      top_of_dense(S, m, nrun);   // the new running top, in order
    }
  }
  __syncthreads();
  double Ssum = 0.0;
#pragma unroll
  for (int w = 0; w < TNW; ++w) Ssum += S.red_d[w];
  const double ln = log(Ssum);
  const uint32_t nout = min(n, V);
  for (uint32_t j = tid; j < n; j += TNT) {
    if (j < nout && j < nrun) {
      const unsigned long long e = S.top[j];
      const double l = (double)okey_value((uint32_t)(e >> 32));
      A.ids[(uint64_t)row * n + j] = (int32_t)(~(uint32_t)e);
      A.logprobs[(uint64_t)row * n + j] = (l - M) - ln;
    } else {
      A.ids[(uint64_t)row * n + j] = -1;
      A.logprobs[(uint64_t)row * n + j] = -INFINITY;
    }
  }
  if (tid == 0) {
    A.status[row] = 0;
    if (A.maximum) A.maximum[row] = M;
    if (A.lognorm) A.lognorm[row] = ln;
    if (A.token_lp) {
      // the picked token's f64(l) - maximum - log_normalizer under the same
      // suppressed logits (token_logprob's `logprob(selected)`); NaN for a
      // row without a token
      const int32_t t = A.token[row];
      double lp = __builtin_nan("");
      if (t >= 0 && (uint32_t)t < V) {
        const uint64_t at = (uint64_t)row * A.stride + (uint32_t)t;
        float l = A.bf16 ? bf16_to_f32(reinterpret_cast<const uint16_t*>(A.logits)[at])
                         : reinterpret_cast<const float*>(A.logits)[at];
        if (A.sup_off) {
          // bias ids increase within a row: binary search for t
          uint32_t lo = A.sup_off[row], hi = A.sup_off[row + 1];
          while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (A.sup_ids[mid] < (uint32_t)t) lo = mid + 1u;
            else hi = mid;
          }
          if (lo < A.sup_off[row + 1] && A.sup_ids[lo] == (uint32_t)t && A.sup_vals[lo] == -INFINITY) l = -FLT_MAX;
        }
        lp = ((double)l - M) - ln;
      }
      A.token_lp[row] = lp;
    }
  }
}

}  // namespace mxs

namespace mxs {

// Argument checks shared by both entry points (nullptr: accepted).
static const char* topn_check(const void* logits, int32_t dtype, uint32_t vocab, uint64_t row_stride, uint32_t n,
                              const int32_t* ids, const double* logprobs, const double* maximum,
                              const double* log_normalizer, const int32_t* status) {
  if (!logits || !maximum || !log_normalizer || !status || (n > 0 && (!ids || !logprobs)))
    return "logits, maximum, log_normalizer and status are required (ids and logprobs when n > 0)";
  if (vocab == 0) return "vocab must be positive";
  if (n > TOPN_MAX) return "n must be at most 64";
  if (dtype != MXS_F32 && dtype != MXS_BF16) return "dtype must be MXS_F32 or MXS_BF16";
  if (row_stride < vocab || (row_stride & 3u)) return "row_stride must be >= vocab and a multiple of 4";
  if (((uintptr_t)logits) % (dtype == MXS_F32 ? 16u : 8u)) return "logits must be 16-byte (f32) or 8-byte (bf16) aligned";
  if ((vocab + TCH - 1u) / TCH > (uint32_t)TMAXC) return "vocab too large for the chunk layout";
  return nullptr;
}

// Queues the chunk pass and the merge on `stream` (current device) with the
// per-chunk statistics and lists at `stat` and `list`.
static hipError_t topn_launch(hipStream_t stream, const void* logits, int32_t dtype, uint32_t rows, uint32_t vocab,
                              uint64_t row_stride, uint32_t n, int32_t* ids, double* logprobs, double* maximum,
                              double* log_normalizer, int32_t* status, TopnStat* stat, unsigned long long* list,
                              const TopnArgs* step = nullptr) {
  const uint32_t C = (vocab + TCH - 1u) / TCH;
  TopnArgs A{};
  if (step) A = *step;
  A.logits = logits;
  A.stride = row_stride;
  A.rows = rows;
  A.V = vocab;
  A.n = n;
  A.C = C;
  A.ids = ids;
  A.logprobs = logprobs;
  A.maximum = maximum;
  A.lognorm = log_normalizer;
  A.status = status;
  A.stat = stat;
  A.list = list;
  A.bf16 = dtype == MXS_BF16 ? 1u : 0u;
  const dim3 grid(8u * C, (rows + 7u) / 8u);
  if (dtype == MXS_F32)
    hipLaunchKernelGGL(topn_kernel<float>, grid, dim3(TNT), 0, stream, A);
  else
    hipLaunchKernelGGL(topn_kernel<uint16_t>, grid, dim3(TNT), 0, stream, A);
  hipLaunchKernelGGL(topn_merge_kernel, dim3(rows), dim3(TNT), 0, stream, A);
  return hipGetLastError();
}

// Scratch bytes the context allocates for mxs_logsoftmax_topn.
size_t topn_scratch_bytes(uint32_t max_rows) {
  return (size_t)max_rows * TMAXC * (sizeof(TopnStat) + TOPN_MAX * sizeof(unsigned long long));
}

// ---------------------------------------------------------------------------
// mxs_logsoftmax_topn_noalloc: the per-chunk statistics and lists live in a
// device array of the library (one copy per GPU, held until the process
// ends).  Its device address is looked up once per device, with that device
// current, and kept; host code passes that address, never the array's name
// (a host-side stand-in).  Calls on one GPU share the array.
static __device__ __align__(256) unsigned char scratch[MXS_TOPN_STATIC_BYTES];
constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES];
static thread_local std::string g_noalloc_error;

static int noalloc_fail(int code, const std::string& msg) {
  g_noalloc_error = msg;
  return code;
}

static int scratch_of_device(int dev, void** out) {
  if (dev < 0 || dev >= MAX_DEVICES) return noalloc_fail(MXS_ENODEV, "device index beyond the library's table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return noalloc_fail(MXS_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MXS_OK;
}

const char* noalloc_last_error() { return g_noalloc_error.empty() ? nullptr : g_noalloc_error.c_str(); }

}  // namespace mxs

extern "C" int mxs_logsoftmax_topn(mxs_ctx* ctx, const void* logits, int32_t dtype, uint32_t rows, uint32_t vocab,
                                   uint64_t row_stride, uint32_t n, int32_t* ids, double* logprobs, double* maximum,
                                   double* log_normalizer, int32_t* status) {
  if (!ctx) return MXS_EINVAL;
  if (rows == 0) return MXS_OK;
  if (const char* m = mxs::topn_check(logits, dtype, vocab, row_stride, n, ids, logprobs, maximum, log_normalizer, status))
    return fail(ctx, MXS_EINVAL, m);
  if (rows > ctx->max_rows || vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  auto* stat = reinterpret_cast<mxs::TopnStat*>(ctx->topn_scratch);
  auto* list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ctx->topn_scratch) +
                                                     (size_t)ctx->max_rows * mxs::TMAXC * sizeof(mxs::TopnStat));
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  const hipError_t e = mxs::topn_launch(ctx->stream, logits, dtype, rows, vocab, row_stride, n, ids, logprobs, maximum,
                                        log_normalizer, status, stat, list);
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "topn launch");
  return MXS_OK;
}

extern "C" int mxs_logsoftmax_topn_noalloc(void* stream, const void* logits, int32_t dtype, uint32_t rows,
                                           uint32_t vocab, uint64_t row_stride, uint32_t n, int32_t* ids,
                                           double* logprobs, double* maximum, double* log_normalizer,
                                           int32_t* status) {
  if (rows == 0) return MXS_OK;
  if (const char* m = mxs::topn_check(logits, dtype, vocab, row_stride, n, ids, logprobs, maximum, log_normalizer, status))
    return mxs::noalloc_fail(MXS_EINVAL, m);
  const uint64_t pairs = (uint64_t)rows * ((vocab + mxs::TCH - 1u) / mxs::TCH);
  const uint64_t stat_bytes = (pairs * sizeof(mxs::TopnStat) + 255u) & ~(uint64_t)255u;
  if (stat_bytes + pairs * n * sizeof(unsigned long long) > (uint64_t)MXS_TOPN_STATIC_BYTES)
    return mxs::noalloc_fail(MXS_EINVAL, "rows * ceil(vocab / 8192) * (24 + 8 n) bytes exceed MXS_TOPN_STATIC_BYTES");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mxs::noalloc_fail(MXS_ENODEV, std::string("hipGetDevice: ") + hipGetErrorString(e));
  void* base = nullptr;
  if (int rc = mxs::scratch_of_device(dev, &base)) return rc;
  auto* stat = reinterpret_cast<mxs::TopnStat*>(base);
  auto* list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(base) + stat_bytes);
  e = mxs::topn_launch((hipStream_t)stream, logits, dtype, rows, vocab, row_stride, n, ids, logprobs, maximum,
                       log_normalizer, status, stat, list);
  if (e != hipSuccess) return mxs::noalloc_fail(MXS_EHIP, std::string("topn launch: ") + hipGetErrorString(e));
  return MXS_OK;
}

// One engine step (engine_loop.rs:1080-1134, ChatTurn::pick at
// chat_turn.rs:290-303): every row's pick and the log-probability receipt of
// the rows that want one, over the logits after suppression: one pass of
// the sample kernel, or, under race-v2, the top-n kernels after the race.
extern "C" int mxs_step(mxs_ctx* ctx, const mxs_batch* batch, const mxs_race* race, const mxs_out* out,
                        const mxs_receipts* receipts) {
  if (!ctx || !batch || !out) return MXS_EINVAL;
  if (receipts) {
    const mxs_receipts& R = *receipts;
    if (R.n == 0 || R.n > mxs::TOPN_MAX) return fail(ctx, MXS_EINVAL, "receipts->n must be in 1..64");
    if (!R.ids || !R.logprobs || !R.token_logprob || !R.status)
      return fail(ctx, MXS_EINVAL, "receipts: ids, logprobs, token_logprob and status are required");
    if (const char* m = mxs::topn_check(batch->logits, batch->dtype, batch->vocab, batch->row_stride, R.n, R.ids,
                                        R.logprobs, R.token_logprob, R.token_logprob, R.status))
      return fail(ctx, MXS_EINVAL, m);
  }
  if (!race) {
    // the receipts come from the pick's own pass over the logits
    if (batch->rows == 0) return MXS_OK;
    return mxs::sample_launch(ctx, batch, out, false, receipts);
  }
  // race-v2: the token comes from the race kernel, so the receipts follow it
  int rc = mxs_sample_race(ctx, batch, race, out);
  if (rc != MXS_OK || !receipts || batch->rows == 0) return rc;
  const mxs_receipts& R = *receipts;
  mxs::TopnArgs X{};
  X.want = R.top;
  X.sup_off = batch->bias_offsets;
  X.sup_ids = batch->bias_ids;
  X.sup_vals = batch->bias_values;
  X.token = out->token;
  X.token_lp = R.token_logprob;
  auto* stat = reinterpret_cast<mxs::TopnStat*>(ctx->topn_scratch);
  auto* list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ctx->topn_scratch) +
                                                     (size_t)ctx->max_rows * mxs::TMAXC * sizeof(mxs::TopnStat));
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  const hipError_t e = mxs::topn_launch(ctx->stream, batch->logits, batch->dtype, batch->rows, batch->vocab,
                                        batch->row_stride, R.n, R.ids, R.logprobs, nullptr, nullptr, R.status, stat,
                                        list, &X);
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "receipt launch");
  return MXS_OK;
}
