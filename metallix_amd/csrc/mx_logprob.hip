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
// One launch: each row is split into C chunks of TCH tokens, one 256-thread
// workgroup per chunk (small register and LDS footprints, so several
// workgroups share a CU and their streams overlap).  A chunk streams its
// logits once and reduces its maximum and its f64 sum of exp(l - chunk
// maximum).  For its top n it takes a threshold that at least n of its
// tokens reach: each wave's n-th largest lane maximum (n lanes each hold a
// token at least that large), the largest over the waves.  The tokens at or
// above it (about n to 2n of 8192 on ordinary rows) are ranked exactly by
// counting, in (total_cmp descending, ID ascending) order.  A chunk whose
// threshold admits more than TWCAP tokens in one wave (near-ties) takes an exact radix
// select over its registers instead.  The last chunk of the row to arrive
// merges the C sorted lists (by binary search ranks, in rounds of at most
// TMCAP entries) and the C (maximum, sum) pairs.

#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

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
constexpr uint32_t TMCAP = 2048;          // list entries one merge round holds

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
  double* maximum;
  double* lognorm;
  int32_t* status;
  uint32_t* ctr;                // [rows] arrival counters, CTR_STRIDE words apart
  TopnStat* stat;               // [rows * C]
  unsigned long long* list;     // [rows * C * n], (okey << 32) | ~id, descending
};

struct alignas(16) TopnSmem {
  union {
    alignas(16) uint32_t hist[3][NBR];               // exact select: three radix passes
    unsigned long long cand[TNW * TWCAP];            // threshold candidates, per-wave regions
    unsigned long long ent[TMCAP];                   // merge round
  } u;
  unsigned long long top[TOPN_MAX];                  // the chunk's list / the merge's running list
  double etab[128];                                  // 2^(j/64) and its low parts
  TopnStat st[TMAXC];
  uint32_t lo[TMAXC + 2];                            // merge: list boundaries within ent
  uint32_t wcnt[TQ * TNW];
  uint32_t red_u[3][TNW];
  double red_d[TNW];
  unsigned long long red64[TNW];
  uint32_t s_cnt, s_last, s_n;
};

__device__ __forceinline__ unsigned long long entry_key(uint32_t k, uint32_t id) {
  return ((unsigned long long)k << 32) | (unsigned long long)(~id);
}

// Entries of the sorted (descending) list ent[b, e) larger than x.
__device__ __forceinline__ uint32_t count_above(const unsigned long long* ent, uint32_t b, uint32_t e,
                                                unsigned long long x) {
  uint32_t lo = b, hi = e;
  while (lo < hi) {
    const uint32_t md = (lo + hi) >> 1;
    if (ent[md] > x) lo = md + 1u; else hi = md;
  }
  return lo - b;
}

// A chunk's exact top `take` (near-ties: the threshold admitted too many
// tokens): radix select over the chunk, reloaded, with ties at the k-th key
// taken in token-ID order; the list goes out sorted.
template <typename In>
__device__ __noinline__ void exact_list(const TopnArgs& A, TopnSmem& S, const In* src, uint32_t row, uint32_t chunk,
                                        uint32_t c0, uint32_t c1, uint32_t take) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t t = tid; t < 3u * NBR / 4u; t += TNT)
    reinterpret_cast<uint4*>(&S.u.hist[0][0])[t] = make_uint4(0u, 0u, 0u, 0u);
  if (tid == 0) S.s_cnt = 0u;
  uint32_t keys[TQ * 4];
  uint64_t act = 0;
  for (int q = 0; q < TQ; ++q) {
    const uint32_t e0 = c0 + (uint32_t)q * TSL + tid * 4u;
    float v[4];
    Quad<In>::unpack(Quad<In>::load(src + (e0 < c1 ? e0 : c0)), v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      keys[q * 4 + e] = okey(v[e]);
      if (e0 + (uint32_t)e < c1) act |= 1ull << (q * 4 + e);
    }
  }
  lds_barrier();
  uint32_t above = 0;
  const uint32_t kth = block_kth_largest<TQ * 4>(keys, act, take, &S.u.hist[0][0], &above);
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
    if (lane() < take) st_dev(&A.list[((uint64_t)row * A.C + chunk) * A.n + rank], mine);
  }
}

template <typename In>
__global__ __launch_bounds__(TNT, 4) void topn_kernel(TopnArgs A) {
  __shared__ TopnSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  const uint32_t V = A.V;
  const uint32_t c0 = chunk * TCH;
  const uint32_t c1 = min(V, c0 + TCH);
  const In* src = reinterpret_cast<const In*>(A.logits) + (uint64_t)row * A.stride;

  // the exp tables first: their loads complete ahead of the stream's
  const double tab = tid < 128u ? (tid < 64u ? kExp2Tab[tid] : kExp2TabLo[tid - 64u]) : 0.0;
  typename Quad<In>::Raw raw[TQ];
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    const uint32_t e0 = c0 + (uint32_t)q * TSL + tid * 4u;
    raw[q] = Quad<In>::load(src + (e0 < c1 ? e0 : c0));
  }
  if (tid < 128u) S.etab[tid] = tab;

  // ---- pass 1: maximum, finite check, lane maxima ---------------------------
  float x[TQ][4];
  float t1 = -INFINITY;
  bool nf = false;
#pragma unroll
  for (int q = 0; q < TQ; ++q) {
    float v[4];
    Quad<In>::unpack(raw[q], v);
    const uint32_t e0 = c0 + (uint32_t)q * TSL + tid * 4u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool inr = e0 + (uint32_t)e < c1;
      x[q][e] = inr ? v[e] : -INFINITY;
      nf |= inr && !__builtin_isfinite(v[e]);
      t1 = fmaxf(t1, x[q][e]);
    }
  }
  const uint32_t n = A.n;
  const uint32_t len = c1 - c0;
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
#pragma unroll
    for (int q = 0; q < TQ; ++q) {
      const uint32_t e0 = c0 + (uint32_t)q * TSL + tid * 4u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t key = okey(x[q][e]);
        const bool c = e0 + (uint32_t)e < c1 && key >= wthr;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(c);
        if (bal) {
          const uint32_t at = woff + lanes_below(bal);
          if (c && at < TWCAP) wc[at] = entry_key(key, e0 + (uint32_t)e);
          woff += (uint32_t)__builtin_popcountll(bal);
        }
      }
    }
  }
  lds_barrier();   // the exp tables are in LDS
  if (t1 > -INFINITY) {
    const double tm = (double)t1;
#pragma unroll
    for (int q = 0; q < TQ; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) part += exp_neg_p((double)x[q][e] - tm);   // -inf -> 0
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
      // ---- rank the candidates at or above the block threshold by counting
      // (keys are distinct; candidates below it never outrank one above it)
      for (uint32_t j = tid; j < ncand; j += TNT) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 1; i < TNW; ++i) w += j >= wb[i] ? 1u : 0u;
        const unsigned long long mine = S.u.cand[w * TWCAP + (j - wb[w])];
        if ((uint32_t)(mine >> 32) < lthr) continue;
        uint32_t rank = 0;
        for (int v = 0; v < TNW; ++v) {
          const unsigned long long* cw = S.u.cand + v * TWCAP;
          const uint32_t cn = S.wcnt[v];
          for (uint32_t i = 0; i < cn; ++i) rank += cw[i] > mine ? 1u : 0u;
        }
        if (rank < take) st_dev(&A.list[((uint64_t)row * A.C + chunk) * n + rank], mine);
      }
      listed = take;
    } else if (take > 0u) {
      __syncthreads();   // the histograms overlay the candidate slots
      exact_list<In>(A, S, src, row, chunk, c0, c1, take);
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
  if (!arrive_last(A.ctr + (uint64_t)row * CTR_STRIDE, A.C, &S.s_last)) return;

  // ---- the row's last chunk: merge ------------------------------------------
  const uint32_t C = A.C;
  for (uint32_t q = tid; q < C; q += TNT) {
    const TopnStat* st = &A.stat[(uint64_t)row * C + q];
    TopnStat v;
    v.maxv = ld_dev(&st->maxv);
    v.flags = ld_dev(&st->flags);
    v.count = ld_dev(&st->count);
    v.sum = ld_dev(&st->sum);
    S.st[q] = v;
  }
  __syncthreads();
  uint32_t rflags = 0;
  float M32 = -INFINITY;
  for (uint32_t q = 0; q < C; ++q) {
    rflags |= S.st[q].flags;
    M32 = fmaxf(M32, S.st[q].maxv);
  }
  if (rflags) {
    for (uint32_t j = tid; j < n; j += TNT) {
      A.ids[(uint64_t)row * n + j] = -1;
      A.logprobs[(uint64_t)row * n + j] = __builtin_nan("");
    }
    if (tid == 0) {
      A.status[row] = MXS_ROW_NON_FINITE_LOGIT;
      A.maximum[row] = __builtin_nan("");
      A.lognorm[row] = __builtin_nan("");
    }
    return;
  }
  const double M = (double)M32;
  double rpart = 0.0;
  for (uint32_t q = tid; q < C; q += TNT)
    if (S.st[q].sum > 0.0) rpart += S.st[q].sum * exp_neg_t((double)S.st[q].maxv - M, S.etab, S.etab + 64);
  rpart = wave_sum_f64(rpart);
  if (lane() == 0) S.red_d[wave()] = rpart;
  // Merge rounds: the running list (sorted, at most n entries) and as many
  // whole chunk lists as fit in TMCAP entries; each entry's rank is its
  // place in its own list plus, per other list, the entries larger than it.
  const uint32_t nout = min(n, V);
  uint32_t nrun = 0;
  uint32_t q0 = 0;
  if (n > 0) {
    while (q0 < C) {
      if (tid == 0) {
        uint32_t at = nrun, q = q0, k = 1;
        S.lo[0] = 0u;
        S.lo[1] = nrun;
        while (q < C && at + S.st[q].count <= TMCAP) {
          at += S.st[q].count;
          S.lo[++k] = at;
          ++q;
        }
        S.s_n = q;   // chunks q0 .. q - 1 join this round
      }
      __syncthreads();
      const uint32_t q1 = S.s_n;
      const uint32_t nl = q1 - q0 + 1u;   // lists: the running list, then the chunks
      const uint32_t total = S.lo[nl];
      for (uint32_t j = tid; j < total; j += TNT) {
        unsigned long long v;
        if (j < nrun) {
          v = S.top[j];
        } else {
          uint32_t l = 1;
          while (S.lo[l + 1] <= j) ++l;
          const uint32_t q = q0 + l - 1u;
          v = __builtin_bit_cast(unsigned long long,
                                 ld_dev(reinterpret_cast<const double*>(&A.list[((uint64_t)row * C + q) * n + (j - S.lo[l])])));
        }
        S.u.ent[j] = v;
      }
      __syncthreads();
      // A list of n entries has n at or above its last: entries below the
      // largest such last entry cannot rank below n.
      unsigned long long tl = 0ull;
      for (uint32_t l = tid; l < nl; l += TNT)
        if (S.lo[l + 1] - S.lo[l] >= n) tl = max(tl, S.u.ent[S.lo[l] + n - 1u]);
      tl = wave_max_u64(tl);
      if (lane() == 0) S.red64[wave()] = tl;
      __syncthreads();
      unsigned long long thr = 0ull;
#pragma unroll
      for (int w = 0; w < TNW; ++w) thr = max(thr, S.red64[w]);
      for (uint32_t j = tid; j < total; j += TNT) {
        const unsigned long long e = S.u.ent[j];
        if (e < thr) continue;
        uint32_t l = 0;
        while (S.lo[l + 1] <= j) ++l;
        uint32_t rank = j - S.lo[l];
        for (uint32_t r = 0; r < nl; ++r)
          if (r != l) rank += count_above(S.u.ent, S.lo[r], S.lo[r + 1], e);
        if (rank < n) S.top[rank] = e;
      }
      nrun = min(n, total);
      q0 = q1;
      __syncthreads();
    }
  }
  __syncthreads();
  double Ssum = 0.0;
#pragma unroll
  for (int w = 0; w < TNW; ++w) Ssum += S.red_d[w];
  const double ln = log(Ssum);
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
    A.maximum[row] = M;
    A.lognorm[row] = ln;
  }
}

}  // namespace mxs

extern "C" int mxs_logsoftmax_topn(mxs_ctx* ctx, const void* logits, int32_t dtype, uint32_t rows, uint32_t vocab,
                                   uint64_t row_stride, uint32_t n, int32_t* ids, double* logprobs, double* maximum,
                                   double* log_normalizer, int32_t* status) {
  if (!ctx) return MXS_EINVAL;
  if (rows == 0) return MXS_OK;
  if (!logits || !maximum || !log_normalizer || !status || (n > 0 && (!ids || !logprobs)))
    return fail(ctx, MXS_EINVAL, "logits, maximum, log_normalizer and status are required (ids and logprobs when n > 0)");
  if (rows > ctx->max_rows || vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  if (vocab == 0) return fail(ctx, MXS_EINVAL, "vocab must be positive");
  if (n > mxs::TOPN_MAX) return fail(ctx, MXS_EINVAL, "n must be at most 64");
  if (dtype != MXS_F32 && dtype != MXS_BF16) return fail(ctx, MXS_EINVAL, "dtype must be MXS_F32 or MXS_BF16");
  if (row_stride < vocab || (row_stride & 3u)) return fail(ctx, MXS_EINVAL, "row_stride must be >= vocab and a multiple of 4");
  if (((uintptr_t)logits) % (dtype == MXS_F32 ? 16u : 8u)) return fail(ctx, MXS_EINVAL, "logits must be 16-byte (f32) or 8-byte (bf16) aligned");
  const uint32_t C = (vocab + mxs::TCH - 1u) / mxs::TCH;
  if (C > (uint32_t)mxs::TMAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  mxs::TopnArgs A;
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
  A.ctr = ctx->topn_ctr;
  A.stat = reinterpret_cast<mxs::TopnStat*>(ctx->topn_scratch);
  A.list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ctx->topn_scratch) +
                                                 (size_t)ctx->max_rows * mxs::TMAXC * sizeof(mxs::TopnStat));
  const dim3 grid(8u * C, (rows + 7u) / 8u);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  if (dtype == MXS_F32)
    hipLaunchKernelGGL(mxs::topn_kernel<float>, grid, dim3(mxs::TNT), 0, ctx->stream, A);
  else
    hipLaunchKernelGGL(mxs::topn_kernel<uint16_t>, grid, dim3(mxs::TNT), 0, ctx->stream, A);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "topn_kernel launch");
  return MXS_OK;
}

namespace mxs {
// Scratch bytes the context allocates for mxs_logsoftmax_topn.
size_t topn_scratch_bytes(uint32_t max_rows) {
  return (size_t)max_rows * TMAXC * (sizeof(TopnStat) + TOPN_MAX * sizeof(unsigned long long));
}
}  // namespace mxs
