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
// One launch: each row is split into C chunks, one 1024-thread workgroup per
// chunk.  A chunk streams its logits once, reduces its maximum and its f64
// sum of exp(l - chunk maximum), and selects its own exact top-n by two
// block radix selects (the n-th largest per-thread maximum bounds the
// candidates, then the n-th largest candidate) with ties taken in ID order.
// The last chunk of the row to finish merges the C sorted lists and the C
// (maximum, sum) pairs.

#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_math.h"

namespace mxs {

constexpr uint32_t TOPN_MAX = 64;         // largest n served
constexpr int TP = 5;                     // quads per thread per chunk (registers hold the chunk)
constexpr int TMAXC = 128;                // chunks per row

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
  uint32_t rows, V, n, C, CH, per;
  int32_t* ids;
  double* logprobs;
  double* maximum;
  double* lognorm;
  int32_t* status;
  uint32_t* ctr;                // [rows] arrival counters
  TopnStat* stat;               // [rows * TMAXC]
  unsigned long long* list;     // [rows * TMAXC * TOPN_MAX], (okey << 32) | ~id, descending
};

struct alignas(16) TopnSmem {
  union {
    alignas(16) uint32_t hist[6][NBR];              // chunk phase: two radix selects, three passes each
    unsigned long long ent[TMAXC * TOPN_MAX];        // merge: every chunk's list
  };
  alignas(16) uint32_t wcnt[TP * NW + 32];
  unsigned long long top[TOPN_MAX];
  uint32_t rank_of[TOPN_MAX];
  TopnStat st[TMAXC];
  uint32_t coff[TMAXC + 1];
  uint32_t red_u[4][NW];
  double red_d[NW];
  uint32_t s_cnt, s_last;
};

__device__ __forceinline__ unsigned long long entry_key(uint32_t k, uint32_t id) {
  return ((unsigned long long)k << 32) | (unsigned long long)(~id);
}

template <typename In>
__global__ __launch_bounds__(NT) void topn_kernel(TopnArgs A) {
  __shared__ TopnSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  const uint32_t V = A.V;
  const uint32_t c0 = chunk * A.CH;
  const uint32_t c1 = min(V, c0 + A.CH);
  const In* src = reinterpret_cast<const In*>(A.logits) + (uint64_t)row * A.stride;

  typename Quad<In>::Raw raw[TP];
#pragma unroll
  for (int i = 0; i < TP; ++i) {
    const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
    raw[i] = Quad<In>::load(src + (e0 < c1 ? e0 : c0));
  }
  for (uint32_t t = tid; t < 6u * NBR / 4u; t += NT)
    reinterpret_cast<uint4*>(&S.hist[0][0])[t] = make_uint4(0u, 0u, 0u, 0u);
  if (tid == 0) S.s_cnt = 0u;

  // ---- pass 1: maximum, finite check, per-thread maximum -------------------
  float lv[TP][4];
  float t1 = -INFINITY;
  uint64_t nf = 0;
  uint32_t nin = 0;
#pragma unroll
  for (int i = 0; i < TP; ++i) {
    float x[4];
    Quad<In>::unpack(raw[i], x);
    const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool inr = i < (int)A.per && e0 + (uint32_t)e < c1;
      lv[i][e] = inr ? x[e] : -INFINITY;
      nf |= __builtin_amdgcn_ballot_w64(inr && !__builtin_isfinite(x[e]));
      t1 = fmaxf(t1, lv[i][e]);
      nin += inr ? 1u : 0u;
    }
  }
  {
    const uint32_t kmax = wave_max_u32(okey(t1));
    const uint32_t nact = wave_sum_u32(t1 > -INFINITY ? 1u : 0u);
    if (lane() == 0) {
      S.red_u[0][wave()] = kmax;
      S.red_u[1][wave()] = nf ? 1u : 0u;
      S.red_u[2][wave()] = nact;
    }
  }
  lds_barrier();
  uint32_t kmax = 0u, flags = 0u, nact = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    kmax = max(kmax, S.red_u[0][w]);
    flags |= S.red_u[1][w];
    nact += S.red_u[2][w];
  }
  const uint32_t cnt_chunk = c1 > c0 ? c1 - c0 : 0u;
  const float m = okey_value(kmax);
  const uint32_t n = A.n;
  const uint32_t take = min(n, cnt_chunk);
  double sum = 0.0;
  uint32_t listed = 0;
  if (!flags && cnt_chunk > 0) {
    // ---- pass 2: f64 sum of exp(l - m) ------------------------------------
    const double md = (double)m;
    double part = 0.0;
#pragma unroll
    for (int i = 0; i < TP; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) part += exp_neg((double)lv[i][e] - md);   // -inf -> 0
    part = wave_sum_f64(part);
    if (lane() == 0) S.red_d[wave()] = part;

    // ---- the chunk's exact top-n ---------------------------------------------
    if (take > 0) {
      uint32_t kth = 0u;
      uint64_t act = 0;
      uint32_t keys[TP * 4];
#pragma unroll
      for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) keys[i * 4 + e] = okey(lv[i][e]);
      const uint32_t KNEG = okey(-INFINITY);   // out-of-range tokens carry -inf
      if (take < cnt_chunk) {
        // The take-th largest per-thread maximum is at most the chunk's
        // take-th largest logit: only keys at or above it take part in
        // the exact select (when enough threads hold a logit).
        uint32_t lo = 0u;
        if (take <= nact) {
          uint32_t dummy;
          const uint32_t tk[1] = {okey(t1)};
          lo = block_kth_largest<1>(tk, t1 > -INFINITY ? 1ull : 0ull, take, &S.hist[0][0], &dummy);
        }
#pragma unroll
        for (int j = 0; j < TP * 4; ++j)
          if (keys[j] > KNEG && keys[j] >= lo) act |= 1ull << j;
        uint32_t above = 0;
        kth = block_kth_largest<TP * 4>(keys, act, take, &S.hist[3][0], &above);
        // keys above kth go straight in; ties at kth in token-ID order
        const uint32_t need_t = take - above;
#pragma unroll
        for (int j = 0; j < TP * 4; ++j) {
          if (((act >> j) & 1ull) && keys[j] > kth) {
            const uint32_t at = atomicAdd(&S.s_cnt, 1u);
            S.top[at] = entry_key(keys[j], c0 + (uint32_t)(j >> 2) * SLICE + tid * 4u + (uint32_t)(j & 3));
          }
        }
        // tie counts per (slice, wave), then ranks in ID order
#pragma unroll
        for (int i = 0; i < TP; ++i) {
          uint32_t cnt = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            cnt += (uint32_t)__builtin_popcountll(
                __builtin_amdgcn_ballot_w64(((act >> (i * 4 + e)) & 1ull) && keys[i * 4 + e] == kth));
          if (lane() == 0) S.wcnt[i * NW + wave()] = cnt;
        }
        lds_barrier();
        const uint32_t nent = (uint32_t)(TP * NW);
        const uint32_t v0 = lane() < nent ? S.wcnt[lane()] : 0u;
        const uint32_t v1 = lane() + 64u < nent ? S.wcnt[lane() + 64u] : 0u;
        const uint32_t v2 = lane() + 128u < nent ? S.wcnt[lane() + 128u] : 0u;
        const uint32_t i0 = wave_scan_u32(v0), i1 = wave_scan_u32(v1), i2 = wave_scan_u32(v2);
        const uint32_t s0 = bcast63(i0), s1 = bcast63(i1);
        const uint32_t x0 = i0 - v0, x1 = i1 - v1 + s0, x2 = i2 - v2 + s0 + s1;
#pragma unroll
        for (int i = 0; i < TP; ++i) {
          const uint32_t idx = (uint32_t)i * NW + wave();
          const uint32_t reg = idx >> 6;
          const uint32_t xv = reg == 0 ? x0 : (reg == 1 ? x1 : x2);
          const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)xv, (int)(idx & 63u));
          if (base >= need_t) continue;
          uint32_t before_me = 0;
          bool tie[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            tie[e] = ((act >> (i * 4 + e)) & 1ull) && keys[i * 4 + e] == kth;
            before_me += lanes_below(__builtin_amdgcn_ballot_w64(tie[e]));
          }
          uint32_t r = base + before_me;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (tie[e]) {
              if (r < need_t) {
                const uint32_t at = atomicAdd(&S.s_cnt, 1u);
                S.top[at] = entry_key(kth, c0 + (uint32_t)i * SLICE + tid * 4u + (uint32_t)e);
              }
              ++r;
            }
          }
        }
      } else {
        // the whole chunk is its own list
#pragma unroll
        for (int j = 0; j < TP * 4; ++j) {
          if (keys[j] > KNEG) {
            const uint32_t at = atomicAdd(&S.s_cnt, 1u);
            S.top[at] = entry_key(keys[j], c0 + (uint32_t)(j >> 2) * SLICE + tid * 4u + (uint32_t)(j & 3));
          }
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += S.red_d[w];
    listed = S.s_cnt;
    // sort the list (at most TOPN_MAX entries) by rank counting in wave 0
    if (wave() == 0) {
      const unsigned long long mine = lane() < listed ? S.top[lane()] : 0ull;
      uint32_t rank = 0;
      for (uint32_t j = 0; j < listed; ++j) rank += S.top[j] > mine ? 1u : 0u;
      if (lane() < listed)
        st_dev(reinterpret_cast<double*>(&A.list[((uint64_t)row * TMAXC + chunk) * TOPN_MAX + rank]),
               __builtin_bit_cast(double, mine));
    }
  }
  if (tid == 0) {
    TopnStat* st = &A.stat[(uint64_t)row * TMAXC + chunk];
    st_dev(&st->maxv, m);
    st_dev(&st->flags, flags);
    st_dev(&st->count, listed);
    st_dev(&st->sum, sum);
  }
  wait_mem();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&A.ctr[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.s_last = (prev == A.C - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!S.s_last) return;

  // ---- the row's last chunk: merge ------------------------------------------
  const uint32_t C = A.C;
  if (tid == 0) st_dev(&A.ctr[row], 0u);
  for (uint32_t q = tid; q < C; q += NT) {
    const TopnStat* st = &A.stat[(uint64_t)row * TMAXC + q];
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
  const uint32_t nout = min(n, V);
  if (rflags) {
    for (uint32_t j = tid; j < n; j += NT) {
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
  if (tid == 0) {
    uint32_t run = 0;
    for (uint32_t q = 0; q < C; ++q) { S.coff[q] = run; run += S.st[q].count; }
    S.coff[C] = run;
  }
  __syncthreads();
  const uint32_t total = S.coff[C];
  for (uint32_t j = tid; j < total; j += NT) {
    uint32_t q = 0;
    while (q + 1 < C && S.coff[q + 1] <= j) ++q;
    S.ent[j] = __builtin_bit_cast(unsigned long long,
                                  ld_dev(reinterpret_cast<const double*>(
                                      &A.list[((uint64_t)row * TMAXC + q) * TOPN_MAX + (j - S.coff[q])])));
  }
  double part = 0.0;
  for (uint32_t q = tid; q < C; q += NT)
    if (S.st[q].count) part += S.st[q].sum * exp_neg((double)S.st[q].maxv - M);
  part = wave_sum_f64(part);
  if (lane() == 0) S.red_d[wave()] = part;
  __syncthreads();
  double Ssum = 0.0;
#pragma unroll
  for (int w = 0; w < NW; ++w) Ssum += S.red_d[w];
  const double ln = log(Ssum);
  // rank of each entry: its place in its own sorted list plus, per other
  // list, the entries larger than it (binary search)
  for (uint32_t j = tid; j < total; j += NT) {
    uint32_t q = 0;
    while (q + 1 < C && S.coff[q + 1] <= j) ++q;
    const unsigned long long e = S.ent[j];
    uint32_t rank = j - S.coff[q];
    for (uint32_t r = 0; r < C; ++r) {
      if (r == q) continue;
      uint32_t lo = S.coff[r], hi = S.coff[r + 1];
      while (lo < hi) {
        const uint32_t md = (lo + hi) >> 1;
        if (S.ent[md] > e) lo = md + 1u; else hi = md;
      }
      rank += lo - S.coff[r];
    }
    if (rank < nout) {
      const uint32_t id = ~(uint32_t)e;
      const double l = (double)okey_value((uint32_t)(e >> 32));
      A.ids[(uint64_t)row * n + rank] = (int32_t)id;
      A.logprobs[(uint64_t)row * n + rank] = (l - M) - ln;
    }
  }
  for (uint32_t j = nout + tid; j < n; j += NT) {
    A.ids[(uint64_t)row * n + j] = -1;
    A.logprobs[(uint64_t)row * n + j] = -INFINITY;
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
  const mxs::ChunkLayout L = mxs::chunk_layout(vocab, mxs::TP);
  if (L.per > (uint32_t)mxs::TP || L.C > (uint32_t)mxs::TMAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  mxs::TopnArgs A;
  A.logits = logits;
  A.stride = row_stride;
  A.rows = rows;
  A.V = vocab;
  A.n = n;
  A.C = L.C;
  A.CH = L.CH;
  A.per = L.per;
  A.ids = ids;
  A.logprobs = logprobs;
  A.maximum = maximum;
  A.lognorm = log_normalizer;
  A.status = status;
  A.ctr = ctx->topn_ctr;
  A.stat = reinterpret_cast<mxs::TopnStat*>(ctx->topn_scratch);
  A.list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ctx->topn_scratch) +
                                                 (size_t)ctx->max_rows * mxs::TMAXC * sizeof(mxs::TopnStat));
  const dim3 grid(8u * L.C, (rows + 7u) / 8u);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  if (dtype == MXS_F32)
    hipLaunchKernelGGL(mxs::topn_kernel<float>, grid, dim3(mxs::NT), 0, ctx->stream, A);
  else
    hipLaunchKernelGGL(mxs::topn_kernel<uint16_t>, grid, dim3(mxs::NT), 0, ctx->stream, A);
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
