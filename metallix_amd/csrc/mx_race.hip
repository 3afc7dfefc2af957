// mx_race.hip -- race-v2 picks: the Gumbel-max winner over each row's kept set.
//
// race-v2 (crates/core/engine/src/sampling/race.rs:1-17, 114-147) picks the
// kept token maximising f64(logit) / T + g, lowest token ID on ties, where g
// is Gumbel noise made from 64 Philox4x32-10 bits keyed by the request seed
// and counted by (token >> 1, position, choice, "race") (race.rs:39-80) and
// turned into -ln E with E = -ln(1 - w), w = (bits + 1/2) 2^-64, each half of
// the bit range taking the form that keeps full relative precision
// (race.rs:82-99).  The kept set is the one mxs_sample builds (bias,
// penalties, grammar mask, top-k -> top-p -> min-p); the reference applies
// race-v2 to its nucleus mask the same way (SamplingPolicy::sample with
// Entropy::Race after nucleus_mask, crates/app/cli/src/qwen_forward.rs:
// 221-278).  sampling_logprob is sample_race's: the winner's shifted logit
// over the kept set minus ln of the kept set's f64 mass.
//
// Scores are computed in f64 on the device.  The inputs of log1p/log are
// formed exactly as the reference forms them (u64 -> f64 rounds to nearest,
// + 0.5 and the power-of-two scale are the same IEEE operations), the
// division by T is correctly rounded on both sides, and only the two log
// evaluations may differ from the reference's libm by an ulp or so.  A
// winner is therefore certified when its score leads the runner-up by more
// than 2^-46 (64 + |s1| + |s2|), far above both sides' rounding
// (about 2^-50 (1 + |g| + |score|) each); otherwise the row's status is 1
// (uncertified) and it carries the device's winner.
//
// Launch: grid (8 C, rows / 8) of RNT-thread workgroups; chunk c of a row covers
// tokens [c RT, (c + 1) RT), 32 tokens RNT apart per thread.
// Each chunk reduces its kept tokens to a RaceStat; the row's last chunk to
// arrive (device-scope counter) merges them and writes the row's result.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mxs_ctx.h"
#include "mxs_device.h"

namespace mxs {

constexpr int RNT = 256;                       // threads per race workgroup
constexpr int RNW = RNT / 64;
constexpr uint32_t RT = (uint32_t)RNT * 32u;    // tokens per race chunk

// One chunk's kept tokens, reduced.
struct alignas(16) RaceStat {
  double best;      // largest score (-inf when the chunk keeps nothing)
  double second;    // largest score of every other kept token of the chunk
  double mass;      // sum of exp((l - m) / T) over the chunk's kept tokens (m the row maximum)
  float m;          // the row's largest adjusted logit (the mass's reference point)
  float lbest;      // the winner's adjusted logit
  uint32_t id;      // the winner's token ID (NONE when empty)
  uint32_t flags;   // RF_* below
  uint32_t pad[2];
};
constexpr uint32_t RF_ANY = 1u;        // the chunk keeps a token
constexpr uint32_t RF_NONFINITE = 2u;  // a kept token's score is not finite

size_t race_scratch_bytes(uint32_t max_rows, uint32_t max_vocab) {
  return (size_t)max_rows * ((max_vocab + RT - 1u) / RT) * sizeof(RaceStat);
}

struct RaceArgs {
  const void* logits;
  uint64_t stride;
  uint32_t rows, V, nwords, C;
  const double* temperature;
  const float* rep;
  const float* pres;
  const float* freq;
  const uint32_t* hoff;
  const uint32_t* hids;
  const uint32_t* boff;
  const uint32_t* bids;
  const float* bvals;
  const uint32_t* kept;     // rows x nwords, written by the row finisher
  const float* rowmax;      // rows: the largest adjusted logit (written by the row finisher)
  const uint64_t* seed;
  const uint32_t* choice;
  const uint32_t* position;
  int32_t* token;
  double* logprob;          // may be null
  int32_t* status;
  uint32_t* ctr;            // per-row arrival counters, CTR_STRIDE words apart (zero between calls)
  RaceStat* stat;           // rows x C
};

// Philox4x32 with 10 rounds (Salmon et al., SC'11; race.rs:39-54).
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

// The 64 noise bits of token `id` (race.rs:66-80).
__device__ __forceinline__ uint64_t race_bits(uint64_t seed, uint32_t choice, uint32_t position, uint32_t id) {
  uint32_t c[4] = {id >> 1, position, choice, 0x72616365u};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const uint32_t hi = (id & 1u) ? c[2] : c[0];
  const uint32_t lo = (id & 1u) ? c[3] : c[1];
  return ((uint64_t)hi << 32) | lo;
}

// Gumbel noise -ln E from 64 bits (race.rs:82-99).
__device__ __forceinline__ double gumbel_from_bits(uint64_t bits) {
  const double s = 0x1p-64;
  double e;
  if (bits < (1ull << 63))
    e = -log1p(-(((double)bits + 0.5) * s));
  else
    e = -log(((double)(~bits) + 0.5) * s);
  return -log(e);
}

// The same noise in f32, for screening: E from the bits' f32 image (relative
// error about 2^-22 either branch; the w branch keeps log1p's precision for
// small w), then f32 logs (about 2 ulp each).  |g32 - g| < 1e-5.
__device__ __forceinline__ float gumbel32(uint64_t bits) {
  const uint32_t hi = (uint32_t)(bits >> 32), lo = (uint32_t)bits;
  float e;
  if (!(hi >> 31)) {
    const float w = ((float)hi + ((float)lo + 0.5f) * 0x1p-32f) * 0x1p-32f;
    e = -log1pf(-w);
  } else {
    const float v = ((float)(~hi) + ((float)(~lo) + 0.5f) * 0x1p-32f) * 0x1p-32f;
    e = -logf(v);
  }
  return -logf(e);
}

// Bound on |s32 - (l / T + g - m / T)| for the f32 screening score
// s32 = (l - m) * (1/T)_f32 + g32 (m the row's largest adjusted logit, at or
// above every kept logit):
// (l - m) / T <= 0 and g <= 45.1 give |(l - m) / T| <= |s32| + 46, whose
// three f32 roundings cost under 2^-22.4 (|s32| + 46); plus |g32 - g| and
// the final rounding.  The form below is several times larger than that.
__device__ __forceinline__ float err32(float s32) { return 0x1p-10f + fabsf(s32) * 0x1p-19f; }

// Certification margin between the two best device scores.
__device__ __forceinline__ double race_margin(double s1, double s2) {
  return 0x1p-46 * (64.0 + fabs(s1) + fabs(s2));
}

// Best-score bookkeeping: the best (score, lowest ID on ties) and the best
// score of everything else seen.
struct Best {
  double s1, s2;
  uint32_t id;
  float l;
};
__device__ __forceinline__ void best_merge(Best& a, double s1, double s2, uint32_t id, float l) {
  if (s1 > a.s1 || (s1 == a.s1 && id < a.id)) {
    a.s2 = fmax(s2, a.s1);
    a.s1 = s1;
    a.id = id;
    a.l = l;
  } else {
    a.s2 = fmax(a.s2, s1);
  }
}

// History counts of a chunk's tokens, two 16-bit counts per LDS word (token
// d of the chunk in half d & 1), so that the table takes 16 KB and eight
// workgroups share a CU.  A row with at most 65535 history entries cannot
// carry a count into its neighbour, and plain adds are exact.  A longer
// history adds with compare-and-swap, saturating at 0xFFFF, and a saturated
// count is recounted from the history itself.
__device__ __forceinline__ void cnt_add_sat(uint32_t* p, uint32_t sh) {
  uint32_t old = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (((old >> sh) & 0xFFFFu) != 0xFFFFu) {
    const uint32_t prev = atomicCAS(p, old, old + (1u << sh));
    if (prev == old) return;
    old = prev;
  }
}

struct RaceSmem {
  uint32_t cnt[RT / 2];      // history counts of the chunk's tokens (16-bit pairs)
  float redf2[RNW];
  double redd[RNW];
  double b1[RNW], b2[RNW];
  uint32_t bid[RNW];
  float bl[RNW];
  uint32_t kw[RNT];          // the chunk's kept-set words
  uint32_t any, last;
};

template <typename In>
__global__ __launch_bounds__(RNT) void race_kernel(RaceArgs A) {
  __shared__ RaceSmem S;
  // blockIdx.x = chunk * 8 + xcd and row = blockIdx.y * 8 + xcd: workgroup
  // i runs on XCD i mod 8, so a row's chunks share one XCD's L2.
  const uint32_t tid = threadIdx.x, chunk = blockIdx.x >> 3, row = blockIdx.y * 8u + (blockIdx.x & 7u);
  if (row >= A.rows) return;
  // Every per-row load goes out at once (the kept words and the row's
  // parameters are in bounds for every row below A.rows).
  const int32_t st0 = A.status[row];
  const double T = A.temperature[row];
  const uint32_t base = chunk * RT;
  const uint32_t w = chunk * (uint32_t)RNT + tid;
  uint32_t word = w < A.nwords ? A.kept[(uint64_t)row * A.nwords + w] : 0u;
  const uint32_t hb = A.hoff[row], he = A.hoff[row + 1];
  const uint32_t bb = A.boff[row], be = A.boff[row + 1];
  const float rep = A.rep[row], pres = A.pres[row], freq = A.freq[row];
  const float mrow = A.rowmax[row];
  // Rows the finisher rejected and greedy rows keep the finisher's result.
  if (st0 < 0 || T == 0.0) return;
  if (tid == 0) S.any = 0u;
  S.kw[tid] = word;
  __syncthreads();
  if (word) S.any = 1u;
  __syncthreads();
  const bool any = S.any != 0u;

  Best b{-INFINITY, -INFINITY, NONE, 0.0f};
  float m = -INFINITY;
  double mass = 0.0;
  uint32_t flags = 0u;
  if (any) {
    const bool longh = he - hb > 0xFFFFu;
    if (he > hb) {
      for (uint32_t i = tid; i < RT / 2u; i += RNT) S.cnt[i] = 0u;
      __syncthreads();
      for (uint32_t h = hb + tid; h < he; h += RNT) {
        const uint32_t d = A.hids[h] - base;
        if (d < RT) {
          if (!longh) atomicAdd(&S.cnt[d >> 1], 1u << ((d & 1u) * 16u));
          else cnt_add_sat(&S.cnt[d >> 1], (d & 1u) * 16u);
        }
      }
      __syncthreads();
    }
    const In* lrow = reinterpret_cast<const In*>(A.logits) + (uint64_t)row * A.stride;
    // The adjusted logit of a kept token (the chunk pass's bias and penalty
    // stage, penalize_logit).
    auto adjusted = [&](uint32_t id) -> float {
      const float l = Quad<In>::one(lrow + id);
      uint32_t cnt = 0u;
      if (he > hb) {
        const uint32_t d = id - base;
        cnt = (S.cnt[d >> 1] >> ((d & 1u) * 16u)) & 0xFFFFu;
        if (cnt == 0xFFFFu) {   // saturated (histories above 65535 entries): recount
          cnt = 0u;
          for (uint32_t h = hb; h < he; ++h) cnt += A.hids[h] == id ? 1u : 0u;
        }
      }
      uint32_t lo = bb, hi = be;   // bias ids are strictly increasing
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (A.bids[mid] < id) lo = mid + 1u; else hi = mid;
      }
      const bool hasb = lo < be && A.bids[lo] == id;
      return penalize_logit(l, cnt, hasb, hasb ? A.bvals[lo] : 0.0f, rep, pres, freq);
    };
    // Thread tid takes the chunk's tokens tid + 256 j (j < 32): a wave's
    // logit loads are consecutive tokens.  Bit j of `mine` is token
    // tid + 256 j's kept bit (word tid / 32 + 8 j, bit tid mod 32).
    uint32_t mine = 0u;
    for (uint32_t j = 0; j < 32u; ++j) mine |= ((S.kw[(tid >> 5) + 8u * j] >> (tid & 31u)) & 1u) << j;
    const uint32_t id0 = base + tid;
    // The reference point of the scores and the mass: the row's largest
    // adjusted logit, which the finisher found (the kept set holds it), so
    // no pass over the chunk's tokens precedes the scoring.
    m = mrow;
    const uint64_t seed = A.seed[row];
    const uint32_t choice = A.choice[row], position = A.position[row];
    const double invT = 1.0 / T;
    const float invT32 = (float)invT;
    // f32 screening scores and the f64 mass
    // This thread's two largest screening scores, and the largest one's
    // token, logit and noise bits.
    float t1 = -INFINITY, t2 = -INFINITY, l1 = 0.0f;
    uint32_t id1 = 0u;
    uint64_t bits1 = 0ull;
    for (uint32_t r = mine; r; r &= r - 1u) {
      const uint32_t id = id0 + 256u * (uint32_t)__builtin_ctz(r);
      const float l = adjusted(id);
      mass += exp(((double)l - (double)m) * invT);   // (within an ulp of the quotient: the mass feeds only the logprob)
      const uint64_t bits = race_bits(seed, choice, position, id);
      const float s32 = (l - m) * invT32 + gumbel32(bits);
      if (s32 > t1) {
        t2 = t1; t1 = s32; id1 = id; l1 = l; bits1 = bits;
      } else {
        t2 = fmaxf(t2, s32);
      }
    }
    float smax = t1;
    smax = wave_max(smax);
    if (lane() == 0) S.redf2[wave()] = smax;
    __syncthreads();
    smax = S.redf2[0];
    for (int i = 1; i < RNW; ++i) smax = fmaxf(smax, S.redf2[i]);
    // Exact f64 scores for tokens whose f32 upper bound reaches the chunk
    // maximum's lower bound (less 2^-10).  A token screened out scores below
    // that threshold plus m / T, at least 2^-10 under the winner: the bound
    // stands in for its score as a runner-up.
    // (No screen when 1/T overflows f32: every kept token is then scored in
    // f64; the finisher has already checked that (l - M) / T is finite.)
    const bool screen = __builtin_isfinite(invT32) && __builtin_isfinite(smax);
    const float cut = smax - err32(smax) - 0x1p-10f;
    // s + err32(s) rises with s, up to f32 rounding far below err32, so a
    // thread whose largest score fails the screen by more than err32 holds
    // no token that passes it.  When its second largest score fails that
    // way, only its largest can pass, and that token was kept in registers;
    // the other threads recompute their screening scores (the same
    // operations, so the same values) token by token.
    uint32_t out = 0u;
    if (screen && !(t1 + err32(t1) + err32(t1) >= cut)) {
      out = __builtin_popcount(mine);
    } else if (screen && !(t2 + err32(t2) + err32(t2) >= cut)) {
      // only the thread's largest score can pass: its token needs no reload
      out = __builtin_popcount(mine) - 1u;
      if (!(t1 + err32(t1) >= cut)) {
        ++out;
      } else {
        const double sc = (double)l1 / T + gumbel_from_bits(bits1);
        if (!isfinite(sc)) flags |= RF_NONFINITE;
        best_merge(b, sc, -INFINITY, id1, l1);
      }
    } else
    for (uint32_t r = mine; r; r &= r - 1u) {
      const uint32_t id = id0 + 256u * (uint32_t)__builtin_ctz(r);
      const float l = adjusted(id);
      const uint64_t bits = race_bits(seed, choice, position, id);
      if (screen) {
        const float s32 = (l - m) * invT32 + gumbel32(bits);
        if (!(s32 + err32(s32) >= cut)) { ++out; continue; }
      }
      const double s = (double)l / T + gumbel_from_bits(bits);
      if (!isfinite(s)) flags |= RF_NONFINITE;
      best_merge(b, s, -INFINITY, id, l);
    }
    if (out) b.s2 = fmax(b.s2, (double)cut + (double)m / T);
  }
  // block reductions: mass, flags, best
  mass = wave_sum(mass);
  for (int o = 32; o > 0; o >>= 1) {
    const double s1 = __shfl_xor(b.s1, o), s2 = __shfl_xor(b.s2, o);
    const uint32_t id = __shfl_xor(b.id, o);
    const float l = __shfl_xor(b.l, o);
    best_merge(b, s1, s2, id, l);
  }
  flags = wave_or_u32(flags);
  if (lane() == 0) {
    S.redd[wave()] = mass;
    S.b1[wave()] = b.s1;
    S.b2[wave()] = b.s2;
    S.bid[wave()] = b.id;
    S.bl[wave()] = b.l;
  }
  __syncthreads();
  if (tid == 0) {
    Best t{-INFINITY, -INFINITY, NONE, 0.0f};
    double ms = 0.0;
    for (int i = 0; i < RNW; ++i) {
      ms += S.redd[i];
      best_merge(t, S.b1[i], S.b2[i], S.bid[i], S.bl[i]);
    }
    RaceStat* p = &A.stat[(uint64_t)row * A.C + chunk];
    if (any) {   // the merge reads only the flags of a chunk that keeps nothing
      st_dev(&p->best, t.s1);
      st_dev(&p->second, t.s2);
      st_dev(&p->mass, ms);
      st_dev(&p->m, m);
      st_dev(&p->lbest, t.l);
      st_dev(&p->id, t.id);
    }
    st_dev(&p->flags, flags | (any ? RF_ANY : 0u));
    // The chunk's record is this thread's own device-scope stores: they
    // complete before the increment (the ordering argument of arrive_last),
    // and the last arriver's acquire fence precedes the merge's loads.
    wait_mem();
    uint32_t* ctr = A.ctr + (uint64_t)row * CTR_STRIDE;
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = prev + 1u == A.C ? 1u : 0u;
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      st_dev(ctr, 0u);
    }
    S.last = last;
  }
  __syncthreads();
  if (!S.last || wave() != 0) return;
  // ---- the row's last chunk: wave 0 merges the chunks' records, lane q
  // taking chunks q, q + 64, ... (all loads in flight at once) ------------
  const uint32_t ln = lane();
  const RaceStat* rs = &A.stat[(uint64_t)row * A.C];
  uint32_t rf = 0u;
  float M = -INFINITY;
  for (uint32_t q = ln; q < A.C; q += 64u) {
    const uint32_t f = ld_dev(&rs[q].flags);
    rf |= f;
    if (f & RF_ANY) M = fmaxf(M, ld_dev(&rs[q].m));
  }
  rf = wave_or_u32(rf);
  M = wave_max(M);
  Best r{-INFINITY, -INFINITY, NONE, 0.0f};
  double S_ = 0.0;
  for (uint32_t q = ln; q < A.C; q += 64u) {
    if (!(ld_dev(&rs[q].flags) & RF_ANY)) continue;
    S_ += ld_dev(&rs[q].mass) * exp(((double)ld_dev(&rs[q].m) - (double)M) / T);
    best_merge(r, ld_dev(&rs[q].best), ld_dev(&rs[q].second), ld_dev(&rs[q].id), ld_dev(&rs[q].lbest));
  }
  S_ = wave_sum(S_);
  for (int o = 32; o > 0; o >>= 1) {
    const double s1 = __shfl_xor(r.s1, o), s2 = __shfl_xor(r.s2, o);
    const uint32_t id = __shfl_xor(r.id, o);
    const float l = __shfl_xor(r.l, o);
    best_merge(r, s1, s2, id, l);
  }
  if (ln != 0) return;
  if (!(rf & RF_ANY)) {
    A.status[row] = MXS_ROW_EMPTY_SUPPORT;
    A.token[row] = -1;
    if (A.logprob) A.logprob[row] = 0.0;
    return;
  }
  if (rf & RF_NONFINITE) {
    A.status[row] = MXS_ROW_INVALID_TEMPERATURE;
    A.token[row] = -1;
    if (A.logprob) A.logprob[row] = 0.0;
    return;
  }
  // a lone kept token (no runner-up) needs no margin
  const bool certified = r.s2 == -INFINITY || r.s1 - r.s2 > race_margin(r.s1, r.s2);
  A.token[row] = (int32_t)r.id;
  A.status[row] = (st0 == MXS_ROW_OK && certified) ? MXS_ROW_OK : MXS_ROW_UNCERTIFIED;
  if (A.logprob) A.logprob[row] = ((double)r.l - (double)M) / T - log(S_);
}

}  // namespace mxs

extern "C" int mxs_sample_race(mxs_ctx* ctx, const mxs_batch* b, const mxs_race* race, const mxs_out* o) {
  if (!ctx || !b || !race || !o) return MXS_EINVAL;
  if (b->rows == 0) return MXS_OK;
  if (!race->seed || !race->position) return fail(ctx, MXS_EINVAL, "race seed and position are required");
  if (!o->token || !o->status) return fail(ctx, MXS_EINVAL, "token and status are required");
  if (b->rows > ctx->max_rows || b->vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  // The kept set comes from mxs_sample's pipeline; race-v2 draws no uniform.
  mxs_batch b2 = *b;
  b2.uniform = ctx->d_race_u;
  mxs_out o2 = *o;
  if (!o2.kept_bits) o2.kept_bits = ctx->race_kept;
  int rc = mxs::sample_launch(ctx, &b2, &o2, true);
  if (rc != MXS_OK) return rc;
  mxs::RaceArgs A;
  A.logits = b->logits;
  A.stride = b->row_stride;
  A.rows = b->rows;
  A.V = b->vocab;
  A.nwords = (b->vocab + 31u) / 32u;
  A.C = (b->vocab + mxs::RT - 1u) / mxs::RT;
  A.temperature = b->temperature;
  A.rep = b->repetition ? b->repetition : ctx->d_one_f32;
  A.pres = b->presence ? b->presence : ctx->d_zero_f32;
  A.freq = b->frequency ? b->frequency : ctx->d_zero_f32;
  A.hoff = b->history_offsets ? b->history_offsets : ctx->d_zero_u32;
  A.hids = b->history_ids ? b->history_ids : ctx->d_zero_u32;
  A.boff = b->bias_offsets ? b->bias_offsets : ctx->d_zero_u32;
  A.bids = b->bias_ids ? b->bias_ids : ctx->d_zero_u32;
  A.bvals = b->bias_values ? b->bias_values : ctx->d_zero_f32;
  A.kept = o2.kept_bits;
  A.rowmax = ctx->race_m;
  A.seed = race->seed;
  A.choice = race->choice ? race->choice : ctx->d_zero_u32;
  A.position = race->position;
  A.token = o->token;
  A.logprob = o->sampling_logprob;
  A.status = o->status;
  A.ctr = ctx->race_ctr;
  A.stat = static_cast<mxs::RaceStat*>(ctx->race_scratch);
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (prev != ctx->device) (void)hipSetDevice(ctx->device);
  const dim3 grid(8u * A.C, (b->rows + 7u) / 8u);
  if (b->dtype == MXS_F32)
    hipLaunchKernelGGL(mxs::race_kernel<float>, grid, dim3(mxs::RNT), 0, ctx->stream, A);
  else
    hipLaunchKernelGGL(mxs::race_kernel<uint16_t>, grid, dim3(mxs::RNT), 0, ctx->stream, A);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "race_kernel launch");
  return MXS_OK;
}
