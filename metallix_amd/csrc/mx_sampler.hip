// mx_sampler.hip -- MI355X (gfx950) token sampler: kernels and the C ABI of
// include/mx_sampler.h.
//
// One launch samples a batch.  Each logit row is split into C chunks of at
// most CHUNK_MAX tokens; one 1024-thread workgroup streams a chunk from HBM
// once into registers (16-byte loads, coalesced), applies logit bias and
// penalties from an LDS count table, the grammar mask and the finite check,
// reduces the chunk's statistics and writes a compact, token-ID-ordered
// candidate list.  The last workgroup of the row to finish (a relaxed
// device-scope counter, no grid barrier) becomes the row's finisher: it
// merges the chunk statistics and candidates and decides top-k, top-p,
// min-p and the inverse-CDF draw in f64.  Decisions the reference makes with
// sequential f64 sums are taken from parallel sums only when a rigorous
// error bound certifies them; otherwise the finisher replays the
// reference's sequential order on one lane, or reports the row uncertified.
//
// Reference semantics (arclabs561/metallix):
//   nucleus_mask            crates/app/cli/src/qwen_forward.rs:474-549
//   sample_categorical      crates/core/engine/src/sampling.rs:56-158
//   greedy_token            crates/app/cli/src/chat_generation.rs:2213-2231
//   masked_argmax           crates/core/engine/src/constraint.rs:895-932
//   fill_legal_mask         crates/core/engine/src/constraint.rs:793-806
// plus the penalty, bias, min-p and mask-with-nucleus stages this sampler
// defines (see the oracle's orc_sample_row for the executable statement).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/mx_sampler.h"
#include "mxs_math.h"

namespace mxs {

constexpr int NT = 1024;                  // threads per workgroup
constexpr int NW = NT / 64;               // waves per workgroup
constexpr int PER_MAX = 10;               // 4-token quads per thread per chunk
constexpr int SLICE = NT * 4;             // tokens per slice (one quad per thread)
constexpr int CHUNK_MAX = SLICE * PER_MAX;
constexpr int MAXC = 64;                  // chunks per row (vocab <= MAXC * CHUNK_MAX)
constexpr int ECAP = 4096;                // finisher's LDS set capacity
constexpr int KCAND_MAX = ECAP;           // top_k served from per-chunk candidates
constexpr int NB = 2048;                  // radix-select bins (11 bits)
constexpr int HB = 1024;                  // chunk top-k histogram bins
constexpr float HRANGE = 32.0f;           // logit units covered by HB bins
constexpr uint32_t NONE = 0xffffffffu;
constexpr double U = 1.1102230246251565e-16;  // 2^-53

enum Mode : uint32_t { M_GREEDY = 0, M_TOPK = 1, M_MINP = 2, M_ALL = 3, M_KEEPALL = 4 };
enum Flag : uint32_t { F_NONFINITE = 1, F_HIST = 2, F_BIAS = 4 };

struct ChunkStat {
  uint32_t maxkey;     // total-order key of the largest legal logit (0: no legal token)
  uint32_t gbest_id;   // IEEE argmax over legal tokens, lowest ID (NONE: none)
  float gbest_val;
  uint32_t nlegal;
  uint32_t ncand;
  uint32_t flags;
  double mass;         // sum of exp((l - chunk max) / T) over legal tokens, when computed
  uint32_t minkey;     // total-order key of the smallest legal logit
  uint32_t pad;
};

struct Work {
  uint32_t* ctr;       // [max_rows] arrival counters (reset by each finisher)
  ChunkStat* stat;     // [max_rows * MAXC]
  float* cand_l;       // [max_rows * max_vocab]
  uint32_t* cand_id;   // [max_rows * max_vocab]
  double* cand_w;      // [max_rows * max_vocab]
  double* seg;         // [max_rows * MAXC * PER_MAX * NW]
};

struct SampleArgs {
  mxs_batch b;
  mxs_out o;
  Work w;
  uint32_t C;          // chunks per row
  uint32_t per;        // quads per thread per chunk (<= PER_MAX)
  uint32_t CH;         // tokens per chunk (multiple of 4)
};

// ---------------------------------------------------------------------------
// Device-scope (coherent across workgroups and XCDs) loads and stores.  Data
// exchanged between a row's workgroups goes through these: they bypass the
// non-coherent caches, so no L2 writeback/invalidate is needed.
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(double* p, double v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_dev(const double* p) {
  return __hip_atomic_load(const_cast<double*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this lane's outstanding memory operations have completed.
__device__ __forceinline__ void wait_mem() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t lane() { return threadIdx.x & 63; }
__device__ __forceinline__ uint32_t wave() { return threadIdx.x >> 6; }
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// ---------------------------------------------------------------------------
// Block-wide reductions and scans (all threads participate and receive the
// result).  `red` is LDS scratch of at least NW elements of the type.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  for (int o = 32; o > 0; o >>= 1) { T t = __shfl_xor(v, o); v = t > v ? t : v; }
  return v;
}
template <typename T>
__device__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  T s = red[0];
  for (int i = 1; i < NW; ++i) s += red[i];
  __syncthreads();
  return s;
}
template <typename T>
__device__ T block_max(T v, T* red) {
  v = wave_max(v);
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  T s = red[0];
  for (int i = 1; i < NW; ++i) s = red[i] > s ? red[i] : s;
  __syncthreads();
  return s;
}
// Inclusive scan in thread order; *total receives the block total.
template <typename T>
__device__ T block_scan_incl(T v, T* red, T* total) {
  const uint32_t l = lane();
  for (int o = 1; o < 64; o <<= 1) {
    T t = __shfl_up(v, o);
    if (l >= (uint32_t)o) v += t;
  }
  if (l == 63) red[wave()] = v;
  __syncthreads();
  T before = T(0), all = T(0);
  for (int i = 0; i < NW; ++i) {
    T r = red[i];
    if (i < (int)wave()) before += r;
    all += r;
  }
  __syncthreads();
  *total = all;
  return before + v;
}

// IEEE argmax with the lowest index on ties (-0.0 ties 0.0): greedy_token's
// and masked_argmax's rule.
__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
  if (ai == NONE) return false;
  if (bi == NONE) return true;
  return av > bv || (av == bv && ai < bi);
}

// ---------------------------------------------------------------------------
// Shared memory: one static pool, carved per phase.
struct ChunkSmem {
  uint32_t tab[SLICE];                 // per-slice history counts
  uint32_t btab[SLICE];                // per-slice bias slot (index + 1)
  uint32_t hist[HB];                   // top-k threshold histogram
  uint32_t wcnt[PER_MAX * NW];         // candidates per (slice, wave)
  uint32_t woff[PER_MAX * NW];
  uint32_t red_u[NW];
  double red_d[NW];
  float red_f[NW];
  uint32_t red_i[NW];
  uint32_t s_flags;
  uint32_t s_thresh_bin;
  uint32_t s_last;
};
struct FinSmem {
  float e_l[ECAP];
  uint32_t e_id[ECAP];
  double e_w[ECAP];
  unsigned long long skey[ECAP];       // sort keys: (key << 32) | ~id, descending
  uint32_t sidx[ECAP];                 // sort payload: index into e_*
  uint32_t hcnt[NB];
  double hmass[NB];
  ChunkStat st[MAXC];
  double cscale[MAXC];
  uint32_t coff[MAXC + 1];
  uint32_t red_u[NW];
  double red_d[NW];
  float red_f[NW];
  uint32_t red_i[NW];
  uint32_t s_u[8];
  double s_d[8];
};
constexpr size_t SMEM_BYTES = sizeof(FinSmem) > sizeof(ChunkSmem) ? sizeof(FinSmem) : sizeof(ChunkSmem);

// ---------------------------------------------------------------------------
// Per-row parameters and their validation (uniform across the workgroup).
struct RowCfg {
  double T, top_p, min_p, u;
  uint32_t k;
  float rep, pres, freq;
  uint32_t hb, he, bb, be;
  int32_t err;          // parameter error (0 = ok)
  bool greedy;
};

__device__ RowCfg load_cfg(const mxs_batch& b, uint32_t row) {
  RowCfg c;
  c.T = b.temperature[row];
  c.top_p = b.top_p ? b.top_p[row] : 1.0;
  c.min_p = b.min_p ? b.min_p[row] : 0.0;
  c.u = b.uniform ? b.uniform[row] : 0.0;
  c.k = b.top_k ? b.top_k[row] : 0u;
  c.rep = b.repetition ? b.repetition[row] : 1.0f;
  c.pres = b.presence ? b.presence[row] : 0.0f;
  c.freq = b.frequency ? b.frequency[row] : 0.0f;
  c.hb = c.he = c.bb = c.be = 0;
  if (b.history_offsets) { c.hb = b.history_offsets[row]; c.he = b.history_offsets[row + 1]; }
  if (b.bias_offsets) { c.bb = b.bias_offsets[row]; c.be = b.bias_offsets[row + 1]; }
  c.err = 0;
  c.greedy = c.T == 0.0;
  if (!(c.T >= 0.0) || !isfinite(c.T)) c.err = MXS_ROW_INVALID_TEMPERATURE;
  else if (!c.greedy && !(c.top_p > 0.0 && c.top_p <= 1.0)) c.err = MXS_ROW_INVALID_TOP_P;
  else if (!c.greedy && !(c.min_p >= 0.0 && c.min_p <= 1.0)) c.err = MXS_ROW_INVALID_MIN_P;
  else if (!(isfinite(c.rep) && c.rep > 0.0f) || !isfinite(c.pres) || !isfinite(c.freq)) c.err = MXS_ROW_INVALID_PENALTY;
  else if (c.he < c.hb) c.err = MXS_ROW_INVALID_HISTORY;
  else if (c.be < c.bb) c.err = MXS_ROW_INVALID_BIAS;
  return c;
}

// Error precedence after the parameter checks: history ids, bias entries,
// uniform, non-finite adjusted logit, empty support.
__device__ int32_t combine_errors(const RowCfg& c, uint32_t flags, uint32_t nlegal) {
  if (c.err) return c.err;
  if (flags & F_HIST) return MXS_ROW_INVALID_HISTORY;
  if (flags & F_BIAS) return MXS_ROW_INVALID_BIAS;
  if (!c.greedy && (!isfinite(c.u) || !(c.u >= 0.0 && c.u < 1.0))) return MXS_ROW_INVALID_UNIFORM;
  if (flags & F_NONFINITE) return MXS_ROW_NON_FINITE_LOGIT;
  if (nlegal == 0) return MXS_ROW_EMPTY_SUPPORT;
  return 0;
}

__device__ __forceinline__ uint32_t chunk_mode(const RowCfg& c, uint32_t V) {
  if (c.greedy) return M_GREEDY;
  const bool k_act = c.k > 0 && c.k < V;
  if (k_act) return c.k <= (uint32_t)KCAND_MAX ? M_TOPK : M_ALL;
  if (c.min_p > 0.0) return M_MINP;
  if (c.top_p < 1.0) return M_ALL;
  return M_KEEPALL;
}

// Logit-bias and penalty stage for one token (BUILD-DEFINED semantics, f32,
// every operation rounded separately).
__device__ __forceinline__ float adjust(float l, uint32_t cnt, uint32_t slot, const RowCfg& c,
                                       const float* bias_values) {
  if (slot) l = l + bias_values[c.bb + slot - 1];
  if (cnt) {
    l = l < 0.0f ? l * c.rep : l / c.rep;
    const float cf = (float)cnt * c.freq;
    l = l - cf;
    l = l - c.pres;
  }
  return l;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

template <typename In>
struct Quad;
template <>
struct Quad<float> {
  using Raw = float4;
  __device__ static Raw load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ static void unpack(const Raw& r, float x[4]) { x[0] = r.x; x[1] = r.y; x[2] = r.z; x[3] = r.w; }
  __device__ static float one(const float* p) { return *p; }
};
template <>
struct Quad<uint16_t> {
  using Raw = uint2;
  __device__ static Raw load(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ static void unpack(const Raw& r, float x[4]) {
    x[0] = bf16_to_f32((uint16_t)(r.x & 0xffffu)); x[1] = bf16_to_f32((uint16_t)(r.x >> 16));
    x[2] = bf16_to_f32((uint16_t)(r.y & 0xffffu)); x[3] = bf16_to_f32((uint16_t)(r.y >> 16));
  }
  __device__ static float one(const uint16_t* p) { return bf16_to_f32(*p); }
};

// Re-derives adjusted logits and legality for `cnt` tokens starting at `id0`
// (one lane per token, cnt <= 64, one wave).  Used by the finisher to locate
// a draw inside a 256-token segment without the chunk's registers.
template <typename In>
__device__ void rederive_token(const SampleArgs& A, const RowCfg& c, uint32_t row, uint32_t id,
                               float* l_out, bool* legal_out) {
  const mxs_batch& b = A.b;
  const In* p = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;
  float l = Quad<In>::one(p + id);
  uint32_t cnt = 0, slot = 0;
  for (uint32_t h = c.hb; h < c.he; ++h) cnt += b.history_ids[h] == id;
  for (uint32_t j = c.bb; j < c.be; ++j)
    if (b.bias_ids[j] == id) slot = j - c.bb + 1;
  *l_out = adjust(l, cnt, slot, c, b.bias_values);
  bool legal = true;
  if (b.mask_words) {
    const uint32_t w = b.mask_words[(uint64_t)row * b.mask_stride + (id >> 5)];
    legal = ((w >> (id & 31)) & 1u) && id < b.tokenizer_vocab;
  }
  *legal_out = legal;
}

// ---------------------------------------------------------------------------
// Finisher helpers.

// Bitonic sort of n (<= ECAP) descending keys with payload, in LDS.
__device__ void bitonic_sort_desc(unsigned long long* key, uint32_t* idx, uint32_t n) {
  uint32_t np = 1;
  while (np < n) np <<= 1;
  for (uint32_t i = n + threadIdx.x; i < np; i += NT) { key[i] = 0ull; idx[i] = NONE; }
  __syncthreads();
  for (uint32_t size = 2; size <= np; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t t = threadIdx.x; t < np / 2; t += NT) {
        const uint32_t i = 2 * stride * (t / stride) + (t % stride);
        const uint32_t j = i + stride;
        const bool desc = ((i & size) == 0);
        unsigned long long a = key[i], bb = key[j];
        if ((a < bb) == desc) {
          key[i] = bb; key[j] = a;
          uint32_t ti = idx[i]; idx[i] = idx[j]; idx[j] = ti;
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ unsigned long long sort_key(float l, uint32_t id) {
  return ((unsigned long long)okey(l) << 32) | (unsigned long long)(~id);
}

// Sum bound: |computed - reference| for two f64 sums of the same n
// non-negative terms, each term within `term_ulps` ulp of the reference's.
__device__ __forceinline__ double sum_bound(double s, uint32_t n, double term_ulps) {
  return (2.0 * (double)n + term_ulps + 4.0) * U * s * 1.0001 + 1e-300;
}

// ---------------------------------------------------------------------------
// Finisher path for a working set E larger than the LDS capacity: E stays in
// the candidate arrays (global memory, token-ID order) and is filtered by a
// predicate on every pass; the nucleus cut comes from a mass-weighted radix
// select (three 11/11/10-bit passes with LDS count and f64 mass histograms)
// whose bin decisions are certified against the same error bounds.
struct LargeCtx {
  const SampleArgs* A;
  const RowCfg* c;
  uint32_t row, mode, C, ncand, ne, nlegal;
  bool k_path;
  uint32_t kappa, id_tie;
  double M, L, Lclose, total, total_err;
  bool have_total;
};

__device__ __forceinline__ uint64_t cand_pos_of(const FinSmem& F, uint32_t C, uint64_t rbase, uint32_t CH, uint32_t j) {
  uint32_t q = 0;
  while (q + 1 < C && F.coff[q + 1] <= j) ++q;
  return rbase + (uint64_t)q * CH + (j - F.coff[q]);
}

__device__ void finish_large(const LargeCtx& X, FinSmem& F, uint64_t rbase, uint32_t* kbits, uint32_t nwords) {
  const SampleArgs& A = *X.A;
  const RowCfg& c = *X.c;
  const uint32_t tid = threadIdx.x;
  const uint32_t n = X.ncand;
  auto member = [&](float l, uint32_t id) -> bool {
    if (X.k_path) {
      const uint32_t key = okey(l);
      return key > X.kappa || (key == X.kappa && id <= X.id_tie);
    }
    if (X.mode == M_MINP) return (((double)l - X.M) / c.T) >= X.L;
    return true;
  };
  auto finish = [&](int32_t status, int32_t token, double lp, uint32_t kept) {
    if (tid == 0) {
      A.o.token[X.row] = token;
      A.o.status[X.row] = status;
      if (A.o.sampling_logprob) A.o.sampling_logprob[X.row] = lp;
      if (A.o.kept_count) A.o.kept_count[X.row] = kept;
    }
  };
  bool uncert = false;
  // P1: exact weights of E into cand_w (0 for non-members), their sum and minimum.
  double wpart = 0.0, wmin = INFINITY;
  uint32_t bad = 0;
  for (uint32_t j = tid; j < n; j += NT) {
    const uint64_t pos = cand_pos_of(F, X.C, rbase, A.CH, j);
    const float l = ld_dev(&A.w.cand_l[pos]);
    const uint32_t id = ld_dev(&A.w.cand_id[pos]);
    double w = 0.0;
    if (member(l, id)) {
      w = exp_neg(((double)l - X.M) / c.T);
      wmin = fmin(wmin, w);
    }
    st_dev(&A.w.cand_w[pos], w);
    wpart += w;
  }
  const double esum = block_sum<double>(wpart, F.red_d);
  wmin = -block_max<double>(-wmin, F.red_d);
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, X.ne, 8.0); }

  // P2: nucleus threshold (tau, id_cut): member kept iff key > tau or (key == tau and id <= id_cut).
  uint32_t tau = 0, id_cut = NONE;   // default: every member
  bool cut = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      // covered reaches kept only at the last head token when every weight
      // is large enough to change the running f64 sum.
      if (!(wmin > 2.3e-16 * esum)) uncert = true;
    } else {
      cut = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, X.ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
    cut = !(esum + sum_bound(esum, X.ne, 8.0) < theta - theta_err);
  }
  if (cut) {
    uint32_t prefix = 0, pmask = 0, above_n = 0;
    double above = 0.0;
    const int shifts[3] = {21, 10, 0};
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass];
      for (uint32_t t = tid; t < (uint32_t)NB; t += NT) { F.hcnt[t] = 0u; F.hmass[t] = 0.0; }
      __syncthreads();
      for (uint32_t j = tid; j < n; j += NT) {
        const uint64_t pos = cand_pos_of(F, X.C, rbase, A.CH, j);
        const float l = ld_dev(&A.w.cand_l[pos]);
        const uint32_t id = ld_dev(&A.w.cand_id[pos]);
        const uint32_t key = okey(l);
        if ((key & pmask) == prefix && member(l, id)) {
          const uint32_t bin = (key >> sh) & (NB - 1);
          atomicAdd(&F.hcnt[bin], 1u);
          atomicAdd(&F.hmass[bin], ld_dev(&A.w.cand_w[pos]));
        }
      }
      __syncthreads();
      const uint32_t b_hi = NB - 1 - 2 * tid, b_lo = b_hi - 1;
      const double mh = F.hmass[b_hi], ml = F.hmass[b_lo];
      const uint32_t nh = F.hcnt[b_hi], nl = F.hcnt[b_lo];
      double mtot;
      uint32_t ntot;
      const double minc = above + block_scan_incl<double>(mh + ml, F.red_d, &mtot);
      const uint32_t ninc = above_n + block_scan_incl<uint32_t>(nh + nl, F.red_u, &ntot);
      const double mexc = minc - mh - ml;
      const uint32_t nexc = ninc - nh - nl;
      if (tid == 0) { F.s_u[4] = NONE; F.s_u[6] = 0u; }
      __syncthreads();
      // the bin where the descending cumulative mass first reaches theta
      const double e1 = sum_bound(mexc + mh, nexc + nh + 64u, 8.0);
      if (nh && mexc < theta && theta <= mexc + mh) {
        F.s_u[4] = b_hi; F.s_u[5] = nexc; F.s_d[4] = mexc;
        const double e0 = sum_bound(mexc, nexc + 64u, 8.0);
        if (!(mexc + e0 < theta - theta_err) || !(mexc + mh - e1 >= theta + theta_err)) F.s_u[6] = 1u;
      } else if (nl && mexc + mh < theta && theta <= minc) {
        F.s_u[4] = b_lo; F.s_u[5] = nexc + nh; F.s_d[4] = mexc + mh;
        const double e2 = sum_bound(minc, ninc + 64u, 8.0);
        if (!(mexc + mh + e1 < theta - theta_err) || !(minc - e2 >= theta + theta_err)) F.s_u[6] = 1u;
      }
      __syncthreads();
      if (F.s_u[4] == NONE) {
        // theta beyond the accumulated mass (rounding): keep every member
        cut = false;
        uncert = true;
        __syncthreads();
        break;
      }
      if (F.s_u[6]) uncert = true;
      prefix |= F.s_u[4] << sh;
      pmask |= (uint32_t)(NB - 1) << sh;
      above = F.s_d[4];
      above_n = F.s_u[5];
      __syncthreads();
    }
    if (cut) {
      tau = prefix;
      // ties at tau share one weight; the reference adds them one by one
      const double wt = exp_neg(((double)okey_value(tau) - X.M) / c.T);
      if (tid == 0) {
        uint32_t jn = 0;
        double cov = above;
        bool close = false;
        for (uint32_t q = 0; q < 1000000u; ++q) {
          cov += wt;
          ++jn;
          const double e = sum_bound(cov, above_n + jn + 64u, 8.0);
          if (fabs(cov - theta) <= e + theta_err) close = true;
          if (cov >= theta || !(wt > 0.0)) break;
        }
        F.s_u[6] = jn;
        F.s_u[7] = close ? 1u : 0u;
      }
      __syncthreads();
      const uint32_t jneed = F.s_u[6];
      if (F.s_u[7]) uncert = true;
      __syncthreads();
      // id of the jneed-th member with key == tau, in ID order
      uint32_t seen = 0;
      if (tid == 0) F.s_u[3] = NONE;
      __syncthreads();
      for (uint32_t base = 0; base < n; base += NT) {
        const uint32_t j = base + tid;
        bool tie = false;
        uint32_t id = 0;
        if (j < n) {
          const uint64_t pos = cand_pos_of(F, X.C, rbase, A.CH, j);
          const float l = ld_dev(&A.w.cand_l[pos]);
          id = ld_dev(&A.w.cand_id[pos]);
          tie = okey(l) == tau && member(l, id);
        }
        uint32_t tt;
        const uint32_t ti = block_scan_incl<uint32_t>(tie ? 1u : 0u, F.red_u, &tt);
        if (tie && seen + ti == jneed) F.s_u[3] = id;
        seen += tt;
      }
      __syncthreads();
      id_cut = F.s_u[3];
      if (id_cut == NONE) { id_cut = 0xfffffffeu; uncert = true; }
      __syncthreads();
    }
  }

  // P3: kept = member, inside the nucleus cut, and (unless E is already the
  // min-p set) at or above ln(min_p).  Draw in token-ID order.
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  auto kept_w = [&](uint32_t j, uint32_t* id_out, double* s_out) -> double {
    const uint64_t pos = cand_pos_of(F, X.C, rbase, A.CH, j);
    const float l = ld_dev(&A.w.cand_l[pos]);
    const uint32_t id = ld_dev(&A.w.cand_id[pos]);
    *id_out = id;
    *s_out = ((double)l - X.M) / c.T;
    if (!member(l, id)) return -1.0;
    if (cut) {
      const uint32_t key = okey(l);
      if (!(key > tau || (key == tau && id <= id_cut))) return -1.0;
    }
    if (apply_minp && !(*s_out >= X.L)) return -1.0;
    return ld_dev(&A.w.cand_w[pos]);
  };
  double kpart = 0.0;
  uint32_t kn = 0, close = 0;
  for (uint32_t j = tid; j < n; j += NT) {
    uint32_t id;
    double s;
    const double w = kept_w(j, &id, &s);
    if (apply_minp && fabs(s - X.L) < X.Lclose) close = 1;
    if (w >= 0.0) { kpart += w; ++kn; if (!isfinite(s)) bad = 1; }
  }
  if (block_max<uint32_t>(bad, F.red_u)) { finish(MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
  if (block_max<uint32_t>(close, F.red_u)) uncert = true;
  const double S = block_sum<double>(kpart, F.red_d);
  const uint32_t nkept = block_sum<uint32_t>(kn, F.red_u);
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
  __syncthreads();
  double run = 0.0;
  for (uint32_t base = 0; base < n; base += NT) {
    const uint32_t j = base + tid;
    uint32_t id = 0;
    double s = 0.0, w = 0.0;
    if (j < n) {
      const double kw = kept_w(j, &id, &s);
      w = kw > 0.0 ? kw : 0.0;
    }
    double tot;
    const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
    const double exc = inc - w;
    if (w > 0.0) {
      atomicMax(&F.s_u[1], j + 1u);
      if (target < inc && !(target < exc)) {
        F.s_u[0] = j;
        F.s_d[0] = s;
        if (fabs(target - exc) <= derr || fabs(inc - target) <= derr) F.s_u[2] = 1u;
      }
    }
    run += tot;
  }
  __syncthreads();
  uint32_t pick = F.s_u[0];
  if (F.s_u[2]) uncert = true;
  double shifted = F.s_d[0];
  if (pick == NONE) {
    uncert = true;
    pick = F.s_u[1] ? F.s_u[1] - 1u : NONE;
    if (pick != NONE) {
      uint32_t id;
      kept_w(pick, &id, &shifted);
    }
  }
  __syncthreads();
  if (pick == NONE) { finish(MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  uint32_t tok;
  double sh2;
  kept_w(pick, &tok, &sh2);
  finish(uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)tok, shifted - log(S), nkept);
  if (kbits) {
    for (uint32_t q = tid; q < nwords; q += NT) kbits[q] = 0u;
    __syncthreads();
    for (uint32_t j = tid; j < n; j += NT) {
      uint32_t id;
      double s;
      if (kept_w(j, &id, &s) >= 0.0) atomicOr(&kbits[id >> 5], 1u << (id & 31u));
    }
  }
}

// ---------------------------------------------------------------------------
// The row finisher.  Runs in the last chunk workgroup of a row, after every
// chunk published its statistics and candidates.
template <typename In>
__device__ void finish_row(const SampleArgs& A, FinSmem& F, const RowCfg& c, uint32_t row, uint32_t mode,
                           uint64_t rbase, double invT) {
  const mxs_batch& b = A.b;
  const uint32_t tid = threadIdx.x;
  const uint32_t V = b.vocab;
  const uint32_t C = A.C;
  if (tid == 0) st_dev(&A.w.ctr[row], 0u);   // ready for the next launch
  for (uint32_t q = tid; q < C; q += NT) {
    const ChunkStat* st = &A.w.stat[(uint64_t)row * MAXC + q];
    ChunkStat v;
    v.maxkey = ld_dev(&st->maxkey);
    v.gbest_id = ld_dev(&st->gbest_id);
    v.gbest_val = ld_dev(&st->gbest_val);
    v.nlegal = ld_dev(&st->nlegal);
    v.ncand = ld_dev(&st->ncand);
    v.flags = ld_dev(&st->flags);
    v.mass = ld_dev(&st->mass);
    v.minkey = ld_dev(&st->minkey);
    F.st[q] = v;
  }
  __syncthreads();
  uint32_t flags = 0, nlegal = 0, Mkey = 0;
  float bv = 0.0f;
  uint32_t bi = NONE;
  for (uint32_t q = 0; q < C; ++q) {
    const ChunkStat& v = F.st[q];
    flags |= v.flags;
    nlegal += v.nlegal;
    if (v.nlegal && v.maxkey > Mkey) Mkey = v.maxkey;
    if (better(v.gbest_val, v.gbest_id, bv, bi)) { bv = v.gbest_val; bi = v.gbest_id; }
  }
  const double M = (double)okey_value(Mkey);
  if (tid == 0) {
    uint32_t run = 0;
    for (uint32_t q = 0; q < C; ++q) {
      F.coff[q] = run;
      run += F.st[q].ncand;
      F.cscale[q] = F.st[q].nlegal ? exp_neg(((double)okey_value(F.st[q].maxkey) - M) * invT) : 0.0;
    }
    F.coff[C] = run;
  }
  __syncthreads();
  const int32_t err = combine_errors(c, flags, nlegal);
  const uint32_t nwords = (V + 31u) / 32u;
  uint32_t* kbits = A.o.kept_bits ? A.o.kept_bits + (uint64_t)row * nwords : nullptr;
  auto finish = [&](int32_t status, int32_t token, double lp, uint32_t kept) {
    if (tid == 0) {
      A.o.token[row] = token;
      A.o.status[row] = status;
      if (A.o.sampling_logprob) A.o.sampling_logprob[row] = lp;
      if (A.o.kept_count) A.o.kept_count[row] = kept;
    }
  };
  if (err) {
    finish(err, -1, 0.0, 0u);
    if (kbits)
      for (uint32_t q = tid; q < nwords; q += NT) kbits[q] = 0u;
    return;
  }
  if (mode == M_GREEDY) {
    finish(0, (int32_t)bi, 0.0, 1u);
    if (kbits)
      for (uint32_t q = tid; q < nwords; q += NT) kbits[q] = (q == (bi >> 5)) ? (1u << (bi & 31u)) : 0u;
    return;
  }
  const bool k_act = c.k > 0 && c.k < nlegal;

  // =================== KEEPALL: every legal token, ID order ===============
  if (mode == M_KEEPALL) {
    uint32_t mink = NONE;
    for (uint32_t q = 0; q < C; ++q)
      if (F.st[q].nlegal && F.st[q].minkey < mink) mink = F.st[q].minkey;
    if (!isfinite(((double)okey_value(mink) - M) / c.T)) { finish(MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
    const uint32_t segs_per_chunk = A.per * NW;
    const uint32_t nseg = C * segs_per_chunk;
    // total mass
    double part = 0.0;
    for (uint32_t s = tid; s < nseg; s += NT) {
      const uint32_t q = s / segs_per_chunk, r = s % segs_per_chunk;
      if (F.st[q].nlegal) part += ld_dev(&A.w.seg[((uint64_t)row * MAXC + q) * PER_MAX * NW + r]) * F.cscale[q];
    }
    const double total = block_sum<double>(part, F.red_d);
    const double target = c.u * total;
    // Bound: each segment mass carries the x = (l - m) / T product rounding
    // (x e^x <= 1/e per token) and 8 ulp per weight; plus the scale factors.
    const double err_b = sum_bound(total, nlegal + nseg, 12.0) + 2.0 * 0.37 * (double)nlegal * U;
    if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
    __syncthreads();
    double run = 0.0;
    for (uint32_t base = 0; base < nseg; base += NT) {
      const uint32_t s = base + tid;
      double w = 0.0;
      if (s < nseg) {
        const uint32_t q = s / segs_per_chunk, r = s % segs_per_chunk;
        if (F.st[q].nlegal) w = ld_dev(&A.w.seg[((uint64_t)row * MAXC + q) * PER_MAX * NW + r]) * F.cscale[q];
      }
      double tot;
      const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
      const double exc = inc - w;
      if (w > 0.0) {
        atomicMax(&F.s_u[1], s + 1u);
        if (target < inc && !(target < exc)) {
          F.s_u[0] = s;
          F.s_d[0] = exc;
          if (fabs(target - exc) <= err_b || fabs(inc - target) <= err_b) F.s_u[2] = 1u;
        }
      }
      run += tot;
    }
    __syncthreads();
    uint32_t seg = F.s_u[0];
    bool near = F.s_u[2] != 0u;
    double before = F.s_d[0];
    if (seg == NONE) {
      // rounding left the variate past the accumulated mass
      seg = F.s_u[1] ? F.s_u[1] - 1u : NONE;
      near = true;
      before = -INFINITY;   // forces the last positive token of the segment
    }
    if (seg == NONE) { finish(MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
    if (wave() == 0) {
      const uint32_t q = seg / segs_per_chunk, r = seg % segs_per_chunk;
      const uint32_t i = r / NW, w = r % NW;
      const uint32_t q1 = min(V, q * A.CH + A.CH);
      const uint32_t id0 = q * A.CH + i * SLICE + w * 256u + lane() * 4u;
      double wl[4];
      double sh[4];
      double lsum = 0.0;
      for (int e = 0; e < 4; ++e) {
        const uint32_t id = id0 + (uint32_t)e;
        wl[e] = 0.0;
        sh[e] = 0.0;
        if (id < q1) {
          float l;
          bool lg;
          rederive_token<In>(A, c, row, id, &l, &lg);
          if (lg) { sh[e] = ((double)l - M) / c.T; wl[e] = exp_neg(sh[e]); }
        }
        lsum += wl[e];
      }
      double inc = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane() >= (uint32_t)o) inc += t;
      }
      double cum = (before == -INFINITY ? 0.0 : before) + inc - lsum;
      uint32_t found = NONE, lastpos = NONE;
      double fsh = 0.0, lsh = 0.0;
      bool fnear = false;
      for (int e = 0; e < 4; ++e) {
        const double prev = cum;
        cum += wl[e];
        if (wl[e] > 0.0) {
          lastpos = id0 + (uint32_t)e;
          lsh = sh[e];
          if (before != -INFINITY && found == NONE && target < cum && !(target < prev)) {
            found = id0 + (uint32_t)e;
            fsh = sh[e];
            fnear = fabs(target - prev) <= err_b || fabs(cum - target) <= err_b;
          }
        }
      }
      const uint64_t fb = __ballot(found != NONE);
      const uint64_t lb = __ballot(lastpos != NONE);
      uint32_t tok = NONE;
      double tsh = 0.0;
      bool tnear = true;
      if (fb) {
        const int sl = __ffsll((unsigned long long)fb) - 1;
        tok = __shfl(found, sl);
        tsh = __shfl(fsh, sl);
        tnear = __shfl(fnear ? 1 : 0, sl) != 0;
      } else if (lb) {
        const int sl = 63 - __clzll((long long)lb);
        tok = __shfl(lastpos, sl);
        tsh = __shfl(lsh, sl);
      }
      if (lane() == 0) { F.s_u[3] = tok; F.s_d[1] = tsh; F.s_u[4] = tnear ? 1u : 0u; }
    }
    __syncthreads();
    const uint32_t tok = F.s_u[3];
    if (tok == NONE) { finish(MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
    near = near || F.s_u[4] != 0u;
    finish(near ? MXS_ROW_UNCERTIFIED : 0, (int32_t)tok, F.s_d[1] - log(total), nlegal);
    if (kbits) {
      for (uint32_t q = tid; q < nwords; q += NT) {
        uint32_t wv = 0xffffffffu;
        if (q == nwords - 1 && (V & 31u)) wv = (1u << (V & 31u)) - 1u;
        if (b.mask_words) {
          wv &= b.mask_words[(uint64_t)row * b.mask_stride + q];
          const uint32_t tv = b.tokenizer_vocab;
          if (q * 32u >= tv) wv = 0u;
          else if (q * 32u + 32u > tv) wv &= (1u << (tv - q * 32u)) - 1u;
        }
        kbits[q] = wv;
      }
    }
    return;
  }

  // =================== candidate paths ====================================
  const uint32_t ncand_total = F.coff[C];
  auto cand_pos = [&](uint32_t j) -> uint64_t {
    uint32_t q = 0;
    while (q + 1 < C && F.coff[q + 1] <= j) ++q;
    return rbase + (uint64_t)q * A.CH + (j - F.coff[q]);
  };
  const double L = c.min_p > 0.0 ? log(c.min_p) : -INFINITY;
  // ln(min_p) is exact for min_p = 1 (and -inf for 0); otherwise device and
  // host logs may differ in the last ulps, so a shifted logit within 4 ulp is
  // an uncertain cut.
  const double Lclose = (c.min_p > 0.0 && c.min_p < 1.0) ? 4.0 * U * fabs(L) : 0.0;

  // total = sum over every legal token of exp((l - M) / T), from chunk masses
  double total = 0.0, total_err = 0.0;
  bool have_total = false;
  if (c.top_p < 1.0 && !k_act && (mode == M_MINP || mode == M_ALL || (mode == M_TOPK && b.mask_words))) {
    for (uint32_t q = 0; q < C; ++q) total += F.st[q].mass * F.cscale[q];
    total_err = sum_bound(total, nlegal + C, 12.0) + 2.0 * 0.37 * (double)nlegal * U;
    have_total = true;
  }

  // top-k head: kappa = the k-th largest key, ties_needed = how many
  // candidates with key == kappa join it, lowest IDs first.
  uint32_t kappa = 0, ties_needed = 0;
  const bool k_path = k_act && (mode == M_TOPK || mode == M_ALL);
  if (k_path) {
    uint32_t prefix = 0, pmask = 0, above = 0;
    const int shifts[3] = {21, 10, 0};
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass];
      for (uint32_t t = tid; t < (uint32_t)NB; t += NT) F.hcnt[t] = 0u;
      __syncthreads();
      for (uint32_t j = tid; j < ncand_total; j += NT) {
        const uint32_t key = okey(ld_dev(&A.w.cand_l[cand_pos(j)]));
        if ((key & pmask) == prefix) atomicAdd(&F.hcnt[(key >> sh) & (NB - 1)], 1u);
      }
      __syncthreads();
      const uint32_t b_hi = NB - 1 - 2 * tid, b_lo = b_hi - 1;
      const uint32_t ch = F.hcnt[b_hi], cl = F.hcnt[b_lo];
      uint32_t tot;
      const uint32_t inc = block_scan_incl<uint32_t>(ch + cl, F.red_u, &tot);
      const uint32_t exc = inc - ch - cl;
      const uint32_t need = c.k - above;
      if (exc < need && need <= exc + ch) { F.s_u[4] = b_hi; F.s_u[5] = above + exc; }
      else if (exc + ch < need && need <= inc) { F.s_u[4] = b_lo; F.s_u[5] = above + exc + ch; }
      __syncthreads();
      prefix |= F.s_u[4] << sh;
      pmask |= (uint32_t)(NB - 1) << sh;
      above = F.s_u[5];
      __syncthreads();
    }
    kappa = prefix;
    ties_needed = c.k - above;
  }

  // ---- working set E in LDS, token-ID order -------------------------------
  // E = the head (k path), the exact min-p set (MINP), or every candidate.
  uint32_t ne = 0, tie_seen = 0;
  bool mp_close = false;
  if (tid == 0) F.s_u[7] = NONE;
  __syncthreads();
  for (uint32_t base = 0; base < ncand_total; base += NT) {
    const uint32_t j = base + tid;
    float l = 0.0f;
    uint32_t id = 0;
    bool in = false, tie = false;
    if (j < ncand_total) {
      const uint64_t pos = cand_pos(j);
      l = ld_dev(&A.w.cand_l[pos]);
      id = ld_dev(&A.w.cand_id[pos]);
      if (k_path) {
        const uint32_t key = okey(l);
        in = key > kappa;
        tie = key == kappa;
      } else if (mode == M_MINP) {
        const double s = ((double)l - M) / c.T;
        in = s >= L;
        if (fabs(s - L) < Lclose) mp_close = true;
      } else {
        in = true;
      }
    }
    uint32_t ttot;
    const uint32_t tinc = block_scan_incl<uint32_t>(tie ? 1u : 0u, F.red_u, &ttot);
    if (tie && tie_seen + tinc <= ties_needed) in = true;
    if (tie && tie_seen + tinc == ties_needed) F.s_u[7] = id;
    tie_seen += ttot;
    uint32_t etot;
    const uint32_t einc = block_scan_incl<uint32_t>(in ? 1u : 0u, F.red_u, &etot);
    if (in && ne + einc - 1u < (uint32_t)ECAP) {
      F.e_l[ne + einc - 1u] = l;
      F.e_id[ne + einc - 1u] = id;
    }
    ne += etot;
  }
  __syncthreads();
  if (block_max<uint32_t>(mp_close ? 1u : 0u, F.red_u)) mp_close = true;
  if (ne > (uint32_t)ECAP) {
    LargeCtx X;
    X.A = &A; X.c = &c; X.row = row; X.mode = mode; X.C = C; X.ncand = ncand_total; X.ne = ne;
    X.nlegal = nlegal; X.k_path = k_path; X.kappa = kappa; X.id_tie = F.s_u[7];
    X.M = M; X.L = L; X.Lclose = Lclose; X.total = total; X.total_err = total_err; X.have_total = have_total;
    __syncthreads();
    finish_large(X, F, rbase, kbits, nwords);
    if (mp_close && tid == 0 && A.o.status[row] == 0) A.o.status[row] = MXS_ROW_UNCERTIFIED;
    return;
  }

  // weights
  double wpart = 0.0;
  for (uint32_t t = tid; t < ne; t += NT) {
    const double s = ((double)F.e_l[t] - M) / c.T;
    const double w = exp_neg(s);
    F.e_w[t] = w;
    wpart += w;
  }
  const double esum = block_sum<double>(wpart, F.red_d);
  if (!have_total && !k_path && mode != M_MINP) {
    total = esum;   // E holds every legal token
    total_err = sum_bound(total, ne, 8.0);
    have_total = true;
  }

  // ---- nucleus over E in (key desc, ID asc) order -------------------------
  bool uncert = false;
  uint32_t n_keep = ne;
  bool walk = false;
  double theta = 0.0, theta_err = 0.0;
  if (k_path) {
    walk = true;
    theta = c.top_p * esum;
    theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
  } else if (c.top_p < 1.0) {
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
    walk = !(esum + sum_bound(esum, ne, 8.0) < theta - theta_err);   // else the nucleus covers E
  }
  if (walk) {
    for (uint32_t t = tid; t < ne; t += NT) { F.skey[t] = sort_key(F.e_l[t], F.e_id[t]); F.sidx[t] = t; }
    __syncthreads();
    bitonic_sort_desc(F.skey, F.sidx, ne);
    bool replay = false;
    if (k_path && c.top_p >= 1.0) {
      // covered reaches kept only at the last head token when every weight
      // is large enough to change the running f64 sum; otherwise replay.
      double wmin_part = INFINITY;
      for (uint32_t t = tid; t < ne; t += NT) wmin_part = fmin(wmin_part, F.e_w[t]);
      const double wmin = -block_max<double>(-wmin_part, F.red_d);
      if (wmin > 2.3e-16 * esum) n_keep = ne;
      else replay = true;
    }
    const bool freeze_done = k_path && c.top_p >= 1.0 && !replay;
    if (!replay && !freeze_done) {
      // first sorted position not certainly below theta
      if (tid == 0) { F.s_u[6] = NONE; F.s_u[7] = 0u; }
      __syncthreads();
      double run = 0.0;
      for (uint32_t base = 0; base < ne; base += NT) {
        const uint32_t t = base + tid;
        const double w = t < ne ? F.e_w[F.sidx[t]] : 0.0;
        double tot;
        const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
        const double exc = inc - w;
        if (t < ne) {
          const double e_inc = sum_bound(inc, t + 65u, 8.0);
          const double e_exc = sum_bound(exc, t + 64u, 8.0);
          const bool lt = inc + e_inc < theta - theta_err;
          if (!lt) {
            const bool prev_lt = t == 0 || exc + e_exc < theta - theta_err;
            if (prev_lt) {
              F.s_u[6] = t;   // unique: the first position not certainly below
              if (!(inc - e_inc >= theta + theta_err)) F.s_u[7] = 1u;
            } else if (t == 0 || !(exc - e_exc >= theta + theta_err)) {
              // previous position is ambiguous as well
              atomicOr(&F.s_u[7], 2u);
            }
          }
        }
        run += tot;
      }
      __syncthreads();
      if (F.s_u[6] == NONE || F.s_u[7]) replay = true;
      else n_keep = F.s_u[6] + 1u;
      __syncthreads();
    }
    if (replay) {
      // The reference's sequential f64 sums in descending order, one lane.
      if (tid == 0) {
        double th = theta;
        if (k_path) {
          double kept = 0.0;
          for (uint32_t q = 0; q < ne; ++q) kept += F.e_w[F.sidx[q]];
          th = c.top_p * kept;
        }
        double cov = 0.0;
        uint32_t nk = ne;
        uint32_t close = 0;
        for (uint32_t q = 0; q < ne; ++q) {
          cov += F.e_w[F.sidx[q]];
          if (!k_path && fabs(cov - th) <= theta_err + sum_bound(cov, q + 1, 8.0)) close = 1;
          if (cov >= th) { nk = q + 1; break; }
        }
        F.s_u[6] = nk;
        F.s_u[7] = close;
      }
      __syncthreads();
      n_keep = F.s_u[6];
      if (F.s_u[7]) uncert = true;
      __syncthreads();
    }
    // flags by E index: kept iff sorted position < n_keep
    for (uint32_t t = tid; t < ne; t += NT) F.skey[t] = 0ull;
    __syncthreads();
    for (uint32_t t = tid; t < n_keep; t += NT) F.skey[F.sidx[t]] = 1ull;
    __syncthreads();
  } else {
    for (uint32_t t = tid; t < ne; t += NT) F.skey[t] = 1ull;
    __syncthreads();
  }

  // ---- min-p after the nucleus (E is already the min-p set under MINP) ----
  if (c.min_p > 0.0 && mode != M_MINP) {
    for (uint32_t t = tid; t < ne; t += NT) {
      const double s = ((double)F.e_l[t] - M) / c.T;
      if (fabs(s - L) < Lclose) mp_close = true;
      if (F.skey[t] && !(s >= L)) F.skey[t] = 0ull;
    }
    __syncthreads();
  }
  if (block_max<uint32_t>(mp_close ? 1u : 0u, F.red_u)) uncert = true;
  {
    // sample_categorical rejects a kept token whose shifted logit overflows
    uint32_t bad = 0;
    for (uint32_t t = tid; t < ne; t += NT)
      if (F.skey[t] && !isfinite(((double)F.e_l[t] - M) / c.T)) bad = 1;
    if (block_max<uint32_t>(bad, F.red_u)) { finish(MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
  }

  // ---- inverse-CDF draw over the kept set, token-ID order -----------------
  double kpart = 0.0;
  uint32_t kn = 0;
  for (uint32_t t = tid; t < ne; t += NT)
    if (F.skey[t]) { kpart += F.e_w[t]; ++kn; }
  const double S = block_sum<double>(kpart, F.red_d);
  const uint32_t nkept = block_sum<uint32_t>(kn, F.red_u);
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
  __syncthreads();
  double run = 0.0;
  for (uint32_t base = 0; base < ne; base += NT) {
    const uint32_t t = base + tid;
    const bool kept = t < ne && F.skey[t] != 0ull;
    const double w = kept ? F.e_w[t] : 0.0;
    double tot;
    const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
    const double exc = inc - w;
    if (w > 0.0) {
      atomicMax(&F.s_u[1], t + 1u);
      if (target < inc && !(target < exc)) {
        F.s_u[0] = t;
        if (fabs(target - exc) <= derr || fabs(inc - target) <= derr) F.s_u[2] = 1u;
      }
    }
    run += tot;
  }
  __syncthreads();
  uint32_t pick = F.s_u[0];
  if (F.s_u[2]) uncert = true;
  if (pick == NONE) {
    pick = F.s_u[1] ? F.s_u[1] - 1u : NONE;   // last positive-weight kept token
    uncert = true;
  }
  if (pick == NONE) { finish(MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  const double shifted = ((double)F.e_l[pick] - M) / c.T;
  finish(uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)F.e_id[pick], shifted - log(S), nkept);
  if (kbits) {
    for (uint32_t q = tid; q < nwords; q += NT) kbits[q] = 0u;
    __syncthreads();
    for (uint32_t t = tid; t < ne; t += NT)
      if (F.skey[t]) atomicOr(&kbits[F.e_id[t] >> 5], 1u << (F.e_id[t] & 31u));
  }
}

// ---------------------------------------------------------------------------
// The sampling kernel.
template <typename In>
__global__ __launch_bounds__(NT) void sample_kernel(SampleArgs A) {
  __shared__ __align__(16) unsigned char smem_raw[SMEM_BYTES];
  ChunkSmem& S = *reinterpret_cast<ChunkSmem*>(smem_raw);
  FinSmem& F = *reinterpret_cast<FinSmem*>(smem_raw);
  const mxs_batch& b = A.b;
  const uint32_t tid = threadIdx.x;

  // Workgroup -> (row, chunk): the chunks of one row share an XCD (workgroup
  // IDs are dealt to the 8 XCDs round robin), so their exchange stays local.
  const uint32_t bid = blockIdx.x;
  const uint32_t xcd = bid & 7u, j8 = bid >> 3;
  const uint32_t row = (j8 / A.C) * 8u + xcd;
  const uint32_t chunk = j8 % A.C;
  if (row >= b.rows) return;

  const uint32_t V = b.vocab;
  const RowCfg c = load_cfg(b, row);
  const uint32_t mode = chunk_mode(c, V);
  const uint32_t c0 = chunk * A.CH;
  const uint32_t c1 = min(V, c0 + A.CH);
  const In* src = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;
  const double invT = c.greedy ? 0.0 : 1.0 / c.T;
  const bool has_tab = (c.he > c.hb) || (c.be > c.bb);

  // ---- stream the chunk: every load issued before any use ----------------
  typename Quad<In>::Raw raw[PER_MAX];
#pragma unroll
  for (int i = 0; i < PER_MAX; ++i) {
    if (i < (int)A.per && !c.err) {
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
      // A quad starting below the chunk end lies inside the row stride (a
      // multiple of 4); past the end, re-read the chunk's first quad.
      raw[i] = Quad<In>::load(src + (e0 < c1 ? e0 : c0));
    }
  }
  if (tid == 0) S.s_flags = 0;
  if (has_tab) {
    for (uint32_t t = tid; t < (uint32_t)SLICE; t += NT) { S.tab[t] = 0u; S.btab[t] = 0u; }
  }
  __syncthreads();

  // ---- bias, penalties, mask, finite check, chunk statistics -------------
  float lv[PER_MAX][4];
  uint64_t lbits = 0;                 // bit 4i+e: token (i, e) is legal
  uint32_t my_flags = 0;
  uint32_t maxkey = 0, nleg = 0;
  float gv = 0.0f;
  uint32_t gi = NONE;
  uint32_t tmaxkey = 0;               // this thread's largest legal key
  uint32_t tminkey = NONE;            // and smallest
#pragma unroll
  for (int i = 0; i < PER_MAX; ++i) {
    if (i < (int)A.per && !c.err) {
      const uint32_t sbase = c0 + (uint32_t)i * SLICE;
      const uint32_t send = min(c1, sbase + (uint32_t)SLICE);
      uint4 tv = make_uint4(0u, 0u, 0u, 0u), bv4 = make_uint4(0u, 0u, 0u, 0u);
      if (has_tab) {
        for (uint32_t h = c.hb + tid; h < c.he; h += NT) {
          const uint32_t id = b.history_ids[h];
          if (i == 0 && id >= V) my_flags |= F_HIST;
          if (id >= sbase && id < send) atomicAdd(&S.tab[id - sbase], 1u);
        }
        for (uint32_t jb = c.bb + tid; jb < c.be; jb += NT) {
          const uint32_t id = b.bias_ids[jb];
          if (i == 0) {
            if (id >= V || !isfinite(b.bias_values[jb]) || (jb > c.bb && b.bias_ids[jb - 1] >= id)) my_flags |= F_BIAS;
          }
          if (id >= sbase && id < send) S.btab[id - sbase] = jb - c.bb + 1u;
        }
        __syncthreads();
        tv = *reinterpret_cast<uint4*>(&S.tab[tid * 4u]);
        bv4 = *reinterpret_cast<uint4*>(&S.btab[tid * 4u]);
        *reinterpret_cast<uint4*>(&S.tab[tid * 4u]) = make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(&S.btab[tid * 4u]) = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
      }
      const uint32_t e0 = sbase + tid * 4u;
      float x[4];
      Quad<In>::unpack(raw[i], x);
      uint32_t mword = NONE;
      if (b.mask_words && e0 < c1) mword = b.mask_words[(uint64_t)row * b.mask_stride + (e0 >> 5)];
      const uint32_t tva[4] = {tv.x, tv.y, tv.z, tv.w};
      const uint32_t bva[4] = {bv4.x, bv4.y, bv4.z, bv4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t id = e0 + (uint32_t)e;
        float l = x[e];
        if (tva[e] | bva[e]) l = adjust(l, tva[e], bva[e], c, b.bias_values);
        lv[i][e] = l;
        if (id < c1) {
          if (!isfinite(l)) my_flags |= F_NONFINITE;
          if (A.o.adjusted) A.o.adjusted[(uint64_t)row * V + id] = l;
          bool legal = true;
          if (b.mask_words) legal = ((mword >> (id & 31u)) & 1u) && id < b.tokenizer_vocab;
          if (legal) {
            lbits |= 1ull << (i * 4 + e);
            ++nleg;
            const uint32_t k = okey(l);
            tmaxkey = k > tmaxkey ? k : tmaxkey;
            tminkey = k < tminkey ? k : tminkey;
            if (better(l, id, gv, gi)) { gv = l; gi = id; }
          }
        }
      }
    }
  }

  // Block reductions.
  if (my_flags) atomicOr(&S.s_flags, my_flags);
  maxkey = block_max<uint32_t>(tmaxkey, S.red_u);
  const uint32_t minkey = ~block_max<uint32_t>(~tminkey, S.red_u);
  nleg = block_sum<uint32_t>(nleg, S.red_u);
  {
    // argmax: reduce within the wave, then across waves
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(gv, o);
      const uint32_t oi = __shfl_xor(gi, o);
      if (better(ov, oi, gv, gi)) { gv = ov; gi = oi; }
    }
    if (lane() == 0) { S.red_f[wave()] = gv; S.red_i[wave()] = gi; }
    __syncthreads();
    gv = S.red_f[0]; gi = S.red_i[0];
    for (int w = 1; w < NW; ++w)
      if (better(S.red_f[w], S.red_i[w], gv, gi)) { gv = S.red_f[w]; gi = S.red_i[w]; }
    __syncthreads();
  }
  const uint32_t cflags = S.s_flags;
  const float m = nleg ? okey_value(maxkey) : 0.0f;   // chunk's largest legal logit
  const double md = (double)m;
  const bool row_ok = !c.err && !(cflags & (F_HIST | F_BIAS | F_NONFINITE));

  // ---- mode-specific chunk output ----------------------------------------
  uint32_t ncand = 0;
  double mass = 0.0;
  const uint64_t rbase = (uint64_t)row * V;
  if (row_ok && mode != M_GREEDY && nleg > 0) {
    // Emission predicate per token: which tokens become candidates.
    uint32_t emit_kind = 0;      // 0 none, 1 all legal, 2 bin <= thresh, 3 min-p superset
    uint32_t thresh_bin = 0;
    float minp_pre = 0.0f;
    double L = 0.0;
    if (mode == M_TOPK) {
      const uint32_t need = min(c.k, nleg);
      if (need >= nleg) {
        emit_kind = 1;
      } else {
        // Histogram over d = (m - l) * HB / HRANGE, bins 0..HB-2 (HB-1 = beyond range).
        for (uint32_t t = tid; t < (uint32_t)HB; t += NT) S.hist[t] = 0u;
        __syncthreads();
        const float scale = (float)HB / HRANGE;
        if (need <= 128u) {
          // The need-th largest per-thread maximum bounds the chunk's need-th
          // largest logit from below: histogram the NT thread maxima only.
          if (tmaxkey) {
            const float d = (m - okey_value(tmaxkey)) * scale;
            const uint32_t bin = d < (float)(HB - 1) ? (uint32_t)d : (uint32_t)(HB - 1);
            if (bin < (uint32_t)(HB - 1)) atomicAdd(&S.hist[bin], 1u);
          }
        } else {
#pragma unroll
          for (int i = 0; i < PER_MAX; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if ((lbits >> (i * 4 + e)) & 1ull) {
                const float d = (m - lv[i][e]) * scale;
                if (d < (float)(HB - 1)) atomicAdd(&S.hist[(uint32_t)d], 1u);
              }
            }
          }
        }
        __syncthreads();
        // first bin whose cumulative count reaches `need`
        uint32_t cnt = S.hist[tid];
        uint32_t tot;
        const uint32_t inc = block_scan_incl<uint32_t>(cnt, S.red_u, &tot);
        if (tid == 0) S.s_thresh_bin = NONE;
        __syncthreads();
        if (inc >= need && inc - cnt < need) S.s_thresh_bin = tid;
        __syncthreads();
        thresh_bin = S.s_thresh_bin;
        emit_kind = thresh_bin == NONE ? 1u : 2u;
      }
    } else if (mode == M_MINP) {
      L = log(c.min_p);
      const double lim = md + c.T * L;
      minp_pre = (float)lim - (fabsf((float)lim) + fabsf(m)) * 1e-5f - 1e-30f;
      emit_kind = 3;
    } else if (mode == M_ALL) {
      emit_kind = 1;
    }

    const bool need_mass = (mode == M_MINP && c.top_p < 1.0) || mode == M_ALL || mode == M_KEEPALL ||
                           (mode == M_TOPK && b.mask_words != nullptr);
    const float scale = (float)HB / HRANGE;
    // Pass 1: per (slice, wave) counts and the chunk mass.
    double mloc = 0.0;
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      uint32_t cnt_i = 0;
      double seg_mass = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool legal = (lbits >> (i * 4 + e)) & 1ull;
        bool emit = false;
        if (legal) {
          const float l = lv[i][e];
          if (emit_kind == 1) emit = true;
          else if (emit_kind == 2) { const float d = (m - l) * scale; emit = d < (float)(HB - 1) && (uint32_t)d <= thresh_bin; }
          else if (emit_kind == 3) emit = l >= minp_pre && (((double)l - md) / c.T) >= L;
          if (need_mass) seg_mass += exp_neg(((double)l - md) * invT);
        }
        cnt_i += emit;
      }
      if (need_mass) mloc += seg_mass;
      if (mode == M_KEEPALL && i < (int)A.per) {
        const double ws = wave_sum(seg_mass);
        if (lane() == 0) st_dev(&A.w.seg[(((uint64_t)row * MAXC + chunk) * PER_MAX + i) * NW + wave()], ws);
      }
      if (emit_kind) {
        const uint32_t wc = wave_sum(cnt_i);
        if (lane() == 0) S.wcnt[i * NW + wave()] = wc;
      }
    }
    if (need_mass) mass = block_sum<double>(mloc, S.red_d);
    if (emit_kind) {
      __syncthreads();
      // exclusive offsets in (slice, wave) order == token-ID order
      if (tid < 64) {
        uint32_t run = 0;
        if (tid == 0) {
          for (int q = 0; q < PER_MAX * NW; ++q) { S.woff[q] = run; run += S.wcnt[q]; }
          S.s_thresh_bin = run;
        }
      }
      __syncthreads();
      ncand = S.s_thresh_bin;
      // Pass 2: write candidates in token-ID order.
      const uint64_t cbase = rbase + c0;
#pragma unroll
      for (int i = 0; i < PER_MAX; ++i) {
        uint32_t base = S.woff[i * NW + wave()];
        bool em[4];
        uint32_t before_me = 0, mine = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool legal = (lbits >> (i * 4 + e)) & 1ull;
          bool emit = false;
          if (legal) {
            const float l = lv[i][e];
            if (emit_kind == 1) emit = true;
            else if (emit_kind == 2) { const float d = (m - l) * scale; emit = d < (float)(HB - 1) && (uint32_t)d <= thresh_bin; }
            else if (emit_kind == 3) emit = l >= minp_pre && (((double)l - md) / c.T) >= L;
          }
          em[e] = emit;
          const uint64_t bal = __ballot(emit);
          before_me += lanes_below(bal);
        }
        if (i < (int)A.per) {
          uint32_t off = base + before_me;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (em[e]) {
              const uint32_t id = c0 + (uint32_t)i * SLICE + tid * 4u + (uint32_t)e;
              const uint64_t pos = cbase + off + mine;
              st_dev(&A.w.cand_l[pos], lv[i][e]);
              st_dev(&A.w.cand_id[pos], id);
              if (mode == M_ALL) st_dev(&A.w.cand_w[pos], exp_neg(((double)lv[i][e] - md) * invT));
              ++mine;
            }
          }
        }
      }
    }
  }

  // ---- publish the chunk's statistics, then count arrivals ---------------
  if (tid == 0) {
    ChunkStat* st = &A.w.stat[(uint64_t)row * MAXC + chunk];
    st_dev(&st->maxkey, nleg ? maxkey : 0u);
    st_dev(&st->gbest_id, gi);
    st_dev(&st->gbest_val, gv);
    st_dev(&st->nlegal, nleg);
    st_dev(&st->ncand, ncand);
    st_dev(&st->flags, cflags);
    st_dev(&st->mass, mass);
    st_dev(&st->minkey, minkey);
  }
  wait_mem();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&A.w.ctr[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.s_last = (prev == A.C - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!S.s_last) return;

  // =========================================================================
  // Finisher: the last chunk workgroup of the row.
  // =========================================================================
  finish_row<In>(A, F, c, row, mode, rbase, invT);
}

}  // namespace mxs

// ===========================================================================
// Host side: context, validation, launch.
// ===========================================================================
struct mxs_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t max_rows = 0, max_vocab = 0;
  mxs::Work work{};
  std::string last_error;
};

namespace {

int fail(mxs_ctx* ctx, int code, const std::string& msg) {
  if (ctx) ctx->last_error = msg;
  return code;
}

int hip_fail(mxs_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, MXS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

extern "C" {

int mxs_abi_version(void) { return MXS_ABI_VERSION; }

const char* mxs_status_string(int32_t s) {
  switch (s) {
    case MXS_ROW_OK: return "ok";
    case MXS_ROW_UNCERTIFIED: return "ok, uncertified: a decision margin fell below the device error bound";
    case MXS_ROW_EMPTY_LOGITS: return "logits must not be empty";
    case MXS_ROW_MASK_LENGTH_MISMATCH: return "logits and legal-token mask must have equal lengths";
    case MXS_ROW_EMPTY_SUPPORT: return "at least one legal token is required";
    case MXS_ROW_INVALID_TEMPERATURE: return "temperature must be finite, greater than zero, and preserve finite transformed logits";
    case MXS_ROW_INVALID_UNIFORM: return "uniform variate must be finite and in [0, 1)";
    case MXS_ROW_NON_FINITE_LOGIT: return "logits must all be finite";
    case MXS_ROW_VOCABULARY_TOO_LARGE: return "model vocabulary exceeds the supported token-ID range";
    case MXS_ROW_INVALID_TOP_P: return "nucleus sampling requires top_p in (0, 1]";
    case MXS_ROW_INVALID_MIN_P: return "min_p must be in [0, 1]";
    case MXS_ROW_INVALID_PENALTY: return "repetition penalty must be finite and positive; presence and frequency finite";
    case MXS_ROW_INVALID_HISTORY: return "history token IDs must be below the vocabulary (at most 65535 per row)";
    case MXS_ROW_INVALID_BIAS: return "logit bias IDs must be strictly increasing, below the vocabulary, with finite values";
    case MXS_ROW_TOKEN_OUT_OF_RANGE: return "drafted token outside the vocabulary";
    case MXS_ROW_PROBABILITIES: return "invalid probability vectors";
    default: return "unknown status";
  }
}

int mxs_create(int device, void* stream, uint32_t max_rows, uint32_t max_vocab, mxs_ctx** out) {
  if (!out) return MXS_EINVAL;
  *out = nullptr;
  if (max_rows == 0 || max_vocab == 0 || max_vocab > (uint32_t)(mxs::MAXC * mxs::CHUNK_MAX)) return MXS_EINVAL;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return MXS_ENODEV;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return MXS_ENODEV;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MXS_ENODEV;
  mxs_ctx* ctx = new mxs_ctx();
  ctx->device = device;
  ctx->stream = (hipStream_t)stream;
  ctx->max_rows = max_rows;
  ctx->max_vocab = max_vocab;
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(device);
  const size_t rv = (size_t)max_rows * max_vocab;
  hipError_t e = hipSuccess;
  e = e ? e : hipMalloc(&ctx->work.ctr, (size_t)max_rows * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->work.stat, (size_t)max_rows * mxs::MAXC * sizeof(mxs::ChunkStat));
  e = e ? e : hipMalloc(&ctx->work.cand_l, rv * sizeof(float));
  e = e ? e : hipMalloc(&ctx->work.cand_id, rv * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->work.cand_w, rv * sizeof(double));
  e = e ? e : hipMalloc(&ctx->work.seg, (size_t)max_rows * mxs::MAXC * mxs::PER_MAX * mxs::NW * sizeof(double));
  e = e ? e : hipMemset(ctx->work.ctr, 0, (size_t)max_rows * sizeof(uint32_t));
  e = e ? e : hipDeviceSynchronize();
  hipSetDevice(prev);
  if (e != hipSuccess) {
    mxs_destroy(ctx);
    return MXS_ENOMEM;
  }
  *out = ctx;
  return MXS_OK;
}

int mxs_destroy(mxs_ctx* ctx) {
  if (!ctx) return MXS_OK;
  int prev = 0;
  hipGetDevice(&prev);
  hipSetDevice(ctx->device);
  hipDeviceSynchronize();
  hipFree(ctx->work.ctr);
  hipFree(ctx->work.stat);
  hipFree(ctx->work.cand_l);
  hipFree(ctx->work.cand_id);
  hipFree(ctx->work.cand_w);
  hipFree(ctx->work.seg);
  hipSetDevice(prev);
  delete ctx;
  return MXS_OK;
}

int mxs_set_stream(mxs_ctx* ctx, void* stream) {
  if (!ctx) return MXS_EINVAL;
  ctx->stream = (hipStream_t)stream;
  return MXS_OK;
}

int mxs_sync(mxs_ctx* ctx) {
  if (!ctx) return MXS_EINVAL;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return MXS_OK;
}

const char* mxs_last_error(const mxs_ctx* ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

int mxs_sample(mxs_ctx* ctx, const mxs_batch* b, const mxs_out* o) {
  if (!ctx || !b || !o) return MXS_EINVAL;
  if (b->rows == 0) return MXS_OK;
  if (!b->logits || !b->temperature || !o->token || !o->status) return fail(ctx, MXS_EINVAL, "logits, temperature, token and status are required");
  if (b->rows > ctx->max_rows || b->vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  if (b->vocab == 0) return fail(ctx, MXS_EINVAL, "vocab must be positive");
  if (b->dtype != MXS_F32 && b->dtype != MXS_BF16) return fail(ctx, MXS_EINVAL, "dtype must be MXS_F32 or MXS_BF16");
  if (b->row_stride < b->vocab || (b->row_stride & 3u)) return fail(ctx, MXS_EINVAL, "row_stride must be >= vocab and a multiple of 4");
  const size_t align = b->dtype == MXS_F32 ? 16 : 8;
  if (((uintptr_t)b->logits) % align) return fail(ctx, MXS_EINVAL, "logits must be 16-byte (f32) or 8-byte (bf16) aligned");
  if (b->mask_words && b->mask_stride < (b->vocab + 31u) / 32u) return fail(ctx, MXS_EINVAL, "mask_stride must be >= ceil(vocab / 32)");
  if ((b->history_offsets == nullptr) != (b->history_ids == nullptr)) return fail(ctx, MXS_EINVAL, "history offsets and ids go together");
  if ((b->bias_offsets == nullptr) != (b->bias_ids == nullptr) || (b->bias_offsets && !b->bias_values)) return fail(ctx, MXS_EINVAL, "bias offsets, ids and values go together");
  mxs::SampleArgs A;
  A.b = *b;
  A.o = *o;
  A.w = ctx->work;
  const uint32_t V = b->vocab;
  const uint32_t quads = (V + 3u) / 4u;
  uint32_t C = (quads + (uint32_t)(mxs::NT * mxs::PER_MAX) - 1u) / (uint32_t)(mxs::NT * mxs::PER_MAX);
  if (C < 1) C = 1;
  uint32_t ch = ((V + C - 1u) / C + 3u) & ~3u;
  A.C = C;
  A.CH = ch;
  A.per = (ch / 4u + (uint32_t)mxs::NT - 1u) / (uint32_t)mxs::NT;
  if (A.per > (uint32_t)mxs::PER_MAX || C > (uint32_t)mxs::MAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  const uint32_t groups = ((b->rows + 7u) / 8u) * 8u * C;
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  if (b->dtype == MXS_F32)
    hipLaunchKernelGGL(mxs::sample_kernel<float>, dim3(groups), dim3(mxs::NT), 0, ctx->stream, A);
  else
    hipLaunchKernelGGL(mxs::sample_kernel<uint16_t>, dim3(groups), dim3(mxs::NT), 0, ctx->stream, A);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "sample_kernel launch");
  return MXS_OK;
}

int mxs_logsoftmax_topn(mxs_ctx* ctx, const void*, int32_t, uint32_t, uint32_t, uint64_t, uint32_t, int32_t*,
                        double*, double*, double*, int32_t*) {
  return fail(ctx, MXS_EINVAL, "mxs_logsoftmax_topn: not built yet");
}

int mxs_spec_verify(mxs_ctx* ctx, const float*, const float*, uint32_t, uint32_t, uint32_t, const int32_t*,
                    const double*, const double*, const double*, const double*, int32_t*, int32_t*, int32_t*,
                    int32_t*) {
  return fail(ctx, MXS_EINVAL, "mxs_spec_verify: not built yet");
}

}  // extern "C"
