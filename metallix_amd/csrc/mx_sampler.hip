// mx_sampler.hip -- MI355X (gfx950) token sampler: kernels and the C ABI of
// include/mx_sampler.h.
//
// One mxs_sample call is one kernel.  sample_kernel splits each logit row
// into C chunks of at most CHUNK_MAX tokens; one 1024-thread workgroup
// streams a chunk from HBM once into registers (16-byte loads, coalesced),
// applies logit bias and penalties from an LDS count table, the grammar mask
// and the finite check, reduces the chunk's statistics and writes a compact,
// token-ID-ordered candidate list with device-scope stores.  The row's last
// chunk to arrive on the row counter (release by every chunk, acquire by the
// last) becomes the row finisher: it merges the chunk statistics and
// candidates and decides top-k, top-p, min-p and the inverse-CDF draw in f64.  Decisions the reference makes with
// sequential f64 sums are taken from parallel sums only when a rigorous
// error bound certifies them; otherwise the finisher replays the
// reference's sequential order, or reports the row uncertified.
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

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_epilogue.h"
#include "mxs_math.h"

namespace mxs {

constexpr int CCAP = 8192;                // candidates the finisher caches in LDS
constexpr int ECAP = 4096;                // finisher's exact working-set capacity
constexpr int KCAND_MAX = ECAP;           // top_k served from per-chunk candidates
constexpr int NB = 2048;                  // radix-select bins (11 bits)
constexpr int HB = 1024;                  // chunk top-k histogram bins (== NT)
constexpr uint32_t TOP1_MAX = 256;        // top_k served by per-thread maxima; above, top-2 maxima
constexpr uint32_t CT_MAXH = 32767;       // longest history the u16 chunk count table takes
constexpr float HRANGE = 32.0f;           // logit units covered by HB bins
constexpr int HCAP = 4 * NT;              // history ids staged in LDS
constexpr int BCAP = 2 * NT;              // bias entries staged in LDS
// mask words of one chunk (CHUNK_MAX / 32 + 2), rounded up to whole
// 1024-word rounds of the LDS staging, which writes every lane's slot
constexpr int MCAP = ((CHUNK_MAX / 32 + 2 + NT - 1) / NT) * NT;
#ifndef MXS_LA
#define MXS_LA 3
#endif
constexpr int LA = MXS_LA;                // slices in flight ahead of pass 1 (lean chunk body)
constexpr uint32_t WIDE_NCAND = 2048;     // a min-p chunk past this many candidates sums its mass in f64
static_assert(HCAP % NT == 0 && BCAP % NT == 0 && MCAP % NT == 0,
              "LDS staging copies whole 1024-entry rounds");
static_assert(HB == NT, "one histogram bin per thread");

enum Mode : uint32_t { M_GREEDY = 0, M_TOPK = 1, M_MINP = 2, M_ALL = 3, M_KEEPALL = 4 };
enum Flag : uint32_t { F_NONFINITE = 1, F_HIST = 2, F_BIAS = 4 };

struct ChunkStat {
  uint32_t maxkey;     // total-order key of the largest legal logit (0: no legal token)
  uint32_t gbest_id;   // IEEE argmax over legal tokens, lowest ID (NONE: none)
  float gbest_val;
  uint32_t nlegal;
  uint32_t ncand;
  uint32_t flags;
  uint32_t minkey;     // total-order key of the smallest legal logit
  float thr;           // candidate threshold used (diagnostics)
  double mass;         // sum of exp((l - chunk max) / T) over legal tokens, when computed
  double mass_err;     // bound on |mass - exact sum| from the f32 path (0 for the f64 path)
};


// Per-chunk receipt statistics (step receipts fused into the pick).
struct RxStat {
  float maxv;          // the chunk's largest logit after suppression
  uint32_t flags;      // 1: a non-finite logit
  uint32_t count;      // entries listed
  uint32_t pad;
  double sum;          // sum of exp(l - maxv) over the chunk
};

struct SampleArgs {
  mxs_batch b;
  mxs_out o;
  Work w;
  uint32_t C;          // chunks per row
  uint32_t per;        // quads per thread per chunk (<= PER_MAX)
  uint32_t CH;         // tokens per chunk (multiple of 4)
  uint64_t* timing;    // optional phase timestamps (diagnostics), see mxs_debug_set_timing
  int32_t* paths;      // optional finisher path per row (diagnostics), see mxs_debug_set_paths
  uint32_t masked;     // a grammar mask was given (else mask_words is an all-ones row)
  uint32_t epoch;      // this call's tag for Work::rowx (never 0; the row's last chunk also clears its word)
  uint32_t nodraw;     // keep-all rows skip the inverse-CDF draw (race-v2 calls)
  float* race_m;       // race-v2 calls: each row's largest adjusted logit (else null)
  // Step receipts fused into the pick (mxs_step without race-v2): rows whose
  // rx_want entry is not MXS_RECEIPT_NONE also get the log-softmax top rx_n
  // of their logits after suppression, read in the same pass; rx_want null:
  // no receipts
  const uint32_t* rx_want;
  uint32_t rx_n;
  int32_t* rx_ids;             // [rows * rx_n]
  double* rx_lps;              // [rows * rx_n]
  double* rx_token_lp;         // [rows]
  int32_t* rx_status;          // [rows]
  RxStat* rx_stat;             // [rows * MAXC]
  unsigned long long* rx_list; // [rows * MAXC * rx_n], (okey << 32) | ~id, descending
};

// Phase timestamps for diagnostics: wall clock (100 MHz) at fixed points of
// each chunk workgroup and each row finisher, TSTAMPS per record.  Slots
// 0-7 are phases; slot 8 is the workgroup's first instruction and slot 9 its
// exit (for the workgroup that finishes the row, in the finisher's record);
// slots 10 and 11 bracket the step receipt's work (chunk share, merge).
// Every lane stores the same value (a uniform branch only): a lane-0
// condition would make the compiler move uniform values into vector
// registers.
__device__ __forceinline__ void stamp(const SampleArgs& A, uint32_t row, uint32_t chunk, uint32_t k) {
  if (A.timing) A.timing[((uint64_t)row * (MAXC + 1) + chunk) * TSTAMPS + k] = wall_clock64();
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
struct WavePart {                     // one wave's share of the chunk statistics
  uint32_t kmax, kmin, nleg, flags;
  unsigned long long arg;              // (okey(value) << 32) | ~id of the wave's argmax
  double m0, m1;                       // mass and its error weight
};
struct alignas(16) ChunkSmem {
  // members read as 16-byte vectors are 16-byte aligned
  union {
    // whole-chunk table: per token a u16, count in bits 0-14, bias flag in bit 15
    alignas(16) uint32_t ct[CHUNK_MAX / 2];
    struct {                           // per-slice tables (histories longer than CT_MAXH)
      alignas(16) uint32_t tab[2][SLICE];   // count | bias flag << 31 (double-buffered)
      alignas(16) float btab[2][SLICE];     // bias value (double-buffered)
    } sl;
  } t;
  alignas(16) uint32_t hids[HCAP];     // the row's history ids (when at most HCAP)
  alignas(16) uint32_t bids[BCAP];     // the row's bias ids and values (when at most BCAP)
  alignas(16) float bvals[BCAP];
  alignas(16) uint32_t mask[MCAP];     // the chunk's grammar-mask words
  alignas(16) uint32_t hist[HB];       // top-k threshold histogram
  alignas(16) uint32_t wcnt[PER_MAX * NW + 32];   // candidates per (slice, wave), padded for the scan
  WavePart wp[NW];
  WavePart wq[NW];
  uint32_t xkey;                       // min-p rows: the exchanged row-maximum lower bound
  double etab[128];                    // exp_neg's tables (f64 weights of keep-all and top-p-only rows)
};
// The row finisher runs 1024 threads: its candidate phase keeps at most
// CCAP / FT = 8 candidates per thread; sets of at most 256 E tokens are
// finished by one wave.
constexpr int FT = 1024;
constexpr int FW = FT / 64;
static_assert(FT == NT, "the block helpers assume NT-thread blocks");
constexpr uint32_t BPT = NB / FT;          // radix bins per finisher thread
// The selection finisher keeps SR candidate slots per chunk and thread in
// registers, histograms them into NBS value bins, and finishes rows whose
// min-p subset P has at most PCAP members (one per lane of a wave).
constexpr int SR = 6;
constexpr int NBS = 2048;
constexpr int PCAP = 64;
constexpr int PMAX = 1024;
static_assert(NBS == 32 * 64, "a lane scans 32 bins");
struct alignas(16) FinSmem {
  float cl[CCAP];                      // candidates cached in LDS, token-ID order
  uint32_t cid[CCAP];
  uint32_t eidx[ECAP];                 // working set E: indices into the candidates
  union {
    struct {
      double ew[ECAP];                 // weights of E
      unsigned long long skey[ECAP];   // sort keys: (key << 32) | ~E-index, descending
    } e;
    struct {
      uint32_t hcnt[NB];               // radix-select histograms
      double hmass[NB];
    } h;
    struct {                           // the fast finisher's histograms and crossing-bin members
      uint32_t cnt[4096];
      unsigned long long mass[4096];   // fixed-point masses
      uint32_t mkey[FT];
      uint32_t mpos[FT];
      unsigned long long mw[FT];
    } f;
    struct {                           // the selection finisher (finish_sel)
      alignas(16) uint32_t cnt[NBS];   // value histogram of the candidates
      alignas(16) unsigned long long mass[NBS];   // fixed-point mass histogram of P
      uint32_t mk[PCAP], mi[PCAP];     // crossing-bin members: key, token ID, fixed-point mass
      unsigned long long mw[PCAP];
      double sw[PCAP];                 // weights in (key desc, ID asc) rank order
      uint32_t pk[PMAX], pid[PMAX];    // P in token-ID order: key, token ID, logit
      float pl[PMAX];
    } s;
  } u;
  uint32_t sc_u[2][FW];                // single-barrier scan slots
  double sc_d[2][FW];
  unsigned long long sc_l[2][FW];
  unsigned long long s_l[4];
  struct {                             // the row header from the chunk statistics
    double mass, mass_err;             // sum of chunk masses scaled to the row maximum, and the row total's error bound
    double L;                          // ln(min_p) (-inf for min_p = 0)
    uint32_t flags, nlegal, Mkey, bi, ncand;
    uint32_t qmax;                     // the largest candidate count of a chunk
    float lo;                          // no candidate is below it (the chunks' smallest threshold)
  } hdr;
  double etab[128];                    // exp_neg's tables: 2^(j/64) (high, low parts)
  double rd[FW][2];                    // multi-value reduction
  uint32_t ru[FW][4];
  unsigned long long rm[FW];
  uint8_t kflag[ECAP];                 // kept flags by E index
  ChunkStat st[MAXC];
  double cscale[MAXC];
  uint32_t coff[MAXC + 1];
  uint32_t red_u[FW];
  double red_d[FW];
  float red_f[FW];
  uint32_t red_i[FW];
  uint32_t s_u[16];
  double s_d[8];
};

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

// Per-row parameter arrays, passed as separate read-only kernel arguments so
// the compiler reads them with scalar loads (uniform per workgroup).  The
// host substitutes default arrays for the ABI's NULLs, so none is null here.
struct RowParams {
  const double* __restrict__ temperature;
  const uint32_t* __restrict__ top_k;
  const double* __restrict__ top_p;
  const double* __restrict__ min_p;
  const float* __restrict__ repetition;
  const float* __restrict__ presence;
  const float* __restrict__ frequency;
  const double* __restrict__ uniform;
  const uint32_t* __restrict__ history_offsets;
  const uint32_t* __restrict__ bias_offsets;
};

__device__ __forceinline__ RowCfg load_cfg(const double* __restrict__ temperature, const uint32_t* __restrict__ top_k,
                                           const double* __restrict__ top_p, const double* __restrict__ min_p,
                                           const float* __restrict__ repetition, const float* __restrict__ presence,
                                           const float* __restrict__ frequency, const double* __restrict__ uniform,
                                           const uint32_t* __restrict__ hoff, const uint32_t* __restrict__ boff,
                                           uint32_t row) {
  RowCfg c;
  c.T = temperature[row];
  c.top_p = top_p[row];
  c.min_p = min_p[row];
  c.u = uniform[row];
  c.k = top_k[row];
  c.rep = repetition[row];
  c.pres = presence[row];
  c.freq = frequency[row];
  c.hb = hoff[row];
  c.he = hoff[row + 1];
  c.bb = boff[row];
  c.be = boff[row + 1];
  // every load goes out before the first wait: the checks below would
  // otherwise pull the loads they guard into their branches, one round
  // trip each
  __asm__ volatile("" ::"s"(c.T), "s"(c.top_p), "s"(c.min_p), "s"(c.u), "s"(c.k), "s"(c.rep), "s"(c.pres),
                   "s"(c.freq), "s"(c.hb), "s"(c.he), "s"(c.bb), "s"(c.be));
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

// A bias value is finite, or -inf (the token is suppressed: f32::MIN).
__device__ __forceinline__ bool bias_ok(float v) { return v == v && v != INFINITY; }

// Error precedence after the parameter checks: history ids, bias entries,
// uniform, non-finite adjusted logit, empty support.
__device__ __forceinline__ int32_t combine_errors(const RowCfg& c, uint32_t flags, uint32_t nlegal) {
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
__device__ __forceinline__ float adjust(float l, uint32_t cnt, uint32_t slot, float bias, const RowCfg& c) {
  return penalize_logit(l, cnt, slot != 0u, bias, c.rep, c.pres, c.freq);
}

// Re-derives the adjusted logit and legality of token `id`, whose history
// count `cnt` the caller supplies.  Used by the finisher to locate a draw
// inside a 256-token segment without the chunk's registers.  Bias ids are
// strictly increasing (the chunk pass rejects the row otherwise): binary
// search.
template <typename In>
__device__ __forceinline__ void rederive_token(const SampleArgs& A, const RowCfg& c, uint32_t row, uint32_t id,
                                               uint32_t cnt, float* l_out, bool* legal_out) {
  const mxs_batch& b = A.b;
  const In* p = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;
  const float l = Quad<In>::one(p + id);
  uint32_t lo = c.bb, hi = c.be;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (b.bias_ids[mid] < id) lo = mid + 1u; else hi = mid;
  }
  const bool hasb = lo < c.be && b.bias_ids[lo] == id;
  *l_out = penalize_logit(l, cnt, hasb, hasb ? b.bias_values[lo] : 0.0f, c.rep, c.pres, c.freq);
  const uint32_t w = b.mask_words[(uint64_t)row * b.mask_stride + (id >> 5)];
  *legal_out = ((w >> (id & 31)) & 1u) && id < b.tokenizer_vocab;
}

// ---------------------------------------------------------------------------
// Finisher helpers.

// Bitonic sort of n (<= ECAP) keys into descending order, in LDS.
__device__ __forceinline__ void bitonic_sort_desc(unsigned long long* key, uint32_t n) {
  uint32_t np = 1;
  while (np < n) np <<= 1;
  for (uint32_t i = n + threadIdx.x; i < np; i += FT) key[i] = 0ull;
  __syncthreads();
  for (uint32_t size = 2; size <= np; size <<= 1) {
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (uint32_t t = threadIdx.x; t < np / 2; t += FT) {
        const uint32_t i = 2 * stride * (t / stride) + (t % stride);
        const uint32_t j = i + stride;
        const bool desc = ((i & size) == 0);
        const unsigned long long a = key[i], bb = key[j];
        if ((a < bb) == desc) { key[i] = bb; key[j] = a; }
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

// top_p = 1 under a top-k: the reference's running f64 sum over the top-k
// weights (descending) stops at its first value equal to the kept mass, so
// weights too small to move the sum (at or below 2.3e-16 of it) may be cut.
// Only members at or above the min-p cut are kept, and each such member's
// weight is at least min_p (to within rounding): when min_p clears that
// stall level, the cut cannot reach a kept member.
__device__ __forceinline__ bool minp_above_stall(const RowCfg& c, double esum) {
  return c.min_p > 0.0 && c.min_p * (1.0 - 1e-12) > 2.3e-16 * esum;
}

// ---------------------------------------------------------------------------
// Finisher state shared by its phases.
struct FinCtx {
  // copies of the launch arguments the decisions need (taking the address
  // of the by-value kernel argument would force it into private memory)
  const float* cand_l;
  const uint32_t* cand_id;
  uint32_t CH;
  mxs_out o;
  RowCfg c;            // a copy (a pointer to the caller's would put it in private memory)
  uint32_t row, mode, C, V, ncand, nlegal;
  uint64_t rbase;
  bool lds_c;          // candidates cached in LDS
  bool k_path;
  uint32_t kappa, id_tie;
  double M, L, Lclose, total, total_err;
  bool have_total;
  bool nodraw;         // race-v2: the draw is discarded, so only the kept set's certificate sets the status
  uint32_t* kbits;
  uint32_t nwords;
  uint64_t* timing;    // phase timestamps (diagnostics), null when off
  int32_t* paths;      // finisher path per row (diagnostics), null when off
  const double* etab;  // exp_neg's tables in LDS
};

// The finisher path a row took (MXS_PATH_*, diagnostics); a later call on
// the same row overwrites an earlier one.
__device__ __forceinline__ void fpath(const FinCtx& X, int32_t p) {
  if (X.paths && threadIdx.x == 0) X.paths[X.row] = p;
}

// Finisher phase timestamp k (slot MAXC of the row's timing record).
__device__ __forceinline__ void fstamp(const FinCtx& X, uint32_t k) {
  if (X.timing) X.timing[((uint64_t)X.row * (MAXC + 1) + MAXC) * TSTAMPS + k] = wall_clock64();
}

__device__ __forceinline__ uint64_t cand_pos_of(const FinSmem& F, uint32_t C, uint64_t rbase, uint32_t CH, uint32_t j) {
  uint32_t q = 0;
  while (q + 1 < C && F.coff[q + 1] <= j) ++q;
  return rbase + (uint64_t)q * CH + (j - F.coff[q]);
}

// Candidate j (token-ID order): from LDS when cached, else from the
// device-scope candidate arrays.
__device__ __forceinline__ float cand_l(const FinCtx& X, const FinSmem& F, uint32_t j) {
  if (X.lds_c) return F.cl[j];
  const float* p = &X.cand_l[cand_pos_of(F, X.C, X.rbase, X.CH, j)];
  return ld_dev(p);
}
__device__ __forceinline__ uint32_t cand_id(const FinCtx& X, const FinSmem& F, uint32_t j) {
  if (X.lds_c) return F.cid[j];
  const uint32_t* p = &X.cand_id[cand_pos_of(F, X.C, X.rbase, X.CH, j)];
  return ld_dev(p);
}
__device__ __forceinline__ bool member(const FinCtx& X, float l, uint32_t id) {
  if (X.k_path) {
    const uint32_t key = okey(l);
    return key > X.kappa || (key == X.kappa && id <= X.id_tie);
  }
  if (X.mode == M_MINP) return (((double)l - X.M) / X.c.T) >= X.L;
  return true;
}

__device__ __forceinline__ void write_result(const FinCtx& X, int32_t status, int32_t token, double lp, uint32_t kept) {
  if (threadIdx.x == 0) {
    const mxs_out& o = X.o;
    o.token[X.row] = token;
    o.status[X.row] = status;
    if (o.sampling_logprob) o.sampling_logprob[X.row] = lp;
    if (o.kept_count) o.kept_count[X.row] = kept;
  }
}

// ---------------------------------------------------------------------------
// Large working set (E beyond the LDS capacity): E is the predicate `member`
// over the candidates; the nucleus cut comes from a mass-weighted radix
// select (11/11/10-bit passes, LDS count and f64 mass histograms) whose bin
// decisions are certified with the same bounds as the exact path.
__device__ __forceinline__ void finish_large(const FinCtx& X, FinSmem& F, uint32_t ne) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x;
  const uint32_t n = X.ncand;
  auto weight = [&](float l) { return exp_neg_t(((double)l - X.M) / c.T, X.etab, X.etab + 64); };
  bool uncert = false;
  double wpart = 0.0, wmin = INFINITY;
  for (uint32_t j = tid; j < n; j += FT) {
    const float l = cand_l(X, F, j);
    if (member(X, l, cand_id(X, F, j))) {
      const double w = weight(l);
      wpart += w;
      wmin = fmin(wmin, w);
    }
  }
  const double esum = block_sum<double>(wpart, F.red_d);
  wmin = -block_max<double>(-wmin, F.red_d);
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, ne, 8.0); }
  fstamp(X, 4);

  uint32_t tau = 0, id_cut = NONE;
  bool cut = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      if (!minp_above_stall(c, esum) && !(wmin > 2.3e-16 * esum)) uncert = true;
    } else {
      cut = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
    cut = !(esum + sum_bound(esum, ne, 8.0) < theta - theta_err);
  }
  if (cut) {
    uint32_t prefix = 0, pmask = 0, above_n = 0;
    double above = 0.0;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      for (uint32_t t = tid; t < (uint32_t)NB; t += FT) { F.u.h.hcnt[t] = 0u; F.u.h.hmass[t] = 0.0; }
      __syncthreads();
      for (uint32_t j = tid; j < n; j += FT) {
        const float l = cand_l(X, F, j);
        const uint32_t key = okey(l);
        if ((key & pmask) == prefix && member(X, l, cand_id(X, F, j))) {
          const uint32_t bin = (key >> sh) & (NB - 1);
          atomicAdd(&F.u.h.hcnt[bin], 1u);
          atomicAdd(&F.u.h.hmass[bin], weight(l));
        }
      }
      __syncthreads();
      // Each thread owns BPT consecutive bins in descending key order; the
      // per-thread intervals (mexc, minc] tile the mass exactly (the
      // exclusive prefix is the previous thread's inclusive value), and so
      // do the per-bin intervals inside a thread, so at most one bin claims
      // theta.
      const uint32_t b0 = NB - 1 - BPT * tid;
      double msum = 0.0;
      uint32_t nsum = 0;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) { msum += F.u.h.hmass[b0 - i]; nsum += F.u.h.hcnt[b0 - i]; }
      double mtot, mexc;
      uint32_t ntot, nexc;
      const double minc = above + block_scan_pair<double>(msum, F.red_d, &mexc, &mtot);
      mexc += above;
      nexc = above_n + block_scan_incl<uint32_t>(nsum, F.red_u, &ntot) - nsum;
      if (tid == 0) { F.s_u[4] = NONE; F.s_u[6] = 0u; }
      __syncthreads();
      double lo = mexc;
      uint32_t nlo = nexc;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) {
        const double mh = F.u.h.hmass[b0 - i];
        const uint32_t nh = F.u.h.hcnt[b0 - i];
        const double hi = i + 1 == BPT ? minc : lo + mh;
        if (nh && lo < theta && theta <= hi) {
          F.s_u[4] = b0 - i; F.s_u[5] = nlo; F.s_d[4] = lo;
          const double e0 = sum_bound(lo, nlo + 64u, 8.0);
          const double e1 = sum_bound(hi, nlo + nh + 64u, 8.0);
          if (!(lo + e0 < theta - theta_err) || !(hi - e1 >= theta + theta_err)) F.s_u[6] = 1u;
        }
        lo = hi;
        nlo += nh;
      }
      __syncthreads();
      const uint32_t bin = F.s_u[4];
      const uint32_t amb = F.s_u[6];
      const uint32_t an = F.s_u[5];
      const double am = F.s_d[4];
      __syncthreads();
      if (bin == NONE) { cut = false; uncert = true; break; }
      if (amb) uncert = true;
      prefix |= bin << sh;
      pmask |= (uint32_t)(NB - 1) << sh;
      above = am;
      above_n = an;
    }
    if (cut) {
      tau = prefix;
      const double wt = weight(okey_value(tau));
      if (tid == 0) {
        uint32_t jn = 0;
        double cov = above;
        bool close = false;
        for (uint32_t q = 0; q < (uint32_t)NB * 64u; ++q) {
          cov += wt;
          ++jn;
          const double e = sum_bound(cov, above_n + jn + 64u, 8.0);
          if (fabs(cov - theta) <= e + theta_err) close = true;
          if (cov >= theta || !(wt > 0.0)) break;
        }
        F.s_u[6] = jn;
        F.s_u[7] = close ? 1u : 0u;
        F.s_u[3] = NONE;
      }
      __syncthreads();
      const uint32_t jneed = F.s_u[6];
      if (F.s_u[7]) uncert = true;
      uint32_t seen = 0;
      for (uint32_t base = 0; base < n; base += FT) {
        const uint32_t j = base + tid;
        bool tie = false;
        uint32_t id = 0;
        if (j < n) {
          const float l = cand_l(X, F, j);
          id = cand_id(X, F, j);
          tie = okey(l) == tau && member(X, l, id);
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

  fstamp(X, 5);
  // kept = member, inside the cut, and (unless E is the min-p set already)
  // at or above ln(min_p); the draw walks kept tokens in ID order.
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  auto kept = [&](float l, uint32_t id, double* s) -> bool {
    *s = ((double)l - X.M) / c.T;
    if (!member(X, l, id)) return false;
    if (cut) {
      const uint32_t key = okey(l);
      if (!(key > tau || (key == tau && id <= id_cut))) return false;
    }
    return !(apply_minp && !(*s >= X.L));
  };
  double kpart = 0.0;
  uint32_t kn = 0, close = 0, bad = 0;
  for (uint32_t j = tid; j < n; j += FT) {
    const float l = cand_l(X, F, j);
    double s;
    const bool k = kept(l, cand_id(X, F, j), &s);
    if (apply_minp && fabs(s - X.L) < X.Lclose) close = 1;
    if (k) { kpart += exp_neg_t(s, X.etab, X.etab + 64); ++kn; if (!isfinite(s)) bad = 1; }
  }
  if (block_max<uint32_t>(bad, F.red_u)) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
  if (block_max<uint32_t>(close, F.red_u)) uncert = true;
  const double S = block_sum<double>(kpart, F.red_d);
  const uint32_t nkept = block_sum<uint32_t>(kn, F.red_u);
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
  __syncthreads();
  fstamp(X, 6);
  double run = 0.0;
  for (uint32_t base = 0; base < n; base += FT) {
    const uint32_t j = base + tid;
    double s = 0.0, w = 0.0;
    uint32_t id = 0;
    if (j < n) {
      const float l = cand_l(X, F, j);
      id = cand_id(X, F, j);
      if (kept(l, id, &s)) w = exp_neg_t(s, X.etab, X.etab + 64);
    }
    double tot;
    const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
    const double exc = inc - w;
    {   // the last positive weight's position: one LDS atomic per wave
      const uint32_t lj = wave_max_u32(w > 0.0 ? j + 1u : 0u);
      if (lane() == 0 && lj) atomicMax(&F.s_u[1], lj);
    }
    if (w > 0.0) {
      if (target < inc && !(target < exc)) {
        F.s_u[0] = id;
        F.s_d[0] = s;
        if (fabs(target - exc) <= derr || fabs(inc - target) <= derr) F.s_u[2] = 1u;
      }
    }
    run += tot;
  }
  __syncthreads();
  uint32_t tok = F.s_u[0];
  double shifted = F.s_d[0];
  if (F.s_u[2] && !X.nodraw) uncert = true;
  if (tok == NONE && F.s_u[1]) {
    // rounding left the variate past the accumulated mass: last positive kept token
    const uint32_t j = F.s_u[1] - 1u;
    tok = cand_id(X, F, j);
    shifted = ((double)cand_l(X, F, j) - X.M) / c.T;
    uncert = uncert || !X.nodraw;
  }
  __syncthreads();
  if (tok == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)tok, shifted - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = tid; q < X.nwords; q += FT) X.kbits[q] = 0u;
    __syncthreads();
    for (uint32_t j = tid; j < n; j += FT) {
      const float l = cand_l(X, F, j);
      const uint32_t id = cand_id(X, F, j);
      double s;
      if (kept(l, id, &s)) atomicOr(&X.kbits[id >> 5], 1u << (id & 31u));
    }
  }
}

// ---------------------------------------------------------------------------
// Exact path: E (token-ID order) fits in LDS as indices into the cached
// candidates.  P = E's min-p prefix.  The nucleus is a prefix of E in
// descending order; when P's mass certainly stays below the nucleus target
// the final set is P with no sort, otherwise the crossing lies inside P and
// only P is sorted.  An uncertain crossing replays the reference's
// sequential f64 sums over E sorted.
__device__ __forceinline__ void finish_exact(const FinCtx& X, FinSmem& F, uint32_t ne, bool mp_close_in) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x;
  auto el = [&](uint32_t t) { return F.cl[F.eidx[t]]; };
  auto eid = [&](uint32_t t) { return F.cid[F.eidx[t]]; };
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  bool uncert = mp_close_in;
  double epart = 0.0, ppart = 0.0, wmin = INFINITY;
  uint32_t pn = 0, close = 0;
  for (uint32_t t = tid; t < ne; t += FT) {
    const double s = ((double)el(t) - X.M) / c.T;
    const double w = exp_neg_t(s, X.etab, X.etab + 64);
    F.u.e.ew[t] = w;
    epart += w;
    wmin = fmin(wmin, w);
    bool inp = true;
    if (apply_minp) {
      inp = s >= X.L;
      if (fabs(s - X.L) < X.Lclose) close = 1;
    }
    F.kflag[t] = inp ? 1 : 0;   // provisional: in P
    if (inp) { ppart += w; ++pn; }
  }
  const double esum = block_sum<double>(epart, F.red_d);
  const double psum = block_sum<double>(ppart, F.red_d);
  const uint32_t np_ = block_sum<uint32_t>(pn, F.red_u);
  wmin = -block_max<double>(-wmin, F.red_d);
  if (block_max<uint32_t>(close, F.red_u)) uncert = true;
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, ne, 8.0); }

  // The nucleus over E in descending order, intersected with P.
  bool theta_set = false, replay = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      // covered reaches kept only at E's last token when every weight is
      // large enough to change the running f64 sum; otherwise replay.
      replay = !minp_above_stall(c, esum) && !(wmin > 2.3e-16 * esum);
    } else {
      theta_set = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta_set = true;
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
  }
  if (theta_set && !(psum + sum_bound(psum, np_, 8.0) < theta - theta_err)) {
    // The crossing lies inside P: sort P and find the first prefix reaching theta.
    fpath(X, MXS_PATH_EXACT_SORTED);
    if (tid == 0) F.s_u[8] = 0u;
    __syncthreads();
    for (uint32_t t = tid; t < ne; t += FT) {
      if (F.kflag[t]) {
        const uint32_t at = atomicAdd(&F.s_u[8], 1u);
        F.u.e.skey[at] = ((unsigned long long)okey(el(t)) << 32) | (unsigned long long)(0xffffffffu - t);
      }
    }
    __syncthreads();
    bitonic_sort_desc(F.u.e.skey, np_);
    if (tid == 0) { F.s_u[6] = NONE; F.s_u[7] = 0u; }
    __syncthreads();
    double run = 0.0;
    for (uint32_t base = 0; base < np_; base += FT) {
      const uint32_t p = base + tid;
      const double w = p < np_ ? F.u.e.ew[0xffffffffu - (uint32_t)F.u.e.skey[p]] : 0.0;
      double tot;
      const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
      const double exc = inc - w;
      if (p < np_) {
        const double e_inc = sum_bound(inc, p + 65u, 8.0);
        const double e_exc = sum_bound(exc, p + 64u, 8.0);
        const bool lt = inc + e_inc < theta - theta_err;
        if (!lt) {
          const bool prev_lt = p == 0 || exc + e_exc < theta - theta_err;
          if (prev_lt) {
            F.s_u[6] = p;   // the first position not certainly below theta
            if (!(inc - e_inc >= theta + theta_err)) F.s_u[7] = 1u;
          }
        }
      }
      run += tot;
    }
    __syncthreads();
    const uint32_t first = F.s_u[6];
    if (first == NONE || F.s_u[7]) {
      replay = true;
    } else {
      // kept = the first `first + 1` sorted positions of P
      for (uint32_t t = tid; t < ne; t += FT) F.kflag[t] = 0;
      __syncthreads();
      for (uint32_t p = tid; p <= first; p += FT) F.kflag[0xffffffffu - (uint32_t)F.u.e.skey[p]] = 1;
    }
    __syncthreads();
  }
  if (replay) {
    // Sort all of E and replay the reference's sequential f64 sums.
    fpath(X, MXS_PATH_EXACT_REPLAY);
    for (uint32_t t = tid; t < ne; t += FT)
      F.u.e.skey[t] = ((unsigned long long)okey(el(t)) << 32) | (unsigned long long)(0xffffffffu - t);
    __syncthreads();
    bitonic_sort_desc(F.u.e.skey, ne);
    if (tid == 0) {
      double th = theta;
      if (X.k_path) {
        double keptsum = 0.0;
        for (uint32_t q = 0; q < ne; ++q) keptsum += F.u.e.ew[0xffffffffu - (uint32_t)F.u.e.skey[q]];
        th = c.top_p * keptsum;
      }
      double cov = 0.0;
      uint32_t nk = ne, cl = 0;
      for (uint32_t q = 0; q < ne; ++q) {
        cov += F.u.e.ew[0xffffffffu - (uint32_t)F.u.e.skey[q]];
        if (!X.k_path && fabs(cov - th) <= theta_err + sum_bound(cov, q + 1, 8.0)) cl = 1;
        if (cov >= th) { nk = q + 1; break; }
      }
      F.s_u[6] = nk;
      F.s_u[7] = cl;
    }
    __syncthreads();
    const uint32_t nk = F.s_u[6];
    if (F.s_u[7]) uncert = true;
    // kept = sorted positions < nk, intersected with P
    for (uint32_t p = tid; p < ne; p += FT) {
      const uint32_t t = 0xffffffffu - (uint32_t)F.u.e.skey[p];
      if (p >= nk) F.kflag[t] = 0;
    }
    __syncthreads();
  }

  // sample_categorical rejects a kept token whose shifted logit overflows.
  uint32_t bad = 0;
  for (uint32_t t = tid; t < ne; t += FT)
    if (F.kflag[t] && !isfinite(((double)el(t) - X.M) / c.T)) bad = 1;
  if (block_max<uint32_t>(bad, F.red_u)) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }

  // Inverse-CDF draw over the kept set in token-ID order.
  double kpart = 0.0;
  uint32_t kn = 0;
  for (uint32_t t = tid; t < ne; t += FT)
    if (F.kflag[t]) { kpart += F.u.e.ew[t]; ++kn; }
  const double S = block_sum<double>(kpart, F.red_d);
  const uint32_t nkept = block_sum<uint32_t>(kn, F.red_u);
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
  __syncthreads();
  double run = 0.0;
  for (uint32_t base = 0; base < ne; base += FT) {
    const uint32_t t = base + tid;
    const double w = (t < ne && F.kflag[t]) ? F.u.e.ew[t] : 0.0;
    double tot;
    const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
    const double exc = inc - w;
    {   // the last positive weight's position: one LDS atomic per wave
      const uint32_t lt = wave_max_u32(w > 0.0 ? t + 1u : 0u);
      if (lane() == 0 && lt) atomicMax(&F.s_u[1], lt);
    }
    if (w > 0.0) {
      if (target < inc && !(target < exc)) {
        F.s_u[0] = t;
        if (fabs(target - exc) <= derr || fabs(inc - target) <= derr) F.s_u[2] = 1u;
      }
    }
    run += tot;
  }
  __syncthreads();
  uint32_t pick = F.s_u[0];
  if (F.s_u[2] && !X.nodraw) uncert = true;
  if (pick == NONE) {
    pick = F.s_u[1] ? F.s_u[1] - 1u : NONE;
    uncert = uncert || !X.nodraw;
  }
  if (pick == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  const double shifted = ((double)el(pick) - X.M) / c.T;
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)eid(pick), shifted - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = tid; q < X.nwords; q += FT) X.kbits[q] = 0u;
    __syncthreads();
    for (uint32_t t = tid; t < ne; t += FT)
      if (F.kflag[t]) atomicOr(&X.kbits[eid(t) >> 5], 1u << (eid(t) & 31u));
  }
}

// ---------------------------------------------------------------------------
// Fast finisher for candidate sets cached in LDS (at most CCAP, token-ID
// order).  The candidate phase runs on the whole workgroup, thread t owning
// the R contiguous candidates from t * R:
//   E     the top-k head (the k-th largest key from a 12-bit LDS histogram
//         and ranks inside the crossing bin; ties at the k-th key kept in ID
//         order), the exact min-p set, or every candidate; compacted to eidx
//         in token-ID order.
// The E phase runs on one wave when E has at most 4 * 64 tokens (no
// workgroup barriers at all), else on the workgroup:
//   sums  f64 weights of E (group-contiguous, at most FE per thread), the
//         min-p subset P, and the sums
//   cut   when the nucleus can end inside P: a histogram of P's keys (4 bins
//         per thread) with exact fixed-point masses finds the crossing bin,
//         and ranks inside that bin the crossing token
//   draw  the inverse-CDF draw over the kept tokens in token-ID order.
// Returns false, having written nothing, for a row the general path decides
// (more candidates or E tokens than fit, an uncertain cut, the top_p = 1
// freeze rule, a crossing bin with more members than threads).
constexpr int FR = CCAP / FT;      // candidates per thread
constexpr int FE = ECAP / FT;      // E tokens per thread
constexpr int FB = 4 * FT;         // the candidate phase's histogram bins
constexpr int FB_BITS = FT == 256 ? 10 : (FT == 512 ? 11 : 12);
static_assert(FB == (1 << FB_BITS), "power-of-two bins");
constexpr double WFIX = 0x1p50;    // fixed-point scale of the cut's masses (every weight is at most 1)
static_assert(FB == 4 * FT, "each thread scans four histogram bins");
static_assert(FR <= 32 && FE <= 32, "per-thread bit masks");

// Bin shift for keys in [kmin, kmax] and 2^bits bins: the bits from the
// highest bit where they differ down (keys share every bit above it).
__device__ __forceinline__ int fast_shift(uint32_t kmin, uint32_t kmax, int bits) {
  const uint32_t diff = kmin ^ kmax;
  const int hb = diff ? 31 - (int)__builtin_clz(diff) : 0;
  return hb >= bits ? hb - bits + 1 : 0;
}

// The k-th largest of the active candidate keys (1 <= k <= active count)
// and how many active keys are larger.  Returns false when the crossing bin
// holds more than FT keys (the caller falls back).
__device__ __forceinline__ bool fast_kth(FinSmem& F, const uint32_t (&key)[FR], uint32_t act, uint32_t k,
                                         uint32_t kmin, uint32_t kmax, uint32_t* kappa, uint32_t* above) {
  const uint32_t tid = threadIdx.x;
  if (kmin == kmax) { *kappa = kmax; *above = 0u; return true; }
  const int sh = fast_shift(kmin, kmax, FB_BITS);
  uint32_t* cnt = F.u.f.cnt;
  reinterpret_cast<uint4*>(cnt)[tid] = make_uint4(0u, 0u, 0u, 0u);
  F.u.f.mkey[tid] = 0u;   // key 0 is no finite logit's: pads the member list
  if (tid == 0) F.s_u[10] = 0u;
  lds_barrier();
#pragma unroll
  for (int r = 0; r < FR; ++r)
    if ((act >> r) & 1u) atomicAdd(&cnt[(key[r] >> sh) & (FB - 1)], 1u);
  lds_barrier();
  // thread t scans bins FB-1-4t down to FB-4-4t
  const uint4 h4 = reinterpret_cast<const uint4*>(cnt)[FT - 1 - tid];
  const uint32_t hv[4] = {h4.w, h4.z, h4.y, h4.x};
  uint32_t tot;
  uint32_t run = block_excl_scan_u32(h4.x + h4.y + h4.z + h4.w, F.sc_u[0], &tot);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (run < k && k <= run + hv[i]) { F.s_u[8] = FB - 1 - 4 * tid - (uint32_t)i; F.s_u[9] = run; }
    run += hv[i];
  }
  lds_barrier();
  const uint32_t bstar = F.s_u[8], abv = F.s_u[9];
  if (sh == 0) { *kappa = (kmax & ~(uint32_t)(FB - 1)) | bstar; *above = abv; return true; }
  // rank the crossing bin's members
#pragma unroll
  for (int r = 0; r < FR; ++r) {
    if (((act >> r) & 1u) && ((key[r] >> sh) & (FB - 1)) == bstar) {
      const uint32_t at = atomicAdd(&F.s_u[10], 1u);
      if (at < (uint32_t)FT) F.u.f.mkey[at] = key[r];
    }
  }
  lds_barrier();
  const uint32_t cm = F.s_u[10];
  if (cm > (uint32_t)FT) return false;
  const uint32_t need = k - abv;
  if (tid < cm) {
    const uint32_t my = F.u.f.mkey[tid];
    uint32_t gt = 0, eq = 0;
    for (uint32_t i = 0; i < cm; i += 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(&F.u.f.mkey[i]);
      gt += (v.x > my) + (v.y > my) + (v.z > my) + (v.w > my);
      eq += (v.x == my) + (v.y == my) + (v.z == my) + (v.w == my);
    }
    if (gt < need && need <= gt + eq) { F.s_u[11] = my; F.s_u[12] = abv + gt; }
  }
  lds_barrier();
  *kappa = F.s_u[11];
  *above = F.s_u[12];
  return true;
}

// Group primitives of the E phase: one wave (G = 64: LDS operations of one
// wave complete in order, so no barrier is needed) or the workgroup (G = FT:
// one LDS barrier per call; consecutive calls alternate their slots).
template <int G>
struct Grp;
template <>
struct Grp<64> {
  __device__ __forceinline__ static uint32_t id() { return lane(); }
  __device__ __forceinline__ static void sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
  __device__ __forceinline__ static uint32_t excl_u32(uint32_t v, uint32_t*, uint32_t* total) {
    const uint32_t i = wave_scan_u32(v);
    *total = bcast63(i);
    return i - v;
  }
  __device__ __forceinline__ static unsigned long long excl_u64(unsigned long long v, unsigned long long*, unsigned long long* total) {
    const unsigned long long i = wave_scan_u64(v);
    *total = readlane64(i, 63);
    return i - v;
  }
  __device__ __forceinline__ static double incl_f64(double v, double*, double* total) {
    const double i = wave_scan_f64(v);
    *total = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, i), 63));
    return i;
  }
  // sums of two f64 and one u32 (one reduction)
  __device__ __forceinline__ static void sum3(double& a, double& b, uint32_t& c, FinSmem&, int) {
    a = wave_sum_f64(a);
    b = wave_sum_f64(b);
    c = wave_sum_u32(c);
  }
  __device__ __forceinline__ static void minmax_u32(uint32_t& mn, uint32_t& mx, FinSmem&) {
    mn = ~wave_max_u32(~mn);
    mx = wave_max_u32(mx);
  }
  __device__ __forceinline__ static unsigned long long min_u64(unsigned long long v, FinSmem&) { return ~wave_max_u64(~v); }
};
template <>
struct Grp<FT> {
  __device__ __forceinline__ static uint32_t id() { return threadIdx.x; }
  __device__ __forceinline__ static void sync() { lds_barrier(); }
  __device__ __forceinline__ static uint32_t excl_u32(uint32_t v, uint32_t* slot, uint32_t* total) {
    return block_excl_scan_u32(v, slot, total);
  }
  __device__ __forceinline__ static unsigned long long excl_u64(unsigned long long v, unsigned long long* slot,
                                                unsigned long long* total) {
    return block_excl_scan_u64(v, slot, total);
  }
  __device__ __forceinline__ static double incl_f64(double v, double* slot, double* total) { return block_incl_scan_f64(v, slot, total); }
  __device__ __forceinline__ static void sum3(double& a, double& b, uint32_t& c, FinSmem& F, int s) {
    a = wave_sum_f64(a);
    b = wave_sum_f64(b);
    c = wave_sum_u32(c);
    if (lane() == 0) { F.rd[wave()][0] = a; F.rd[wave()][1] = b; F.ru[wave()][s] = c; }
    lds_barrier();
    const bool wl = lane() < (uint32_t)FW;
    const uint32_t q = wl ? lane() : 0u;
    a = wave_sum_f64(wl ? F.rd[q][0] : 0.0);
    b = wave_sum_f64(wl ? F.rd[q][1] : 0.0);
    c = wave_sum_u32(wl ? F.ru[q][s] : 0u);
  }
  __device__ __forceinline__ static void minmax_u32(uint32_t& mn, uint32_t& mx, FinSmem& F) {
    mn = ~wave_max_u32(~mn);
    mx = wave_max_u32(mx);
    if (lane() == 0) { F.ru[wave()][2] = mn; F.ru[wave()][3] = mx; }
    lds_barrier();
    const bool wl = lane() < (uint32_t)FW;
    const uint32_t q = wl ? lane() : 0u;
    mn = ~wave_max_u32(wl ? ~F.ru[q][2] : 0u);
    mx = wave_max_u32(wl ? F.ru[q][3] : 0u);
  }
  __device__ __forceinline__ static unsigned long long min_u64(unsigned long long v, FinSmem& F) {
    v = ~wave_max_u64(~v);
    if (lane() == 0) F.rm[wave()] = v;
    lds_barrier();
    const bool wl = lane() < (uint32_t)FW;
    return ~wave_max_u64(wl ? ~F.rm[wl ? lane() : 0u] : 0ull);
  }
};

// The E phase (see finish_fast) on a group of G threads; E is eidx[0, ne)
// in token-ID order, at most FE per thread.  `unc0` carries the candidate
// phase's min-p closeness flag.  Returns false, having written nothing, for
// the general path.
template <int G>
__device__ __forceinline__ bool e_finish(const FinCtx& X, FinSmem& F, uint32_t ne, uint32_t unc0) {
  using Gr = Grp<G>;
  constexpr int NBG = 4 * G;                 // cut histogram bins
  constexpr int BITS = G == 64 ? 8 : (G == 256 ? 10 : (G == 512 ? 11 : 12));
  static_assert(NBG == (1 << BITS), "4 bins per thread");
  const RowCfg& c = X.c;
  const uint32_t gi = Gr::id();
  const uint32_t RE = (ne + G - 1u) / G;
  const uint32_t p0 = gi * RE;
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  double w[FE];
  uint32_t ek[FE];
  uint32_t inP = 0, unc = 0;
  double esum = 0.0, psum = 0.0;
  uint32_t np_unc = 0;   // P count | close flags << 16
#pragma unroll
  for (int r = 0; r < FE; ++r) {
    w[r] = 0.0;
    ek[r] = 0u;
    if ((uint32_t)r < RE && p0 + (uint32_t)r < ne) {
      const float l = F.cl[F.eidx[p0 + r]];
      ek[r] = okey(l);
      const double s = ((double)l - X.M) / c.T;
      w[r] = exp_neg_t(s, X.etab, X.etab + 64);
      esum += w[r];
      bool p = true;
      if (apply_minp) {
        p = s >= X.L;
        if (fabs(s - X.L) < X.Lclose) unc = 1;
      }
      if (p) { inP |= 1u << r; psum += w[r]; ++np_unc; }
    }
  }
  np_unc |= unc << 16;
  Gr::sum3(esum, psum, np_unc, F, 0);
  const uint32_t NP = np_unc & 0xffffu;
  unc = unc0 | (np_unc >> 16);

  // ---- the nucleus cut ------------------------------------------------------
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, ne, 8.0); }
  bool theta_set = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      unsigned long long wk = ~0ull;   // smallest weight (non-negative doubles order as u64)
#pragma unroll
      for (int r = 0; r < FE; ++r)
        if ((uint32_t)r < RE && p0 + (uint32_t)r < ne) {
          const unsigned long long b = __builtin_bit_cast(unsigned long long, w[r]);
          wk = b < wk ? b : wk;
        }
      const double wmin = __builtin_bit_cast(double, Gr::min_u64(wk, F));
      if (!minp_above_stall(c, esum) && !(wmin > 2.3e-16 * esum)) return false;   // the running sum may stall: replay
    } else {
      theta_set = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta_set = true;
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
  }
  uint32_t kept = inP;
  if (theta_set && !(psum + sum_bound(psum, NP, 8.0) < theta - theta_err)) {
    // The nucleus can end inside P.  P's keys, histogrammed with exact
    // fixed-point masses, in descending key order: the crossing bin is where
    // the mass prefix reaches theta; inside it the members are ordered by
    // (key desc, token ID asc), E positions being in token-ID order.
    uint32_t pkmin = NONE, pkmax = 0;
#pragma unroll
    for (int r = 0; r < FE; ++r)
      if ((inP >> r) & 1u) { pkmin = min(pkmin, ek[r]); pkmax = max(pkmax, ek[r]); }
    Gr::minmax_u32(pkmin, pkmax, F);
    const int sh = fast_shift(pkmin, pkmax, BITS);
    uint32_t* cnt = F.u.f.cnt;
    unsigned long long* mass = F.u.f.mass;
    reinterpret_cast<uint4*>(cnt)[gi] = make_uint4(0u, 0u, 0u, 0u);
    reinterpret_cast<ulonglong2*>(mass)[2 * gi] = make_ulonglong2(0ull, 0ull);
    reinterpret_cast<ulonglong2*>(mass)[2 * gi + 1] = make_ulonglong2(0ull, 0ull);
    F.u.f.mkey[gi] = 0u;   // pads the member list (key 0 is no finite logit's)
    if (gi == 0) { F.s_u[10] = 0u; F.s_u[11] = NONE; F.s_u[13] = 0u; }
    Gr::sync();
    unsigned long long W[FE];
#pragma unroll
    for (int r = 0; r < FE; ++r) {
      W[r] = __double2ull_rn(w[r] * WFIX);
      if ((inP >> r) & 1u) {
        const uint32_t b = (ek[r] >> sh) & (NBG - 1);
        atomicAdd(&cnt[b], 1u);
        atomicAdd(&mass[b], W[r]);
      }
    }
    Gr::sync();
    const double theta_fx = theta * WFIX;
    const uint4 h4 = reinterpret_cast<const uint4*>(cnt)[G - 1 - gi];
    const ulonglong2 m01 = reinterpret_cast<const ulonglong2*>(mass)[2 * (G - 1 - gi)];
    const ulonglong2 m23 = reinterpret_cast<const ulonglong2*>(mass)[2 * (G - 1 - gi) + 1];
    const uint32_t hv[4] = {h4.w, h4.z, h4.y, h4.x};
    const unsigned long long mv[4] = {m23.y, m23.x, m01.y, m01.x};
    unsigned long long mtot;
    unsigned long long before = Gr::excl_u64(mv[0] + mv[1] + mv[2] + mv[3], F.sc_l[0], &mtot);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (hv[i] && (double)before < theta_fx && theta_fx <= (double)(before + mv[i])) {
        F.s_u[8] = NBG - 1 - 4 * gi - (uint32_t)i;
        F.s_l[0] = before;
      }
      before += mv[i];
    }
    if (gi == 0 && !((double)mtot >= theta_fx)) F.s_u[8] = NONE;   // no crossing inside P
    Gr::sync();
    const uint32_t bstar = F.s_u[8];
    if (bstar == NONE) return false;
    const unsigned long long bbefore = F.s_l[0];
#pragma unroll
    for (int r = 0; r < FE; ++r) {
      if (((inP >> r) & 1u) && ((ek[r] >> sh) & (NBG - 1)) == bstar) {
        const uint32_t at = atomicAdd(&F.s_u[10], 1u);
        if (at < (uint32_t)G) {
          F.u.f.mkey[at] = ek[r];
          F.u.f.mpos[at] = p0 + r;
          F.u.f.mw[at] = W[r];
          // (key, ~position) in one word: ordered before <=> larger (the
          // mass histogram is read by now)
          if (G == FT) F.u.f.mass[at] = ((unsigned long long)ek[r] << 32) | (unsigned long long)(~(p0 + (uint32_t)r));
        }
      }
    }
    Gr::sync();
    const uint32_t cm = F.s_u[10];
    if (cm > (uint32_t)G) return false;
    const uint32_t mk = gi < cm ? F.u.f.mkey[gi] : 0u, mp = gi < cm ? F.u.f.mpos[gi] : 0u;
    const unsigned long long mwv = gi < cm ? F.u.f.mw[gi] : 0ull;
    unsigned long long ahead = 0;   // mass of the members ordered before this one
    if (G == 64) {
      // one wave: the members sit in lanes 0..cm-1; read them lane by lane
      for (uint32_t i = 0; i < cm; ++i) {
        const uint32_t k2 = (uint32_t)__builtin_amdgcn_readlane((int)mk, (int)i);
        const uint32_t p2 = (uint32_t)__builtin_amdgcn_readlane((int)mp, (int)i);
        const unsigned long long w2 = readlane64(mwv, i);
        if (k2 > mk || (k2 == mk && p2 < mp)) ahead += w2;
      }
    } else if (gi < cm) {
      // two members per 16-byte read of the packed (key, ~position) words
      // and of the weights (the crossing bin of a tied row holds hundreds)
      const unsigned long long my = ((unsigned long long)mk << 32) | (unsigned long long)(~mp);
      const unsigned long long* cp = F.u.f.mass;
      uint32_t i = 0;
      for (; i + 2u <= cm; i += 2u) {
        const ulonglong2 c2 = *reinterpret_cast<const ulonglong2*>(&cp[i]);
        const ulonglong2 w2 = *reinterpret_cast<const ulonglong2*>(&F.u.f.mw[i]);
        ahead += (c2.x > my ? w2.x : 0ull) + (c2.y > my ? w2.y : 0ull);
      }
      if (i < cm) ahead += cp[i] > my ? F.u.f.mw[i] : 0ull;
    }
    if (gi < cm) {
      const unsigned long long prev = bbefore + ahead, incl = prev + mwv;
      if ((double)prev < theta_fx && theta_fx <= (double)incl) {
        F.s_u[11] = mk;
        F.s_u[12] = mp;
        // Certificate: the fixed-point prefixes are exact sums of weights
        // rounded to 2^-51 (NP 2^-51 in all), the weights are within 8 ulp
        // of the reference's, and its sequential sums in sorted order are
        // within sum_bound; the f64 conversion adds one rounding.
        const double dp = (double)prev / WFIX, di = (double)incl / WFIX;
        const double fx = (double)NP * 0x1p-51;
        const double ep = sum_bound(dp, NP, 8.0) + fx + U * dp, ei = sum_bound(di, NP, 8.0) + fx + U * di;
        if (!(dp + ep < theta - theta_err) || !(di - ei >= theta + theta_err)) F.s_u[13] = 1u;
      }
    }
    Gr::sync();
    const uint32_t cut_key = F.s_u[11], cut_pos = F.s_u[12];
    if (cut_key == NONE || F.s_u[13]) return false;   // uncertain cut: replay
    kept = 0;
#pragma unroll
    for (int r = 0; r < FE; ++r)
      if (((inP >> r) & 1u) && (ek[r] > cut_key || (ek[r] == cut_key && p0 + (uint32_t)r <= cut_pos))) kept |= 1u << r;
  }

  // ---- overflow check and the inverse-CDF draw in token-ID order ----------
  double kpart = 0.0;
  uint32_t kn = 0;
  bool bad = false;
#pragma unroll
  for (int r = 0; r < FE; ++r) {
    if (!((kept >> r) & 1u)) continue;
    kpart += w[r];
    ++kn;
    if (!isfinite(((double)okey_value(ek[r]) - X.M) / c.T)) bad = true;
  }
  if (gi == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; F.s_u[3] = 0u; }
  uint32_t nkept;
  (void)Gr::excl_u32(kn | (bad ? 0x10000u : 0u), F.sc_u[1], &nkept);
  const bool any_bad = (nkept >> 16) != 0u;
  nkept &= 0xffffu;
  double S;
  const double kinc = Gr::incl_f64(kpart, F.sc_d[0], &S);
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  double cum = kinc - kpart;
  uint32_t lastp = 0u;   // this lane's last positive kept weight, position + 1
#pragma unroll
  for (int r = 0; r < FE; ++r) {
    if (!((kept >> r) & 1u)) continue;
    const double prev = cum;
    cum += w[r];
    if (w[r] > 0.0) {
      lastp = p0 + (uint32_t)r + 1u;
      if (target < cum && !(target < prev)) {
        F.s_u[0] = p0 + (uint32_t)r;
        if (fabs(target - prev) <= derr || fabs(cum - target) <= derr) F.s_u[2] = 1u;
      }
    }
  }
  {   // one LDS atomic per wave, not per kept slot (they all hit one word)
    const uint32_t lp = wave_max_u32(lastp);
    if (lane() == 0 && lp) atomicMax(&F.s_u[1], lp);
  }
  Gr::sync();
  if (any_bad) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return true; }
  bool uncert = unc != 0u || (F.s_u[2] != 0u && !X.nodraw);
  uint32_t pick = F.s_u[0];
  if (pick == NONE) {
    // rounding left the variate past the accumulated mass: last positive kept token
    pick = F.s_u[1] ? F.s_u[1] - 1u : NONE;
    uncert = uncert || !X.nodraw;
  }
  if (pick == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return true; }
  const uint32_t jp = F.eidx[pick];
  const double shifted = ((double)F.cl[jp] - X.M) / c.T;
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)F.cid[jp], shifted - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = gi; q < X.nwords; q += G) X.kbits[q] = 0u;
    __builtin_amdgcn_s_waitcnt(0);   // the zeroing lands before the atomics (one group, in program order)
    if (G == FT) __syncthreads();
#pragma unroll
    for (int r = 0; r < FE; ++r) {
      if (!((kept >> r) & 1u)) continue;
      const uint32_t tok = F.cid[F.eidx[p0 + r]];
      atomicOr(&X.kbits[tok >> 5], 1u << (tok & 31u));
    }
  }
  return true;
}

// The E phase on one wave (at most 256 E tokens; the other waves wait for
// its verdict) or on the workgroup.
__device__ __forceinline__ bool finish_e(const FinCtx& X, FinSmem& F, uint32_t ne, uint32_t unc) {
  if (ne <= 256u) {
    if (wave() == 0) {
      const bool ok = e_finish<64>(X, F, ne, unc);
      if (lane() == 0) F.s_u[15] = ok ? 1u : 0u;
    }
    lds_barrier();
    return F.s_u[15] != 0u;
  }
  return e_finish<FT>(X, F, ne, unc);
}

// ---------------------------------------------------------------------------
// The row finish on one wave, for rows with at most WR * 64 candidates (lane
// l holds candidates WR l .. WR l + WR - 1, so lane order is token-ID order).
// Every step is a wave operation (DPP, ballots, LDS ops that complete in
// order within the wave): no workgroup barrier between the candidate load
// and the result.  The decisions and their certificates are e_finish's; a
// row this path cannot certify returns false having written nothing.
constexpr int WR = 8;

// Lanes of one wave exchange data through LDS below: the hardware completes
// one wave's LDS operations in order, and this compiler barrier keeps a
// lane's own earlier store from being forwarded to its later load of a
// location another lane has written since.
__device__ __forceinline__ void wave_lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// The k-th largest (1 <= k <= active count) of the wave's active keys (WR
// per lane) and how many are larger: radix select on 8-bit digits from the
// highest bit where the keys differ, over a 256-bin LDS histogram.
__device__ __forceinline__ bool wave_kth(uint32_t* h, const uint32_t (&key)[WR], uint32_t act, uint32_t k,
                                         uint32_t* kappa, uint32_t* above) {
  const uint32_t ln = lane();
  uint32_t kmin = NONE, kmax = 0;
#pragma unroll
  for (int r = 0; r < WR; ++r)
    if ((act >> r) & 1u) { kmin = min(kmin, key[r]); kmax = max(kmax, key[r]); }
  kmin = ~wave_max_u32(~kmin);
  kmax = wave_max_u32(kmax);
  if (kmin == kmax) { *kappa = kmax; *above = 0u; return true; }
  int hb = 31 - (int)__builtin_clz(kmin ^ kmax);
  uint32_t pmask = hb >= 31 ? 0u : ~((2u << hb) - 1u);
  uint32_t prefix = kmax & pmask, need = k, abv = 0;
  while (hb >= 0) {
    const int sh = hb >= 7 ? hb - 7 : 0;
    const uint32_t dm = (2u << (hb - sh)) - 1u;
    *reinterpret_cast<uint4*>(&h[4u * ln]) = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if (((act >> r) & 1u) && (key[r] & pmask) == prefix) atomicAdd(&h[(key[r] >> sh) & dm], 1u);
    wave_lds_sync();
    // lane l reads bins 255 - 4l .. 252 - 4l: lane order is descending digit order
    const uint4 v = *reinterpret_cast<const uint4*>(&h[252u - 4u * ln]);
    const uint32_t c4[4] = {v.w, v.z, v.y, v.x};
    const uint32_t s = c4[0] + c4[1] + c4[2] + c4[3];
    const uint32_t inc = wave_scan_u32(s);
    const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
    if (!reach) return false;   // fewer active keys than k: the caller's contract is broken
    const uint32_t L = (uint32_t)__builtin_ctzll(reach);
    uint32_t run = inc - s, dig = 0u, bef = 0u;
    bool found = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!found && run + c4[i] >= need) { found = true; dig = 255u - 4u * ln - (uint32_t)i; bef = run; }
      run += c4[i];
    }
    dig = (uint32_t)__builtin_amdgcn_readlane((int)dig, (int)L);
    bef = (uint32_t)__builtin_amdgcn_readlane((int)bef, (int)L);
    need -= bef;
    abv += bef;
    prefix |= dig << sh;
    pmask |= dm << sh;
    hb = sh - 1;
  }
  *kappa = prefix;
  *above = abv;
  return true;
}

// Bitonic sort of one (key, position) pair per lane into descending key
// order, ascending position among equal keys (sort_key order).
__device__ __forceinline__ unsigned long long wave_sort_desc(unsigned long long v) {
  const uint32_t ln = lane();
#pragma unroll
  for (uint32_t size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
      const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, (int)stride);
      const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), (int)stride);
      const unsigned long long o = ((unsigned long long)hi << 32) | lo;
      // descending blocks when (lane & size) == 0; the lower lane keeps the larger
      const bool desc = (ln & size) == 0u;
      const bool lower = (ln & stride) == 0u;
      const bool take_max = desc == lower;
      v = take_max ? (o > v ? o : v) : (o < v ? o : v);
    }
  }
  return v;
}

__device__ __forceinline__ bool wave_finish(const FinCtx& X, FinSmem& F) {
  const RowCfg& c = X.c;
  const uint32_t n = X.ncand, ln = lane(), j0 = ln * (uint32_t)WR;
  if (n == 0u) return false;
  float lv[WR];
  uint32_t key[WR];
  uint32_t act = 0;
  {
    const float4 a0 = *reinterpret_cast<const float4*>(&F.cl[j0]);
    const float4 a1 = *reinterpret_cast<const float4*>(&F.cl[j0 + 4u]);
    lv[0] = a0.x; lv[1] = a0.y; lv[2] = a0.z; lv[3] = a0.w;
    lv[4] = a1.x; lv[5] = a1.y; lv[6] = a1.z; lv[7] = a1.w;
  }
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    const bool a = j0 + (uint32_t)r < n;
    act |= a ? 1u << r : 0u;
    key[r] = a ? okey(lv[r]) : 0u;
  }

  // ---- E: the top-k head, the exact min-p set, or every candidate --------
  uint32_t inE = 0;
  bool unc = false;
  double s[WR];
#pragma unroll
  for (int r = 0; r < WR; ++r) s[r] = ((act >> r) & 1u) ? ((double)lv[r] - X.M) / c.T : 0.0;
  if (X.k_path) {
    if (c.k > n) return false;
    uint32_t kappa, above;
    if (!wave_kth(F.u.f.cnt, key, act, c.k, &kappa, &above)) return false;
    // the keys above kappa and the first (k - above) ties at kappa in token-ID order
    const uint32_t need_t = c.k - above;
    uint32_t tie = 0;
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      if (!((act >> r) & 1u)) continue;
      if (key[r] > kappa) inE |= 1u << r;
      if (key[r] == kappa) tie |= 1u << r;
    }
    const uint32_t tc = (uint32_t)__builtin_popcount(tie);
    uint32_t t = wave_scan_u32(tc) - tc;
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if ((tie >> r) & 1u) { if (t < need_t) inE |= 1u << r; ++t; }
  } else if (X.mode == M_MINP) {
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      if (!((act >> r) & 1u)) continue;
      if (s[r] >= X.L) inE |= 1u << r;
      if (fabs(s[r] - X.L) < X.Lclose) unc = true;
    }
  } else {
    inE = act;
  }

  // ---- weights, the min-p subset P and the sums ---------------------------
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  double w[WR];
  uint32_t inP = 0, ne = 0, np = 0;
  double esum = 0.0, psum = 0.0;
  unsigned long long wmin = ~0ull;   // smallest weight (non-negative doubles order as u64)
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    w[r] = 0.0;
    if (!((inE >> r) & 1u)) continue;
    w[r] = exp_neg_t(s[r], X.etab, X.etab + 64);
    esum += w[r];
    ++ne;
    const unsigned long long bits = __builtin_bit_cast(unsigned long long, w[r]);
    wmin = bits < wmin ? bits : wmin;
    bool p = true;
    if (apply_minp) {
      p = s[r] >= X.L;
      if (fabs(s[r] - X.L) < X.Lclose) unc = true;
    }
    if (p) { inP |= 1u << r; psum += w[r]; ++np; }
  }
  esum = wave_sum_f64(esum);
  psum = wave_sum_f64(psum);
  const uint32_t cnts = wave_sum_u32(ne | (np << 16));
  ne = cnts & 0xffffu;
  np = cnts >> 16;
  unc = __builtin_amdgcn_ballot_w64(unc) != 0ull;
  if (ne == 0u) return false;

  // ---- the nucleus cut ------------------------------------------------------
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, ne, 8.0); }
  bool theta_set = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      // the running sum may stall before reaching the total: the general path replays it
      const double wm = __builtin_bit_cast(double, ~wave_max_u64(~wmin));
      if (!minp_above_stall(c, esum) && !(wm > 2.3e-16 * esum)) return false;
    } else {
      theta_set = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta_set = true;
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
  }
  uint32_t kept = inP;
  if (theta_set && !(psum + sum_bound(psum, np, 8.0) < theta - theta_err)) {
    // The nucleus can end inside P: sort P (at most 64 members, one per
    // lane) by (key desc, token ID asc) and walk the prefix sums.
    if (np > 64u) return false;
    const uint32_t pc = (uint32_t)__builtin_popcount(inP);
    uint32_t at = wave_scan_u32(pc) - pc;
    unsigned long long* mk = F.u.f.mass;   // sort keys (key << 32 | ~position), slot by P rank
    double* mw = reinterpret_cast<double*>(F.u.f.mw);
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if ((inP >> r) & 1u) {
        mk[at] = ((unsigned long long)key[r] << 32) | (unsigned long long)(~(j0 + (uint32_t)r));
        mw[at] = w[r];
        ++at;
      }
    wave_lds_sync();
    const bool mine = ln < np;
    const unsigned long long sk = wave_sort_desc(mine ? mk[ln] : 0ull);
    const uint32_t pos = ~(uint32_t)sk;   // candidate index of this lane's sorted member
    // the member's weight, fetched by its P rank: P ranks follow candidate order
    uint32_t wr = 0;
    if (mine) {
      // rank of `pos` in P = number of P members before it in candidate order;
      // search the rank table written above
      for (uint32_t i = 0; i < np; ++i) wr += (~(uint32_t)mk[i]) < pos ? 1u : 0u;
    }
    const double wv = mine ? mw[wr] : 0.0;
    const double cum = wave_scan_f64(wv);   // inclusive, in sorted order
    const double prev = cum - wv;
    // the reference stops at the first member whose running sum reaches theta
    const double e_i = sum_bound(cum, ln + 1u, 8.0), e_p = sum_bound(prev, ln + 1u, 8.0);
    const bool reach = mine && cum >= theta;
    const uint64_t rb = __builtin_amdgcn_ballot_w64(reach);
    if (!rb) return false;   // the bound allowed a crossing the sums do not show: replay
    const uint32_t istar = (uint32_t)__builtin_ctzll(rb);
    const bool cert_i = cum - e_i >= theta + theta_err;
    const bool cert_p = ln == 0u || prev + e_p < theta - theta_err;
    if (!__builtin_amdgcn_readlane((int)(cert_i && cert_p), (int)istar)) return false;
    // kept = the sorted members 0 .. istar: flag them by candidate index
    uint8_t* kf = F.kflag;
#pragma unroll
    for (int r = 0; r < WR; ++r) kf[j0 + (uint32_t)r] = 0u;
    wave_lds_sync();
    if (mine && ln <= istar) kf[pos] = 1u;
    wave_lds_sync();
    kept = 0;
#pragma unroll
    for (int r = 0; r < WR; ++r) kept |= kf[j0 + (uint32_t)r] ? 1u << r : 0u;
  }

  // ---- overflow check and the inverse-CDF draw in token-ID order ----------
  double kpart = 0.0;
  uint32_t kn = 0;
  bool bad = false;
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    if (!((kept >> r) & 1u)) continue;
    kpart += w[r];
    ++kn;
    if (!isfinite(s[r])) bad = true;
  }
  const uint32_t nkept = wave_sum_u32(kn);
  if (__builtin_amdgcn_ballot_w64(bad)) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return true; }
  const double kinc = wave_scan_f64(kpart);
  const double S = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, kinc), 63));
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  double cum = kinc - kpart;
  uint32_t found = NONE, last = NONE;
  bool fnear = false;
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    if (!((kept >> r) & 1u)) continue;
    const double prev = cum;
    cum += w[r];
    if (w[r] > 0.0) {
      last = j0 + (uint32_t)r;
      if (found == NONE && target < cum && !(target < prev)) {
        found = j0 + (uint32_t)r;
        fnear = fabs(target - prev) <= derr || fabs(cum - target) <= derr;
      }
    }
  }
  bool uncert = unc;
  uint32_t pick = NONE;
  const uint64_t fb = __builtin_amdgcn_ballot_w64(found != NONE);
  if (fb) {
    const uint32_t L = (uint32_t)__builtin_ctzll(fb);
    pick = (uint32_t)__builtin_amdgcn_readlane((int)found, (int)L);
    uncert = uncert || (__builtin_amdgcn_readlane((int)fnear, (int)L) != 0 && !X.nodraw);
  } else {
    // rounding left the variate past the accumulated mass: the last positive kept token
    const uint64_t lb = __builtin_amdgcn_ballot_w64(last != NONE);
    if (lb) pick = (uint32_t)__builtin_amdgcn_readlane((int)last, (int)(63 - __builtin_clzll(lb)));
    uncert = uncert || !X.nodraw;
  }
  if (pick == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return true; }
  const double shifted = ((double)F.cl[pick] - X.M) / c.T;
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)F.cid[pick], shifted - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = ln; q < X.nwords; q += 64u) X.kbits[q] = 0u;
    __builtin_amdgcn_s_waitcnt(0);   // the zeroing lands before the atomics (one wave, in program order)
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      if (!((kept >> r) & 1u)) continue;
      const uint32_t tok = F.cid[j0 + (uint32_t)r];
      atomicOr(&X.kbits[tok >> 5], 1u << (tok & 31u));
    }
  }
  return true;
}

__device__ __forceinline__ bool finish_fast(const FinCtx& X, FinSmem& F) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x;
  const uint32_t n = X.ncand;
  if (X.timing) X.timing[((uint64_t)X.row * (MAXC + 1) + MAXC) * TSTAMPS + 3] = n;   // candidate count (diagnostics)
  if (n == 0 || n > (uint32_t)CCAP || !X.lds_c) return false;
  const uint32_t R = (n + FT - 1u) / FT;
  const uint32_t j0 = tid * R;
  uint32_t key[FR];
  uint32_t act = 0;
#pragma unroll
  for (int r = 0; r < FR; ++r) {
    const bool a = (uint32_t)r < R && j0 + (uint32_t)r < n;
    key[r] = a ? okey(F.cl[j0 + r]) : 0u;
    act |= a ? 1u << r : 0u;
  }

  // ---- E: the top-k head, the exact min-p set, or every candidate --------
  uint32_t inE = 0, unc = 0;
  if (X.k_path) {
    if (c.k > (uint32_t)ECAP) return false;
    uint32_t kmin = NONE, kmax = 0;
#pragma unroll
    for (int r = 0; r < FR; ++r)
      if ((act >> r) & 1u) { kmin = min(kmin, key[r]); kmax = max(kmax, key[r]); }
    Grp<FT>::minmax_u32(kmin, kmax, F);
    uint32_t kappa, above;
    if (!fast_kth(F, key, act, c.k, kmin, kmax, &kappa, &above)) return false;
    // E = the keys above kappa and the first (k - above) ties at kappa in
    // token-ID order: one scan of (above count << 16 | tie count) places
    // both (at most FR each per thread, k <= ECAP in all).
    uint32_t gt = 0, nt = 0;
#pragma unroll
    for (int r = 0; r < FR; ++r)
      if ((act >> r) & 1u) { gt += key[r] > kappa; nt += key[r] == kappa; }
    uint32_t ttot;
    const uint32_t ex = block_excl_scan_u32((gt << 16) | nt, F.sc_u[1], &ttot);
    const uint32_t need_t = c.k - above;
    uint32_t tb = ex & 0xffffu;
    uint32_t ep = (ex >> 16) + min(need_t, tb);
#pragma unroll
    for (int r = 0; r < FR; ++r) {
      if (!((act >> r) & 1u)) continue;
      bool in = key[r] > kappa;
      if (key[r] == kappa) { in = tb < need_t; ++tb; }
      if (in) F.eidx[ep++] = j0 + r;
    }
    lds_barrier();
    fstamp(X, 4);
    return finish_e(X, F, c.k, 0u);
  } else if (X.mode == M_MINP) {
#pragma unroll
    for (int r = 0; r < FR; ++r) {
      if (!((act >> r) & 1u)) continue;
      const double s = ((double)F.cl[j0 + r] - X.M) / c.T;
      if (s >= X.L) inE |= 1u << r;
      if (fabs(s - X.L) < X.Lclose) unc = 1;
    }
  } else {
    inE = act;
  }
  uint32_t ne;
  uint32_t ep = block_excl_scan_u32((uint32_t)__builtin_popcount(inE) | (unc << 16), F.sc_u[0], &ne);
  unc = ne >> 16 ? 1u : 0u;
  ne &= 0xffffu;
  ep &= 0xffffu;
  if (ne == 0 || ne > (uint32_t)ECAP) return false;
#pragma unroll
  for (int r = 0; r < FR; ++r)
    if ((inE >> r) & 1u) F.eidx[ep++] = j0 + r;
  lds_barrier();
  fstamp(X, 4);
  return finish_e(X, F, ne, unc);
}

// ---------------------------------------------------------------------------
// The finisher's candidate slots.  For C <= FW chunks, wave w serves chunk
// w mod C as its (w div C)-th wave, so a row's chunks spread over the four
// SIMDs (wave w runs on SIMD w mod 4) and lane order within a wave is
// candidate order; for C > FW, thread t serves chunk t div (FT / C).
// Thread (q, j) holds slots SR j .. SR j + SR - 1 of chunk q, so every
// chunk's first slot_cov(C) slots are in registers.
__device__ __forceinline__ void slot_map(uint32_t C, uint32_t* q, uint32_t* j) {
  const uint32_t tid = threadIdx.x;
  if (C <= (uint32_t)FW) {
    const uint32_t w = tid >> 6;
    *q = w % C;
    *j = (w / C) * 64u + (tid & 63u);
  } else {
    const uint32_t spc = FT / C;
    *q = tid / spc;
    *j = tid - *q * spc;
  }
}
__device__ __forceinline__ uint32_t slot_cov(uint32_t C) {
  return C <= (uint32_t)FW ? (uint32_t)SR * 64u * ((uint32_t)FW / C) : (uint32_t)SR * ((uint32_t)FT / C);
}

// The finisher's first loads, issued before anything waits: the chunk
// statistics (waves 0 and 1, lane q <-> chunk q) and the register slots
// (slot_map).  Slots past a chunk's count hold stale values and are
// ignored once the statistics are in.
struct FinLoads {
  float l[SR];
  uint32_t id[SR];
  ChunkStat v;
};
static_assert(SR % 2 == 0, "slot pairs");
__device__ __forceinline__ void fin_issue(const SampleArgs& A, uint32_t row, FinLoads& P) {
  const uint32_t C = A.C, V = A.b.vocab, CH = A.CH;
  uint32_t sq, sj;
  slot_map(C, &sq, &sj);
  // the row's region ends at V, the chunk's at CH: slots below both are in bounds
  const uint32_t lim = sq < C ? min(CH, V - sq * CH) : 0u;
  const uint64_t base = (uint64_t)row * V + (uint64_t)sq * CH + (uint64_t)sj * SR;
  // an even vocabulary makes base even (CH and SR are): 8-byte pairs
  const bool pairs = (V & 1u) == 0u;
#pragma unroll
  for (int u = 0; u < SR; u += 2) {
    const uint32_t slot = sj * (uint32_t)SR + (uint32_t)u;
    float2 lv = make_float2(0.0f, 0.0f);
    uint2 iv = make_uint2(0u, 0u);
    if (pairs && slot + 1u < lim) {
      lv = ld_dev(reinterpret_cast<const float2*>(&A.w.cand_l[base + u]));
      iv = ld_dev(reinterpret_cast<const uint2*>(&A.w.cand_id[base + u]));
    } else {
      if (slot < lim) {
        lv.x = ld_dev(&A.w.cand_l[base + u]);
        iv.x = ld_dev(&A.w.cand_id[base + u]);
      }
      if (slot + 1u < lim) {
        lv.y = ld_dev(&A.w.cand_l[base + u + 1]);
        iv.y = ld_dev(&A.w.cand_id[base + u + 1]);
      }
    }
    P.l[u] = lv.x; P.l[u + 1] = lv.y;
    P.id[u] = iv.x; P.id[u + 1] = iv.y;
  }
  ChunkStat& v = P.v;
  v.maxkey = 0u; v.gbest_id = NONE; v.gbest_val = 0.0f; v.nlegal = 0u; v.ncand = 0u; v.flags = 0u;
  v.minkey = NONE; v.thr = 0.0f; v.mass = 0.0; v.mass_err = 0.0;
  if (wave() < 2u && lane() < C) {   // wave 0: the header; wave 1: the chunk masses
    const ChunkStat* st = &A.w.stat[(uint64_t)row * MAXC + lane()];
    v.maxkey = ld_dev(&st->maxkey);
    v.gbest_id = ld_dev(&st->gbest_id);
    v.gbest_val = ld_dev(&st->gbest_val);
    v.nlegal = ld_dev(&st->nlegal);
    v.ncand = ld_dev(&st->ncand);
    v.flags = ld_dev(&st->flags);
    v.mass = ld_dev(&st->mass);
    v.mass_err = ld_dev(&st->mass_err);
    v.minkey = ld_dev(&st->minkey);
    v.thr = ld_dev(&st->thr);
  }
}

// ---------------------------------------------------------------------------
// The selection finisher: top-k and min-p rows of at most FW chunks whose
// candidates all sit in the register slots (slot_map: lane order within a
// wave is candidate order; waves order by (chunk, rank in the chunk)).  The
// decisions and their certificates
// are wave_finish's and e_finish's; the work is spread differently:
//   - E's top-k bound comes from a value histogram of the register-held
//     candidates: bin (M - l) (NBS - 1) / (M - lo) is non-increasing in l
//     (each f32 step is monotone), so the k-th largest candidate lies in the
//     first bin where the running count from bin 0 reaches k; the crossing
//     bin's members (at most PCAP) are ranked by (key desc, ID asc);
//   - E's mass (which only sets theta = top_p * mass) is summed from f32
//     weights 2^((l - M) log2(e) / T) with an error bound, like the chunk
//     masses; only P's members (E with the min-p test, decided in f32 away
//     from the threshold and in f64 near it) get f64 weights;
//   - P is compacted in token-ID order by a block scan; P of at most 64
//     members is finished by one wave (lane = P member), larger P (at most
//     PMAX) by the workgroup: the nucleus cut from a fixed-point mass
//     histogram on the same value bins, the draw from a block scan.
// Returns false, having written nothing, for the general paths; every
// early return is taken by all waves alike (it depends only on values
// every wave computes identically, or on LDS read after a barrier).
struct SelSums {
  double esum, esum_err;   // E's mass (from f32 weights) and its error bound
  double wlo;              // a lower bound of E's smallest weight
  uint32_t ne, np;
  bool unc;
};

// The value bin of logit l (non-increasing in l; l <= M).
__device__ __forceinline__ uint32_t sel_bin(float l, float Mf, float sc) {
  const float d = (Mf - l) * sc;
  return d < (float)(NBS - 1) ? (uint32_t)d : (uint32_t)(NBS - 1);
}

// theta (the nucleus mass) and its error; false when the general path must
// replay the row
__device__ __forceinline__ bool sel_theta(const FinCtx& X, const SelSums& Q, bool* set, double* theta,
                                          double* theta_err) {
  const RowCfg& c = X.c;
  *set = false;
  *theta = 0.0;
  *theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      // the running sum may stall before reaching the total
      if (!minp_above_stall(c, Q.esum + Q.esum_err) && !(Q.wlo > 2.3e-16 * (Q.esum + Q.esum_err))) return false;
    } else {
      *set = true;
      *theta = c.top_p * Q.esum;
      *theta_err = c.top_p * Q.esum_err + U * *theta;
    }
  } else if (c.top_p < 1.0) {
    const double total = X.have_total ? X.total : Q.esum;
    const double total_err = X.have_total ? X.total_err : Q.esum_err;
    *set = true;
    *theta = c.top_p * total;
    *theta_err = c.top_p * total_err + U * *theta;
  }
  return true;
}

// The first position (0-based) where an inclusive prefix of the wave's
// lane-ordered counts reaches `need`, scanning 32-entry groups: lane i holds
// the total of group i (hs) and its inclusive scan (inc); the crossing
// group's 32 entries are then read lane-parallel from `h`.  Returns NONE
// when the total stays below need; *before receives the count ahead of the
// position.
__device__ __forceinline__ uint32_t wave_cross32(const uint32_t* h, uint32_t hs, uint32_t inc, uint32_t need,
                                                 uint32_t* before) {
  const uint32_t ln = lane();
  const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
  if (!reach) return NONE;
  const uint32_t g = (uint32_t)__builtin_ctzll(reach);
  const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - hs), (int)g);
  const uint32_t v = ln < 32u ? h[32u * g + ln] : 0u;
  const uint32_t vi = base + wave_scan_u32(v);
  const uint64_t r2 = __builtin_amdgcn_ballot_w64(ln < 32u && vi >= need);
  const uint32_t i = (uint32_t)__builtin_ctzll(r2);
  *before = (uint32_t)__builtin_amdgcn_readlane((int)(vi - v), (int)i);
  return 32u * g + i;
}

// The draw over the kept members of P in token-ID order (one wave: lane =
// member); writes the result.
__device__ __forceinline__ void sel_draw_wave(const FinCtx& X, bool kept, double w, double s, uint32_t id, bool unc) {
  const RowCfg& c = X.c;
  const uint32_t nkept = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(kept));
  if (__builtin_amdgcn_ballot_w64(kept && !isfinite(s))) {
    write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
    return;
  }
  const double dw = kept ? w : 0.0;
  const double inc = wave_scan_f64(dw);
  const double S = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, inc), 63));
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  const double before = inc - dw;
  const bool hit = dw > 0.0 && target < inc && !(target < before);
  const bool near = fabs(target - before) <= derr || fabs(inc - target) <= derr;
  bool uncert = unc;
  uint32_t pick = NONE;
  const uint64_t fb = __builtin_amdgcn_ballot_w64(hit);
  if (fb) {
    pick = (uint32_t)__builtin_ctzll(fb);
    uncert = uncert || (__builtin_amdgcn_readlane((int)near, (int)pick) != 0 && !X.nodraw);
  } else {
    // rounding left the variate past the accumulated mass: the last positive kept token
    const uint64_t lb = __builtin_amdgcn_ballot_w64(dw > 0.0);
    if (lb) pick = (uint32_t)(63 - __builtin_clzll(lb));
    uncert = uncert || !X.nodraw;
  }
  if (pick == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  const int32_t tok = __builtin_amdgcn_readlane((int)id, (int)pick);
  const double sp = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, s), pick));
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, tok, sp - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = lane(); q < X.nwords; q += 64u) X.kbits[q] = 0u;
    __builtin_amdgcn_s_waitcnt(0);   // the zeroing lands before the atomics (one wave, in program order)
    if (kept) atomicOr(&X.kbits[id >> 5], 1u << (id & 31u));
  }
}

// P of at most 64 members, on one wave: lane i holds P member i (ID order).
__device__ __forceinline__ bool sel_small(const FinCtx& X, FinSmem& F, const SelSums& Q) {
  const RowCfg& c = X.c;
  const uint32_t ln = lane(), np = Q.np;
  const bool mine = ln < np;
  const uint32_t mk = mine ? F.u.s.pk[ln] : 0u, mi = mine ? F.u.s.pid[ln] : NONE;
  const float ml = mine ? F.u.s.pl[ln] : 0.0f;
  const double s = mine ? ((double)ml - X.M) / c.T : 0.0;
  const double mw = mine ? exp_neg_t(s, X.etab, X.etab + 64) : 0.0;
  const double psum = wave_sum_f64(mw);
  bool theta_set;
  double theta, theta_err;
  if (!sel_theta(X, Q, &theta_set, &theta, &theta_err)) return false;
  bool kept = mine;
  if (theta_set && !(psum + sum_bound(psum, np, 8.0) < theta - theta_err)) {
    // The nucleus can end inside P: prefix sums in (key desc, ID asc)
    // order; the reference stops at the first member whose running sum
    // reaches theta.
    uint32_t rk = 0;
    for (uint32_t j = 0; j < np; ++j) {
      const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)mk, (int)j);
      const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)mi, (int)j);
      rk += (kj > mk || (kj == mk && ij < mi)) ? 1u : 0u;
    }
    double* sw = F.u.s.sw;
    if (mine) sw[rk] = mw;
    wave_lds_sync();
    const double wv = mine ? sw[ln] : 0.0;
    const double cum = wave_scan_f64(wv);   // inclusive, in rank order
    const double prev = cum - wv;
    const double e_i = sum_bound(cum, ln + 1u, 8.0), e_p = sum_bound(prev, ln + 1u, 8.0);
    const uint64_t rb = __builtin_amdgcn_ballot_w64(mine && cum >= theta);
    if (!rb) return false;   // the bound allowed a crossing the sums do not show: replay
    const uint32_t istar = (uint32_t)__builtin_ctzll(rb);
    const bool cert_i = cum - e_i >= theta + theta_err;
    const bool cert_p = ln == 0u || prev + e_p < theta - theta_err;
    if (!__builtin_amdgcn_readlane((int)(cert_i && cert_p), (int)istar)) return false;
    kept = mine && rk <= istar;
  }
  sel_draw_wave(X, kept, mw, s, mi, Q.unc);
  return true;
}

// P of more than 64 (at most PMAX = FT) members, on the workgroup: thread i
// holds P member i (ID order).
__device__ __forceinline__ bool sel_large(const FinCtx& X, FinSmem& F, const SelSums& Q) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x, np = Q.np;
  const bool mine = tid < np;
  const uint32_t mk = mine ? F.u.s.pk[tid] : 0u, mi = mine ? F.u.s.pid[tid] : NONE;
  const float ml = mine ? F.u.s.pl[tid] : 0.0f;
  const double s = mine ? ((double)ml - X.M) / c.T : 0.0;
  const double mw = mine ? exp_neg_t(s, X.etab, X.etab + 64) : 0.0;
  // theta, and whether the nucleus can end inside P (P's f32 mass could not
  // rule it out), come from finish_sel
  const bool cut = F.s_u[15] != 0u;
  bool kept = mine;
  if (cut) {
    // The nucleus can end inside P.  P's weights, as exact fixed-point
    // masses, histogrammed on the value bins; the bin where the mass prefix
    // in descending value order reaches theta, then its members ranked by
    // (key desc, ID asc), give the crossing member, certified as e_finish
    // does.
    const double theta = F.s_d[3], theta_err = F.s_d[4];
    const double theta_fx = theta * WFIX;
    // integer threshold: the first prefix at or above theta_fx
    const unsigned long long tfx = (unsigned long long)ceil(theta_fx);
    const float Mf = okey_value(F.hdr.Mkey), lo = F.hdr.lo;
    const float span = Mf - lo;
    const float sc = span > 1e-30f ? (float)(NBS - 1) / span : 0.0f;
    unsigned long long* mass = F.u.s.mass;
    const unsigned long long W = __double2ull_rn(mw * WFIX);
    const uint32_t bn = sel_bin(ml, Mf, sc);
    if (mine) atomicAdd(&mass[bn], W);
    if (tid == 0) F.s_u[10] = 0u;
    lds_barrier();
    if (wave() == 0) {
      // lane i: bins 32i .. 32i + 31; the crossing group, then its bins lane-parallel
      const uint32_t ln = lane();
      unsigned long long hs = 0;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const ulonglong2 m2 = *reinterpret_cast<const ulonglong2*>(&mass[32u * ln + 2u * (uint32_t)q]);
        hs += m2.x + m2.y;
      }
      const unsigned long long inc = wave_scan_u64(hs);
      const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= tfx);
      uint32_t bc = NONE, nocut = 0u;
      unsigned long long bb = 0;
      if (!reach) {
        // P's exact mass stays below theta: every member is kept when the
        // bound clears it
        const double dt = (double)readlane64(inc, 63) / WFIX;
        const double et = sum_bound(dt, np, 8.0) + (double)np * 0x1p-51 + U * dt;
        nocut = dt + et < theta - theta_err ? 1u : 0u;
      } else {
        const uint32_t g = (uint32_t)__builtin_ctzll(reach);
        const unsigned long long base = readlane64(inc - hs, g);
        const unsigned long long v = ln < 32u ? mass[32u * g + ln] : 0ull;
        const unsigned long long vi = base + wave_scan_u64(v);
        const uint64_t r2 = __builtin_amdgcn_ballot_w64(ln < 32u && vi >= tfx);
        const uint32_t i = (uint32_t)__builtin_ctzll(r2);
        bc = 32u * g + i;
        bb = readlane64(vi - v, i);
      }
      if (ln == 0) { F.s_u[12] = bc; F.s_u[13] = nocut; F.s_l[0] = bb; }
    }
    lds_barrier();
    const uint32_t bc = F.s_u[12];
    if (bc == NONE && !F.s_u[13]) return false;   // no certified crossing or total: replay
  }
  if (cut && F.s_u[12] != NONE) {
    const double theta = F.s_d[3], theta_err = F.s_d[4];
    const double theta_fx = theta * WFIX;
    const float Mf = okey_value(F.hdr.Mkey), lo = F.hdr.lo;
    const float span = Mf - lo;
    const float sc = span > 1e-30f ? (float)(NBS - 1) / span : 0.0f;
    const unsigned long long W = __double2ull_rn(mw * WFIX);
    const uint32_t bn = sel_bin(ml, Mf, sc);
    const uint32_t bc = F.s_u[12];
    if (mine && bn == bc) {
      const uint32_t at = atomicAdd(&F.s_u[10], 1u);
      if (at < 64u) { F.u.s.mk[at] = mk; F.u.s.mi[at] = mi; F.u.s.mw[at] = W; }
    }
    lds_barrier();
    const uint32_t cm = F.s_u[10];
    if (cm > 64u) return false;
    if (wave() == 0) {
      const uint32_t ln = lane();
      const bool mm = ln < cm;
      const uint32_t a = mm ? F.u.s.mk[ln] : 0u, bi = mm ? F.u.s.mi[ln] : NONE;
      const unsigned long long aw = mm ? F.u.s.mw[ln] : 0ull;
      unsigned long long ahead = 0;   // mass of the members ordered before this one
      for (uint32_t j = 0; j < cm; ++j) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)j);
        const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)bi, (int)j);
        const unsigned long long wj = readlane64(aw, j);
        if (kj > a || (kj == a && ij < bi)) ahead += wj;
      }
      const unsigned long long prev = F.s_l[0] + ahead, incl = prev + aw;
      const bool cross = mm && (double)prev < theta_fx && theta_fx <= (double)incl;
      // Certificate: the fixed-point prefixes are exact sums of weights
      // rounded to 2^-51 (np 2^-51 in all), the weights are within 8 ulp
      // of the reference's, and its sequential sums in sorted order are
      // within sum_bound; the f64 conversion adds one rounding.
      const double dp = (double)prev / WFIX, di = (double)incl / WFIX;
      const double fx = (double)np * 0x1p-51;
      const double ep = sum_bound(dp, np, 8.0) + fx + U * dp, ei = sum_bound(di, np, 8.0) + fx + U * di;
      const bool cert = dp + ep < theta - theta_err && di - ei >= theta + theta_err;
      const uint64_t xb = __builtin_amdgcn_ballot_w64(cross);
      uint32_t ok = 0u, ck = 0u, ci = 0u;
      if (xb) {
        const uint32_t Lx = (uint32_t)__builtin_ctzll(xb);
        ck = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)Lx);
        ci = (uint32_t)__builtin_amdgcn_readlane((int)bi, (int)Lx);
        ok = __builtin_amdgcn_readlane((int)cert, (int)Lx) ? 1u : 0u;
      }
      if (ln == 0) { F.s_u[12] = ck; F.s_u[13] = ci; F.s_u[14] = ok; }
    }
    lds_barrier();
    if (!F.s_u[14]) return false;   // no certified crossing inside P: replay
    const uint32_t ck = F.s_u[12], ci = F.s_u[13];
    kept = mine && (mk > ck || (mk == ck && mi <= ci));
  }

  // ---- overflow check and the inverse-CDF draw in token-ID order ----------
  const double dw = kept ? mw : 0.0;
  const double winc = wave_scan_f64(dw);
  const uint32_t wk = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(kept));
  const bool wbad = __builtin_amdgcn_ballot_w64(kept && !isfinite(s)) != 0ull;
  const uint64_t pos = __builtin_amdgcn_ballot_w64(dw > 0.0);
  if (lane() == 63) {
    F.rd[wave()][0] = winc;
    F.ru[wave()][2] = wk;
    F.ru[wave()][3] = wbad ? 1u : 0u;
  }
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; }
  if (X.kbits) {
    for (uint32_t q = tid; q < X.nwords; q += FT) X.kbits[q] = 0u;
    __builtin_amdgcn_s_waitcnt(0);   // the zeroing lands before any wave's atomics below
  }
  lds_barrier();
  const bool wl = lane() < (uint32_t)FW;
  const double ws = wave_scan_f64(wl ? F.rd[lane()][0] : 0.0);
  const double S = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, ws), 63));
  const double wbefore =
      wave() ? __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, ws), wave() - 1)) : 0.0;
  const uint32_t nkept = wave_sum_u32(wl ? F.ru[lane()][2] : 0u);
  const bool bad = __builtin_amdgcn_ballot_w64(wl && F.ru[lane()][3] != 0u) != 0ull;
  if (bad) {
    write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u);
    return true;
  }
  const double cum = wbefore + winc, before = cum - dw;
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  // the last positive kept member: one atomic per wave
  if (pos && lane() == 0) atomicMax(&F.s_u[1], wave() * 64u + (uint32_t)(64 - __builtin_clzll(pos)));
  if (dw > 0.0 && target < cum && !(target < before)) {
    F.kflag[tid] = (fabs(target - before) <= derr || fabs(cum - target) <= derr) ? 1u : 0u;
    atomicMin(&F.s_u[0], tid);
  }
  lds_barrier();
  uint32_t pick = F.s_u[0];
  bool uncert = Q.unc;
  if (pick != NONE) {
    uncert = uncert || (F.kflag[pick] != 0u && !X.nodraw);
  } else {
    // rounding left the variate past the accumulated mass: the last positive kept token
    pick = F.s_u[1] ? F.s_u[1] - 1u : NONE;
    uncert = uncert || !X.nodraw;
  }
  if (pick == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return true; }
  const double sp = ((double)F.u.s.pl[pick] - X.M) / c.T;
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)F.u.s.pid[pick], sp - log(S), nkept);
  if (X.kbits && kept) atomicOr(&X.kbits[mi >> 5], 1u << (mi & 31u));
  return true;
}

__device__ __forceinline__ bool finish_sel(const FinCtx& X, FinSmem& F, const FinLoads& P, uint32_t sq, uint32_t sj) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x;
  const uint32_t nq = sq < X.C ? F.st[sq].ncand : 0u;
  uint32_t act = 0, key[SR];
#pragma unroll
  for (int u = 0; u < SR; ++u) {
    const bool a = sj * (uint32_t)SR + (uint32_t)u < nq;
    act |= a ? 1u << u : 0u;
    key[u] = a ? okey(P.l[u]) : 0u;
  }
  const float Mf = okey_value(F.hdr.Mkey);   // the row maximum (X.M in f64)
  // waves holding no candidate skip the per-slot work (the rows' few
  // candidates sit in one wave per chunk); they still meet every barrier
  const bool wact = __builtin_amdgcn_ballot_w64(act != 0u) != 0ull;
  uint32_t kap = 0, idk = 0, bstar = NONE;
  bool whole = false;     // E takes the whole crossing bin (exactly, or as a bracket)
  bool bracket = false;   // ... with surplus members whose mass bext bounds
  double bext = 0.0;
  uint32_t bin[SR];
  if (X.k_path) {
    if (c.k > X.ncand) return false;
    const float lo = F.hdr.lo;
    const float span = Mf - lo;
    const float sc = span > 1e-30f ? (float)(NBS - 1) / span : 0.0f;
    if (wact) {
#pragma unroll
      for (int u = 0; u < SR; ++u) {
        bin[u] = sel_bin(P.l[u], Mf, sc);
        if ((act >> u) & 1u) atomicAdd(&F.u.s.cnt[bin[u]], 1u);
      }
    }
    lds_barrier();
    // wave 0 finds the crossing bin (bin order = descending value)
    if (wave() == 0) {
      const uint32_t ln = lane();
      uint32_t hs = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint4 h4 = *reinterpret_cast<const uint4*>(&F.u.s.cnt[32u * ln + 4u * (uint32_t)q]);
        hs += h4.x + h4.y + h4.z + h4.w;
      }
      uint32_t bb = 0;
      const uint32_t bf = wave_cross32(F.u.s.cnt, hs, wave_scan_u32(hs), c.k, &bb);
      // NONE: fewer candidates than k.  Whole: the crossing bin holds
      // exactly the members E still needs, so E is every candidate in bins
      // 0 .. bf.  Bracket: the crossing bin lies below the min-p band (no
      // member is in P), so E may take the whole bin too; its surplus
      // members' mass (at most (count - need) times the largest weight the
      // bin allows, one bin wider for the f32 binning) widens E's mass bound.
      const uint32_t cb = bf != NONE ? F.u.s.cnt[bf] : 0u;
      uint32_t mode = 0u;
      double extra = 0.0;
      if (bf != NONE) {
        if (bb + cb == c.k) {
          mode = 1u;
        } else if (c.min_p > 0.0 && sc > 0.0f) {
          const float band = 1e-5f * (fabsf(Mf) + fabsf((float)(c.T * X.L))) + 1e-30f;
          const float llo = Mf + (float)(c.T * X.L) - band;
          const float top = Mf - (float)((int)bf - 1) / sc;   // above every value in bin bf
          if (__builtin_isfinite(llo) && top < llo) {
            mode = 2u;
            const float c2 = (float)(1.4426950408889634 / c.T);
            const double whi = fmin(1.0, (double)__builtin_amdgcn_exp2f((top - Mf) * c2) * 1.0001);
            extra = (double)(bb + cb - c.k) * whi;
          }
        }
      }
      if (ln == 0) { F.s_u[12] = bf; F.s_u[13] = bb; F.s_u[8] = mode; F.s_d[5] = extra; }
    }
    lds_barrier();
    bstar = F.s_u[12];
    const uint32_t abv = F.s_u[13];
    if (bstar == NONE) return false;
    whole = F.s_u[8] != 0u;
    bracket = F.s_u[8] == 2u;
    bext = F.s_d[5];
    if (!whole) {   // rank the crossing bin's members
      // the crossing bin's members
      if (wact) {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
          if (((act >> u) & 1u) && bin[u] == bstar) {
            const uint32_t at = atomicAdd(&F.s_u[10], 1u);
            if (at < (uint32_t)PCAP) { F.u.s.mk[at] = key[u]; F.u.s.mi[at] = P.id[u]; }
          }
        }
      }
      lds_barrier();
      const uint32_t cm = F.s_u[10];
      if (cm > (uint32_t)PCAP) return false;
      // wave 0 ranks the members: the (k - abv)-th in (key desc, ID asc)
      // order is the last one E takes (the need-th exists: cm >= need >= 1)
      if (wave() == 0) {
        const uint32_t need = c.k - abv;
        const uint32_t ln = lane();
        const bool mm = ln < cm;
        const uint32_t a = mm ? F.u.s.mk[ln] : 0u, bi = mm ? F.u.s.mi[ln] : NONE;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < cm; ++j) {
          const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)j);
          const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)bi, (int)j);
          rank += (kj > a || (kj == a && ij < bi)) ? 1u : 0u;
        }
        if (ln == 0) F.s_u[12] = NONE;   // no finite logit's key
        if (mm && rank == need - 1u) { F.s_u[12] = a; F.s_u[13] = bi; }
      }
      lds_barrier();
      kap = F.s_u[12];
      idk = F.s_u[13];
      if (kap == NONE) return false;   // not reached: the members hold the need-th
    }
  }

  // ---- E, its f32 mass, and P ----------------------------------------------
  // The min-p test s = (l - M) / T >= L, i.e. l >= M + T L, on the f32
  // logit away from that threshold (the band is far wider than the f32
  // threshold's rounding), in f64 near it (with the closeness flag).
  const bool need_wlo = X.k_path && c.top_p >= 1.0;   // only this case reads the minimum weight
  bool unc = false;
  uint32_t inP = 0, ne = 0;
  float e32 = 0.0f, eab32 = 0.0f, p32 = 0.0f, pab32 = 0.0f;
  float wlo = FLT_MAX;
  if (wact) {
    const double L = X.L;
    const bool minp_on = c.min_p > 0.0;
    const float lthr = minp_on ? Mf + (float)(c.T * L) : -FLT_MAX;
    const float band = minp_on ? 1e-5f * (fabsf(Mf) + fabsf((float)(c.T * L))) + 1e-30f : 0.0f;
    // (a non-finite threshold or band sends every candidate to the f64 test)
    const bool lfin = __builtin_isfinite(lthr + band) && __builtin_isfinite(lthr - band);
    const float lhi = lfin ? lthr + band : INFINITY, llo = lfin ? lthr - band : -INFINITY;
    const float c2 = (float)(1.4426950408889634 / c.T);   // log2(e) / T
    // Branch-free per slot (a slot outside E adds +0 to every sum, which
    // leaves it unchanged); only the rare f64 min-p test near the threshold
    // is a branch, taken by the waves that need it.
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const bool a = (act >> u) & 1u;
      const float l = P.l[u];
      bool pm = l >= lhi;   // the min-p test (every token when min_p = 0)
      const bool near = a && minp_on && l >= llo && l < lhi;
      if (__builtin_amdgcn_ballot_w64(near)) {
        if (near) {
          const double sd = ((double)l - X.M) / c.T;
          pm = sd >= L;
          if (fabs(sd - L) < X.Lclose) unc = true;
        }
      }
      const bool in = a && (!X.k_path ? pm
                            : whole ? bin[u] <= bstar
                                    : (key[u] > kap || (key[u] == kap && P.id[u] <= idk)));
      // (a stale slot's logit may be anything: it is replaced by Mf, so y
      // stays finite and 0 times -y stays 0)
      const float y = vmax(((a ? l : Mf) - Mf) * c2, -200.0f);   // <= 0 (clamped: f32::MIN would give -inf)
      const float wx = __builtin_amdgcn_exp2f(y);
      const float wf = in ? wx : 0.0f;
      ne += in ? 1u : 0u;
      e32 += wf;
      eab32 = __builtin_fmaf(wf, -y, eab32);
      if (need_wlo && in) wlo = fminf(wlo, wf * (1.0f - (0x1p-21f + 2.5e-7f * -y)));
      const bool pin = in && pm;
      inP |= pin ? 1u << u : 0u;
      const float wp = pin ? wf : 0.0f;
      p32 += wp;
      pab32 = __builtin_fmaf(wp, -y, pab32);
    }
  }
  // per-thread partial sums to LDS (the E index space is free); wave 0
  // alone reduces them
  static_assert(FT * sizeof(float4) <= ECAP * sizeof(uint32_t), "partial sums fit eidx");
  float4* part = reinterpret_cast<float4*>(F.eidx);
  part[tid] = make_float4(e32, eab32, p32, pab32);
  const uint32_t pc = (uint32_t)__builtin_popcount(inP);
  uint32_t pinc = 0;
  if (wact) {
    pinc = wave_scan_u32(pc);
    const uint32_t wne = wave_sum_u32(ne);
    const bool uw = __builtin_amdgcn_ballot_w64(unc) != 0ull;
    if (need_wlo) wlo = okey_value(~wave_max_u32(~okey(wlo)));   // the wave's minimum
    if (lane() == 63) {
      F.ru[wave()][0] = pinc;
      F.ru[wave()][1] = wne;
      F.ru[wave()][2] = uw ? 1u : 0u;
      F.red_f[wave()] = wlo;
    }
  } else if (lane() == 0) {
    F.ru[wave()][0] = 0u;
    F.ru[wave()][1] = 0u;
    F.ru[wave()][2] = 0u;
    F.red_f[wave()] = FLT_MAX;
  }
  lds_barrier();
  SelSums Q;
  {
    const uint32_t ln = lane();
    const bool wl = ln < (uint32_t)FW;
    const uint32_t cw = wl ? F.ru[ln][0] : 0u;
    Q.np = wave_sum_u32(cw);
    Q.ne = wave_sum_u32(wl ? F.ru[ln][1] : 0u);
    if (Q.ne == 0u || Q.np > (uint32_t)PMAX) return false;
    // P in token-ID order: waves order by (chunk, rank in the chunk), lanes
    // and slots in order within a wave
    if (__builtin_amdgcn_ballot_w64(inP != 0u)) {
      const uint32_t C = X.C, w = wave();
      const uint32_t q = w % C, m = w / C, lq = ln % C, lm = ln / C;
      const uint32_t ahead = wave_sum_u32(wl && (lq < q || (lq == q && lm < m)) ? cw : 0u);
      uint32_t at = ahead + pinc - pc;
#pragma unroll
      for (int u = 0; u < SR; ++u) {
        if ((inP >> u) & 1u) {
          F.u.s.pk[at] = key[u];
          F.u.s.pid[at] = P.id[u];
          F.u.s.pl[at] = P.l[u];
          ++at;
        }
      }
    }
    if (wave() == 0) {
      // E's mass: f32 weights, summed in f32 per thread (at most SR terms)
      // and in f64 across threads (any order: the bound holds for every
      // order).  |f32 weight - exact| <= 2^-22 w (exp2f) + ln2 3.0001 2^-24
      // w |y| (the three f32 roundings of y) + 2^-120 below 2^-126; the
      // per-thread f32 sums add (SR + 1) 2^-24 of the mass; plus both sides'
      // f64 sums (sum_bound, 8 ulp terms).
      double e = 0.0, ea = 0.0, pp = 0.0, pa = 0.0;
#pragma unroll
      for (int i = 0; i < FT / 64; ++i) {
        const float4 v = part[ln + 64u * (uint32_t)i];
        e += (double)v.x;
        ea += (double)v.y;
        pp += (double)v.z;
        pa += (double)v.w;
      }
      Q.esum = wave_sum_f64(e);
      const double eab = wave_sum_f64(ea);
      Q.esum_err = 1.01 * ((0x1p-22 + (double)(SR + 1) * 0x1p-24) * Q.esum +
                           0.6931471805599453 * 3.0001 * 0x1p-24 * eab) +
                   (double)Q.ne * 0x1p-120 + sum_bound(Q.esum, Q.ne, 8.0);
      if (bracket) {
        // E's mass lies in [sum - extra, sum]: take the middle
        Q.esum -= 0.5 * bext;
        Q.esum_err += 0.5 * bext * 1.0001;
      }
      Q.unc = __builtin_amdgcn_ballot_w64(wl && F.ru[ln][2] != 0u) != 0ull;
      Q.wlo = need_wlo ? (double)okey_value(~wave_max_u32(wl ? ~okey(F.red_f[ln]) : 0u)) : 0.0;
      // For the workgroup finish of a large P: theta, and whether the
      // nucleus can end inside P, from P's f32 mass (same bound as E's).
      bool theta_set = false;
      double theta = 0.0, theta_err = 0.0;
      const bool tok = sel_theta(X, Q, &theta_set, &theta, &theta_err);
      bool cut = false;
      if (Q.np > 64u && tok && theta_set) {
        const double ps = wave_sum_f64(pp), pab = wave_sum_f64(pa);
        const double ps_err = 1.01 * ((0x1p-22 + (double)(SR + 1) * 0x1p-24) * ps +
                                      0.6931471805599453 * 3.0001 * 0x1p-24 * pab) +
                              (double)Q.np * 0x1p-120 + sum_bound(ps, Q.np, 8.0);
        cut = !(ps + ps_err < theta - theta_err);
      }
      if (ln == 0) {
        F.s_d[0] = Q.esum;
        F.s_d[1] = Q.esum_err;
        F.s_d[2] = Q.wlo;
        F.s_u[9] = Q.unc ? 1u : 0u;
        F.s_u[14] = tok ? 1u : 0u;
        F.s_u[15] = cut ? 1u : 0u;
        F.s_d[3] = theta;
        F.s_d[4] = theta_err;
      }
    }
  }
  lds_barrier();
  if (Q.np <= 64u) {
    if (wave() == 0) {
      const bool ok = sel_small(X, F, Q);
      if (lane() == 0) F.s_u[15] = ok ? 1u : 0u;
    }
    lds_barrier();
    return F.s_u[15] != 0u;
  }
  if (!F.s_u[14]) return false;   // the running sum may stall: the general path replays it
  Q.esum = F.s_d[0];
  Q.esum_err = F.s_d[1];
  Q.wlo = F.s_d[2];
  Q.unc = F.s_u[9] != 0u;
  return sel_large(X, F, Q);
}

// ---------------------------------------------------------------------------
// finish_large for candidates cached in LDS (n <= FT * FR): each thread
// holds a contiguous range of R = ceil(n / FT) candidates in registers, with
// its shifted logits and weights computed once, so every later pass is one
// loop over registers and each prefix is one block scan (the draw's scan in
// token-ID order included) instead of one block scan per FT candidates.
// The decisions and certificates are finish_large's.
__device__ __forceinline__ void finish_large_r(const FinCtx& X, FinSmem& F, uint32_t ne) {
  const RowCfg& c = X.c;
  const uint32_t tid = threadIdx.x;
  const uint32_t n = X.ncand;
  const uint32_t R = (n + FT - 1u) / FT, j0 = tid * R;
  uint32_t kv[FR];
  double sv[FR], wv[FR];
  uint32_t have = 0, mem = 0;
  bool uncert = false;
  double wpart = 0.0, wmin = INFINITY;
  // The shifted logit decides membership (min-p rows) and the min-p test:
  // there it is the reference's quotient.  Otherwise it only feeds weights,
  // and the product with 1/T (within 2 ulp of the quotient) moves a weight
  // by at most w |s| 2^-51 <= 2^-51 / e, inside the bounds' allowance for
  // every prefix from the top (each holds the maximum, weight 1).
  const bool exact_s = X.mode == M_MINP || (c.min_p > 0.0 && X.mode != M_MINP);
  const double invT = 1.0 / c.T;
  float lmin = INFINITY;   // the smallest member logit
#pragma unroll
  for (int r = 0; r < FR; ++r) {
    kv[r] = 0u;
    sv[r] = 0.0;
    wv[r] = 0.0;
    if ((uint32_t)r < R && j0 + (uint32_t)r < n) {
      const float l = F.cl[j0 + r];
      const uint32_t id = F.cid[j0 + r];
      const uint32_t key = okey(l);
      const double sh = exact_s ? ((double)l - X.M) / c.T : ((double)l - X.M) * invT;
      kv[r] = key;
      sv[r] = sh;
      have |= 1u << r;
      const bool m = X.k_path ? (key > X.kappa || (key == X.kappa && id <= X.id_tie))
                              : (X.mode == M_MINP ? sh >= X.L : true);
      if (m) {
        mem |= 1u << r;
        const double w = exp_neg_t(sh, X.etab, X.etab + 64);
        wv[r] = w;
        wpart += w;
        wmin = fmin(wmin, w);
        lmin = fminf(lmin, l);
      }
    }
  }
  if (tid == 0) { F.s_u[13] = 0u; F.s_u[14] = 0u; }   // the kept pass's flags (ordered by the barriers below)
  double esum = wpart, nwmin = -wmin;
  float nlmin = -lmin;
  block_sum_max_max(&esum, &nwmin, &nlmin, F.rd, F.red_f);
  wmin = -nwmin;
  lmin = -nlmin;
  double total = X.total, total_err = X.total_err;
  if (!X.have_total) { total = esum; total_err = sum_bound(esum, ne, 8.0); }
  fstamp(X, 4);

  uint32_t tau = 0, id_cut = NONE;
  bool cut = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      if (!minp_above_stall(c, esum) && !(wmin > 2.3e-16 * esum)) uncert = true;
    } else {
      cut = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    theta = c.top_p * total;
    theta_err = c.top_p * total_err + U * theta;
    cut = !(esum + sum_bound(esum, ne, 8.0) < theta - theta_err);
  }
  bool binned = false;
  if (cut) {
    // One mass histogram on NB value bins (bin 0 holds the largest logits;
    // a bin index never decreases as the logit decreases), its block scan,
    // and the crossing bin's members ranked exactly by one wave: the cut
    // member's (key, ID) in one pass.  More than 64 members in the
    // crossing bin: the radix passes below.
    const float Mf = (float)X.M;
    const float span = Mf - fmaxf(lmin, Mf - (float)(746.0 * c.T));   // zero-weight members share the last bin
    const float sc = span > 1e-30f ? (float)(NB - 1) / span : 0.0f;
    for (uint32_t t = tid; t < (uint32_t)NB; t += FT) { F.u.h.hcnt[t] = 0u; F.u.h.hmass[t] = 0.0; }
    if (tid == 0) { F.s_u[4] = NONE; F.s_u[6] = 0u; F.s_u[10] = 0u; }
    __syncthreads();
    uint32_t bins[FR];
#pragma unroll
    for (int r = 0; r < FR; ++r) {
      bins[r] = 0u;
      if ((mem >> r) & 1u) {
        const float d = (Mf - okey_value(kv[r])) * sc;
        bins[r] = d < (float)(NB - 1) ? (uint32_t)d : (uint32_t)(NB - 1);
        atomicAdd(&F.u.h.hcnt[bins[r]], 1u);
        atomicAdd(&F.u.h.hmass[bins[r]], wv[r]);
      }
    }
    __syncthreads();
    const uint32_t b0 = BPT * tid;   // this thread's bins, in descending value order
    double msum = 0.0;
    uint32_t nsum = 0;
#pragma unroll
    for (uint32_t i = 0; i < BPT; ++i) { msum += F.u.h.hmass[b0 + i]; nsum += F.u.h.hcnt[b0 + i]; }
    double mtot, mexc;
    uint32_t ntot, ninc;
    const double minc = block_scan_pair_du(msum, nsum, F.red_d, F.red_u, &mexc, &mtot, &ninc, &ntot);
    const uint32_t nexc = ninc - nsum;
    {
      double lo = mexc;
      uint32_t nlo = nexc;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) {
        const double mh = F.u.h.hmass[b0 + i];
        const uint32_t nh = F.u.h.hcnt[b0 + i];
        const double hi = i + 1 == BPT ? minc : lo + mh;
        if (nh && lo < theta && theta <= hi) { F.s_u[4] = b0 + i; F.s_u[5] = nlo; F.s_d[4] = lo; }
        lo = hi;
        nlo += nh;
      }
    }
    __syncthreads();
    const uint32_t bstar = F.s_u[4];
    if (bstar != NONE) {
#pragma unroll
      for (int r = 0; r < FR; ++r)
        if (((mem >> r) & 1u) && bins[r] == bstar) {
          const uint32_t at = atomicAdd(&F.s_u[10], 1u);
          if (at < 64u) { F.u.h.hcnt[at] = kv[r]; F.eidx[at] = F.cid[j0 + r]; }
        }
    }
    __syncthreads();
    const uint32_t cm = F.s_u[10];
    if (bstar != NONE && cm <= 64u) {
      binned = true;
      if (wave() == 0) {
        // rank the members by (key desc, ID asc): each lane sums the weights
        // of the members ahead of it (one pass over the members, no sort)
        const uint32_t ln = lane();
        const bool live = ln < cm;
        const uint32_t key = live ? F.u.h.hcnt[ln] : 0u, id = live ? F.eidx[ln] : NONE;
        const double sh = exact_s ? ((double)okey_value(key) - X.M) / c.T : ((double)okey_value(key) - X.M) * invT;
        const double w = live ? exp_neg_t(sh, X.etab, X.etab + 64) : 0.0;
        double pre = 0.0;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < cm; ++j) {
          const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)key, (int)j);
          const uint32_t ij = (uint32_t)__builtin_amdgcn_readlane((int)id, (int)j);
          const double wj = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, w), j));
          const bool ahead = kj > key || (kj == key && ij < id);
          pre += ahead ? wj : 0.0;
          rank += ahead ? 1u : 0u;
        }
        const double above = F.s_d[4];
        const uint32_t above_n = F.s_u[5];
        const double prev = above + pre, cum = prev + w;   // before and after this member
        const uint64_t hit = __builtin_amdgcn_ballot_w64(live && prev < theta && theta <= cum);
        if (ln == 0) { F.s_u[3] = NONE; F.s_u[11] = NONE; F.s_u[7] = 1u; }
        if (hit) {
          const uint32_t i = (uint32_t)__builtin_ctzll(hit);
          if (ln == i) {
            const double e1 = sum_bound(cum, above_n + rank + 65u, 8.0), e0 = sum_bound(prev, above_n + rank + 64u, 8.0);
            const bool cert = prev + e0 < theta - theta_err && cum - e1 >= theta + theta_err;
            F.s_u[3] = id;
            F.s_u[11] = key;
            F.s_u[7] = cert && __builtin_popcountll(hit) == 1 ? 0u : 1u;
          }
        }
      }
      __syncthreads();
      if (F.s_u[11] == NONE) { cut = false; uncert = true; }
      else { tau = F.s_u[11]; id_cut = F.s_u[3]; if (F.s_u[7]) uncert = true; }
      __syncthreads();
    }
  }
  if (cut && !binned) {
    uint32_t prefix = 0, pmask = 0, above_n = 0;
    double above = 0.0;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      for (uint32_t t = tid; t < (uint32_t)NB; t += FT) { F.u.h.hcnt[t] = 0u; F.u.h.hmass[t] = 0.0; }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < FR; ++r) {
        if (((mem >> r) & 1u) && (kv[r] & pmask) == prefix) {
          const uint32_t bin = (kv[r] >> sh) & (NB - 1);
          atomicAdd(&F.u.h.hcnt[bin], 1u);
          atomicAdd(&F.u.h.hmass[bin], wv[r]);
        }
      }
      __syncthreads();
      // as in finish_large: per-thread bin intervals tile the mass exactly
      const uint32_t b0 = NB - 1 - BPT * tid;
      double msum = 0.0;
      uint32_t nsum = 0;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) { msum += F.u.h.hmass[b0 - i]; nsum += F.u.h.hcnt[b0 - i]; }
      double mtot, mexc;
      uint32_t ntot, nexc;
      const double minc = above + block_scan_pair<double>(msum, F.red_d, &mexc, &mtot);
      mexc += above;
      nexc = above_n + block_scan_incl<uint32_t>(nsum, F.red_u, &ntot) - nsum;
      if (tid == 0) { F.s_u[4] = NONE; F.s_u[6] = 0u; }
      __syncthreads();
      double lo = mexc;
      uint32_t nlo = nexc;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) {
        const double mh = F.u.h.hmass[b0 - i];
        const uint32_t nh = F.u.h.hcnt[b0 - i];
        const double hi = i + 1 == BPT ? minc : lo + mh;
        if (nh && lo < theta && theta <= hi) {
          F.s_u[4] = b0 - i; F.s_u[5] = nlo; F.s_d[4] = lo;
          const double e0 = sum_bound(lo, nlo + 64u, 8.0);
          const double e1 = sum_bound(hi, nlo + nh + 64u, 8.0);
          if (!(lo + e0 < theta - theta_err) || !(hi - e1 >= theta + theta_err)) F.s_u[6] = 1u;
        }
        lo = hi;
        nlo += nh;
      }
      __syncthreads();
      const uint32_t bin = F.s_u[4];
      const uint32_t amb = F.s_u[6];
      const uint32_t an = F.s_u[5];
      const double am = F.s_d[4];
      __syncthreads();
      if (bin == NONE) { cut = false; uncert = true; break; }
      if (amb) uncert = true;
      prefix |= bin << sh;
      pmask |= (uint32_t)(NB - 1) << sh;
      above = am;
      above_n = an;
    }
    if (cut) {
      tau = prefix;
      const double wt = exp_neg_t(((double)okey_value(tau) - X.M) / c.T, X.etab, X.etab + 64);
      if (tid == 0) {
        uint32_t jn = 0;
        double cov = above;
        bool close = false;
        for (uint32_t q = 0; q < (uint32_t)NB * 64u; ++q) {
          cov += wt;
          ++jn;
          const double e = sum_bound(cov, above_n + jn + 64u, 8.0);
          if (fabs(cov - theta) <= e + theta_err) close = true;
          if (cov >= theta || !(wt > 0.0)) break;
        }
        F.s_u[6] = jn;
        F.s_u[7] = close ? 1u : 0u;
        F.s_u[3] = NONE;
      }
      __syncthreads();
      const uint32_t jneed = F.s_u[6];
      if (F.s_u[7]) uncert = true;
      // the jneed-th member at tau in token-ID order (ranges are in ID order)
      uint32_t tie = 0;
#pragma unroll
      for (int r = 0; r < FR; ++r) tie |= ((mem >> r) & 1u) && kv[r] == tau ? 1u << r : 0u;
      uint32_t ttot;
      uint32_t t = block_excl_scan_u32((uint32_t)__builtin_popcount(tie), F.sc_u[0], &ttot);
#pragma unroll
      for (int r = 0; r < FR; ++r)
        if ((tie >> r) & 1u) { ++t; if (t == jneed) F.s_u[3] = F.cid[j0 + r]; }
      __syncthreads();
      id_cut = F.s_u[3];
      if (id_cut == NONE) { id_cut = 0xfffffffeu; uncert = true; }
      __syncthreads();
    }
  }

  fstamp(X, 5);
  // kept = member, inside the cut, and (unless E is the min-p set already)
  // at or above ln(min_p); the draw walks kept tokens in ID order.
  const bool apply_minp = c.min_p > 0.0 && X.mode != M_MINP;
  uint32_t kept = 0, kn = 0, close = 0, bad = 0;
  double kpart = 0.0;
#pragma unroll
  for (int r = 0; r < FR; ++r) {
    if (!((have >> r) & 1u)) continue;
    if (apply_minp && fabs(sv[r] - X.L) < X.Lclose) close = 1;
    if (!((mem >> r) & 1u)) continue;
    if (cut && !(kv[r] > tau || (kv[r] == tau && F.cid[j0 + r] <= id_cut))) continue;
    if (apply_minp && !(sv[r] >= X.L)) continue;
    kept |= 1u << r;
    kpart += wv[r];
    ++kn;
    if (!isfinite(sv[r]) && !isfinite(((double)F.cl[j0 + r] - X.M) / c.T)) bad = 1;
  }
  if (bad) F.s_u[13] = 1u;
  if (close) F.s_u[14] = 1u;
  if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
  // the draw: one scan of the per-thread kept masses (and counts); the
  // threads' intervals tile (0, S] exactly, and inside a thread the last
  // positive weight's interval ends at the thread's inclusive prefix
  double kexc, S;
  uint32_t kninc, nkept;
  const double kinc = block_scan_pair_du(kpart, kn, F.red_d, F.red_u, &kexc, &S, &kninc, &nkept);
  if (F.s_u[13]) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
  if (F.s_u[14]) uncert = true;
  const double target = c.u * S;
  const double derr = sum_bound(S, nkept + 64u, 8.0);
  fstamp(X, 6);
  uint32_t lastw = 0;   // bit r: the last slot of this thread with a positive kept weight
#pragma unroll
  for (int r = 0; r < FR; ++r) if (((kept >> r) & 1u) && wv[r] > 0.0) lastw = 1u << r;
  double run = kexc;
#pragma unroll
  for (int r = 0; r < FR; ++r) {
    if (!((kept >> r) & 1u) || !(wv[r] > 0.0)) continue;
    const double prev = run;
    run = ((lastw >> r) & 1u) ? kinc : run + wv[r];
    if (target < run && !(target < prev)) {
      F.s_u[0] = F.cid[j0 + r];
      F.s_u[8] = kv[r];
      F.s_d[0] = sv[r];
      if (fabs(target - prev) <= derr || fabs(run - target) <= derr) F.s_u[2] = 1u;
    }
  }
  {   // the last positive kept weight's position: one LDS atomic per wave
    const uint32_t lp = wave_max_u32(lastw ? j0 + (uint32_t)__builtin_ctz(lastw) + 1u : 0u);
    if (lane() == 0 && lp) atomicMax(&F.s_u[1], lp);
  }
  __syncthreads();
  uint32_t tok = F.s_u[0];
  double shifted = F.s_d[0];
  if (F.s_u[2] && !X.nodraw) uncert = true;
  if (tok == NONE && F.s_u[1]) {
    // rounding left the variate past the accumulated mass: last positive kept token
    const uint32_t j = F.s_u[1] - 1u;
    tok = F.cid[j];
    shifted = ((double)F.cl[j] - X.M) / c.T;
    uncert = uncert || !X.nodraw;
  } else if (tok != NONE && !exact_s) {
    // the output takes the reference's quotient
    shifted = ((double)okey_value(F.s_u[8]) - X.M) / c.T;
  }
  __syncthreads();
  if (tok == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
  write_result(X, uncert ? MXS_ROW_UNCERTIFIED : 0, (int32_t)tok, shifted - log(S), nkept);
  if (X.kbits) {
    for (uint32_t q = tid; q < X.nwords; q += FT) X.kbits[q] = 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < FR; ++r)
      if ((kept >> r) & 1u) {
        const uint32_t id = F.cid[j0 + r];
        atomicOr(&X.kbits[id >> 5], 1u << (id & 31u));
      }
  }
}

// ---------------------------------------------------------------------------
// The k-th largest (1 <= k <= active count) of the wave's active keys (WR per
// lane, logits lv) and how many are larger, from one value histogram: 256
// bins between lo (no active logit is below it) and the maximum Mf, the bin
// index never decreasing as the logit decreases, the crossing bin found by a
// scan, and its members ranked exactly.  False when the range is degenerate
// or the crossing bin holds more than 64 members (ties, a narrow crowd): the
// caller then takes the radix select.
__device__ __forceinline__ bool wave_kth_bin(uint32_t* h, uint32_t* mk, const float (&lv)[WR],
                                             const uint32_t (&key)[WR], uint32_t act, uint32_t k, float Mf, float lo,
                                             uint32_t* kappa, uint32_t* above) {
  const float span = Mf - lo;
  if (!(span > 1e-30f) || !__builtin_isfinite(span)) return false;
  const float sc = 255.0f / span;
  const uint32_t ln = lane();
  *reinterpret_cast<uint4*>(&h[4u * ln]) = make_uint4(0u, 0u, 0u, 0u);
  wave_lds_sync();
  uint32_t bin[WR];
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    const float d = (Mf - lv[r]) * sc;
    bin[r] = d < 255.0f ? (uint32_t)d : 255u;
    if ((act >> r) & 1u) atomicAdd(&h[bin[r]], 1u);
  }
  wave_lds_sync();
  const uint4 v = *reinterpret_cast<const uint4*>(&h[4u * ln]);
  const uint32_t c4[4] = {v.x, v.y, v.z, v.w};
  const uint32_t s = c4[0] + c4[1] + c4[2] + c4[3];
  const uint32_t inc = wave_scan_u32(s);
  const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= k);
  if (!reach) return false;
  const uint32_t L = (uint32_t)__builtin_ctzll(reach);
  uint32_t run = inc - s, b = 0u, bef = 0u;
  bool found = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!found && run + c4[i] >= k) { found = true; b = 4u * ln + (uint32_t)i; bef = run; }
    run += c4[i];
  }
  b = (uint32_t)__builtin_amdgcn_readlane((int)b, (int)L);
  bef = (uint32_t)__builtin_amdgcn_readlane((int)bef, (int)L);
  // the crossing bin's members, packed to lanes
  uint32_t mb = 0;
#pragma unroll
  for (int r = 0; r < WR; ++r) mb |= ((act >> r) & 1u) && bin[r] == b ? 1u << r : 0u;
  const uint32_t cnt = (uint32_t)__builtin_popcount(mb);
  const uint32_t pinc = wave_scan_u32(cnt);
  const uint32_t cm = bcast63(pinc);
  if (cm > 64u) return false;
  wave_lds_sync();   // every lane has read h before mk (which may share it) is written
  {
    uint32_t at = pinc - cnt;
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if ((mb >> r) & 1u) mk[at++] = key[r];
  }
  wave_lds_sync();
  const bool mine = ln < cm;
  const uint32_t a = mine ? mk[ln] : 0u;
  uint32_t ge = 0, gt = 0;
  for (uint32_t j = 0; j < cm; ++j) {
    const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)j);
    ge += kj >= a ? 1u : 0u;
    gt += kj > a ? 1u : 0u;
  }
  // kappa: the largest member key with at least `need` members at or above it
  const uint32_t need = k - bef;
  const bool cand = mine && ge >= need;
  const uint32_t kap = wave_max_u32(cand ? a : 0u);
  const uint64_t at_k = __builtin_amdgcn_ballot_w64(mine && a == kap);
  const uint32_t g = (uint32_t)__builtin_amdgcn_readlane((int)gt, (int)__builtin_ctzll(at_k));
  *kappa = kap;
  *above = bef + g;
  return true;
}

// ---------------------------------------------------------------------------
// The short one-wave finisher: top-k rows with k <= 64 and min-p rows, at
// most WR * 64 candidates (lane l holds candidates WR l .. WR l + WR - 1 from
// LDS, so lane order is token-ID order) and a working set E of at most 64
// members.  It makes wave_finish's decisions with far fewer dependent steps,
// which is what a single wave's finish time is made of:
//   - E (the top-k head, or the min-p set) is compacted to one member per
//     lane in token-ID order; each lane then takes one exact f64 shifted
//     logit (the reference's division) and one weight;
//   - the nucleus cut needs the mass ahead of each member of P (E with the
//     min-p test) in (key desc, ID asc) order: each lane sums the weights of
//     the P members ranked before it, one ballot-driven pass over P, instead
//     of a sort;
//   - the draw is sel_draw_wave (one inclusive scan in token-ID order).
// Every decision carries the same certificate as elsewhere: a margin inside
// the bound returns false having written nothing, and the row goes on to
// the other finishers (which replay it where needed).
__device__ __forceinline__ bool finish_w1(const FinCtx& X, FinSmem& F) {
  const RowCfg& c = X.c;
  const uint32_t n = X.ncand, ln = lane(), j0 = ln * (uint32_t)WR;
  if (n == 0u || n > (uint32_t)(WR * 64)) return false;
  float lv[WR];
  uint32_t key[WR];
  uint32_t act = 0;
  {
    const float4 a0 = *reinterpret_cast<const float4*>(&F.cl[j0]);
    const float4 a1 = *reinterpret_cast<const float4*>(&F.cl[j0 + 4u]);
    lv[0] = a0.x; lv[1] = a0.y; lv[2] = a0.z; lv[3] = a0.w;
    lv[4] = a1.x; lv[5] = a1.y; lv[6] = a1.z; lv[7] = a1.w;
  }
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    const bool a = j0 + (uint32_t)r < n;
    act |= a ? 1u << r : 0u;
    key[r] = a ? okey(lv[r]) : 0u;
  }
  // ---- E: the top-k head (key above kappa, then the lowest-ID ties) or the
  // min-p set (the f32 logit decides away from the threshold, the exact
  // shifted logit near it)
  uint32_t inE = 0;
  bool unc = false;
  if (X.k_path) {
    if (c.k > 64u || c.k > n) return false;
    uint32_t kappa, above;
    if (!wave_kth_bin(F.eidx, F.eidx + 256, lv, key, act, c.k, (float)X.M, F.hdr.lo, &kappa, &above) &&
        !wave_kth(F.eidx, key, act, c.k, &kappa, &above))
      return false;
    const uint32_t need_t = c.k - above;
    uint32_t tie = 0;
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      inE |= ((act >> r) & 1u) && key[r] > kappa ? 1u << r : 0u;
      tie |= ((act >> r) & 1u) && key[r] == kappa ? 1u << r : 0u;
    }
    const uint32_t tc = (uint32_t)__builtin_popcount(tie);
    uint32_t t = wave_scan_u32(tc) - tc;
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if ((tie >> r) & 1u) { if (t < need_t) inE |= 1u << r; ++t; }
  } else {
    const float Mf = (float)X.M;
    const float lthr = Mf + (float)(c.T * X.L);
    const float band = 1e-5f * (fabsf(Mf) + fabsf((float)(c.T * X.L))) + 1e-30f;
    const bool lfin = __builtin_isfinite(lthr + band) && __builtin_isfinite(lthr - band);
    const float lhi = lfin ? lthr + band : INFINITY, llo = lfin ? lthr - band : -INFINITY;
#pragma unroll
    for (int r = 0; r < WR; ++r) {
      if (!((act >> r) & 1u)) continue;
      bool in = lv[r] >= lhi;
      if (lv[r] >= llo && lv[r] < lhi) {
        const double sd = ((double)lv[r] - X.M) / c.T;
        in = sd >= X.L;
        if (fabs(sd - X.L) < X.Lclose) unc = true;
      }
      inE |= in ? 1u << r : 0u;
    }
  }
  // ---- E compacted to lanes in token-ID order --------------------------------
  const uint32_t ec = (uint32_t)__builtin_popcount(inE);
  const uint32_t einc = wave_scan_u32(ec);
  const uint32_t ne = bcast63(einc);
  if (ne == 0u || ne > 64u) return false;
  uint32_t* ek = F.eidx + 256;   // past wave_kth's histogram
  uint32_t* ep = ek + 64;
  {
    uint32_t at = einc - ec;
#pragma unroll
    for (int r = 0; r < WR; ++r)
      if ((inE >> r) & 1u) { ek[at] = key[r]; ep[at] = j0 + (uint32_t)r; ++at; }
  }
  wave_lds_sync();
  const bool mine = ln < ne;
  const uint32_t mk = mine ? ek[ln] : 0u, mp = mine ? ep[ln] : 0u;
  const float ml = mine ? F.cl[mp] : 0.0f;
  const uint32_t mid = mine ? F.cid[mp] : NONE;
  const double s = mine ? ((double)ml - X.M) / c.T : 0.0;
  const double w = mine ? exp_neg_t(s, X.etab, X.etab + 64) : 0.0;
  // P: E with the min-p test (top-k rows; E already is the min-p set otherwise)
  bool inp = mine;
  if (mine && X.k_path && c.min_p > 0.0) {
    inp = s >= X.L;
    if (fabs(s - X.L) < X.Lclose) unc = true;
  }
  const uint64_t pmask = __builtin_amdgcn_ballot_w64(inp);
  const uint32_t np = (uint32_t)__builtin_popcountll(pmask);
  const double esum = wave_sum_f64(w);
  const double psum = wave_sum_f64(inp ? w : 0.0);
  unc = __builtin_amdgcn_ballot_w64(unc) != 0ull;

  // ---- the nucleus cut --------------------------------------------------------
  bool theta_set = false;
  double theta = 0.0, theta_err = 0.0;
  if (X.k_path) {
    if (c.top_p >= 1.0) {
      // the running sum may stall before reaching the total: the other paths replay it
      const unsigned long long wb = mine ? __builtin_bit_cast(unsigned long long, w) : ~0ull;
      const double wm = __builtin_bit_cast(double, ~wave_max_u64(~wb));
      if (!minp_above_stall(c, esum) && !(wm > 2.3e-16 * esum)) return false;
    } else {
      theta_set = true;
      theta = c.top_p * esum;
      theta_err = c.top_p * sum_bound(esum, ne, 8.0) + U * theta;
    }
  } else if (c.top_p < 1.0) {
    // the reference walks the tokens whose weight reaches 1e-9 of the total:
    // every min-p member must clear that level
    if (!(c.min_p * (1.0 - 1e-12) > 1e-9 * (X.total + X.total_err) * (1.0 + 1e-12))) return false;
    theta_set = true;
    theta = c.top_p * X.total;
    theta_err = c.top_p * X.total_err + U * theta;
  }
  bool kept = inp;
  if (theta_set && !(psum + sum_bound(psum, np, 8.0) < theta - theta_err)) {
    // The nucleus can end inside P.  P's masses on 64 value bins (bin 0
    // holds the largest logits; lane b reads bin b), one scan finds the bin
    // where the prefix reaches theta, and only that bin's members take the
    // mass of the members ranked before them; the reference keeps a member
    // whose running sum before it is still below theta.
    const float Mf = (float)X.M;
    // P's smallest logit, not below M - 746 T (members further down weigh 0
    // and share the last bin)
    const float plo = fmaxf(okey_value(~wave_max_u32(inp ? ~okey(ml) : 0u)), Mf - (float)(746.0 * c.T));
    const float span = Mf - plo;
    const float sc = span > 1e-30f && __builtin_isfinite(span) ? 63.0f / span : 0.0f;
    const float d = (Mf - ml) * sc;
    const uint32_t pb = d < 63.0f ? (uint32_t)d : 63u;
    double* bm = reinterpret_cast<double*>(F.eidx + 512);
    bm[ln] = 0.0;
    wave_lds_sync();
    if (inp) atomicAdd(&bm[pb], w);
    wave_lds_sync();
    const double bv = bm[ln];
    const double binc = wave_scan_f64(bv);
    const uint64_t cross = __builtin_amdgcn_ballot_w64(binc >= theta);
    if (!cross) {
      // P's mass stays below theta: every member is kept when the bound clears it
      const double tot = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, binc), 63));
      if (!(tot + sum_bound(tot, np + 64u, 8.0) < theta - theta_err)) return false;
    } else {
      const uint32_t b = (uint32_t)__builtin_ctzll(cross);
      const double bef = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, binc - bv), b));
      const uint64_t inb = __builtin_amdgcn_ballot_w64(inp && pb == b);
      const uint32_t nbef = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(inp && pb < b));
      double pre = 0.0;
      uint32_t rank = 0;
      uint64_t m = inb;
      while (m) {
        const uint32_t j = (uint32_t)__builtin_ctzll(m);
        m &= m - 1ull;
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)mk, (int)j);
        const uint32_t pj = (uint32_t)__builtin_amdgcn_readlane((int)mp, (int)j);
        const double wj = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, w), j));
        const bool ahead = kj > mk || (kj == mk && pj < mp);
        pre += ahead ? wj : 0.0;
        rank += ahead ? 1u : 0u;
      }
      const bool mb = inp && pb == b;
      const double prev = bef + pre, cum = prev + w;
      const uint64_t hit = __builtin_amdgcn_ballot_w64(mb && prev < theta && theta <= cum);
      if (__builtin_popcountll(hit) != 1) return false;
      const uint32_t hx = (uint32_t)__builtin_ctzll(hit);
      const uint32_t nb = nbef + rank;
      const bool cert = prev + sum_bound(prev, nb + 64u, 8.0) < theta - theta_err &&
                        cum - sum_bound(cum, nb + 65u, 8.0) >= theta + theta_err;
      if (!__builtin_amdgcn_readlane((int)cert, (int)hx)) return false;
      const uint32_t ck = (uint32_t)__builtin_amdgcn_readlane((int)mk, (int)hx);
      const uint32_t cp = (uint32_t)__builtin_amdgcn_readlane((int)mp, (int)hx);
      kept = inp && (pb < b || (pb == b && (mk > ck || (mk == ck && mp <= cp))));
    }
  }
  sel_draw_wave(X, kept, w, s, mid, unc);
  return true;
}

// ---------------------------------------------------------------------------
// The row finisher.  Runs in the last chunk workgroup of a row, after every
// chunk published its statistics and candidates.
// The kept set of a keep-all row: every legal token.
__device__ __forceinline__ void keepall_bits(const SampleArgs& A, uint32_t row, uint32_t* kbits, uint32_t nwords,
                                             uint32_t V) {
  if (!kbits) return;
  const mxs_batch& b = A.b;
  for (uint32_t q = threadIdx.x; q < nwords; q += FT) {
    uint32_t wv = 0xffffffffu;
    if (q == nwords - 1 && (V & 31u)) wv = (1u << (V & 31u)) - 1u;
    if (A.masked) {
      wv &= b.mask_words[(uint64_t)row * b.mask_stride + q];
      const uint32_t tv = b.tokenizer_vocab;
      if (q * 32u >= tv) wv = 0u;
      else if (q * 32u + 32u > tv) wv &= (1u << (tv - q * 32u)) - 1u;
    }
    kbits[q] = wv;
  }
}

#ifndef MXS_REDUCE_RW
#define MXS_REDUCE_RW 4u
#endif
// A top-k row whose chunk lists exceed the finisher's LDS cache (heads above
// 1024, or flat rows): one pass histograms the lists on a value grid below
// the row maximum (NBS bins of HRANGE / NBS logits), and the candidates in
// the bins down to the one where the count reaches k (the head and every tie
// at its edge: every bin above holds fewer than k) are compacted into the
// LDS cache in token-ID order when they fit.  Returns their count, or NONE
// (the lists do not reduce to the cache).  The lists themselves stay as they
// are (mxs_export_candidates reads them).
__device__ __forceinline__ uint32_t reduce_head(const float* cand_l, const uint32_t* cand_id, uint64_t rbase,
                                             uint32_t CH, uint32_t C, uint32_t k, uint32_t Mkey, FinSmem& F,
                                             uint64_t* timing, uint32_t row) {
  const uint32_t tid = threadIdx.x;
  uint32_t res = NONE;
  constexpr uint32_t RW = MXS_REDUCE_RW;   // list entries per thread per round (loads in flight)
  static_assert(RW >= 1u && RW <= 16u, "the offset tables hold 16 entries per wave");
  const float Mf = okey_value(Mkey);
  const float sc = (float)NBS / HRANGE;
  auto vb = [&](float x) -> uint32_t {
    const float d = (Mf - x) * sc;
    return d < (float)(NBS - 1) ? (uint32_t)d : (uint32_t)(NBS - 1);
  };
  // 8 copies of the histogram, lane l adding to copy l % 8: lanes whose
  // entries share a bin mostly hit different words (the bulk of a row's
  // values falls in a few hundred bins)
  constexpr uint32_t HCP = 8;
  uint32_t* hc = reinterpret_cast<uint32_t*>(&F.u);   // HCP x NBS words; F.u.s is cleared again below
  static_assert(sizeof(F.u) >= HCP * NBS * sizeof(uint32_t), "histogram copies fit the finisher's union");
  for (uint32_t i = tid; i < HCP * (uint32_t)NBS; i += FT) hc[i] = 0u;
  __syncthreads();
  if (timing) timing[((uint64_t)row * (MAXC + 1) + MAXC) * TSTAMPS + 12] = wall_clock64();
  // A chunk with at least k candidates holds k tokens at or above its
  // threshold, so the head's k-th value is at least the largest such
  // threshold: entries below it are never in the head's bins.
  float hthr = -INFINITY;
  for (uint32_t q = 0; q < C; ++q)
    if (F.st[q].ncand >= k) hthr = fmaxf(hthr, F.st[q].thr);
  uint32_t* hl = hc + (lane() % HCP) * (uint32_t)NBS;
  for (uint32_t q = 0; q < C; ++q) {   // coalesced, RW loads in flight per thread
    const uint32_t nq = F.st[q].ncand;
    const float* cl = cand_l + rbase + (uint64_t)q * CH;
    for (uint32_t j0 = tid; j0 < nq; j0 += (uint32_t)FT * RW) {
      float xv[RW];
#pragma unroll
      for (uint32_t u = 0; u < RW; ++u) {
        const uint32_t j = j0 + u * (uint32_t)FT;
        xv[u] = j < nq ? ld_dev(&cl[j]) : -INFINITY;
      }
#pragma unroll
      for (uint32_t u = 0; u < RW; ++u)
        if (j0 + u * (uint32_t)FT < nq && xv[u] >= hthr) atomicAdd(&hl[vb(xv[u])], 1u);
    }
  }
  __syncthreads();
  if (wave() == 0) {   // lane l: bins 32 l .. 32 l + 31, from the row maximum down
    auto bin = [&](uint32_t i) {
      uint32_t t = 0u;
#pragma unroll
      for (uint32_t p = 0; p < HCP; ++p) t += hc[p * (uint32_t)NBS + i];
      return t;
    };
    uint32_t hs = 0u;
    for (uint32_t i = 0; i < 32u; ++i) hs += bin(lane() * 32u + i);
    const uint32_t inc = wave_scan_u32(hs);
    const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= k);
    uint32_t bs = (uint32_t)(NBS - 1), kept = bcast63(inc);
    if (reach) {
      const uint32_t gi = (uint32_t)__builtin_ctzll(reach);
      const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - hs), (int)gi);
      const uint32_t hv = lane() < 32u ? bin(32u * gi + lane()) : 0u;
      const uint32_t vi = base + wave_scan_u32(hv);
      const uint32_t lb = (uint32_t)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lane() < 32u && vi >= k));
      bs = 32u * gi + lb;
      kept = (uint32_t)__builtin_amdgcn_readlane((int)vi, (int)lb);
    }
    if (lane() == 0) { F.s_u[12] = bs; F.s_u[14] = kept; }
  }
  __syncthreads();
  if (timing) timing[((uint64_t)row * (MAXC + 1) + MAXC) * TSTAMPS + 13] = wall_clock64();
  const uint32_t bs = F.s_u[12], kept = F.s_u[14];
  if (kept <= (uint32_t)CCAP) {
    // Compaction in token-ID order from coalesced rounds: entry
    // r0 + u FT + tid of a round goes after every kept entry of the
    // round's earlier u, then of the earlier waves at this u, then of the
    // wave's lower lanes (ballots); wave 0 turns the waves' per-u counts
    // into offsets, one exchange per round.
    uint32_t* wc = hc;              // [NW][16] kept counts per wave and u
    uint32_t* off = hc + NW * 16u;  // [NW][16] offsets; [NW * 16]: the round's total
    uint32_t n = 0;
    const uint32_t w = wave();
    for (uint32_t q = 0; q < C; ++q) {
      const uint32_t nq = F.st[q].ncand;
      const uint64_t cb = rbase + (uint64_t)q * CH;
      for (uint32_t r0 = 0; r0 < nq; r0 += (uint32_t)FT * RW) {   // uniform trip count
        float xv[RW];
        uint32_t iv[RW];
        uint32_t keep = 0u;
#pragma unroll
        for (uint32_t u = 0; u < RW; ++u) {
          const uint32_t j = r0 + u * (uint32_t)FT + tid;
          xv[u] = j < nq ? ld_dev(&cand_l[cb + j]) : -INFINITY;
          iv[u] = j < nq ? ld_dev(&cand_id[cb + j]) : 0u;
        }
        uint32_t pl[RW];
#pragma unroll
        for (uint32_t u = 0; u < RW; ++u) {
          const bool in = r0 + u * (uint32_t)FT + tid < nq && xv[u] >= hthr && vb(xv[u]) <= bs;
          keep |= in ? 1u << u : 0u;
          const uint64_t bm = __builtin_amdgcn_ballot_w64(in);
          pl[u] = lanes_below(bm);
          if (lane() == u) wc[w * 16u + u] = (uint32_t)__builtin_popcountll(bm);
        }
        __syncthreads();
        if (w == 0) {
          // lane u < 16: the per-wave offsets at u, then the scan over u
          uint32_t tu = 0u;
          uint32_t cv[NW];
#pragma unroll
          for (int v = 0; v < NW; ++v) {
            cv[v] = lane() < RW ? wc[(uint32_t)v * 16u + lane()] : 0u;
            tu += cv[v];
          }
          const uint32_t bu = wave_scan_u32(tu) - tu;
          if (lane() < RW) {
            uint32_t run = n + bu;
#pragma unroll
            for (int v = 0; v < NW; ++v) {
              off[(uint32_t)v * 16u + lane()] = run;
              run += cv[v];
            }
          }
          if (lane() == RW - 1u) off[NW * 16u] = bu + tu;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t u = 0; u < RW; ++u)
          if ((keep >> u) & 1u) {
            const uint32_t at = off[w * 16u + u] + pl[u];
            F.cl[at] = xv[u];
            F.cid[at] = iv[u];
          }
        n += off[NW * 16u];
        __syncthreads();   // wc and off are rewritten next round
      }
    }
    res = n;
  }
  if (timing) timing[((uint64_t)row * (MAXC + 1) + MAXC) * TSTAMPS + 14] = wall_clock64();
  __syncthreads();
  reinterpret_cast<uint2*>(F.u.s.cnt)[tid] = make_uint2(0u, 0u);
  reinterpret_cast<ulonglong2*>(F.u.s.mass)[tid] = make_ulonglong2(0ull, 0ull);
  __syncthreads();
  return res;
}

template <typename In>
__device__ __forceinline__ void finish_row(const SampleArgs& A, FinSmem& F, const RowCfg& c, uint32_t row, uint32_t mode,
                           uint64_t rbase, double invT, const FinLoads& P) {
  const mxs_batch& b = A.b;
  const uint32_t tid = threadIdx.x;
  const uint32_t V = b.vocab;
  const uint32_t C = A.C;
  // exp_neg's tables into LDS (waves 2-3) while waves 0-1 reduce the chunk
  // statistics; the selection finisher's histogram and list counters are
  // cleared in the same interval.
  if (tid >= 128 && tid < 256) {
    const uint32_t j = tid - 128u;
    F.etab[j] = j < 64u ? kExp2Tab[j] : kExp2TabLo[j - 64u];
  }
  reinterpret_cast<uint2*>(F.u.s.cnt)[tid] = make_uint2(0u, 0u);
  reinterpret_cast<ulonglong2*>(F.u.s.mass)[tid] = make_ulonglong2(0ull, 0ull);
  static_assert(NBS == 2 * FT && PMAX == FT, "two histogram bins per thread; one P member per thread");
  if (tid == 256) {   // wave 4: off the statistics' waves
    F.s_u[10] = 0u;
    F.s_u[11] = 0u;
    F.hdr.L = c.min_p > 0.0 ? log(c.min_p) : -INFINITY;
  }
  if (tid == 0) A.w.cand_rows[row] = -1;   // no candidate list unless a candidate path runs
  uint32_t sq, sj;                // this thread's chunk and slot group (slot_map)
  slot_map(C, &sq, &sj);
  const uint32_t cov = slot_cov(C);   // candidates per chunk held in registers
  // Chunk statistics (lane q of wave 0 holds chunk q's, C <= 64): reduced
  // with DPP into the row header, and copied to LDS.
  if (wave() == 0) {
    const uint32_t q = lane();
    const ChunkStat& v = P.v;
    const uint32_t fl = wave_or_u32(v.flags);
    const uint32_t nl = wave_sum_u32(v.nlegal);
    const uint32_t mkey = wave_max_u32(v.nlegal ? v.maxkey : 0u);
    const uint32_t qmax = wave_max_u32(v.ncand);
    // the smallest candidate threshold (order keys; chunks without candidates do not count)
    const uint32_t lokey = ~wave_max_u32(v.ncand ? ~okey(v.thr) : 0u);
    // the greedy argmax: largest (value key, ~id); chunk values are +0.0-normalised
    const unsigned long long garg = wave_max_u64(
        v.gbest_id != NONE ? ((unsigned long long)okey(v.gbest_val) << 32) | (unsigned long long)(~v.gbest_id) : 0ull);
    const uint32_t cinc = wave_scan_u32(v.ncand);
    if (q < C) {
      F.st[q] = v;
      F.coff[q] = cinc - v.ncand;
    }
    if (q == 0) {
      F.coff[C] = bcast63(cinc);
      F.hdr.flags = fl; F.hdr.nlegal = nl; F.hdr.Mkey = mkey; F.hdr.bi = garg ? ~(uint32_t)garg : NONE;
      F.hdr.ncand = bcast63(cinc);
      F.hdr.qmax = qmax;
      // The value bins' lower end: no candidate below it matters to a bin's
      // position, and members more than 746 T below the maximum weigh 0
      // (exp underflows), so they share the last bin (a suppressed legal
      // token's f32::MIN would otherwise stretch the bins over 3.4e38 and
      // put every other candidate in bin 0).
      F.hdr.lo = fmaxf(okey_value(lokey), okey_value(mkey) - (float)(746.0 * c.T));
    }
  } else if (wave() == 1 && !c.greedy) {
    // the chunk masses rescaled to the row maximum (f64: off wave 0's path)
    const uint32_t q = lane();
    const bool qa = q < C;
    const uint32_t nlg = P.v.nlegal, mxk = P.v.maxkey;
    const double ms = P.v.mass, me = P.v.mass_err;
    const uint32_t mkey = wave_max_u32(nlg ? mxk : 0u);
    const double Mw = (double)okey_value(mkey);
    const double cs = nlg ? exp_neg_p(((double)okey_value(mxk) - Mw) * invT) : 0.0;
    const double t = wave_sum_f64(ms * cs), te = wave_sum_f64(me * cs);
    const uint32_t nl = wave_sum_u32(nlg);
    if (qa) F.cscale[q] = cs;
    if (q == 0) {
      F.hdr.mass = t;
      // chunk error bounds (f32 weights), scaled; plus both sides' f64
      // rounding of weights and sums, and the x e^x <= 1/e product term
      F.hdr.mass_err = te * 1.000001 + sum_bound(t, nl + C, 12.0) + 2.0 * 0.37 * (double)nl * U;
    }
  }
  lds_barrier();
  const uint32_t flags = F.hdr.flags, nlegal = F.hdr.nlegal, bi = F.hdr.bi;
  const double M = (double)okey_value(F.hdr.Mkey);
  const int32_t err = combine_errors(c, flags, nlegal);
  if (A.race_m && tid == 0) A.race_m[row] = (float)M;   // the race kernel's reference point
  const uint32_t nwords = (V + 31u) / 32u;
  uint32_t* kbits = A.o.kept_bits ? A.o.kept_bits + (uint64_t)row * nwords : nullptr;
  FinCtx X;
  X.cand_l = A.w.cand_l; X.cand_id = A.w.cand_id; X.CH = A.CH; X.o = A.o; X.c = c; X.row = row; X.mode = mode; X.C = C; X.V = V; X.nlegal = nlegal; X.rbase = rbase;
  X.kbits = kbits; X.nwords = nwords; X.M = M; X.timing = A.timing; X.paths = A.paths; X.etab = F.etab;
  X.nodraw = A.nodraw != 0u;
  if (err) {
    fpath(X, MXS_PATH_ERROR);
    write_result(X, err, -1, 0.0, 0u);
    if (kbits)
      for (uint32_t q = tid; q < nwords; q += FT) kbits[q] = 0u;
    return;
  }
  if (mode == M_GREEDY) {
    fpath(X, MXS_PATH_GREEDY);
    write_result(X, 0, (int32_t)bi, 0.0, 1u);
    if (kbits)
      for (uint32_t q = tid; q < nwords; q += FT) kbits[q] = (q == (bi >> 5)) ? (1u << (bi & 31u)) : 0u;
    return;
  }
  const bool k_act = c.k > 0 && c.k < nlegal;

  // =================== KEEPALL: every legal token, ID order ===============
  if (mode == M_KEEPALL) {
    uint32_t mink = NONE;
    for (uint32_t q = 0; q < C; ++q)
      if (F.st[q].nlegal && F.st[q].minkey < mink) mink = F.st[q].minkey;
    if (!isfinite(((double)okey_value(mink) - M) / c.T)) { write_result(X, MXS_ROW_INVALID_TEMPERATURE, -1, 0.0, 0u); return; }
    if (A.nodraw) {   // race-v2: the kept set is every legal token; the race kernel picks
      fpath(X, MXS_PATH_KEEPALL_RACE);
      write_result(X, 0, -1, 0.0, nlegal);
      keepall_bits(A, row, kbits, nwords, V);
      return;
    }
    fpath(X, MXS_PATH_KEEPALL);
    const uint32_t segs_per_chunk = A.per * NW;   // the chunk kernel's 256-token (slice, wave) segments
    const uint32_t nseg = C * segs_per_chunk;
    double part = 0.0;
    for (uint32_t s = tid; s < nseg; s += FT) {
      const uint32_t q = s / segs_per_chunk, r = s % segs_per_chunk;
      if (F.st[q].nlegal) part += ld_dev(&A.w.seg[((uint64_t)row * MAXC + q) * PER_MAX * NW + r]) * F.cscale[q];
    }
    const double total = block_sum<double>(part, F.red_d);
    const double target = c.u * total;
    // Each segment mass carries the x = (l - m) / T product rounding
    // (x e^x <= 1/e per token) and 8 ulp per weight; plus the scale factors.
    const double err_b = sum_bound(total, nlegal + nseg, 12.0) + 2.0 * 0.37 * (double)nlegal * U;
    if (tid == 0) { F.s_u[0] = NONE; F.s_u[1] = 0u; F.s_u[2] = 0u; }
    __syncthreads();
    double run = 0.0;
    for (uint32_t base = 0; base < nseg; base += FT) {
      const uint32_t s = base + tid;
      double w = 0.0;
      if (s < nseg) {
        const uint32_t q = s / segs_per_chunk, r = s % segs_per_chunk;
        if (F.st[q].nlegal) w = ld_dev(&A.w.seg[((uint64_t)row * MAXC + q) * PER_MAX * NW + r]) * F.cscale[q];
      }
      double tot;
      const double inc = run + block_scan_incl<double>(w, F.red_d, &tot);
      const double exc = inc - w;
      {   // the last positive segment: one LDS atomic per wave
        const uint32_t ls = wave_max_u32(w > 0.0 ? s + 1u : 0u);
        if (lane() == 0 && ls) atomicMax(&F.s_u[1], ls);
      }
      if (w > 0.0) {
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
      seg = F.s_u[1] ? F.s_u[1] - 1u : NONE;
      near = true;
      before = -INFINITY;   // forces the last positive token of the segment
    }
    if (seg == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
    if (wave() == 0) {
      const uint32_t q = seg / segs_per_chunk, r = seg % segs_per_chunk;
      const uint32_t i = r / NW, w = r % NW;
      const uint32_t q1 = min(V, q * A.CH + A.CH);
      const uint32_t seg0 = q * A.CH + i * SLICE + w * 256u;
      const uint32_t id0 = seg0 + lane() * 4u;
      // the segment's history counts, counted by the whole wave in LDS
      // (one coalesced pass over the row's history)
      uint32_t* scnt = F.eidx;
      for (uint32_t j = lane(); j < 256u; j += 64u) scnt[j] = 0u;
      wave_lds_sync();
      for (uint32_t h = c.hb + lane(); h < c.he; h += 64u) {
        const uint32_t d = b.history_ids[h] - seg0;
        if (d < 256u) atomicAdd(&scnt[d], 1u);
      }
      wave_lds_sync();
      double wl[4], sh[4];
      double lsum = 0.0;
      for (int e = 0; e < 4; ++e) {
        const uint32_t id = id0 + (uint32_t)e;
        wl[e] = 0.0;
        sh[e] = 0.0;
        if (id < q1) {
          float l;
          bool lg;
          rederive_token<In>(A, c, row, id, scnt[lane() * 4u + (uint32_t)e], &l, &lg);
          if (lg) { sh[e] = ((double)l - M) / c.T; wl[e] = exp_neg_t(sh[e], F.etab, F.etab + 64); }
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
    if (tok == NONE) { write_result(X, MXS_ROW_EMPTY_SUPPORT, -1, 0.0, 0u); return; }
    near = near || F.s_u[4] != 0u;
    write_result(X, near ? MXS_ROW_UNCERTIFIED : 0, (int32_t)tok, F.s_d[1] - log(total), nlegal);
    keepall_bits(A, row, kbits, nwords, V);
    return;
  }

  // =================== candidate paths ====================================
  uint32_t ncand = F.hdr.ncand;
  if (tid == 0) A.w.cand_rows[row] = (int32_t)ncand;   // mxs_export_candidates
  // A top-k row whose chunk lists exceed the LDS cache (heads above 1024,
  // or flat rows): one pass histograms the lists on a value grid below the
  // row maximum (NBS bins of HRANGE / NBS logits), and the candidates in
  // the bins down to the one where the count reaches k (the head and every
  // tie at its edge: every bin above holds fewer than k) are compacted into
  // the LDS cache in token-ID order when they fit; the lists themselves stay
  // as they are (mxs_export_candidates reads them).
  bool pre = false;   // the LDS cache holds the reduced list
  if (ncand > (uint32_t)CCAP && k_act && (mode == M_TOPK || mode == M_ALL)) {
    const uint32_t n = reduce_head(A.w.cand_l, A.w.cand_id, rbase, A.CH, C, c.k, F.hdr.Mkey, F, A.timing, row);
    if (n != NONE) {
      ncand = n;
      pre = true;
    }
  }
  X.ncand = ncand;
  X.lds_c = ncand <= (uint32_t)CCAP;
  const double L = F.hdr.L;
  // ln(min_p) is exact for min_p = 1 (and -inf for 0); otherwise device and
  // host logs may differ in the last ulps, so a shifted logit within 4 ulp is
  // an uncertain cut.
  X.L = L;
  X.Lclose = (c.min_p > 0.0 && c.min_p < 1.0) ? 4.0 * U * fabs(L) : 0.0;

  // total = sum over every legal token of exp((l - M) / T), from chunk masses
  X.total = 0.0;
  X.total_err = 0.0;
  X.have_total = false;
  // (an all-candidates row's working set is every legal token: its sum is
  // the total)
  if (c.top_p < 1.0 && !k_act && (mode == M_MINP || (mode == M_TOPK && A.masked))) {
    X.total = F.hdr.mass;
    X.total_err = F.hdr.mass_err;
    X.have_total = true;
  }

  // top-k head: kappa = the k-th largest key; the head takes every candidate
  // above it and the lowest-ID ties at it.
  X.k_path = k_act && (mode == M_TOPK || mode == M_ALL);
  X.kappa = 0;
  X.id_tie = NONE;

  // One bulk load of every candidate into LDS, all loads in flight at once.
  // Candidate j lives in chunk q's region at j - coff[q]; j grows with u,
  // so each thread walks the chunk offsets once.
  auto bulk_load = [&]() {
    // the register slots first (every chunk's first cov candidates)
    {
      const uint32_t nq = sq < C ? F.st[sq].ncand : 0u;
      const uint32_t o = sq < C ? F.coff[sq] : 0u;
#pragma unroll
      for (int u = 0; u < SR; ++u) {
        const uint32_t slot = sj * (uint32_t)SR + (uint32_t)u;
        if (slot < nq) { F.cl[o + slot] = P.l[u]; F.cid[o + slot] = P.id[u]; }
      }
    }
    float lv[FR];
    uint32_t iv[FR];
    uint32_t need = 0;   // bit u: candidate u * FT + tid is past the speculative slots
    uint32_t qj = 0, nxt = C > 1 ? F.coff[1] : NONE;
#pragma unroll
    for (int u = 0; u < FR; ++u) {
      const uint32_t j = (uint32_t)u * FT + tid;
      if (j < ncand) {
        while (j >= nxt) { ++qj; nxt = qj + 1 < C ? F.coff[qj + 1] : NONE; }
        const uint32_t local = j - F.coff[qj];
        if (local >= cov) {
          const uint64_t pos = rbase + (uint64_t)qj * A.CH + local;
          lv[u] = ld_dev(&A.w.cand_l[pos]);
          iv[u] = ld_dev(&A.w.cand_id[pos]);
          need |= 1u << u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < FR; ++u) {
      const uint32_t j = (uint32_t)u * FT + tid;
      if ((need >> u) & 1u) { F.cl[j] = lv[u]; F.cid[j] = iv[u]; }
    }
    lds_barrier();
  };
  // short rows first: the one-wave finisher
  bool loaded = pre;
  if (((mode == M_TOPK && c.k <= 64u) || mode == M_MINP) && ncand > 0u && ncand <= (uint32_t)(WR * 64) &&
      X.lds_c) {
    if (!loaded) bulk_load();
    loaded = true;
    if (wave() == 0) {
      const bool ok = finish_w1(X, F);
      if (lane() == 0) F.s_u[15] = ok ? 1u : 0u;
    }
    lds_barrier();
    if (F.s_u[15]) {
      fpath(X, MXS_PATH_SHORT);
      stamp(A, row, MAXC, 2);
      return;
    }
    lds_barrier();   // wave 0's LDS scratch is reused below
  }
  // rows whose candidates all sit in the register slots: the selection finisher
  if ((mode == M_TOPK || mode == M_MINP) && ncand > 0u && C <= (uint32_t)FW && F.hdr.qmax <= cov) {
    if (finish_sel(X, F, P, sq, sj)) {
      fpath(X, MXS_PATH_SELECT);
      stamp(A, row, MAXC, 2);
      return;
    }
  }
  if (X.lds_c && !loaded) bulk_load();
  stamp(A, row, MAXC, 1);
  if (mode != M_KEEPALL && X.lds_c && ncand <= (uint32_t)(WR * 64)) {
    // at most WR * 64 candidates: one wave finishes the row
    if (wave() == 0) {
      const bool ok = wave_finish(X, F);
      if (lane() == 0) F.s_u[15] = ok ? 1u : 0u;
    }
    lds_barrier();
    if (F.s_u[15]) {
      fpath(X, MXS_PATH_WAVE);
      stamp(A, row, MAXC, 2);
      return;
    }
    lds_barrier();   // wave 0's LDS scratch is reused below
  }
  if (mode != M_KEEPALL && finish_fast(X, F)) {
    fpath(X, MXS_PATH_FAST);
    stamp(A, row, MAXC, 2);
    return;
  }
  __syncthreads();   // the general path below reuses LDS the lean finisher touched
  uint32_t ties_needed = 0;
  if (X.k_path) {
    // Radix select from the first bit where the candidates' keys differ:
    // the shared high bits would put every candidate in one bin.
    uint32_t kmin_p = NONE, kmax_p = 0;
    for (uint32_t j = tid; j < ncand; j += FT) {
      const uint32_t key = okey(cand_l(X, F, j));
      kmin_p = min(kmin_p, key);
      kmax_p = max(kmax_p, key);
    }
    const uint32_t kmax = block_max<uint32_t>(kmax_p, F.red_u);
    const uint32_t kmin = ~block_max<uint32_t>(~kmin_p, F.red_u);
    const uint32_t diff = kmin ^ kmax;
    int hb = diff ? 31 - __clz((int)diff) : -1;   // highest differing bit
    uint32_t pmask = hb >= 0 ? (uint32_t)(~0ull << (hb + 1)) : 0xffffffffu;
    uint32_t prefix = kmin & pmask, above = 0;
    while (hb >= 0) {
      const int sh = hb >= 10 ? hb - 10 : 0;
      const uint32_t dmask = (uint32_t)((1ull << (hb - sh + 1)) - 1ull);
      for (uint32_t t = tid; t < (uint32_t)NB; t += FT) F.u.h.hcnt[t] = 0u;
      __syncthreads();
      for (uint32_t j = tid; j < ncand; j += FT) {
        const uint32_t key = okey(cand_l(X, F, j));
        if ((key & pmask) == prefix) atomicAdd(&F.u.h.hcnt[(key >> sh) & dmask], 1u);
      }
      __syncthreads();
      const uint32_t b0 = NB - 1 - BPT * tid;
      uint32_t csum = 0;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) csum += F.u.h.hcnt[b0 - i];
      uint32_t tot;
      uint32_t lo = block_scan_incl<uint32_t>(csum, F.red_u, &tot) - csum;
      const uint32_t need = c.k - above;
#pragma unroll
      for (uint32_t i = 0; i < BPT; ++i) {
        const uint32_t ch = F.u.h.hcnt[b0 - i];
        if (lo < need && need <= lo + ch) { F.s_u[4] = b0 - i; F.s_u[5] = above + lo; }
        lo += ch;
      }
      __syncthreads();
      prefix |= F.s_u[4] << sh;
      pmask |= dmask << sh;
      above = F.s_u[5];
      __syncthreads();
      hb = sh - 1;
    }
    X.kappa = prefix;
    ties_needed = c.k - above;
  }
  stamp(A, row, MAXC, 2);

  // ---- working set E: the head (k path), the exact min-p set (MINP) or
  // every candidate; token-ID order.
  uint32_t ne = 0, tie_seen = 0;
  bool mp_close = false;
  if (tid == 0) F.s_u[7] = NONE;
  __syncthreads();
  if (X.lds_c) {
    // contiguous per-thread ranges of the cached candidates (ID order runs
    // through the threads): one block scan for the ties, one for E
    const uint32_t R = (ncand + FT - 1u) / FT, j0 = tid * R;
    uint32_t inb = 0, tieb = 0;
#pragma unroll
    for (int r = 0; r < FR; ++r) {
      const uint32_t j = j0 + (uint32_t)r;
      if ((uint32_t)r < R && j < ncand) {
        const float l = F.cl[j];
        if (X.k_path) {
          const uint32_t key = okey(l);
          inb |= key > X.kappa ? 1u << r : 0u;
          tieb |= key == X.kappa ? 1u << r : 0u;
        } else if (mode == M_MINP) {
          const double sd = ((double)l - M) / c.T;
          inb |= sd >= L ? 1u << r : 0u;
          if (fabs(sd - L) < X.Lclose) mp_close = true;
        } else {
          inb |= 1u << r;
        }
      }
    }
    if (X.k_path) {
      uint32_t ttot;
      uint32_t t = block_excl_scan_u32((uint32_t)__builtin_popcount(tieb), F.sc_u[0], &ttot);
#pragma unroll
      for (int r = 0; r < FR; ++r)
        if ((tieb >> r) & 1u) {
          ++t;
          if (t <= ties_needed) inb |= 1u << r;
          if (t == ties_needed) F.s_u[7] = F.cid[j0 + r];
        }
    }
    uint32_t at = block_excl_scan_u32((uint32_t)__builtin_popcount(inb), F.sc_u[1], &ne);
    if (ne <= (uint32_t)ECAP) {
#pragma unroll
      for (int r = 0; r < FR; ++r)
        if ((inb >> r) & 1u) F.eidx[at++] = j0 + (uint32_t)r;
    }
  } else
  for (uint32_t base = 0; base < ncand; base += FT) {
    const uint32_t j = base + tid;
    bool in = false, tie = false;
    uint32_t id = 0;
    if (j < ncand) {
      const float l = cand_l(X, F, j);
      id = cand_id(X, F, j);
      if (X.k_path) {
        const uint32_t key = okey(l);
        in = key > X.kappa;
        tie = key == X.kappa;
      } else if (mode == M_MINP) {
        const double s = ((double)l - M) / c.T;
        in = s >= L;
        if (fabs(s - L) < X.Lclose) mp_close = true;
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
    if (in && ne + einc - 1u < (uint32_t)ECAP) F.eidx[ne + einc - 1u] = j;
    ne += etot;
  }
  __syncthreads();
  X.id_tie = F.s_u[7];
  mp_close = block_max<uint32_t>(mp_close ? 1u : 0u, F.red_u) != 0u;
  stamp(A, row, MAXC, 3);
  if (ne <= (uint32_t)ECAP && X.lds_c) {
    fpath(X, MXS_PATH_EXACT);
    finish_exact(X, F, ne, mp_close);
  } else {
    fpath(X, MXS_PATH_LARGE);
    if (X.lds_c) finish_large_r(X, F, ne);
    else finish_large(X, F, ne);
    if (mp_close && tid == 0 && A.o.status[row] == 0) A.o.status[row] = MXS_ROW_UNCERTIFIED;
  }
}

// ---------------------------------------------------------------------------
// The sampling kernel.
// The chunk pass and the row finisher share the workgroup's LDS (the
// finisher starts after the chunk is published).
union alignas(16) FusedSmem {
  ChunkSmem s;
  FinSmem f;
};
__device__ __forceinline__ ChunkSmem& chunk_smem(FusedSmem& u) { return u.s; }

// ---------------------------------------------------------------------------
// Step receipts fused into the pick.  A receipt is the log-softmax top n of
// the row's logits after suppression (ChatFormat::suppress writes f32::MIN,
// crates/core/chat-format/src/lib.rs:771-780) and the picked token's log
// probability (token_logprob, crates/app/cli/src/chat_turn.rs:506-563): what
// mx_logprob.hip's top-n kernels compute for a receipt, here from the chunk
// pass's own read of the logits.  Each chunk publishes its maximum, its sum
// of exp(l - maximum) and its exact top min(n, length) entries (key desc,
// token ID asc); the row's finisher merges them after the pick.
constexpr uint32_t RX_CAP = 2048;   // entries at or above the lower bound, collected in LDS
static_assert(offsetof(ChunkSmem, bvals) == offsetof(ChunkSmem, bids) + BCAP * 4 && BCAP * 2 >= (int)RX_CAP,
              "the receipt candidates take bids and bvals");
static_assert(MCAP >= 1024 + 128, "the receipt histogram, wave values and counters take mask");
static_assert(offsetof(FinSmem, cid) == offsetof(FinSmem, cl) + CCAP * 4 && CCAP * 8 >= (MAXC * 64 + 16) * 8,
              "the receipt merge takes the finisher's candidate cache (cl, then cid)");

// f(i) for the slices i < A.per: unrolled (UNR > 1: a getter over register
// arrays needs compile-time indices) or rolled.
template <int UNR, typename F>
__device__ __forceinline__ void rx_slices(const SampleArgs& A, F f) {
  if constexpr (UNR > 1) {
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i)
      if (i < (int)A.per) f(i);
  } else {
#pragma unroll 1
    for (int i = 0; i < (int)A.per; ++i) f(i);
  }
}

__device__ __forceinline__ unsigned long long rx_entry(uint32_t k, uint32_t id) {
  return ((unsigned long long)k << 32) | (unsigned long long)(~id);
}

// The rank (descending) of `mine` among m distinct nonzero entries v[0, m),
// by counting.  v must hold zeros up to the next multiple of 8 (they count
// for no entry); the comparisons read 8 entries per round as 4 independent
// 16-byte loads, not one dependent load each.
__device__ __forceinline__ uint32_t rx_rank_of(const unsigned long long* v, uint32_t m, unsigned long long mine) {
  const uint32_t m8 = (m + 7u) & ~7u;
  uint32_t rank = 0;
  for (uint32_t k = 0; k < m8; k += 8u) {
    ulonglong2 q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u] = *reinterpret_cast<const ulonglong2*>(&v[k + 2u * (uint32_t)u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) rank += (q[u].x > mine ? 1u : 0u) + (q[u].y > mine ? 1u : 0u);
  }
  return rank;
}

// The entries of v[0, m) ranked below `want`, stored in rank order to out
// (device scope); v padded as rx_rank_of needs.
__device__ __forceinline__ void rx_rank(const unsigned long long* v, uint32_t m, uint32_t want,
                                        unsigned long long* out) {
  for (uint32_t j = threadIdx.x; j < m; j += NT) {
    const unsigned long long mine = v[j];
    const uint32_t rank = rx_rank_of(v, m, mine);
    if (rank < want) st_dev(reinterpret_cast<double*>(&out[rank]), __builtin_bit_cast(double, mine));
  }
}

// The receipt's exact top-take of a chunk, where the fast path of
// receipt_chunk failed: the take-th largest key K by a bit search over block
// counts (one counter per round), then the keys above K and the ties at K in
// token-ID order, ranked and written out.
template <typename GetQ>
__device__ __forceinline__ void receipt_exact(const SampleArgs& A, ChunkSmem& S, uint32_t row, uint32_t chunk,
                                              uint32_t c0, uint32_t take, GetQ getq) {
  const uint32_t tid = threadIdx.x;
  uint32_t* rcnt = S.mask + 1088;
  unsigned long long* rc = reinterpret_cast<unsigned long long*>(S.bids);
  unsigned long long* list = A.rx_list + ((uint64_t)row * MAXC + chunk) * A.rx_n;
  lds_barrier();   // every thread has read the fast path's counters
  if (tid < 40u) rcnt[tid] = 0u;
  lds_barrier();
    uint32_t K = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = K | (1u << bit);
      uint32_t cnt = 0;
#pragma unroll 1
      for (int i = 0; i < (int)A.per; ++i) {
        float r[4];
        uint32_t rb;
        getq(i, r, rb);
#pragma unroll
        for (int e = 0; e < 4; ++e) cnt += (((rb >> e) & 1u) && okey(r[e]) >= cand) ? 1u : 0u;
      }
      cnt = wave_sum_u32(cnt);
      if (lane() == 0) atomicAdd(&rcnt[2 + bit], cnt);
      lds_barrier();
      if (rcnt[2 + bit] >= take) K = cand;
    }
    // keys above K (fewer than take) first, then the ties: counts per
    // (slice, wave) in token-ID order
#pragma unroll 1
    for (int i = 0; i < (int)A.per; ++i) {
      uint32_t tq = 0;
      float r[4];
      uint32_t rb;
      getq(i, r, rb);
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool inr = (rb >> e) & 1u;
        const uint32_t k = okey(r[e]);
        if (inr && k > K) rc[atomicAdd(&rcnt[1], 1u)] = rx_entry(k, e0 + (uint32_t)e);
        tq += (inr && k == K) ? 1u : 0u;
      }
      const uint32_t wt = wave_sum_u32(tq);
      if (lane() == 0) S.wcnt[i * NW + wave()] = wt;
    }
    lds_barrier();
    const uint32_t above = rcnt[1], need = take - above;
    const uint32_t nent = A.per * NW;
    const uint32_t v0 = lane() < nent ? S.wcnt[lane()] : 0u;
    const uint32_t v1 = lane() + 64u < nent ? S.wcnt[lane() + 64u] : 0u;
    const uint32_t v2 = lane() + 128u < nent ? S.wcnt[lane() + 128u] : 0u;
    const uint32_t i0 = wave_scan_u32(v0), i1 = wave_scan_u32(v1), i2 = wave_scan_u32(v2);
    const uint32_t s0 = (uint32_t)__builtin_amdgcn_readlane((int)i0, 63);
    const uint32_t s1 = (uint32_t)__builtin_amdgcn_readlane((int)i1, 63);
    const uint32_t x0 = i0 - v0, x1 = i1 - v1 + s0, x2 = i2 - v2 + s0 + s1;
#pragma unroll 1
    for (int i = 0; i < (int)A.per; ++i) {
      {
        float r[4];
        uint32_t rb;
        getq(i, r, rb);
        bool tie[4];
        uint32_t tq = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          tie[e] = ((rb >> e) & 1u) && okey(r[e]) == K;
          tq += tie[e] ? 1u : 0u;
        }
        const uint32_t idx = (uint32_t)i * NW + wave();
        const uint32_t xv = (idx >> 6) == 0 ? x0 : ((idx >> 6) == 1 ? x1 : x2);
        uint32_t rk = (uint32_t)__builtin_amdgcn_readlane((int)xv, (int)(idx & 63u)) + (wave_scan_u32(tq) - tq);
        const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (tie[e]) {
            if (rk < need) rc[above + rk] = rx_entry(K, e0 + (uint32_t)e);
            ++rk;
          }
        }
      }
    }
    lds_barrier();
  if (tid < 16u) rc[take + tid] = 0ull;
  lds_barrier();
  rx_rank(rc, take, take, list);
}

// getq(i, r, rb): this thread's quad of slice i after suppression (f32::MIN)
// into r, its in-range bits into rb.  UNR: PER_MAX for a getter over
// register arrays (compile-time slice indices), 1 for one that loads (the
// slice loop stays rolled, so no pass holds the whole chunk in registers).
// Uses mask, bids, bvals and wcnt of the chunk's LDS; every thread of the
// workgroup calls it.
template <int UNR, typename GetQ>
__device__ __forceinline__ bool receipt_chunk(const SampleArgs& A, ChunkSmem& S, uint32_t row, uint32_t chunk,
                                              uint32_t c0, uint32_t c1, GetQ getq) {
  const uint32_t tid = threadIdx.x;
  const uint32_t len = c1 - c0;
  const uint32_t n = A.rx_n, take = min(n, len);
  uint32_t* rh = S.mask;                                   // [1024] histogram of the thread maxima
  uint32_t* rwk = S.mask + 1024;                           // [NW] wave maxima (keys)
  uint32_t* rwf = S.mask + 1040;                           // [NW] wave non-finite flags
  double* rws = reinterpret_cast<double*>(S.mask + 1056);  // [NW] wave sums
  uint32_t* rcnt = S.mask + 1088;                          // [40] counters, each used once
  unsigned long long* rc = reinterpret_cast<unsigned long long*>(S.bids);   // [RX_CAP]
  unsigned long long* list = A.rx_list + ((uint64_t)row * MAXC + chunk) * n;
  rh[tid] = 0u;
  if (tid < 40u) rcnt[tid] = 0u;
  float tmax = -INFINITY;
  bool nf = false;
  rx_slices<UNR>(A, [&](int i) {
    float r[4];
    uint32_t rb;
    getq(i, r, rb);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool inr = (rb >> e) & 1u;
      nf |= inr && !__builtin_isfinite(r[e]);
      tmax = fmaxf(tmax, inr ? r[e] : -INFINITY);
    }
  });
  stamp(A, row, chunk, 12);
  // Each weight 2^y, y = (l - tmax) log2(e) <= 0, in f32: the subtraction
  // and the product each round y by at most 2^-24 |y|, and the exp2 adds an
  // ulp, so a weight is within 2^-23 (1 + ln2 |y|) of exp(l - tmax); a
  // quad's four weights are summed in f32 (3 more roundings), the quads in
  // f64.  Relative to this thread's sum S_t, which holds the maximum's exact
  // weight 1 besides at most 39 others, the error is at most
  // 2^-23 (1 + ln2 max_t(39 t 2^-t / (1 + 39 2^-t)) + 1.5) < 2^-20.9 (the
  // ratio peaks near 2.7); rescaled in f64 and summed, the row's S is within
  // 2^-20.9 (S - 1) of the exact sum, so ln S and every log probability
  // (l - M) - ln S, of magnitude at least (S - 1) / S, within 2^-20.9
  // relative.  y is clamped at -200 (2^-200 is 0 in f32): suppressed and
  // out-of-range tokens weigh 0.
  double part = 0.0;
  if (tmax > -INFINITY) {
    rx_slices<UNR>(A, [&](int i) {
      float r[4];
      uint32_t rb;
      getq(i, r, rb);
      float qs = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y = fmaxf((((rb >> e) & 1u) ? r[e] - tmax : -INFINITY) * 1.44269504f, -200.0f);
        qs += __builtin_amdgcn_exp2f(y);
      }
      part += (double)qs;
    });
  }
  stamp(A, row, chunk, 13);
  {
    const uint32_t wk = wave_max_u32(okey(tmax));
    const bool wf = __builtin_amdgcn_ballot_w64(nf) != 0ull;
    if (lane() == 0) {
      rwk[wave()] = wk;
      rwf[wave()] = wf ? 1u : 0u;
    }
  }
  lds_barrier();
  uint32_t ck = 0u, flags = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ck = max(ck, rwk[w]);
    flags |= rwf[w];
  }
  const float cmax = okey_value(ck);
  const bool listing = !flags && take > 0u;
  bool exact = false;
  // the thread's sum rescaled to the chunk maximum; the thread maxima
  // histogrammed on a 1/32-logit grid below it
  if (tmax > -INFINITY) part *= exp_neg_p((double)tmax - (double)cmax);
  part = wave_sum_f64(part);
  if (lane() == 0) rws[wave()] = part;
  if (listing && tmax > -INFINITY) {
    const float d = (cmax - tmax) * 32.0f;
    if (d < 1023.0f) atomicAdd(&rh[(uint32_t)d], 1u);
  }
  lds_barrier();
  if (listing) {
    // take threads hold a maximum at or above the crossing bin's lower edge,
    // so the chunk's take-th largest logit is too (one bin of margin for
    // the rounding of d): every wave finds the bin (lane j: bins 16 j ..)
    float L = -INFINITY;
    {
      uint32_t sm = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 h4 = *reinterpret_cast<const uint4*>(&rh[lane() * 16u + (uint32_t)q * 4u]);
        sm += h4.x + h4.y + h4.z + h4.w;
      }
      const uint32_t inc = wave_scan_u32(sm);
      const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= take);
      if (reach) {
        const uint32_t g = (uint32_t)__builtin_ctzll(reach);
        const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - sm), (int)g);
        const uint32_t v = lane() < 16u ? rh[16u * g + lane()] : 0u;
        const uint32_t vi = base + wave_scan_u32(v);
        const uint64_t r2 = __builtin_amdgcn_ballot_w64(lane() < 16u && vi >= take);
        const uint32_t tb = 16u * g + (uint32_t)__builtin_ctzll(r2);
        L = cmax - (float)(tb + 2u) / 32.0f;
      }
    }
    const uint32_t Lk = okey(L);
    stamp(A, row, chunk, 14);
    // the tokens at or above L, into LDS
    // the tokens at or above L, into LDS
    rx_slices<UNR>(A, [&](int i) {
      float r[4];
      uint32_t rb;
      getq(i, r, rb);
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k = okey(r[e]);
        if (((rb >> e) & 1u) && k >= Lk) {
          const uint32_t at = atomicAdd(&rcnt[0], 1u);
          if (at < RX_CAP) rc[at] = rx_entry(k, e0 + (uint32_t)e);
        }
      }
    });
    lds_barrier();
    stamp(A, row, chunk, 15);
    const uint32_t m = rcnt[0];
    // too many at or above L (ties, or a flat chunk), or (logits past 2^19
    // in magnitude, where the bin edges round) too few: the exact path
    if (m > RX_CAP - 16u || m < take) exact = true;
    // rank by counting (entries are distinct), the first take out in order
    if (!exact) {
      if (tid < 16u && m + tid < RX_CAP) rc[m + tid] = 0ull;   // (m <= RX_CAP - 16: see above)
      lds_barrier();
      rx_rank(rc, m, take, list);
    }
  }
  if (tid == 0) {
    double sum = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) sum += rws[w];
    RxStat* st = &A.rx_stat[(uint64_t)row * MAXC + chunk];
    st_dev(&st->maxv, cmax);
    st_dev(&st->flags, flags);
    st_dev(&st->count, listing ? take : 0u);
    st_dev(&st->sum, sum);
  }
  return !exact;
}

// The row's suppressed tokens (bias entries of -inf) in the chunk, as a
// bitmap (bit t - c0) over the count table, dead after the chunk body.
__device__ __forceinline__ void rx_supmap(const SampleArgs& A, ChunkSmem& S, uint32_t c0, uint32_t c1, uint32_t bb,
                                          uint32_t bn) {
  const uint32_t tid = threadIdx.x;
  const mxs_batch& b = A.b;
  uint32_t* supw = S.t.ct;
  lds_barrier();   // the candidates' copy-out has read the staging area
  const uint32_t nwd = A.per * ((uint32_t)SLICE / 32u);
  for (uint32_t t = tid; t < nwd; t += NT) supw[t] = 0u;
  lds_barrier();
  for (uint32_t j = tid; j < bn; j += NT) {
    const uint32_t d = b.bias_ids[bb + j] - c0;
    if (d < c1 - c0 && b.bias_values[bb + j] == -INFINITY) atomicOr(&supw[d >> 5], 1u << (d & 31u));
  }
  lds_barrier();
}

// The row's receipt from its chunks' statistics and lists, on the finisher's
// workgroup after the pick (thread 0 wrote the token).  The merge of the
// top-n kernel: a list of n entries has n at or above its last, so only
// entries at or above the largest such last entry can rank below n.  The
// loads go out together: every thread its list entries and their chunks'
// counts, wave 0 the statistics, wave 1 the row's suppressed IDs, thread 0
// the token's logit; one barrier later the filter, the rank and the writes.
template <typename In>
__device__ __forceinline__ void receipt_finish(const SampleArgs& A, FinSmem& F, uint32_t row) {
  const uint32_t tid = threadIdx.x;
  const uint32_t n = A.rx_n, C = A.C, V = A.b.vocab;
  const mxs_batch& b = A.b;
  const RxStat* st = A.rx_stat + (uint64_t)row * MAXC;
  const unsigned long long* lists = A.rx_list + (uint64_t)row * MAXC * n;
  unsigned long long* dense = reinterpret_cast<unsigned long long*>(F.cl);   // [MAXC * 64 + 16] over cl, cid
  uint32_t* supl = F.eidx;                                                   // [64] suppressed IDs
  constexpr int RL = (MAXC * 64 + NT - 1) / NT;   // list entries per thread
  unsigned long long ent[RL];
  uint32_t ecnt[RL];
#pragma unroll
  for (int u = 0; u < RL; ++u) {
    const uint32_t jj = tid + (uint32_t)u * NT;
    ent[u] = 0ull;
    ecnt[u] = 0u;
    if (jj < C * n) {
      const uint32_t q = jj / n;
      ent[u] = __builtin_bit_cast(unsigned long long, ld_dev(reinterpret_cast<const double*>(&lists[jj])));
      ecnt[u] = ld_dev(&st[q].count) > jj - q * n ? 1u : 0u;
    }
  }
  int32_t t = -1;
  float tl = 0.0f;
  if (tid == 0) {
    t = A.o.token[row];
    if (t >= 0 && (uint32_t)t < V) tl = Quad<In>::one(reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride + (uint32_t)t);
  }
  const uint32_t b0 = b.bias_offsets[row], b1 = b.bias_offsets[row + 1];
  const uint32_t bn = b1 > b0 ? b1 - b0 : 0u;
  if (wave() == 1 && bn <= 64u) {
    const uint32_t l = lane();
    const bool sp = l < bn && b.bias_values[b0 + l] == -INFINITY;
    const uint32_t id = l < bn ? b.bias_ids[b0 + l] : NONE;
    supl[l] = sp ? id : NONE;
  }
  if (wave() == 0) {
    const uint32_t q = lane();   // chunk q (C <= MAXC = 64)
    float cm = -INFINITY;
    double cs = 0.0;
    uint32_t fl = 0u;
    unsigned long long last = 0ull;
    if (q < C) {
      cm = ld_dev(&st[q].maxv);
      cs = ld_dev(&st[q].sum);
      fl = ld_dev(&st[q].flags);
      if (ld_dev(&st[q].count) == n)
        last = __builtin_bit_cast(unsigned long long, ld_dev(reinterpret_cast<const double*>(&lists[(uint64_t)q * n + n - 1u])));
    }
    const uint32_t flags = wave_or_u32(fl);
    const uint32_t mkey = wave_max_u32(okey(cm));
    const double M = (double)okey_value(mkey);
    const double S = wave_sum_f64(cs > 0.0 ? cs * exp_neg_p((double)cm - M) : 0.0);
    const unsigned long long thr = wave_max_u64(last);
    if (lane() == 0) {
      F.s_u[0] = flags;
      F.s_u[1] = 0u;
      F.s_d[0] = M;
      F.s_d[1] = S;
      F.s_l[0] = thr;
    }
  }
  lds_barrier();
  const uint32_t flags = F.s_u[0];
  const double M = F.s_d[0];
  int32_t* ids = A.rx_ids + (uint64_t)row * n;
  double* lps = A.rx_lps + (uint64_t)row * n;
  if (flags) {   // a non-finite logit: the chunks listed nothing
    for (uint32_t j = tid; j < n; j += NT) {
      ids[j] = -1;
      lps[j] = __builtin_nan("");
    }
    if (tid == 0) {
      A.rx_status[row] = MXS_ROW_NON_FINITE_LOGIT;
      A.rx_token_lp[row] = __builtin_nan("");
    }
    return;
  }
  const unsigned long long thr = F.s_l[0];
#pragma unroll
  for (int u = 0; u < RL; ++u)
    if (ecnt[u] && ent[u] >= thr) dense[atomicAdd(&F.s_u[1], 1u)] = ent[u];
  lds_barrier();
  const uint32_t m = F.s_u[1];
  if (tid < 16u) dense[m + tid] = 0ull;
  lds_barrier();
  const double ln = log(F.s_d[1]);
  const uint32_t nout = min(n, V);
  for (uint32_t j = tid; j < m; j += NT) {
    const unsigned long long mine = dense[j];
    const uint32_t rank = rx_rank_of(dense, m, mine);
    if (rank < nout) {
      ids[rank] = (int32_t)(~(uint32_t)mine);
      lps[rank] = ((double)okey_value((uint32_t)(mine >> 32)) - M) - ln;
    }
  }
  for (uint32_t j = min(m, nout) + tid; j < n; j += NT) {
    ids[j] = -1;
    lps[j] = -INFINITY;
  }
  if (tid == 0) {
    A.rx_status[row] = 0;
    // the picked token's f64(l) - maximum - log_normalizer under the same
    // suppressed logits; NaN for a row without a token
    double lp = __builtin_nan("");
    if (t >= 0 && (uint32_t)t < V) {
      bool sup = false;
      if (bn <= 64u) {
        for (uint32_t l = 0; l < bn; ++l) sup |= supl[l] == (uint32_t)t;
      } else {
        uint32_t lo = b0, hi = b1;
        while (lo < hi) {   // bias ids increase within a row
          const uint32_t mid = (lo + hi) >> 1;
          if (b.bias_ids[mid] < (uint32_t)t) lo = mid + 1u;
          else hi = mid;
        }
        sup = lo < b1 && b.bias_ids[lo] == (uint32_t)t && b.bias_values[lo] == -INFINITY;
      }
      lp = ((double)(sup ? -FLT_MAX : tl) - M) - ln;
    }
    A.rx_token_lp[row] = lp;
  }
}

// What a chunk body leaves of the step receipt for the kernel to do after
// it: nothing, or the chunk's share (RX_FULL: the general body, whose raw
// logits are not in registers, or a lean chunk whose fast path failed).
// The kernel's share re-reads the chunk into registers after the body: in
// a body, next to its live registers, the reread share made it spill.
constexpr uint32_t RX_FULL = 2u;

// The row's last chunk to finish becomes its finisher.  Every wave waits for
// its own device-scope stores to complete before the workgroup barrier,
// which comes before thread 0's increment of the row counter; the last
// arriver's acquire fence, then the barrier, order its workgroup's loads
// after all of the row's stores (the ordering argument of arrive_last: a
// relaxed increment, no L2 write-back per arrival).
__device__ __forceinline__ bool arrive_row(const SampleArgs& A, ChunkSmem& S, uint32_t row) {
  wait_mem();
  __syncthreads();
  uint32_t last = 0;
  if (threadIdx.x == 0) {
    uint32_t* ctr = A.w.ctr + (uint64_t)row * CTR_STRIDE;
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev + 1u == A.C ? 1u : 0u;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    S.xkey = last;
  }
  __syncthreads();
  last = S.xkey;
  lds_barrier();   // the finisher's LDS overlays the chunk's
  return last != 0u;
}

// ---------------------------------------------------------------------------
// The lean chunk body: rows with no grammar mask, no logit bias and a history
// that fits the register staging (at most HCAP ids), in the greedy, top-k or
// min-p mode.  It writes the same chunk statistics and token-ID-ordered
// candidate list as the general body below, so the row finisher is shared.
// It differs in how it spends instructions:
//   - one pass per slice, as the slice's load lands: the count table is
//     built from registers right after the history ids arrive (they are
//     issued ahead of all but the first slice), so pass 1 overlaps the
//     stream instead of starting after it;
//   - every per-token decision is specialised at compile time (MODE, HIST):
//     no per-slice mode tests;
//   - min-p rows that need the row mass accumulate it online during the
//     stream, relative to a running per-thread maximum (each rescale is one
//     f32 exp2 per slice; the error bound below accounts for it), instead of
//     in a second pass over the registers after the chunk maximum is known;
//   - each wave publishes its maximum to the row's exchange word as soon as
//     its pass 1 ends, so the min-p threshold sees the other chunks' maxima
//     as early as possible.
template <typename In, uint32_t MODE, bool HIST, bool RX>
__device__ __forceinline__ uint32_t chunk_fast(const SampleArgs& A, FusedSmem& U, const RowCfg& c,
                                           const uint32_t row, const uint32_t chunk, const uint32_t c0,
                                           const uint32_t c1, const uint32_t hn, const uint32_t bn, const bool rx) {
  ChunkSmem& S = chunk_smem(U);
  const mxs_batch& b = A.b;
  const uint32_t tid = threadIdx.x;
  const uint32_t V = b.vocab;
  // The loads are issued here, per instantiation, so that no stream register
  // is live across the kernel's dispatch between the bodies (values live
  // across it made the register allocator spill, and a spill reload, being a
  // vector memory instruction, waits for every earlier load of the wave: the
  // whole stream).  The history ids go out first: the count table needs them
  // before pass 1.
  // (identical loads in every instantiation would otherwise be hoisted above
  // the dispatch as common code; an opaque use of the chunk offset keeps them
  // inside this body)
  uint32_t c0k = c0;
  __asm__ volatile("" : "+s"(c0k));
  uint32_t hreg[HCAP / NT];
  // the row's logit-bias entry `tid` (at most NT entries, none above 0) and
  // its predecessor's id
  uint32_t bid = NONE, bprev = 0u;
  float bval = 0.0f;
  if constexpr (HIST) {
    const uint32_t* hp = b.history_ids + c.hb;
    if (hn) {
#pragma unroll
      for (int r = 0; r < HCAP / NT; ++r) hreg[r] = hp[min((uint32_t)r * NT + tid, hn - 1u)];
    } else {
#pragma unroll
      for (int r = 0; r < HCAP / NT; ++r) hreg[r] = 0u;
    }
    if (tid < bn) {
      bid = b.bias_ids[c.bb + tid];
      bval = b.bias_values[c.bb + tid];
      if (tid > 0u) bprev = b.bias_ids[c.bb + tid - 1u];
    }
  }
  // The slices stream through a window of LA loads in flight per wave: slice
  // i + LA is issued as slice i is processed.  A wave issues in order, and a
  // load waits at issue while the CU's memory pipeline is full, so issuing
  // every slice up front would hold each wave at its last load until most
  // of the chunk had arrived, with pass 1 only starting after it.
  typename Quad<In>::Raw raw[PER_MAX];
  const In* src = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;
  auto issue = [&](int i) {
    const uint32_t e0 = c0k + (uint32_t)i * SLICE + tid * 4u;
    raw[i] = Quad<In>::load(src + (e0 < c1 ? e0 : c0k));
  };
  // (every thread issues all PER_MAX slices, past the chunk re-reading its
  // first quad, so each wave's count of loads in flight is known at compile
  // time and every wait is exact)
#pragma unroll
  for (int i = 0; i < LA; ++i) issue(i);
  const uint32_t clen = c1 - c0;
  const double invT = MODE == M_GREEDY ? 0.0 : 1.0 / c.T;
  uint32_t my_flags = 0;
  // T ln(min_p) for the min-p threshold, computed while the loads are in
  // flight (the empty asm keeps the f64 logarithm here instead of on the
  // path after the chunk reduction)
  double tlnmp = 0.0;
  if constexpr (MODE == M_MINP) {
    tlnmp = c.T * log(c.min_p);
    __asm__ volatile("" : "+v"(tlnmp));
  }

  // ---- the chunk's history count table (u16 per token) -------------------
  // Penalties in this body never raise a logit (repetition >= 1, frequency
  // and presence >= 0; other rows take the general body), and they touch
  // few tokens.  Pass 1 leaves every penalised token out of the statistics
  // (-inf), and the thread whose count-table increment came first for a
  // token (its owner) computes the token's adjusted logit from its own load
  // of the logit and adds it back; the candidate pass swaps the adjusted
  // logit in where a slice can hold a candidate (a penalised logit at or
  // above a threshold was at or above it before the penalty).  The owner
  // leaves the adjusted logit in pvals and marks the token's table entry
  // 0x8000 | slot.  Logit-bias entries join the same scheme when none of a
  // row's values is above 0 (the kernel checks), so the bias never raises a
  // logit either: each entry marks its token with 0x4000 before the history
  // counts go in, and owns it (bias ids are distinct), adding the bias as
  // bias_and_penalize does; its slot is hn + its index.
  uint32_t own = 0;              // bit r < 4: this thread owns history entry r's token; bit 4: bias entry tid's
  float hraw[HCAP / NT];         // the owned tokens' logits
  float braw = 0.0f;             // the biased token's logit
  float* pvals = reinterpret_cast<float*>(S.hids);   // HCAP adjusted logits by slot (the lean body stages no history)
  if constexpr (HIST) {
    const uint32_t n4 = A.per * (SLICE / 8);   // uint4 words covering per slices
    for (uint32_t t = tid; t < n4; t += NT) reinterpret_cast<uint4*>(S.t.ct)[t] = make_uint4(0u, 0u, 0u, 0u);
  }
  if constexpr (MODE == M_TOPK) S.hist[tid] = 0u;   // HB == NT
  if constexpr (HIST) {
    lds_barrier();
    if (bn) {   // (uniform) the bias marks, then a barrier before the history counts
      if (tid < bn) {
        if (bid >= V || !bias_ok(bval) || (tid > 0u && bprev >= bid)) my_flags |= F_BIAS;
        const uint32_t t = bid - c0;
        if (t < clen) {
          atomicAdd(&S.t.ct[t >> 1], (RX && bval == -INFINITY ? 0x6000u : 0x4000u) << ((t & 1u) * 16u));
          own |= 1u << 4;
        }
      }
      lds_barrier();
    }
#pragma unroll
    for (int r = 0; r < HCAP / NT; ++r) {
      const uint32_t j = (uint32_t)r * NT + tid;
      if (j < hn) {
        const uint32_t id = hreg[r];
        if (id >= V) my_flags |= F_HIST;
        const uint32_t t = id - c0;
        if (t < clen) {
          const uint32_t sh = (t & 1u) * 16u;
          const uint32_t old = atomicAdd(&S.t.ct[t >> 1], 1u << sh);
          if (((old >> sh) & 0xffffu) == 0u) own |= 1u << r;
        }
      }
    }
    // every thread issues its HCAP / NT loads (a non-owner re-reads the
    // chunk's first token): a fixed count of loads in flight per wave
#pragma unroll
    for (int r = 0; r < HCAP / NT; ++r) hraw[r] = Quad<In>::one(src + (((own >> r) & 1u) ? hreg[r] : c0k));
    braw = Quad<In>::one(src + (((own >> 4) & 1u) ? bid : c0k));
    lds_barrier();
  }
  stamp(A, row, chunk, 3);

  // ---- pass 1: penalties, finite check, statistics, online mass ----------
  const bool top2 = MODE == M_TOPK && c.k > TOP1_MAX;
  const bool do_mass = MODE == M_MINP && c.top_p < 1.0;
  const float c2 = (float)(invT * 1.4426950408889634);   // log2(e) / T
  const double inv_rep = 1.0 / (double)c.rep;
  float lv[PER_MAX][4];
  float qm[PER_MAX];
  float t1 = -INFINITY, t2 = -INFINITY, gv = -INFINITY;
  uint32_t gi = NONE;
  uint64_t nf = 0;
  // online mass: acc = sum of 2^((l - mrun) c2) over this thread's tokens so
  // far, eacc = the same weights times |(l - mrun) c2| (for the error
  // bound); mrun is the running maximum.  f32 throughout: one fused rescale
  // and add per slice.
  float mrun = -FLT_MAX;
  float acc = 0.0f, eacc = 0.0f;
  uint32_t pq = 0;   // bit i: this thread's quad of slice i holds a penalised token
#pragma unroll
  for (int i = 0; i < PER_MAX; ++i) {
    qm[i] = -INFINITY;
    if (i + LA < PER_MAX) issue(i + LA);
    if (i < (int)A.per) {
      const uint32_t sbase = c0 + (uint32_t)i * SLICE;
      const uint32_t e0 = sbase + tid * 4u;
      const bool full = sbase + (uint32_t)SLICE <= c1;   // uniform
      const uint32_t rb = full ? 0xfu : (e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u);
      float x[4];
      Quad<In>::unpack(raw[i], x);
      // xe: the logits the statistics see (penalised tokens left out)
      float xe[4] = {x[0], x[1], x[2], x[3]};
      if constexpr (HIST) {
        const uint2 cw = *reinterpret_cast<const uint2*>(&S.t.ct[((uint32_t)i * SLICE + tid * 4u) >> 1]);
        xe[0] = (cw.x & 0xffffu) ? -INFINITY : x[0];
        xe[1] = (cw.x >> 16) ? -INFINITY : x[1];
        xe[2] = (cw.y & 0xffffu) ? -INFINITY : x[2];
        xe[3] = (cw.y >> 16) ? -INFINITY : x[3];
        pq |= (cw.x | cw.y) ? 1u << i : 0u;
      }
      if (A.o.adjusted) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((rb >> e) & 1u) A.o.adjusted[(uint64_t)row * V + e0 + (uint32_t)e] = x[e];
      }
      if (full) {
#pragma unroll
        for (int e = 0; e < 4; ++e) nf |= __builtin_amdgcn_ballot_w64(!__builtin_isfinite(x[e]));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool inr = (rb >> e) & 1u;
          nf |= __builtin_amdgcn_ballot_w64(inr && !__builtin_isfinite(x[e]));
          x[e] = inr ? x[e] : -INFINITY;
          xe[e] = inr ? xe[e] : -INFINITY;
        }
      }
      if constexpr (MODE == M_GREEDY) {
        // IEEE >, first index wins (ids grow with e and i in this thread)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool g = xe[e] > gv;
          gv = g ? xe[e] : gv;
          gi = g ? e0 + (uint32_t)e : gi;
        }
      } else {
        // qm: the slice screen of the candidate pass (raw logits: a superset);
        // qe: the statistics' quad maximum
        qm[i] = vmax(vmax3(x[0], x[1], x[2]), x[3]);
        const float qe = HIST ? vmax(vmax3(xe[0], xe[1], xe[2]), xe[3]) : qm[i];
        if (top2) {
#pragma unroll
          for (int e = 0; e < 4; ++e) { t2 = vmed3(t1, t2, xe[e]); t1 = vmax(t1, xe[e]); }
        } else {
          t1 = vmax(t1, qe);
        }
        if (do_mass) {
          const float mnew = vmax(mrun, qe);
          const float ys = (mrun - mnew) * c2;                 // <= 0
          const float s = __builtin_amdgcn_exp2f(ys);
          float sw = 0.0f, ew = 0.0f;
          if (full) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // a left-out token (-inf) weighs 0 with a finite exponent
              const float y = HIST ? vmax((xe[e] - mnew) * c2, -200.0f) : (xe[e] - mnew) * c2;
              const float w = __builtin_amdgcn_exp2f(y);
              sw += w;
              ew = __builtin_fmaf(w, -y, ew);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool inr = (rb >> e) & 1u;
              const float y = HIST ? vmax((xe[e] - mnew) * c2, -200.0f) : (xe[e] - mnew) * c2;
              const float w = inr ? __builtin_amdgcn_exp2f(y) : 0.0f;
              sw += w;
              ew = inr ? __builtin_fmaf(w, -y, ew) : ew;
            }
          }
          // rescale what is accumulated to the new running maximum (s = 1
          // when it did not move); a zero accumulator stays zero
          const bool live = acc > 0.0f;
          eacc = live ? __builtin_fmaf(__builtin_fmaf(acc, -ys, eacc), s, ew) : ew;
          acc = live ? __builtin_fmaf(acc, s, sw) : sw;
          mrun = mnew;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) lv[i][e] = x[e];
    }
  }
  if constexpr (HIST) {
    // The owners' adjusted logits join the statistics (their loads landed
    // with the slices), go to pvals and mark their table entries.  Pass 1
    // wrote the penalised tokens' raw logits to the adjusted output: those
    // writes complete before the owners overwrite them.
    if (A.o.adjusted) {
      wait_mem();
      __syncthreads();
    }
    auto fold = [&](const float pv, const uint32_t id, const uint32_t t, const uint32_t slot) {
      if (!__builtin_isfinite(pv)) my_flags |= F_NONFINITE;
      if (A.o.adjusted) A.o.adjusted[(uint64_t)row * V + id] = pv;
      pvals[slot] = pv;
      // (with step receipts, a suppressed token's 0x2000, set with its bias
      // mark, stays: the receipt reads it)
      const uint32_t sflag = RX ? (S.t.ct[t >> 1] >> ((t & 1u) * 16u)) & 0x2000u : 0u;
      reinterpret_cast<uint16_t*>(S.t.ct)[t] = (uint16_t)(0x8000u | sflag | slot);
      if constexpr (MODE == M_GREEDY) {
        if (better(pv, id, gv, gi)) { gv = pv; gi = id; }
      } else {
        if (top2) {
          t2 = vmed3(t1, t2, pv);
          t1 = vmax(t1, pv);
        } else {
          t1 = vmax(t1, pv);
        }
        if (do_mass) {   // one more online step
          const float mnew = vmax(mrun, pv);
          const float ys = (mrun - mnew) * c2;
          const float sc = __builtin_amdgcn_exp2f(ys);
          const float y = vmax((pv - mnew) * c2, -200.0f);
          const float w = __builtin_amdgcn_exp2f(y);
          const bool live = acc > 0.0f;
          eacc = live ? __builtin_fmaf(__builtin_fmaf(acc, -ys, eacc), sc, w * -y) : w * -y;
          acc = live ? __builtin_fmaf(acc, sc, w) : w;
          mrun = mnew;
        }
      }
    };
#pragma unroll
    for (int r = 0; r < HCAP / NT; ++r) {
      if (!((own >> r) & 1u)) continue;
      const uint32_t id = hreg[r], t = id - c0, sh = (t & 1u) * 16u;
      const uint32_t cnt = (S.t.ct[t >> 1] >> sh) & 0xffffu;   // an unbiased token: its history count
      fold(bias_and_penalize(hraw[r], cnt, 0.0f, c.rep, inv_rep, c.freq, c.pres), id, t, (uint32_t)r * NT + tid);
    }
    if ((own >> 4) & 1u) {
      const uint32_t t = bid - c0, sh = (t & 1u) * 16u;
      const uint32_t cnt = (S.t.ct[t >> 1] >> sh) & 0x1fffu;   // the history count under the bias marks
      fold(bias_and_penalize(braw, 0x80000000u | cnt, bval, c.rep, inv_rep, c.freq, c.pres), bid, t, hn + tid);
    }
  }
  stamp(A, row, chunk, 6);

  // ---- chunk statistics: one block reduction ------------------------------
  const uint32_t nleg = clen;   // no mask: every token of the chunk is legal
  unsigned long long xprev = 0ull;   // min-p rows: the exchange word before this wave's update (lane 0)
  {
    const uint32_t kmax = wave_max_u32(okey(MODE == M_GREEDY ? gv : t1));
    if constexpr (MODE == M_MINP) {
      // this wave's maximum goes to the row's exchange word right away; the
      // value it replaces (the other chunks' maxima published so far)
      // returns while the workgroup reduces, and feeds the threshold
      if (lane() == 0)
        xprev = __hip_atomic_fetch_max(A.w.rowx + (uint64_t)row * ROWX_STRIDE,
                                       ((unsigned long long)A.epoch << 32) | kmax, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t wf = wave_or_u32(my_flags) | (nf ? (uint32_t)F_NONFINITE : 0u);
    unsigned long long arg = 0ull;
    if constexpr (MODE == M_GREEDY) {
      // -0.0 ties +0.0 under IEEE >: key both as +0.0 so the lower ID wins
      arg = gi == NONE ? 0ull : ((unsigned long long)okey(gv + 0.0f) << 32) | (unsigned long long)(~gi);
      arg = wave_max_u64(arg);
    }
    double w0s = 0.0, w1s = 0.0;
    if (do_mass) {
      // each lane's sum, rescaled from its running maximum to the wave's
      // (one more f32 rescale step, counted in the bound)
      const float wm = okey_value(kmax);
      const float ys = (mrun - wm) * c2;
      const float s = __builtin_amdgcn_exp2f(ys);
      const bool live = acc > 0.0f;
      const double e1 = live ? ((double)eacc + (double)acc * (double)(-ys)) * (double)s : 0.0;
      const double a1 = live ? (double)acc * (double)s : 0.0;
      w0s = wave_sum_f64(a1);
      w1s = wave_sum_f64(e1);
    }
    if (lane() == 0) {
      WavePart& p = S.wp[wave()];
      p.kmax = kmax; p.kmin = 0u; p.nleg = 0u; p.flags = wf; p.arg = arg; p.m0 = w0s; p.m1 = w1s;
    }
  }
  lds_barrier();
  uint32_t maxkey = 0u, cflags = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    maxkey = max(maxkey, S.wp[w].kmax);
    cflags |= S.wp[w].flags;
  }
  stamp(A, row, chunk, 1);
  const float m = okey_value(maxkey);   // chunk's largest logit
  const double md = (double)m;
  const bool row_ok = !(cflags & (F_HIST | F_NONFINITE));

  // ---- the step receipt's share of this chunk, from the raw logits in
  // registers (before the candidate pass swaps adjusted logits in); a
  // suppressed token (a bias entry of -inf) carries 0x2000 in the table.
  // Where its fast path fails, the kernel redoes the share after the body.
  bool rx_left = rx;
  if (RX && rx) {
    stamp(A, row, chunk, 10);
    rx_left = !receipt_chunk<PER_MAX>(A, S, row, chunk, c0, c1, [&](int i, float* r, uint32_t& rb) {
      const uint32_t sbase = c0 + (uint32_t)i * SLICE, e0 = sbase + tid * 4u;
      rb = sbase + (uint32_t)SLICE <= c1 ? 0xfu : (e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u);
      uint32_t sup = 0u;
      if constexpr (HIST) {
        if ((pq >> i) & 1u) {
          const uint2 cw = *reinterpret_cast<const uint2*>(&S.t.ct[((uint32_t)i * SLICE + tid * 4u) >> 1]);
          sup = ((cw.x & 0x2000u) ? 1u : 0u) | ((cw.x & 0x20000000u) ? 2u : 0u) | ((cw.y & 0x2000u) ? 4u : 0u) |
                ((cw.y & 0x20000000u) ? 8u : 0u);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = ((sup >> e) & 1u) ? -FLT_MAX : lv[i][e];
    });
    stamp(A, row, chunk, 11);
  }

  // ---- candidate threshold and counts --------------------------------------
  float thr = -INFINITY;
  bool emit = false;
  if (MODE == M_TOPK && row_ok) {
    emit = true;
    const uint32_t need = min(c.k, nleg);
    if (need < nleg) {
      // The need-th largest of the per-thread maxima (top-2 maxima for
      // large k) is at most the chunk's need-th largest logit.  Histogram
      // them on a 1/32-logit grid below m, find the bin where the count
      // reaches need, and emit down to one bin below it.
      const float scale = (float)HB / HRANGE;
      {
        const float d1 = (m - t1) * scale;
        if (d1 < (float)(HB - 1)) atomicAdd(&S.hist[(uint32_t)d1], 1u);
        if (top2) {
          const float d2 = (m - t2) * scale;
          if (d2 < (float)(HB - 1)) atomicAdd(&S.hist[(uint32_t)d2], 1u);
        }
      }
      lds_barrier();
      // every wave: lane j sums bins 16 j .. 16 j + 15; the crossing group's
      // bins are then scanned lane-parallel (no per-bin serial walk)
      uint32_t s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 h4 = *reinterpret_cast<const uint4*>(&S.hist[lane() * 16u + (uint32_t)q * 4u]);
        s += h4.x + h4.y + h4.z + h4.w;
      }
      const uint32_t inc = wave_scan_u32(s);
      const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
      if (reach) {
        const uint32_t g = (uint32_t)__builtin_ctzll(reach);
        const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - s), (int)g);
        const uint32_t v = lane() < 16u ? S.hist[16u * g + lane()] : 0u;
        const uint32_t vi = base + wave_scan_u32(v);
        const uint64_t r2 = __builtin_amdgcn_ballot_w64(lane() < 16u && vi >= need);
        const uint32_t tb = 16u * g + (uint32_t)__builtin_ctzll(r2);
        thr = m - (float)(tb + 2u) / scale;
      }
    }
  } else if (MODE == M_MINP && row_ok) {
    // The largest chunk maximum of the row published by now is a lower
    // bound of the row maximum: any lower bound gives a superset of the
    // min-p set, a tighter one fewer candidates.  ln(min_p) in f64 (an f32
    // logarithm's error, T * 2^-24 absolute, is not covered by a margin
    // relative to the logits when they and T ln(min_p) are near 0).
    emit = true;
    const uint32_t xhi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(xprev >> 32));
    const uint32_t xlo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)xprev);
    const uint32_t xkey = xhi == A.epoch ? max(maxkey, xlo) : maxkey;
    const float mx = okey_value(xkey);
    const double lim_d = (double)mx + tlnmp;
    thr = (float)lim_d - (fabsf((float)lim_d) + fabsf(mx)) * 1e-5f - 1e-30f;
  }
  uint32_t cnt_i[PER_MAX];
  // Out-of-range tokens hold -inf: a finite threshold needs no range mask
  // (a threshold of -inf takes every in-range token, so it does).
  const bool thr_fin = thr > -INFINITY;   // uniform
  if (emit) {
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      cnt_i[i] = 0u;
      if (i < (int)A.per) {
        // screen the slice on the quad maxima first
        uint32_t cnt = 0;
        if (__builtin_amdgcn_ballot_w64(qm[i] >= thr)) {
          if (HIST && __builtin_amdgcn_ballot_w64(((pq >> i) & 1u) && qm[i] >= thr)) {
            // a penalised token can only be a candidate if its raw logit is
            // (penalties never raise a logit): then its owner's adjusted
            // logit comes in
            if (((pq >> i) & 1u) && qm[i] >= thr) {
              const uint2 cw = *reinterpret_cast<const uint2*>(&S.t.ct[((uint32_t)i * SLICE + tid * 4u) >> 1]);
              const uint32_t h[4] = {cw.x & 0xffffu, cw.x >> 16, cw.y & 0xffffu, cw.y >> 16};
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (h[e] && lv[i][e] >= thr) lv[i][e] = pvals[h[e] & 0xfffu];
            }
          }
          if (thr_fin) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              cnt += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lv[i][e] >= thr));
          } else {
            const uint32_t sbase = c0 + (uint32_t)i * SLICE;
            const uint32_t e0 = sbase + tid * 4u;
            const uint32_t rb = sbase + (uint32_t)SLICE <= c1 ? 0xfu
                                : (e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              cnt += (uint32_t)__builtin_popcountll(
                  __builtin_amdgcn_ballot_w64(((rb >> e) & 1u) && lv[i][e] >= thr));
          }
        }
        cnt_i[i] = cnt;
        if (lane() == 0) S.wcnt[i * NW + wave()] = cnt;
      }
    }
  }
  // the chunk mass, relative to the chunk maximum: wave 0 rescales the
  // waves' sums (lane w <-> wave w) in f64
  double mass = 0.0, mass_err = 0.0;
  if (do_mass && row_ok && wave() == 0) {
    // lane w rescales wave w's sum from the wave maximum to the chunk
    // maximum (one more f32 rescale step, counted in the bound)
    const uint32_t w = lane();
    double a = 0.0, e = 0.0;
    if (w < (uint32_t)NW) {
      const float ys = (okey_value(S.wp[w].kmax) - m) * c2;   // <= 0
      const double sc = (double)__builtin_amdgcn_exp2f(ys);
      const double m0w = S.wp[w].m0;
      a = m0w > 0.0 ? m0w * sc : 0.0;
      e = m0w > 0.0 ? (S.wp[w].m1 + m0w * (double)(-ys)) * sc : 0.0;
    }
    const double S0 = wave_sum_f64(a), E0 = wave_sum_f64(e);
    mass = S0;
    // |mass - sum of exact weights| <= 1.01 (2^-22 S (per + 3) +
    // (per + 5) 2^-24 S) for the f32 exp2 of each weight and of each of at
    // most per + 2 rescale factors (2 ulp each), the 4-term f32 slice sums
    // and the per fused f32 rescale-and-adds, + 1.01 ln2 3 2^-24 sum w |y|
    // for the rounding of the exponents (three f32 roundings each,
    // relative; a term's exponent and the rescale exponents applied to it
    // telescope to its distance from the chunk maximum), + n 2^-120 for
    // weights and factors below 2^-126, + 2^-40 S for the f64 sums.
    // (each owned history token is one more step)
    const uint32_t steps = A.per + (HIST ? (uint32_t)(HCAP / NT) + 1u : 0u);
    mass_err = 1.01 * (0x1p-22 * S0 * (double)(steps + 3u) + (double)(steps + 5u) * 0x1p-24 * S0 +
                       0.6931471805599453 * 3.0001 * 0x1p-24 * E0) +
               (double)nleg * 0x1p-120 + 0x1p-40 * S0;
  }
  stamp(A, row, chunk, 5);
  uint32_t ncand = 0;
  if (emit) {
    lds_barrier();
    // exclusive offsets in (slice, wave) order == token-ID order; every wave
    // scans the PER_MAX * NW counts itself (lane j holds j, j + 64, j + 128)
    const uint32_t nent = A.per * NW;
    const uint32_t v0 = lane() < nent ? S.wcnt[lane()] : 0u;
    const uint32_t v1 = lane() + 64u < nent ? S.wcnt[lane() + 64u] : 0u;
    const uint32_t v2 = lane() + 128u < nent ? S.wcnt[lane() + 128u] : 0u;
    const uint32_t i0 = wave_scan_u32(v0), i1 = wave_scan_u32(v1), i2 = wave_scan_u32(v2);
    const uint32_t s0 = (uint32_t)__builtin_amdgcn_readlane((int)i0, 63);
    const uint32_t s1 = (uint32_t)__builtin_amdgcn_readlane((int)i1, 63);
    const uint32_t s2 = (uint32_t)__builtin_amdgcn_readlane((int)i2, 63);
    ncand = s0 + s1 + s2;
    if constexpr (MODE == M_MINP) {
      if (do_mass && row_ok && ncand > WIDE_NCAND) {
        // A wide min-p set: its nucleus cut can fall between tokens that
        // each carry about 1e-5 of the row mass, finer than the f32 mass's
        // bound, so the chunk mass is summed again from f64 weights relative
        // to the chunk maximum (penalised tokens by their owners; the count
        // table, still intact here, marks them).
        double part = 0.0;
#pragma unroll
        for (int i = 0; i < PER_MAX; ++i) {
          if (i < (int)A.per) {
            uint32_t skip = 0;
            if constexpr (HIST) {
              if ((pq >> i) & 1u) {
                const uint2 cw = *reinterpret_cast<const uint2*>(&S.t.ct[((uint32_t)i * SLICE + tid * 4u) >> 1]);
                skip = ((cw.x & 0xffffu) ? 1u : 0u) | ((cw.x >> 16) ? 2u : 0u) | ((cw.y & 0xffffu) ? 4u : 0u) |
                       ((cw.y >> 16) ? 8u : 0u);
              }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (!((skip >> e) & 1u)) part += exp_neg_p(((double)lv[i][e] - md) * invT);
          }
        }
        if constexpr (HIST) {
#pragma unroll
          for (int r = 0; r < HCAP / NT; ++r)
            if ((own >> r) & 1u) part += exp_neg_p(((double)pvals[(uint32_t)r * NT + tid] - md) * invT);
          if ((own >> 4) & 1u) part += exp_neg_p(((double)pvals[hn + tid] - md) * invT);
        }
        mass = block_sum<double>(part, reinterpret_cast<double*>(S.wq));
        // 2 ulp per weight plus the sums (sum_bound), and the rounding of
        // (l - m) / T as a product (at most 3 ulp of it: w |x| 3 2^-53 <= 3 2^-53 / e)
        mass_err = sum_bound(mass, nleg + (uint32_t)NT, 8.0) + 3.0 * 0.37 * (double)nleg * mxs::U;
      }
    }
    const uint32_t x0 = i0 - v0, x1 = i1 - v1 + s0, x2 = i2 - v2 + s0 + s1;
    const uint64_t cbase = (uint64_t)row * V + c0;
    // Candidates are staged in LDS (the count table is dead by now) and then
    // copied out with coalesced stores: scattered per-element global stores
    // cost an address-unit pass per store instruction, tens per wave.
    const bool staged = ncand <= (uint32_t)(CHUNK_MAX / 4);   // uniform
    float* stl = reinterpret_cast<float*>(S.t.ct);
    uint32_t* sti = S.t.ct + CHUNK_MAX / 4;
    if (staged && thr_fin) {
      // the common case: staged, and a finite threshold (no range masks)
#pragma unroll
      for (int i = 0; i < PER_MAX; ++i) {
        if (i < (int)A.per && cnt_i[i]) {
          const uint32_t idx = (uint32_t)i * NW + wave();
          const uint32_t src = idx & 63u;
          const uint32_t reg = idx >> 6;
          const uint32_t xv = reg == 0 ? x0 : (reg == 1 ? x1 : x2);
          const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)xv, (int)src);
          const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
          uint32_t off = base;
#pragma unroll
          for (int e = 0; e < 4; ++e) off += lanes_below(__builtin_amdgcn_ballot_w64(lv[i][e] >= thr));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (lv[i][e] >= thr) {
              stl[off] = lv[i][e];
              sti[off] = e0 + (uint32_t)e;
              ++off;
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < PER_MAX; ++i) {
        if (i < (int)A.per && cnt_i[i]) {
          const uint32_t idx = (uint32_t)i * NW + wave();
          const uint32_t src = idx & 63u;
          const uint32_t reg = idx >> 6;
          const uint32_t xv = reg == 0 ? x0 : (reg == 1 ? x1 : x2);
          const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)xv, (int)src);
          const uint32_t sbase = c0 + (uint32_t)i * SLICE;
          const uint32_t e0 = sbase + tid * 4u;
          const uint32_t rb = sbase + (uint32_t)SLICE <= c1 ? 0xfu
                              : (e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u);
          bool em[4];
          uint32_t before_me = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            em[e] = (thr_fin || ((rb >> e) & 1u)) && lv[i][e] >= thr;
            before_me += lanes_below(__builtin_amdgcn_ballot_w64(em[e]));
          }
          uint32_t off = base + before_me;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (em[e]) {
              if (staged) {
                stl[off] = lv[i][e];
                sti[off] = e0 + (uint32_t)e;
              } else {
                const uint64_t pos = cbase + off;
                st_dev(&A.w.cand_l[pos], lv[i][e]);
                st_dev(&A.w.cand_id[pos], e0 + (uint32_t)e);
              }
              ++off;
            }
          }
        }
      }
    }
    if (staged) {
      lds_barrier();
      for (uint32_t j = tid; j < ncand; j += NT) {
        st_dev(&A.w.cand_l[cbase + j], stl[j]);
        st_dev(&A.w.cand_id[cbase + j], sti[j]);
      }
    }
  }

  // ---- publish the chunk's statistics (the row finisher kernel reads them)
  stamp(A, row, chunk, 7);
  if (tid == 0) {
    unsigned long long garg = 0ull;
    if constexpr (MODE == M_GREEDY)
      for (int w = 0; w < NW; ++w) garg = garg > S.wp[w].arg ? garg : S.wp[w].arg;
    ChunkStat& st = A.w.stat[(uint64_t)row * MAXC + chunk];
    st_dev(&st.maxkey, nleg ? maxkey : 0u);
    st_dev(&st.gbest_id, garg ? ~(uint32_t)garg : NONE);
    st_dev(&st.gbest_val, garg ? okey_value((uint32_t)(garg >> 32)) : 0.0f);
    st_dev(&st.nlegal, nleg);
    st_dev(&st.ncand, ncand);
    st_dev(&st.flags, cflags);
    st_dev(&st.mass, mass);
    st_dev(&st.mass_err, mass_err);
    st_dev(&st.minkey, 0u);
    st_dev(&st.thr, thr);
  }
  stamp(A, row, chunk, 2);
  return rx_left ? RX_FULL : 0u;
}

// The general chunk body: every row the lean body does not cover (grammar
// masks, logit bias, long histories, parameter errors, the all-candidates
// and keep-all modes).  The kernel has
// already read the row's parameters (c).  The kernel's own load of the
// first slice is not passed in (it would stay live across both bodies): the
// general body issues its slices itself.
template <typename In>
__device__ __forceinline__ uint32_t chunk_general(const SampleArgs& A, FusedSmem& U, const RowCfg& c,
                                              const uint32_t row, const uint32_t chunk, const bool rx) {
  ChunkSmem& S = chunk_smem(U);
  const mxs_batch& b = A.b;
  const uint32_t tid = threadIdx.x;
  const uint32_t V = b.vocab;
  stamp(A, row, chunk, 0);
  const uint32_t c0 = chunk * A.CH;
  const uint32_t c1 = min(V, c0 + A.CH);
  const In* src = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;

  // ---- stream the chunk ---------------------------------------------------
  // Vector loads complete in issue order, so the issue order below is the
  // order data becomes usable: the first slice, then
  // the row's history and bias lists and the chunk's mask words (staged into
  // LDS), then the rest of the chunk.  A quad starting below the chunk end
  // lies inside the row stride (a multiple of 4); past the end, the chunk's
  // first quad is re-read and ignored.
  typename Quad<In>::Raw raw[PER_MAX];
  raw[0] = Quad<In>::load(src + (c0 + tid * 4u < c1 ? c0 + tid * 4u : c0));
  const uint32_t mode = chunk_mode(c, V);
  const double invT = c.greedy ? 0.0 : 1.0 / c.T;
  const uint32_t hn = c.he > c.hb ? c.he - c.hb : 0u, bn = c.be > c.bb ? c.be - c.bb : 0u;
  const bool has_tab = hn || bn;
  const bool h_lds = hn <= (uint32_t)HCAP, b_lds = bn <= (uint32_t)BCAP;
  const uint32_t w0 = c0 >> 5, nmw = ((c1 - 1u) >> 5) - w0 + 1u;
  // The row's history and bias lists (when they fit in LDS) and, for masked
  // rows, the chunk's mask words go through registers into LDS.  They are
  // issued before the bulk of the logits, so they land first (vector loads
  // complete in issue order); each lane loads whole 1024-entry rounds,
  // repeating the last entry past the list's end.
  const bool stage_h = hn && h_lds, stage_b = bn && b_lds, stage_m = A.masked != 0u;
  uint32_t hreg[HCAP / NT], breg[BCAP / NT], mreg[MCAP / NT];
  float vreg[BCAP / NT];
  if (stage_h) {
    const uint32_t* hp = b.history_ids + c.hb;
#pragma unroll
    for (int r = 0; r < HCAP / NT; ++r) hreg[r] = hp[min((uint32_t)r * NT + tid, hn - 1u)];
  }
  if (stage_b) {
    const uint32_t* ip = b.bias_ids + c.bb;
    const float* vp = b.bias_values + c.bb;
#pragma unroll
    for (int r = 0; r < BCAP / NT; ++r) {
      breg[r] = ip[min((uint32_t)r * NT + tid, bn - 1u)];
      vreg[r] = vp[min((uint32_t)r * NT + tid, bn - 1u)];
    }
  }
  if (stage_m) {
    const uint32_t* mp = b.mask_words + (uint64_t)row * b.mask_stride + w0;
#pragma unroll
    for (int r = 0; r < MCAP / NT; ++r) mreg[r] = mp[min((uint32_t)r * NT + tid, nmw - 1u)];
  }
  const double etab_v = tid < 128u ? (tid < 64u ? kExp2Tab[tid] : kExp2TabLo[tid - 64u]) : 0.0;
#pragma unroll
  for (int i = 1; i < PER_MAX; ++i) {
    const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
    raw[i] = Quad<In>::load(src + (e0 < c1 ? e0 : c0));
  }
  if (stage_h) {
#pragma unroll
    for (int r = 0; r < HCAP / NT; ++r) S.hids[r * NT + tid] = hreg[r];
  }
  if (tid < 128u) S.etab[tid] = etab_v;
  if (stage_b) {
#pragma unroll
    for (int r = 0; r < BCAP / NT; ++r) { S.bids[r * NT + tid] = breg[r]; S.bvals[r * NT + tid] = vreg[r]; }
  }
  if (stage_m) {
#pragma unroll
    for (int r = 0; r < MCAP / NT; ++r) S.mask[r * NT + tid] = mreg[r];
  }
  // History counts and bias flags: one table for the whole chunk, built
  // once, when no count can pass 15 bits and the bias list is in LDS (its
  // values are found by binary search there); otherwise per-slice u32 tables.
  const bool tab_chunk = has_tab && hn <= CT_MAXH && b_lds;
  const bool tab_slices = has_tab && !tab_chunk;
  if (tab_chunk) {
    const uint32_t n4 = A.per * (SLICE / 8);   // uint4 words covering per slices
    for (uint32_t t = tid; t < n4; t += NT) reinterpret_cast<uint4*>(S.t.ct)[t] = make_uint4(0u, 0u, 0u, 0u);
  } else if (tab_slices) {
    for (uint32_t t = tid; t < (uint32_t)(2 * SLICE); t += NT) (&S.t.sl.tab[0][0])[t] = 0u;
  }
  if (mode == M_TOPK) S.hist[tid] = 0u;   // HB == NT
  lds_barrier();
  uint32_t my_flags = 0;
  if (has_tab && !c.err) {
    // validation: history ids below the vocabulary; bias ids strictly
    // increasing, below the vocabulary, with finite values
    // (LDS and global copies in separate loops: a pointer select between
    // them would compile to flat loads, which wait on every global load)
    if (h_lds) {
      for (uint32_t j = tid; j < hn; j += NT)
        if (S.hids[j] >= V) my_flags |= F_HIST;
    } else {
      for (uint32_t j = tid; j < hn; j += NT)
        if (b.history_ids[c.hb + j] >= V) my_flags |= F_HIST;
    }
    if (b_lds) {
      for (uint32_t j = tid; j < bn; j += NT) {
        const uint32_t id = S.bids[j];
        const uint32_t prev = j == 0 ? 0u : S.bids[j - 1];
        if (id >= V || !bias_ok(S.bvals[j]) || (j > 0 && prev >= id)) my_flags |= F_BIAS;
      }
    } else {
      for (uint32_t j = tid; j < bn; j += NT) {
        const uint32_t id = b.bias_ids[c.bb + j];
        const uint32_t prev = j == 0 ? 0u : b.bias_ids[c.bb + j - 1];
        if (id >= V || !bias_ok(b.bias_values[c.bb + j]) || (j > 0 && prev >= id)) my_flags |= F_BIAS;
      }
    }
  }
  const uint32_t clen = c1 - c0;
  if (tab_chunk) {
    if (h_lds) {
      for (uint32_t j = tid; j < hn; j += NT) {
        const uint32_t t = S.hids[j] - c0;
        if (t < clen) atomicAdd(&S.t.ct[t >> 1], 1u << ((t & 1u) * 16u));
      }
    } else {
      for (uint32_t j = tid; j < hn; j += NT) {
        const uint32_t t = b.history_ids[c.hb + j] - c0;
        if (t < clen) atomicAdd(&S.t.ct[t >> 1], 1u << ((t & 1u) * 16u));
      }
    }
    for (uint32_t j = tid; j < bn; j += NT) {
      const uint32_t t = S.bids[j] - c0;
      if (t < clen) atomicOr(&S.t.ct[t >> 1], 0x8000u << ((t & 1u) * 16u));
    }
    lds_barrier();
  }

  stamp(A, row, chunk, 3);
  // ---- pass 1: bias, penalties, mask, finite check, chunk statistics ------
  // Full slices of unmasked rows take a path with no per-token legality
  // work; partial slices and masked rows carry 4 legal bits per slice.
  // Penalised tokens are rare: each of the quad's 4 lanes enters the
  // penalty arithmetic only when some lane of the wave needs it.
  const bool masked_row = A.masked != 0u;
  const uint32_t lim = masked_row ? min(c1, b.tokenizer_vocab) : c1;   // no legal token at or past lim
  const bool want_top2 = mode == M_TOPK && c.k > (uint32_t)TOP1_MAX;
  const bool want_min = mode == M_KEEPALL;
  const bool want_arg = mode == M_GREEDY;
  const double inv_rep = 1.0 / (double)c.rep;
  float lv[PER_MAX][4];
  float qm[PER_MAX];                  // per slice: the largest legal logit of this thread's quad
#pragma unroll
  for (int i = 0; i < PER_MAX; ++i) qm[i] = -INFINITY;
  uint64_t lq = 0;                    // legal bits of partial / masked slices, 4 per slice
  float t1 = -INFINITY, t2 = -INFINITY, tmin = INFINITY, gv = -INFINITY;
  uint32_t gi = NONE, nleg = 0;
  uint64_t nf = 0;                    // wave-uniform: a lane saw a non-finite logit
#pragma unroll
  for (int i = 0; i < PER_MAX; ++i) {
    if (i < (int)A.per) {
      const uint32_t sbase = c0 + (uint32_t)i * SLICE;
      const uint32_t send = min(c1, sbase + (uint32_t)SLICE);
      uint32_t tva[4] = {0u, 0u, 0u, 0u};   // count | bias flag << 31
      float bva[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      bool tab_hit = false;   // wave-uniform: some lane's quad has a history or bias entry
      if (tab_chunk) {
        const uint2 cw = *reinterpret_cast<const uint2*>(&S.t.ct[((uint32_t)i * SLICE + tid * 4u) >> 1]);
        // Most quads of most waves hold no entry: decode only when one does.
        tab_hit = __builtin_amdgcn_ballot_w64((cw.x | cw.y) != 0u) != 0ull;
        if (tab_hit) {
          const uint32_t h[4] = {cw.x & 0xffffu, cw.x >> 16, cw.y & 0xffffu, cw.y >> 16};
#pragma unroll
          for (int e = 0; e < 4; ++e) tva[e] = (h[e] & 0x7fffu) | ((h[e] & 0x8000u) << 16);
        }
      } else if (tab_slices) {
        tab_hit = true;
        const int buf = i & 1;
        // Scatter this slice's history ids (counts) and bias ids (flag and
        // value) into the LDS table; a buffer is rewritten two slices later,
        // after the next slice's barrier, so one barrier per slice suffices.
        for (uint32_t j = tid; j < hn; j += NT) {
          const uint32_t id = b.history_ids[c.hb + j];
          if (id >= sbase && id < send) atomicAdd(&S.t.sl.tab[buf][id - sbase], 1u);
        }
        if (b_lds) {
          for (uint32_t j = tid; j < bn; j += NT) {
            const uint32_t id = S.bids[j];
            if (id >= sbase && id < send) {
              atomicOr(&S.t.sl.tab[buf][id - sbase], 0x80000000u);
              S.t.sl.btab[buf][id - sbase] = S.bvals[j];
            }
          }
        } else {
          for (uint32_t j = tid; j < bn; j += NT) {
            const uint32_t id = b.bias_ids[c.bb + j];
            if (id >= sbase && id < send) {
              atomicOr(&S.t.sl.tab[buf][id - sbase], 0x80000000u);
              S.t.sl.btab[buf][id - sbase] = b.bias_values[c.bb + j];
            }
          }
        }
        lds_barrier();
        const uint4 tv = *reinterpret_cast<uint4*>(&S.t.sl.tab[buf][tid * 4u]);
        const float4 bv4 = *reinterpret_cast<float4*>(&S.t.sl.btab[buf][tid * 4u]);
        *reinterpret_cast<uint4*>(&S.t.sl.tab[buf][tid * 4u]) = make_uint4(0u, 0u, 0u, 0u);
        tva[0] = tv.x; tva[1] = tv.y; tva[2] = tv.z; tva[3] = tv.w;
        bva[0] = bv4.x; bva[1] = bv4.y; bva[2] = bv4.z; bva[3] = bv4.w;
      }
      float x[4];
      Quad<In>::unpack(raw[i], x);
      if (tab_hit) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool hit = tva[e] != 0u;
          if (__builtin_amdgcn_ballot_w64(hit)) {
            float bias = bva[e];
            if (tab_chunk && (tva[e] >> 31)) {
              // the bias value: binary search over the strictly increasing ids
              const uint32_t id = sbase + tid * 4u + (uint32_t)e;
              uint32_t lo = 0, hi = bn;
              while (lo < hi) { const uint32_t md2 = (lo + hi) >> 1; if (S.bids[md2] < id) lo = md2 + 1u; else hi = md2; }
              bias = S.bvals[min(lo, bn - 1u)];
            }
            x[e] = hit ? bias_and_penalize(x[e], tva[e], bias, c.rep, inv_rep, c.freq, c.pres) : x[e];
          }
        }
      }
      const uint32_t e0 = sbase + tid * 4u;
      const bool full = !masked_row && send - sbase == (uint32_t)SLICE;   // uniform
      uint32_t qb = 0xfu, rb = 0xfu;  // legal bits, in-range bits of the quad
      if (!full) {
        rb = e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u;
        const uint32_t lb = e0 < lim ? (lim - e0 >= 4u ? 0xfu : (1u << (lim - e0)) - 1u) : 0u;
        const uint32_t mw = (masked_row && e0 < c1) ? (S.mask[(e0 >> 5) - w0] >> (e0 & 31u)) & 0xfu : 0xfu;
        qb = lb & mw;
        lq |= (uint64_t)qb << (4 * i);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) lv[i][e] = x[e];
      if (full) {
        // every token of the quad is in range and legal
#pragma unroll
        for (int e = 0; e < 4; ++e) nf |= __builtin_amdgcn_ballot_w64(!__builtin_isfinite(x[e]));
        if (want_arg) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool g = x[e] > gv;
            gv = g ? x[e] : gv;
            gi = g ? e0 + (uint32_t)e : gi;
          }
        } else if (want_top2) {
          // top two per thread: with t1 >= t2, med3(t1, t2, x) is the new second
#pragma unroll
          for (int e = 0; e < 4; ++e) { t2 = vmed3(t1, t2, x[e]); t1 = vmax(t1, x[e]); }
          qm[i] = vmax(vmax3(x[0], x[1], x[2]), x[3]);
        } else if (want_min) {
          t1 = vmax3(vmax3(t1, x[0], x[1]), x[2], x[3]);
          tmin = vmin3(vmin3(tmin, x[0], x[1]), x[2], x[3]);
        } else {
          qm[i] = vmax(vmax3(x[0], x[1], x[2]), x[3]);
          t1 = vmax(t1, qm[i]);
        }
      } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool inr = (rb >> e) & 1u;
        nf |= __builtin_amdgcn_ballot_w64(inr && !__builtin_isfinite(x[e]));
        const bool lg = (qb >> e) & 1u;
        const float lm = lg ? x[e] : -INFINITY;
        if (want_top2) t2 = fmaxf(t2, fminf(t1, lm));
        t1 = fmaxf(t1, lm);
        qm[i] = fmaxf(qm[i], lm);
        if (want_min) tmin = fminf(tmin, lg ? x[e] : INFINITY);
        if (want_arg) {
          const bool g = lm > gv;
          gv = g ? lm : gv;
          gi = g ? e0 + (uint32_t)e : gi;
        }
      }
      }
      if (A.o.adjusted) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((rb >> e) & 1u) A.o.adjusted[(uint64_t)row * V + e0 + (uint32_t)e] = x[e];
      }
      nleg += full ? 4u : (uint32_t)__builtin_popcount(qb);
    }
  }
  stamp(A, row, chunk, 6);

  // ---- chunk statistics: one block reduction ------------------------------
  {
    const uint32_t kmax = wave_max_u32(okey(t1));
    const uint32_t kmin = want_min ? ~wave_max_u32(~okey(tmin)) : 0u;
    const uint32_t wn = wave_sum_u32(nleg);
    const uint32_t wf = wave_or_u32(my_flags) | (nf ? (uint32_t)F_NONFINITE : 0u);
    unsigned long long arg = 0ull;
    if (want_arg) {
      // -0.0 ties +0.0 under IEEE >: key both as +0.0 so the lower ID wins
      arg = gi == NONE ? 0ull : ((unsigned long long)okey(gv + 0.0f) << 32) | (unsigned long long)(~gi);
      arg = wave_max_u64(arg);
    }
    if (lane() == 0) {
      WavePart& p = S.wp[wave()];
      p.kmax = kmax; p.kmin = kmin; p.nleg = wn; p.flags = wf; p.arg = arg;
    }
  }
  lds_barrier();
  uint32_t maxkey = 0u, minkey = NONE, cflags = 0u;
  nleg = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const WavePart& p = S.wp[w];
    maxkey = max(maxkey, p.kmax);
    minkey = min(minkey, p.kmin);
    nleg += p.nleg;
    cflags |= p.flags;
  }
  stamp(A, row, chunk, 1);
  const float m = nleg ? okey_value(maxkey) : 0.0f;   // chunk's largest legal logit
  const double md = (double)m;
  const bool row_ok = !c.err && !(cflags & (F_HIST | F_BIAS | F_NONFINITE));

  // ---- pass 2: candidate threshold, counts, chunk mass --------------------
  // Candidates are emitted in token-ID order: per (slice, wave) counts, an
  // exclusive scan, then the writes.  A token is a candidate when it is
  // legal and its logit is at least `thr`.
  uint32_t ncand = 0;
  double mass = 0.0, mass_err = 0.0;
  const uint64_t rbase = (uint64_t)row * V;
  bool emit = false;
  float thr = -INFINITY;
  // Min-p rows: the row maximum is at least every chunk maximum, so each
  // chunk publishes its maximum key (epoch-tagged atomic max, one word per
  // row) and later takes the largest published so far as a lower bound of
  // the row maximum.  Any lower bound gives a superset of the min-p set;
  // the exchange only makes it tighter.
  bool minp_x = false;
  uint32_t xkey = maxkey;
  if (row_ok && nleg > 0) {
    if (mode == M_TOPK) {
      emit = true;
      const uint32_t need = min(c.k, nleg);
      if (need < nleg) {
        // The need-th largest of the per-thread maxima (top-2 maxima for
        // large k) is at most the chunk's need-th largest legal logit.
        // Histogram them on a 1/32-logit grid below m, find the bin where
        // the count reaches need, and emit down to one bin below it.
        const float scale = (float)HB / HRANGE;
        {
          const float d1 = (m - t1) * scale;
          if (d1 < (float)(HB - 1)) atomicAdd(&S.hist[(uint32_t)d1], 1u);
          if (want_top2) {
            const float d2 = (m - t2) * scale;
            if (d2 < (float)(HB - 1)) atomicAdd(&S.hist[(uint32_t)d2], 1u);
          }
        }
        lds_barrier();
        // Every wave finds the bin itself: lane j sums bins [16j, 16j + 16).
        uint32_t hv[16];
        uint32_t s = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint4 h4 = *reinterpret_cast<const uint4*>(&S.hist[lane() * 16u + (uint32_t)q * 4u]);
          hv[q * 4 + 0] = h4.x; hv[q * 4 + 1] = h4.y; hv[q * 4 + 2] = h4.z; hv[q * 4 + 3] = h4.w;
          s += h4.x + h4.y + h4.z + h4.w;
        }
        const uint32_t inc = wave_scan_u32(s);
        const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
        if (reach) {
          const uint32_t L = (uint32_t)__builtin_ctzll(reach);
          uint32_t run = inc - s, bin = 16u * lane() + 15u;
          bool found = false;
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            run += hv[q];
            if (!found && run >= need) { found = true; bin = 16u * lane() + (uint32_t)q; }
          }
          const uint32_t tb = (uint32_t)__builtin_amdgcn_readlane((int)bin, (int)L);
          thr = m - (float)(tb + 2u) / scale;
        }
      }
    } else if (mode == M_MINP) {
      // The threshold comes after the mass pass, from the largest chunk
      // maximum of the row published by then (see below).
      emit = true;
      minp_x = true;
      if (tid == 0) {
        const unsigned long long old = __hip_atomic_fetch_max(
            A.w.rowx + (uint64_t)row * ROWX_STRIDE, ((unsigned long long)A.epoch << 32) | maxkey, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(old >> 32) == A.epoch) xkey = max(xkey, (uint32_t)old);
      }
    } else if (mode == M_ALL) {
      emit = true;
    }
  }
  stamp(A, row, chunk, 4);
  const bool mass32 = row_ok && nleg > 0 &&
                      ((mode == M_MINP && c.top_p < 1.0) || (mode == M_TOPK && masked_row));
  // (all-candidates rows emit every legal token: the finisher's own f64
  // sum over its working set is their row total, no chunk mass needed; a
  // keep-all row under race-v2 draws nothing here, the race kernel takes
  // its own mass)
  const bool mass64 = row_ok && nleg > 0 && mode == M_KEEPALL && !A.nodraw;
  uint32_t cnt_i[PER_MAX];
  double m0 = 0.0, m1 = 0.0;
  {
    // f32 weights 2^((l - m) * c2) with c2 = log2(e) / T; see the chunk
    // error bound below.  f64 weights (exp_neg) for the modes whose draw
    // walks the full row.
    const float c2 = (float)(invT * 1.4426950408889634);
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      cnt_i[i] = 0u;
      if (i < (int)A.per) {
        const uint32_t sbase = c0 + (uint32_t)i * SLICE;
        const bool full = !masked_row && min(c1, sbase + (uint32_t)SLICE) - sbase == (uint32_t)SLICE;
        const uint32_t qb = full ? 0xfu : (uint32_t)(lq >> (4 * i)) & 0xfu;
        if (emit && !minp_x) {
          // screen the slice on the quad maxima (legal tokens only) first
          uint32_t cnt = 0;
          if (__builtin_amdgcn_ballot_w64(qm[i] >= thr)) {
            if (full) {
#pragma unroll
              for (int e = 0; e < 4; ++e) cnt += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lv[i][e] >= thr));
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                cnt += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(((qb >> e) & 1u) && lv[i][e] >= thr));
            }
          }
          cnt_i[i] = cnt;
          if (lane() == 0) S.wcnt[i * NW + wave()] = cnt;
        }
        if (mass32) {
          float sw = 0.0f, ew = 0.0f;
          // (y is clamped at -200: a suppressed token's f32::MIN logit
          // would make it -inf, and its weight 0 times -y a NaN bound;
          // exp2f is 0 below -149 either way)
          if (full) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float y = vmax((lv[i][e] - m) * c2, -200.0f);
              const float w = __builtin_amdgcn_exp2f(y);
              sw += w;
              ew = __builtin_fmaf(w, -y, ew);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float y = vmax((lv[i][e] - m) * c2, -200.0f);
              const float w = __builtin_amdgcn_exp2f(y);
              const bool lg = (qb >> e) & 1u;
              sw += lg ? w : 0.0f;
              ew = lg ? __builtin_fmaf(w, -y, ew) : ew;
            }
          }
          m0 += (double)sw;
          m1 += (double)ew;
        } else if (mass64) {
          double sw = 0.0;
          if (masked_row) {
            // legal tokens are sparse: the wave's legal logits of the slice
            // are packed into its own 256-float stretch of the count table
            // (dead after pass 1) and weighted one per lane, instead of an
            // f64 weight per element position any lane holds
            float* cb = reinterpret_cast<float*>(S.t.ct) + wave() * 256u;
            uint32_t nb = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const bool lg = (qb >> e) & 1u;
              const uint64_t bm = __builtin_amdgcn_ballot_w64(lg);
              if (lg) cb[nb + lanes_below(bm)] = lv[i][e];
              nb += (uint32_t)__builtin_popcountll(bm);
            }
            wave_lds_sync();
            for (uint32_t k = lane(); k < nb; k += 64u)
              sw += exp_neg_t(((double)cb[k] - md) * invT, S.etab, S.etab + 64);
            wave_lds_sync();
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              sw += ((qb >> e) & 1u) ? exp_neg_t(((double)lv[i][e] - md) * invT, S.etab, S.etab + 64) : 0.0;
          }
          m0 += sw;
          if (mode == M_KEEPALL) {
            const double ws = wave_sum_f64(sw);
            if (lane() == 0) st_dev(&A.w.seg[(((uint64_t)row * MAXC + chunk) * PER_MAX + i) * NW + wave()], ws);
          }
        }
      } else if (lane() == 0 && emit) {
        S.wcnt[i * NW + wave()] = 0u;
      }
    }
    if (mass32 || mass64) {
      const double w0s = wave_sum_f64(m0), w1s = wave_sum_f64(m1);
      if (lane() == 0) { S.wq[wave()].m0 = w0s; S.wq[wave()].m1 = w1s; }
    }
  }
  if (minp_x) {
    // the largest chunk maximum of the row published by now
    if (tid == 0) {
      const unsigned long long cur = __hip_atomic_load(A.w.rowx + (uint64_t)row * ROWX_STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)(cur >> 32) == A.epoch) xkey = max(xkey, (uint32_t)cur);
      S.xkey = xkey;
    }
    lds_barrier();
    const float mx = okey_value(S.xkey);
    const double lim_d = (double)mx + c.T * log(c.min_p);
    thr = (float)lim_d - (fabsf((float)lim_d) + fabsf(mx)) * 1e-5f - 1e-30f;
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      cnt_i[i] = 0u;
      if (i < (int)A.per) {
        const uint32_t sbase = c0 + (uint32_t)i * SLICE;
        const bool full = !masked_row && min(c1, sbase + (uint32_t)SLICE) - sbase == (uint32_t)SLICE;
        const uint32_t qb = full ? 0xfu : (uint32_t)(lq >> (4 * i)) & 0xfu;
        uint32_t cnt = 0;
        if (__builtin_amdgcn_ballot_w64(qm[i] >= thr)) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            cnt += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(((qb >> e) & 1u) && lv[i][e] >= thr));
        }
        cnt_i[i] = cnt;
        if (lane() == 0) S.wcnt[i * NW + wave()] = cnt;
      } else if (lane() == 0) {
        S.wcnt[i * NW + wave()] = 0u;
      }
    }
  }
  stamp(A, row, chunk, 5);
  if (emit || mass32 || mass64) lds_barrier();
  if (mass32 || mass64) {
    double s0 = 0.0, s1 = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) { s0 += S.wq[w].m0; s1 += S.wq[w].m1; }
    mass = s0;
    if (mass32) {
      // |mass - sum of exact weights| <= 1.01 (2^-22 S + 3 2^-24 S) for the
      // f32 exp (2 ulp) and the 4-term f32 slice sums, + 1.01 ln2 3 2^-24
      // sum w |y| for the rounding of y (three f32 roundings, relative),
      // + n 2^-124 for weights below 2^-126, + 2^-40 S for the f64 sums.
      const double S0 = s0, E0 = s1;
      mass_err = 1.01 * (0x1p-22 * S0 + 3.0 * 0x1p-24 * S0 + 0.6931471805599453 * 3.0001 * 0x1p-24 * E0) +
                 (double)nleg * 0x1p-124 + 0x1p-40 * S0;
    }
  }
  if (emit) {
    // exclusive offsets in (slice, wave) order == token-ID order; every wave
    // scans the PER_MAX * NW counts itself (lane j holds j, j + 64, j + 128)
    const uint32_t nent = A.per * NW;
    const uint32_t v0 = lane() < nent ? S.wcnt[lane()] : 0u;
    const uint32_t v1 = lane() + 64u < nent ? S.wcnt[lane() + 64u] : 0u;
    const uint32_t v2 = lane() + 128u < nent ? S.wcnt[lane() + 128u] : 0u;
    const uint32_t i0 = wave_scan_u32(v0), i1 = wave_scan_u32(v1), i2 = wave_scan_u32(v2);
    const uint32_t t0 = (uint32_t)__builtin_amdgcn_readlane((int)i0, 63);
    const uint32_t t1s = (uint32_t)__builtin_amdgcn_readlane((int)i1, 63);
    const uint32_t t2s = (uint32_t)__builtin_amdgcn_readlane((int)i2, 63);
    ncand = t0 + t1s + t2s;
    const uint32_t x0 = i0 - v0, x1 = i1 - v1 + t0, x2 = i2 - v2 + t0 + t1s;
    const uint64_t cbase = rbase + c0;
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      if (i < (int)A.per && cnt_i[i]) {
        const uint32_t idx = (uint32_t)i * NW + wave();
        const uint32_t src = idx & 63u;
        const uint32_t reg = idx >> 6;
        const uint32_t xv = reg == 0 ? x0 : (reg == 1 ? x1 : x2);
        const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)xv, (int)src);
        const uint32_t sbase = c0 + (uint32_t)i * SLICE;
        const bool full = !masked_row && min(c1, sbase + (uint32_t)SLICE) - sbase == (uint32_t)SLICE;
        const uint32_t qb = full ? 0xfu : (uint32_t)(lq >> (4 * i)) & 0xfu;
        bool em[4];
        uint32_t before_me = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          em[e] = ((qb >> e) & 1u) && lv[i][e] >= thr;
          before_me += lanes_below(__builtin_amdgcn_ballot_w64(em[e]));
        }
        uint32_t off = base + before_me;
        const uint32_t e0 = sbase + tid * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (em[e]) {
            const uint64_t pos = cbase + off;
            st_dev(&A.w.cand_l[pos], lv[i][e]);
            st_dev(&A.w.cand_id[pos], e0 + (uint32_t)e);
            ++off;
          }
        }
      }
    }
  }

  // ---- publish the chunk's statistics (the row finisher kernel reads them)
  stamp(A, row, chunk, 7);
  if (tid == 0) {
    // the greedy argmax: the largest (value key, ~id) of the waves' argmaxes
    unsigned long long garg = 0ull;
    if (want_arg)
      for (int w = 0; w < NW; ++w) garg = garg > S.wp[w].arg ? garg : S.wp[w].arg;
    ChunkStat& st = A.w.stat[(uint64_t)row * MAXC + chunk];
    st_dev(&st.maxkey, nleg ? maxkey : 0u);
    st_dev(&st.gbest_id, garg ? ~(uint32_t)garg : NONE);
    st_dev(&st.gbest_val, garg ? okey_value((uint32_t)(garg >> 32)) : 0.0f);
    st_dev(&st.nlegal, nleg);
    st_dev(&st.ncand, ncand);
    st_dev(&st.flags, cflags);
    st_dev(&st.mass, mass);
    st_dev(&st.mass_err, mass_err);
    st_dev(&st.minkey, minkey);
    st_dev(&st.thr, thr);
  }
  stamp(A, row, chunk, 2);
  return rx ? RX_FULL : 0u;
}

// ---------------------------------------------------------------------------
// The chunk kernel.  Workgroup -> (row, chunk) as in the general body.  The
// row's parameters decide the body: rows the lean body covers issue the
// history ids and the stream there and run it, the others run the general
// body (which issues its own loads).
template <typename In, bool RX>
__global__ __launch_bounds__(NT) void sample_kernel(
    SampleArgs A, const double* __restrict__ p_temperature, const uint32_t* __restrict__ p_top_k,
    const double* __restrict__ p_top_p, const double* __restrict__ p_min_p, const float* __restrict__ p_rep,
    const float* __restrict__ p_pres, const float* __restrict__ p_freq, const double* __restrict__ p_uniform,
    const uint32_t* __restrict__ p_hoff, const uint32_t* __restrict__ p_boff) {
  __shared__ __align__(16) FusedSmem U;
  const mxs_batch& b = A.b;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= b.rows) return;
  stamp(A, row, chunk, 8);
  const uint32_t V = b.vocab;
  const uint32_t c0 = chunk * A.CH;
  const uint32_t c1 = min(V, c0 + A.CH);
  const RowCfg c = load_cfg(p_temperature, p_top_k, p_top_p, p_min_p, p_rep, p_pres, p_freq, p_uniform, p_hoff,
                            p_boff, row);
  const uint32_t mode = chunk_mode(c, V);
  // a step receipt for this row (mxs_step)
  const bool rx = RX && A.rx_want[row] != MXS_RECEIPT_NONE;
  uint32_t rxw;   // the receipt work left after the body
  {
    const uint32_t hn = c.he > c.hb ? c.he - c.hb : 0u, bn = c.be > c.bb ? c.be - c.bb : 0u;
    // A logit bias of at most NT entries, none above 0 (-inf suppresses),
    // never raises a logit: the lean body takes it (NaN and +inf values fail
    // the test, and the general body reports them).
    bool lean_bias = bn == 0u;
    if (bn && bn <= (uint32_t)NT && hn + bn <= (uint32_t)HCAP && !c.err && A.masked == 0u) {
      const float v = threadIdx.x < bn ? b.bias_values[c.bb + threadIdx.x] : 0.0f;
      lean_bias = __syncthreads_and(v <= 0.0f) != 0;
    }
    // (the lean body's penalties never raise a logit: others take the general body)
    if (!c.err && A.masked == 0u && lean_bias && hn <= (uint32_t)HCAP &&
        (hn == 0u || (c.rep >= 1.0f && c.freq >= 0.0f && c.pres >= 0.0f)) &&
        (mode == M_GREEDY || mode == M_TOPK || mode == M_MINP)) {
      stamp(A, row, chunk, 0);
      if (hn || bn) {
        if (mode == M_GREEDY) rxw = chunk_fast<In, M_GREEDY, true, RX>(A, U, c, row, chunk, c0, c1, hn, bn, rx);
        else if (mode == M_TOPK) rxw = chunk_fast<In, M_TOPK, true, RX>(A, U, c, row, chunk, c0, c1, hn, bn, rx);
        else rxw = chunk_fast<In, M_MINP, true, RX>(A, U, c, row, chunk, c0, c1, hn, bn, rx);
      } else {
        if (mode == M_GREEDY) rxw = chunk_fast<In, M_GREEDY, false, RX>(A, U, c, row, chunk, c0, c1, 0u, 0u, rx);
        else if (mode == M_TOPK) rxw = chunk_fast<In, M_TOPK, false, RX>(A, U, c, row, chunk, c0, c1, 0u, 0u, rx);
        else rxw = chunk_fast<In, M_MINP, false, RX>(A, U, c, row, chunk, c0, c1, 0u, 0u, rx);
      }
    } else {
      rxw = chunk_general<In>(A, U, c, row, chunk, rx);
    }
  }
  // The step receipt's reload paths run here, after the body, where its
  // registers are dead (inside a body they made the kernel spill), then the
  // row arrival.
  if (RX && rxw) {
    stamp(A, row, chunk, 10);
    ChunkSmem& S = chunk_smem(U);
    rx_supmap(A, S, c0, c1, c.bb, c.be > c.bb ? c.be - c.bb : 0u);
    const uint32_t* supw = S.t.ct;
    const In* src = reinterpret_cast<const In*>(b.logits) + (uint64_t)row * b.row_stride;
    // each pass reads the chunk again (just streamed: from the caches), its
    // slice loop rolled: held in registers across the passes, the chunk made
    // the kernel spill (the opaque pointer keeps the passes' loads apart)
    const auto getq = [&](int i, float* r, uint32_t& rb) {
      const uint32_t sbase = c0 + (uint32_t)i * SLICE, e0 = sbase + threadIdx.x * 4u;
      rb = sbase + (uint32_t)SLICE <= c1 ? 0xfu : (e0 < c1 ? (c1 - e0 >= 4u ? 0xfu : (1u << (c1 - e0)) - 1u) : 0u);
      const In* p = src;
      __asm__ volatile("" : "+s"(p));
      Quad<In>::unpack(Quad<In>::load(p + (e0 < c1 ? e0 : c0)), r);
      const uint32_t sb = supw[(uint32_t)i * ((uint32_t)SLICE / 32u) + (threadIdx.x >> 3)] >> ((threadIdx.x & 7u) * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((sb >> e) & 1u) r[e] = -FLT_MAX;
    };
    if (!receipt_chunk<1>(A, S, row, chunk, c0, c1, getq))
      receipt_exact(A, S, row, chunk, c0, min(A.rx_n, c1 - c0), getq);
    stamp(A, row, chunk, 11);
  }
  const bool last = arrive_row(A, chunk_smem(U), row);
  // The row finisher: one copy for every chunk body.  The finisher runs once
  // per row, mostly down code no other wave of the workgroup has run, so its
  // instruction fetches miss the instruction cache; one shared copy keeps the
  // kernel's code (and the lines every row's finisher fetches) small.
  if (!last) {
    stamp(A, row, chunk, 9);
    return;
  }
  stamp(A, row, MAXC, 0);
  FinLoads P;
  fin_issue(A, row, P);
  finish_row<In>(A, U.f, c, row, mode, (uint64_t)row * V, c.greedy ? 0.0 : 1.0 / c.T, P);
  stamp(A, row, MAXC, 7);
  if (RX && rx) {
    __syncthreads();   // the finisher's LDS is free
    stamp(A, row, MAXC, 10);
    receipt_finish<In>(A, U.f, row);
    stamp(A, row, MAXC, 11);
  }
  // The row's counter and exchange word are cleared for the next call here,
  // after the finisher: every chunk has arrived (its exchange update came
  // before), and stores issued at the arrival would hold the finisher's
  // first loads behind their completion (a wave's memory counter is in
  // order).
  if (threadIdx.x == 0) {
    st_dev(A.w.ctr + (uint64_t)row * CTR_STRIDE, 0u);
    st_dev(A.w.rowx + (uint64_t)row * ROWX_STRIDE, 0ull);
  }
  stamp(A, row, MAXC, 9);
}

size_t sample_lds_bytes() { return sizeof(FusedSmem); }

// A batch whose chunks would not fill the CUs streams each row with twice
// as many workgroups (half the quads per thread), while the doubled count
// stays within the register-slot finishers' FW chunks.
ChunkLayout sample_layout(uint32_t rows, uint32_t V) {
  ChunkLayout L = chunk_layout(V);
  if ((uint64_t)rows * L.C < 256u) {
    const ChunkLayout L2 = chunk_layout(V, (uint32_t)PER_MAX / 2u);
    if (L2.C <= (uint32_t)FW) L = L2;
  }
  return L;
}

}  // namespace mxs

// ===========================================================================
// Host side: context, validation, launch.
// ===========================================================================

namespace mxs {

int sample_launch(mxs_ctx* ctx, const mxs_batch* b, const mxs_out* o, bool nodraw, const mxs_receipts* rx) {
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
  A.timing = ctx->timing;
  A.paths = ctx->paths;
  if (++ctx->epoch == 0u) ctx->epoch = 1u;   // 0 is the zeroed scratch's tag
  A.epoch = ctx->epoch;
  A.nodraw = nodraw ? 1u : 0u;
  A.race_m = nodraw ? ctx->race_m : nullptr;
  A.masked = b->mask_words != nullptr;
  A.rx_want = nullptr;
  if (rx) {
    // step receipts in the same pass: a NULL top asks one of every row (the
    // zeros stand in); the per-chunk statistics and lists take the top-n
    // scratch, which is larger
    static_assert(sizeof(mxs::RxStat) == 24, "RxStat layout");
    A.rx_want = rx->top ? rx->top : ctx->d_zero_u32;
    A.rx_n = rx->n;
    A.rx_ids = rx->ids;
    A.rx_lps = rx->logprobs;
    A.rx_token_lp = rx->token_logprob;
    A.rx_status = rx->status;
    A.rx_stat = reinterpret_cast<mxs::RxStat*>(ctx->topn_scratch);
    A.rx_list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ctx->topn_scratch) +
                                                      (size_t)ctx->max_rows * mxs::MAXC * sizeof(mxs::RxStat));
    if ((size_t)ctx->max_rows * mxs::MAXC * (sizeof(mxs::RxStat) + (size_t)rx->n * 8u) > topn_scratch_bytes(ctx->max_rows))
      return fail(ctx, MXS_EINVAL, "receipt scratch too small");
  }
  if (!A.masked) {
    A.b.mask_words = ctx->d_mask_ones;
    A.b.mask_stride = 0;
    A.b.tokenizer_vocab = b->vocab;
  }
  if (!b->history_offsets) { A.b.history_offsets = ctx->d_zero_u32; A.b.history_ids = ctx->d_zero_u32; }
  if (!b->bias_offsets) { A.b.bias_offsets = ctx->d_zero_u32; A.b.bias_ids = ctx->d_zero_u32; A.b.bias_values = ctx->d_zero_f32; }
  const double* p_tp = b->top_p ? b->top_p : ctx->d_one_f64;
  const double* p_mp = b->min_p ? b->min_p : ctx->d_zero_f64;
  const double* p_u = b->uniform ? b->uniform : ctx->d_zero_f64;
  const uint32_t* p_k = b->top_k ? b->top_k : ctx->d_zero_u32;
  const float* p_rep = b->repetition ? b->repetition : ctx->d_one_f32;
  const float* p_pres = b->presence ? b->presence : ctx->d_zero_f32;
  const float* p_freq = b->frequency ? b->frequency : ctx->d_zero_f32;
  const mxs::ChunkLayout L = sample_layout(b->rows, b->vocab);
  const uint32_t C = L.C;
  A.C = L.C;
  A.CH = L.CH;
  A.per = L.per;
  if (A.per > (uint32_t)mxs::PER_MAX || C > (uint32_t)mxs::MAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  const dim3 grid(8u * C, (b->rows + 7u) / 8u);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  // One kernel: each row's last chunk to finish decides the row.
#define MXS_ARGS A, b->temperature, p_k, p_tp, p_mp, p_rep, p_pres, p_freq, p_u, A.b.history_offsets, A.b.bias_offsets
  // (step receipts: their own instantiation, so picks without receipts run
  // the kernel's code unchanged)
  if (b->dtype == MXS_F32) {
    if (A.rx_want) hipLaunchKernelGGL((mxs::sample_kernel<float, true>), grid, dim3(mxs::NT), 0, ctx->stream, MXS_ARGS);
    else hipLaunchKernelGGL((mxs::sample_kernel<float, false>), grid, dim3(mxs::NT), 0, ctx->stream, MXS_ARGS);
  } else {
    if (A.rx_want) hipLaunchKernelGGL((mxs::sample_kernel<uint16_t, true>), grid, dim3(mxs::NT), 0, ctx->stream, MXS_ARGS);
    else hipLaunchKernelGGL((mxs::sample_kernel<uint16_t, false>), grid, dim3(mxs::NT), 0, ctx->stream, MXS_ARGS);
  }
#undef MXS_ARGS
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    mask_note_read(ctx, b->mask_words);
    ctx->last_rows = b->rows;
    ctx->last_C = L.C;
    ctx->last_CH = L.CH;
    ctx->last_V = b->vocab;
  }
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "sample_kernel launch");
  return MXS_OK;
}

// ---------------------------------------------------------------------------
// Candidate export (mxs_export_candidates): row r's candidate list from the
// last mxs_sample / mxs_step call, chunk q's candidates at r V + q CH
// (ncand of them, token-ID order), copied out whole when at most `width`,
// else its top `width` by (logit desc, ID asc): a radix select of the
// width-th largest order key over four 8-bit digits, then every key above it
// and the lowest-ID ties at it.  Output in token-ID order.
__global__ __launch_bounds__(NT) void cand_export_kernel(Work w, uint32_t C, uint32_t CH, uint32_t V,
                                                         uint32_t width, int32_t* count, int32_t* ids,
                                                         float* logits) {
  __shared__ uint32_t coff[MAXC + 1];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t red[NW];
  __shared__ uint32_t s_u[2];
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const int32_t n0 = w.cand_rows[row];
  if (n0 < 0) {
    if (tid == 0) count[row] = -1;
    return;
  }
  if (tid < 64u) {   // chunk offsets (C <= MAXC = 64)
    const uint32_t nq = tid < C ? w.stat[(uint64_t)row * MAXC + tid].ncand : 0u;
    const uint32_t inc = wave_scan_u32(nq);
    if (tid < C) coff[tid] = inc - nq;
    const uint32_t tot = bcast63(inc);
    if (tid == 0) coff[C] = tot;
  }
  __syncthreads();
  const uint32_t n = min((uint32_t)n0, coff[C]);
  const uint64_t rbase = (uint64_t)row * V;
  // candidate j's position: the last chunk q < C with coff[q] <= j
  auto pos_of = [&](uint32_t j) -> uint64_t {
    uint32_t lo = 0, hi = C - 1u;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1u) >> 1;
      if (coff[mid] <= j) lo = mid; else hi = mid - 1u;
    }
    return rbase + (uint64_t)lo * CH + (j - coff[lo]);
  };
  int32_t* oi = ids + (uint64_t)row * width;
  float* ol = logits + (uint64_t)row * width;
  if (n <= width) {
    for (uint32_t j = tid; j < n; j += NT) {
      const uint64_t p = pos_of(j);
      oi[j] = (int32_t)ld_dev(&w.cand_id[p]);
      ol[j] = ld_dev(&w.cand_l[p]);
    }
    if (tid == 0) count[row] = (int32_t)n;
    return;
  }
  uint32_t prefix = 0u, need = width;   // the key's fixed high digits; members still to take at or below them
  for (int d = 3; d >= 0; --d) {
    if (tid < 256u) hist[tid] = 0u;
    __syncthreads();
    const uint32_t pm = d == 3 ? 0u : (0xffffffffu << (8 * (d + 1)));
    for (uint32_t j = tid; j < n; j += NT) {
      const uint32_t key = okey(ld_dev(&w.cand_l[pos_of(j)]));
      if ((key & pm) == prefix) atomicAdd(&hist[(key >> (8 * d)) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {   // the digit, from the top, where the count above reaches `need`
      uint32_t cum = 0u;
      int b = 255;
      for (; b > 0; --b) {
        if (cum + hist[b] >= need) break;
        cum += hist[b];
      }
      s_u[0] = (uint32_t)b;
      s_u[1] = cum;
    }
    __syncthreads();
    prefix |= s_u[0] << (8 * d);
    need -= s_u[1];
    __syncthreads();
  }
  // keys above `prefix` (width - need of them), then the first `need` ties in ID order
  uint32_t base = 0u, tbase = 0u;
  for (uint32_t j0 = 0; j0 < n; j0 += NT) {
    const uint32_t j = j0 + tid;
    uint32_t key = 0u, id = 0u;
    float l = 0.0f;
    if (j < n) {
      const uint64_t p = pos_of(j);
      l = ld_dev(&w.cand_l[p]);
      id = ld_dev(&w.cand_id[p]);
      key = okey(l);
    }
    const bool tie = j < n && key == prefix;
    uint32_t ttot;
    const uint32_t trank = tbase + block_scan_incl<uint32_t>(tie ? 1u : 0u, red, &ttot) - (tie ? 1u : 0u);
    const bool take = (j < n && key > prefix) || (tie && trank < need);
    uint32_t tot;
    const uint32_t at = base + block_scan_incl<uint32_t>(take ? 1u : 0u, red, &tot) - (take ? 1u : 0u);
    if (take && at < width) {
      oi[at] = (int32_t)id;
      ol[at] = l;
    }
    base += tot;
    tbase += ttot;
  }
  if (tid == 0) count[row] = (int32_t)min(base, width);
}

// ---------------------------------------------------------------------------
// Finish-only pick over a logits producer's tile statistics
// (mxs_finish_tiles; the producer's epilogue wrote them with mxs_epilogue.h):
// one workgroup per row builds the one-chunk statistics and candidate list
// the row finisher takes, reading the logits of only the tiles a top-k head
// can reach, then runs finish_row as the sample kernel's last chunk does.
//   - greedy: the argmax is the largest tile gkey (ties: lowest token);
//   - top-k: kappa = the k-th largest tile maximum (order keys).  A tile
//     holding a member of the head has its maximum at or above the head's
//     k-th value, which is at least kappa (the k largest tile maxima are k
//     distinct tokens' values), so the tokens at or above kappa of the tiles
//     whose maximum reaches kappa hold the head and every tie at its edge.
//     kappa is the candidate threshold, as a chunk's is in the sample kernel.
//     With k above the tile count the tile maxima bound nothing: the row is
//     histogrammed on the sample kernel's value grid (HB bins of HRANGE / HB
//     logits below the row maximum) and the candidates are the tokens in
//     the bins down to the one where the count reaches k (two reads of the
//     row instead of one; every bin above holds fewer than k tokens, so the
//     head and its edge ties are inside).
__global__ __launch_bounds__(NT) void tile_finish_kernel(SampleArgs A, const EpiTileStat* __restrict__ ts,
                                                         uint32_t ntiles, const double* __restrict__ p_temperature,
                                                         const uint32_t* __restrict__ p_top_k,
                                                         const double* __restrict__ p_top_p,
                                                         const double* __restrict__ p_min_p,
                                                         const double* __restrict__ p_uniform,
                                                         const float* __restrict__ p_one, const float* __restrict__ p_zero,
                                                         const uint32_t* __restrict__ p_zero_u) {
  __shared__ __align__(16) FusedSmem U;
  const mxs_batch& b = A.b;
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const uint32_t V = b.vocab;
  const RowCfg c = load_cfg(p_temperature, p_top_k, p_top_p, p_min_p, p_one, p_zero, p_zero, p_uniform, p_zero_u,
                            p_zero_u, row);
  const uint32_t mode = chunk_mode(c, V);
  if (!c.err && mode != M_GREEDY && mode != M_TOPK) {
    if (tid == 0) {
      A.o.token[row] = -1;
      A.o.status[row] = MXS_ROW_UNSUPPORTED_RULE;
      if (A.o.sampling_logprob) A.o.sampling_logprob[row] = 0.0;
      if (A.o.kept_count) A.o.kept_count[row] = 0u;
      A.w.cand_rows[row] = -1;
    }
    return;
  }
  // scratch in the finisher's LDS, before the finisher writes it
  uint32_t* tk = reinterpret_cast<uint32_t*>(&U);   // [1024] the tiles' maxima
  uint32_t* tl = tk + 1024;                         // [1024] candidate tiles, ascending
  uint32_t* hist = tl + 1024;                       // [256]
  uint32_t* red = hist + 256;                       // [NW]
  uint32_t* su = red + NW;                          // [4]
  stamp(A, row, 0, 8);
  const EpiTileStat* rs = ts + (uint64_t)row * ntiles;
  uint32_t tm = 0u, bad = 0u;
  for (uint32_t t = tid; t < ntiles; t += NT) {
    const EpiTileStat s = rs[t];
    tm = max(tm, s.tmax);
    bad |= s.bad;
    tk[t] = s.tmax;
  }
  tm = block_max<uint32_t>(tm, red);
  bad = block_max<uint32_t>(bad, red);
  uint32_t kappa = 0u, n = 0u, bstar = 0u, gid = NONE;
  bool hmode = false;   // k above the tile count: the value-grid histogram decides
  const uint64_t rbase = (uint64_t)row * V;
  const float Mrow = okey_value(tm);
  const float hscale = (float)HB / HRANGE;
  // the value grid: bin 0 holds the row maximum, HB - 1 everything more than
  // HRANGE below it (monotone non-increasing in the value)
  auto vbin = [&](float x) -> uint32_t {
    const float d = (Mrow - x) * hscale;
    return d < (float)(HB - 1) ? (uint32_t)d : (uint32_t)(HB - 1);
  };
  if (!c.err && !bad && (mode == M_TOPK || mode == M_GREEDY)) {
    const float* lg = reinterpret_cast<const float*>(b.logits) + (uint64_t)row * b.row_stride;
    uint32_t m;   // candidate tiles in tl[0 .. m), ascending
    if (mode == M_GREEDY) {
      // the tiles holding the row maximum, and their tokens equal to it
      // (-0.0 and +0.0 are adjacent order keys: a zero maximum takes both)
      kappa = Mrow == 0.0f ? okey(-0.0f) : tm;
      const bool ct = tid < ntiles && tk[tid] >= kappa;
      const uint32_t at = block_scan_incl<uint32_t>(ct ? 1u : 0u, red, &m) - (ct ? 1u : 0u);
      if (ct) tl[at] = tid;
      __syncthreads();
    } else if (c.k <= ntiles) {
      // kappa: a lower bound of the k-th largest tile maximum.  One pass
      // puts the tile maxima on the value grid below the row maximum (tl
      // holds the HB bins until the compaction below): the bin where their
      // count reaches k, less one bin for rounding, bounds the k-th from
      // below.  A k-th maximum beyond the grid takes the exact k-th by four
      // 8-bit digit passes instead.
      for (uint32_t i = tid; i < (uint32_t)HB; i += NT) tl[i] = 0u;
      __syncthreads();
      if (tid < ntiles) atomicAdd(&tl[vbin(okey_value(tk[tid]))], 1u);
      __syncthreads();
      if (wave() == 0) {   // lane j: bins 16 j .. 16 j + 15
        uint32_t hs = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) hs += tl[lane() * 16u + (uint32_t)i];
        const uint32_t inc = wave_scan_u32(hs);
        const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= c.k);   // k <= ntiles: some lane reaches it
        const uint32_t gi = (uint32_t)__builtin_ctzll(reach);
        const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - hs), (int)gi);
        const uint32_t hv = lane() < 16u ? tl[16u * gi + lane()] : 0u;
        const uint32_t vi = base + wave_scan_u32(hv);
        const uint32_t lb = (uint32_t)__builtin_ctzll(__builtin_amdgcn_ballot_w64(lane() < 16u && vi >= c.k));
        if (lane() == 0) su[3] = 16u * gi + lb;
      }
      __syncthreads();
      const uint32_t bk = su[3];
      if (bk + 2u < (uint32_t)HB) {
        kappa = okey(Mrow - (float)(bk + 2u) / hscale);
      } else {
        uint32_t prefix = 0u, need = c.k;
        for (int d = 3; d >= 0; --d) {
          if (tid < 256u) hist[tid] = 0u;
          __syncthreads();
          const uint32_t pm = d == 3 ? 0u : (0xffffffffu << (8 * (d + 1)));
          if (tid < ntiles && (tk[tid] & pm) == prefix) atomicAdd(&hist[(tk[tid] >> (8 * d)) & 255u], 1u);
          __syncthreads();
          if (wave() == 0) {   // lane l: bins 255 - 4l .. 252 - 4l, from the top
            uint32_t hb[4], hs = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) { hb[i] = hist[255u - 4u * lane() - (uint32_t)i]; hs += hb[i]; }
            const uint32_t inc = wave_scan_u32(hs);
            const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
            const uint32_t L = (uint32_t)__builtin_ctzll(reach);   // need <= the matching count: some lane reaches it
            if (lane() == L) {
              uint32_t cum = inc - hs;
              uint32_t bin = 252u - 4u * L;
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (cum + hb[i] >= need) { bin = 255u - 4u * L - (uint32_t)i; break; }
                cum += hb[i];
              }
              su[0] = bin;
              su[1] = cum;
            }
          }
          __syncthreads();
          prefix |= su[0] << (8 * d);
          need -= su[1];
          __syncthreads();
        }
        kappa = prefix;
      }
      const bool ct = tid < ntiles && tk[tid] >= kappa;
      const uint32_t at = block_scan_incl<uint32_t>(ct ? 1u : 0u, red, &m) - (ct ? 1u : 0u);
      if (ct) tl[at] = tid;
      __syncthreads();
    } else {
      // More heads than tiles: the tile maxima bound nothing, so the whole
      // row is histogrammed on the value grid (tk becomes the HB bins) and
      // the head is the bins down to the one where the count reaches k.
      hmode = true;
      m = ntiles;
      if (tid < ntiles) tl[tid] = tid;
      for (uint32_t i = tid; i < (uint32_t)HB; i += NT) tk[i] = 0u;
      __syncthreads();
      for (uint32_t v0 = tid * 16u; v0 < V; v0 += NT * 16u) {
        float4 xv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t v = v0 + 4u * (uint32_t)u;
          xv[u] = v < V ? *reinterpret_cast<const float4*>(lg + v) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float e4[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (v0 + 4u * (uint32_t)u + (uint32_t)e < V) atomicAdd(&tk[vbin(e4[e])], 1u);
        }
      }
      __syncthreads();
      if (wave() == 0) {   // lane j: bins 16 j .. 16 j + 15, from the top value down
        uint32_t hs = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) hs += tk[lane() * 16u + (uint32_t)i];
        const uint32_t inc = wave_scan_u32(hs);
        const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= c.k);
        uint32_t bs = (uint32_t)(HB - 1);
        if (reach) {
          const uint32_t gi = (uint32_t)__builtin_ctzll(reach);
          const uint32_t base = (uint32_t)__builtin_amdgcn_readlane((int)(inc - hs), (int)gi);
          const uint32_t hv = lane() < 16u ? tk[16u * gi + lane()] : 0u;
          const uint32_t vi = base + wave_scan_u32(hv);
          const uint64_t r2 = __builtin_amdgcn_ballot_w64(lane() < 16u && vi >= c.k);
          bs = 16u * gi + (uint32_t)__builtin_ctzll(r2);
        }
        if (lane() == 0) su[0] = bs;
      }
      __syncthreads();
      bstar = su[0];
    }
    stamp(A, row, 0, 1);
    // the candidate tiles' tokens in the head's range, in token-ID order:
    // 16 threads per tile, 16 consecutive tokens each, 64 tiles a pass
    for (uint32_t t0 = 0; t0 < m; t0 += NT / 16u) {
      const uint32_t ti = t0 + tid / 16u;
      const uint32_t v0 = ti < m ? tl[ti] * EPI_TILE + (tid % 16u) * 16u : V;
      float4 xv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t v = v0 + 4u * (uint32_t)u;
        xv[u] = v < V ? *reinterpret_cast<const float4*>(lg + v) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      uint32_t keep = 0u;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float e4[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t v = v0 + 4u * (uint32_t)u + (uint32_t)e;
          const bool in = v < V && (hmode ? vbin(e4[e]) <= bstar : okey(e4[e]) >= kappa);
          keep |= in ? 1u << (4 * u + e) : 0u;
        }
      }
      if (mode == M_GREEDY) {   // the argmax: the lowest ID holding the maximum, no list
        if (keep) gid = min(gid, v0 + (uint32_t)__builtin_ctz(keep));
        continue;
      }
      const uint32_t cnt = (uint32_t)__builtin_popcount(keep);
      uint32_t tot;
      uint32_t pos = n + block_scan_incl<uint32_t>(cnt, red, &tot) - cnt;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float e4[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((keep >> (4 * u + e)) & 1u) {
            st_dev(&A.w.cand_l[rbase + pos], e4[e]);
            st_dev(&A.w.cand_id[rbase + pos], v0 + 4u * (uint32_t)u + (uint32_t)e);
            ++pos;
          }
      }
      n += tot;
    }
    if (mode == M_GREEDY) gid = ~block_max<uint32_t>(~gid, red);
  }
  stamp(A, row, 0, 2);
  if (tid == 0) {
    ChunkStat* st = &A.w.stat[(uint64_t)row * MAXC];
    st_dev(&st->maxkey, tm);
    st_dev(&st->gbest_id, gid);
    st_dev(&st->gbest_val, Mrow == 0.0f ? 0.0f : Mrow);
    st_dev(&st->nlegal, V);
    st_dev(&st->ncand, n);
    st_dev(&st->flags, bad ? (uint32_t)F_NONFINITE : 0u);
    st_dev(&st->minkey, 0u);
    st_dev(&st->thr, hmode ? -INFINITY : okey_value(kappa));
    st_dev(&st->mass, 0.0);
    st_dev(&st->mass_err, 0.0);
  }
  wait_mem();
  __syncthreads();
  FinLoads P;
  fin_issue(A, row, P);
  finish_row<float>(A, U.f, c, row, mode, rbase, c.greedy ? 0.0 : 1.0 / c.T, P);
}

}  // namespace mxs

extern "C" {

int mxs_abi_version(void) { return MXS_ABI_VERSION; }

int mxs_finish_tiles(mxs_ctx* ctx, const mxs_batch* b, const void* tile_stats, const mxs_out* o) {
  using namespace mxs;
  if (!ctx || !b || !o) return MXS_EINVAL;
  if (b->rows == 0) return MXS_OK;
  if (!b->logits || !b->temperature || !tile_stats || !o->token || !o->status)
    return fail(ctx, MXS_EINVAL, "logits, temperature, tile_stats, token and status are required");
  if (b->rows > ctx->max_rows || b->vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  if (b->vocab == 0 || b->vocab > 1024u * EPI_TILE) return fail(ctx, MXS_EINVAL, "vocab must be in 1..262144");
  if (b->dtype != MXS_F32) return fail(ctx, MXS_EINVAL, "the finish-only pick reads f32 logits");
  if (b->row_stride < b->vocab || (b->row_stride & 3u)) return fail(ctx, MXS_EINVAL, "row_stride must be >= vocab and a multiple of 4");
  if (((uintptr_t)b->logits) % 16u) return fail(ctx, MXS_EINVAL, "logits must be 16-byte aligned");
  if (b->history_offsets || b->bias_offsets || b->mask_words || b->repetition || b->presence || b->frequency)
    return fail(ctx, MXS_EINVAL, "the finish-only pick takes no penalties, bias or mask");
  if (o->adjusted) return fail(ctx, MXS_EINVAL, "the finish-only pick writes no adjusted logits");
  SampleArgs A;
  A.b = *b;
  A.o = *o;
  A.w = ctx->work;
  A.timing = ctx->timing;
  A.paths = ctx->paths;
  if (++ctx->epoch == 0u) ctx->epoch = 1u;
  A.epoch = ctx->epoch;
  A.nodraw = 0u;
  A.race_m = nullptr;
  A.masked = 0u;
  A.rx_want = nullptr;
  A.b.mask_words = ctx->d_mask_ones;
  A.b.mask_stride = 0;
  A.b.tokenizer_vocab = b->vocab;
  A.b.history_offsets = ctx->d_zero_u32;
  A.b.history_ids = ctx->d_zero_u32;
  A.b.bias_offsets = ctx->d_zero_u32;
  A.b.bias_ids = ctx->d_zero_u32;
  A.b.bias_values = ctx->d_zero_f32;
  A.C = 1u;
  A.CH = b->vocab;
  A.per = 1u;
  const uint32_t ntiles = (b->vocab + EPI_TILE - 1u) / EPI_TILE;
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  hipLaunchKernelGGL(tile_finish_kernel, dim3(b->rows), dim3(NT), 0, ctx->stream, A,
                     reinterpret_cast<const EpiTileStat*>(tile_stats), ntiles, b->temperature,
                     b->top_k ? b->top_k : ctx->d_zero_u32, b->top_p ? b->top_p : ctx->d_one_f64,
                     b->min_p ? b->min_p : ctx->d_zero_f64, b->uniform ? b->uniform : ctx->d_zero_f64,
                     ctx->d_one_f32, ctx->d_zero_f32, ctx->d_zero_u32);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    ctx->last_rows = b->rows;
    ctx->last_C = 1u;
    ctx->last_CH = b->vocab;
    ctx->last_V = b->vocab;
  }
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "tile_finish_kernel launch");
  return MXS_OK;
}

int mxs_export_candidates(mxs_ctx* ctx, uint32_t rows, uint32_t width, int32_t* count, int32_t* ids,
                          float* logits) {
  using namespace mxs;
  if (!ctx) return MXS_EINVAL;
  if (rows == 0) return MXS_OK;
  if (!count || !ids || !logits || width == 0)
    return fail(ctx, MXS_EINVAL, "count, ids and logits are required and width must be positive");
  if (ctx->last_rows == 0) return fail(ctx, MXS_EINVAL, "no mxs_sample or mxs_step call on this context yet");
  if (rows > ctx->last_rows) return fail(ctx, MXS_EINVAL, "rows exceeds the last call's batch");
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  hipLaunchKernelGGL(cand_export_kernel, dim3(rows), dim3(NT), 0, ctx->stream, ctx->work, ctx->last_C,
                     ctx->last_CH, ctx->last_V, width, count, ids, logits);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "cand_export_kernel launch");
  return MXS_OK;
}

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
    case MXS_ROW_INVALID_HISTORY: return "history token IDs must be below the vocabulary";
    case MXS_ROW_INVALID_BIAS: return "logit bias IDs must be strictly increasing, below the vocabulary, with finite values (or -inf: suppressed)";
    case MXS_ROW_TOKEN_OUT_OF_RANGE: return "drafted token outside the vocabulary";
    case MXS_ROW_PROBABILITIES: return "invalid probability vectors";
    case MXS_ROW_UNSUPPORTED_RULE: return "the finish-only pick serves greedy and top-k (k <= 4096) rows";
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
  e = e ? e : hipMalloc(&ctx->work.ctr, (size_t)max_rows * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->work.rowx, (size_t)max_rows * mxs::ROWX_STRIDE * sizeof(unsigned long long));
  e = e ? e : hipMalloc(&ctx->work.stat, (size_t)max_rows * mxs::MAXC * sizeof(mxs::ChunkStat));
  e = e ? e : hipMalloc(&ctx->work.cand_l, rv * sizeof(float));
  e = e ? e : hipMalloc(&ctx->work.cand_id, rv * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->work.seg, (size_t)max_rows * mxs::MAXC * mxs::PER_MAX * mxs::NW * sizeof(double));
  e = e ? e : hipMalloc(&ctx->work.cand_rows, (size_t)max_rows * sizeof(int32_t));
  e = e ? e : hipMemset(ctx->work.cand_rows, 0xff, (size_t)max_rows * sizeof(int32_t));
  e = e ? e : hipMemset(ctx->work.rowx, 0, (size_t)max_rows * mxs::ROWX_STRIDE * sizeof(unsigned long long));
  e = e ? e : hipMemset(ctx->work.ctr, 0, (size_t)max_rows * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->topn_scratch, mxs::topn_scratch_bytes(max_rows));
  e = e ? e : hipMalloc(&ctx->spec_ctr, (size_t)max_rows * mxs::SPEC_COUNTERS_PER_ROW * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMemset(ctx->spec_ctr, 0, (size_t)max_rows * mxs::SPEC_COUNTERS_PER_ROW * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->spec_scratch, mxs::spec_scratch_bytes(max_rows, max_vocab));
  e = e ? e : hipMalloc(&ctx->race_ctr, (size_t)max_rows * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMemset(ctx->race_ctr, 0, (size_t)max_rows * mxs::CTR_STRIDE * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->race_scratch, mxs::race_scratch_bytes(max_rows, max_vocab));
  e = e ? e : hipMalloc(&ctx->race_kept, (size_t)max_rows * ((max_vocab + 31u) / 32u) * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->race_m, (size_t)max_rows * sizeof(float));
  const size_t nr = (size_t)max_rows + 1, nwords = (size_t)max_vocab / 32 + 2;
  e = e ? e : hipMalloc(&ctx->d_zero_u32, nr * sizeof(uint32_t));
  e = e ? e : hipMalloc(&ctx->d_one_f64, nr * sizeof(double));
  e = e ? e : hipMalloc(&ctx->d_race_u, nr * sizeof(double));
  e = e ? e : hipMalloc(&ctx->d_zero_f64, nr * sizeof(double));
  e = e ? e : hipMalloc(&ctx->d_one_f32, nr * sizeof(float));
  e = e ? e : hipMalloc(&ctx->d_zero_f32, nr * sizeof(float));
  e = e ? e : hipMalloc(&ctx->d_mask_ones, nwords * sizeof(uint32_t));
  if (e == hipSuccess) {
    std::vector<double> one64(nr, 1.0);
    std::vector<float> one32(nr, 1.0f);
    e = hipMemset(ctx->d_zero_u32, 0, nr * sizeof(uint32_t));
    e = e ? e : hipMemset(ctx->d_zero_f64, 0, nr * sizeof(double));
    e = e ? e : hipMemset(ctx->d_zero_f32, 0, nr * sizeof(float));
    e = e ? e : hipMemset(ctx->d_mask_ones, 0xff, nwords * sizeof(uint32_t));
    e = e ? e : hipMemcpy(ctx->d_one_f64, one64.data(), nr * sizeof(double), hipMemcpyHostToDevice);
    e = e ? e : hipMemcpy(ctx->d_one_f32, one32.data(), nr * sizeof(float), hipMemcpyHostToDevice);
    const std::vector<double> race_u(nr, mxs::RACE_DRAW_UNIFORM);
    e = e ? e : hipMemcpy(ctx->d_race_u, race_u.data(), nr * sizeof(double), hipMemcpyHostToDevice);
  }
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
  hipFree(ctx->work.rowx);
  hipFree(ctx->work.stat);
  hipFree(ctx->work.cand_l);
  hipFree(ctx->work.cand_id);
  hipFree(ctx->work.seg);
  hipFree(ctx->work.cand_rows);
  hipFree(ctx->d_zero_u32);
  hipFree(ctx->d_one_f64);
  hipFree(ctx->d_race_u);
  hipFree(ctx->d_zero_f64);
  hipFree(ctx->d_one_f32);
  hipFree(ctx->d_zero_f32);
  hipFree(ctx->d_mask_ones);
  hipFree(ctx->topn_scratch);
  hipFree(ctx->spec_ctr);
  hipFree(ctx->spec_scratch);
  hipFree(ctx->race_ctr);
  hipFree(ctx->race_scratch);
  hipFree(ctx->race_kept);
  hipFree(ctx->race_m);
  mxs::mask_release(ctx);
  hipSetDevice(prev);
  delete ctx;
  return MXS_OK;
}

int mxs_set_stream(mxs_ctx* ctx, void* stream) {
  if (!ctx) return MXS_EINVAL;
  ctx->stream = (hipStream_t)stream;
  return MXS_OK;
}

int mxs_debug_set_paths(mxs_ctx* ctx, void* device_buffer) {
  if (!ctx) return MXS_EINVAL;
  ctx->paths = (int32_t*)device_buffer;
  return MXS_OK;
}

int mxs_debug_set_timing(mxs_ctx* ctx, void* device_buffer) {
  if (!ctx) return MXS_EINVAL;
  ctx->timing = (uint64_t*)device_buffer;
  return MXS_OK;
}

int mxs_sync(mxs_ctx* ctx) {
  if (!ctx) return MXS_EINVAL;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamSynchronize");
  return MXS_OK;
}

const char* mxs_last_error(const mxs_ctx* ctx) {
  if (ctx) return ctx->last_error.c_str();
  const char* m = mxs::noalloc_last_error();   // the context-free entry point's
  return m ? m : "null context";
}

int mxs_sample(mxs_ctx* ctx, const mxs_batch* b, const mxs_out* o) { return mxs::sample_launch(ctx, b, o, false); }

}  // extern "C"
