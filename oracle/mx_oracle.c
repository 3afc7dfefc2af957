/* mx_oracle.c -- CPU restatement of the metallix token-sampler path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); see
 * mx_oracle.h.  Compile with -O2 -ffp-contract=off and without fast-math so
 * every f64 operation rounds as the Rust reference's does.
 *
 * Pins (what checks each function besides this restatement):
 *   orc_unit_uniform, orc_chacha8_*    -> GOLDEN_ICDF_V1 (qwen_forward.rs:1852-1876),
 *                                          uniform bit tests (qwen_forward.rs:2107-2135)
 *   orc_sample_categorical             -> sampling.rs:160-379 cases and error matrix
 *   orc_nucleus_mask                   -> kept-set table (qwen_forward.rs:2491-2518), brute force
 *   orc_greedy_token/orc_masked_argmax -> tie tests (qwen_forward.rs:1774-1795), brute force
 *   orc_token_logprob_top              -> analytic logsumexp cases, brute force sort
 *   orc_accept_or_resample             -> speculative/tests.rs:579-605, exact-law check
 *   orc_philox4x32_10, race            -> Random123 KATs, noise vectors, race-v2 golden tokens
 *                                          (race.rs:221-289)
 *   BUILD-DEFINED stages               -> closed forms (identity parameters, single-token
 *                                          histories, min_p 0/1, single legal id)
 */
#include "mx_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* f32 total order, as Rust's f32::total_cmp.                               */
static inline int32_t total_key(float x) {
  int32_t b;
  memcpy(&b, &x, 4);
  b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
  return b;
}

/* Descending total order, ascending index on ties: the `descending`
 * comparator of nucleus_mask (qwen_forward.rs:501-505) and of token_logprob
 * (chat_turn.rs:527-531). Returns nonzero when a sorts strictly before b. */
static inline int before(const float* x, uint32_t a, uint32_t b) {
  int32_t ka = total_key(x[a]), kb = total_key(x[b]);
  return ka > kb || (ka == kb && a < b);
}

static void insertion_sort(const float* x, uint32_t* v, size_t n) {
  for (size_t i = 1; i < n; ++i) {
    uint32_t t = v[i];
    size_t j = i;
    while (j > 0 && before(x, t, v[j - 1])) {
      v[j] = v[j - 1];
      --j;
    }
    v[j] = t;
  }
}

static void sift_down(const float* x, uint32_t* v, size_t n, size_t i) {
  for (;;) {
    size_t c = 2 * i + 1;
    if (c >= n) return;
    if (c + 1 < n && before(x, v[c], v[c + 1])) ++c;  /* max-heap of "later" elements */
    if (!before(x, v[i], v[c])) return;
    uint32_t t = v[i]; v[i] = v[c]; v[c] = t;
    i = c;
  }
}

static void heap_sort(const float* x, uint32_t* v, size_t n) {
  for (size_t i = n / 2; i-- > 0;) sift_down(x, v, n, i);
  for (size_t e = n; e-- > 1;) {
    uint32_t t = v[0]; v[0] = v[e]; v[e] = t;
    sift_down(x, v, e, 0);
  }
}

static size_t partition(const float* x, uint32_t* v, size_t n) {
  /* median of three as pivot, moved to v[0] */
  size_t m = n / 2;
  if (before(x, v[m], v[0])) { uint32_t t = v[m]; v[m] = v[0]; v[0] = t; }
  if (before(x, v[n - 1], v[0])) { uint32_t t = v[n - 1]; v[n - 1] = v[0]; v[0] = t; }
  if (before(x, v[n - 1], v[m])) { uint32_t t = v[n - 1]; v[n - 1] = v[m]; v[m] = t; }
  { uint32_t t = v[m]; v[m] = v[0]; v[0] = t; }
  uint32_t p = v[0];
  size_t i = 1, j = n - 1;
  for (;;) {
    while (i <= j && before(x, v[i], p)) ++i;
    while (j >= i && before(x, p, v[j])) --j;
    if (i >= j) break;
    uint32_t t = v[i]; v[i] = v[j]; v[j] = t;
    ++i; --j;
  }
  uint32_t t = v[j]; v[j] = v[0]; v[0] = t;
  return j;
}

static void intro_sort(const float* x, uint32_t* v, size_t n, int depth) {
  while (n > 16) {
    if (depth-- == 0) { heap_sort(x, v, n); return; }
    size_t p = partition(x, v, n);
    if (p < n - p) { intro_sort(x, v, p, depth); v += p + 1; n -= p + 1; }
    else { intro_sort(x, v + p + 1, n - p - 1, depth); n = p; }
  }
  insertion_sort(x, v, n);
}

/* sort_unstable_by(descending) */
static void sort_desc(const float* x, uint32_t* v, size_t n) {
  int depth = 2;
  for (size_t m = n; m > 1; m >>= 1) depth += 2;
  intro_sort(x, v, n, depth);
}

/* select_nth_unstable_by(nth, descending): afterwards v[0..nth) all sort
 * before v[nth]. */
static void select_nth_desc(const float* x, uint32_t* v, size_t n, size_t nth) {
  size_t lo = 0, hi = n;
  while (hi - lo > 16) {
    size_t p = lo + partition(x, v + lo, hi - lo);
    if (p == nth) return;
    if (p < nth) lo = p + 1; else hi = p;
  }
  insertion_sort(x, v + lo, hi - lo);
}

/* ------------------------------------------------------------------------ */
/* unit_uniform (qwen_forward.rs:551-559): top 53 bits of a u64 divided by
 * 2^53, split as 32 + 21 bits so every step is exact. */
double orc_unit_uniform(uint64_t word) {
  const double two_to_21 = 2097152.0;
  const double two_to_53 = 9007199254740992.0;
  uint64_t top53 = word >> 11;
  uint32_t high = (uint32_t)(top53 >> 21);
  uint32_t low = (uint32_t)(top53 & ((1u << 21) - 1));
  return ((double)high * two_to_21 + (double)low) / two_to_53;
}

/* ChaCha8Rng::seed_from_u64 (rand_chacha 0.9.0 over rand_core 0.9.3, pinned in
 * the reference's Cargo.lock): the u64 seed is expanded to the 32-byte key by
 * rand_core's PCG32 step (multiplier 6364136223846793005, increment
 * 11634580027462260723, XSH-RR output), block counter and stream start at
 * zero.  Restated from the published algorithms; pinned by GOLDEN_ICDF_V1. */
void orc_chacha8_seed_from_u64(orc_chacha8* rng, uint64_t state) {
  const uint64_t mul = 6364136223846793005ULL;
  const uint64_t inc = 11634580027462260723ULL;
  for (int i = 0; i < 8; ++i) {
    state = state * mul + inc;
    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    rng->key[i] = (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
  }
  rng->counter = 0;
  rng->index = 64;
}

static inline uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

static void chacha8_block(const uint32_t key[8], uint64_t counter, uint32_t out[16]) {
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                    key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                    (uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
  uint32_t w[16];
  memcpy(w, s, sizeof w);
#define QR(a, b, c, d)                 \
  w[a] += w[b]; w[d] ^= w[a]; w[d] = rotl32(w[d], 16); \
  w[c] += w[d]; w[b] ^= w[c]; w[b] = rotl32(w[b], 12); \
  w[a] += w[b]; w[d] ^= w[a]; w[d] = rotl32(w[d], 8);  \
  w[c] += w[d]; w[b] ^= w[c]; w[b] = rotl32(w[b], 7);
  for (int r = 0; r < 4; ++r) {
    QR(0, 4, 8, 12) QR(1, 5, 9, 13) QR(2, 6, 10, 14) QR(3, 7, 11, 15)
    QR(0, 5, 10, 15) QR(1, 6, 11, 12) QR(2, 7, 8, 13) QR(3, 4, 9, 14)
  }
#undef QR
  for (int i = 0; i < 16; ++i) out[i] = w[i] + s[i];
}

/* BlockRng::next_u64 over a 64-word buffer of four consecutive blocks: two
 * consecutive words, low word first. */
uint64_t orc_chacha8_next_u64(orc_chacha8* rng) {
  if (rng->index >= 63) {
    if (rng->index == 63) {
      uint32_t lo = rng->buf[63];
      for (int b = 0; b < 4; ++b) chacha8_block(rng->key, rng->counter + (uint64_t)b, rng->buf + 16 * b);
      rng->counter += 4;
      rng->index = 1;
      return ((uint64_t)rng->buf[0] << 32) | lo;
    }
    for (int b = 0; b < 4; ++b) chacha8_block(rng->key, rng->counter + (uint64_t)b, rng->buf + 16 * b);
    rng->counter += 4;
    rng->index = 0;
  }
  uint64_t v = ((uint64_t)rng->buf[rng->index + 1] << 32) | rng->buf[rng->index];
  rng->index += 2;
  return v;
}

/* ------------------------------------------------------------------------ */
/* sample_categorical (crates/core/engine/src/sampling.rs:56-103) with
 * check_row (:106-120), legal_shifted_sum (:122-149), shifted_logit
 * (:151-158).  `legal` may be NULL (every row legal). */
static inline int shifted_logit(float logit, double maximum, double temperature, double* out) {
  double s = ((double)logit - maximum) / temperature;
  if (!isfinite(s)) return ORC_INVALID_TEMPERATURE;
  *out = s;
  return ORC_OK;
}

int orc_sample_categorical(const float* logits, const uint8_t* legal, size_t n, double temperature,
                           double uniform, uint32_t* token, double* sampling_logprob) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  if (n > UINT32_MAX) return ORC_VOCABULARY_TOO_LARGE;
  if (!isfinite(temperature) || temperature <= 0.0) return ORC_INVALID_TEMPERATURE;
  if (!isfinite(uniform) || !(uniform >= 0.0 && uniform < 1.0)) return ORC_INVALID_UNIFORM;
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(logits[i])) return ORC_NON_FINITE_LOGIT;
  /* legal_shifted_sum */
  double maximum = -INFINITY;
  int has = 0;
  for (size_t i = 0; i < n; ++i) {
    if (legal && !legal[i]) continue;
    maximum = fmax(maximum, (double)logits[i]);
    has = 1;
  }
  if (!has) return ORC_EMPTY_SUPPORT;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    if (legal && !legal[i]) continue;
    double s;
    int st = shifted_logit(logits[i], maximum, temperature, &s);
    if (st) return st;
    sum += exp(s);
  }
  double log_normalizer = log(sum);
  double target = uniform * sum;
  double cumulative = 0.0;
  int have_final = 0;
  uint32_t final_token = 0;
  double final_shifted = 0.0;
  for (size_t i = 0; i < n; ++i) {
    if (legal && !legal[i]) continue;
    double s;
    int st = shifted_logit(logits[i], maximum, temperature, &s);
    if (st) return st;
    double w = exp(s);
    cumulative += w;
    if (w > 0.0) { have_final = 1; final_token = (uint32_t)i; final_shifted = s; }
    if (target < cumulative) {
      *token = (uint32_t)i;
      *sampling_logprob = s - log_normalizer;
      return ORC_OK;
    }
  }
  if (!have_final) return ORC_EMPTY_SUPPORT;
  *token = final_token;
  *sampling_logprob = final_shifted - log_normalizer;
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* nucleus_mask (crates/app/cli/src/qwen_forward.rs:474-549).  top_k == 0
 * stands for None.  The full-row `total` is computed on every path, as the
 * reference does, so the CPU baseline carries the reference's cost. */
int orc_nucleus_mask(const float* logits, size_t n, double temperature, double top_p, size_t top_k,
                     uint8_t* mask) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  int valid = top_p > 0.0 && top_p <= 1.0 && temperature > 0.0 && isfinite(temperature);
  if (!valid) return (top_p > 0.0 && top_p <= 1.0) ? ORC_INVALID_TEMPERATURE : ORC_INVALID_TOP_P;
  size_t k = (top_k > 0 && top_k < n) ? top_k : 0;
  int keep_all = top_p >= 1.0 && k == 0;
  memset(mask, keep_all ? 1 : 0, n);
  if (keep_all) return ORC_OK;
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(logits[i])) return ORC_NON_FINITE_LOGIT;
  float mf = -INFINITY;
  for (size_t i = 0; i < n; ++i) mf = fmaxf(mf, logits[i]);
  const double maximum = (double)mf;
#define WEIGHT(l) exp(((double)(l) - maximum) / temperature)
  double total = 0.0;
  for (size_t i = 0; i < n; ++i) total += WEIGHT(logits[i]);
  const double target = top_p * total;
  uint32_t* order = (uint32_t*)malloc(n * sizeof(uint32_t));
  if (!order) abort();
  if (k) {
    for (size_t i = 0; i < n; ++i) order[i] = (uint32_t)i;
    select_nth_desc(logits, order, n, k - 1);
    sort_desc(logits, order, k);
    double kept = 0.0;
    for (size_t j = 0; j < k; ++j) kept += WEIGHT(logits[order[j]]);
    double covered = 0.0;
    for (size_t j = 0; j < k; ++j) {
      mask[order[j]] = 1;
      covered += WEIGHT(logits[order[j]]);
      if (covered >= top_p * kept) break;
    }
    free(order);
    return ORC_OK;
  }
  size_t m = 0;
  for (size_t i = 0; i < n; ++i)
    if (WEIGHT(logits[i]) >= total * 1e-9) order[m++] = (uint32_t)i;
  sort_desc(logits, order, m);
  double covered = 0.0;
  for (size_t j = 0; j < m; ++j) {
    mask[order[j]] = 1;
    covered += WEIGHT(logits[order[j]]);
    if (covered >= target) { free(order); return ORC_OK; }
  }
  for (size_t i = 0; i < n; ++i) order[i] = (uint32_t)i;
  sort_desc(logits, order, n);
  memset(mask, 0, n);
  covered = 0.0;
  for (size_t j = 0; j < n; ++j) {
    mask[order[j]] = 1;
    covered += WEIGHT(logits[order[j]]);
    if (covered >= target) break;
  }
#undef WEIGHT
  free(order);
  return ORC_OK;
}

/* greedy_token (crates/app/cli/src/chat_generation.rs:2213-2231): IEEE `>`,
 * first index wins, every value must be finite. */
int orc_greedy_token(const float* logits, size_t n, int32_t* token) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  if (!isfinite(logits[0])) return ORC_NON_FINITE_LOGIT;
  size_t best = 0;
  for (size_t i = 1; i < n; ++i) {
    if (!isfinite(logits[i])) return ORC_NON_FINITE_LOGIT;
    if (logits[i] > logits[best]) best = i;
  }
  if (best > INT32_MAX) return ORC_VOCABULARY_TOO_LARGE;
  *token = (int32_t)best;
  return ORC_OK;
}

/* masked_argmax (crates/core/engine/src/constraint.rs:895-932): the best
 * mask-legal logit below `width`, lowest ID on ties (-0.0 ties 0.0).
 * *index = -1 when no legal token exists. */
int orc_masked_argmax(const uint32_t* words, size_t nwords, const float* logits, size_t width,
                      int64_t* index) {
  int have = 0;
  size_t best_i = 0;
  float best_v = 0.0f;
  for (size_t w = 0; w < nwords; ++w) {
    size_t base = w * 32;
    if (base >= width) break;
    uint32_t bits = words[w];
    if (bits == 0) continue;
    if (bits == UINT32_MAX && base + 32 <= width) {
      float mx = -INFINITY;
      for (int j = 0; j < 32; ++j) mx = fmaxf(mx, logits[base + j]);
      if (!have || mx > best_v) {
        int off = -1;
        for (int j = 0; j < 32; ++j)
          if (logits[base + j] == mx) { off = j; break; }
        if (off < 0) { *index = -1; return ORC_OK; }
        have = 1; best_i = base + (size_t)off; best_v = mx;
      }
      continue;
    }
    while (bits) {
      size_t i = base + (size_t)__builtin_ctz(bits);
      bits &= bits - 1;
      if (i >= width) break;
      if (!have || logits[i] > best_v) { have = 1; best_i = i; best_v = logits[i]; }
    }
  }
  *index = have ? (int64_t)best_i : -1;
  return ORC_OK;
}

/* fill_legal_mask (constraint.rs:793-806): bit b of word w <-> token 32w+b,
 * tokens at or past the tokenizer vocabulary are never legal. */
void orc_fill_legal_mask(const uint32_t* words, size_t nwords, size_t tokenizer_vocab, uint8_t* legal,
                         size_t n) {
  memset(legal, 0, n);
  for (size_t w = 0; w < nwords; ++w) {
    uint32_t bits = words[w];
    while (bits) {
      size_t i = w * 32 + (size_t)__builtin_ctz(bits);
      bits &= bits - 1;
      if (i >= tokenizer_vocab) return;
      if (i < n) legal[i] = 1;
    }
  }
}

/* selected_model_logprob (qwen_forward.rs:1577-1594). */
int orc_selected_model_logprob(const float* logits, size_t n, uint32_t token, double* logprob) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(logits[i])) return ORC_NON_FINITE_LOGIT;
  if (token >= n) return ORC_TOKEN_OUT_OF_RANGE;
  double maximum = -INFINITY;
  for (size_t i = 0; i < n; ++i) maximum = fmax(maximum, (double)logits[i]);
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) sum += exp((double)logits[i] - maximum);
  *logprob = (double)logits[token] - maximum - log(sum);
  return ORC_OK;
}

/* token_logprob (crates/app/cli/src/chat_turn.rs:506-563) without the
 * tokenizer spelling filter: the `top` most likely IDs by (total_cmp desc,
 * ID asc) and their f64 log-softmax values.  The reference over-selects
 * top + 8 to skip unspellable IDs; a caller asks for top + 8 here and
 * filters. */
int orc_token_logprob_top(const float* logits, size_t n, size_t top, int32_t* ids, double* logprobs,
                          double* maximum_out, double* log_normalizer_out) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  double maximum = -INFINITY;
  for (size_t i = 0; i < n; ++i) maximum = fmax(maximum, (double)logits[i]);
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) sum += exp((double)logits[i] - maximum);
  double log_normalizer = log(sum);
  size_t head = top < n ? top : n;
  uint32_t* order = (uint32_t*)malloc(n * sizeof(uint32_t));
  if (!order) abort();
  for (size_t i = 0; i < n; ++i) order[i] = (uint32_t)i;
  if (head < n) select_nth_desc(logits, order, n, head);
  sort_desc(logits, order, head);
  for (size_t j = 0; j < head; ++j) {
    ids[j] = (int32_t)order[j];
    logprobs[j] = (double)logits[order[j]] - maximum - log_normalizer;
  }
  free(order);
  if (maximum_out) *maximum_out = maximum;
  if (log_normalizer_out) *log_normalizer_out = log_normalizer;
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* accept_or_resample (crates/core/engine/src/speculative.rs:369-429) and
 * categorical (:431-444). *accepted = 1, or 0 with *resampled set. */
static int categorical_f64(const double* weights, size_t n, double threshold, size_t* index) {
  double cumulative = 0.0;
  int have = 0;
  size_t last = 0;
  for (size_t i = 0; i < n; ++i) {
    if (weights[i] > 0.0) { have = 1; last = i; }
    cumulative += weights[i];
    if (threshold < cumulative) { *index = i; return ORC_OK; }
  }
  if (!have) return ORC_PROBABILITIES;
  *index = last;
  return ORC_OK;
}

int orc_accept_or_resample(const double* target, const double* draft, size_t n, size_t drafted,
                           double accept_uniform, double resample_uniform, int* accepted,
                           size_t* resampled) {
  double tsum = 0.0, dsum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    if (!isfinite(target[i]) || !(target[i] >= 0.0)) return ORC_PROBABILITIES;
    tsum += target[i];
  }
  if (!(tsum > 0.0)) return ORC_PROBABILITIES;
  for (size_t i = 0; i < n; ++i) {
    if (!isfinite(draft[i]) || !(draft[i] >= 0.0)) return ORC_PROBABILITIES;
    dsum += draft[i];
  }
  if (!(dsum > 0.0)) return ORC_PROBABILITIES;
  double us[2] = {accept_uniform, resample_uniform};
  for (int j = 0; j < 2; ++j)
    if (!isfinite(us[j]) || !(us[j] >= 0.0 && us[j] < 1.0)) return ORC_INVALID_UNIFORM;
  double target_total = 0.0, draft_total = 0.0;
  for (size_t i = 0; i < n; ++i) target_total += target[i];
  for (size_t i = 0; i < n; ++i) draft_total += draft[i];
  if (drafted >= n) return ORC_TOKEN_OUT_OF_RANGE;
  double p = target[drafted] / target_total, q = draft[drafted] / draft_total;
  if (q <= 0.0) return ORC_PROBABILITIES;
  if (accept_uniform < p / q) { *accepted = 1; return ORC_OK; }
  *accepted = 0;
#define RESIDUAL(i) fmax(target[i] / target_total - draft[i] / draft_total, 0.0)
  double mass = 0.0;
  for (size_t i = 0; i < n; ++i) mass += RESIDUAL(i);
  if (mass <= 0.0) return categorical_f64(target, n, resample_uniform * target_total, resampled);
  double threshold = resample_uniform * mass;
  double cumulative = 0.0;
  int have = 0;
  size_t last = 0;
  for (size_t i = 0; i < n; ++i) {
    double w = RESIDUAL(i);
    if (w > 0.0) { have = 1; last = i; }
    cumulative += w;
    if (threshold < cumulative) { *resampled = i; return ORC_OK; }
  }
#undef RESIDUAL
  if (!have) return ORC_PROBABILITIES;
  *resampled = last;
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* race-v2 (crates/core/engine/src/sampling/race.rs:21-151). */
void orc_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
  const uint32_t m0 = 0xD2511F53u, m1 = 0xCD9E8D57u, w0 = 0x9E3779B9u, w1 = 0xBB67AE85u;
  uint32_t c0 = counter[0], c1 = counter[1], c2 = counter[2], c3 = counter[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int round = 0; round < 10; ++round) {
    if (round > 0) { k0 += w0; k1 += w1; }
    uint64_t p0 = (uint64_t)m0 * c0, p1 = (uint64_t)m1 * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

uint64_t orc_race_bits(uint64_t seed, uint32_t choice, uint32_t position, uint32_t row) {
  uint32_t counter[4] = {row >> 1, position, choice, 0x72616365u};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t w[4];
  orc_philox4x32_10(counter, key, w);
  uint32_t hi = (row & 1) ? w[2] : w[0];
  uint32_t lo = (row & 1) ? w[3] : w[1];
  return ((uint64_t)hi << 32) | lo;
}

/* gumbel_from_bits (race.rs:84-101).  The reference calls the pure-Rust
 * `libm` crate 0.2.16 (a musl port); glibc log/log1p are used here, which
 * the reference's own noise test bounds at 1e-15 (race.rs:241-259). */
double orc_gumbel_from_bits(uint64_t bits) {
  const double two_to_minus_64 = 1.0 / 18446744073709551616.0;
  double e;
  if (bits < (1ULL << 63)) e = -log1p(-(((double)bits + 0.5) * two_to_minus_64));
  else e = -log(((double)(~bits) + 0.5) * two_to_minus_64);
  return -log(e);
}

double orc_race_score(float logit, double temperature, uint64_t seed, uint32_t choice,
                      uint32_t position, uint32_t row) {
  return (double)logit / temperature + orc_gumbel_from_bits(orc_race_bits(seed, choice, position, row));
}

int orc_sample_race(const float* logits, const uint8_t* legal, size_t n, double temperature,
                    uint64_t seed, uint32_t choice, uint32_t position, uint32_t* token,
                    double* sampling_logprob) {
  if (n == 0) return ORC_EMPTY_LOGITS;
  if (n > UINT32_MAX) return ORC_VOCABULARY_TOO_LARGE;
  if (!isfinite(temperature) || temperature <= 0.0) return ORC_INVALID_TEMPERATURE;
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(logits[i])) return ORC_NON_FINITE_LOGIT;
  double maximum = -INFINITY;
  int has = 0;
  for (size_t i = 0; i < n; ++i)
    if (!legal || legal[i]) { maximum = fmax(maximum, (double)logits[i]); has = 1; }
  if (!has) return ORC_EMPTY_SUPPORT;
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) {
    if (legal && !legal[i]) continue;
    double s;
    int st = shifted_logit(logits[i], maximum, temperature, &s);
    if (st) return st;
    sum += exp(s);
  }
  int have = 0;
  uint32_t best = 0;
  double top = 0.0;
  for (size_t i = 0; i < n; ++i) {
    if (legal && !legal[i]) continue;
    double score = orc_race_score(logits[i], temperature, seed, choice, position, (uint32_t)i);
    if (!isfinite(score)) return ORC_INVALID_TEMPERATURE;
    if (!have || score > top) { have = 1; best = (uint32_t)i; top = score; }
  }
  double s;
  int st = shifted_logit(logits[best], maximum, temperature, &s);
  if (st) return st;
  *token = best;
  *sampling_logprob = s - log(sum);
  return ORC_OK;
}

/* ------------------------------------------------------------------------ */
float orc_bf16_to_f32(uint16_t h) {
  uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* BUILD-DEFINED penalty stage.  For each token, in f32 with every operation
 * rounded separately (no contraction):
 *   l = logit (+ bias, when the token is listed in the strictly increasing
 *       bias ids)
 *   c = occurrences of the token in the history
 *   if c > 0:
 *     l = l < 0 ? l * repetition : l / repetition
 *     l = l - (float)c * frequency
 *     l = l - presence
 * repetition follows the Hugging Face RepetitionPenaltyLogitsProcessor
 * (applied once per distinct token); frequency and presence follow OpenAI's
 * definitions.  A bias value of -inf suppresses its token: the adjusted
 * logit is f32::MIN after everything else, as ChatFormat::suppress writes it
 * (crates/core/chat-format/src/lib.rs:771-780; the reference has no bias or
 * penalties, so there suppression is exactly "logit = f32::MIN"). */
int orc_adjust_logits(const float* logits, size_t n, const orc_row_params* p, float* adjusted) {
  if (!(isfinite(p->repetition) && p->repetition > 0.0f) || !isfinite(p->presence) ||
      !isfinite(p->frequency))
    return ORC_INVALID_PENALTY;
  for (size_t j = 0; j < p->history_len; ++j)
    if (p->history[j] >= n) return ORC_INVALID_HISTORY;
  for (size_t j = 0; j < p->bias_len; ++j) {
    const float v = p->bias_values[j];
    if (p->bias_ids[j] >= n || isnan(v) || v == INFINITY) return ORC_INVALID_BIAS;
    if (j > 0 && p->bias_ids[j] <= p->bias_ids[j - 1]) return ORC_INVALID_BIAS;
  }
  memcpy(adjusted, logits, n * sizeof(float));
  for (size_t j = 0; j < p->bias_len; ++j) {
    if (p->bias_values[j] == -INFINITY) continue;   /* suppressed: set below */
    volatile float sum = adjusted[p->bias_ids[j]] + p->bias_values[j];
    adjusted[p->bias_ids[j]] = sum;
  }
  if (p->history_len) {
    uint32_t* counts = (uint32_t*)calloc(n, sizeof(uint32_t));
    if (!counts) abort();
    for (size_t j = 0; j < p->history_len; ++j) counts[p->history[j]]++;
    for (size_t i = 0; i < n; ++i) {
      uint32_t c = counts[i];
      if (!c) continue;
      float l = adjusted[i];
      l = l < 0.0f ? l * p->repetition : l / p->repetition;
      volatile float cf = (float)c * p->frequency;
      l = l - cf;
      l = l - p->presence;
      adjusted[i] = l;
    }
    free(counts);
  }
  for (size_t j = 0; j < p->bias_len; ++j)
    if (p->bias_values[j] == -INFINITY) adjusted[p->bias_ids[j]] = -FLT_MAX;
  return ORC_OK;
}

/* BUILD-DEFINED row sampler (see the header).  Error precedence:
 * temperature, top_p, min_p, penalties, history ids, bias ids, uniform,
 * non-finite adjusted logit, empty support, temperature overflow. */
int orc_sample_row(const float* logits, size_t n, const orc_row_params* p, float* adjusted,
                   uint8_t* kept, orc_row_result* r) {
  r->token = -1;
  r->sampling_logprob = 0.0;
  r->kept_count = 0;
  if (kept) memset(kept, 0, n);
#define FAIL(code) do { r->status = (code); return (code); } while (0)
  if (n == 0) FAIL(ORC_EMPTY_LOGITS);
  if (n > (size_t)INT32_MAX) FAIL(ORC_VOCABULARY_TOO_LARGE);
  const double T = p->temperature;
  if (!(T >= 0.0) || !isfinite(T)) FAIL(ORC_INVALID_TEMPERATURE);
  const int greedy = T == 0.0;
  if (!greedy && !(p->top_p > 0.0 && p->top_p <= 1.0)) FAIL(ORC_INVALID_TOP_P);
  if (!greedy && !(p->min_p >= 0.0 && p->min_p <= 1.0)) FAIL(ORC_INVALID_MIN_P);
  int st = orc_adjust_logits(logits, n, p, adjusted);
  if (st) FAIL(st);
  if (!greedy && (!isfinite(p->uniform) || !(p->uniform >= 0.0 && p->uniform < 1.0)))
    FAIL(ORC_INVALID_UNIFORM);
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(adjusted[i])) FAIL(ORC_NON_FINITE_LOGIT);
  /* legal set */
  uint8_t* legal = NULL;
  size_t nl = n;
  if (p->mask_words) {
    legal = (uint8_t*)malloc(n);
    if (!legal) abort();
    orc_fill_legal_mask(p->mask_words, p->mask_nwords, p->tokenizer_vocab, legal, n);
    nl = 0;
    for (size_t i = 0; i < n; ++i) nl += legal[i];
    if (nl == 0) { free(legal); FAIL(ORC_EMPTY_SUPPORT); }
  }
  if (greedy) {
    int32_t tok;
    if (legal) {
      int64_t idx;
      orc_masked_argmax(p->mask_words, p->mask_nwords, adjusted,
                        p->tokenizer_vocab < n ? p->tokenizer_vocab : n, &idx);
      free(legal);
      if (idx < 0) FAIL(ORC_EMPTY_SUPPORT);
      tok = (int32_t)idx;
    } else {
      st = orc_greedy_token(adjusted, n, &tok);
      if (st) FAIL(st);
    }
    r->token = tok;
    r->kept_count = 1;
    if (kept) kept[tok] = 1;
    r->status = ORC_OK;
    return ORC_OK;
  }
  /* compact row of legal tokens in ID order */
  uint32_t* ids = (uint32_t*)malloc(nl * sizeof(uint32_t));
  float* compact = (float*)malloc(nl * sizeof(float));
  uint8_t* mask = (uint8_t*)malloc(nl);
  if (!ids || !compact || !mask) abort();
  for (size_t i = 0, j = 0; i < n; ++i)
    if (!legal || legal[i]) { ids[j] = (uint32_t)i; compact[j] = adjusted[i]; ++j; }
  free(legal);
  st = orc_nucleus_mask(compact, nl, T, p->top_p, p->top_k, mask);
  if (st) { free(ids); free(compact); free(mask); FAIL(st); }
  if (p->min_p > 0.0) {
    /* BUILD-DEFINED min-p: keep kept tokens whose shifted logit
     * (f64(l) - M) / T reaches ln(min_p), M the compact row's maximum
     * (p_i >= min_p * p_max). */
    float mf = -INFINITY;
    for (size_t j = 0; j < nl; ++j) mf = fmaxf(mf, compact[j]);
    const double maximum = (double)mf, threshold = log(p->min_p);
    for (size_t j = 0; j < nl; ++j)
      if (mask[j] && !((((double)compact[j] - maximum) / T) >= threshold)) mask[j] = 0;
  }
  uint32_t pick;
  double lp;
  st = orc_sample_categorical(compact, mask, nl, T, p->uniform, &pick, &lp);
  if (!st) {
    r->token = (int32_t)ids[pick];
    r->sampling_logprob = lp;
    for (size_t j = 0; j < nl; ++j) {
      r->kept_count += mask[j];
      if (kept && mask[j]) kept[ids[j]] = 1;
    }
  }
  free(ids); free(compact); free(mask);
  if (st) FAIL(st);
  r->status = ORC_OK;
  return ORC_OK;
#undef FAIL
}

/* BUILD-DEFINED speculative verify of one row: temperature weights
 * w = exp((f64(l) - max) / T) of the target and draft rows feed
 * accept_or_resample position by position (speculative.rs:369-429); the
 * first rejection emits the resampled token and stops; when every draft is
 * accepted the bonus token is sample_categorical over target row k. */
int orc_spec_verify_row(const float* target, const float* draft, size_t vocab, size_t k,
                        const int32_t* draft_tokens, double temperature, const double* accept_u,
                        const double* resample_u, double bonus_u, int32_t* out_tokens,
                        int32_t* out_count, int32_t* out_accepted) {
  if (!isfinite(temperature) || temperature <= 0.0) return ORC_INVALID_TEMPERATURE;
  double* tw = (double*)malloc(vocab * sizeof(double));
  double* dw = (double*)malloc(vocab * sizeof(double));
  if (!tw || !dw) abort();
  int st = ORC_OK;
  *out_count = 0;
  *out_accepted = 0;
  for (size_t j = 0; j < k; ++j) {
    const float* t = target + j * vocab;
    const float* d = draft + j * vocab;
    double tm = -INFINITY, dm = -INFINITY;
    for (size_t i = 0; i < vocab; ++i) {
      if (!isfinite(t[i]) || !isfinite(d[i])) { st = ORC_NON_FINITE_LOGIT; goto done; }
      tm = fmax(tm, (double)t[i]);
      dm = fmax(dm, (double)d[i]);
    }
    for (size_t i = 0; i < vocab; ++i) {
      tw[i] = exp(((double)t[i] - tm) / temperature);
      dw[i] = exp(((double)d[i] - dm) / temperature);
    }
    if (draft_tokens[j] < 0) { st = ORC_TOKEN_OUT_OF_RANGE; goto done; }
    int accepted = 0;
    size_t resampled = 0;
    st = orc_accept_or_resample(tw, dw, vocab, (size_t)draft_tokens[j], accept_u[j], resample_u[j],
                                &accepted, &resampled);
    if (st) goto done;
    if (accepted) {
      out_tokens[j] = draft_tokens[j];
      *out_count = (int32_t)(j + 1);
      *out_accepted = (int32_t)(j + 1);
      continue;
    }
    out_tokens[j] = (int32_t)resampled;
    *out_count = (int32_t)(j + 1);
    goto done;
  }
  {
    uint32_t tok;
    double lp;
    st = orc_sample_categorical(target + k * vocab, NULL, vocab, temperature, bonus_u, &tok, &lp);
    if (!st) { out_tokens[k] = (int32_t)tok; *out_count = (int32_t)(k + 1); }
  }
done:
  free(tw);
  free(dw);
  return st;
}

/* ------------------------------------------------------------------------ */
static void batch_row_params(const orc_batch* b, size_t row, orc_row_params* p) {
  memset(p, 0, sizeof *p);
  p->temperature = b->temperature[row];
  p->top_p = b->top_p ? b->top_p[row] : 1.0;
  p->min_p = b->min_p ? b->min_p[row] : 0.0;
  p->uniform = b->uniform ? b->uniform[row] : 0.0;
  p->top_k = b->top_k ? b->top_k[row] : 0;
  p->repetition = b->repetition ? b->repetition[row] : 1.0f;
  p->presence = b->presence ? b->presence[row] : 0.0f;
  p->frequency = b->frequency ? b->frequency[row] : 0.0f;
  if (b->history_offsets) {
    p->history = b->history_ids + b->history_offsets[row];
    p->history_len = b->history_offsets[row + 1] - b->history_offsets[row];
  }
  if (b->bias_offsets) {
    p->bias_ids = b->bias_ids + b->bias_offsets[row];
    p->bias_values = b->bias_values + b->bias_offsets[row];
    p->bias_len = b->bias_offsets[row + 1] - b->bias_offsets[row];
  }
  if (b->mask_words) {
    p->mask_words = b->mask_words + row * b->mask_nwords;
    p->mask_nwords = b->mask_nwords;
    p->tokenizer_vocab = b->tokenizer_vocab;
  }
}

int orc_sample_batch(const orc_batch* b, size_t row_begin, size_t row_end, int32_t* tokens,
                     double* logprobs, int32_t* status, float* adjusted_scratch, uint8_t* kept_out) {
  float* scratch = adjusted_scratch;
  int own = 0;
  if (!scratch) { scratch = (float*)malloc(b->vocab * sizeof(float)); own = 1; }
  if (!scratch) abort();
  for (size_t row = row_begin; row < row_end; ++row) {
    orc_row_params p;
    batch_row_params(b, row, &p);
    orc_row_result r;
    float* adj = own ? scratch : scratch + row * b->vocab;
    orc_sample_row(b->logits + row * b->vocab, b->vocab, &p, adj,
                   kept_out ? kept_out + row * b->vocab : NULL, &r);
    tokens[row] = r.token;
    logprobs[row] = r.sampling_logprob;
    status[row] = r.status;
  }
  if (own) free(scratch);
  return ORC_OK;
}

typedef struct {
  const orc_batch* b; size_t begin, end; int32_t* tokens; double* logprobs; int32_t* status;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  orc_sample_batch(j->b, j->begin, j->end, j->tokens, j->logprobs, j->status, NULL, NULL);
  return NULL;
}

int orc_sample_batch_threads(const orc_batch* b, int threads, int32_t* tokens, double* logprobs,
                             int32_t* status) {
  if (threads < 1) threads = 1;
  if ((size_t)threads > b->rows) threads = (int)b->rows;
  pthread_t* th = (pthread_t*)malloc((size_t)threads * sizeof(pthread_t));
  batch_job* jobs = (batch_job*)malloc((size_t)threads * sizeof(batch_job));
  if (!th || !jobs) abort();
  for (int t = 0; t < threads; ++t) {
    jobs[t].b = b;
    jobs[t].begin = b->rows * (size_t)t / (size_t)threads;
    jobs[t].end = b->rows * (size_t)(t + 1) / (size_t)threads;
    jobs[t].tokens = tokens; jobs[t].logprobs = logprobs; jobs[t].status = status;
    pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
  return ORC_OK;
}
