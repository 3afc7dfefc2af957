/* sanitize_check.c -- test infrastructure: drives every function of the
 * oracle (mx_oracle.c) over seeded random and edge-case inputs in a build
 * with AddressSanitizer and UndefinedBehaviorSanitizer (`make -C oracle
 * sanitize`), so an out-of-bounds access, a use of uninitialised heap
 * memory by index, a signed overflow or a misaligned access in the checker
 * stops the run.  Also checks a few contracts each function states (a token
 * in range on success, kept sets within the legal set, one accepted or
 * resampled outcome per verify).  Exit status 0: clean. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mx_oracle.h"

static uint64_t g_state = 0x5eed5eed5eedull;
static uint64_t next_u64(void) {   /* SplitMix64 */
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static double unif(void) { return (double)(next_u64() >> 11) * 0x1p-53; }
static size_t below(size_t n) { return n ? (size_t)(next_u64() % n) : 0; }

static int failures = 0;
static long ok_calls = 0;   /* calls that returned ORC_OK: how much of each path ran */
#define CHECK(cond, ...)                 \
  do {                                   \
    if (!(cond)) {                       \
      fprintf(stderr, __VA_ARGS__);      \
      fputc('\n', stderr);               \
      ++failures;                        \
    }                                    \
  } while (0)

/* logits with ties, plateaus, a spread of scales and (rarely) non-finite values */
static void fill_logits(float* x, size_t n, int allow_nonfinite) {
  const double scale = 0.1 + 4.0 * unif();
  for (size_t i = 0; i < n; ++i) {
    double v = scale * (unif() * 2.0 - 1.0) * 3.0;
    if (below(8) == 0) v = floor(v);            /* ties */
    x[i] = (float)v;
  }
  if (n && below(4) == 0) x[below(n)] += 8.0f;  /* a peak */
  if (allow_nonfinite && n && below(16) == 0) x[below(n)] = below(2) ? INFINITY : NAN;
}

static void check_categorical_and_nucleus(size_t n) {
  float* x = malloc((n ? n : 1) * sizeof(float));
  uint8_t* legal = malloc(n ? n : 1);
  uint8_t* mask = malloc(n ? n : 1);
  fill_logits(x, n, 1);
  for (size_t i = 0; i < n; ++i) legal[i] = below(5) != 0;
  const double temps[] = {0.0, 1e-3, 0.7, 1.0, 3.0, -1.0, NAN};
  const double t = temps[below(7)];
  const double u = below(10) == 0 ? 0.0 : (below(10) == 0 ? 1.0 - 0x1p-53 : unif());
  uint32_t tok = 0;
  double lp = 0.0;
  int st = orc_sample_categorical(x, legal, n, t, u, &tok, &lp);
  if (st == ORC_OK) { ++ok_calls; CHECK(tok < n && legal[tok], "categorical: token %u of %zu not legal", tok, n); }
  const double ps[] = {1.0, 0.9, 0.5, 1e-9, 0.0, 1.5};
  const size_t ks[] = {0, 1, 2, 20, n, n + 5};
  st = orc_nucleus_mask(x, n, t > 0 ? t : 1.0, ps[below(6)], ks[below(6)], mask);
  if (st == ORC_OK) {
    size_t kept = 0;
    for (size_t i = 0; i < n; ++i) kept += mask[i] != 0;
    CHECK(kept >= 1 || n == 0, "nucleus: empty kept set over %zu tokens", n);
  }
  int32_t g = -1;
  st = orc_greedy_token(x, n, &g);
  if (st == ORC_OK) CHECK(g >= 0 && (size_t)g < n, "greedy: token %d of %zu", g, n);
  free(x);
  free(legal);
  free(mask);
}

static void check_masks_and_logprobs(size_t n) {
  const size_t words = (n + 31) / 32 + below(3);
  uint32_t* w = malloc((words ? words : 1) * sizeof(uint32_t));
  for (size_t i = 0; i < words; ++i) w[i] = (uint32_t)next_u64() & (uint32_t)next_u64();
  float* x = malloc((n ? n : 1) * sizeof(float));
  uint8_t* legal = malloc(n ? n : 1);
  fill_logits(x, n, 0);
  const size_t width = below(2) ? n : n + below(40);
  int64_t idx = -2;
  if (orc_masked_argmax(w, words, x, width < n ? width : n, &idx) == ORC_OK)
    CHECK(idx >= -1 && idx < (int64_t)n, "masked argmax: index %lld of %zu", (long long)idx, n);
  orc_fill_legal_mask(w, words, below(n + 8), legal, n);
  double lp = 0.0;
  if (n) orc_selected_model_logprob(x, n, (uint32_t)below(n + 2), &lp);
  const size_t top = below(n + 10);
  int32_t* ids = malloc((top ? top : 1) * sizeof(int32_t));
  double* lps = malloc((top ? top : 1) * sizeof(double));
  double mx = 0.0, ln = 0.0;
  if (orc_token_logprob_top(x, n, top, ids, lps, &mx, &ln) == ORC_OK) {
    const size_t k = top < n ? top : n;
    for (size_t i = 0; i < k; ++i) CHECK(ids[i] >= 0 && (size_t)ids[i] < n, "top: id %d of %zu", ids[i], n);
    for (size_t i = 1; i < k; ++i) CHECK(lps[i] <= lps[i - 1], "top: logprobs not descending at %zu", i);
  }
  free(w);
  free(x);
  free(legal);
  free(ids);
  free(lps);
}

static void check_speculative(size_t n) {
  double* p = malloc(n * sizeof(double));
  double* q = malloc(n * sizeof(double));
  double sp = 0.0, sq = 0.0;
  for (size_t i = 0; i < n; ++i) {
    p[i] = below(4) ? unif() : 0.0;
    q[i] = below(4) ? unif() : 0.0;
    sp += p[i];
    sq += q[i];
  }
  for (size_t i = 0; i < n && sp > 0 && sq > 0; ++i) { p[i] /= sp; q[i] /= sq; }
  if (below(10) == 0) p[below(n)] = NAN;
  int acc = -1;
  size_t res = (size_t)-1;
  if (orc_accept_or_resample(p, q, n, below(n + 2), unif(), unif(), &acc, &res) == ORC_OK)
    CHECK(acc == 1 || res < n, "accept_or_resample: no outcome (accepted %d, resampled %zu of %zu)", acc, res, n);
  free(p);
  free(q);

  const size_t k = 1 + below(6);
  float* tgt = malloc((k + 1) * n * sizeof(float));
  float* drf = malloc(k * n * sizeof(float));
  int32_t dt[8];
  double au[8], ru[8];
  for (size_t j = 0; j <= k; ++j) fill_logits(tgt + j * n, n, 0);
  for (size_t j = 0; j < k; ++j) {
    for (size_t i = 0; i < n; ++i) drf[j * n + i] = tgt[j * n + i] + (float)(unif() - 0.5);
    dt[j] = below(12) == 0 ? (int32_t)(n + 3) : (int32_t)below(n);
    au[j] = unif();
    ru[j] = unif();
  }
  int32_t out[9], cnt = -1, nacc = -1;
  if (orc_spec_verify_row(tgt, drf, n, k, dt, below(8) ? 0.3 + unif() : 0.0, au, ru, unif(), out, &cnt, &nacc) ==
      ORC_OK) {
    CHECK(cnt >= 1 && cnt <= (int32_t)k + 1 && nacc >= 0 && nacc < cnt, "spec verify: count %d accepted %d", cnt,
          nacc);
    for (int32_t j = 0; j < cnt; ++j) CHECK(out[j] >= 0 && (size_t)out[j] < n, "spec verify: token %d", out[j]);
  }
  free(tgt);
  free(drf);
}

static void check_race(size_t n) {
  float* x = malloc(n * sizeof(float));
  uint8_t* legal = malloc(n);
  fill_logits(x, n, 1);
  for (size_t i = 0; i < n; ++i) legal[i] = below(3) != 0;
  uint32_t ctr[4] = {(uint32_t)next_u64(), (uint32_t)next_u64(), (uint32_t)next_u64(), (uint32_t)next_u64()};
  uint32_t key[2] = {(uint32_t)next_u64(), (uint32_t)next_u64()}, out[4];
  orc_philox4x32_10(ctr, key, out);
  const uint64_t bits = orc_race_bits(next_u64(), (uint32_t)below(4), (uint32_t)below(1u << 20), (uint32_t)below(n));
  const double gmb = orc_gumbel_from_bits(bits);
  CHECK(isfinite(gmb), "gumbel not finite for bits %llx", (unsigned long long)bits);
  uint32_t tok = 0;
  double lp = 0.0;
  if (orc_sample_race(x, legal, n, below(6) ? 0.1 + 2.0 * unif() : 0.0, next_u64(), (uint32_t)below(4),
                      (uint32_t)below(1000), &tok, &lp) == ORC_OK)
    CHECK(tok < n && legal[tok], "race: token %u of %zu not legal", tok, n);
  free(x);
  free(legal);
}

static void check_rows_and_batches(size_t rows, size_t n) {
  float* x = malloc(rows * n * sizeof(float));
  double *t = malloc(rows * sizeof(double)), *tp = malloc(rows * sizeof(double));
  double *mp = malloc(rows * sizeof(double)), *u = malloc(rows * sizeof(double));
  uint32_t* tk = malloc(rows * sizeof(uint32_t));
  float *rep = malloc(rows * sizeof(float)), *pres = malloc(rows * sizeof(float)), *freq = malloc(rows * sizeof(float));
  uint32_t *hoff = malloc((rows + 1) * sizeof(uint32_t)), *boff = malloc((rows + 1) * sizeof(uint32_t));
  uint32_t* hids = malloc(rows * 16 * sizeof(uint32_t));
  uint32_t* bids = malloc(rows * 8 * sizeof(uint32_t));
  float* bvals = malloc(rows * 8 * sizeof(float));
  const size_t words = (n + 31) / 32;
  uint32_t* mw = malloc(rows * words * sizeof(uint32_t));
  hoff[0] = boff[0] = 0;
  for (size_t r = 0; r < rows; ++r) {
    fill_logits(x + r * n, n, 1);
    t[r] = below(5) ? 0.2 + 2.0 * unif() : 0.0;
    tp[r] = below(3) ? 0.3 + 0.7 * unif() : 1.0;
    mp[r] = below(3) ? 0.0 : unif() * 0.2;
    u[r] = unif();
    tk[r] = (uint32_t)(below(3) ? below(n + 4) : 0);
    rep[r] = (float)(0.5 + unif());
    pres[r] = (float)(unif() - 0.5);
    freq[r] = (float)(unif() - 0.5);
    const size_t hn = below(16), bn = below(8);
    for (size_t j = 0; j < hn; ++j) hids[hoff[r] + j] = (uint32_t)(below(40) ? below(n) : n);   /* rarely invalid */
    hoff[r + 1] = hoff[r] + (uint32_t)hn;
    uint32_t id = (uint32_t)below(4);
    for (size_t j = 0; j < bn; ++j) {
      bids[boff[r] + j] = id;
      bvals[boff[r] + j] = below(6) ? (float)(unif() * 4.0 - 2.0) : -INFINITY;
      id += 1 + (uint32_t)below(n / 4 + 1);
    }
    boff[r + 1] = boff[r] + (uint32_t)bn;
    for (size_t w = 0; w < words; ++w) mw[r * words + w] = below(8) ? (uint32_t)next_u64() : 0u;
  }
  const int masked = below(2);
  orc_batch b = {x, rows, n, t, tp, mp, u, tk, rep, pres, freq, hoff, hids, boff, bids, bvals,
                 masked ? mw : NULL, words, masked ? n - below(n / 2 + 1) : 0};
  int32_t *tok = malloc(rows * sizeof(int32_t)), *st = malloc(rows * sizeof(int32_t));
  double* lp = malloc(rows * sizeof(double));
  float* adj = malloc(rows * n * sizeof(float));
  uint8_t* kept = malloc(rows * n);
  orc_sample_batch(&b, 0, rows, tok, lp, st, adj, kept);
  for (size_t r = 0; r < rows; ++r)
    if (st[r] == ORC_OK) { ++ok_calls; CHECK(tok[r] >= 0 && (size_t)tok[r] < n, "batch row %zu: token %d", r, tok[r]); }
  int32_t *tok2 = malloc(rows * sizeof(int32_t)), *st2 = malloc(rows * sizeof(int32_t));
  double* lp2 = malloc(rows * sizeof(double));
  orc_sample_batch_threads(&b, 3, tok2, lp2, st2);
  for (size_t r = 0; r < rows; ++r)
    CHECK(st2[r] == st[r] && (st[r] != ORC_OK || tok2[r] == tok[r]), "threaded batch differs on row %zu", r);
  /* one row through the row API, with the same parameters */
  orc_row_params p = {t[0], tp[0], mp[0], u[0], tk[0], rep[0], pres[0], freq[0], hids, hoff[1], bids, bvals, boff[1],
                      masked ? mw : NULL, words, masked ? b.tokenizer_vocab : 0};
  orc_row_result res;
  orc_adjust_logits(x, n, &p, adj);
  orc_sample_row(x, n, &p, adj, kept, &res);
  CHECK(res.status == st[0] && (res.status != ORC_OK || res.token == tok[0]), "row API differs from batch row 0");
  for (size_t i = 0; i < 64; ++i) (void)orc_bf16_to_f32((uint16_t)next_u64());
  free(x); free(t); free(tp); free(mp); free(u); free(tk); free(rep); free(pres); free(freq);
  free(hoff); free(boff); free(hids); free(bids); free(bvals); free(mw);
  free(tok); free(st); free(lp); free(adj); free(kept); free(tok2); free(st2); free(lp2);
}

int main(void) {
  orc_chacha8 rng;
  orc_chacha8_seed_from_u64(&rng, 42);
  for (int i = 0; i < 200; ++i) {
    const double v = orc_unit_uniform(orc_chacha8_next_u64(&rng));
    CHECK(v >= 0.0 && v < 1.0, "unit_uniform out of [0, 1): %g", v);
  }
  const size_t sizes[] = {0, 1, 2, 3, 31, 32, 33, 64, 100, 257};
  for (int it = 0; it < 400; ++it) {
    const size_t n = sizes[below(10)];
    check_categorical_and_nucleus(n);
    check_masks_and_logprobs(n);
    if (n) {
      check_speculative(n);
      check_race(n);
      check_rows_and_batches(1 + below(6), n);
    }
  }
  if (failures) fprintf(stderr, "%d contract failures\n", failures);
  else printf("sanitize_check: clean (%ld successful picks checked)\n", ok_calls);
  return failures ? 1 : 0;
}
