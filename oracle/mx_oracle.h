/* mx_oracle.h -- CPU restatement of the metallix token-sampler path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * sampler in metallix_amd/, and the timed CPU baseline of bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product path never calls it.
 *
 * Every function restates one reference function (file:line in the
 * arclabs561/metallix tree) in plain C11: f64 where the reference uses f64,
 * the same iteration orders, the same strict/non-strict comparisons, glibc
 * libm exp/log (the libm Rust std links on Linux).  Build-defined stages the
 * reference does not have (penalties, logit bias, min-p, mask + nucleus) are
 * marked BUILD-DEFINED and follow the semantics written in the design notes
 * shipped with this repository.
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0 ok, negative = error.  The first seven mirror
 * engine::sampling::SamplingError (crates/core/engine/src/sampling.rs:19-43). */
enum {
  ORC_OK = 0,
  ORC_EMPTY_LOGITS = -1,
  ORC_MASK_LENGTH_MISMATCH = -2,
  ORC_EMPTY_SUPPORT = -3,
  ORC_INVALID_TEMPERATURE = -4,
  ORC_INVALID_UNIFORM = -5,
  ORC_NON_FINITE_LOGIT = -6,
  ORC_VOCABULARY_TOO_LARGE = -7,
  ORC_INVALID_TOP_P = -8,      /* nucleus_mask: top_p outside (0, 1] */
  ORC_INVALID_MIN_P = -9,      /* BUILD-DEFINED: min_p outside [0, 1] */
  ORC_INVALID_PENALTY = -10,   /* BUILD-DEFINED: repetition <= 0 or non-finite penalty */
  ORC_INVALID_HISTORY = -11,   /* BUILD-DEFINED: history id >= vocabulary */
  ORC_INVALID_BIAS = -12,      /* BUILD-DEFINED: bias id >= vocabulary, ids not increasing, NaN or +inf bias */
  ORC_TOKEN_OUT_OF_RANGE = -13,/* speculative: drafted token outside the row */
  ORC_PROBABILITIES = -14,     /* speculative: invalid probability vectors */
};

/* ---- entropy (host side of icdf-v1) ------------------------------------ */
double orc_unit_uniform(uint64_t word);
typedef struct { uint32_t key[8]; uint64_t counter; uint32_t buf[64]; uint32_t index; } orc_chacha8;
void orc_chacha8_seed_from_u64(orc_chacha8* rng, uint64_t seed);
uint64_t orc_chacha8_next_u64(orc_chacha8* rng);

/* ---- reference primitives ---------------------------------------------- */
int orc_sample_categorical(const float* logits, const uint8_t* legal, size_t n, double temperature,
                           double uniform, uint32_t* token, double* sampling_logprob);
int orc_nucleus_mask(const float* logits, size_t n, double temperature, double top_p, size_t top_k,
                     uint8_t* mask);
int orc_greedy_token(const float* logits, size_t n, int32_t* token);
int orc_masked_argmax(const uint32_t* words, size_t nwords, const float* logits, size_t width,
                      int64_t* index);
void orc_fill_legal_mask(const uint32_t* words, size_t nwords, size_t tokenizer_vocab, uint8_t* legal,
                         size_t n);
int orc_selected_model_logprob(const float* logits, size_t n, uint32_t token, double* logprob);
int orc_token_logprob_top(const float* logits, size_t n, size_t top, int32_t* ids, double* logprobs,
                          double* maximum, double* log_normalizer);
int orc_accept_or_resample(const double* target, const double* draft, size_t n, size_t drafted,
                           double accept_uniform, double resample_uniform, int* accepted,
                           size_t* resampled);
void orc_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]);
uint64_t orc_race_bits(uint64_t seed, uint32_t choice, uint32_t position, uint32_t row);
double orc_gumbel_from_bits(uint64_t bits);
double orc_race_score(float logit, double temperature, uint64_t seed, uint32_t choice,
                      uint32_t position, uint32_t row);
int orc_sample_race(const float* logits, const uint8_t* legal, size_t n, double temperature,
                    uint64_t seed, uint32_t choice, uint32_t position, uint32_t* token,
                    double* sampling_logprob);

/* ---- BUILD-DEFINED composed row sampler --------------------------------
 * One row of the batched sampler: logit bias, penalties, grammar mask, then
 * greedy (temperature 0) or nucleus (top-k -> top-p) -> min-p -> inverse-CDF
 * draw.  The nucleus and draw are the reference's own nucleus_mask and
 * sample_categorical applied to the compact row of legal tokens in ID order,
 * the same compaction the reference uses in
 * SamplingPolicy::sample_top_k_candidates (qwen_forward.rs:404-428). */
typedef struct {
  double temperature;      /* 0 => greedy */
  double top_p;            /* (0, 1]; 1 => off */
  double min_p;            /* [0, 1]; 0 => off */
  double uniform;          /* [0, 1) */
  uint32_t top_k;          /* 0 => off */
  float repetition;        /* > 0; 1 => off */
  float presence;          /* finite */
  float frequency;         /* finite */
  const uint32_t* history; size_t history_len;
  const uint32_t* bias_ids; const float* bias_values; size_t bias_len;
  const uint32_t* mask_words; size_t mask_nwords; size_t tokenizer_vocab; /* mask_words NULL => no mask */
} orc_row_params;

typedef struct {
  int32_t status;
  int32_t token;
  double sampling_logprob;
  uint32_t kept_count;
} orc_row_result;

/* Writes the adjusted (biased, penalised) logits to `adjusted` (n floats,
 * required) and the final kept set to `kept` (n bytes, may be NULL). */
int orc_sample_row(const float* logits, size_t n, const orc_row_params* params, float* adjusted,
                   uint8_t* kept, orc_row_result* result);
/* Penalty/bias stage alone (BUILD-DEFINED), exposed for stage tests. */
int orc_adjust_logits(const float* logits, size_t n, const orc_row_params* params, float* adjusted);

/* BUILD-DEFINED speculative verify of one batch row (Leviathan rule of
 * speculative.rs:369-444 on temperature weights of two logit rows). */
int orc_spec_verify_row(const float* target, const float* draft, size_t vocab, size_t k,
                        const int32_t* draft_tokens, double temperature, const double* accept_u,
                        const double* resample_u, double bonus_u, int32_t* out_tokens,
                        int32_t* out_count, int32_t* out_accepted);

/* bf16 -> f32 widening (exact). */
float orc_bf16_to_f32(uint16_t h);

/* Batched drivers for the CPU baseline: rows [row_begin, row_end). */
typedef struct {
  const float* logits; size_t rows, vocab;
  const double* temperature; const double* top_p; const double* min_p; const double* uniform;
  const uint32_t* top_k; const float* repetition; const float* presence; const float* frequency;
  const uint32_t* history_offsets; const uint32_t* history_ids;
  const uint32_t* bias_offsets; const uint32_t* bias_ids; const float* bias_values;
  const uint32_t* mask_words; size_t mask_nwords; size_t tokenizer_vocab;
} orc_batch;
int orc_sample_batch(const orc_batch* batch, size_t row_begin, size_t row_end, int32_t* tokens,
                     double* logprobs, int32_t* status, float* adjusted_scratch, uint8_t* kept_out);
/* Same as orc_sample_batch, spread over `threads` POSIX threads (rows partitioned). */
int orc_sample_batch_threads(const orc_batch* batch, int threads, int32_t* tokens, double* logprobs,
                             int32_t* status);

#ifdef __cplusplus
}
#endif
#endif
