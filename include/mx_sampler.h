/* mx_sampler.h -- C ABI of the MI355X (gfx950) token sampler, libmx_sampler.so.
 *
 * The drop-in boundary for metallix's device pick.  Each entry point names
 * the reference interface it replaces (paths relative to the
 * arclabs561/metallix tree):
 *
 *   mxs_create / mxs_destroy  <- mlx_kernels::MetalKernel::new + Drop
 *                                (crates/metal/mlx-kernels/src/lib.rs:203-215, 444-450):
 *                                one handle owns the compiled kernels and scratch.
 *   mxs_sample                <- Qwen3TokenPicks::start_with(rows, binding, rule)
 *                                (crates/models/qwen/src/forward/picks.rs:279-381) with
 *                                Qwen3Selection::{Greedy, TopKNucleus}; the arithmetic is
 *                                TokenPicker::pick -> SamplingPolicy::sample_nucleus ->
 *                                nucleus_mask + sample_categorical
 *                                (crates/app/cli/src/qwen_forward.rs:264-278, 474-549;
 *                                crates/core/engine/src/sampling.rs:56-158), greedy_token
 *                                (crates/app/cli/src/chat_generation.rs:2213-2231) and the
 *                                grammar-mask consumption of
 *                                crates/core/engine/src/constraint.rs:793-806, 895-932.
 *   mxs_sample_race           <- Qwen3TokenPicks::start_with with Qwen3Selection::Race
 *                                (picks.rs:40-66, 296-336) and its host settle, SamplingPolicy::
 *                                sample under Entropy::Race (qwen_forward.rs:221-278, 310-341)
 *                                -> sample_race (crates/core/engine/src/sampling/race.rs:114-147).
 *   mxs_logsoftmax_topn       <- token_logprob (crates/app/cli/src/chat_turn.rs:506-563) and
 *                                Qwen3RowCandidates (picks.rs:97-129).
 *   mxs_spec_verify           <- engine::speculative::accept_or_resample
 *                                (crates/core/engine/src/speculative.rs:369-444) applied
 *                                position by position as in speculative_step (:202-227).
 *   mxs_step                  <- the per-row pick loop of EngineLoop::decode_now
 *                                (crates/app/cli/src/engine_loop.rs:1080-1134) through
 *                                TurnLoop::pick (chat_turn.rs:290-303): ChatFormat::suppress,
 *                                the pick, and token_logprob's receipt (chat_turn.rs:506-563)
 *                                for every row of the batch in one call.
 *   mxs_mask_host,            <- the per-step SimpleVob words (crates/core/engine/src/
 *   mxs_mask_upload              constraint.rs:777-806) on their way to the device: pinned
 *                                staging, an upload on a copy stream, double-buffered.
 *   mxs_export_candidates     <- Qwen3TokenPicks::wait_with_candidates (picks.rs:429-466), the
 *                                candidates TurnLoop::settle_row hands pick_from_candidates
 *                                (chat_turn.rs:332-358; chat_generation.rs:2088-2131).
 *   mxs_lmhead_bf16,          <- the lm_head that feeds Qwen3TokenPicks::start_with in
 *   mxs_finish_tiles             Qwen3ForwardExecutor::append_picks (crates/models/qwen/src/
 *                                forward.rs:1745-1761), with the pick fused into its epilogue:
 *                                the GEMM's tiles publish mxs_epilogue.h statistics and the
 *                                finish-only pick reads those and the tiles a head can reach.
 *   mxs_sync                  <- Qwen3TokenPicks::wait (picks.rs:390-401).
 *   mxs_last_error            <- KernelError's message (mlx-kernels/src/lib.rs:444-450).
 *
 * Conventions.  Every buffer is caller-owned device memory unless stated.
 * Calls are asynchronous on the context's stream and never synchronise the
 * host (except mxs_sync).  Return codes: 0 = accepted, negative = rejected
 * before launch (see mxs_last_error).  Per-row results carry a status:
 * 0 = ok, 1 = ok but uncertified (a decision margin fell below the device's
 * rigorous floating-point error bound; the token is the device's best
 * decision and a caller that owes bit-exact parity re-derives the row on the
 * host, as TokenPicker does when candidates cannot settle a pick,
 * chat_turn.rs:348-358), negative = the row's error (MXS_ROW_* below, the
 * first seven mirroring engine::sampling::SamplingError,
 * sampling.rs:19-43).  One context belongs to one host thread at a time.
 */
#ifndef MX_SAMPLER_H
#define MX_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXS_ABI_VERSION 2

/* Call return codes. */
enum {
  MXS_OK = 0,
  MXS_EINVAL = -1,     /* bad argument: null pointer, size over the context limits, misalignment */
  MXS_EHIP = -2,       /* a HIP runtime call failed */
  MXS_ENOMEM = -3,     /* device allocation failed */
  MXS_ENODEV = -4      /* no gfx950 device */
};

/* Per-row status codes (mxs_out.status). */
enum {
  MXS_ROW_OK = 0,
  MXS_ROW_UNCERTIFIED = 1,
  MXS_ROW_EMPTY_LOGITS = -1,
  MXS_ROW_MASK_LENGTH_MISMATCH = -2,
  MXS_ROW_EMPTY_SUPPORT = -3,
  MXS_ROW_INVALID_TEMPERATURE = -4,
  MXS_ROW_INVALID_UNIFORM = -5,
  MXS_ROW_NON_FINITE_LOGIT = -6,
  MXS_ROW_VOCABULARY_TOO_LARGE = -7,
  MXS_ROW_INVALID_TOP_P = -8,
  MXS_ROW_INVALID_MIN_P = -9,
  MXS_ROW_INVALID_PENALTY = -10,
  MXS_ROW_INVALID_HISTORY = -11,
  MXS_ROW_INVALID_BIAS = -12,
  MXS_ROW_TOKEN_OUT_OF_RANGE = -13,
  MXS_ROW_PROBABILITIES = -14,
  MXS_ROW_UNSUPPORTED_RULE = -15  /* mxs_finish_tiles: a rule other than greedy or top-k <= 4096 */
};

typedef enum { MXS_F32 = 0, MXS_BF16 = 1 } mxs_dtype;

typedef struct mxs_ctx mxs_ctx;

/* One batch of logit rows and the per-row sampling rule.  Per-row arrays
 * are device arrays of `rows` entries; NULL selects the default shown.
 * These fields are Qwen3Selection::TopKNucleus's (temperature, top_p,
 * top_k, uniforms; picks.rs:20-40) plus the stages the reference rejects
 * at its HTTP layer and this sampler defines (penalties, logit bias,
 * min_p) and the grammar mask (constraint.rs:793-806). */
typedef struct {
  const void* logits;             /* rows x row_stride elements of `dtype` */
  int32_t dtype;                  /* mxs_dtype */
  uint32_t rows;
  uint32_t vocab;
  uint64_t row_stride;            /* elements between row starts; multiple of 4 */
  const double* temperature;      /* required; 0 => greedy */
  const uint32_t* top_k;          /* NULL => 0 (off) */
  const double* top_p;            /* NULL => 1 (off) */
  const double* min_p;            /* NULL => 0 (off) */
  const float* repetition;        /* NULL => 1 (off) */
  const float* presence;          /* NULL => 0 */
  const float* frequency;         /* NULL => 0 */
  const double* uniform;          /* required unless every row is greedy; [0, 1) */
  const uint32_t* history_offsets;/* rows + 1 offsets into history_ids (CSR); NULL => none */
  const uint32_t* history_ids;
  const uint32_t* bias_offsets;   /* rows + 1 offsets into bias_ids/bias_values; NULL => none */
  const uint32_t* bias_ids;       /* strictly increasing within a row */
  const float* bias_values;       /* finite, or -INFINITY: the token is suppressed, its adjusted
                                     logit f32::MIN (ChatFormat::suppress,
                                     crates/core/chat-format/src/lib.rs:771-780) */
  const uint32_t* mask_words;     /* rows x mask_stride u32 words, bit b of word w <-> token 32w+b; NULL => none */
  uint64_t mask_stride;           /* words between row masks; >= ceil(vocab / 32) */
  uint32_t tokenizer_vocab;       /* with a mask: tokens at or past it are never legal */
  uint32_t reserved;
} mxs_batch;

/* Outputs of mxs_sample: device arrays of `rows` entries; the debug
 * outputs may be NULL. */
typedef struct {
  int32_t* token;                 /* required */
  double* sampling_logprob;       /* NULL => not written */
  int32_t* status;                /* required */
  uint32_t* kept_count;           /* NULL => not written */
  float* adjusted;                /* debug: rows x vocab penalised, biased logits */
  uint32_t* kept_bits;            /* debug: rows x ceil(vocab / 32) final kept set */
} mxs_out;

int mxs_create(int device, void* stream, uint32_t max_rows, uint32_t max_vocab, mxs_ctx** out);
int mxs_destroy(mxs_ctx* ctx);
int mxs_set_stream(mxs_ctx* ctx, void* stream);
int mxs_sample(mxs_ctx* ctx, const mxs_batch* batch, const mxs_out* out);
/* race-v2 keys (engine::sampling::race::RaceKey plus the generated
 * position, race.rs:29-37, 66-80): device arrays of `rows` entries. */
typedef struct {
  const uint64_t* seed;           /* required: the request seed of each row */
  const uint32_t* choice;         /* NULL => 0: the completion index within the request */
  const uint32_t* position;       /* required: the generated position of each row's token */
} mxs_race;

/* As mxs_sample, but every non-greedy row takes the race-v2 winner over its
 * kept set: the kept token with the largest f64(adjusted logit) / T +
 * Gumbel(Philox4x32-10 bits of (seed, choice, position, token)), lowest ID on
 * ties.  batch->uniform is ignored (race-v2 draws none).  sampling_logprob is
 * the winner's log probability over the kept set at temperature T.  Status 1
 * when the two best scores are too close to order against the reference's
 * libm.  out->kept_bits may be NULL (the context's scratch holds the set). */
int mxs_sample_race(mxs_ctx* ctx, const mxs_batch* batch, const mxs_race* race, const mxs_out* out);
int mxs_logsoftmax_topn(mxs_ctx* ctx, const void* logits, int32_t dtype, uint32_t rows,
                        uint32_t vocab, uint64_t row_stride, uint32_t n, int32_t* ids,
                        double* logprobs, double* maximum, double* log_normalizer, int32_t* status);
int mxs_spec_verify(mxs_ctx* ctx, const float* target_logits, const float* draft_logits,
                    uint32_t rows, uint32_t draft_len, uint32_t vocab,
                    const int32_t* draft_tokens, const double* temperature,
                    const double* accept_uniform, const double* resample_uniform,
                    const double* bonus_uniform, int32_t* out_tokens, int32_t* out_count,
                    int32_t* out_accepted, int32_t* status);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mxs_logsoftmax_topn without a context.  The kernels run
 * on `stream` (a hipStream_t; NULL = the default stream) on the current
 * device, with their per-chunk statistics and lists in a device array the
 * library holds per GPU until the process ends: rows * ceil(vocab / 8192) *
 * (24 + 8 n) bytes must fit in MXS_TOPN_STATIC_BYTES (MXS_EINVAL otherwise).
 * Calls on one GPU share that array, so calls that overlap in time on one
 * GPU (other streams, other threads) race; calls in order on one stream do
 * not.  Allocates nothing.  mxs_last_error(NULL) reads this thread's last
 * error message. */
#define MXS_TOPN_STATIC_BYTES (8u << 20)
int mxs_logsoftmax_topn_noalloc(void* stream, const void* logits, int32_t dtype, uint32_t rows,
                                uint32_t vocab, uint64_t row_stride, uint32_t n, int32_t* ids,
                                double* logprobs, double* maximum, double* log_normalizer,
                                int32_t* status);
/* Log-probability receipts of one step (TokenLogprob, chat_turn.rs:506-563):
 * over each row's logits after suppression (the batch's bias entries of
 * -INFINITY read as f32::MIN, ChatFormat::suppress, chat-format/src/lib.rs:
 * 771-780) and nothing else, the n most likely IDs by (total_cmp
 * descending, ID ascending) with f64(l) - maximum - log_normalizer, and the
 * picked token's log probability.  n is the largest top_logprobs + 8, the
 * over-selection the reference ranks before it drops unspellable IDs.
 * Device arrays; rows whose `top` entry is MXS_RECEIPT_NONE are not
 * written.  A `top` entry of 0 is a receipt with no top entries (the
 * reference's `logprobs: true` without top_logprobs, Some(0):
 * chat_completions.rs:241-243): the picked token's log probability is
 * still written, with the ranked IDs (the caller keeps none of them). */
#define MXS_RECEIPT_NONE 0xFFFFFFFFu
typedef struct {
  const uint32_t* top;            /* rows entries: the row's top_logprobs, MXS_RECEIPT_NONE => no receipt; NULL => every row */
  uint32_t n;                     /* entries per row of ids and logprobs, 1..64 */
  uint32_t reserved;
  int32_t* ids;                   /* rows x n; -1 past the vocabulary */
  double* logprobs;               /* rows x n; -inf past the vocabulary */
  double* token_logprob;          /* rows: the picked token's; NaN when the row has no token */
  int32_t* status;                /* rows: 0, or MXS_ROW_NON_FINITE_LOGIT */
} mxs_receipts;

/* One engine step: the pick of every row (mxs_sample, or mxs_sample_race
 * when `race` is given), then, when `receipts` is given, the receipts of
 * the rows that want one, queued behind the picks on the context's stream
 * (their token_logprob reads out->token on the device).  Replaces the
 * reference's per-row host loop; which receipts to keep (a stop token takes
 * none, TurnLoop::receipt_wanted, chat_turn.rs:413-418) and the drop of
 * unspellable IDs stay with the caller. */
int mxs_step(mxs_ctx* ctx, const mxs_batch* batch, const mxs_race* race, const mxs_out* out,
             const mxs_receipts* receipts);
/* Grammar-mask staging.  The constraint's allowed-token words for a step
 * (SimpleVob: bit b of word w <-> token 32w+b, constraint.rs:793-806) are
 * written by the host into a pinned staging slot (0 or 1) the context owns,
 * then uploaded.  mxs_mask_host returns the slot's host words (max_rows rows
 * of *stride_words words; allocated at the first call) after waiting until
 * the slot's previous upload has read them.  mxs_mask_upload queues the copy
 * of the slot's first `rows` rows on the context's copy stream, behind the
 * last pick that read the slot's device words, and orders the context's
 * stream after the copy; *device_words is the slot's device copy, to pass as
 * batch->mask_words with mask_stride = *stride_words.  Two slots
 * double-buffer consecutive steps: fill and upload slot 1 - s while the pick
 * of slot s runs. */
/* Candidates of the context's last mxs_sample or mxs_step call, per row of
 * its first `rows` rows, queued on the context's stream behind that call:
 * the list the row's finisher chose from (every candidate at or above its
 * chunk's threshold; it holds the row's top-k head for a top-k row and its
 * min-p set for a min-p row), as adjusted logits (penalties, bias, mask
 * applied) with their token IDs, in token-ID order.  count[r] = the list's
 * length when at most `width`; else its top `width` by (logit desc, ID asc)
 * and count[r] = width; -1 for a row with no list (greedy, keep-all, error
 * rows).  ids and logits are rows x width.  The settle of an uncertified
 * (status 1) top-k row with k <= width: sort by (logit desc, ID asc), keep
 * the first k, and apply the row's rule to them, as pick_from_candidates'
 * sample_top_k_candidates does; the row need not be read back.  A later
 * pick on the context overwrites the lists. */
int mxs_export_candidates(mxs_ctx* ctx, uint32_t rows, uint32_t width, int32_t* count, int32_t* ids,
                          float* logits);
/* A bf16 lm_head for gfx950: logits[n][v] = sum_k hidden[n][k] weight[v][k]
 * (f32 accumulate), hidden rows x hidden_dim, weight vocab x hidden_dim, both
 * row-major bf16 and 16-byte aligned; rows <= 64, hidden_dim a multiple of
 * 128, vocab a multiple of 4; logits f32 rows x logits_stride.  When
 * tile_stats is non-null, the epilogue also writes, per (row, 256-token
 * tile), the statistics mxs_finish_tiles reads (MXS_TILE_STAT_BYTES each,
 * rows x ceil(vocab / MXS_TILE_TOKENS); the layout is mxs::EpiTileStat of
 * metallix_amd/csrc/mxs_epilogue.h, whose device functions any producer's
 * epilogue can call). */
#define MXS_TILE_TOKENS 256      /* vocabulary entries per tile of the epilogue statistics */
#define MXS_TILE_STAT_BYTES 8    /* bytes per (row, tile): the tile maximum's order key, a non-finite flag */
int mxs_lmhead_bf16(mxs_ctx* ctx, const void* hidden, const void* weight, uint32_t rows, uint32_t hidden_dim,
                    uint32_t vocab, float* logits, uint64_t logits_stride, void* tile_stats);
/* The pick of mxs_sample from a producer's tile statistics: batch->logits
 * (f32) are the producer's logits, of which only the tiles a row's top-k
 * head can reach are read; the rows' rules are greedy (temperature 0) or
 * top-k with 1 <= top_k <= 4096 (with top_p, min_p and the uniform as in
 * mxs_sample); no penalties, bias or mask (the reference's device picks
 * take none, picks.rs:273-381); a row with another rule reports
 * MXS_ROW_UNSUPPORTED_RULE.  vocab <= 262144.  Outputs as mxs_sample's
 * (adjusted must be NULL); results are identical to mxs_sample's on the
 * same logits.  One workgroup per row reads the tiles whose maximum reaches
 * the k-th largest tile maximum, so the read shrinks with k / tile count:
 * greedy and small-k rows (k up to about 128 at vocab 151936) finish faster
 * than mxs_sample; a row with k above the tile count reads its row twice in
 * one workgroup, slower than mxs_sample's chunked read. */
int mxs_finish_tiles(mxs_ctx* ctx, const mxs_batch* batch, const void* tile_stats, const mxs_out* out);
int mxs_mask_host(mxs_ctx* ctx, uint32_t slot, uint32_t** words, uint64_t* stride_words);
int mxs_mask_upload(mxs_ctx* ctx, uint32_t slot, uint32_t rows, const uint32_t** device_words);
int mxs_sync(mxs_ctx* ctx);
/* Diagnostics (no reference counterpart): when `device_buffer` is non-null,
 * mxs_sample records 100 MHz wall-clock stamps at fixed phase boundaries:
 * u64 [rows][MXS_DEBUG_TIMING_SLOTS][MXS_DEBUG_TIMING_STAMPS], chunk
 * workgroups at slot = chunk, the row finisher at slot
 * MXS_DEBUG_TIMING_SLOTS - 1; stamp 8 is a workgroup's first instruction,
 * stamp 9 its exit, stamps 10 and 11 bracket a step receipt's work, and
 * the finisher's stamps 12 to 14 its reduction of candidate lists beyond its
 * LDS cache (histogram start, histogram end, compaction end).  NULL
 * disables. */
#define MXS_DEBUG_TIMING_SLOTS 65
#define MXS_DEBUG_TIMING_STAMPS 16
int mxs_debug_set_timing(mxs_ctx* ctx, void* device_buffer);
/* Diagnostics (no reference counterpart): measurement floors in
 * mxs_sample's launch shape (grid, workgroup size, LDS per workgroup) on the
 * context's stream.  mode 0: every workgroup exits at once (the launch
 * floor); mode 1: every workgroup reads its chunk of the logits once and
 * writes its maximum (the stream floor); mode 2: mode 1 that also writes
 * each workgroup's 100 MHz wall-clock stamps at entry and exit to `stamps`
 * (device u64 [rows][MXS_DEBUG_TIMING_SLOTS - 1][2]; NULL otherwise).
 * `out`: device f32 [rows][MXS_DEBUG_TIMING_SLOTS - 1]. */
int mxs_debug_floor(mxs_ctx* ctx, const void* logits, int32_t dtype, uint32_t rows, uint32_t vocab,
                    uint32_t row_stride, uint32_t mode, float* out, uint64_t* stamps);
/* Diagnostics (no reference counterpart): when `device_buffer` (int32
 * [rows]) is non-null, mxs_sample writes the finisher path each row took. */
enum {
  MXS_PATH_ERROR = 1,          /* a row error status */
  MXS_PATH_GREEDY = 2,         /* temperature 0: the chunks' argmax */
  MXS_PATH_KEEPALL = 3,        /* every legal token kept: draw by segment masses */
  MXS_PATH_KEEPALL_RACE = 4,   /* the same rows under race-v2 (no draw) */
  MXS_PATH_SELECT = 5,         /* candidates in registers: the selection finisher */
  MXS_PATH_WAVE = 6,           /* few candidates: one wave */
  MXS_PATH_FAST = 7,           /* the k head or min-p set in LDS */
  MXS_PATH_EXACT = 8,          /* working set in LDS, the nucleus certified without a sort */
  MXS_PATH_EXACT_SORTED = 9,   /* ... the crossing inside the min-p prefix: that prefix sorted */
  MXS_PATH_EXACT_REPLAY = 10,  /* ... an uncertain crossing: the reference's sums replayed */
  MXS_PATH_LARGE = 11,         /* working set beyond LDS: mass-weighted radix select */
  MXS_PATH_SHORT = 12          /* top-k <= 64 or min-p rows, at most 512 candidates: one wave, one E member per lane */
};
int mxs_debug_set_paths(mxs_ctx* ctx, void* device_buffer);
const char* mxs_last_error(const mxs_ctx* ctx);
const char* mxs_status_string(int32_t status);
int mxs_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
