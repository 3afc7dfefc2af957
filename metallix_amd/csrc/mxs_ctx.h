// mxs_ctx.h -- the host-side context behind the C ABI's mxs_ctx handle,
// shared by the entry points of the sampler, log-softmax and speculative
// verification kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/mx_sampler.h"

namespace mxs {

struct ChunkStat;

// mxs_sample_race runs mxs_sample's pipeline for the kept set and discards
// its inverse-CDF draw; with `nodraw` set, the draw's nearness to a CDF
// boundary never flags a row (only the kept set's own certificate does).
// Keep-all rows skip the draw; other rows still make one with this uniform
// (the golden-ratio conjugate, any value in (0, 1) would do).
constexpr double RACE_DRAW_UNIFORM = 0.6180339887498949;

// mxs_sample's launch; `nodraw` makes keep-all rows skip the inverse-CDF
// draw (token -1, status 0, the kept set still written) and keeps every
// row's draw out of its status; `rx` (checked by the caller) adds the step
// receipts of the rows that want one, computed in the same pass.
int sample_launch(mxs_ctx* ctx, const mxs_batch* b, const mxs_out* o, bool nodraw,
                  const mxs_receipts* rx = nullptr);

// The sample kernel's LDS bytes per workgroup and its chunk layout for a
// batch of `rows` rows of V tokens (mx_floor.hip launches with both).
size_t sample_lds_bytes();
struct ChunkLayout;
ChunkLayout sample_layout(uint32_t rows, uint32_t V);

// A pick queued on ctx->stream read `words`: when they are a staging
// slot's device words, the slot's next upload waits for that pick
// (mx_mask.hip).
void mask_note_read(mxs_ctx* ctx, const uint32_t* words);
void mask_release(mxs_ctx* ctx);   // frees the staging slots (mxs_destroy)

// Scratch sizes of the entry points other than mxs_sample (defined beside
// their kernels).
size_t topn_scratch_bytes(uint32_t max_rows);
const char* noalloc_last_error();   // this thread's last mxs_logsoftmax_topn_noalloc error, or nullptr
size_t spec_scratch_bytes(uint32_t max_rows, uint32_t max_vocab);
size_t race_scratch_bytes(uint32_t max_rows, uint32_t max_vocab);
constexpr uint32_t SPEC_COUNTERS_PER_ROW = 10;   // one per (row, position <= 8), one per row

// Rows' counters and exchange words sit on their own 128-byte lines, so the
// atomics of different rows do not queue on one line.
constexpr uint32_t CTR_STRIDE = 32;    // u32 words between arrival counters (one 128-byte line each)
constexpr uint32_t ROWX_STRIDE = 16;   // u64 words per row of Work::rowx

// Device scratch of mxs_sample, sized for the context's limits.
struct Work {
  uint32_t* ctr;              // [max_rows * CTR_STRIDE] chunks of the row done (the row's last chunk resets it)
  unsigned long long* rowx;   // [max_rows * ROWX_STRIDE] (call epoch << 32) | largest chunk-maximum key published so far;
                              // the row's last chunk clears it, so an entry never outlives its call
  ChunkStat* stat;            // [max_rows * MAXC]
  float* cand_l;              // [max_rows * max_vocab]
  uint32_t* cand_id;          // [max_rows * max_vocab]
  double* seg;                // [max_rows * MAXC * PER_MAX * NW]
  int32_t* cand_rows;         // [max_rows] candidates the row's finisher chose from (-1: no list)
};

}  // namespace mxs

struct mxs_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  uint32_t max_rows = 0, max_vocab = 0;
  mxs::Work work{};
  // Defaults standing in for the ABI's NULL arrays, so the kernel never tests
  // a pointer: zeros (u32, max_rows + 1), ones/zeros (f64), ones/zeros (f32),
  // and one all-ones mask row.
  uint32_t* d_zero_u32 = nullptr;
  double* d_one_f64 = nullptr;
  double* d_zero_f64 = nullptr;
  float* d_one_f32 = nullptr;
  float* d_zero_f32 = nullptr;
  uint32_t* d_mask_ones = nullptr;
  uint64_t* timing = nullptr;
  int32_t* paths = nullptr;             // finisher path per row (diagnostics)
  uint32_t epoch = 0;                 // mxs_sample calls so far (tags Work::rowx entries)
  // the last mxs_sample / mxs_step call's layout (mxs_export_candidates)
  uint32_t last_rows = 0, last_C = 0, last_CH = 0, last_V = 0;
  // mxs_logsoftmax_topn: per-chunk results
  void* topn_scratch = nullptr;
  // mxs_spec_verify: per-position arrival counters and per-chunk results
  uint32_t* spec_ctr = nullptr;
  void* spec_scratch = nullptr;
  // mxs_sample_race: per-row arrival counters, per-chunk results and the
  // kept set when the caller asks for none
  uint32_t* race_ctr = nullptr;
  void* race_scratch = nullptr;
  uint32_t* race_kept = nullptr;
  float* race_m = nullptr;   // each row's largest adjusted logit, from the finisher to the race kernel
  // the uniform of the inverse-CDF draw mxs_sample_race discards (below)
  double* d_race_u = nullptr;
  // grammar-mask staging (mxs_mask_host / mxs_mask_upload, mx_mask.hip):
  // two slots of max_rows rows of mask_stride words, pinned on the host and
  // on the device, allocated at the first mxs_mask_host; copies run on
  // their own stream (default priority)
  uint32_t* mask_host[2] = {nullptr, nullptr};
  uint32_t* mask_dev[2] = {nullptr, nullptr};
  uint64_t mask_stride = 0;
  hipStream_t copy_stream = nullptr;
  hipEvent_t mask_copied[2] = {nullptr, nullptr};   // the slot's last upload has read the host words
  hipEvent_t mask_read[2] = {nullptr, nullptr};     // the last pick that read the device slot is done
  bool copy_queued[2] = {false, false};
  bool read_queued[2] = {false, false};
  std::string last_error;
};

namespace {

inline int fail(mxs_ctx* ctx, int code, const std::string& msg) {
  if (ctx) ctx->last_error = msg;
  return code;
}

inline int hip_fail(mxs_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, MXS_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace
