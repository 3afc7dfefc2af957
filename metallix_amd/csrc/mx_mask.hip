// mx_mask.hip -- grammar-mask staging: the host side of the mask's trip from
// the constraint engine to the sampler (mxs_mask_host / mxs_mask_upload of
// include/mx_sampler.h).
//
// Reference: each step the constraint computes the allowed tokens on the CPU
// as an llguidance SimpleVob (crates/core/engine/src/constraint.rs:777-789)
// whose u32 words, LSB first, are the per-row mask (:793-806, 4748 words for
// V = 151936).  Here the host writes those words straight into a pinned
// staging slot the context owns; the upload copies the slot to device memory
// on a copy stream of its own and makes the context's stream wait for it, so
// the copy overlaps whatever runs before the pick (the forward pass).  Two
// slots double-buffer consecutive steps: while step n's pick reads slot s,
// the host fills slot 1 - s for step n + 1.  Two events per slot keep the
// reuse safe: the host rewrites a slot only after its last copy has read it
// (mask_copied, waited in mxs_mask_host), and a copy overwrites a device
// slot only after the last pick that read it (mask_read, recorded by every
// pick whose batch points into the slot, waited on the copy stream).

#include <hip/hip_runtime.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"

namespace mxs {

static int mask_alloc(mxs_ctx* ctx) {
  if (ctx->mask_host[0]) return MXS_OK;
  // rows start 16-byte aligned (the kernels read the words as uint4)
  const uint64_t stride = (((uint64_t)ctx->max_vocab + 31u) / 32u + 3u) & ~(uint64_t)3u;
  const size_t bytes = (size_t)ctx->max_rows * stride * sizeof(uint32_t);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  hipError_t e = hipSuccess;
  for (int s = 0; s < 2 && e == hipSuccess; ++s) {
    e = hipHostMalloc((void**)&ctx->mask_host[s], bytes, hipHostMallocDefault);
    e = e ? e : hipMalloc((void**)&ctx->mask_dev[s], bytes);
    e = e ? e : hipEventCreateWithFlags(&ctx->mask_copied[s], hipEventDisableTiming);
    e = e ? e : hipEventCreateWithFlags(&ctx->mask_read[s], hipEventDisableTiming);
  }
  e = e ? e : hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking);
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) {
    mask_release(ctx);
    return hip_fail(ctx, e, "mask staging allocation");
  }
  ctx->mask_stride = stride;
  return MXS_OK;
}

void mask_release(mxs_ctx* ctx) {
  for (int s = 0; s < 2; ++s) {
    if (ctx->mask_host[s]) hipHostFree(ctx->mask_host[s]);
    if (ctx->mask_dev[s]) hipFree(ctx->mask_dev[s]);
    if (ctx->mask_copied[s]) hipEventDestroy(ctx->mask_copied[s]);
    if (ctx->mask_read[s]) hipEventDestroy(ctx->mask_read[s]);
    ctx->mask_host[s] = nullptr;
    ctx->mask_dev[s] = nullptr;
    ctx->mask_copied[s] = nullptr;
    ctx->mask_read[s] = nullptr;
    ctx->copy_queued[s] = ctx->read_queued[s] = false;
  }
  if (ctx->copy_stream) hipStreamDestroy(ctx->copy_stream);
  ctx->copy_stream = nullptr;
  ctx->mask_stride = 0;
}

void mask_note_read(mxs_ctx* ctx, const uint32_t* words) {
  if (!words || !ctx->mask_dev[0]) return;
  const uint64_t n = (uint64_t)ctx->max_rows * ctx->mask_stride;
  for (int s = 0; s < 2; ++s) {
    if (words >= ctx->mask_dev[s] && words < ctx->mask_dev[s] + n) {
      hipEventRecord(ctx->mask_read[s], ctx->stream);
      ctx->read_queued[s] = true;
    }
  }
}

}  // namespace mxs

extern "C" int mxs_mask_host(mxs_ctx* ctx, uint32_t slot, uint32_t** words, uint64_t* stride_words) {
  if (!ctx || slot > 1u || !words || !stride_words) return MXS_EINVAL;
  if (int rc = mxs::mask_alloc(ctx)) return rc;
  if (ctx->copy_queued[slot]) {
    // the slot's last upload must have read the host words before they change
    const hipError_t e = hipEventSynchronize(ctx->mask_copied[slot]);
    if (e != hipSuccess) return hip_fail(ctx, e, "waiting for the slot's last upload");
    ctx->copy_queued[slot] = false;
  }
  *words = ctx->mask_host[slot];
  *stride_words = ctx->mask_stride;
  return MXS_OK;
}

extern "C" int mxs_mask_upload(mxs_ctx* ctx, uint32_t slot, uint32_t rows, const uint32_t** device_words) {
  if (!ctx || slot > 1u || !device_words) return MXS_EINVAL;
  if (!ctx->mask_host[0]) return fail(ctx, MXS_EINVAL, "mxs_mask_host must stage the slot before its upload");
  if (rows > ctx->max_rows) return fail(ctx, MXS_EINVAL, "rows exceed the context's max_rows");
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  hipError_t e = hipSuccess;
  // the device slot is overwritten only after the last pick that read it
  if (ctx->read_queued[slot]) e = hipStreamWaitEvent(ctx->copy_stream, ctx->mask_read[slot], 0);
  const size_t bytes = (size_t)rows * ctx->mask_stride * sizeof(uint32_t);
  if (e == hipSuccess && bytes)
    e = hipMemcpyAsync(ctx->mask_dev[slot], ctx->mask_host[slot], bytes, hipMemcpyHostToDevice, ctx->copy_stream);
  e = e ? e : hipEventRecord(ctx->mask_copied[slot], ctx->copy_stream);
  // the picks queued from here on read the new words
  e = e ? e : hipStreamWaitEvent(ctx->stream, ctx->mask_copied[slot], 0);
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "mask upload");
  ctx->copy_queued[slot] = true;
  *device_words = ctx->mask_dev[slot];
  return MXS_OK;
}
