// mx_spec.hip -- speculative-decoding verification (mxs_spec_verify).
#include <hip/hip_runtime.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"

extern "C" int mxs_spec_verify(mxs_ctx* ctx, const float*, const float*, uint32_t, uint32_t, uint32_t,
                               const int32_t*, const double*, const double*, const double*, const double*,
                               int32_t*, int32_t*, int32_t*, int32_t*) {
  return fail(ctx, MXS_EINVAL, "mxs_spec_verify: not built yet");
}
