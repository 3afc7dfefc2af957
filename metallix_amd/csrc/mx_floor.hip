// mx_floor.hip -- measurement floors for mxs_sample (diagnostics only, no
// reference counterpart).  Both kernels take mxs_sample's launch shape: the
// grid (8 * C, ceil(B / 8)), NT threads, a row's chunks on one XCD, and the
// sample kernel's LDS footprint (so one workgroup per CU, as there):
//   mode 0, launch floor: every workgroup writes one value and exits;
//   mode 1, stream floor: every workgroup reads its chunk of the row once,
//           with all of a thread's quad loads issued up front, and writes
//           the chunk's maximum;
//   mode 2: mode 1 that also writes each workgroup's wall-clock stamps
//           (100 MHz) at its first instruction and at its exit.
// Their durations bound what any single-pass sampler with this grid can
// reach: the stream floor is the achievable HBM time of the logits.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxs_ctx.h"
#include "mxs_device.h"

namespace mxs {

template <typename In, int MODE>
__global__ __launch_bounds__(NT) void floor_kernel(const In* __restrict__ logits, uint32_t rows, uint32_t V,
                                                   uint64_t stride, uint32_t CH, float* __restrict__ out,
                                                   uint64_t* __restrict__ stamps) {
  extern __shared__ __align__(16) float red[];
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= rows) return;
  const uint64_t t_entry = MODE == 2 ? wall_clock64() : 0u;
  if (MODE == 0) {
    if (threadIdx.x == 0) out[(uint64_t)row * MAXC + chunk] = (float)chunk;
    return;
  }
  const uint32_t c0 = chunk * CH, c1 = min(V, c0 + CH);
  const In* p = logits + (uint64_t)row * stride + c0;
  const uint32_t nq = c0 < c1 ? (c1 - c0) / 4u : 0u;   // whole quads of the chunk
  float m = -INFINITY;
  if (sizeof(In) == 4) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 v[PER_MAX];
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      const uint32_t j = (uint32_t)i * NT + threadIdx.x;
      v[i] = j < nq ? q[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) m = fmaxf(m, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
  } else {
    const uint2* q = reinterpret_cast<const uint2*>(p);
    uint2 v[PER_MAX];
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      const uint32_t j = (uint32_t)i * NT + threadIdx.x;
      v[i] = j < nq ? q[j] : make_uint2(0xff80ff80u, 0xff80ff80u);
    }
#pragma unroll
    for (int i = 0; i < PER_MAX; ++i) {
      m = fmaxf(m, fmaxf(__uint_as_float(v[i].x << 16), __uint_as_float(v[i].x & 0xffff0000u)));
      m = fmaxf(m, fmaxf(__uint_as_float(v[i].y << 16), __uint_as_float(v[i].y & 0xffff0000u)));
    }
  }
  for (uint32_t t = c0 + nq * 4u + threadIdx.x; t < c1; t += NT) {   // the chunk's last 1-3 tokens
    const float x = sizeof(In) == 4 ? (float)p[t - c0]
                                    : __uint_as_float((uint32_t)(*(const uint16_t*)(p + (t - c0))) << 16);
    m = fmaxf(m, x);
  }
  m = block_max(m, red);
  if (threadIdx.x == 0) out[(uint64_t)row * MAXC + chunk] = m;
  if (MODE == 2 && threadIdx.x == 0) {
    stamps[((uint64_t)row * MAXC + chunk) * 2] = t_entry;
    stamps[((uint64_t)row * MAXC + chunk) * 2 + 1] = wall_clock64();
  }
}

}  // namespace mxs

extern "C" int mxs_debug_floor(mxs_ctx* ctx, const void* logits, int32_t dtype, uint32_t rows, uint32_t vocab,
                               uint32_t row_stride, uint32_t mode, float* out, uint64_t* stamps) {
  if (!ctx || !logits || !out || rows == 0 || vocab == 0 || mode > 2u || (mode == 2u && !stamps)) return MXS_EINVAL;
  if (dtype != MXS_F32 && dtype != MXS_BF16) return fail(ctx, MXS_EINVAL, "dtype must be MXS_F32 or MXS_BF16");
  if (row_stride < vocab || (row_stride & 3u)) return fail(ctx, MXS_EINVAL, "row_stride must be >= vocab and a multiple of 4");
  if (((uintptr_t)logits) % (dtype == MXS_F32 ? 16u : 8u)) return fail(ctx, MXS_EINVAL, "logits misaligned");
  const mxs::ChunkLayout L = mxs::sample_layout(rows, vocab);   // small-batch doubling included
  if (L.per > (uint32_t)mxs::PER_MAX || L.C > (uint32_t)mxs::MAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  const dim3 grid(8u * L.C, (rows + 7u) / 8u);
  const size_t lds = mxs::sample_lds_bytes();
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  hipError_t e = hipSuccess;
#define MXS_FLOOR(T, M)                                                                                     \
  do {                                                                                                      \
    e = hipFuncSetAttribute((const void*)mxs::floor_kernel<T, M>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                            (int)lds);                                                                      \
    if (e == hipSuccess)                                                                                    \
      hipLaunchKernelGGL((mxs::floor_kernel<T, M>), grid, dim3(mxs::NT), lds, ctx->stream,                  \
                         (const T*)logits, rows, vocab, (uint64_t)row_stride, L.CH, out, stamps);           \
  } while (0)
  if (dtype == MXS_F32) {
    if (mode == 0u) MXS_FLOOR(float, 0); else if (mode == 1u) MXS_FLOOR(float, 1); else MXS_FLOOR(float, 2);
  } else {
    if (mode == 0u) MXS_FLOOR(uint16_t, 0); else if (mode == 1u) MXS_FLOOR(uint16_t, 1); else MXS_FLOOR(uint16_t, 2);
  }
#undef MXS_FLOOR
  if (e == hipSuccess) e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "floor_kernel launch");
  return MXS_OK;
}
