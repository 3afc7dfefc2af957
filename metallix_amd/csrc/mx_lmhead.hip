// mx_lmhead.hip -- a bf16 lm_head GEMM for gfx950 (mxs_lmhead_bf16): the
// logits producer whose epilogue writes the tile statistics of
// mxs_epilogue.h for mxs_finish_tiles.
//
// logits[n][v] = sum_k hidden[n][k] weight[v][k] (bf16 in, f32 accumulate),
// the lm_head of a Qwen3-shaped forward (the reference computes it in MLX
// before its picks, crates/models/qwen/src/forward.rs:1745-1761).  One
// 256-thread workgroup per 256-row vocabulary tile; wave w owns the tile's
// vocabulary rows 64 w .. 64 w + 63 against every batch row (at most 64), as
// 4 x 4 blocks of v_mfma_f32_16x16x32_bf16 (A: 16 vocabulary rows x 32 k, B:
// 32 k x 16 batch rows; lane l holds row l % 16 and k (l / 16) 8 .. + 7 of
// each, 16 contiguous bytes; D: lane l holds vocabulary rows (l / 16) 4 + j
// of batch row l % 16).  The weights stream from HBM once (the roofline:
// V K 2 bytes); the hidden states are re-read from L2 by every wave.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_epilogue.h"

namespace mxs {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

static_assert(sizeof(EpiTileStat) == MXS_TILE_STAT_BYTES && EPI_TILE == MXS_TILE_TOKENS, "the header's tile layout");

constexpr uint32_t LM_ROWS = 64;   // batch rows per launch (four 16-row MFMA blocks)
constexpr uint32_t LM_KC = 128;    // hidden-state k staged in LDS per chunk
constexpr uint32_t LM_BST = LM_KC + 8u;   // LDS row stride (bf16): rows 16 B apart in the banks

template <bool STATS>
__global__ __launch_bounds__(256) void lmhead_kernel(const __bf16* __restrict__ H, const __bf16* __restrict__ W,
                                                     uint32_t rows, uint32_t K, uint32_t V,
                                                     float* __restrict__ logits, uint64_t ld,
                                                     EpiTileStat* __restrict__ stats, uint32_t ntiles) {
  __shared__ EpiPartial part[4][LM_ROWS];
  __shared__ __align__(16) __bf16 Bs[2][LM_ROWS * LM_BST];   // staged hidden-state chunks
  const uint32_t tile = blockIdx.x, w = threadIdx.x >> 6, l = threadIdx.x & 63u;
  const uint32_t lr = l & 15u, lg = l >> 4;
  const uint32_t vw = tile * EPI_TILE + w * 64u;   // this wave's first vocabulary row
  // weight rows, clamped in range (the clamped rows' results are dropped)
  const __bf16* ap[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const uint32_t v = min(vw + (uint32_t)mb * 16u + lr, V - 1u);
    ap[mb] = W + (uint64_t)v * K + lg * 8u;
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // The hidden states pass through LDS in chunks of LM_KC k, double
  // buffered: thread t stages 32 k of row t / 4 (rows clamped; the clamped
  // rows' results are dropped), once per workgroup instead of once per wave.
  const uint32_t sn = min(threadIdx.x >> 2, rows - 1u), sk = (threadIdx.x & 3u) * 32u;
  const __bf16* hsrc = H + (uint64_t)sn * K + sk;
  bf16x8 st[4];
  auto stage_load = [&](uint32_t c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) st[j] = *reinterpret_cast<const bf16x8*>(hsrc + c * LM_KC + 8u * (uint32_t)j);
  };
  auto stage_store = [&](uint32_t buf) {
    __bf16* dst = &Bs[buf][(threadIdx.x >> 2) * LM_BST + sk];
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<bf16x8*>(dst + 8u * (uint32_t)j) = st[j];
  };
  // The weights stream from HBM into registers two K steps ahead: step
  // s + 2's rows load while step s's products issue.  The loads are
  // unconditional (past the last step they repeat it, in bounds, unused) so
  // the memory counter waits stay exact.
  const uint32_t steps = K / 32u, nch = K / LM_KC;
  bf16x8 a[2][4];
  auto load_a = [&](bf16x8* d, uint32_t s) {
    const uint32_t k0 = min(s, steps - 1u) * 32u;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) d[mb] = *reinterpret_cast<const bf16x8*>(ap[mb] + k0);
  };
  stage_load(0u);
  load_a(a[0], 0u);
  load_a(a[1], 1u);
  stage_store(0u);
  __syncthreads();
  for (uint32_t c = 0; c < nch; ++c) {
    if (c + 1u < nch) stage_load(c + 1u);
    const __bf16* bs = &Bs[c & 1u][0];
#pragma unroll
    for (uint32_t ks = 0; ks < LM_KC / 32u; ++ks) {
      bf16x8 b[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        b[nb] = *reinterpret_cast<const bf16x8*>(bs + ((uint32_t)nb * 16u + lr) * LM_BST + ks * 32u + lg * 8u);
      bf16x8* ac = a[ks & 1u];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[mb], b[nb], acc[mb][nb], 0, 0, 0);
      load_a(ac, c * (LM_KC / 32u) + ks + 2u);
    }
    if (c + 1u < nch) stage_store((c + 1u) & 1u);
    __syncthreads();
  }
  // acc[mb][nb][j]: token vw + 16 mb + 4 lg + j of batch row 16 nb + lr
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    const uint32_t n = (uint32_t)nb * 16u + lr;
    EpiPartial p = epi_empty();
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const uint32_t v0 = vw + (uint32_t)mb * 16u + lg * 4u;
      if (v0 < V) {   // V % 4 == 0: the quad is in range
        if (n < rows) *reinterpret_cast<f32x4*>(logits + (uint64_t)n * ld + v0) = acc[mb][nb];
        if (STATS) {
#pragma unroll
          for (int j = 0; j < 4; ++j) epi_add(p, acc[mb][nb][j]);
        }
      }
    }
    if (STATS) {
      epi_xor(p, 16);
      epi_xor(p, 32);
      if (lg == 0u) part[w][n] = p;
    }
  }
  if (STATS) {
    __syncthreads();
    if (threadIdx.x < rows) {
      const uint32_t n = threadIdx.x;
      EpiPartial p = part[0][n];
#pragma unroll
      for (int q = 1; q < 4; ++q) epi_merge(p, part[q][n]);
      epi_store(&stats[(uint64_t)n * ntiles + tile], p);
    }
  }
}

}  // namespace mxs

extern "C" int mxs_lmhead_bf16(mxs_ctx* ctx, const void* hidden, const void* weight, uint32_t rows,
                               uint32_t hidden_dim, uint32_t vocab, float* logits, uint64_t logits_stride,
                               void* tile_stats) {
  using namespace mxs;
  if (!ctx) return MXS_EINVAL;
  if (rows == 0) return MXS_OK;
  if (!hidden || !weight || !logits) return fail(ctx, MXS_EINVAL, "hidden, weight and logits are required");
  if (rows > LM_ROWS) return fail(ctx, MXS_EINVAL, "rows must be at most 64");
  if (hidden_dim == 0 || hidden_dim % LM_KC) return fail(ctx, MXS_EINVAL, "hidden_dim must be a positive multiple of 128");
  if (vocab == 0 || vocab % 4u) return fail(ctx, MXS_EINVAL, "vocab must be a positive multiple of 4");
  if (logits_stride < vocab || logits_stride % 4u) return fail(ctx, MXS_EINVAL, "logits_stride must be >= vocab and a multiple of 4");
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)logits) % 16u)
    return fail(ctx, MXS_EINVAL, "hidden, weight and logits must be 16-byte aligned");
  const uint32_t ntiles = (vocab + EPI_TILE - 1u) / EPI_TILE;
  int prev = 0;
  (void)hipGetDevice(&prev);
  if (prev != ctx->device) (void)hipSetDevice(ctx->device);
  const __bf16* H = reinterpret_cast<const __bf16*>(hidden);
  const __bf16* W = reinterpret_cast<const __bf16*>(weight);
  EpiTileStat* S = reinterpret_cast<EpiTileStat*>(tile_stats);
  if (S)
    hipLaunchKernelGGL(lmhead_kernel<true>, dim3(ntiles), dim3(256), 0, ctx->stream, H, W, rows, hidden_dim, vocab,
                       logits, logits_stride, S, ntiles);
  else
    hipLaunchKernelGGL(lmhead_kernel<false>, dim3(ntiles), dim3(256), 0, ctx->stream, H, W, rows, hidden_dim, vocab,
                       logits, logits_stride, S, ntiles);
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "lmhead_kernel launch");
  return MXS_OK;
}
