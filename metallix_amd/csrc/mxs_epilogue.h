// mxs_epilogue.h -- device functions a logits-producing kernel's epilogue
// calls per output tile so that mxs_finish_tiles can pick without reading
// the whole logits row back.
//
// A tile is EPI_TILE consecutive vocabulary entries of one row; tile t of a
// row covers tokens [t EPI_TILE, (t + 1) EPI_TILE).  For every (row, tile)
// the producer stores one EpiTileStat at stats[row * ntiles + t]:
//   - tmax: the order key (total order: -0.0 below +0.0) of the tile's
//     largest value, which bounds the tile's members of a top-k head and
//     marks the tiles holding the row maximum (the greedy argmax, lowest ID
//     on ties with -0.0 equal to +0.0, greedy_token,
//     chat_generation.rs:2213-2231, is found in those tiles);
//   - bad: 1 when a value of the tile is NaN or infinite.
// The logits themselves are still written (mxs_finish_tiles re-reads only
// the tiles a row's pick can reach).  Accumulate with epi_add per value the
// lane holds, merge lanes with epi_merge (shuffles, DPP or LDS: the merge is
// associative and commutative), store one partial per (row, tile); start
// from epi_empty().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxs_math.h"

namespace mxs {

constexpr uint32_t EPI_TILE = 256;   // vocabulary entries per tile

struct EpiTileStat {
  uint32_t tmax;                     // order key of the tile's largest value (0: none)
  uint32_t bad;                      // a non-finite value
};

struct EpiPartial {
  uint32_t tmax;
  uint32_t bad;
};

__device__ __forceinline__ EpiPartial epi_empty() {
  EpiPartial p;
  p.tmax = 0u;
  p.bad = 0u;
  return p;
}

__device__ __forceinline__ void epi_add(EpiPartial& p, float v) {
  const uint32_t t = okey(v);
  p.tmax = t > p.tmax ? t : p.tmax;
  p.bad |= __builtin_isfinite(v) ? 0u : 1u;
}

__device__ __forceinline__ void epi_merge(EpiPartial& p, const EpiPartial& q) {
  p.tmax = q.tmax > p.tmax ? q.tmax : p.tmax;
  p.bad |= q.bad;
}

// Merges the partials of lanes l, l ^ m for each m in the xor masks (a
// butterfly over lane groups, e.g. {16, 32} joins the four lanes l % 16).
__device__ __forceinline__ void epi_xor(EpiPartial& p, int m) {
  EpiPartial q;
  q.tmax = (uint32_t)__shfl_xor((int)p.tmax, m);
  q.bad = (uint32_t)__shfl_xor((int)p.bad, m);
  epi_merge(p, q);
}

__device__ __forceinline__ void epi_store(EpiTileStat* dst, const EpiPartial& p) {
  EpiTileStat s;
  s.tmax = p.tmax;
  s.bad = p.bad;
  *dst = s;
}

}  // namespace mxs
