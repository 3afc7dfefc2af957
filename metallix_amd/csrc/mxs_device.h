// mxs_device.h -- device building blocks shared by the sampler kernels:
// the chunk layout, coherent cross-workgroup loads and stores, barriers,
// DPP wave reductions and scans, block reductions, and the logit loaders.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxs_math.h"

namespace mxs {

constexpr int NT = 1024;                  // threads per workgroup
constexpr int NW = NT / 64;               // waves per workgroup
constexpr int PER_MAX = 10;               // 4-token quads per thread per chunk
constexpr int SLICE = NT * 4;             // tokens per slice (one quad per thread)
constexpr int CHUNK_MAX = SLICE * PER_MAX;
constexpr int MAXC = 64;                  // chunks per row (vocab <= MAXC * CHUNK_MAX)
constexpr int TSTAMPS = 16;               // diagnostic timestamps per timing record
constexpr uint32_t NONE = 0xffffffffu;
constexpr double U = 1.1102230246251565e-16;  // 2^-53

// Chunk layout of a row of V tokens: C chunks of CH tokens (a multiple of
// 4), each streamed by one workgroup as `per` quads per thread.
struct ChunkLayout {
  uint32_t C, CH, per;
};
inline ChunkLayout chunk_layout(uint32_t V, uint32_t per_max = PER_MAX) {
  const uint32_t quads = (V + 3u) / 4u;
  uint32_t C = (quads + (uint32_t)NT * per_max - 1u) / ((uint32_t)NT * per_max);
  if (C < 1) C = 1;
  const uint32_t ch = ((V + C - 1u) / C + 3u) & ~3u;
  return {C, ch, (ch / 4u + (uint32_t)NT - 1u) / (uint32_t)NT};
}

// ---------------------------------------------------------------------------
// Device-scope (coherent across workgroups and XCDs) loads and stores.  Data
// exchanged between a row's workgroups goes through these: they bypass the
// non-coherent caches, so no L2 writeback/invalidate is needed.
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(double* p, double v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_dev(const double* p) {
  return __hip_atomic_load(const_cast<double*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_dev(const float2* p) {
  const unsigned long long v = __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<float2*>(p)),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
__device__ __forceinline__ uint2 ld_dev(const uint2* p) {
  const unsigned long long v = __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<uint2*>(p)),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}
__device__ __forceinline__ void st_dev(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this lane's outstanding memory operations have completed.
__device__ __forceinline__ void wait_mem() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Arrival of one workgroup on a counter shared by the `total` workgroups
// that split one unit of work (a row, a row position).  Returns true in every
// thread of the last workgroup to arrive, which also returns the counter to
// zero for the next launch.  `flag` is a word of LDS.
//
// Ordering.  Everything the workgroups exchange is written with the
// device-scope stores above (st_dev: scope bits sc1, written through to the
// level every XCD reads) and read with the device-scope loads (ld_dev).  Each
// wave waits for its own stores to complete (s_waitcnt vmcnt(0): complete
// means performed at device scope), the workgroup barrier puts every wave's
// wait before thread 0's increment, and the last arriver issues its loads
// only after its increment returned the final count, that is after every
// other workgroup's increment, each issued after that workgroup's stores had
// completed.  The increment itself is relaxed: a release increment would add
// a write-back of the XCD's whole L2 (buffer_wbl2) per arrival, which the
// device-scope stores do not need (measured: +25 us per config-4 pick with
// 1792 arrivals, +250 us per config-4 top-n with 8192).  The last arriver
// still takes an acquire fence (a cache invalidate, cheap) before its loads.
__device__ __forceinline__ bool arrive_last(uint32_t* ctr, uint32_t total, uint32_t* flag) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = prev + 1u == total ? 1u : 0u;
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *flag = last;
  }
  __syncthreads();
  return *flag != 0u;
}
// Workgroup barrier for LDS traffic: waits for this wave's LDS (and scalar)
// operations only.  __syncthreads() also drains every outstanding global
// load and store first, which would stall the chunk phase until its whole
// stream has landed; the chunk phase tracks its global loads itself.
__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lane() { return threadIdx.x & 63; }
__device__ __forceinline__ uint32_t wave() { return threadIdx.x >> 6; }
// The block helpers are for NT-thread blocks, the size every kernel here
// launches with (a compile-time count spares a kernel-argument load before
// each use).
__device__ __forceinline__ uint32_t nwaves() { return (uint32_t)NW; }
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// ---------------------------------------------------------------------------
// Wave primitives on DPP lane moves (no LDS round trip).  A row is 16 lanes;
// row_shr:n shifts within a row, row_bcast:15 / row_bcast:31 carry a row's
// last lane into the following rows.  Lanes with no source receive `old`
// (the operation's identity), so the scans below are Hillis-Steele scans
// within rows followed by the two cross-row carries.
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, RM, 0xf, false);
}
constexpr int DPP_SHR1 = 0x111, DPP_SHR2 = 0x112, DPP_SHR4 = 0x114, DPP_SHR8 = 0x118;
constexpr int DPP_BC15 = 0x142, DPP_BC31 = 0x143;

// Inclusive sum scan in lane order.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += dpp<DPP_SHR1>(0u, v);
  v += dpp<DPP_SHR2>(0u, v);
  v += dpp<DPP_SHR4>(0u, v);
  v += dpp<DPP_SHR8>(0u, v);
  v += dpp<DPP_BC15, 0xa>(0u, v);
  v += dpp<DPP_BC31, 0xc>(0u, v);
  return v;
}
__device__ __forceinline__ uint32_t bcast63(uint32_t v) { return (uint32_t)__builtin_amdgcn_readlane((int)v, 63); }
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return bcast63(wave_scan_u32(v)); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp<DPP_SHR1>(0u, v));
  v = max(v, dpp<DPP_SHR2>(0u, v));
  v = max(v, dpp<DPP_SHR4>(0u, v));
  v = max(v, dpp<DPP_SHR8>(0u, v));
  v = max(v, dpp<DPP_BC15, 0xa>(0u, v));
  v = max(v, dpp<DPP_BC31, 0xc>(0u, v));
  return bcast63(v);
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  v |= dpp<DPP_SHR1>(0u, v);
  v |= dpp<DPP_SHR2>(0u, v);
  v |= dpp<DPP_SHR4>(0u, v);
  v |= dpp<DPP_SHR8>(0u, v);
  v |= dpp<DPP_BC15, 0xa>(0u, v);
  v |= dpp<DPP_BC31, 0xc>(0u, v);
  return bcast63(v);
}
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ unsigned long long dpp64(unsigned long long v) {
  const uint32_t lo = dpp<CTRL, RM>(0u, (uint32_t)v), hi = dpp<CTRL, RM>(0u, (uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  unsigned long long t;
  t = dpp64<DPP_SHR1>(v); v = t > v ? t : v;
  t = dpp64<DPP_SHR2>(v); v = t > v ? t : v;
  t = dpp64<DPP_SHR4>(v); v = t > v ? t : v;
  t = dpp64<DPP_SHR8>(v); v = t > v ? t : v;
  t = dpp64<DPP_BC15, 0xa>(v); v = t > v ? t : v;
  t = dpp64<DPP_BC31, 0xc>(v); v = t > v ? t : v;
  const uint32_t lo = bcast63((uint32_t)v), hi = bcast63((uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
// Sum over the wave (identity +0.0; addition order fixed by the lane tree).
__device__ __forceinline__ double wave_sum_f64(double v) {
  unsigned long long b;
  b = dpp64<DPP_SHR1>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR2>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR4>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR8>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_BC15, 0xa>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_BC31, 0xc>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  const unsigned long long r = __builtin_bit_cast(unsigned long long, v);
  const uint32_t lo = bcast63((uint32_t)r), hi = bcast63((uint32_t)(r >> 32));
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}


// f32 max / min / median of three as single VALU instructions, without the
// NaN-quieting canonicalisation the compiler puts before fmaxf/fminf.  For
// finite operands they equal the IEEE results; callers flag non-finite
// logits separately, so the value they give a NaN does not matter.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float vmin3(float a, float b, float c) {
  float r;
  __asm__("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float vmed3(float a, float b, float c) {
  float r;
  __asm__("v_med3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  __asm__("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Logit-bias and penalty stage for one token (BUILD-DEFINED semantics, f32,
// every operation rounded separately): bias, then for a token seen cnt > 0
// times the repetition penalty once (l < 0 ? l * rep : l / rep), then
// - cnt * freq, then - pres.  A bias of -inf suppresses the token (f32::MIN,
// as bias_and_penalize).
__device__ __forceinline__ float penalize_logit(float l, uint32_t cnt, bool has_bias, float bias, float rep,
                                                float pres, float freq) {
  if (has_bias && bias == -INFINITY) return kF32Min;
  if (has_bias) l = l + bias;
  if (cnt) {
    l = l < 0.0f ? l * rep : l / rep;
    const float cf = (float)cnt * freq;
    l = l - cf;
    l = l - pres;
  }
  return l;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

template <typename In>
struct Quad;
template <>
struct Quad<float> {
  using Raw = float4;
  __device__ static Raw load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ static void unpack(const Raw& r, float x[4]) { x[0] = r.x; x[1] = r.y; x[2] = r.z; x[3] = r.w; }
  __device__ static float one(const float* p) { return *p; }
};
template <>
struct Quad<uint16_t> {
  using Raw = uint2;
  __device__ static Raw load(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ static void unpack(const Raw& r, float x[4]) {
    x[0] = bf16_to_f32((uint16_t)(r.x & 0xffffu)); x[1] = bf16_to_f32((uint16_t)(r.x >> 16));
    x[2] = bf16_to_f32((uint16_t)(r.y & 0xffffu)); x[3] = bf16_to_f32((uint16_t)(r.y >> 16));
  }
  __device__ static float one(const uint16_t* p) { return bf16_to_f32(*p); }
};


// ---------------------------------------------------------------------------
// Block primitives with one barrier each.  `slot` is LDS scratch of the
// given shape; consecutive calls must alternate between two slots (the
// next-but-one call may overwrite a slot, by which time every thread has
// read it).

// Exclusive scan of u32 in thread order; *total receives the block total.
// The waves' totals are combined lane-parallel: lane w reads wave w's.
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* slot /* [NW] */, uint32_t* total) {
  const uint32_t inc = wave_scan_u32(v);
  if (lane() == 63) slot[wave()] = inc;
  lds_barrier();
  const uint32_t ws = wave_scan_u32(lane() < nwaves() ? slot[lane()] : 0u);
  *total = bcast63(ws);
  const uint32_t before = wave() ? (uint32_t)__builtin_amdgcn_readlane((int)ws, (int)(wave() - 1)) : 0u;
  return before + inc - v;
}

// Exclusive scan of u64 in thread order (exact); *total receives the block total.
__device__ __forceinline__ unsigned long long wave_scan_u64(unsigned long long v) {
  v += dpp64<DPP_SHR1>(v);
  v += dpp64<DPP_SHR2>(v);
  v += dpp64<DPP_SHR4>(v);
  v += dpp64<DPP_SHR8>(v);
  v += dpp64<DPP_BC15, 0xa>(v);
  v += dpp64<DPP_BC31, 0xc>(v);
  return v;
}
__device__ __forceinline__ unsigned long long readlane64(unsigned long long v, uint32_t l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, (int)l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), (int)l);
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long block_excl_scan_u64(unsigned long long v, unsigned long long* slot,
                                                                  unsigned long long* total) {
  const unsigned long long inc = wave_scan_u64(v);
  if (lane() == 63) slot[wave()] = inc;
  lds_barrier();
  const unsigned long long ws = wave_scan_u64(lane() < nwaves() ? slot[lane()] : 0ull);
  *total = readlane64(ws, 63);
  const unsigned long long before = wave() ? readlane64(ws, wave() - 1) : 0ull;
  return before + inc - v;
}

// Inclusive scan of f64 in thread order (the addition order: lanes in a
// fixed DPP tree, then waves in order); *total receives the block total.
__device__ __forceinline__ double wave_scan_f64(double v) {
  unsigned long long b;
  b = dpp64<DPP_SHR1>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR2>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR4>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_SHR8>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_BC15, 0xa>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  b = dpp64<DPP_BC31, 0xc>(__builtin_bit_cast(unsigned long long, v)); v += __builtin_bit_cast(double, b);
  return v;
}
__device__ __forceinline__ double block_incl_scan_f64(double v, double* slot /* [NW] */, double* total) {
  const double inc = wave_scan_f64(v);
  if (lane() == 63) slot[wave()] = inc;
  lds_barrier();
  const double ws = wave_scan_f64(lane() < nwaves() ? slot[lane()] : 0.0);
  const unsigned long long wb = __builtin_bit_cast(unsigned long long, ws);
  *total = __builtin_bit_cast(double, readlane64(wb, 63));
  const double before = wave() ? __builtin_bit_cast(double, readlane64(wb, wave() - 1)) : 0.0;
  return before + inc;
}

// ---------------------------------------------------------------------------
// Block-wide reductions and scans for NT-thread blocks (all threads
// participate and receive the result), on the DPP wave primitives: the
// waves' results meet in `red` (LDS, at least NW elements of the type) and
// one wave-wide pass combines them lane-parallel.
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ unsigned long long dpp64o(unsigned long long old, unsigned long long v) {
  const uint32_t lo = dpp<CTRL, RM>((uint32_t)old, (uint32_t)v);
  const uint32_t hi = dpp<CTRL, RM>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ double bcast63(double v) {
  return __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, v), 63));
}
__device__ __forceinline__ float bcast63(float v) { return __uint_as_float(bcast63(__float_as_uint(v))); }
__device__ __forceinline__ double readlane_t(double v, uint32_t l) {
  return __builtin_bit_cast(double, readlane64(__builtin_bit_cast(unsigned long long, v), l));
}
__device__ __forceinline__ uint32_t readlane_t(uint32_t v, uint32_t l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}
// f32 and f64 maxima: lanes with no source read -inf; `t > v ? t : v` as the
// scalar code compares
__device__ __forceinline__ float wave_max_f32(float v) {
  const uint32_t ninf = 0xff800000u;
  float t;
  t = __uint_as_float(dpp<DPP_SHR1>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  t = __uint_as_float(dpp<DPP_SHR2>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  t = __uint_as_float(dpp<DPP_SHR4>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  t = __uint_as_float(dpp<DPP_SHR8>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  t = __uint_as_float(dpp<DPP_BC15, 0xa>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  t = __uint_as_float(dpp<DPP_BC31, 0xc>(ninf, __float_as_uint(v))); v = t > v ? t : v;
  return bcast63(v);
}
__device__ __forceinline__ double wave_max_f64(double v) {
  const unsigned long long ninf = 0xfff0000000000000ull;
  double t;
#define MXS_MAXSTEP(C, R) \
  t = __builtin_bit_cast(double, dpp64o<C, R>(ninf, __builtin_bit_cast(unsigned long long, v))); v = t > v ? t : v;
  MXS_MAXSTEP(DPP_SHR1, 0xf) MXS_MAXSTEP(DPP_SHR2, 0xf) MXS_MAXSTEP(DPP_SHR4, 0xf) MXS_MAXSTEP(DPP_SHR8, 0xf)
  MXS_MAXSTEP(DPP_BC15, 0xa) MXS_MAXSTEP(DPP_BC31, 0xc)
#undef MXS_MAXSTEP
  return bcast63(v);
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += __uint_as_float(dpp<DPP_SHR1>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<DPP_SHR2>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<DPP_SHR4>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<DPP_SHR8>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<DPP_BC15, 0xa>(0u, __float_as_uint(v)));
  v += __uint_as_float(dpp<DPP_BC31, 0xc>(0u, __float_as_uint(v)));
  return bcast63(v);
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) { return wave_sum_u32(v); }
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32(v); }
__device__ __forceinline__ double wave_sum(double v) { return wave_sum_f64(v); }
__device__ __forceinline__ uint32_t wave_max(uint32_t v) { return wave_max_u32(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_max_f32(v); }
__device__ __forceinline__ double wave_max(double v) { return wave_max_f64(v); }
__device__ __forceinline__ uint32_t wave_scan(uint32_t v) { return wave_scan_u32(v); }
__device__ __forceinline__ double wave_scan(double v) { return wave_scan_f64(v); }
template <typename T>
__device__ __forceinline__ T max_identity() { return T(0); }
template <>
__device__ __forceinline__ float max_identity<float>() { return -INFINITY; }
template <>
__device__ __forceinline__ double max_identity<double>() { return -INFINITY; }

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  const T s = wave_sum(lane() < nwaves() ? red[lane()] : T(0));
  __syncthreads();
  return s;
}
template <typename T>
__device__ __forceinline__ T block_max(T v, T* red) {
  v = wave_max(v);
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  const T s = wave_max(lane() < nwaves() ? red[lane()] : max_identity<T>());
  __syncthreads();
  return s;
}
// Inclusive scan in thread order; *total receives the block total.
template <typename T>
__device__ __forceinline__ T block_scan_incl(T v, T* red, T* total) {
  v = wave_scan(v);
  if (lane() == 63) red[wave()] = v;
  __syncthreads();
  const T ws = wave_scan(lane() < nwaves() ? red[lane()] : T(0));
  const T before = wave() ? readlane_t(ws, wave() - 1u) : T(0);
  *total = readlane_t(ws, nwaves() - 1u);
  __syncthreads();
  return before + v;
}
// As block_scan_incl, and *excl receives the exclusive prefix computed so
// that it is bit-identical to the previous thread's inclusive value: the
// per-thread intervals (excl, incl] then tile (0, total] with no gap or
// overlap even in floating point.
template <typename T>
__device__ __forceinline__ T block_scan_pair(T v, T* red, T* excl, T* total) {
  const uint32_t l = lane();
  v = wave_scan(v);
  const T prev = __shfl_up(v, 1);
  if (l == 63) red[wave()] = v;
  __syncthreads();
  const T ws = wave_scan(l < nwaves() ? red[l] : T(0));
  const T before = wave() ? readlane_t(ws, wave() - 1u) : T(0);
  *total = readlane_t(ws, nwaves() - 1u);
  __syncthreads();
  *excl = l == 0 ? before : before + prev;
  return before + v;
}

// Two or three reductions for the price of one barrier pair: the block's
// sum of s, maximum of a and maximum of b (all threads receive them).
__device__ __forceinline__ void block_sum_max_max(double* s, double* a, float* b, double (*rd)[2], float* rf) {
  double vs = wave_sum(*s), va = wave_max(*a);
  float vb = wave_max(*b);
  if (lane() == 0) { rd[wave()][0] = vs; rd[wave()][1] = va; rf[wave()] = vb; }
  __syncthreads();
  const bool l = lane() < nwaves();
  *s = wave_sum(l ? rd[lane()][0] : 0.0);
  *a = wave_max(l ? rd[lane()][1] : -INFINITY);
  *b = wave_max(l ? rf[lane()] : -INFINITY);
  __syncthreads();
}
// block_scan_pair of an f64 together with an inclusive u32 scan (one
// barrier pair for both).
__device__ __forceinline__ double block_scan_pair_du(double v, uint32_t n, double* red_d, uint32_t* red_u, double* excl,
                                                     double* total, uint32_t* nincl, uint32_t* ntotal) {
  const uint32_t l = lane();
  v = wave_scan(v);
  n = wave_scan(n);
  const double prev = __shfl_up(v, 1);
  if (l == 63) { red_d[wave()] = v; red_u[wave()] = n; }
  __syncthreads();
  const double ws = wave_scan(l < nwaves() ? red_d[l] : 0.0);
  const uint32_t wn = wave_scan(l < nwaves() ? red_u[l] : 0u);
  const double before = wave() ? readlane_t(ws, wave() - 1u) : 0.0;
  const uint32_t nbefore = wave() ? readlane_t(wn, wave() - 1u) : 0u;
  *total = readlane_t(ws, nwaves() - 1u);
  *ntotal = readlane_t(wn, nwaves() - 1u);
  __syncthreads();
  *excl = l == 0 ? before : before + prev;
  *nincl = nbefore + n;
  return before + v;
}

constexpr int NBR = 2048;                 // radix-select bins (11 bits)

// LDS word of histogram bin b.  Lane j of a wave owns the 32 bins
// [NBR - 32 (j + 1), NBR - 32 j) and reads them as eight 4-bin groups; the
// groups are stored transposed (group g of owner o at word 256 g + 4 o), so
// the 64 lanes' 16-byte reads of one group index are consecutive and the
// bin search is free of bank conflicts.
__device__ __forceinline__ uint32_t hpos(uint32_t b) { return ((b & 31u) >> 2) * 256u + (b >> 5) * 4u + (b & 3u); }

// The k-th largest (k >= 1) of the active 32-bit keys the workgroup's
// threads hold (up to R each; bit r of `act` marks key[r] active), by three
// radix passes (11, 11 and 10 bits) over one NBR-word LDS histogram, which it
// clears before each pass; *above receives how many active keys are larger.
// Needs at least k active keys.
template <int R>
__device__ __forceinline__ uint32_t block_kth_largest(const uint32_t (&key)[R], uint64_t act, uint32_t k, uint32_t* hist,
                                      uint32_t* above) {
  uint32_t prefix = 0, pmask = 0, need = k, abv = 0;
  const uint32_t own = 4u * (63u - lane());   // this lane's word within a group row
#pragma unroll 1
  for (int p = 0; p < 3; ++p) {
    const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0);
    const uint32_t dmask = p == 2 ? 0x3ffu : 0x7ffu;
    uint32_t* h = hist;
    __syncthreads();   // every wave has finished reading the previous pass's counts
    for (uint32_t t = threadIdx.x; t < (uint32_t)NBR / 4u; t += blockDim.x)
      reinterpret_cast<uint4*>(h)[t] = make_uint4(0u, 0u, 0u, 0u);
    lds_barrier();
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (((act >> r) & 1ull) && (key[r] & pmask) == prefix) atomicAdd(&h[hpos((key[r] >> sh) & dmask)], 1u);
    lds_barrier();
    // Every wave finds the bin itself, each lane over its own 32 bins from
    // the highest (group 7 down to group 0).
    const uint32_t hi = (uint32_t)NBR - 32u * lane();
    uint32_t c[32];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const uint4 v = *reinterpret_cast<const uint4*>(&h[(uint32_t)(7 - g) * 256u + own]);
      c[4 * g + 0] = v.w; c[4 * g + 1] = v.z; c[4 * g + 2] = v.y; c[4 * g + 3] = v.x;
    }
    uint32_t s = 0;
#pragma unroll
    for (int q = 0; q < 32; ++q) s += c[q];
    const uint32_t inc = wave_scan_u32(s);
    const uint64_t reach = __builtin_amdgcn_ballot_w64(inc >= need);
    if (!reach) break;   // fewer than k active keys: the caller's contract is broken
    const uint32_t L = (uint32_t)__builtin_ctzll(reach);
    // the crossing bin inside lane L's range (every lane walks its own)
    uint32_t run = inc - s, bin = hi - 1u, before = run;
    bool found = false;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      if (!found && run + c[q] >= need) {
        found = true;
        bin = hi - 1u - (uint32_t)q;
        before = run;
      }
      run += c[q];
    }
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)bin, (int)L);
    const uint32_t cnt_above = (uint32_t)__builtin_amdgcn_readlane((int)before, (int)L);
    need -= cnt_above;
    abv += cnt_above;
    prefix |= b << sh;
    pmask |= dmask << sh;
  }
  *above = abv;
  return prefix;
}

}  // namespace mxs
