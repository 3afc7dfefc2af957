// mx_spec.hip -- speculative-decoding verification (mxs_spec_verify of
// include/mx_sampler.h).
//
// Reference semantics (arclabs561/metallix):
//   accept_or_resample  crates/core/engine/src/speculative.rs:369-429
//   categorical         crates/core/engine/src/speculative.rs:431-444
//   the position walk   speculative_step / accept_and_roll_back (:202-227, :318-347)
//   bonus draw          sample_categorical, crates/core/engine/src/sampling.rs:56-158
// For each row, position j < K carries target and draft logits; both become
// f64 weights exp((l - row max) / T).  Position j accepts the drafted token
// d when u_accept < (t[d] / sum t) / (q[d] / sum q); the first rejection
// emits a draw from max(0, t / sum t - q / sum q) and stops; when every draft
// is accepted, the bonus token is sample_categorical over target row K.
//
// Two launches on the context's stream.
//   Pass 1, one workgroup per (row, chunk), streaming that chunk of all the
//   row's 2K + 1 logit rows: per row of logits the chunk's maximum and
//   weight sum, the weights from the f32 exp2 summed in f64 (a few 2^-23
//   relative, plus a term in sum w |y| for the rounding of y; spec_sum_err).
//   The row's last workgroup decides acceptance at every position: the ratio
//   p/q needs only that relative accuracy to be certified.
//   Pass 2, one workgroup per (row, chunk): the first rejected position (or
//   the bonus position) from pass 1's verdicts, then the drawn
//   distribution's weights at that position in f64 (exp_neg16_t, its
//   16-entry table read from LDS without bank conflicts).  The residual
//   max(0, t_i / sum t - q_i / sum q) needs the totals to f64 accuracy, which
//   pass 1 does not have; its approximate totals only classify each token's
//   sign with a margin, so that each 256-token segment stores the exact sums
//   of t_i and q_i over its positive tokens and the residual mass follows
//   once the row's exact totals (summed here too) are known.  Tokens inside
//   the margin (|p_i - q_i| within a few 2^-22 of p_i + q_i) count as 0 and
//   their possible mass joins the error bound.  The row's last chunk locates
//   the draw: the segment by a prefix over segment masses, then the token by
//   re-deriving the segment's 256 residual weights in f64.
// Every comparison against a reference f64 sum is taken only when a
// rigorous error bound certifies it; otherwise the row is reported
// uncertified (status 1) with the device's decision.

#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

#include <type_traits>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_math.h"

namespace mxs {

constexpr int SP = 5;                 // quads per thread per chunk (vocabularies past SMAXC default chunks)
constexpr int SMAXC = 128;            // chunks per row
constexpr uint32_t SPEC_KMAX = 8;     // draft positions per row
constexpr uint32_t SPART = 5;         // pass 2's per-chunk partials

struct SpecStat {                     // per (row, position, chunk)
  float tmax, dmax, tmin;
  uint32_t tflags, dflags;            // a non-finite target / draft logit
  float te, de;                       // sums of w |y|, y = (l - chunk max) log2(e) / T
  uint32_t pad;
  double tsum, dsum;                  // sums of exp((l - chunk max) / T)
};

struct SpecPos {                      // per (row, position): pass 1's verdict
  int32_t err;                        // this position's error status (0: none)
  int32_t accept;                     // 1: drafted token accepted
  int32_t unc;                        // the decision is not certified
  int32_t pad;
  float mt, md;                       // row maxima of target and draft
  double tt, td;                      // totals of exp((l - row max) / T), weight2 terms
  double tterr, tderr;                // bounds on |total - reference total|
};

struct SpecArgs {
  const float* target;                // [rows][K + 1][V]
  const float* draft;                 // [rows][K][V]
  uint32_t rows, K, V, C, CH, per;
  const int32_t* tok;                 // [rows][K]
  const double* T;                    // [rows]
  const double* ua;                   // [rows][K]
  const double* ur;                   // [rows][K]
  const double* ub;                   // [rows]
  int32_t* out_tokens;                // [rows][K + 1]
  int32_t* out_count;
  int32_t* out_accepted;
  int32_t* status;
  uint32_t* ctr1;                     // [rows * (SPEC_KMAX + 1)], CTR_STRIDE words apart
  uint32_t* ctr2;                     // [rows], CTR_STRIDE words apart
  SpecStat* stat;                     // [rows * (SPEC_KMAX + 1) * SMAXC]
  SpecPos* pos;                       // [rows * (SPEC_KMAX + 1)]
  uint32_t C2, CH2, per2;             // pass 2's chunk layout
  // pass 2, per row (seg_stride doubles): the segments' positive sums
  // (sum t, sum q) at [2 s, 2 s + 1], s = chunk * per2 * NW + slice * NW +
  // wave in token order, then at 2 nseg_cap + SPART chunk the chunk's
  // partials: sum t, sum q, margin mass, positive sum t, positive sum q
  double* seg;
  uint64_t seg_stride;
  uint32_t nseg_cap;
};

struct SpecSmem {
  double etab[32];                    // exp_neg16_t's tables: 2^(j/16), hi then lo
  SpecPos ps[SPEC_KMAX + 1];
  uint32_t red_u[4][NW];
  double red_d[8][NW];
  double s_d[4];
  uint32_t s_u[8];
};

// Pass 1's per (item, wave) statistics.
struct WaveStat {
  float m, mn;                        // the wave's maximum and minimum
  float e;                            // sum of w |y|, y relative to the wave maximum
  uint32_t bad;                       // a non-finite logit
  double s;                           // sum of weights relative to the wave maximum
};
struct SpecSmem1 {
  WaveStat w[NW][2 * SPEC_KMAX + 1];  // [wave][item]: the per-item combine reads consecutive entries
  uint32_t s_u[4];
};

// Weight exp(x) of x = (l - M) / T <= 0 as 2^y, y = (l - M) c2 with c2 =
// log2(e) / T, formed in f64 and clamped at -1000 (2^-1000 is 0 in f32):
// the f32 exp2 of y's f32 head corrected by its tail (|tail| <= 2^-24 |head|,
// one fma).  Within 2^-22 relative of 2^y where the result is in f32's
// normal range, within 2^-125 absolute below it; the maximum weighs exactly
// 1 and l = -inf weighs 0.
__device__ __forceinline__ double weight2(float l, double M, double c2) {
  const double y = fmax(((double)l - M) * c2, -1000.0);
  const float yh = (float)y;
  const float yl = (float)(y - (double)yh);
  const float eh = __builtin_amdgcn_exp2f(yh);
  return (double)__builtin_fmaf(eh, yl * 0.69314718f, eh);
}

// Bound on |device sum - reference sum| for n weights exp(x), x = (l - M) / T
// <= 0, both in f64 (4 ulp per term against the reference's exp), summed in
// different orders; the rounding of x (x e^x <= 1/e per term).
__device__ __forceinline__ double weight_sum_err(double s, uint32_t n) {
  return (2.0 * (double)n + 16.0) * U * s * 1.0001 + 1.5 * (double)n * U + 1e-300;
}
// Bound on |device total - reference total| for a row total s of n
// weights exp(x), x = (l - M) / T, from pass 1's weights: each 2^y with y =
// (l - wave max) c2 rounded three times in f32 (3.0001 2^-24 |y| relative, so
// ln2 3.0001 2^-24 |y| w in the weight), exp2f (2^-23), the 4-term f32 sums
// (3 2^-24), and the wave-to-chunk factor (the same, its |y| joining the
// token's in e = sum of w |y| with y relative to the chunk maximum; weight2
// terms instead: 2^-22 each, e = 0), 2^-21 s in all; weights below f32's
// normal range 2^-125 each; f64 sums in different orders and the rounding of
// x as weight_sum_err.
__device__ __forceinline__ double spec_sum_err(double s, double e, uint32_t n) {
  return (0x1p-21 + (2.0 * (double)n + 16.0) * U) * s * 1.0001 +
         0.6931471805599453 * 3.0001 * 0x1p-24 * e * 1.01 + (double)n * (2.5 * U + 0x1p-125) + 1e-300;
}

template <bool ALIGNED>
__device__ __forceinline__ void load_quad(const float* p, uint32_t e0, uint32_t c1, float x[4]) {
  if (ALIGNED) {
    const float4 v = *reinterpret_cast<const float4*>(p + e0);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = p[e0 + (uint32_t)e < c1 ? e0 + (uint32_t)e : e0];
  }
}

__device__ __forceinline__ bool temperature_ok(double T) { return T > 0.0 && isfinite(T); }
__device__ __forceinline__ bool uniform_ok(double u) { return isfinite(u) && u >= 0.0 && u < 1.0; }
// 1 / T capped at 2^1000: below T = 2^-1000 every weight but the maximum's
// is 0 either way (|l - M| >= 2^-149 otherwise), and the maximum's x stays 0
// instead of 0 * inf.
__device__ __forceinline__ double inv_temperature(double T) {
  return temperature_ok(T) ? fmin(1.0 / T, 0x1p1000) : 0.0;
}

// ---------------------------------------------------------------------------
// Pass 1: one workgroup per (row, chunk) streams the chunk of the row's
// 2K + 1 logit rows (items: target position j at j <= K, draft position j at
// K + 1 + j), two items in flight per thread.  Each wave reduces its part of
// an item to statistics on its own (no barrier per item); the workgroup
// combines them per item at its end.  The row's last workgroup takes the
// K + 1 verdicts, wave j position j.
template <bool ALIGNED, int Q>
__global__ __launch_bounds__(NT) void spec_pass1(SpecArgs A) {
  __shared__ SpecSmem1 S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  const uint32_t K = A.K, V = A.V, nit = 2u * K + 1u;
  const uint32_t c0 = chunk * A.CH, c1 = min(V, c0 + A.CH);
  const double T = A.T[row];
  const bool tok_T = temperature_ok(T);
  const double invT = inv_temperature(T);
  const double c2 = invT * 1.4426950408889634;
  const bool f32w = c2 <= 0x1p126;   // y in f32 (c2 a normal f32); weight2's f64 y above
  const float c2f = (float)c2;
  const float* tb = A.target + (uint64_t)row * (K + 1u) * V;
  const float* db = A.draft + (uint64_t)row * K * V;

  // wave j's position for the verdict, should this workgroup take them:
  // the drafted token, its uniforms and logits (wave-uniform, so scalar
  // loads into scalar registers, off the verdict's critical path)
  const uint32_t wj = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave());
  int32_t d = -1;
  double ua = 0.0, ur = 0.0;
  float tpd = 0.0f, dpd = 0.0f;
  if (wj < K) {
    d = A.tok[(uint64_t)row * K + wj];
    ua = A.ua[(uint64_t)row * K + wj];
    ur = A.ur[(uint64_t)row * K + wj];
    if (d >= 0 && (uint32_t)d < V) {
      tpd = tb[(uint64_t)wj * V + (uint32_t)d];
      dpd = db[(uint64_t)wj * V + (uint32_t)d];
    }
  }

  auto item_row = [&](uint32_t it) -> const float* {   // past the last item: the last item again
    it = min(it, nit - 1u);
    return it <= K ? tb + (uint64_t)it * V : db + (uint64_t)(it - K - 1u) * V;
  };
  auto load = [&](float (&x)[Q][4], const float* p) {
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
      load_quad<ALIGNED>(p, e0 < c1 ? e0 : c0, c1, x[i]);
    }
  };
  // one item: non-finite flag, wave maximum (and minimum, for the bonus
  // position), the wave's sum of weights relative to its maximum and the
  // sum of w |y| for the bound.  FULL: a whole chunk (every chunk but a
  // row's last), whose quads 0..Q-2 are in range ((per - 1) SLICE < CH); only
  // the last quad is masked.
  auto process = [&](auto full_tag, float (&x)[Q][4], uint32_t it) {
    constexpr bool FULL = decltype(full_tag)::value;
    float mx = -INFINITY, mn = INFINITY;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool inr = (FULL && i < Q - 1) || e0 + (uint32_t)e < c1;
        bad = bad || (inr && !__builtin_isfinite(x[i][e]));
        if (!(FULL && i < Q - 1)) x[i][e] = inr ? x[i][e] : -INFINITY;
        mx = fmaxf(mx, x[i][e]);
      }
    }
    if (it == K) {
#pragma unroll
      for (int i = 0; i < Q; ++i) {
        const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
        for (int e = 0; e < 4; ++e) mn = ((FULL && i < Q - 1) || e0 + (uint32_t)e < c1) ? fminf(mn, x[i][e]) : mn;
      }
    }
    const float Mw = okey_value(wave_max_u32(okey(mx)));
    const float Mn = it == K ? okey_value(~wave_max_u32(~okey(mn))) : INFINITY;
    const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
    double s = 0.0;
    float E = 0.0f;
    if (tok_T && !wbad && Mw > -INFINITY) {
      if (f32w) {
        // every in-range logit is finite here; out-of-range ones are -inf
        // (weight 0, and w y taken as 0)
#pragma unroll
        for (int i = 0; i < Q; ++i) {
          float q = 0.0f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float y = (x[i][e] - Mw) * c2f;
            const float w = __builtin_amdgcn_exp2f(y);
            q += w;
            E = fmaf(w, (FULL && i < Q - 1) ? y : fmaxf(y, -1e30f), E);
          }
          s += (double)q;
        }
        E = -E;
      } else {
#pragma unroll
        for (int i = 0; i < Q; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) s += weight2(x[i][e], (double)Mw, c2);
      }
    }
    s = wave_sum_f64(s);
    E = wave_sum_f32(E);
    if (lane() == 0) {
      WaveStat& ws = S.w[wave()][it];
      ws.m = Mw;
      ws.mn = Mn;
      ws.e = E;
      ws.bad = wbad ? 1u : 0u;
      ws.s = s;
    }
  };
  const bool full = c1 - c0 == A.CH;
  using FullT = std::integral_constant<bool, true>;
  using PartT = std::integral_constant<bool, false>;

  float xa[Q][4], xb[Q][4];
  load(xa, item_row(0u));
  load(xb, item_row(1u));
  if (full) {
    for (uint32_t it = 0; it < nit; it += 2u) {
      process(FullT(), xa, it);
      load(xa, item_row(it + 2u));
      if (it + 1u < nit) process(FullT(), xb, it + 1u);
      load(xb, item_row(it + 3u));
    }
  } else {
    for (uint32_t it = 0; it < nit; it += 2u) {
      process(PartT(), xa, it);
      load(xa, item_row(it + 2u));
      if (it + 1u < nit) process(PartT(), xb, it + 1u);
      load(xb, item_row(it + 3u));
    }
  }
  lds_barrier();

  // per item, the chunk's statistics from the waves': maximum, minimum,
  // flag, and the waves' sums rescaled to the chunk maximum (their E with
  // the rescale's own |y|)
  if (tid < nit) {
    const uint32_t it = tid;
    float M = -INFINITY, Mn = INFINITY;
    uint32_t bad = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      M = fmaxf(M, S.w[w][it].m);
      Mn = fminf(Mn, S.w[w][it].mn);
      bad |= S.w[w][it].bad;
    }
    double s = 0.0;
    float E = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const WaveStat& ws = S.w[w][it];
      if (ws.s > 0.0) {
        if (f32w) {
          const float dy = (ws.m - M) * c2f;
          const float f = __builtin_amdgcn_exp2f(dy);
          s += ws.s * (double)f;
          E += f * (ws.e + (float)ws.s * fminf(-dy, 1e30f));
        } else {
          s += ws.s * weight2(ws.m, (double)M, c2);
        }
      }
    }
    const uint32_t j = it <= K ? it : it - K - 1u;
    SpecStat* st = &A.stat[((uint64_t)row * (SPEC_KMAX + 1) + j) * SMAXC + chunk];
    if (it <= K) {
      st_dev(&st->tmax, M);
      st_dev(&st->tmin, Mn);
      st_dev(&st->tflags, bad);
      st_dev(&st->tsum, s);
      st_dev(&st->te, E);
    } else {
      st_dev(&st->dmax, M);
      st_dev(&st->dflags, bad);
      st_dev(&st->dsum, s);
      st_dev(&st->de, E);
    }
  }
  if (!arrive_last(&A.ctr1[row * (SPEC_KMAX + 1) * CTR_STRIDE], A.C, &S.s_u[0])) return;

  // ---- the verdicts: wave j reduces position j's chunk statistics (two
  // chunks per lane, C <= SMAXC = 128), lane 0 decides
  if (wj > K) return;
  const uint32_t j = wj;
  const bool has_draft = j < K;
  const uint32_t slot = row * (SPEC_KMAX + 1) + j;
  const uint32_t C = A.C;
  float cmt[2], cmd[2], cte[2], cde[2];
  double cts[2], cds[2];
  uint32_t fl = 0u, kt = 0u, kd = 0u, kn = 0u;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t q = lane() + 64u * (uint32_t)h;
    cmt[h] = cmd[h] = -INFINITY;
    cte[h] = cde[h] = 0.0f;
    cts[h] = cds[h] = 0.0;
    if (q < C) {
      const SpecStat* st = &A.stat[(uint64_t)slot * SMAXC + q];
      cmt[h] = ld_dev(&st->tmax);
      kn = max(kn, ~okey(ld_dev(&st->tmin)));
      fl |= ld_dev(&st->tflags);
      cts[h] = ld_dev(&st->tsum);
      cte[h] = ld_dev(&st->te);
      if (has_draft) {
        cmd[h] = ld_dev(&st->dmax);
        fl |= ld_dev(&st->dflags) << 1;
        cds[h] = ld_dev(&st->dsum);
        cde[h] = ld_dev(&st->de);
      }
      kt = max(kt, okey(cmt[h]));
      kd = max(kd, okey(cmd[h]));
    }
  }
  fl = wave_or_u32(fl);
  const float Mt = okey_value(wave_max_u32(kt)), Md = okey_value(wave_max_u32(kd));
  const float Mn = okey_value(~wave_max_u32(kn));
  // totals: the chunk sums rescaled from the chunk maxima to the row maxima
  double tt = 0.0, td = 0.0, et = 0.0, ed = 0.0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const double ft = exp_neg_p(((double)cmt[h] - (double)Mt) * invT);
    const double fd = exp_neg_p(((double)cmd[h] - (double)Md) * invT);
    tt += cts[h] * ft;
    et += (double)cte[h] * ft;
    td += cds[h] * fd;
    ed += (double)cde[h] * fd;
  }
  tt = wave_sum_f64(tt);
  et = wave_sum_f64(et);
  if (has_draft) {
    td = wave_sum_f64(td);
    ed = wave_sum_f64(ed);
  }
  if (lane() != 0) return;
  const uint32_t nsum = V + C * NW;
  SpecPos P;
  P.err = 0;
  P.accept = 0;
  P.unc = 0;
  P.pad = 0;
  P.mt = Mt;
  P.md = Md;
  P.tt = P.td = P.tterr = P.tderr = 0.0;
  if (!tok_T) {
    P.err = MXS_ROW_INVALID_TEMPERATURE;
  } else if (has_draft) {
    if (fl) P.err = MXS_ROW_NON_FINITE_LOGIT;
    else if (d < 0) P.err = MXS_ROW_TOKEN_OUT_OF_RANGE;
    else if (!uniform_ok(ua) || !uniform_ok(ur)) P.err = MXS_ROW_INVALID_UNIFORM;
    else if ((uint32_t)d >= V) P.err = MXS_ROW_TOKEN_OUT_OF_RANGE;
    if (!P.err) {
      P.tt = tt;
      P.td = td;
      P.tterr = spec_sum_err(tt, et, nsum);
      P.tderr = spec_sum_err(td, ed, nsum);
      const double xt = ((double)tpd - (double)Mt) * invT;
      const double xq = ((double)dpd - (double)Md) * invT;
      const double wt = exp_neg_p(xt);
      const double wd = exp_neg_p(xq);
      if (wd <= 0.0) {
        // the reference's q <= 0 rejection; near the f64 underflow edge the
        // two exp implementations may disagree
        P.err = MXS_ROW_PROBABILITIES;
        if (xq > -746.0) P.unc = 1;
      } else {
        const double p = wt / tt, qq = wd / td;
        const double ratio = p / qq;
        // relative error of the ratio: both weights (exp 2 ulp and the
        // rounding of x, 4 ulp each with margin), both totals, the divisions
        const double rel = 16.0 * U + P.tterr / tt + P.tderr / td + 2e-15 * (fabs(xq) + fabs(xt) + 1.0);
        P.accept = ua < ratio ? 1 : 0;
        if (fabs(ua - ratio) <= rel * ratio + 1e-300) P.unc = 1;
        if (xq < -700.0) P.unc = 1;   // q in the subnormal range
      }
    }
  } else {
    // bonus position: sample_categorical's checks in its order
    if (!uniform_ok(A.ub[row])) P.err = MXS_ROW_INVALID_UNIFORM;
    else if (fl & 1u) P.err = MXS_ROW_NON_FINITE_LOGIT;
    else if (!isfinite(((double)Mn - (double)Mt) / T)) P.err = MXS_ROW_INVALID_TEMPERATURE;
    else {
      P.tt = tt;
      P.tterr = spec_sum_err(tt, et, nsum);
    }
  }
  SpecPos* out = &A.pos[slot];
  st_dev(reinterpret_cast<uint32_t*>(&out->err), (uint32_t)P.err);
  st_dev(reinterpret_cast<uint32_t*>(&out->accept), (uint32_t)P.accept);
  st_dev(reinterpret_cast<uint32_t*>(&out->unc), (uint32_t)P.unc);
  st_dev(&out->mt, P.mt);
  st_dev(&out->md, P.md);
  st_dev(&out->tt, P.tt);
  st_dev(&out->td, P.td);
  st_dev(&out->tterr, P.tterr);
  st_dev(&out->tderr, P.tderr);
}

// The row's plan after pass 1: the position to draw at (K: the bonus), the
// error ending the walk (0: none), and whether a decision was uncertified.
struct Plan {
  uint32_t r;
  int32_t err;
  bool unc;
};
__device__ Plan row_plan(const SpecPos* ps, uint32_t K) {
  Plan pl{K, 0, false};
  for (uint32_t j = 0; j < K; ++j) {
    if (ps[j].err) { pl.r = j; pl.err = ps[j].err; pl.unc = pl.unc || ps[j].unc; return pl; }
    pl.unc = pl.unc || ps[j].unc;
    if (!ps[j].accept) { pl.r = j; return pl; }
  }
  if (ps[K].err) pl.err = ps[K].err;
  return pl;
}

// Margin of pass 2's sign classification: |(t_i a' - q_i b') - (p_i - q_i)|
// <= rho (t_i a' + q_i b') with a' = 1 / tt', b' = 1 / td' from pass 1's
// totals; their relative errors, the f64 weights' (4 ulp and 2 ulp |x| for
// the rounding of x, |x| <= 746) and the products' roundings.
__device__ __forceinline__ double sign_margin(const SpecPos& P) {
  return 1.01 * (P.tterr / P.tt + P.tderr / P.td) + 2000.0 * U;
}

// ---------------------------------------------------------------------------
// Pass 2: the drawn distribution's segment and chunk sums; the row's last
// chunk draws.
template <bool ALIGNED, int Q>
__global__ __launch_bounds__(NT) void spec_pass2(SpecArgs A) {
  __shared__ SpecSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  const uint32_t K = A.K, V = A.V;
  if (tid < 32u) S.etab[tid] = tid < 16u ? kExp2Tab[4u * tid] : kExp2TabLo[4u * (tid - 16u)];
  for (uint32_t j = tid; j <= K; j += NT) {
    const SpecPos* src = &A.pos[row * (SPEC_KMAX + 1) + j];
    SpecPos P;
    P.err = (int32_t)ld_dev(reinterpret_cast<const uint32_t*>(&src->err));
    P.accept = (int32_t)ld_dev(reinterpret_cast<const uint32_t*>(&src->accept));
    P.unc = (int32_t)ld_dev(reinterpret_cast<const uint32_t*>(&src->unc));
    P.pad = 0;
    P.mt = ld_dev(&src->mt);
    P.md = ld_dev(&src->md);
    P.tt = ld_dev(&src->tt);
    P.td = ld_dev(&src->td);
    P.tterr = ld_dev(&src->tterr);
    P.tderr = ld_dev(&src->tderr);
    S.ps[j] = P;
  }
  __syncthreads();
  const Plan pl = row_plan(S.ps, K);
  const bool bonus = pl.r == K;
  const double invT = inv_temperature(A.T[row]);
  const uint32_t C = A.C2, CH = A.CH2, per = A.per2;
  const uint32_t c0 = chunk * CH, c1 = min(V, c0 + CH);
  const uint32_t spc = per * NW;                          // segments per chunk
  double* rs = A.seg + (uint64_t)row * A.seg_stride;     // [2 * nseg_cap] segments
  double* parts = rs + 2u * (uint64_t)A.nseg_cap;        // [SPART * C] chunk partials
  const float* tp = A.target + ((uint64_t)row * (K + 1u) + pl.r) * V;
  const float* dp = A.draft + ((uint64_t)row * K + (bonus ? 0u : pl.r)) * V;
  if (!pl.err) {
    const SpecPos& P = S.ps[pl.r];
    const double ra = bonus ? 1.0 : 1.0 / P.tt, rb = bonus ? 0.0 : 1.0 / P.td;
    const double rho = bonus ? 0.0 : sign_margin(P);
    float t[Q][4], q[Q][4];
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
      const uint32_t es = e0 < c1 ? e0 : c0;
      q[i][0] = q[i][1] = q[i][2] = q[i][3] = 0.0f;
      load_quad<ALIGNED>(tp, es, c1, t[i]);
      if (!bonus) load_quad<ALIGNED>(dp, es, c1, q[i]);
    }
    // per thread: sum t, sum q, margin mass, positive sum t, positive sum q
    double pt = 0.0, pd = 0.0, pe = 0.0, pa = 0.0, pb = 0.0;
#pragma unroll
    for (int i = 0; i < Q; ++i) {
      if (i < (int)per) {
        const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
        double sa = 0.0, sb = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (e0 + (uint32_t)e < c1) {
            const double wt = exp_neg16_t(((double)t[i][e] - (double)P.mt) * invT, S.etab, S.etab + 16);
            pt += wt;
            if (bonus) {
              sa += wt;
            } else {
              const double wq = exp_neg16_t(((double)q[i][e] - (double)P.md) * invT, S.etab, S.etab + 16);
              pd += wq;
              const double x = wt * ra, y = wq * rb;
              const double dd = x - y, ss = x + y;
              if (dd > rho * ss) { sa += wt; sb += wq; }
              else if (dd >= -(rho * ss)) pe += ss;
            }
          }
        }
        pa += sa;
        pb += sb;
        sa = wave_sum_f64(sa);
        if (!bonus) sb = wave_sum_f64(sb);
        if (lane() == 0) {
          double* o = rs + 2u * (chunk * spc + (uint32_t)i * NW + wave());
          st_dev(o, sa);
          st_dev(o + 1, sb);
        }
      }
    }
    // the chunk's partials: wave sums, then lanes f < SPART of wave 0 add
    // the waves' values of partial f
    pt = wave_sum_f64(pt);
    pa = wave_sum_f64(pa);
    if (!bonus) { pd = wave_sum_f64(pd); pe = wave_sum_f64(pe); pb = wave_sum_f64(pb); }
    if (lane() == 0) {
      S.red_d[0][wave()] = pt;
      S.red_d[1][wave()] = pd;
      S.red_d[2][wave()] = pe;
      S.red_d[3][wave()] = pa;
      S.red_d[4][wave()] = pb;
    }
    lds_barrier();
    if (tid < SPART) {
      double v = 0.0;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += S.red_d[tid][w];
      st_dev(&parts[SPART * chunk + tid], v);
    }
  }
  // The residual draw's error bound, before the arrive (every workgroup has
  // the inputs; the row's last one then adds the margin mass): the bound on
  // |device cumulative - reference cumulative| at any index, for cumulatives
  // of chunk masses, then segment masses, then the segment's own residual
  // terms.  Every term p_i - q_i carries the two totals' relative errors
  // (weight_sum_err of a total over the total, at most weight_sum_err(1, n):
  // the row maximum weighs 1) and 8 ulp, over sum p = sum q = 1, plus each
  // side's f64 summation; tokens inside the classification margin, counted
  // as 0 in the sums, weigh at most 2 rho (p_i + q_i) each.  (The bonus
  // draw's bound is weight_sum_err of its mass.)
  const uint32_t nseg = C * spc;
  const uint32_t nsum = V + nseg + C;
  double errm = 0.0, erra = 0.0;
  if (!pl.err && !bonus) {
    const double rel = 16.0 * U + 2.0 * weight_sum_err(1.0, V + C);
    errm = 2.02 * sign_margin(S.ps[pl.r]);
    erra = 2.0 * rel + (2.0 * (double)nsum + 32.0) * U * 1.0001 + 1e-300;
  }
  if (!arrive_last(&A.ctr2[row * CTR_STRIDE], C, &S.s_u[0])) return;

  // ---- the row's last chunk: outputs and the draw, in wave 0 ---------------
  if (wave() != 0) return;
  int32_t* ot = A.out_tokens + (uint64_t)row * (K + 1u);
  for (uint32_t j = lane(); j <= K; j += 64u) ot[j] = (j < pl.r) ? A.tok[(uint64_t)row * K + j] : -1;
  if (pl.err) {
    if (lane() == 0) {
      A.status[row] = pl.err;
      A.out_count[row] = (int32_t)pl.r;
      A.out_accepted[row] = (int32_t)pl.r;
    }
    return;
  }
  const SpecPos& P = S.ps[pl.r];
  const double u = bonus ? A.ub[row] : A.ur[(uint64_t)row * K + pl.r];
  // chunk partials: lane l holds chunks 2l and 2l + 1 (C <= SMAXC = 128)
  double cp[2][SPART];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t qc = 2u * lane() + (uint32_t)h;
#pragma unroll
    for (uint32_t f = 0; f < SPART; ++f) cp[h][f] = qc < C ? ld_dev(&parts[SPART * qc + f]) : 0.0;
  }
  const double tt = wave_sum_f64(cp[0][0] + cp[1][0]);
  const double td = bonus ? 1.0 : wave_sum_f64(cp[0][1] + cp[1][1]);
  const double emass = bonus ? 0.0 : wave_sum_f64(cp[0][2] + cp[1][2]);
  const double a = bonus ? 1.0 : 1.0 / tt, b = bonus ? 0.0 : 1.0 / td;
  double cm[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) cm[h] = fmax(cp[h][3] * a - cp[h][4] * b, 0.0);
  const double lsum2 = cm[0] + cm[1];
  const double cinc = wave_scan(lsum2);                           // inclusive over lanes
  const double mass = readlane_t(cinc, 63u);
  const double err = bonus ? weight_sum_err(mass, nsum) : errm * emass + erra;
  const double thr = u * mass;
  bool unc = pl.unc;
  if (!bonus && !(mass > 2.0 * err)) unc = true;   // the reference's mass <= 0 fallback may apply
  // the chunk: first qc with thr < cumulative through qc
  uint32_t fq = NONE, lastq = NONE;
  bool near = false;
  double fbefore = 0.0;
  {
    double cum = cinc - lsum2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const double prev = cum;
      cum += cm[h];
      if (cm[h] > 0.0) {
        lastq = 2u * lane() + (uint32_t)h;
        if (fq == NONE && thr < cum && !(thr < prev)) {
          fq = 2u * lane() + (uint32_t)h;
          fbefore = prev;
          near = fabs(thr - prev) <= err || fabs(cum - thr) <= err;
        }
      }
    }
  }
  uint32_t qc = NONE;
  double before = 0.0;
  {
    const uint64_t fb = __ballot(fq != NONE), lb = __ballot(lastq != NONE);
    if (fb) {
      const int sl = __ffsll((unsigned long long)fb) - 1;
      qc = __shfl(fq, sl);
      before = __shfl(fbefore, sl);
      if (__shfl(near ? 1 : 0, sl)) unc = true;
    } else if (lb) {
      // rounding left the target past the accumulated mass: the last
      // positive chunk, from its start
      const int sl = 63 - __clzll((long long)lb);
      qc = __shfl(lastq, sl);
      before = -INFINITY;
      unc = true;
    }
  }
  uint32_t tok = NONE;
  bool tunc = true;
  if (qc != NONE) {
    // the segment within chunk qc: lane l holds segments l, l + 64 (spc <= SP * NW = 80)
    double sm[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t s = lane() + 64u * (uint32_t)h;
      double sa = 0.0, sb = 0.0;
      if (s < spc) {
        sa = ld_dev(&rs[2u * (qc * spc + s)]);
        sb = ld_dev(&rs[2u * (qc * spc + s) + 1u]);
      }
      sm[h] = fmax(sa * a - sb * b, 0.0);
    }
    // token order within the chunk is segment order (slice-major, then wave)
    const double s0inc = wave_scan(sm[0]);
    const double s0tot = readlane_t(s0inc, 63u);
    const double s1inc = wave_scan(sm[1]) + s0tot;
    uint32_t fs = NONE, lasts = NONE;
    double sbefore = 0.0;
    bool snear = false;
    const double base = before == -INFINITY ? 0.0 : before;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const double inc = base + (h == 0 ? s0inc : s1inc);
      const double exc = inc - sm[h];
      const uint32_t s = lane() + 64u * (uint32_t)h;
      if (sm[h] > 0.0) {
        lasts = s;
        if (fs == NONE && before != -INFINITY && thr < inc && !(thr < exc)) {
          fs = s;
          sbefore = exc;
          snear = fabs(thr - exc) <= err || fabs(inc - thr) <= err;
        }
      }
    }
    // first found segment (lowest s), or the last positive one
    uint32_t seg = NONE;
    {
      const uint32_t fmin = ~wave_max_u32(~fs);
      const uint32_t lmax = lasts == NONE ? 0u : lasts + 1u;
      const uint32_t lm = wave_max_u32(lmax);
      if (fmin != NONE) {
        seg = fmin;
        const int sl = (int)(fmin & 63u);
        before = __shfl(sbefore, sl);
        if (__shfl(snear ? 1 : 0, sl)) unc = true;
      } else if (lm) {
        seg = lm - 1u;
        before = -INFINITY;
        unc = true;
      }
    }
    if (seg != NONE) {
      const uint32_t i = seg / NW, w = seg % NW;
      const uint32_t qc1 = min(V, qc * CH + CH);
      const uint32_t id0 = qc * CH + i * SLICE + w * 256u + lane() * 4u;
      float lt[4], lq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t id = min(id0 + (uint32_t)e, V - 1u);
        lt[e] = tp[id];
        lq[e] = bonus ? 0.0f : dp[id];
      }
      double wl[4], lsum = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double wt = exp_neg16_t(((double)lt[e] - (double)P.mt) * invT, S.etab, S.etab + 16);
        double wv = bonus ? wt : fmax(wt * a - exp_neg16_t(((double)lq[e] - (double)P.md) * invT, S.etab, S.etab + 16) * b, 0.0);
        wl[e] = id0 + (uint32_t)e < qc1 ? wv : 0.0;
        lsum += wl[e];
      }
      const double inc = wave_scan(lsum);
      double cum = (before == -INFINITY ? 0.0 : before) + inc - lsum;
      uint32_t found = NONE, lastpos = NONE;
      bool fnear = false;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double prev = cum;
        cum += wl[e];
        if (wl[e] > 0.0) {
          lastpos = id0 + (uint32_t)e;
          if (before != -INFINITY && found == NONE && thr < cum && !(thr < prev)) {
            found = id0 + (uint32_t)e;
            fnear = fabs(thr - prev) <= err || fabs(cum - thr) <= err;
          }
        }
      }
      const uint64_t fb = __ballot(found != NONE);
      const uint64_t lb = __ballot(lastpos != NONE);
      if (fb) {
        const int sl = __ffsll((unsigned long long)fb) - 1;
        tok = __shfl(found, sl);
        tunc = __shfl(fnear ? 1 : 0, sl) != 0;
      } else if (lb) {
        const int sl = 63 - __clzll((long long)lb);
        tok = __shfl(lastpos, sl);
      }
    }
  }
  if (lane() == 0) {
    unc = unc || tunc;
    if (tok == NONE) {
      A.status[row] = unc ? MXS_ROW_UNCERTIFIED : MXS_ROW_PROBABILITIES;
      A.out_count[row] = (int32_t)pl.r;
      A.out_accepted[row] = (int32_t)pl.r;
    } else {
      ot[pl.r] = (int32_t)tok;
      A.status[row] = unc ? MXS_ROW_UNCERTIFIED : 0;
      A.out_count[row] = (int32_t)pl.r + 1;
      A.out_accepted[row] = (int32_t)pl.r;
    }
  }
}

// Chunk layouts of a vocabulary.  Pass 1 (a workgroup per (row, chunk)
// streams all of the row's logit rows): chunks enough for about 256
// workgroups over the batch, at least what SP quads per thread need, at most
// SMAXC.  Pass 2 (one position per row): one quad per thread, for more
// workgroups over the CUs, under the same limit.
static ChunkLayout spec_layout1(uint32_t V, uint32_t rows) {
  const uint32_t quads = (V + 3u) / 4u;
  const uint32_t cmin = (quads + (uint32_t)NT * SP - 1u) / ((uint32_t)NT * SP);
  const uint32_t cw = (256u + rows - 1u) / rows;
  uint32_t C = min((uint32_t)SMAXC, max(max(cmin, cw), 1u));
  const uint32_t ch = ((V + C - 1u) / C + 3u) & ~3u;
  C = (V + ch - 1u) / ch;
  return {C, ch, (ch / 4u + (uint32_t)NT - 1u) / (uint32_t)NT};
}
static ChunkLayout spec_layout2(uint32_t V) {
  const ChunkLayout L = chunk_layout(V, 1);
  return L.C <= (uint32_t)SMAXC ? L : chunk_layout(V, SP);
}

// Pass 2's segment capacity per row for vocabularies up to max_vocab: chunk
// counts grow with V within a layout, so each layout's count at the largest
// vocabulary it serves bounds the smaller ones.
static uint32_t spec_nseg_cap(uint32_t max_vocab) {
  const ChunkLayout a = chunk_layout(max_vocab, 1);
  uint32_t ns = min(a.C, (uint32_t)SMAXC) * NW;
  if (a.C > (uint32_t)SMAXC) ns = max(ns, chunk_layout(max_vocab, SP).C * (uint32_t)SP * NW);
  return ns;
}

static uint64_t spec_seg_stride(uint32_t max_vocab) {
  return 2ull * spec_nseg_cap(max_vocab) + (uint64_t)SPART * SMAXC;
}

size_t spec_scratch_bytes(uint32_t max_rows, uint32_t max_vocab) {
  const size_t pairs = (size_t)max_rows * (SPEC_KMAX + 1);
  return pairs * SMAXC * sizeof(SpecStat) + pairs * sizeof(SpecPos) +
         (size_t)max_rows * spec_seg_stride(max_vocab) * sizeof(double);
}

}  // namespace mxs

extern "C" int mxs_spec_verify(mxs_ctx* ctx, const float* target_logits, const float* draft_logits, uint32_t rows,
                               uint32_t draft_len, uint32_t vocab, const int32_t* draft_tokens,
                               const double* temperature, const double* accept_uniform,
                               const double* resample_uniform, const double* bonus_uniform, int32_t* out_tokens,
                               int32_t* out_count, int32_t* out_accepted, int32_t* status) {
  using namespace mxs;
  if (!ctx) return MXS_EINVAL;
  if (rows == 0) return MXS_OK;
  if (!target_logits || !temperature || !bonus_uniform || !out_tokens || !out_count || !out_accepted || !status)
    return fail(ctx, MXS_EINVAL, "target_logits, temperature, bonus_uniform and the outputs are required");
  if (draft_len > 0 && (!draft_logits || !draft_tokens || !accept_uniform || !resample_uniform))
    return fail(ctx, MXS_EINVAL, "draft logits, tokens and uniforms are required when draft_len > 0");
  if (rows > ctx->max_rows || vocab > ctx->max_vocab) return fail(ctx, MXS_EINVAL, "batch exceeds the context's max_rows/max_vocab");
  if (vocab == 0) return fail(ctx, MXS_EINVAL, "vocab must be positive");
  if (draft_len > SPEC_KMAX) return fail(ctx, MXS_EINVAL, "draft_len must be at most 8");
  const ChunkLayout L = spec_layout1(vocab, rows), L2 = spec_layout2(vocab);
  if (L.per > (uint32_t)SP || L.C > (uint32_t)SMAXC || L2.per > (uint32_t)SP || L2.C > (uint32_t)SMAXC ||
      L2.C * L2.per * NW > spec_nseg_cap(ctx->max_vocab))
    return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  const bool q2 = L2.per <= 1u;
  SpecArgs A;
  A.target = target_logits;
  A.draft = draft_len ? draft_logits : target_logits;
  A.rows = rows;
  A.K = draft_len;
  A.V = vocab;
  A.C = L.C;
  A.CH = L.CH;
  A.per = L.per;
  A.C2 = L2.C;
  A.CH2 = L2.CH;
  A.per2 = L2.per;
  A.tok = draft_tokens;
  A.T = temperature;
  A.ua = accept_uniform;
  A.ur = resample_uniform;
  A.ub = bonus_uniform;
  A.out_tokens = out_tokens;
  A.out_count = out_count;
  A.out_accepted = out_accepted;
  A.status = status;
  A.ctr1 = ctx->spec_ctr;
  A.ctr2 = ctx->spec_ctr + (size_t)ctx->max_rows * (SPEC_KMAX + 1) * CTR_STRIDE;
  char* base = reinterpret_cast<char*>(ctx->spec_scratch);
  const size_t pairs = (size_t)ctx->max_rows * (SPEC_KMAX + 1);
  A.stat = reinterpret_cast<SpecStat*>(base);
  A.pos = reinterpret_cast<SpecPos*>(base + pairs * SMAXC * sizeof(SpecStat));
  A.seg = reinterpret_cast<double*>(base + pairs * SMAXC * sizeof(SpecStat) + pairs * sizeof(SpecPos));
  A.seg_stride = spec_seg_stride(ctx->max_vocab);
  A.nseg_cap = spec_nseg_cap(ctx->max_vocab);
  const bool aligned = (vocab % 4u) == 0 && ((uintptr_t)target_logits % 16u) == 0 &&
                       ((uintptr_t)A.draft % 16u) == 0;
  const dim3 grid1(8u * L.C, (rows + 7u) / 8u);
  const dim3 grid2(8u * L2.C, (rows + 7u) / 8u);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
#define MXS_SPEC(AL)                                                                                     \
  do {                                                                                                   \
    switch (L.per) {                                                                                     \
      case 1: hipLaunchKernelGGL((spec_pass1<AL, 1>), grid1, dim3(NT), 0, ctx->stream, A); break;        \
      case 2: hipLaunchKernelGGL((spec_pass1<AL, 2>), grid1, dim3(NT), 0, ctx->stream, A); break;        \
      case 3: hipLaunchKernelGGL((spec_pass1<AL, 3>), grid1, dim3(NT), 0, ctx->stream, A); break;        \
      case 4: hipLaunchKernelGGL((spec_pass1<AL, 4>), grid1, dim3(NT), 0, ctx->stream, A); break;        \
      default: hipLaunchKernelGGL((spec_pass1<AL, 5>), grid1, dim3(NT), 0, ctx->stream, A); break;       \
    }                                                                                                    \
    if (q2) hipLaunchKernelGGL((spec_pass2<AL, 1>), grid2, dim3(NT), 0, ctx->stream, A);                \
    else hipLaunchKernelGGL((spec_pass2<AL, SP>), grid2, dim3(NT), 0, ctx->stream, A);                  \
  } while (0)
  if (aligned) MXS_SPEC(true); else MXS_SPEC(false);
#undef MXS_SPEC
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "spec kernels launch");
  return MXS_OK;
}
