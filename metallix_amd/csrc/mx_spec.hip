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
// Two launches on the context's stream.  Pass 1 (one workgroup per (row,
// position, chunk)) reduces each chunk's maxima and f64 weight sums; the
// last chunk of a (row, position) decides acceptance.  Pass 2 (one
// workgroup per (row, chunk)) finds the first rejected position (or the
// bonus position), writes 256-token segment masses of the distribution to
// draw from, and the row's last chunk locates the draw: the segment by a
// prefix over segment masses, then the token by re-deriving the segment's
// 256 weights in f64.  Every comparison against a reference f64 sum is
// taken only when a rigorous error bound certifies it; otherwise the row is
// reported uncertified (status 1) with the device's decision.

#include <hip/hip_runtime.h>

#include <math.h>
#include <string.h>

#include "../../include/mx_sampler.h"
#include "mxs_ctx.h"
#include "mxs_device.h"
#include "mxs_math.h"

namespace mxs {

constexpr int SP = 5;                 // quads per thread per chunk
constexpr int SMAXC = 128;            // chunks per row
constexpr uint32_t SPEC_KMAX = 8;     // draft positions per row
constexpr int SSEG = SP * NW;         // 256-token segments per chunk

struct SpecStat {                     // per (row, position, chunk)
  float tmax, dmax, tmin;
  uint32_t flags;                     // 1: non-finite target logit, 2: non-finite draft logit
  double tsum, dsum;                  // sums of exp((l - chunk max) / T)
};

struct SpecPos {                      // per (row, position): pass 1's verdict
  int32_t err;                        // this position's error status (0: none)
  int32_t accept;                     // 1: drafted token accepted
  int32_t unc;                        // the decision is not certified
  int32_t pad;
  float mt, md;                       // row maxima of target and draft
  double tt, td;                      // totals of exp((l - row max) / T)
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
  double* seg;                        // [rows * SMAXC * SSEG]
};

struct SpecSmem {
  double etab[128];                   // exp_neg's tables
  SpecStat st[SMAXC];
  SpecPos ps[SPEC_KMAX + 1];
  uint32_t red_u[4][NW];
  double red_d[4][NW];
  double s_d[4];
  uint32_t s_u[8];
};

// Bound on |device sum - reference sum| for n weights exp(x), x = (l - M) / T
// <= 0, summed in different orders: each side's f64 rounding of the sums and
// of the terms (8 ulp), and the rounding of x (x e^x <= 1/e per term).
__device__ __forceinline__ double weight_sum_err(double s, uint32_t n) {
  return (2.0 * (double)n + 16.0) * U * s * 1.0001 + 1.5 * (double)n * U + 1e-300;
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

// ---------------------------------------------------------------------------
// Pass 1: per (row, position, chunk) maxima and weight sums; the last chunk
// of a (row, position) decides acceptance.
template <bool ALIGNED>
__global__ __launch_bounds__(NT) void spec_pass1(SpecArgs A) {
  __shared__ SpecSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t pair = blockIdx.y * 8u + xcd;
  const uint32_t K = A.K, V = A.V;
  if (pair >= A.rows * (K + 1u)) return;
  const uint32_t row = pair / (K + 1u), j = pair % (K + 1u);
  const bool has_draft = j < K;
  const uint32_t c0 = chunk * A.CH, c1 = min(V, c0 + A.CH);
  const float* tp = A.target + (uint64_t)pair * V;
  const float* dp = A.draft + ((uint64_t)row * K + (has_draft ? j : 0u)) * V;
  const double T = A.T[row];
  const bool tok_T = temperature_ok(T);
  const double invT = tok_T ? 1.0 / T : 0.0;

  if (tid < 128u) S.etab[tid] = tid < 64u ? kExp2Tab[tid] : kExp2TabLo[tid - 64u];
  float tv[SP][4], dv[SP][4];
#pragma unroll
  for (int i = 0; i < SP; ++i) {
    const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
    const uint32_t es = e0 < c1 ? e0 : c0;
    load_quad<ALIGNED>(tp, es, c1, tv[i]);
    if (has_draft) load_quad<ALIGNED>(dp, es, c1, dv[i]);
  }
  float tmax = -INFINITY, dmax = -INFINITY, tmin = INFINITY;
  uint64_t nft = 0, nfd = 0;
#pragma unroll
  for (int i = 0; i < SP; ++i) {
    const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool inr = i < (int)A.per && e0 + (uint32_t)e < c1;
      nft |= __builtin_amdgcn_ballot_w64(inr && !__builtin_isfinite(tv[i][e]));
      tv[i][e] = inr ? tv[i][e] : -INFINITY;
      tmax = fmaxf(tmax, tv[i][e]);
      tmin = inr ? fminf(tmin, tv[i][e]) : tmin;
      if (has_draft) {
        nfd |= __builtin_amdgcn_ballot_w64(inr && !__builtin_isfinite(dv[i][e]));
        dv[i][e] = inr ? dv[i][e] : -INFINITY;
        dmax = fmaxf(dmax, dv[i][e]);
      }
    }
  }
  {
    const uint32_t a = wave_max_u32(okey(tmax)), b = wave_max_u32(okey(dmax));
    const uint32_t c = ~wave_max_u32(~okey(tmin));
    if (lane() == 0) {
      S.red_u[0][wave()] = a;
      S.red_u[1][wave()] = b;
      S.red_u[2][wave()] = c;
      S.red_u[3][wave()] = (nft ? 1u : 0u) | (nfd ? 2u : 0u);
    }
  }
  lds_barrier();
  uint32_t ka = 0u, kb = 0u, kc = NONE, flags = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ka = max(ka, S.red_u[0][w]);
    kb = max(kb, S.red_u[1][w]);
    kc = min(kc, S.red_u[2][w]);
    flags |= S.red_u[3][w];
  }
  const float mt = okey_value(ka), md = okey_value(kb), mn = okey_value(kc);
  double tsum = 0.0, dsum = 0.0;
  if (tok_T && !flags && c1 > c0) {
    const double mtd = (double)mt, mdd = (double)md;
    double pt = 0.0, pd = 0.0;
#pragma unroll
    for (int i = 0; i < SP; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pt += exp_neg_t(((double)tv[i][e] - mtd) * invT, S.etab, S.etab + 64);
        if (has_draft) pd += exp_neg_t(((double)dv[i][e] - mdd) * invT, S.etab, S.etab + 64);
      }
    pt = wave_sum_f64(pt);
    pd = wave_sum_f64(pd);
    if (lane() == 0) { S.red_d[0][wave()] = pt; S.red_d[1][wave()] = pd; }
    lds_barrier();
#pragma unroll
    for (int w = 0; w < NW; ++w) { tsum += S.red_d[0][w]; dsum += S.red_d[1][w]; }
  }
  if (tid == 0) {
    SpecStat* st = &A.stat[((uint64_t)row * (SPEC_KMAX + 1) + j) * SMAXC + chunk];
    st_dev(&st->tmax, mt);
    st_dev(&st->dmax, md);
    st_dev(&st->tmin, mn);
    st_dev(&st->flags, flags);
    st_dev(&st->tsum, tsum);
    st_dev(&st->dsum, dsum);
  }
  if (!arrive_last(&A.ctr1[(row * (SPEC_KMAX + 1) + j) * CTR_STRIDE], A.C, &S.s_u[0])) return;

  // ---- the position's verdict (one thread does the arithmetic) -------------
  const uint32_t slot = row * (SPEC_KMAX + 1) + j;
  const uint32_t C = A.C;
  for (uint32_t q = tid; q < C; q += NT) {
    const SpecStat* st = &A.stat[(uint64_t)slot * SMAXC + q];
    SpecStat v;
    v.tmax = ld_dev(&st->tmax);
    v.dmax = ld_dev(&st->dmax);
    v.tmin = ld_dev(&st->tmin);
    v.flags = ld_dev(&st->flags);
    v.tsum = ld_dev(&st->tsum);
    v.dsum = ld_dev(&st->dsum);
    S.st[q] = v;
  }
  __syncthreads();
  if (tid != 0) return;
  uint32_t fl = 0;
  float Mt = -INFINITY, Md = -INFINITY, Mn = INFINITY;
  for (uint32_t q = 0; q < C; ++q) {
    fl |= S.st[q].flags;
    Mt = fmaxf(Mt, S.st[q].tmax);
    Md = fmaxf(Md, S.st[q].dmax);
    Mn = fminf(Mn, S.st[q].tmin);
  }
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
    const int32_t d = A.tok[(uint64_t)row * K + j];
    const double ua = A.ua[(uint64_t)row * K + j], ur = A.ur[(uint64_t)row * K + j];
    if (fl) P.err = MXS_ROW_NON_FINITE_LOGIT;
    else if (d < 0) P.err = MXS_ROW_TOKEN_OUT_OF_RANGE;
    else if (!uniform_ok(ua) || !uniform_ok(ur)) P.err = MXS_ROW_INVALID_UNIFORM;
    else if ((uint32_t)d >= V) P.err = MXS_ROW_TOKEN_OUT_OF_RANGE;
    if (!P.err) {
      double tt = 0.0, td = 0.0;
      for (uint32_t q = 0; q < C; ++q) {
        tt += S.st[q].tsum * exp_neg(((double)S.st[q].tmax - (double)Mt) * invT);
        td += S.st[q].dsum * exp_neg(((double)S.st[q].dmax - (double)Md) * invT);
      }
      P.tt = tt;
      P.td = td;
      P.tterr = weight_sum_err(tt, V + C);
      P.tderr = weight_sum_err(td, V + C);
      const double wt = exp_neg(((double)tp[d] - (double)Mt) * invT);
      const double wd = exp_neg(((double)dp[d] - (double)Md) * invT);
      const double xq = ((double)dp[d] - (double)Md) * invT;
      const double xt = ((double)tp[d] - (double)Mt) * invT;
      if (wd <= 0.0) {
        // the reference's q <= 0 rejection; near the f64 underflow edge the
        // two exp implementations may disagree
        P.err = MXS_ROW_PROBABILITIES;
        if (xq > -746.0) P.unc = 1;
      } else {
        const double p = wt / tt, qq = wd / td;
        const double ratio = p / qq;
        // relative error of the ratio: both weights (exp 1 ulp and the
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
      double tt = 0.0;
      for (uint32_t q = 0; q < C; ++q) tt += S.st[q].tsum * exp_neg(((double)S.st[q].tmax - (double)Mt) * invT);
      P.tt = tt;
      P.tterr = weight_sum_err(tt, V + C);
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

// Weight of token i in the distribution drawn at the plan's position:
// the residual max(0, t_i / sum t - q_i / sum q), or the target weight t_i
// for the bonus draw.
__device__ __forceinline__ double draw_weight(bool bonus, float t, float q, const SpecPos& P, double invT,
                                              const double* etab) {
  const double wt = exp_neg_t(((double)t - (double)P.mt) * invT, etab, etab + 64);
  if (bonus) return wt;
  const double wq = exp_neg_t(((double)q - (double)P.md) * invT, etab, etab + 64);
  return fmax(wt / P.tt - wq / P.td, 0.0);
}

// ---------------------------------------------------------------------------
// Pass 2: segment masses of the drawn distribution; the row's last chunk
// draws.
template <bool ALIGNED>
__global__ __launch_bounds__(NT) void spec_pass2(SpecArgs A) {
  __shared__ SpecSmem S;
  const uint32_t tid = threadIdx.x;
  const uint32_t xcd = blockIdx.x & 7u;
  const uint32_t chunk = blockIdx.x >> 3;
  const uint32_t row = blockIdx.y * 8u + xcd;
  if (row >= A.rows) return;
  const uint32_t K = A.K, V = A.V;
  if (tid < 128u) S.etab[tid] = tid < 64u ? kExp2Tab[tid] : kExp2TabLo[tid - 64u];
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
  const double T = A.T[row];
  const double invT = temperature_ok(T) ? 1.0 / T : 0.0;
  const uint32_t c0 = chunk * A.CH, c1 = min(V, c0 + A.CH);
  if (!pl.err) {
    const SpecPos& P = S.ps[pl.r];
    const float* tp = A.target + ((uint64_t)row * (K + 1u) + pl.r) * V;
    const float* dp = A.draft + ((uint64_t)row * K + (bonus ? 0u : pl.r)) * V;
#pragma unroll
    for (int i = 0; i < SP; ++i) {
      double s = 0.0;
      if (i < (int)A.per) {
        const uint32_t e0 = c0 + (uint32_t)i * SLICE + tid * 4u;
        const uint32_t es = e0 < c1 ? e0 : c0;
        float t[4], q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        load_quad<ALIGNED>(tp, es, c1, t);
        if (!bonus) load_quad<ALIGNED>(dp, es, c1, q);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e0 + (uint32_t)e < c1) s += draw_weight(bonus, t[e], q[e], P, invT, S.etab);
      }
      const double ws = wave_sum_f64(s);
      if (lane() == 0) st_dev(&A.seg[((uint64_t)row * SMAXC + chunk) * SSEG + i * NW + wave()], ws);
    }
  }
  if (!arrive_last(&A.ctr2[row * CTR_STRIDE], A.C, &S.s_u[0])) return;

  // ---- the row's last chunk: outputs and the draw ---------------------------
  int32_t* ot = A.out_tokens + (uint64_t)row * (K + 1u);
  for (uint32_t j = tid; j <= K; j += NT) ot[j] = (j < pl.r) ? A.tok[(uint64_t)row * K + j] : -1;
  if (pl.err) {
    if (tid == 0) {
      A.status[row] = pl.err;
      A.out_count[row] = (int32_t)pl.r;
      A.out_accepted[row] = (int32_t)pl.r;
    }
    return;
  }
  const SpecPos& P = S.ps[pl.r];
  const double u = bonus ? A.ub[row] : A.ur[(uint64_t)row * K + pl.r];
  const uint32_t C = A.C;
  const uint32_t segs_per_chunk = A.per * NW;
  const uint32_t nseg = C * segs_per_chunk;
  auto seg_mass = [&](uint32_t s) {
    const uint32_t q = s / segs_per_chunk, r = s % segs_per_chunk;
    return ld_dev(&A.seg[((uint64_t)row * SMAXC + q) * SSEG + r]);
  };
  double part = 0.0;
  for (uint32_t s = tid; s < nseg; s += NT) part += seg_mass(s);
  part = wave_sum_f64(part);
  if (lane() == 0) S.red_d[0][wave()] = part;
  __syncthreads();
  double mass = 0.0;
#pragma unroll
  for (int w = 0; w < NW; ++w) mass += S.red_d[0][w];
  // Bound on |device cumulative - reference cumulative| at any index.  Bonus:
  // target weights as in the sampler's full-row draw.  Residual: every term
  // p_i - q_i carries the two totals' relative errors and 8 ulp, over
  // sum p = sum q = 1, plus each side's f64 summation.
  double err;
  if (bonus) {
    err = weight_sum_err(mass, V + nseg);
  } else {
    const double rel = 16.0 * U + P.tterr / P.tt + P.tderr / P.td;
    err = 2.0 * rel + (2.0 * (double)(V + nseg) + 16.0) * U * 1.0001 + 1e-300;
  }
  const double thr = u * mass;
  bool unc = pl.unc;
  if (!bonus && !(mass > 2.0 * err)) unc = true;   // the reference's mass <= 0 fallback may apply
  // the segment: first s with thr < cumulative through s
  if (tid == 0) { S.s_u[1] = NONE; S.s_u[2] = 0u; S.s_u[3] = 0u; }
  __syncthreads();
  double run = 0.0;
  for (uint32_t base = 0; base < nseg; base += NT) {
    const uint32_t s = base + tid;
    const double w = s < nseg ? seg_mass(s) : 0.0;
    double tot;
    const double inc = run + block_scan_incl<double>(w, S.red_d[1], &tot);
    const double exc = inc - w;
    if (w > 0.0) {
      atomicMax(&S.s_u[2], s + 1u);
      if (thr < inc && !(thr < exc)) {
        S.s_u[1] = s;
        S.s_d[0] = exc;
        if (fabs(thr - exc) <= err || fabs(inc - thr) <= err) S.s_u[3] = 1u;
      }
    }
    run += tot;
  }
  __syncthreads();
  uint32_t seg = S.s_u[1];
  double before = S.s_d[0];
  if (S.s_u[3]) unc = true;
  if (seg == NONE) {
    // rounding left the target past the accumulated mass: last positive token
    seg = S.s_u[2] ? S.s_u[2] - 1u : NONE;
    unc = true;
    before = -INFINITY;
  }
  if (wave() == 0) {
    uint32_t tok = NONE;
    bool tunc = true;
    if (seg != NONE) {
      const uint32_t q = seg / segs_per_chunk, r = seg % segs_per_chunk;
      const uint32_t i = r / NW, w = r % NW;
      const uint32_t qc1 = min(V, q * A.CH + A.CH);
      const uint32_t id0 = q * A.CH + i * SLICE + w * 256u + lane() * 4u;
      const float* tp = A.target + ((uint64_t)row * (K + 1u) + pl.r) * V;
      const float* dp = A.draft + ((uint64_t)row * K + (bonus ? 0u : pl.r)) * V;
      double wl[4], lsum = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t id = id0 + (uint32_t)e;
        wl[e] = id < qc1 ? draw_weight(bonus, tp[id], bonus ? 0.0f : dp[id], P, invT, S.etab) : 0.0;
        lsum += wl[e];
      }
      double inc = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane() >= (uint32_t)o) inc += t;
      }
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
}

size_t spec_scratch_bytes(uint32_t max_rows) {
  const size_t pairs = (size_t)max_rows * (SPEC_KMAX + 1);
  return pairs * SMAXC * sizeof(SpecStat) + pairs * sizeof(SpecPos) + (size_t)max_rows * SMAXC * SSEG * sizeof(double);
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
  const ChunkLayout L = chunk_layout(vocab, SP);
  if (L.per > (uint32_t)SP || L.C > (uint32_t)SMAXC) return fail(ctx, MXS_EINVAL, "vocab too large for the chunk layout");
  SpecArgs A;
  A.target = target_logits;
  A.draft = draft_len ? draft_logits : target_logits;
  A.rows = rows;
  A.K = draft_len;
  A.V = vocab;
  A.C = L.C;
  A.CH = L.CH;
  A.per = L.per;
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
  const bool aligned = (vocab % 4u) == 0 && ((uintptr_t)target_logits % 16u) == 0 &&
                       ((uintptr_t)A.draft % 16u) == 0;
  const dim3 grid1(8u * L.C, (rows * (draft_len + 1u) + 7u) / 8u);
  const dim3 grid2(8u * L.C, (rows + 7u) / 8u);
  int prev = 0;
  hipGetDevice(&prev);
  if (prev != ctx->device) hipSetDevice(ctx->device);
  if (aligned) {
    hipLaunchKernelGGL(spec_pass1<true>, grid1, dim3(NT), 0, ctx->stream, A);
    hipLaunchKernelGGL(spec_pass2<true>, grid2, dim3(NT), 0, ctx->stream, A);
  } else {
    hipLaunchKernelGGL(spec_pass1<false>, grid1, dim3(NT), 0, ctx->stream, A);
    hipLaunchKernelGGL(spec_pass2<false>, grid2, dim3(NT), 0, ctx->stream, A);
  }
  hipError_t e = hipGetLastError();
  if (prev != ctx->device) hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(ctx, e, "spec kernels launch");
  return MXS_OK;
}
