// mxs_math.h -- numeric building blocks shared by the HIP sampler kernels and
// their host-side unit checks.  Compiles as HIP (device + host) and as plain
// C++ (host only, MXS_HD empty).
#pragma once
#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#define MXS_HD __host__ __device__ __forceinline__
#else
#define MXS_HD inline
#endif

namespace mxs {

// 2^(j/64), j = 0..63, correctly rounded to f64.
#if defined(__HIPCC__)
__device__ __constant__
#endif
static const double kExp2Tab[64] = {0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0, 0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0, 0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0, 0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0, 0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, 0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0, 0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0, 0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0, 0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0, 0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0, 0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0, 0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0, 0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0, 0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0, 0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0, 0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0};
// 2^(j/64) - kExp2Tab[j], rounded to f64.
#if defined(__HIPCC__)
__device__ __constant__
#endif
static const double kExp2TabLo[64] = {0x0.0p+0, -0x1.19083535b085dp-56, 0x1.d73e2a475b465p-55, 0x1.186be4bb284ffp-57, 0x1.8a62e4adc610bp-54, 0x1.03a1727c57b53p-59, -0x1.6c51039449b3ap-54, -0x1.32fbf9af1369ep-54, -0x1.19041b9d78a76p-55, 0x1.e5b4c7b4968e4p-55, 0x1.e016e00a2643cp-54, 0x1.dc775814a8495p-55, 0x1.9b07eb6c70573p-54, 0x1.2bd339940e9d9p-55, 0x1.612e8afad1255p-55, 0x1.0024754db41d5p-54, 0x1.6f46ad23182e4p-55, 0x1.32721843659a6p-54, -0x1.63aeabf42eae2p-54, -0x1.5e436d661f5e3p-56, 0x1.ada0911f09ebcp-55, -0x1.ef3691c309278p-58, 0x1.89b7a04ef80d0p-59, 0x1.3c1a3b69062f0p-56, 0x1.d4397afec42e2p-56, -0x1.4b309d25957e3p-54, -0x1.07abe1db13cadp-55, 0x1.9bb2c011d93adp-54, 0x1.6324c054647adp-54, 0x1.ba6f93080e65ep-54, -0x1.383c17e40b497p-54, -0x1.bb60987591c34p-54, -0x1.bdd3413b26456p-54, -0x1.bbe3a683c88abp-57, -0x1.16e4786887a99p-55, -0x1.0245957316dd3p-54, -0x1.41577ee04992fp-55, 0x1.05d02ba15797ep-56, -0x1.d4c1dd41532d8p-54, -0x1.fc6f89bd4f6bap-54, 0x1.6e9f156864b27p-54, 0x1.5cc13a2e3976cp-55, -0x1.75fc781b57ebcp-57, -0x1.d185b7c1b85d1p-54, 0x1.c7c46b071f2bep-56, -0x1.359495d1cd533p-54, -0x1.d2f6edb8d41e1p-54, 0x1.0fac90ef7fd31p-54, 0x1.7a1cd345dcc81p-54, -0x1.2805e3084d708p-57, -0x1.5584f7e54ac3bp-56, 0x1.23dd07a2d9e84p-55, 0x1.11065895048ddp-55, 0x1.2884dff483cadp-54, 0x1.503cbd1e949dbp-56, -0x1.cbc3743797a9cp-54, 0x1.2ed02d75b3707p-55, 0x1.c2300696db532p-54, -0x1.1a5cd4f184b5cp-54, 0x1.39e8980a9cc8fp-55, -0x1.e9c23179c2893p-54, 0x1.dc7f486a4b6b0p-54, 0x1.9d3e12dd8a18bp-54, 0x1.74853f3a5931ep-55};

// f32 total order (Rust f32::total_cmp) as an unsigned key: larger key sorts
// first in descending order; -0.0 ranks below +0.0.
MXS_HD uint32_t okey(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
MXS_HD float okey_value(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

// l / r rounded to f32, for finite r > 0, without an f32 division: the f64
// product l * (1/r) carries at most 2^-52 relative error, while the exact
// quotient of two f32 values (24-bit significands) is either exact in f64
// arithmetic here (r a power of two) or at least 2^-49 (relative) away from
// every f32 rounding midpoint, normal or subnormal.  So the single f64->f32
// rounding lands where the IEEE f32 division rounds.  Checked against the
// f32 division on the host over random and edge-case operands.
MXS_HD float div_by_recip(float l, double inv_r) { return (float)((double)l * inv_r); }

// The lowest finite f32 (Rust's f32::MIN): a suppressed token's logit.
constexpr float kF32Min = -0x1.fffffep+127f;

// Logit bias and penalties for one token, every step rounded to f32 in this
// order: l + bias (when the token has a bias entry), then for a token seen
// `cnt` > 0 times in the history: repetition (l < 0 ? l * rep : l / rep),
// minus cnt * frequency, minus presence.  `tv` packs cnt in bits 0-30 and
// "has a bias entry" in bit 31.  A bias entry of -inf suppresses the token:
// its adjusted logit is f32::MIN whatever the penalties
// (ChatFormat::suppress, crates/core/chat-format/src/lib.rs:771-780).
MXS_HD float bias_and_penalize(float l, uint32_t tv, float bias, float rep, double inv_rep, float freq,
                               float pres) {
  if ((tv >> 31) && bias == -INFINITY) return kF32Min;
  const uint32_t cnt = tv & 0x7fffffffu;
  const float a = (tv >> 31) ? l + bias : l;
  const float r = a < 0.0f ? a * rep : div_by_recip(a, inv_rep);
  const float cf = (float)cnt * freq;
  const float p = (r - cf) - pres;
  return cnt ? p : a;
}

// exp(x) for x <= 0 in f64: x = n ln2/64 + r, |r| <= ln2/128, degree-6 Taylor
// polynomial for e^r - 1 (truncation below 3e-20 relative), 2^(n mod 64 / 64)
// as a two-part table so one final rounding dominates, scaled by
// 2^(n div 64).  Within 1 ulp of glibc's exp (checked in tests); the
// certificate bounds in the kernels budget 4 ulp per term.  Returns 0 below -746 and for -inf.
// exp_neg_t takes the two tables by pointer (a kernel may keep a copy in
// LDS); exp_neg reads the constant tables.
MXS_HD double exp_neg_t(double x, const double* tab_hi, const double* tab_lo) {
  if (!(x > -746.0)) return 0.0;
  const double kInvL = 92.33248261689366;          // 64 / ln 2
  const double kLHi = 0.010830424696249145;        // ln 2 / 64, high part
  const double kLLo = 3.623510646634843e-19;       // ln 2 / 64 - kLHi
  double t = rint(x * kInvL);
  int n = (int)t;
  double r = fma(-t, kLHi, x);
  r = fma(-t, kLLo, r);
  double p = fma(r, 1.0 / 720.0, 1.0 / 120.0);
  p = fma(r, p, 1.0 / 24.0);
  p = fma(r, p, 1.0 / 6.0);
  p = fma(r, p, 0.5);
  double q = fma(r * r, p, r);  // e^r - 1
  int j = n & 63;
  int k = n >> 6;  // arithmetic shift: floor division
  const double th = tab_hi[j], tl = tab_lo[j];
  return ldexp(th + fma(th, q, tl), k);
}
MXS_HD double exp_neg(double x) { return exp_neg_t(x, kExp2Tab, kExp2TabLo); }

// exp(x) for x <= 0 in f64 from a 16-entry two-part table, 2^(j/16) for j <
// 16 (entries 4j of the 64-entry one): a kernel's LDS copy, 16 doubles per
// part, is read without bank conflicts (distinct entries fall in distinct
// banks, equal ones broadcast).  x = n ln2/16 + r, |r| <= ln2/32, degree-7
// Taylor polynomial for e^r - 1 (truncation below 2e-18 relative), scaled
// by 2^(n div 16).  Within 1 ulp of glibc's exp (checked in tests).
// Returns 0 below -746 and for -inf.
MXS_HD double exp_neg16_t(double x, const double* tab_hi, const double* tab_lo) {
  if (!(x > -746.0)) return 0.0;
  const double kInvL = 23.083120654223414;         // 16 / ln 2
  const double kLHi = 0.04332169878499658;         // ln 2 / 16, high part (trailing zero bits: t kLHi exact)
  const double kLLo = 1.4494042586539372e-18;      // ln 2 / 16 - kLHi
  double t = rint(x * kInvL);
  int n = (int)t;
  double r = fma(-t, kLHi, x);
  r = fma(-t, kLLo, r);
  double p = fma(r, 1.0 / 5040.0, 1.0 / 720.0);
  p = fma(r, p, 1.0 / 120.0);
  p = fma(r, p, 1.0 / 24.0);
  p = fma(r, p, 1.0 / 6.0);
  p = fma(r, p, 0.5);
  double q = fma(r * r, p, r);  // e^r - 1
  int j = n & 15;
  int k = n >> 4;  // arithmetic shift: floor division
  const double th = tab_hi[j], tl = tab_lo[j];
  return ldexp(th + fma(th, q, tl), k);
}

// exp(x) for x <= 0 in f64 without tables (for loops over registers, where
// table gathers would be hoisted and held): x = n ln2 + r, |r| <= ln2 / 2
// (Cody-Waite reduction with a 32-bit high part of ln2, so n * hi is exact
// for |n| < 2^21), degree-13 Taylor polynomial for e^r (truncation below
// 5e-18 relative), scaled by 2^n.  Within 2 ulp of glibc's exp (checked in
// tests).  Returns 0 below -746 and for -inf.
MXS_HD double exp_neg_p(double x) {
  if (!(x > -746.0)) return 0.0;
  const double kLn2Hi = 0.6931471803691238;       // ln 2, low 21 bits of the significand clear
  const double kLn2Lo = 1.9082149292705877e-10;   // ln 2 - kLn2Hi
  const double t = rint(x * 1.4426950408889634);
  double r = fma(-t, kLn2Hi, x);
  r = fma(-t, kLn2Lo, r);
  double p = 1.0 / 6227020800.0;                  // 1/13!
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  return ldexp(fma(p, r, 1.0), (int)t);
}

}  // namespace mxs
