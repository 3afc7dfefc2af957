// Host-side checks of the numeric building blocks the kernels share
// (metallix_amd/csrc/mxs_math.h), built with g++ by tests/test_math_host.py.
// Prints one line per check: "<name> <failures> <cases> [detail]".
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../metallix_amd/csrc/mxs_math.h"

static uint64_t sm_state = 0x6d78000000000001ull;
static uint64_t splitmix(void) {
  uint64_t z = (sm_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static float f_of(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t b_of(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static uint64_t d_bits(double d) { uint64_t b; memcpy(&b, &d, 8); return b; }

// l / r through the f64 reciprocal must equal the IEEE f32 quotient bit for bit.
static void check_division(long n) {
  long fail = 0, cases = 0;
  const float reps[] = {1.05f, 1.1f, 1.2f, 1.3f, 1.5f, 2.0f, 0.5f, 0.9f, 3.0f, 7.0f, 1.0f, 0.7f};
  for (long i = 0; i < n; ++i) {
    uint64_t z = splitmix();
    float l = f_of((uint32_t)z);
    float r;
    if (i % 3 == 0) r = reps[(z >> 40) % (sizeof(reps) / sizeof(reps[0]))];
    else r = fabsf(f_of((uint32_t)(z >> 32)));
    if (!isfinite(l) || !isfinite(r) || !(r > 0.0f)) continue;
    ++cases;
    const float want = l / r;
    const float got = mxs::div_by_recip(l, 1.0 / (double)r);
    if (b_of(want) != b_of(got)) {
      if (fail < 5) printf("#division mismatch l=%a r=%a want=%a got=%a\n", l, r, want, got);
      ++fail;
    }
  }
  // subnormal quotients, exact halving of odd subnormals, overflow edge
  for (uint32_t m = 1; m < 4096; ++m) {
    const float l = f_of(m), ln = -f_of(m);
    const float rs[] = {2.0f, 4.0f, 1.1f, 3.0f, 0.75f};
    for (float r : rs) {
      cases += 2;
      if (b_of(l / r) != b_of(mxs::div_by_recip(l, 1.0 / (double)r))) ++fail;
      if (b_of(ln / r) != b_of(mxs::div_by_recip(ln, 1.0 / (double)r))) ++fail;
    }
  }
  const float big[] = {3.4028235e38f, 3.0e38f, 1.7e38f};
  const float small_r[] = {0.99999994f, 0.5f, 0.9f};
  for (float l : big)
    for (float r : small_r) {
      ++cases;
      if (b_of(l / r) != b_of(mxs::div_by_recip(l, 1.0 / (double)r))) ++fail;
    }
  printf("division %ld %ld\n", fail, cases);
}

// The composed bias + penalty stage against the same steps with the f32 division.
static void check_penalize(long n) {
  long fail = 0;
  for (long i = 0; i < n; ++i) {
    uint64_t z = splitmix(), y = splitmix();
    const float l = (float)((int32_t)(uint32_t)z) * 1e-8f;
    const uint32_t cnt = (uint32_t)(y % 5);
    const bool hb = (y >> 8) & 1;
    const float bias = (float)((int32_t)(uint32_t)(y >> 16) % 2000) * 0.01f;
    const float rep = 0.5f + (float)((y >> 40) % 200) * 0.01f;
    const float freq = 0.3f, pres = 0.5f;
    float a = hb ? l + bias : l;
    float want = a;
    if (cnt) {
      float r = a < 0.0f ? a * rep : a / rep;
      float cf = (float)cnt * freq;
      r = r - cf;
      want = r - pres;
    }
    const uint32_t tv = cnt | (hb ? 0x80000000u : 0u);
    const float got = mxs::bias_and_penalize(l, tv, bias, rep, 1.0 / (double)rep, freq, pres);
    if (b_of(want) != b_of(got)) ++fail;
  }
  printf("penalize %ld %ld\n", fail, n);
}

// exp_neg against the C library's exp: at most 1 ulp apart.
static void check_exp(long n) {
  long fail = 0, diff = 0;
  for (long i = 0; i < n; ++i) {
    const double x = -746.0 * (double)(splitmix() >> 11) * 0x1.0p-53;
    const double a = exp(x), b = mxs::exp_neg(x);
    const int64_t u = (int64_t)d_bits(a) - (int64_t)d_bits(b);
    if (u != 0) ++diff;
    if (u > 1 || u < -1) ++fail;
  }
  const double edge[] = {0.0, -0.0, -1e-300, -745.1, -746.0, -800.0, -INFINITY, -708.39, -1.0};
  for (double x : edge) {
    const double a = exp(x), b = mxs::exp_neg(x);
    const int64_t u = (int64_t)d_bits(a) - (int64_t)d_bits(b);
    if (x < -746.0 || x == -746.0) { if (b != 0.0) ++fail; }
    else if (u > 1 || u < -1) ++fail;
  }
  printf("exp_neg %ld %ld differing=%ld\n", fail, n, diff);
}

// exp_neg16_t (1 ulp) and exp_neg_p (2 ulp) against the C library's exp.
static void check_exp_variants(long n) {
  double hi16[16], lo16[16];
  for (int j = 0; j < 16; ++j) { hi16[j] = mxs::kExp2Tab[4 * j]; lo16[j] = mxs::kExp2TabLo[4 * j]; }
  long f16 = 0, fp = 0, d16 = 0, dp = 0;
  auto one = [&](double x) {
    const double a = exp(x), b = mxs::exp_neg16_t(x, hi16, lo16), c = mxs::exp_neg_p(x);
    if (!(x > -746.0)) {
      if (b != 0.0) ++f16;
      if (c != 0.0) ++fp;
      return;
    }
    const int64_t u = (int64_t)d_bits(a) - (int64_t)d_bits(b), v = (int64_t)d_bits(a) - (int64_t)d_bits(c);
    if (u) ++d16;
    if (v) ++dp;
    if (u > 1 || u < -1) ++f16;
    if (v > 2 || v < -2) ++fp;
  };
  for (long i = 0; i < n; ++i) one(-746.0 * (double)(splitmix() >> 11) * 0x1.0p-53);
  for (long i = 0; i < n / 4; ++i) one(-(double)(splitmix() >> 11) * 0x1.0p-53);   // |x| < 1
  const double edge[] = {0.0, -0.0, -1e-300, -745.1, -746.0, -800.0, -INFINITY, -708.39, -1.0, -0.02166, -0.0433};
  for (double x : edge) one(x);
  printf("exp_neg16 %ld %ld differing=%ld\n", f16, n, d16);
  printf("exp_neg_p %ld %ld differing=%ld\n", fp, n, dp);
}

static void check_okey(long n) {
  long fail = 0;
  for (long i = 0; i < n; ++i) {
    uint64_t z = splitmix();
    const float a = f_of((uint32_t)z), b = f_of((uint32_t)(z >> 32));
    if (isnan(a) || isnan(b)) continue;
    // total order: key order == numeric order, with -0 below +0
    const bool lt = a < b || (a == b && signbit(a) && !signbit(b));
    if ((mxs::okey(a) < mxs::okey(b)) != lt) ++fail;
    if (b_of(mxs::okey_value(mxs::okey(a))) != b_of(a)) ++fail;
  }
  printf("okey %ld %ld\n", fail, n);
}

int main(void) {
  check_division(20000000);
  check_penalize(2000000);
  check_exp(2000000);
  check_exp_variants(2000000);
  check_okey(2000000);
  return 0;
}
