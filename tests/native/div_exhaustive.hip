// Host-side check of the kernels' quotients (div_recip64, the fp64-product quotient of the
// dynamic-scale encoders, and div_by_recip, the fp32 FMA quotient of the static scales, in
// tmo_device.h, the same source the gfx950 kernels compile) against IEEE fp32 division.
//
//   bf16 : every positive finite bf16 amax whose scale amax/127 is on the fast path, against
//          every bf16 x with 0 <= x <= amax (the quotient is odd in x, so this covers -x);
//          both quotients.
//   f16  : the same over all finite fp16 values.
//   f32  : random fp32 (amax, x) pairs over the fast-path exponent range plus, for each
//          scale, inputs within +-3 ulps of (k + 0.5) * scale for every k in [-127, 127];
//          both quotients.
//   scale: the divide-free row scale (scale_of) against IEEE amax / 127 for EVERY fp32 amax
//          the kernels send through it (2^-100 up to the largest finite value).
//   static: the static-scale quotient (static_quotients, per-element lane logic) for random
//          scales 2^-60 <= |s| <= 2^100 of both signs, against x with quotients spread over
//          2^-40 .. 2^24, within +-3 ulps of int8 ties (k + 0.5) * s and of fp8 e4m3 ties
//          m * s, near |x| = 2^-100, and +-0; the int8 code and the fp8 code (with the sign
//          of a zero quotient put back, as the fp8 paths do) must always match, the quotient
//          bits whenever |x| >= 2^-100 and the IEEE quotient is normal, or x is zero.
//   fp8:   fp8e4m3_bits against a nearest-value search over the 127 positive e4m3 values
//          (ties to the even code) for EVERY fp32 value in [-448, 448].
//   sqrt:  sqrt_choose (the correction step of the fused rope's square root) for EVERY fp32
//          a in [2^-96, FLT_MAX], given the correctly rounded root or a neighbour of it.
//
// Two properties are checked on every pair:
//   * the int8 code (clamp to [-128, 127], round half to even) of the kernel quotient equals
//     the code of the IEEE quotient -- always;
//   * the quotient bits themselves are identical: for div_by_recip whenever |x| >= 2^-100
//     (below that the FMA residual can underflow and the last bit may differ, but
//     |x / s| < 2^-40 there), for div_recip64 whenever the IEEE quotient is normal or zero.
// Prints "mismatches=<n> checked=<m>" and exits non-zero on any mismatch.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "tmo_device.h"

static float f_from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits_of(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
static float bf16(uint32_t h) { return f_from_bits(h << 16); }
static float f16(uint32_t h) {
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return (float)m * 5.9604644775390625e-08f;
  return f_from_bits(((e + 112u) << 23) | (m << 13));
}

struct Count {
  unsigned long long bad = 0, checked = 0;
};

static int code_of(float q) { return (int)std::nearbyintf(std::fmin(std::fmax(q, -128.0f), 127.0f)); }

// True when the pair violates one of the two properties above.
static bool differs(float x, float q, float r) {
  if (code_of(q) != code_of(r)) return true;
  return std::fabs(x) >= 0x1p-100f && bits_of(q) != bits_of(r);
}
static bool differs64(float q, float r) {
  if (code_of(q) != code_of(r)) return true;
  return (std::fabs(r) >= 0x1p-126f || r == 0.0f) && bits_of(q) != bits_of(r);
}

// Both quotients of one pair against the IEEE quotient r.
static void check_pair(float amax, float x, float s, float y, double y64, Count& c) {
  const float q = tmo::div_by_recip(x, s, y);
  const float q64 = tmo::div_recip64(x, y64);
  const float r = x / s;
  ++c.checked;
  if (differs(x, q, r) || differs64(q64, r)) {
    if (c.bad < 5)
      std::printf("mismatch amax=%a x=%a s=%a fma=%a fp64=%a ieee=%a\n", amax, x, s, q, q64, r);
    ++c.bad;
  }
}

// One amax: all x in [0, amax] of the format.
template <class Conv>
static void check_amax(uint32_t a, Conv conv, Count& c) {
  const float amax = conv(a);
  const float s = amax / 127.0f;
  if (!(s >= tmo::kFastDivMinScale) || !(s < INFINITY)) return;  // IEEE path in the kernel
  const float y = 1.0f / s;
  const double y64 = 1.0 / (double)s;
  for (uint32_t xb = 0; xb <= a; ++xb) check_pair(amax, conv(xb), s, y, y64, c);
}

template <class Conv>
static Count run_format(uint32_t max_bits, Conv conv, int nthreads) {
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      for (uint32_t a = 1 + t; a <= max_bits; a += nthreads) check_amax(a, conv, per[t]);
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  return total;
}

static Count run_f32(unsigned long long n, int nthreads) {
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      std::mt19937_64 rng(1234 + t);
      Count& c = per[t];
      for (unsigned long long i = t; i < n; i += nthreads) {
        // amax: exponent 2^-60 .. 2^127, random significand
        const uint32_t e = 67 + (uint32_t)(rng() % 188);
        const float amax = f_from_bits((e << 23) | (uint32_t)(rng() & 0x7fffff));
        const float s = amax / 127.0f;
        if (!(s >= tmo::kFastDivMinScale) || !(s < INFINITY)) continue;
        const float y = 1.0f / s;
        const double y64 = 1.0 / (double)s;
        float xs[15];
        // random x in [-amax, amax] and near-ties around (k + 0.5) * s
        const double u = (double)(rng() >> 11) / 9007199254740992.0;
        xs[0] = (float)((2.0 * u - 1.0) * amax);
        const int k = (int)(rng() % 255) - 127;
        const float t0 = (float)((k + 0.5) * (double)s);
        for (int d = 0; d < 7; ++d) xs[1 + d] = f_from_bits(bits_of(t0) + (uint32_t)(d - 3));
        // x near m * s for a midpoint m between two adjacent fp32 quotients in (0, 127]: the
        // quotient's own rounding boundary
        const float qa = f_from_bits(0x3f800000u + (uint32_t)(rng() % (0x42fe0000u - 0x3f800000u)));
        const double mq = 0.5 * ((double)qa + (double)f_from_bits(bits_of(qa) + 1u));
        const float t1 = (float)(mq * (double)s) * ((rng() & 1) ? -1.0f : 1.0f);
        for (int d = 0; d < 7; ++d) xs[8 + d] = f_from_bits(bits_of(t1) + (uint32_t)(d - 3));
        for (float x : xs) {
          if (!(std::fabs(x) <= amax)) continue;
          check_pair(amax, x, s, y, y64, c);
        }
      }
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  return total;
}

static Count run_scale(int nthreads) {
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  const uint32_t lo = bits_of(tmo::kScaleDivMin), hi = 0x7f7fffffu;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      Count& c = per[t];
      for (uint32_t b = lo + t; b <= hi; b += nthreads) {
        const float amax = f_from_bits(b);
        const float s = tmo::scale_of(amax), r = amax / 127.0f;
        ++c.checked;
        if (bits_of(s) != bits_of(r)) {
          if (c.bad < 5) std::printf("scale mismatch amax=%a fast=%a ieee=%a\n", amax, s, r);
          ++c.bad;
        }
      }
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  return total;
}

// ---- square root choice

// sqrt_choose (the kernels' sqrt_rn after v_sqrt_f32) for EVERY fp32 a in [2^-96, FLT_MAX]:
// given the correctly rounded root r = sqrtf(a) or either of its neighbours as the approximate
// root s, it must return r.
static Count run_sqrt(int nthreads) {
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  const uint32_t lo = bits_of(tmo::kSqrtMin), hi = 0x7f7fffffu;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      Count& c = per[t];
      for (uint32_t b = lo + t; b <= hi; b += nthreads) {
        const float a = f_from_bits(b);
        const float r = std::sqrt(a);
        for (int d = -1; d <= 1; ++d) {
          const float s = f_from_bits(bits_of(r) + (uint32_t)d);
          const float got = tmo::sqrt_choose(a, s);
          ++c.checked;
          if (bits_of(got) != bits_of(r)) {
            if (c.bad < 5) std::printf("sqrt mismatch a=%a s=%a got=%a ieee=%a\n", a, s, got, r);
            ++c.bad;
          }
        }
      }
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  return total;
}

// ---- static scales

static uint32_t fp8_of(float q) { return tmo::fp8e4m3_bits(std::fmin(std::fmax(q, -448.0f), 448.0f)); }

// Value of positive e4m3 code c (1..126).
static double e4m3_value(int c) {
  const int e = c >> 3, m = c & 7;
  return e == 0 ? m * std::ldexp(1.0, -9) : (8 + m) * std::ldexp(1.0, e - 10);
}

static Count run_static(unsigned long long n, int nthreads) {
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      std::mt19937_64 rng(777 + t);
      Count& c = per[t];
      for (unsigned long long i = t; i < n; i += nthreads) {
        const uint32_t e = 67 + (uint32_t)(rng() % 161);  // 2^-60 .. 2^100
        const uint32_t sign = (rng() % 5 == 0) ? 0x80000000u : 0u;
        const float s = f_from_bits(sign | (e << 23) | (uint32_t)(rng() & 0x7fffff));
        if (!tmo::static_scale_fast(s)) continue;
        const float y = 1.0f / s;
        float xs[20];
        int nx = 0;
        // quotient magnitude log-uniform in 2^-40 .. 2^24, either sign
        const double lq = -40.0 + 64.0 * (double)(rng() >> 11) / 9007199254740992.0;
        xs[nx++] = (float)(std::ldexp(1.0, 0) * std::exp2(lq) * (double)s * ((rng() & 1) ? -1.0 : 1.0));
        const int k = (int)(rng() % 261) - 130;
        const float t0 = (float)((k + 0.5) * (double)s);
        for (int d = 0; d < 7; ++d) xs[nx++] = f_from_bits(bits_of(t0) + (uint32_t)(d - 3));
        // midpoint between two adjacent e4m3 values
        const int c8 = 1 + (int)(rng() % 125);
        const double mid = 0.5 * (e4m3_value(c8) + e4m3_value(c8 + 1)) * ((rng() & 1) ? -1.0 : 1.0);
        const float t1 = (float)(mid * (double)s);
        for (int d = 0; d < 7; ++d) xs[nx++] = f_from_bits(bits_of(t1) + (uint32_t)(d - 3));
        xs[nx++] = f_from_bits(bits_of(0x1p-100f) + (uint32_t)(rng() % 64)) * ((rng() & 1) ? -1.0f : 1.0f);
        xs[nx++] = 0.0f;
        xs[nx++] = -0.0f;
        for (int j = 0; j < nx; ++j) {
          const float x = xs[j];
          if (!std::isfinite(x)) continue;
          float q, qs;
          tmo::static_quotients<1>(&x, &s, &y, true, &q);
          tmo::static_quotients<1, true>(&x, &s, &y, true, &qs);  // the fp8 paths' quotient
          const float r = x / s;
          ++c.checked;
          const bool exact = std::fabs(x) >= 0x1p-100f && std::fabs(r) >= 0x1p-126f;
          const bool bad = code_of(q) != code_of(r) || fp8_of(qs) != fp8_of(r) ||
                           (exact && bits_of(q) != bits_of(r)) ||
                           ((exact || x == 0.0f) && bits_of(qs) != bits_of(r));
          if (bad) {
            if (c.bad < 5) std::printf("static mismatch s=%a x=%a fast=%a ieee=%a\n", s, x, qs, r);
            ++c.bad;
          }
        }
      }
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  return total;
}

// ---- fp8 encoder

static uint32_t fp8_reference(float f) {
  const double a = std::fabs((double)f);
  int best = 0;
  double bd = a;  // distance to code 0
  for (int c = 1; c <= 126; ++c) {
    const double d = std::fabs(a - e4m3_value(c));
    if (d < bd || (d == bd && (c & 1) == 0 && (best & 1) == 1)) {
      bd = d;
      best = c;
    }
  }
  return (std::signbit(f) ? 0x80u : 0u) | (uint32_t)best;
}

static Count run_fp8(int nthreads) {
  // table of the 127 positive values for a binary search
  std::vector<double> vals(127);
  for (int c = 0; c <= 126; ++c) vals[c] = c ? e4m3_value(c) : 0.0;
  std::vector<Count> per(nthreads);
  std::vector<std::thread> th;
  const uint32_t hi = bits_of(448.0f);
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      Count& c = per[t];
      for (uint32_t b = t; b <= hi; b += nthreads) {
        for (uint32_t sgn = 0; sgn < 2; ++sgn) {
          const float f = f_from_bits(b | (sgn << 31));
          const double a = std::fabs((double)f);
          // nearest of vals[lo], vals[lo + 1] with ties to the even code
          int lo = (int)(std::upper_bound(vals.begin(), vals.end(), a) - vals.begin()) - 1;
          int best = lo;
          if (lo < 126) {
            const double d0 = a - vals[lo], d1 = vals[lo + 1] - a;
            if (d1 < d0 || (d1 == d0 && ((lo + 1) & 1) == 0)) best = lo + 1;
          }
          const uint32_t want = (sgn ? 0x80u : 0u) | (uint32_t)best;
          ++c.checked;
          if (tmo::fp8e4m3_bits(f) != want) {
            if (c.bad < 5) std::printf("fp8 mismatch f=%a got=%#x want=%#x\n", f, tmo::fp8e4m3_bits(f), want);
            ++c.bad;
          }
        }
      }
    });
  for (auto& x : th) x.join();
  Count total;
  for (auto& p : per) {
    total.bad += p.bad;
    total.checked += p.checked;
  }
  // spot-check the search against the brute-force reference
  for (float f : {0.0f, -0.0f, 1.0f / 1024, 3.0f / 1024, 0.0087890625f, 240.0f, 248.0f, 440.0f, 448.0f, -13.0f})
    if (fp8_reference(f) != tmo::fp8e4m3_bits(f)) ++total.bad;
  return total;
}

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "bf16";
  const int nthreads = argc > 2 ? std::atoi(argv[2]) : 8;
  Count c;
  if (!std::strcmp(mode, "bf16")) {
    c = run_format(0x7f7fu, bf16, nthreads);
  } else if (!std::strcmp(mode, "f16")) {
    c = run_format(0x7bffu, f16, nthreads);
  } else if (!std::strcmp(mode, "scale")) {
    c = run_scale(nthreads);
  } else if (!std::strcmp(mode, "static")) {
    c = run_static(argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 4000000ull, nthreads);
  } else if (!std::strcmp(mode, "fp8")) {
    c = run_fp8(nthreads);
  } else if (!std::strcmp(mode, "sqrt")) {
    c = run_sqrt(nthreads);
  } else {
    const unsigned long long n = argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 20000000ull;
    c = run_f32(n, nthreads);
  }
  std::printf("mismatches=%llu checked=%llu\n", c.bad, c.checked);
  return c.bad == 0 ? 0 : 1;
}
