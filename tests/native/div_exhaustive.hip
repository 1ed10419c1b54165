// Host-side check of the kernels' quotient (div_by_recip in tmo_device.h, the same source the
// gfx950 kernels compile) against IEEE fp32 division.
//
//   bf16 : every positive finite bf16 amax whose scale amax/127 is on the fast path, against
//          every bf16 x with 0 <= x <= amax (the quotient is odd in x, so this covers -x).
//   f16  : the same over all finite fp16 values.
//   f32  : random fp32 (amax, x) pairs over the fast-path exponent range plus, for each
//          scale, inputs within +-3 ulps of (k + 0.5) * scale for every k in [-127, 127].
//   scale: the divide-free row scale (scale_of) against IEEE amax / 127 for EVERY fp32 amax
//          the kernels send through it (2^-100 up to the largest finite value).
//
// Two properties are checked on every pair:
//   * the int8 code (clamp to [-128, 127], round half to even) of the kernel quotient equals
//     the code of the IEEE quotient -- always;
//   * the quotient bits themselves are identical whenever |x| >= 2^-100 (below that the FMA
//     residual can underflow and the last bit may differ, but |x / s| < 2^-40 there).
// Prints "mismatches=<n> checked=<m>" and exits non-zero on any mismatch.
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

// One amax: all x in [0, amax] of the format.
template <class Conv>
static void check_amax(uint32_t a, Conv conv, Count& c) {
  const float amax = conv(a);
  const float s = amax / 127.0f;
  if (!(s >= tmo::kFastDivMinScale) || !(s < INFINITY)) return;  // IEEE path in the kernel
  const float y = 1.0f / s;
  for (uint32_t xb = 0; xb <= a; ++xb) {
    const float x = conv(xb);
    const float q = tmo::div_by_recip(x, s, y);
    const float r = x / s;
    ++c.checked;
    if (differs(x, q, r)) {
      if (c.bad < 5)
        std::printf("mismatch amax=%a x=%a s=%a fast=%a ieee=%a\n", amax, x, s, q, r);
      ++c.bad;
    }
  }
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
        float xs[8];
        // random x in [-amax, amax] and near-ties around (k + 0.5) * s
        const double u = (double)(rng() >> 11) / 9007199254740992.0;
        xs[0] = (float)((2.0 * u - 1.0) * amax);
        const int k = (int)(rng() % 255) - 127;
        const float t0 = (float)((k + 0.5) * (double)s);
        for (int d = 0; d < 7; ++d) xs[1 + d] = f_from_bits(bits_of(t0) + (uint32_t)(d - 3));
        for (float x : xs) {
          if (!(std::fabs(x) <= amax)) continue;
          const float q = tmo::div_by_recip(x, s, y);
          const float r = x / s;
          ++c.checked;
          if (differs(x, q, r)) {
            if (c.bad < 5) std::printf("mismatch amax=%a x=%a s=%a fast=%a ieee=%a\n", amax, x, s, q, r);
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
  } else {
    const unsigned long long n = argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 20000000ull;
    c = run_f32(n, nthreads);
  }
  std::printf("mismatches=%llu checked=%llu\n", c.bad, c.checked);
  return c.bad == 0 ? 0 : 1;
}
