// GPU checks of the two gfx950 hardware operations the static quantiser relies on, against
// their IEEE / software definitions, over every input the kernels can give them:
//
//   rcp: recip_rn(s) (v_rcp_f32 + one FMA Newton step, tmo_device.h) == IEEE 1.0f / s for
//        every fp32 s with 2^-60 <= s <= 2^100 (the range static_scale_fast admits; the
//        operations are odd in s, so the negative range follows).
//   fp8: fp8x4 (v_cvt_pk_fp8_f32) == fp8e4m3_bits (the integer encoder, itself checked on
//        the host against a nearest-value search by div_exhaustive.hip "fp8") for every fp32
//        value in [-448, 448].
//   mfma: the operand / result lane layouts of v_mfma_f32_16x16x16_bf16 and _f16 that the
//        decode-attention kernel assumes -- lane l holds A[l % 16][4 (l / 16) + e],
//        B[4 (l / 16) + e][l % 16] and C[4 (l / 16) + e][l % 16], e = 0..3 -- on small integer
//        matrices whose products are exact, against the host's matrix product.
//   scan: wave_incl_sum_u32 (the DPP prefix sum of the grouped smooth quantiser) equals the
//        serial inclusive prefix sum over the 64 lanes, on 2^21 wavefronts of hashed counts in
//        [0, 2^25) (and on all-ones, to catch a lane that reads the wrong row).
//   recip64: the dynamic scales' fp64 reciprocal (v_rcp_f32 + two fp64 Newton steps) has
//        |1 - s * recip64(s)| <= 2^-52 for every fp32 s with 2^-60 <= s <= 2^126.
//   div64: div_recip64 (the dynamic-scale encoders' quotient: v_cvt_f64_f32, v_mul_f64,
//        v_cvt_f32_f64 with y64 = recip64(s)) against the IEEE quotient x / s for every bf16
//        and every fp16 pair 0 <= x <= amax with s = amax / 127 on the fast path: the int8
//        codes always, the quotient bits wherever the IEEE quotient is normal or 0.
//   fp8dec: the float8_e4m3fn readers of the attention and dequant kernels -- fp8_value
//        (v_cvt_f32_fp8, byte k of a dword) and the two-code v_cvt_pk_f32_fp8 +
//        v_cvt_pkrtz_f16_f32 path to f16 operands -- equal the closed-form value
//        (-1)^s (8 + m) 2^(e - 10) (m 2^-9 for e = 0) for every non-NaN code in every byte
//        position (and NaN codes decode to NaN).
//   sqrt: __builtin_sqrtf (the fused rope's rms) is correctly rounded for every positive
//        finite fp32 x: with m- and m+ the midpoints between r = sqrtf(x) and its neighbours,
//        m-^2 < x < m+^2 (25-bit midpoints square exactly in fp64; no x sits on a midpoint);
//        and so is sqrt_rn (v_sqrt_f32 + residual choice) for every x in [2^-96, FLT_MAX].
//
// Each mode launches one grid-stride kernel that counts mismatches with vector atomics and
// prints "mismatches=<n> checked=<m>"; the exit status is non-zero on any mismatch.  Built by
// __graft_entry__.build() into tests/native/_build/; run by tests/test_gpu_builtins.py.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "tmo_device.h"

namespace {

__global__ void check_rcp(uint32_t lo, uint32_t count, unsigned long long* bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned long long b = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float s = __uint_as_float(lo + i);
    if (__float_as_uint(tmo::recip_rn(s)) != __float_as_uint(1.0f / s)) ++b;
  }
  if (b) atomicAdd(bad, b);
}

// Bit patterns 0 .. hi of both signs, four consecutive patterns per conversion.
__global__ void check_fp8(uint32_t hi, unsigned long long* bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  const uint32_t quads = hi / 4 + 1;
  unsigned long long b = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < quads; i += stride) {
    for (uint32_t sign = 0; sign < 2; ++sign) {
      float f[4];
      for (int j = 0; j < 4; ++j) {
        const uint32_t u = 4 * i + j;
        f[j] = __uint_as_float((u <= hi ? u : hi) | (sign << 31));
      }
      const uint32_t hw = tmo::fp8x4(f[0], f[1], f[2], f[3]);
      for (int j = 0; j < 4; ++j)
        if (((hw >> (8 * j)) & 0xffu) != tmo::fp8e4m3_bits(f[j])) ++b;
    }
  }
  if (b) atomicAdd(bad, b);
}

// The e4m3fn value of code c by the closed form (a power-of-two scaling of an integer: exact).
__device__ float e4m3_closed_form(uint32_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  const float v = e == 0 ? __builtin_ldexpf((float)m, -9) : __builtin_ldexpf((float)(8 + m), e - 10);
  return (c & 0x80u) ? -v : v;
}

// Thread t: code c = t % 256 in byte position k = (t / 256) % 4 of a dword whose other bytes
// are other codes; checks fp8_value and the f16 operand path for the whole dword.
__global__ __launch_bounds__(256) void check_fp8dec(unsigned long long* bad) {
  const uint32_t t = blockIdx.x * 256 + threadIdx.x;  // 1024 threads
  const uint32_t c = t & 255u, k = (t >> 8) & 3u;
  uint32_t w = 0;
  for (uint32_t j = 0; j < 4; ++j) w |= ((j == k ? c : (c * 37u + 11u * j + 5u) & 255u) << (8 * j));
  unsigned long long b = 0;
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  const uint32_t h0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo[0], lo[1]));
  const uint32_t h1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(hi[0], hi[1]));
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t cj = (w >> (8 * j)) & 255u;
    const float got = tmo::fp8_value(w, (int)j);
    const float pk = j < 2 ? lo[j] : hi[j - 2];
    const uint32_t hb = ((j < 2 ? h0 : h1) >> (16 * (j & 1))) & 0xffffu;
    const float f16v = (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
    if ((cj & 0x7fu) == 0x7fu) {
      if (!__builtin_isnan(got) || !__builtin_isnan(pk)) ++b;
      continue;
    }
    const float want = e4m3_closed_form(cj);
    if (__float_as_uint(got) != __float_as_uint(want)) ++b;
    if (__float_as_uint(pk) != __float_as_uint(want)) ++b;
    if (__float_as_uint(f16v) != __float_as_uint(want)) ++b;
  }
  if (b) atomicAdd(bad, b);
}

__device__ __forceinline__ uint32_t scan_value(uint32_t wave, uint32_t lane) {
  if (wave == 0) return 1u;  // all ones: lane l must hold l + 1
  uint32_t h = wave * 0x9E3779B1u ^ (lane + 0x7F4A7C15u) * 0x85EBCA77u;
  h ^= h >> 15;
  h *= 0x2C1B3C6Du;
  h ^= h >> 12;
  // mostly small counts, sometimes zero, sometimes near the 2^25 bound
  const uint32_t k = h & 3u;
  return k == 0 ? 0u : (k == 1 ? (h >> 8) & 0x1FFu : (k == 2 ? (h >> 7) & 0x1FFFFFFu : 1u));
}

__global__ __launch_bounds__(256) void check_scan(uint32_t waves, unsigned long long* bad) {
  const uint32_t lane = threadIdx.x & 63u;
  unsigned long long b = 0;
  for (uint32_t w = blockIdx.x * 4 + threadIdx.x / 64; w < waves; w += gridDim.x * 4) {
    const uint32_t got = tmo::wave_incl_sum_u32(scan_value(w, lane));
    uint32_t want = 0;
    for (uint32_t j = 0; j <= lane; ++j) want += scan_value(w, j);
    if (got != want) ++b;
  }
  if (b) atomicAdd(bad, b);
}

__global__ void check_recip64(uint32_t lo, uint32_t count, unsigned long long* bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned long long b = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float s = __uint_as_float(lo + i);
    const double e = __builtin_fma(-(double)s, tmo::recip64(s), 1.0);  // exact 1 - s*y, rounded once
    if (!(__builtin_fabs(e) <= 0x1p-52)) ++b;
  }
  if (b) atomicAdd(bad, b);
}

// One workgroup per amax bit pattern (blockIdx.x + 1), its threads striding over x in [0, amax].
template <bool kF16>
__global__ __launch_bounds__(256) void check_div64(uint32_t max_bits, unsigned long long* bad) {
  const uint32_t a = blockIdx.x + 1;
  if (a > max_bits) return;
  const float amax = kF16 ? tmo::f16_bits_to_f32(a) : __uint_as_float(a << 16);
  const float s = amax / 127.0f;
  if (!(s >= tmo::kFastDivMinScale) || !(s < __builtin_inff())) return;
  const double y64 = tmo::recip64(s);
  unsigned long long b = 0;
  for (uint32_t xb = threadIdx.x; xb <= a; xb += blockDim.x) {
    const float x = kF16 ? tmo::f16_bits_to_f32(xb) : __uint_as_float(xb << 16);
    const float q = tmo::div_recip64(x, y64), r = x / s;
    const float cq = __builtin_rintf(__builtin_amdgcn_fmed3f(q, -128.0f, 127.0f));
    const float cr = __builtin_rintf(__builtin_amdgcn_fmed3f(r, -128.0f, 127.0f));
    const bool exact = __builtin_fabsf(r) >= 0x1p-126f || r == 0.0f;
    if (cq != cr || (exact && __float_as_uint(q) != __float_as_uint(r))) ++b;
  }
  if (b) atomicAdd(bad, b);
}

// Pairs check_div64 compares (the same fast-path test on the host's IEEE division).
unsigned long long div64_pairs(uint32_t max_bits, bool f16) {
  unsigned long long n = 0;
  for (uint32_t a = 1; a <= max_bits; ++a) {
    float amax;
    if (f16) {
      const uint32_t e = (a >> 10) & 0x1f, m = a & 0x3ff;
      if (e == 0) {
        amax = (float)m * 5.9604644775390625e-08f;
      } else {
        const uint32_t u = ((e + 112u) << 23) | (m << 13);
        std::memcpy(&amax, &u, 4);
      }
    } else {
      const uint32_t u = a << 16;
      std::memcpy(&amax, &u, 4);
    }
    const float s = amax / 127.0f;
    if (s >= tmo::kFastDivMinScale && s < __builtin_inff()) n += a + 1;
  }
  return n;
}

__global__ void check_sqrt(unsigned long long* bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned long long b = 0;
  for (uint32_t u = 1 + blockIdx.x * blockDim.x + threadIdx.x; u < 0x7f800000u; u += stride) {
    const float x = __uint_as_float(u);
    const double xd = (double)x;
    auto rounded = [xd](float r) {
      const uint32_t rb = __float_as_uint(r);
      const double rd = (double)r;
      const double lo = 0.5 * (rd + (double)__uint_as_float(rb - 1));
      const double hi = 0.5 * (rd + (double)__uint_as_float(rb + 1));
      return lo * lo < xd && xd < hi * hi;
    };
    if (!rounded(__builtin_sqrtf(x))) ++b;
    if (x >= tmo::kSqrtMin && !rounded(tmo::sqrt_rn(x))) ++b;
  }
  if (b) atomicAdd(bad, b);
}

typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One wavefront: operands gathered from row-major 16x16 A and B by the assumed layout, the
// four result registers of every lane written to c[lane][e].  kF16: f16 inputs, else bf16.
template <bool kF16>
__global__ void mfma_layout(const float* a, const float* b, float* c) {
  const int l = threadIdx.x;
  const int r = l % 16, g = l / 16;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kF16) {
    f16x4 av, bv;
    for (int e = 0; e < 4; ++e) {
      av[e] = (_Float16)a[r * 16 + 4 * g + e];
      bv[e] = (_Float16)b[(4 * g + e) * 16 + r];
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bv, acc, 0, 0, 0);
  } else {
    bf16x4 av, bv;
    for (int e = 0; e < 4; ++e) {  // small integers: the upper half of the fp32 is exact bf16
      av[e] = (short)(__float_as_uint(a[r * 16 + 4 * g + e]) >> 16);
      bv[e] = (short)(__float_as_uint(b[(4 * g + e) * 16 + r]) >> 16);
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc, 0, 0, 0);
  }
  for (int e = 0; e < 4; ++e) c[l * 4 + e] = acc[e];
}

// Host side of "mfma": both input types; returns the mismatch count.
unsigned long long run_mfma(unsigned long long& checked) {
  float ha[256], hb[256], want[256], got[256];
  for (int m = 0; m < 16; ++m)
    for (int k = 0; k < 16; ++k) {
      ha[m * 16 + k] = (float)((m * 3 + k * 7) % 17 - 8);
      hb[m * 16 + k] = (float)((m * 5 + k * 11) % 13 - 6);
    }
  for (int m = 0; m < 16; ++m)
    for (int n = 0; n < 16; ++n) {
      float s = 0.0f;
      for (int k = 0; k < 16; ++k) s += ha[m * 16 + k] * hb[k * 16 + n];
      want[m * 16 + n] = s;
    }
  float *da = nullptr, *db = nullptr, *dc = nullptr;
  if (hipMalloc(&da, sizeof ha) != hipSuccess || hipMalloc(&db, sizeof hb) != hipSuccess ||
      hipMalloc(&dc, sizeof got) != hipSuccess ||
      hipMemcpy(da, ha, sizeof ha, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(db, hb, sizeof hb, hipMemcpyHostToDevice) != hipSuccess)
    return ~0ull;
  unsigned long long bad = 0;
  for (int variant = 0; variant < 2; ++variant) {
    if (variant == 0) {
      mfma_layout<false><<<dim3(1), dim3(64)>>>(da, db, dc);
    } else {
      mfma_layout<true><<<dim3(1), dim3(64)>>>(da, db, dc);
    }
    if (hipMemcpy(got, dc, sizeof got, hipMemcpyDeviceToHost) != hipSuccess) return ~0ull;
    for (int l = 0; l < 64; ++l)
      for (int e = 0; e < 4; ++e) {
        ++checked;
        if (got[l * 4 + e] != want[(4 * (l / 16) + e) * 16 + l % 16]) ++bad;
      }
  }
  hipFree(da);
  hipFree(db);
  hipFree(dc);
  return bad;
}

}  // namespace

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "rcp";
  unsigned long long* d_bad = nullptr;
  if (hipMalloc(&d_bad, sizeof(unsigned long long)) != hipSuccess ||
      hipMemset(d_bad, 0, sizeof(unsigned long long)) != hipSuccess) {
    std::printf("device setup failed\n");
    return 2;
  }
  unsigned long long checked = 0;
  if (!std::strcmp(mode, "rcp")) {
    uint32_t lo, hi;
    const float flo = tmo::kStaticMinScale, fhi = tmo::kStaticMaxScale;
    std::memcpy(&lo, &flo, 4);
    std::memcpy(&hi, &fhi, 4);
    checked = (unsigned long long)(hi - lo) + 1;
    check_rcp<<<dim3(8192), dim3(256)>>>(lo, hi - lo + 1, d_bad);
  } else if (!std::strcmp(mode, "fp8")) {
    uint32_t hi;
    const float fhi = 448.0f;
    std::memcpy(&hi, &fhi, 4);
    checked = 2ull * ((unsigned long long)(hi / 4) + 1) * 4;
    check_fp8<<<dim3(8192), dim3(256)>>>(hi, d_bad);
  } else if (!std::strcmp(mode, "fp8dec")) {
    checked = 1024ull * 4;
    check_fp8dec<<<dim3(4), dim3(256)>>>(d_bad);
  } else if (!std::strcmp(mode, "mfma")) {
    const unsigned long long b = run_mfma(checked);
    if (b == ~0ull) {
      std::printf("mfma setup failed\n");
      return 2;
    }
    std::printf("mode=%s mismatches=%llu checked=%llu\n", mode, b, checked);
    return b == 0 ? 0 : 1;
  } else if (!std::strcmp(mode, "scan")) {
    const uint32_t waves = 1u << 21;
    checked = 64ull * waves;
    check_scan<<<dim3(4096), dim3(256)>>>(waves, d_bad);
  } else if (!std::strcmp(mode, "recip64")) {
    uint32_t lo, hi;
    const float flo = tmo::kFastDivMinScale, fhi = 0x1p126f;
    std::memcpy(&lo, &flo, 4);
    std::memcpy(&hi, &fhi, 4);
    checked = (unsigned long long)(hi - lo) + 1;
    check_recip64<<<dim3(8192), dim3(256)>>>(lo, hi - lo + 1, d_bad);
  } else if (!std::strcmp(mode, "div64")) {
    checked = div64_pairs(0x7f7fu, false) + div64_pairs(0x7bffu, true);
    check_div64<false><<<dim3(0x7f7fu), dim3(256)>>>(0x7f7fu, d_bad);
    check_div64<true><<<dim3(0x7bffu), dim3(256)>>>(0x7bffu, d_bad);
  } else if (!std::strcmp(mode, "sqrt")) {
    float smin = tmo::kSqrtMin;
    uint32_t umin;
    std::memcpy(&umin, &smin, 4);
    checked = (0x7f800000ull - 1) + (0x7f800000ull - umin);
    check_sqrt<<<dim3(8192), dim3(256)>>>(d_bad);
  } else {
    std::printf("unknown mode %s\n", mode);
    return 2;
  }
  unsigned long long bad = 0;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&bad, d_bad, sizeof(bad), hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("kernel failed\n");
    return 3;
  }
  std::printf("mode=%s mismatches=%llu checked=%llu\n", mode, bad, checked);
  return bad == 0 ? 0 : 1;
}
