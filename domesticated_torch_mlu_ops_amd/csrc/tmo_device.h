// Device-side building blocks shared by the gfx950 kernels of libtmo_hip.so.
//
// Everything here is wave64-native: row reductions run inside DPP rows (16 lanes) or
// across the whole wavefront, loads and stores are 16-byte vectors, and the int8 encoder
// is written so that the per-element cost stays a handful of VALU ops (the path is
// HBM-bound, the division must not make it VALU-bound).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

#include "tmo_hip.h"

namespace tmo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// MI355X: 8 XCDs of 32 CUs, each with its own L2; workgroups are dispatched round-robin over
// them, so workgroup b runs on XCD b % kXcds.
constexpr int kXcds = 8;

// XCD-aware (token tile, head) of workgroup b for kernels whose grid is tiles x heads: the
// heads of one tile run on one XCD (slot = b / 8, head = slot % heads, tile = 8 * (slot /
// heads) + b % 8), so a tile's bytes meet in one L2 -- per-token scale lines shared by
// neighbouring heads are written or read whole, and the tile's rows go to HBM from one XCD.
// The grid must hold a whole number of groups of 8 tiles (xcd_grid_tiles).
__device__ __forceinline__ void xcd_tile_head(uint32_t b, int heads, int& h, int64_t& tile) {
  const uint32_t slot = b / kXcds;
  h = (int)(slot % (uint32_t)heads);
  tile = (int64_t)(slot / (uint32_t)heads) * kXcds + b % kXcds;
}
inline int64_t xcd_grid_tiles(int64_t tiles) { return (tiles + kXcds - 1) / kXcds * kXcds; }

// ---------------------------------------------------------------------------- element types

// Storage tags for the three input/output float formats.  Each maps a 16-byte vector to
// `kPerVec` fp32 values and back.
struct F32 {
  static constexpr int kBytes = 4;
  static constexpr int kPerVec = 4;
};
struct F16 {
  static constexpr int kBytes = 2;
  static constexpr int kPerVec = 8;
};
struct BF16 {
  static constexpr int kBytes = 2;
  static constexpr int kPerVec = 8;
};

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Unpack one 16-byte vector into fp32 values (exact for all three formats).
__device__ __forceinline__ void unpack(F32, const u32x4& w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
}
__device__ __forceinline__ void unpack(BF16, const u32x4& w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack(F16, const u32x4& w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
    v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
  }
}

// Scalar element load (generic / unaligned paths).
__device__ __forceinline__ float load1(F32, const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
__device__ __forceinline__ float load1(BF16, const void* p, int64_t i) {
  return __uint_as_float((uint32_t) static_cast<const uint16_t*>(p)[i] << 16);
}
__device__ __forceinline__ float load1(F16, const void* p, int64_t i) {
  return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// fp32 -> 16-bit formats, round to nearest even (hardware conversions: v_cvt_pk_bf16_f32
// on gfx950, v_cvt_f16_f32 for fp16; both honour the default RNE mode).
//
// The value is pinned in a VGPR first: without the barrier the backend folds a preceding
// fp32 multiply into the conversion (v_fma_mixlo_f16), which rounds the exact product once
// to fp16 instead of rounding it to fp32 and then to fp16 as the reference's
// `(code.to(float32) * scale).to(dtype)` does -- a 1-ulp difference on double-rounding cases.
__device__ __forceinline__ float materialize(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint16_t to_bits(BF16, float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)materialize(v));
}
__device__ __forceinline__ uint16_t to_bits(F16, float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)materialize(v));
}
template <class Tag>
__device__ __forceinline__ uint32_t pack2(Tag, float lo, float hi) {
  return (uint32_t)to_bits(Tag{}, lo) | ((uint32_t)to_bits(Tag{}, hi) << 16);
}
__device__ __forceinline__ void store1(F32, void* p, int64_t i, float v) {
  static_cast<float*>(p)[i] = v;
}
template <class Tag>
__device__ __forceinline__ void store1(Tag, void* p, int64_t i, float v) {
  static_cast<uint16_t*>(p)[i] = to_bits(Tag{}, v);
}

// ---------------------------------------------------------------------------- reductions

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadSwap1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i inside each 8-lane half row
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i inside each 16-lane row

// All controls used here permute inside a row, so no lane reads out of bounds and
// bound_ctrl only lets the compiler fold the move into the consuming max (v_max_u32_dpp).
template <int Ctrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Ctrl, 0xF, 0xF, true);
}

// Max over aligned groups of G lanes (G a power of two <= 64).  Every lane of the group
// receives the result.  Groups of <= 16 lanes never leave their DPP row; 32/64 use
// cross-row lane shuffles.  The whole group must be active.
template <int G>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  if constexpr (G >= 2) v = max(v, dpp<kDppQuadSwap1>(v));
  if constexpr (G >= 4) v = max(v, dpp<kDppQuadSwap2>(v));
  if constexpr (G >= 8) v = max(v, dpp<kDppRowHalfMirror>(v));
  if constexpr (G >= 16) v = max(v, dpp<kDppRowMirror>(v));
  if constexpr (G >= 32) v = max(v, (uint32_t)__shfl_xor((int)v, 16, 64));
  if constexpr (G >= 64) v = max(v, (uint32_t)__shfl_xor((int)v, 32, 64));
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wavefront, in DPP steps (no LDS round trips):
// sums inside each 16-lane row (row_shr 1, 2, 4, 8, lanes shifted in from outside the row
// read 0), then row 1 and row 3 add the last lane of the row before them (row_bcast:15), then
// rows 2 and 3 add lane 31 (row_bcast:31).  The whole wavefront must be active.
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;
__device__ __forceinline__ uint32_t wave_incl_sum_u32(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr1, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr2, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr4, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr8, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast15, 0xA, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast31, 0xC, 0xF, false);
  return v;
}

// Maximum over the whole wavefront as a scalar: the 16-lane DPP reduction, then the four row
// results read into scalar registers (no cross-row lane shuffle through LDS).
__device__ __forceinline__ uint32_t wave_max_u32_sgpr(uint32_t v) {
  v = group_max_u32<16>(v);
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Maximum over the whole wavefront, returned as a wave-uniform value: every lane holds the
// same result after group_max_u32<64>, and readfirstlane tells the compiler so, which turns
// branches on values derived from it (the encoder's fast / IEEE path choice) into scalar
// branches instead of exec-masked code that keeps both paths' registers live.
__device__ __forceinline__ float wave_max_uniform(float m) {
  return __uint_as_float(
      (uint32_t)__builtin_amdgcn_readfirstlane((int)group_max_u32<kWave>(__float_as_uint(m))));
}

// ---------------------------------------------------------------------------- int8 encoder

// Rows whose scale is below this use a true IEEE divide per element; above it the
// reciprocal-based quotient div_recip64 below gives the IEEE quotient for every x.
constexpr float kFastDivMinScale = 8.6736174e-19f;  // 2^-60

// x / s given y = RN(1 / s) and kFastDivMinScale <= s < inf, in fp32 arithmetic (the static
// scales' quotient, where y is computed per channel).
// q0 = RN(x*y) is within ~2 ulp of x/s; one FMA correction step makes it faithful; a second
// (Markstein's theorem: y within 1/2 ulp of 1/s and q faithful => r = x - s*q is exact and
// RN(q + r*y) = RN(x/s)) makes it the IEEE quotient.  P. Markstein, IBM J. Res. Dev. 34(1),
// 1990; Muller et al., Handbook of Floating-Point Arithmetic, 2nd ed., ch. 4 (FMA division).
// The theorem needs the residual not to underflow: for |x| >= 2^-100 the result is the IEEE
// quotient bit for bit; below that its last bit may differ, but then |x / s| < 2^-40 and the
// int8 code (0) is the same.  tests/native/div_exhaustive.hip checks both statements on
// every bf16 and every fp16 (amax, x) pair and on random / near-tie fp32 pairs.
__host__ __device__ __forceinline__ float div_by_recip(float x, float s, float y) {
  float q0 = x * y;
  float r0 = __builtin_fmaf(-s, q0, x);
  float q1 = __builtin_fmaf(r0, y, q0);
  float r1 = __builtin_fmaf(-s, q1, x);
  return __builtin_fmaf(r1, y, q1);
}

// x / s given y64 within 2^-51 (relative) of 1 / s (recip64 below), for finite x and finite
// s > 0: the fp64 product rounded to fp32 is the IEEE fp32 quotient.  Why: a quotient x / s of
// two fp32 numbers is either an fp32 number or at least 2^-49 (relative) away from every
// midpoint m = M * 2^c between adjacent fp32 numbers (M odd, 2^24 < M < 2^25).  x - s * m is
// never 0, since its odd part would need x's 24-bit significand to hold the odd factor
// M > 2^24.  It is a multiple of 2^min(e_x, e_s + c), which bounds |x / s - m| / m below by
// 1 / (S * M) > 2^-49 or by 1 / X > 2^-24, with X, S the 24-bit significands.  y64 and the
// RN64 product add at most 2^-51 + 2^-53 relative error, so x * y64 lies on the same side of
// every midpoint as x / s, and within 2^-50 of x / s where that is an fp32 number.  Where the
// IEEE quotient is subnormal (|x / s| < 2^-126) the last bit may differ.  The int8, int4 and
// fp8 codes are 0 there either way, and the sign is x's, as in the IEEE quotient, zero
// quotients included.  Three VALU instructions (v_cvt_f64_f32, v_mul_f64, v_cvt_f32_f64, all
// full rate on gfx950) against div_by_recip's five.  tests/native/div_exhaustive.hip checks it
// with y64 = RN64(1 / s) against IEEE division on every bf16 and every fp16 (amax, x) pair and
// on random and near-tie fp32 pairs; tests/native/gfx950_builtins.hip ("div64") checks it on
// the GPU with recip64 on every bf16 and fp16 pair.
__host__ __device__ __forceinline__ float div_recip64(float x, double y64) {
  return (float)((double)x * y64);
}

// 1 / s in fp64 for the dynamic scales, 2^-60 <= s <= 2^126 (kFastDivMinScale up to amax / 7,
// amax / 127 or amax / 448 of a finite amax): v_rcp_f32 (within 1 ulp, a normal number over
// this range) and two fp64 Newton steps y + y * (1 - s * y), each squaring the relative error
// and adding at most 2^-53: 2^-23 -> ~2^-46 -> ~2^-53.
// tests/native/gfx950_builtins.hip ("recip64") checks |1 - s * y| <= 2^-52 on the GPU for
// every fp32 s of the range.
__device__ __forceinline__ double recip64(float s) {
  const double s64 = (double)s;
  double y = (double)__builtin_amdgcn_rcpf(s);
  y = __builtin_fma(__builtin_fma(-s64, y, 1.0), y, y);
  return __builtin_fma(__builtin_fma(-s64, y, 1.0), y, y);
}

// int8 code of an fp32 quotient: clamp to [-128, 127] (v_med3_f32), then round to nearest
// even by adding 1.5*2^23 (the sum's ulp is 1, so the hardware RNE add performs the
// rounding, and the low byte of its bit pattern is the two's-complement code).  Returns the
// code in bits 0..7 of the result (upper bits are garbage).
__device__ __forceinline__ uint32_t rne_bits(float q) { return __float_as_uint(q + 12582912.0f); }
__device__ __forceinline__ uint32_t code_bits(float q) {
  return rne_bits(__builtin_amdgcn_fmed3f(q, -128.0f, 127.0f));
}

// Placed in the rarely-taken IEEE-divide branch.  The IR cost model counts an fdiv as one
// instruction, so without a side effect in the branch the optimiser speculates it and every
// lane computes both quotients (an IEEE divide is ~10 VALU ops) and selects -- which more
// than doubled the quantiser's VALU work in some instantiations.
__host__ __device__ __forceinline__ void keep_branch() { asm volatile(""); }

// Per-row quantisation state: the scale and, on the fast path, its reciprocal.
struct RowScale {
  float s;      // fp32(amax) / 127
  double y64;   // recip64(s) on the fast path (div_recip64); 0 for an all-zero row
  bool fast;    // kFastDivMinScale <= s < inf, or s == 0
};

// RN(amax / 127) without a divide: q0 = amax * RN(1/127) is within ~1 ulp, and one FMA
// correction with the constant reciprocal (Markstein) rounds it correctly.
// tests/native/div_exhaustive.hip checks it against IEEE division for every fp32 amax from
// 2^-100 to the largest finite value; below 2^-100 the correction's residual can be
// inexact, and the IEEE divide is used.
constexpr float kInv127 = 1.0f / 127.0f;
constexpr float kScaleDivMin = 7.88860905e-31f;  // 2^-100
__host__ __device__ __forceinline__ float scale_of(float amax) {
  const float q0 = amax * kInv127;
  const float r = __builtin_fmaf(-127.0f, q0, amax);
  return __builtin_fmaf(r, kInv127, q0);
}

__device__ __forceinline__ RowScale make_row_scale(float amax) {
  RowScale r;
  if (amax >= kScaleDivMin && amax < __builtin_inff()) {
    r.s = scale_of(amax);
  } else {
    keep_branch();
    r.s = amax / 127.0f;  // IEEE divide (hipcc default: correctly rounded fp32 division)
  }
  if (r.s >= kFastDivMinScale && r.s < __builtin_inff()) {
    r.fast = true;
    r.y64 = recip64(r.s);  // once per row
  } else if (r.s == 0.0f) {
    // All-zero row: with y64 = 0 every quotient is +-0, so all codes are 0 and the scale
    // stays 0 (the literal 0/0 of the reference math is not evaluated).
    r.fast = true;
    r.y64 = 0.0;
  } else {
    r.fast = false;
    r.y64 = 0.0;
  }
  return r;
}

// Pack the low bytes of four code_bits() results little-endian into one u32.
__device__ __forceinline__ uint32_t pack_codes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // [b0.0, b1.0, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);  // [0, 0, b2.0, b3.0]
  return lo | hi;
}

// Encode N (multiple of 4) fp32 values of one row into N int8 codes, packed 4 per u32.
// The fast/slow choice is made once per row so the element loop is straight-line code.
template <int N>
__device__ __forceinline__ void encode_row(const float* v, const RowScale& r, uint32_t* out) {
  float q[N];
  if (r.fast) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = div_recip64(v[i], r.y64);
  } else {
    keep_branch();
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = v[i] / r.s;  // IEEE divide (tiny or non-finite scale)
  }
  if (r.fast) {
    // |x| <= amax and s = RN(amax / 127) bound |q| by 127 * (1 + 2^-23), so the clamp of the
    // reference math cannot fire here and the round-half-even add alone gives the code.
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      out[i] = pack_codes(rne_bits(q[4 * i]), rne_bits(q[4 * i + 1]), rne_bits(q[4 * i + 2]),
                          rne_bits(q[4 * i + 3]));
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      out[i] = pack_codes(code_bits(q[4 * i]), code_bits(q[4 * i + 1]), code_bits(q[4 * i + 2]),
                          code_bits(q[4 * i + 3]));
  }
}

__device__ __forceinline__ int8_t encode1(float v, const RowScale& r) {
  float q;
  if (r.fast) {
    q = div_recip64(v, r.y64);
  } else {
    keep_branch();
    q = v / r.s;
  }
  return (int8_t)(uint8_t)(code_bits(q) & 0xffu);
}

// ---------------------------------------------------------------------------- static scales

// Static (offline) scales: code = clip(RNE(RN(x / s)), lo, hi) with a caller-given s per
// channel or per tensor.  The reciprocal quotient is used when kStaticMinScale <= |s| <=
// kStaticMaxScale (y = RN(1/s) is then a normal number and s * q cannot overflow) and every
// |x * y| of the lane is below kStaticQuotientLimit (beyond it the code saturates either
// way, and the correction steps could overflow); otherwise an IEEE divide per element.
// tests/native/div_exhaustive.hip ("static") checks the int8 and fp8 codes, and the quotient
// bits for |x| >= 2^-100 with a normal quotient, against IEEE division.
constexpr float kStaticMinScale = 8.6736174e-19f;   // 2^-60
constexpr float kStaticMaxScale = 1.2676506e30f;    // 2^100
constexpr float kStaticQuotientLimit = 4194304.0f;  // 2^22

__host__ __device__ __forceinline__ bool static_scale_fast(float s) {
  const float a = __builtin_fabsf(s);
  return a >= kStaticMinScale && a <= kStaticMaxScale;
}

// The IEEE quotient x / s carries the sign sign(x) ^ sign(s) also when it is zero; the FMA
// steps of div_by_recip return +0 for x = -0 and s > 0 (r0 = (-s)(-0) + (-0) = +0).  int8
// codes do not see the difference; float8_e4m3fn has a -0 code, so the fp8 paths put the sign
// back after div_by_recip (for a non-zero finite s and a non-zero quotient it is already right).
__host__ __device__ __forceinline__ uint32_t fbits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
__host__ __device__ __forceinline__ float bitsf(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
template <int N>
__host__ __device__ __forceinline__ void quotient_signs(float* q, const float* x, const float* s) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    q[i] = bitsf((fbits(q[i]) & 0x7fffffffu) | ((fbits(x[i]) ^ fbits(s[i])) & 0x80000000u));
}

// N quotients x[i] / s[i] (IEEE bits, see above; with kSignedZero also the sign of a zero
// quotient, for fp8 codes).  y[i] = RN(1 / s[i]) when `fast` (static_scale_fast for every
// s[i]), ignored otherwise.
template <int N, bool kSignedZero = false>
__host__ __device__ __forceinline__ void static_quotients(const float* x, const float* s,
                                                          const float* y, bool fast, float* q) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) m = fmaxf(m, __builtin_fabsf(x[i] * y[i]));
  if (fast && m < kStaticQuotientLimit) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = div_by_recip(x[i], s[i], y[i]);
    if constexpr (kSignedZero) quotient_signs<N>(q, x, s);
  } else {
    keep_branch();
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = x[i] / s[i];  // IEEE divide
  }
}

// RN(1 / s) for kStaticMinScale <= |s| <= kStaticMaxScale: v_rcp_f32 (within 1 ulp) and one
// FMA Newton step, y0 + y0 * (1 - s * y0).  tests/native/gfx950_builtins.hip ("rcp") checks it
// on the GPU against IEEE 1.0f / s for every fp32 s of the range (the steps are odd in s).
__device__ __forceinline__ float recip_rn(float s) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  return __builtin_fmaf(__builtin_fmaf(-s, y0, 1.0f), y0, y0);
}

// RN(sqrt(a)) for kSqrtMin <= a <= FLT_MAX in 8 VALU instructions (the IEEE square root
// adds input scaling for tiny a and special-value handling, 17 in all): v_sqrt_f32 (within
// 1 ulp), then s, its lower neighbour or its upper neighbour by the signs of the exact FMA
// residuals a - c * c+ of the adjacent pairs (c, c+) = (s-, s) and (s, s+).  With u = ulp(c),
// c = C u, the midpoint satisfies (c + u/2)^2 = c * c+ + u^2 / 4, and a, an fp32 number of
// about c^2, is a multiple of 2^23 u^2, so it never lies strictly between c * c+ and the
// squared midpoint: a > c * c+ exactly when sqrt(a) is above the midpoint, and a = c * c+
// (possible, e.g. C = 2^23) is below it.  The residuals are multiples of u^2 >= 2^-144 for
// a >= 2^-96, so their signs survive the FMA's rounding (fp32 denormals are kept).
// tests/native/div_exhaustive.hip ("sqrt") checks the choice on the CPU, given the correctly
// rounded root or either neighbour as s; tests/native/gfx950_builtins.hip ("sqrt") checks
// sqrt_rn on the GPU for every fp32 a of the range.
constexpr float kSqrtMin = 1.26217745e-29f;  // 2^-96
__host__ __device__ __forceinline__ float sqrt_choose(float a, float s) {
  const float dn = bitsf(fbits(s) - 1u);
  const float up = bitsf(fbits(s) + 1u);
  float r = __builtin_fmaf(-dn, s, a) <= 0.0f ? dn : s;
  r = __builtin_fmaf(-up, s, a) > 0.0f ? up : r;
  return r;
}
__device__ __forceinline__ float sqrt_rn(float a) {
  return sqrt_choose(a, __builtin_amdgcn_sqrtf(a));
}

// Four values already clamped to [-448, 448] -> four float8_e4m3fn bytes (little-endian in
// the result) with gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn, round to nearest even, two values
// per instruction).  tests/native/gfx950_builtins.hip ("fp8") checks it on the GPU against
// fp8e4m3_bits below for every fp32 value in [-448, 448].
__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// fp32 -> float8_e4m3fn bits (1-4-3, bias 7, no infinities, max 448), round to nearest
// even, for finite |f| <= 448 (callers clamp first, as the reference math clips to +-448
// before the cast).  Below 2^-6 the result is a subnormal multiple of 2^-9: RNE(|f| * 2^9)
// (exact scaling) is its bit pattern, and 8 lands on the smallest normal, 0x08.  Above, the
// fp32 pattern is rounded to 3 fraction bits (add half-ulp-minus-one plus the kept lsb) and
// the exponent rebased from 127 to 7.  Negative values (and -0) set bit 7.
__host__ __device__ __forceinline__ uint32_t fp8e4m3_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a < 0x3c800000u) {  // |f| < 2^-6
    float af;
    __builtin_memcpy(&af, &a, 4);
    code = (uint32_t)__builtin_rintf(af * 512.0f);
  } else {
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
  }
  return sign | code;
}

// Bytes of N quotients, packed 4 per u32: int8 codes (clamp, round half even) or
// float8_e4m3fn (clamp to +-448, round to nearest even; hardware conversion).
template <int N, bool kFp8>
__device__ __forceinline__ void encode_static(const float* q, uint32_t* out) {
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    if constexpr (kFp8) {
      float c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_fmed3f(q[4 * i + j], -448.0f, 448.0f);
      out[i] = fp8x4(c[0], c[1], c[2], c[3]);
    } else {
      out[i] = pack_codes(code_bits(q[4 * i]), code_bits(q[4 * i + 1]), code_bits(q[4 * i + 2]),
                          code_bits(q[4 * i + 3]));
    }
  }
}

// ---------------------------------------------------------------------------- fp8 dynamic scales

// float8_e4m3fn dynamic scale of a row / group: RN(amax / 448) (IEEE divide, once per row) and,
// when kFastDivMinScale <= s < inf, y64 = recip64(s) for the quotient div_recip64 (the IEEE
// quotient there, as for the int8 scale).  s == 0 (an all-zero row): every code is +0.
__device__ __forceinline__ RowScale make_fp8_scale(float amax) {
  RowScale r;
  r.s = amax / 448.0f;
  r.fast = r.s >= kFastDivMinScale && r.s < __builtin_inff();
  r.y64 = r.fast ? recip64(r.s) : 0.0;
  return r;
}

// N values (multiple of 4) -> N e4m3fn codes packed 4 per u32: e4m3fn_RNE(clip(RN(x / s), +-448)),
// all +0 when s == 0.
template <int N>
__device__ __forceinline__ void encode_fp8_row(const float* v, const RowScale& r, uint32_t* out) {
  float q[N];
  if (r.fast) {
    // div_recip64 keeps the sign of a zero quotient (x * y64 with y64 > 0), as IEEE x / s
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = div_recip64(v[i], r.y64);
  } else {
    keep_branch();
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = v[i] / r.s;  // IEEE divide
  }
  encode_static<N, true>(q, out);
  if (r.s == 0.0f) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) out[i] = 0u;
  }
}

// One value of the same encoding (generic paths).
__device__ __forceinline__ uint8_t encode1_fp8(float v, float s) {
  if (s == 0.0f) return 0;
  return (uint8_t)fp8e4m3_bits(__builtin_amdgcn_fmed3f(v / s, -448.0f, 448.0f));  // IEEE divide
}

// ---------------------------------------------------------------------------- cache readers

// float8_e4m3fn byte k (0..3) of a dword as fp32: gfx950's v_cvt_f32_fp8 decodes the OCP
// e4m3fn format exactly (every e4m3fn value is an fp32, f16 and bf16 value);
// tests/native/gfx950_builtins.hip ("fp8dec") checks all 256 codes in every byte position.
__device__ __forceinline__ float fp8_value(uint32_t w, int k) {
  switch (k) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8((int)w, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8((int)w, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8((int)w, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8((int)w, 3);
  }
}

// Byte k of a dword of cache codes as fp32: an int8 code, or a float8_e4m3fn value.
__device__ __forceinline__ float code_byte(uint32_t w, int k, bool fp8) {
  return fp8 ? fp8_value(w, k) : (float)(int8_t)(w >> (8 * k));
}

// Scale element i of an fp32 or bf16 scale tensor (bf16 widens to fp32 exactly).
__device__ __forceinline__ float scale_at(const void* s, int64_t i, int bf16) {
  return bf16 ? __uint_as_float((uint32_t) static_cast<const uint16_t*>(s)[i] << 16)
              : static_cast<const float*>(s)[i];
}

// Element e (0..7) of 8 consecutive scales held raw: fp32 in w[0], w[1] (4 each), or bf16 in
// w[0] (8).
template <bool kBf16>
__device__ __forceinline__ float scale_of8(const u32x4 (&w)[2], int e) {
  if constexpr (kBf16) {
    const uint32_t x = w[0][e / 2];
    return __uint_as_float((e & 1) ? (x & 0xffff0000u) : (x << 16));
  }
  return __uint_as_float(w[e / 4][e % 4]);
}

// ---------------------------------------------------------------------------- stores

// Non-temporal 4- and 8-byte vector stores of int8 codes.  __builtin_nontemporal_store carries
// the hint as IR metadata, and an IR pass drops it when it merges the two 32-bit halves of a
// code vector in some instantiations (the 16-lane, one-vector-per-lane quantiser lost it and
// ran ~30% slower on scattered page writes), so these emit the `nt` store form directly.
// They are plain vector-memory stores; the compiler's waitcnt bookkeeping only ever
// over-waits around them, and the kernels issue no loads after their stores.
__device__ __forceinline__ void store_nt(uint32_t* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off nt" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_nt(u32x2* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off nt" : : "v"(p), "v"(v) : "memory");
}

// ---------------------------------------------------------------------------- misc

// Launch `kernel(p)` and return TMO_OK or TMO_ERR_LAUNCH from the launch's own status
// (hipLaunchKernel reports it directly; no sticky-error peeking).
template <typename Params>
inline int launch_kernel(void (*kernel)(Params), dim3 grid, dim3 block, hipStream_t stream,
                         const Params& p, unsigned shared_bytes = 0) {
  Params copy = p;
  void* args[] = {&copy};
  const hipError_t e =
      hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, args, shared_bytes, stream);
  return e == hipSuccess ? TMO_OK : TMO_ERR_LAUNCH;
}

// Kernels of three parameters (the params struct and two pointers); the argument types are
// taken from the kernel (non-deduced), so pointers convert to the kernel's const-qualified ones.
template <class A, class B, class C>
inline int launch_kernel(void (*kernel)(A, B, C), dim3 grid, dim3 block, hipStream_t stream,
                         const typename std::common_type<A>::type& a,
                         typename std::common_type<B>::type b,
                         typename std::common_type<C>::type c) {
  A a_copy = a;
  void* args[] = {&a_copy, &b, &c};
  const hipError_t e =
      hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, args, 0, stream);
  return e == hipSuccess ? TMO_OK : TMO_ERR_LAUNCH;
}

__device__ __forceinline__ float abs_max(float m, float v) { return fmaxf(m, fabsf(v)); }

__host__ __device__ __forceinline__ int ilog2_if_pow2(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

}  // namespace tmo
