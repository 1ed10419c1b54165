// fused_rope (norm_type "rmsnorm") into paged caches, for gfx950: one pass over qkv that
// RMS-normalises Q (optional) and K per head, applies the fold rotary embedding to both, writes
// Q back into qkv and stores K and V into [num_blocks, kv_heads, block_size, head_size] pages
// through slot_mapping -- unquantised, or int8 with dynamic per-token or static per-channel
// scales.
//
// Semantics: reference _ops.py:3469-3601 (fused_rope, rmsnorm branch :3504-3509) and
// _ops.py:6356-6423 (fused_rmsnorm_rope_store_paged_cache); rotary math _ops.py:1116-1127
// (interleaved False).  Arithmetic is fp32 with one rounding at the end:
//   ss  = sum of x^2 over 8-element chunks in order, then a balanced tree over the chunk sums
//   inv = RN(1 / RN(sqrt(RN(RN(ss / D) + eps))));  y = RN(RN(x * inv) * gamma)
//   out = RN(RN(rot * sin) + RN(y * cos)),  rot = (-y[half:], y[:half]) over the rope window
// K is quantised (or rounded) from the fp32 result, V from its input values.  A position
// outside the sin/cos table leaves the row unrotated.
// Entry point: tmo_hip_fused_rope_paged (include/tmo_hip.h).
//
// Vector path: a (token, head) row of D elements is G = D / 8 lanes holding 16 bytes each, so
// a lane's 8 elements are exactly one chunk of the sum of squares; the chunk tree is the DPP
// row reduction (its pairings combine adjacent blocks in natural order, and fp32 addition is
// commutative, so every lane gets the tree's value).  The rotary partner of a lane is
// lane +- (rope_dim / 2) / 8 inside the group (ds_bpermute).  Rows are numbered token-major
// (t * (Hq + 2 Hk) + head), which is qkv's memory order, so a workgroup reads contiguous bytes.
#include <type_traits>

#include "tmo_device.h"

namespace tmo {
namespace {

struct FusedRopeParams {
  void* qkv;
  int64_t tokens;
  int64_t seq_len;
  int32_t hq, hk, heads, head_dim;
  const void* sin_t;
  const void* cos_t;
  int64_t table_rows;
  int64_t table_stride;  // elements
  int32_t rope_dim, rope_off;
  const int32_t* position;
  const void* k_gamma;
  const void* k_beta;   // nullable (layernorm only)
  const void* q_gamma;  // nullable (rmsnorm only)
  float eps;
  int32_t norm;         // 0 rmsnorm (before the rotation), 1 layernorm of K (after it)
  void* cache[2];
  float* scale[2];
  int32_t scale_mode;  // 0 none (caches of qkv's dtype), 1 dynamic per token, 2 static per channel
  const int32_t* slot;       // paged target: slot per token
  const int32_t* bs_id;      // linear target: cache batch per sequence (nullable: b)
  const int32_t* seq_off;    // linear target: first cache position per sequence (nullable: 0)
  int64_t max_batch;         // linear target: cache batches
  int32_t linear;            // 1: linear target, 0: paged
  int64_t num_slots;
  int32_t block_size;        // page rows, or the linear cache's length
  int32_t bs_shift;
};

// K (kv 0) or V (kv 1) cache and scale pointers by value.  kv differs between the lane groups
// of a wavefront, and indexing the kernel argument's array with it reads the pointer from
// argument memory with a vector load, whose wait (the memory counter is in order) also waited
// for the stores of the rows before it.
__device__ __forceinline__ void* cache_of(const FusedRopeParams& p, int kv) {
  return kv == 0 ? p.cache[0] : p.cache[1];
}
__device__ __forceinline__ float* scale_of_kv(const FusedRopeParams& p, int kv) {
  return kv == 0 ? p.scale[0] : p.scale[1];
}

// Slot of token t.  A linear cache [max_batch, kv_heads, cache_len, head_size] is the paged
// layout with one page of cache_len rows per cache batch, so token s of sequence b goes to
// slot cache_bs_id[b] * cache_len + cache_seq_offsets[b] + s, or nowhere (-1) when the cache
// batch or the position falls outside the cache.
__device__ __forceinline__ int32_t token_slot(const FusedRopeParams& p, int64_t t) {
  if (!p.linear) return p.slot[t];
  const int64_t b = t / p.seq_len;
  const int64_t cb = p.bs_id ? (int64_t)p.bs_id[b] : b;
  const int64_t pos = (p.seq_off ? (int64_t)p.seq_off[b] : 0) + (t - b * p.seq_len);
  if (cb < 0 || cb >= p.max_batch || pos < 0 || pos >= p.block_size) return -1;
  return (int32_t)(cb * p.block_size + pos);
}

__device__ __forceinline__ bool page_row_of(const FusedRopeParams& p, int32_t slot, int h,
                                            int64_t& page_row) {
  if (slot < 0 || (int64_t)slot >= p.num_slots) return false;
  int32_t blk, off;
  if (p.bs_shift >= 0) {
    blk = slot >> p.bs_shift;
    off = slot & (p.block_size - 1);
  } else {
    blk = slot / p.block_size;
    off = slot - blk * p.block_size;
  }
  page_row = ((int64_t)blk * p.hk + h) * p.block_size + off;
  return true;
}

// Sum over aligned groups of G lanes with the same pairings as group_max_u32: adjacent
// blocks of 1, 2, 4, 8 lanes (DPP inside a row), then 16 and 32 (lane shuffles).
template <int G>
__device__ __forceinline__ float group_sum_f32(float v) {
  auto dppf = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value,
                                                      0xF, 0xF, true));
  };
  if constexpr (G >= 2) v = v + dppf(v, std::integral_constant<int, kDppQuadSwap1>{});
  if constexpr (G >= 4) v = v + dppf(v, std::integral_constant<int, kDppQuadSwap2>{});
  if constexpr (G >= 8) v = v + dppf(v, std::integral_constant<int, kDppRowHalfMirror>{});
  if constexpr (G >= 16) v = v + dppf(v, std::integral_constant<int, kDppRowMirror>{});
  if constexpr (G >= 32) v = v + __shfl_xor(v, 16, 64);
  if constexpr (G >= 64) v = v + __shfl_xor(v, 32, 64);
  return v;
}

// RN(1 / RN(sqrt(RN(RN(ss / D) + eps)))): IEEE division and square root (hipcc's defaults are
// correctly rounded; tests/native/gfx950_builtins.hip "sqrt" checks the square root).
__device__ __forceinline__ float rms_inverse(float ss, int d, float eps) {
  const float mean = ss / (float)d;
  const float r = __builtin_sqrtf(mean + eps);
  return 1.0f / r;
}

// The same value for a power-of-two row length D fixed at compile time (the vector kernels'
// D = 8 * G), in ~25 fewer VALU instructions per row:
//  - ss / D is ss * 2^-log2(D): the quotient and the product are the same real number, and
//    both operations round it once, subnormal and non-finite results included;
//  - for a = mean + eps in [2^-96, FLT_MAX], sqrt is sqrt_rn(a) and 1 / r is recip_rn(r)
//    (RN(1 / r), v_rcp_f32 and one FMA Newton step), since r lies in [2^-48, 2^64], inside
//    recip_rn's range [2^-60, 2^100]; any other a (tiny, 0, inf, NaN) takes the IEEE square
//    root and divide.
template <int D>
__device__ __forceinline__ float rms_inverse_pow2(float ss, float eps) {
  static_assert(D > 0 && (D & (D - 1)) == 0, "D must be a power of two");
  const float mean = ss * (1.0f / (float)D);
  const float a = mean + eps;
  if (a >= kSqrtMin && a <= __FLT_MAX__) return recip_rn(sqrt_rn(a));
  keep_branch();
  return 1.0f / __builtin_sqrtf(a);
}

// Layernorm of a row held as G lanes x 8 values, D = 8 * G (reference _ops.py:3501-3504):
// mean = RN(s1 / D), s1 the chunked sum of the values; d = RN(y - mean); var = RN(s2 / D), s2
// the chunked sum of RN(d * d); inv = RN(1 / RN(sqrt(RN(var + eps))));
// y = RN(RN(d * inv) * gamma) [+ beta, rounded].  D is a power of two, so the divisions by D
// are exact products (rms_inverse_pow2).
template <int G>
__device__ __forceinline__ void layernorm8(float* y, const float* g, const float* b, bool has_beta,
                                           float eps) {
  constexpr int D = 8 * G;
  float s1 = y[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) s1 = s1 + y[e];
  const float mean = group_sum_f32<G>(s1) * (1.0f / (float)D);
  float dv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dv[e] = y[e] - mean;
  float s2 = dv[0] * dv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    const float sq = dv[e] * dv[e];
    s2 = s2 + sq;
  }
  const float inv = rms_inverse_pow2<D>(group_sum_f32<G>(s2), eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float n = dv[e] * inv;
    y[e] = n * g[e];
    if (has_beta) y[e] = y[e] + b[e];
  }
}

constexpr int kDppRowRor8 = 0x128;  // rotate right by 8 lanes inside each 16-lane row

#ifndef TMO_FUSED_ROPE_TOKEN_MAJOR
#define TMO_FUSED_ROPE_TOKEN_MAJOR 1
#endif

template <class Tag>
__device__ __forceinline__ void pack8(Tag, const float* f, u32x4& w) {
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack2(Tag{}, f[2 * i], f[2 * i + 1]);
}

// Vector path: head_dim = 8 * G (G a power of two <= 64), rope window on 8-element chunks.
// kNorm (0 rmsnorm, 1 layernorm) is p.norm as a template argument, so the rmsnorm instance
// carries no layernorm registers (p.norm is still what the generic kernel reads).
template <class Tag, int G, int kNorm>
__global__ __launch_bounds__(256) void fused_rope_vec(FusedRopeParams p) {
  constexpr int kRows = 256 / G;
  const int lane = threadIdx.x & (G - 1);
  const int64_t row = (int64_t)blockIdx.x * kRows + threadIdx.x / G;
  const int64_t nrows = p.tokens * p.heads;
  // a group past the last row still runs the shuffles below (with its own lanes only) and
  // returns before any store
  const bool live = row < nrows;
  const int64_t t = live ? row / p.heads : 0;
  const int hh = live ? (int)(row - t * p.heads) : 0;
  const int kind = hh < p.hq ? 0 : (hh < p.hq + p.hk ? 1 : 2);  // q, k, v
  char* xrow = static_cast<char*>(p.qkv) + (row * p.head_dim + lane * 8) * Tag::kBytes;

  // ---- loads: x, then (q/k) gamma and the sin/cos of this lane's window chunk, slot
  u32x4 xw = {0u, 0u, 0u, 0u}, gw = {0u, 0u, 0u, 0u}, sw = {0u, 0u, 0u, 0u}, cw = {0u, 0u, 0u, 0u};
  u32x4 bw = {0u, 0u, 0u, 0u};
  int32_t slot = -1;
  const int c0 = p.rope_off / 8, nwin = p.rope_dim / 8;  // window in chunks
  const bool in_win = lane >= c0 && lane < c0 + nwin;
  int64_t pos = -1;
  const void* gamma = kind == 0 ? p.q_gamma : p.k_gamma;
  if (live) {
    xw = *reinterpret_cast<const u32x4*>(xrow);
    if (kind != 0) slot = token_slot(p, t);
    if (kind != 2) {
      const int64_t b = t / p.seq_len;
      pos = (int64_t)p.position[b] + (t - b * p.seq_len);
      if (gamma) gw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(gamma) + lane * 16);
      if (kind == 1 && kNorm == 1 && p.k_beta)
        bw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.k_beta) + lane * 16);
      if (pos >= 0 && pos < p.table_rows && in_win) {
        const int64_t e = pos * p.table_stride + (lane - c0) * 8;
        sw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.sin_t) + e * Tag::kBytes);
        cw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.cos_t) + e * Tag::kBytes);
      }
    }
  }
  float x[8];
  unpack(Tag{}, xw, x);

  // ---- q / k: rmsnorm, rope
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = x[e];
  if (kind != 2 && kNorm == 0 && (kind == 1 || p.q_gamma)) {
    float acc = x[0] * x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) {
      const float sq = x[e] * x[e];
      acc = acc + sq;
    }
    const float inv = rms_inverse_pow2<8 * G>(group_sum_f32<G>(acc), p.eps);
    float g[8];
    unpack(Tag{}, gw, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float n = x[e] * inv;
      y[e] = n * g[e];
    }
  }
  const bool rotate = kind != 2 && pos >= 0 && pos < p.table_rows;  // group-uniform
  if (kind != 2) {
    // partner chunk: +half in the first half of the window, -half in the second
    const int hc = nwin / 2;
    float partner[8];
    if (G == 16 && nwin == 16) {
      // whole 16-lane row: the partner is lane +- 8 = lane ^ 8, a DPP row rotation by 8
#pragma unroll
      for (int e = 0; e < 8; ++e)
        partner[e] = __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(y[e]), kDppRowRor8, 0xF, 0xF, true));
    } else {
      const int base = (threadIdx.x & (kWave - 1)) & ~(G - 1);  // the group's first lane
      const int src = in_win ? (lane < c0 + hc ? lane + hc : lane - hc) : lane;
#pragma unroll
      for (int e = 0; e < 8; ++e) partner[e] = __shfl(y[e], base + src, 64);
    }
    if (rotate && in_win) {
      float sn[8], cs[8];
      unpack(Tag{}, sw, sn);
      unpack(Tag{}, cw, cs);
      // rot = -partner in the first half of the window: fold the sign into sin (exact)
      const float sign = lane < c0 + hc ? -1.0f : 1.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = partner[e] * (sn[e] * sign);
        const float b = y[e] * cs[e];
        y[e] = a + b;
      }
    }
    if (kind == 1 && kNorm == 1) {  // layernorm of K after its rotation
      float g[8], bt[8];
      unpack(Tag{}, gw, g);
      unpack(Tag{}, bw, bt);
      layernorm8<G>(y, g, bt, p.k_beta != nullptr, p.eps);
    }
  }
  if (!live) return;
  if (kind == 0) {
    u32x4 o;
    pack8(Tag{}, y, o);
    *reinterpret_cast<u32x4*>(xrow) = o;
    return;
  }

  // ---- k / v: store into the page
  const int h = kind == 1 ? hh - p.hq : hh - p.hq - p.hk;
  const int kv = kind - 1;
  int64_t page_row;
  if (!page_row_of(p, slot, h, page_row)) return;  // group-uniform
  if (p.scale_mode == 0) {
    u32x4 o;
    pack8(Tag{}, y, o);
    *reinterpret_cast<u32x4*>(static_cast<char*>(cache_of(p, kv)) +
                              (page_row * p.head_dim + lane * 8) * Tag::kBytes) = o;
    return;
  }
  uint32_t c[2];
  if (p.scale_mode == 1) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = abs_max(m, y[e]);
    const RowScale rs = make_row_scale(__uint_as_float(group_max_u32<G>(__float_as_uint(m))));
    encode_row<8>(y, rs, c);
    if (lane == 0) scale_of_kv(p, kv)[page_row] = rs.s;
  } else {
    const float* sp = scale_of_kv(p, kv) + (int64_t)h * p.head_dim + lane * 8;
    float s[8], yr[8], q[8];
    bool fast = true;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[e] = sp[e];
      fast &= static_scale_fast(s[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) yr[e] = fast ? recip_rn(s[e]) : 0.0f;
    static_quotients<8>(y, s, yr, fast, q);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      c[i] = pack_codes(code_bits(q[4 * i]), code_bits(q[4 * i + 1]), code_bits(q[4 * i + 2]),
                        code_bits(q[4 * i + 3]));
  }
  u32x2 c2;
  c2[0] = c[0];
  c2[1] = c[1];
  *reinterpret_cast<u32x2*>(static_cast<int8_t*>(cache_of(p, kv)) + page_row * p.head_dim + lane * 8) = c2;
}

// Token-major vector path: a workgroup of kThreads (256 or 512) owns one token (its position
// and slot are scalar loads, no per-lane index division) and the kThreads/G lane groups walk
// its heads, kR rows per group, all kR rows loaded before the first is processed.  sin/cos
// (with the rotation's sign folded in) are unpacked once per workgroup, both gammas loaded
// once.  Same arithmetic, in the same order, as fused_rope_vec.
template <class Tag, int G, int kR, int kNorm, int kThreads>
__global__ __launch_bounds__(kThreads) void fused_rope_tok(FusedRopeParams p) {
  constexpr int kGroups = kThreads / G;
  const int lane = threadIdx.x & (G - 1);
  const int grp = threadIdx.x / G;
  const int64_t t = blockIdx.x;
  const int64_t b = t / p.seq_len;  // workgroup-uniform (scalar)
  const int64_t pos = (int64_t)p.position[b] + (t - b * p.seq_len);
  const int32_t slot = token_slot(p, t);
  const int c0 = p.rope_off / 8, nwin = p.rope_dim / 8, hc = nwin / 2;
  const bool in_win = lane >= c0 && lane < c0 + nwin;
  const bool rotate = pos >= 0 && pos < p.table_rows;  // workgroup-uniform

  // rows of this group: heads grp, grp + kGroups, ... (kR of them at most)
  char* xbase = static_cast<char*>(p.qkv) + (t * p.heads * p.head_dim + lane * 8) * Tag::kBytes;
  // unconditional loads (a row past the last head re-reads the last head, in bounds, and is
  // not used): with the loads under a branch the compiler merged the array through register
  // copies that waited for each load before the next was issued
  u32x4 xw[kR];
#pragma unroll
  for (int j = 0; j < kR; ++j) {
    const int hh = min(grp + j * kGroups, p.heads - 1);
    xw[j] = *reinterpret_cast<const u32x4*>(xbase + (int64_t)hh * p.head_dim * Tag::kBytes);
  }
  u32x4 sw = {0u, 0u, 0u, 0u}, cw = {0u, 0u, 0u, 0u}, kgw = {0u, 0u, 0u, 0u}, qgw = {0u, 0u, 0u, 0u};
  if (rotate && in_win) {
    const int64_t e = pos * p.table_stride + (lane - c0) * 8;
    sw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.sin_t) + e * Tag::kBytes);
    cw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.cos_t) + e * Tag::kBytes);
  }
  kgw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.k_gamma) + lane * 16);
  if (p.q_gamma) qgw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.q_gamma) + lane * 16);
  u32x4 kbw = {0u, 0u, 0u, 0u};
  if (kNorm == 1 && p.k_beta)
    kbw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.k_beta) + lane * 16);
  // Every loaded register is used once here, before the first store: the stores count in the
  // same in-order memory counter as the loads, and a first use after a store (the rows after
  // the first, the gammas and sin/cos loaded under branches) made the compiler wait for that
  // store as well.
#pragma unroll
  for (int j = 0; j < kR; ++j) asm volatile("" ::"v"(xw[j]));
  asm volatile("" ::"v"(sw), "v"(cw), "v"(kgw), "v"(qgw), "v"(kbw));
  // sin (with the rotation's sign folded in: rot = -partner in the window's first half, and
  // the product with +-1 is exact) and cos, unpacked once for all rows of the group; the
  // gammas and beta stay packed until their use in each row (fewer live VGPRs)
  float sns[8], cs[8];
  {
    const float sign = lane < c0 + hc ? -1.0f : 1.0f;
    unpack(Tag{}, sw, sns);
    unpack(Tag{}, cw, cs);
#pragma unroll
    for (int e = 0; e < 8; ++e) sns[e] = sns[e] * sign;
  }
  const bool store_kv = slot >= 0 && (int64_t)slot < p.num_slots;  // workgroup-uniform

#pragma unroll
  for (int j = 0; j < kR; ++j) {
    const int hh = grp + j * kGroups;
    if (hh >= p.heads) break;  // group-uniform
    const int kind = hh < p.hq ? 0 : (hh < p.hq + p.hk ? 1 : 2);
    if (kind != 0 && !store_kv) continue;
    float y[8];
    unpack(Tag{}, xw[j], y);
    if (kind != 2) {
      if (kNorm == 0 && (kind == 1 || p.q_gamma)) {
        float acc = y[0] * y[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) {
          const float sq = y[e] * y[e];
          acc = acc + sq;
        }
        const float inv = rms_inverse_pow2<8 * G>(group_sum_f32<G>(acc), p.eps);
        float g[8];
        unpack(Tag{}, kind == 1 ? kgw : qgw, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float n = y[e] * inv;
          y[e] = n * g[e];
        }
      }
      float partner[8];
      if (G == 16 && nwin == 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          partner[e] = __int_as_float(
              __builtin_amdgcn_update_dpp(0, __float_as_int(y[e]), kDppRowRor8, 0xF, 0xF, true));
      } else {
        const int base = (threadIdx.x & (kWave - 1)) & ~(G - 1);
        const int src = in_win ? (lane < c0 + hc ? lane + hc : lane - hc) : lane;
#pragma unroll
        for (int e = 0; e < 8; ++e) partner[e] = __shfl(y[e], base + src, 64);
      }
      if (rotate && in_win) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float a = partner[e] * sns[e];
          const float c = y[e] * cs[e];
          y[e] = a + c;
        }
      }
      if (kind == 1 && kNorm == 1) {
        float kg[8], kb[8];
        unpack(Tag{}, kgw, kg);
        unpack(Tag{}, kbw, kb);
        layernorm8<G>(y, kg, kb, p.k_beta != nullptr, p.eps);
      }
    }
    if (kind == 0) {
      u32x4 o;
      pack8(Tag{}, y, o);
      *reinterpret_cast<u32x4*>(xbase + (int64_t)hh * p.head_dim * Tag::kBytes) = o;
      continue;
    }
    const int h = kind == 1 ? hh - p.hq : hh - p.hq - p.hk;
    const int kv = kind - 1;
    int64_t page_row;
    page_row_of(p, slot, h, page_row);
    if (p.scale_mode == 0) {
      u32x4 o;
      pack8(Tag{}, y, o);
      *reinterpret_cast<u32x4*>(static_cast<char*>(cache_of(p, kv)) +
                                (page_row * p.head_dim + lane * 8) * Tag::kBytes) = o;
      continue;
    }
    uint32_t c[2];
    if (p.scale_mode == 1) {
      float m = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) m = abs_max(m, y[e]);
      const RowScale rs = make_row_scale(__uint_as_float(group_max_u32<G>(__float_as_uint(m))));
      encode_row<8>(y, rs, c);
      if (lane == 0) scale_of_kv(p, kv)[page_row] = rs.s;
    } else {
      const float* sp = scale_of_kv(p, kv) + (int64_t)h * p.head_dim + lane * 8;
      float sc[8], yr[8], q[8];
      bool fast = true;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sc[e] = sp[e];
        fast &= static_scale_fast(sc[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) yr[e] = fast ? recip_rn(sc[e]) : 0.0f;
      static_quotients<8>(y, sc, yr, fast, q);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        c[i] = pack_codes(code_bits(q[4 * i]), code_bits(q[4 * i + 1]), code_bits(q[4 * i + 2]),
                          code_bits(q[4 * i + 3]));
    }
    u32x2 c2;
    c2[0] = c[0];
    c2[1] = c[1];
    *reinterpret_cast<u32x2*>(static_cast<int8_t*>(cache_of(p, kv)) + page_row * p.head_dim + lane * 8) = c2;
  }
}

// Generic path (any head_dim <= 512, any even rope window): one wavefront per row, the row
// staged in LDS as fp32 (all reads of the row finish before Q is written back in place).
template <class Tag>
__global__ __launch_bounds__(256) void fused_rope_generic(FusedRopeParams p) {
  __shared__ float stage[4][512];
  __shared__ float normed[4][512];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  // every wave reaches both barriers; a wave past the last row only skips the work
  const bool active = row < p.tokens * p.heads;
  const int64_t t = active ? row / p.heads : 0;
  const int hh = active ? (int)(row - t * p.heads) : 0;
  const int kind = hh < p.hq ? 0 : (hh < p.hq + p.hk ? 1 : 2);
  const int D = p.head_dim;
  float* xs = stage[wave];
  float* ys = normed[wave];
  const int64_t base = row * D;
  if (active)
    for (int d = lane; d < D; d += kWave) xs[d] = load1(Tag{}, p.qkv, base + d);
  __syncthreads();
  const void* gamma = kind == 0 ? p.q_gamma : p.k_gamma;
  const bool norm = p.norm == 0 && (kind == 1 || (kind == 0 && p.q_gamma));
  if (active) {
    float inv = 1.0f;
    if (kind != 2 && norm) {
      // chunk `lane` of the sum of squares, then the 64-lane tree (zeros past the last chunk)
      float acc = 0.0f;
      const int e0 = lane * 8;
      if (e0 < D) {
        acc = xs[e0] * xs[e0];
        for (int e = e0 + 1; e < e0 + 8 && e < D; ++e) {
          const float sq = xs[e] * xs[e];
          acc = acc + sq;
        }
      }
      inv = rms_inverse(group_sum_f32<kWave>(acc), D, p.eps);
    }
    for (int d = lane; d < D; d += kWave) {
      float v = xs[d];
      if (kind != 2 && norm) {
        const float n = v * inv;
        v = n * load1(Tag{}, gamma, d);
      }
      ys[d] = v;
    }
  }
  __syncthreads();
  if (!active) return;
  int64_t pos = -1;
  if (kind != 2) {
    const int64_t b = t / p.seq_len;
    pos = (int64_t)p.position[b] + (t - b * p.seq_len);
  }
  const bool rotate0 = kind != 2 && pos >= 0 && pos < p.table_rows;
  const int half = p.rope_dim / 2;
  bool rotate = rotate0;
  if (kind == 1 && p.norm == 1) {
    // layernorm of K after its rotation: rotate into xs (the row's stage, free after the copy
    // into ys), then normalise there; out_at then reads the finished values unrotated
    for (int d = lane; d < D; d += kWave) {
      float v = ys[d];
      if (rotate0 && d >= p.rope_off && d < p.rope_off + p.rope_dim) {
        const int j = d - p.rope_off;
        const float rot = j < half ? -ys[d + half] : ys[d - half];
        const float a = rot * load1(Tag{}, p.sin_t, pos * p.table_stride + j);
        const float b = v * load1(Tag{}, p.cos_t, pos * p.table_stride + j);
        v = a + b;
      }
      xs[d] = v;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // chunk `lane` of the sums, then the 64-lane tree (zeros past the last chunk)
    const int e0 = lane * 8;
    float s1 = 0.0f;
    if (e0 < D) {
      s1 = xs[e0];
      for (int e = e0 + 1; e < e0 + 8 && e < D; ++e) s1 = s1 + xs[e];
    }
    const float mean = group_sum_f32<kWave>(s1) / (float)D;
    float s2 = 0.0f;
    if (e0 < D) {
      const float d0 = xs[e0] - mean;
      s2 = d0 * d0;
      for (int e = e0 + 1; e < e0 + 8 && e < D; ++e) {
        const float de = xs[e] - mean;
        const float sq = de * de;
        s2 = s2 + sq;
      }
    }
    const float inv = rms_inverse(group_sum_f32<kWave>(s2), D, p.eps);
    for (int d = lane; d < D; d += kWave) {
      const float dv = xs[d] - mean;
      const float n = dv * inv;
      float v = n * load1(Tag{}, p.k_gamma, d);
      if (p.k_beta) v = v + load1(Tag{}, p.k_beta, d);
      ys[d] = v;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    rotate = false;
  }
  auto out_at = [&](int d) -> float {
    const float yv = ys[d];
    if (!rotate || d < p.rope_off || d >= p.rope_off + p.rope_dim) return yv;
    const int j = d - p.rope_off;
    const float rot = j < half ? -ys[d + half] : ys[d - half];
    const float sn = load1(Tag{}, p.sin_t, pos * p.table_stride + j);
    const float cs = load1(Tag{}, p.cos_t, pos * p.table_stride + j);
    const float a = rot * sn;
    const float b = yv * cs;
    return a + b;
  };
  if (kind == 0) {
    for (int d = lane; d < D; d += kWave) store1(Tag{}, p.qkv, base + d, out_at(d));
    return;
  }
  const int h = kind == 1 ? hh - p.hq : hh - p.hq - p.hk;
  const int kv = kind - 1;
  int64_t page_row;
  if (!page_row_of(p, token_slot(p, t), h, page_row)) return;
  if (p.scale_mode == 0) {
    for (int d = lane; d < D; d += kWave) store1(Tag{}, cache_of(p, kv), page_row * D + d, out_at(d));
    return;
  }
  int8_t* dst = static_cast<int8_t*>(cache_of(p, kv)) + page_row * D;
  if (p.scale_mode == 1) {
    float m = 0.0f;
    for (int d = lane; d < D; d += kWave) m = abs_max(m, out_at(d));
    const RowScale rs = make_row_scale(__uint_as_float(group_max_u32<kWave>(__float_as_uint(m))));
    for (int d = lane; d < D; d += kWave) dst[d] = encode1(out_at(d), rs);
    if (lane == 0) scale_of_kv(p, kv)[page_row] = rs.s;
  } else {
    for (int d = lane; d < D; d += kWave) {
      const float q = out_at(d) / scale_of_kv(p, kv)[(int64_t)h * D + d];  // IEEE divide
      dst[d] = (int8_t)(uint8_t)(code_bits(q) & 0xffu);
    }
  }
}

#ifndef TMO_FUSED_ROPE_MAX_ROWS
#define TMO_FUSED_ROPE_MAX_ROWS 8
#endif
constexpr int kFusedRopeMaxRows = TMO_FUSED_ROPE_MAX_ROWS;

// fused_rope_tok in kThreads-thread workgroups (one per token) with the smallest row count
// R >= r of its instances (R <= kMaxR)
template <class Tag, int G, int kNorm, int kThreads, int kMaxR, int R = 1>
int launch_tok(int r, hipStream_t stream, const FusedRopeParams& p) {
  if constexpr (R < kMaxR) {
    if (r > R) return launch_tok<Tag, G, kNorm, kThreads, kMaxR, R + 1>(r, stream, p);
  }
  return launch_kernel(fused_rope_tok<Tag, G, R, kNorm, kThreads>, dim3((unsigned)p.tokens),
                       dim3(kThreads), stream, p);
}

template <class Tag, int kNorm>
int launch(const FusedRopeParams& p, hipStream_t stream) {
  const int D = p.head_dim;
  const int G = D / 8;
  auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  bool vec = D % 8 == 0 && G >= 1 && G <= kWave && (G & (G - 1)) == 0 &&
             p.rope_off % 8 == 0 && p.rope_dim % 16 == 0 && al16(p.qkv) && al16(p.k_gamma) && (!p.k_beta || al16(p.k_beta)) &&
             (!p.q_gamma || al16(p.q_gamma)) && al16(p.sin_t) && al16(p.cos_t) &&
             (p.table_stride * Tag::kBytes) % 16 == 0 && al16(p.cache[0]) && al16(p.cache[1]) &&
             (p.scale_mode != 2 || (al16(p.scale[0]) && al16(p.scale[1])));
  // Token-major kernel, one workgroup per token: 256 threads while the token's heads take at
  // most 3 rows per lane group, else 512 threads (twice the lane groups, half the rows, fewer
  // VGPRs per thread) up to kFusedRopeMaxRows rows; more heads take the row-major kernel.
  if (TMO_FUSED_ROPE_TOKEN_MAJOR && vec && p.tokens <= 0x7fffffffLL) {
    const int64_t r = (p.heads + 256 / G - 1) / (256 / G);
    const int64_t r2 = (p.heads + 512 / G - 1) / (512 / G);
    if (r <= 3) {
      switch (G) {
        case 1: return launch_tok<Tag, 1, kNorm, 256, 3>((int)r, stream, p);
        case 2: return launch_tok<Tag, 2, kNorm, 256, 3>((int)r, stream, p);
        case 4: return launch_tok<Tag, 4, kNorm, 256, 3>((int)r, stream, p);
        case 8: return launch_tok<Tag, 8, kNorm, 256, 3>((int)r, stream, p);
        case 16: return launch_tok<Tag, 16, kNorm, 256, 3>((int)r, stream, p);
        case 32: return launch_tok<Tag, 32, kNorm, 256, 3>((int)r, stream, p);
        case 64: return launch_tok<Tag, 64, kNorm, 256, 3>((int)r, stream, p);
        default: break;
      }
    } else if (r2 <= kFusedRopeMaxRows) {
      switch (G) {
        case 1: return launch_tok<Tag, 1, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 2: return launch_tok<Tag, 2, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 4: return launch_tok<Tag, 4, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 8: return launch_tok<Tag, 8, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 16: return launch_tok<Tag, 16, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 32: return launch_tok<Tag, 32, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        case 64: return launch_tok<Tag, 64, kNorm, 512, kFusedRopeMaxRows, 2>((int)r2, stream, p);
        default: break;
      }
    }
  }
  const int64_t nrows = p.tokens * p.heads;
  const int rows = vec ? 256 / G : 4;
  const int64_t blocks = (nrows + rows - 1) / rows;
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)blocks), block(256);
  if (!vec) return launch_kernel(fused_rope_generic<Tag>, grid, block, stream, p);
  switch (G) {
    case 1: return launch_kernel(fused_rope_vec<Tag, 1, kNorm>, grid, block, stream, p);
    case 2: return launch_kernel(fused_rope_vec<Tag, 2, kNorm>, grid, block, stream, p);
    case 4: return launch_kernel(fused_rope_vec<Tag, 4, kNorm>, grid, block, stream, p);
    case 8: return launch_kernel(fused_rope_vec<Tag, 8, kNorm>, grid, block, stream, p);
    case 16: return launch_kernel(fused_rope_vec<Tag, 16, kNorm>, grid, block, stream, p);
    case 32: return launch_kernel(fused_rope_vec<Tag, 32, kNorm>, grid, block, stream, p);
    default: return launch_kernel(fused_rope_vec<Tag, 64, kNorm>, grid, block, stream, p);
  }
}

}  // namespace
}  // namespace tmo

namespace {

// Both targets: slot_mapping (paged) or, with `linear`, cache_bs_id / cache_seq_offsets over
// max_batch cache batches of block_size = cache_len rows.
int fused_rope_run(
    void* qkv, int64_t num_tokens, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
    int64_t head_size, const void* sin_table, const void* cos_table, int64_t table_rows,
    int64_t table_stride, int64_t rope_dim, int64_t rope_offset, const int32_t* position_ids,
    int64_t batch, const void* k_gamma, const void* k_beta, const void* q_gamma, float eps,
    int norm_type, void* k_cache, void* v_cache, float* k_scale, float* v_scale, int scale_mode,
    bool linear, const int32_t* slot_mapping, const int32_t* cache_bs_id,
    const int32_t* cache_seq_offsets, int64_t max_batch, int64_t num_blocks, int64_t block_size,
    int dtype, void* stream) {
  using namespace tmo;
  if (dtype != TMO_DTYPE_F16 && dtype != TMO_DTYPE_BF16) return TMO_ERR_UNSUPPORTED_DTYPE;
  if (scale_mode < 0 || scale_mode > 2 || norm_type < 0 || norm_type > 1)
    return TMO_ERR_UNSUPPORTED_MODE;
  // q_gamma is an rmsnorm-only argument: layernorm ignores it, as the reference does
  // (_ops.py:3469-3601 normalises Q only in the rmsnorm branch)
  if (norm_type == 1) q_gamma = nullptr;
  if (norm_type == 0 && k_beta) return TMO_ERR_INVALID_ARGUMENT;   // layernorm-only argument
  if (!qkv || !sin_table || !cos_table || !position_ids || !k_gamma || !k_cache || !v_cache ||
      (!linear && !slot_mapping))
    return TMO_ERR_INVALID_ARGUMENT;
  // linear target: every slot cache_batch * cache_len + position must fit an int32
  if (linear && block_size > 0 && num_blocks > 0x7fffffffLL / block_size)
    return TMO_ERR_INVALID_ARGUMENT;
  if (scale_mode != 0 && (!k_scale || !v_scale)) return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens < 0 || seq_len <= 0 || q_heads < 0 || kv_heads <= 0 || head_size <= 0 ||
      head_size > 512 || num_blocks < 0 || block_size <= 0 || batch < 0 || table_rows < 0 ||
      table_stride < rope_dim)
    return TMO_ERR_INVALID_ARGUMENT;
  if (rope_dim < 0 || rope_dim % 2 != 0 || rope_offset < 0 || rope_offset + rope_dim > head_size)
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens > batch * seq_len) return TMO_ERR_INVALID_ARGUMENT;  // position_ids[t / seq_len]
  if (q_heads + 2 * kv_heads > 0x7fffffffLL || block_size > 0x7fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0) return TMO_OK;

  FusedRopeParams p{};
  p.qkv = qkv;
  p.tokens = num_tokens;
  p.seq_len = seq_len;
  p.hq = (int32_t)q_heads;
  p.hk = (int32_t)kv_heads;
  p.heads = (int32_t)(q_heads + 2 * kv_heads);
  p.head_dim = (int32_t)head_size;
  p.sin_t = sin_table;
  p.cos_t = cos_table;
  p.table_rows = table_rows;
  p.table_stride = table_stride;
  p.rope_dim = (int32_t)rope_dim;
  p.rope_off = (int32_t)rope_offset;
  p.position = position_ids;
  p.k_gamma = k_gamma;
  p.k_beta = k_beta;
  p.q_gamma = q_gamma;
  p.eps = eps;
  p.norm = norm_type;
  p.cache[0] = k_cache;
  p.cache[1] = v_cache;
  p.scale[0] = k_scale;
  p.scale[1] = v_scale;
  p.scale_mode = scale_mode;
  p.slot = slot_mapping;
  p.bs_id = cache_bs_id;
  p.seq_off = cache_seq_offsets;
  p.max_batch = max_batch;
  p.linear = linear ? 1 : 0;
  p.num_slots = num_blocks * block_size;
  p.block_size = (int32_t)block_size;
  p.bs_shift = ilog2_if_pow2(block_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (norm_type == 1)
    return dtype == TMO_DTYPE_F16 ? launch<F16, 1>(p, s) : launch<BF16, 1>(p, s);
  return dtype == TMO_DTYPE_F16 ? launch<F16, 0>(p, s) : launch<BF16, 0>(p, s);
}

}  // namespace

extern "C" int tmo_hip_fused_rope_paged(
    void* qkv, int64_t num_tokens, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
    int64_t head_size, const void* sin_table, const void* cos_table, int64_t table_rows,
    int64_t table_stride, int64_t rope_dim, int64_t rope_offset, const int32_t* position_ids,
    int64_t batch, const void* k_gamma, const void* k_beta, const void* q_gamma, float eps,
    int norm_type, void* k_cache, void* v_cache, float* k_scale, float* v_scale, int scale_mode,
    const int32_t* slot_mapping, int64_t num_blocks, int64_t block_size, int dtype,
    void* stream) {
  return fused_rope_run(qkv, num_tokens, seq_len, q_heads, kv_heads, head_size, sin_table,
                        cos_table, table_rows, table_stride, rope_dim, rope_offset, position_ids,
                        batch, k_gamma, k_beta, q_gamma, eps, norm_type, k_cache, v_cache, k_scale,
                        v_scale, scale_mode, false, slot_mapping, nullptr, nullptr, 0,
                        num_blocks, block_size, dtype, stream);
}

extern "C" int tmo_hip_fused_rope_linear(
    void* qkv, int64_t num_tokens, int64_t seq_len, int64_t q_heads, int64_t kv_heads,
    int64_t head_size, const void* sin_table, const void* cos_table, int64_t table_rows,
    int64_t table_stride, int64_t rope_dim, int64_t rope_offset, const int32_t* position_ids,
    int64_t batch, const void* k_gamma, const void* k_beta, const void* q_gamma, float eps,
    int norm_type, void* k_cache, void* v_cache, float* k_scale, float* v_scale, int scale_mode,
    const int32_t* cache_bs_id, const int32_t* cache_seq_offsets, int64_t max_batch,
    int64_t cache_len, int dtype, void* stream) {
  return fused_rope_run(qkv, num_tokens, seq_len, q_heads, kv_heads, head_size, sin_table,
                        cos_table, table_rows, table_stride, rope_dim, rope_offset, position_ids,
                        batch, k_gamma, k_beta, q_gamma, eps, norm_type, k_cache, v_cache, k_scale,
                        v_scale, scale_mode, true, nullptr, cache_bs_id, cache_seq_offsets,
                        max_batch, max_batch, cache_len, dtype, stream);
}
