// quant_to_paged_cache for gfx950: dynamic per-(token, head) quantisation of K/V rows into
// int8 (scale = amax / 127) or float8_e4m3fn (scale = amax / 448) codes, scattered into
// [num_blocks, heads, block_size, head_dim] pages through slot_mapping.
//
// Semantics: reference _ops.py:1511-1565 (math block :1524-1537, slot convention :1262-1268).
// Entry point: tmo_hip_quant_to_paged_cache (include/tmo_hip.h).
//
// Also offline_quant_to_paged_cache (reference _ops.py:1639-1706): the same pages written
// with static per-channel or per-tensor scales into an int8 or float8_e4m3fn cache
// (tmo_hip_offline_quant_to_paged_cache), on the same token/head mapping.
//
// Mapping (vector path): a row of head_dim elements is G = head_dim / (16 B / elem) lanes,
// one 16-byte load per lane.  A 256-thread workgroup owns consecutive tokens of ONE head, so
// with consecutive slots (prefill) its code stores fill whole pages contiguously and its
// scale stores one contiguous run.  K and V of the same (token, head) are handled by the same
// lanes, and each lane group takes several tokens, so every lane has several independent
// 16-byte loads in flight.  The row amax
// is a DPP reduction inside the lane group; the divide is the fp64-product quotient of
// tmo_device.h (div_recip64, bit-identical to IEEE division); codes are written with
// non-temporal stores (the cache is written once per step and read by other kernels), the
// 4-byte scales with plain stores (neighbouring heads' scales share a line).
#include "tmo_device.h"

namespace tmo {
namespace {

struct QuantPagedParams {
  const void* src[2];
  int64_t stride_tok[2];   // elements
  int64_t stride_head[2];  // elements
  int8_t* cache[2];
  float* scale[2];
  const int32_t* slot;
  int64_t num_tokens;
  int64_t num_slots;  // num_blocks * block_size
  int32_t heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) or -1
  int32_t nkv;       // 1 (K only) or 2 (K and V)
};

// Page row of (slot, head); false for a skipped slot (negative, or past the last page).
__device__ __forceinline__ bool locate_slot(const QuantPagedParams& p, int32_t slot, int h,
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
  page_row = ((int64_t)blk * p.heads + h) * p.block_size + off;
  return true;
}

#ifndef TMO_QUANT_TOKENS_PER_THREAD
#define TMO_QUANT_TOKENS_PER_THREAD 1
#endif
#ifndef TMO_QUANT_XCD
#define TMO_QUANT_XCD 1
#endif
#ifndef TMO_QUANT_VEC_PER_LANE
#define TMO_QUANT_VEC_PER_LANE 1
#endif
constexpr int kTokensPerThread = TMO_QUANT_TOKENS_PER_THREAD;

// Vector path: head_dim == G * V * Tag::kPerVec, 16-byte aligned rows.  A row is G lanes,
// each holding V 16-byte vectors (lane l of the group owns vectors l, l + G, ...), so the
// per-row work -- the amax reduction, the scale and its reciprocal -- is shared by V * kPerVec
// elements per lane.  A workgroup (256 threads, or 64 for decode-sized launches, see launch())
// owns kTokensPerThread * blockDim.x / G consecutive tokens of one head.
// Every load of the lane group (slots, K rows, V rows) is issued before the first wait: the
// input address does not depend on the slot, only the store address does.
template <class Tag, int G, int V, bool kFp8>
__global__ __launch_bounds__(256) void quant_paged_vec(QuantPagedParams p) {
  const int kGroups = blockDim.x / G;  // lane groups per workgroup
  constexpr int kPer = Tag::kPerVec;
  constexpr int kT = kTokensPerThread;
  const int lane = threadIdx.x & (G - 1);
#if TMO_QUANT_XCD
  // XCD-aware order: the tile's per-token scale lines (64 bytes of each of two heads in one
  // 128-byte line for block size 16) are written whole from one L2
  int h;
  int64_t tile;
  xcd_tile_head(blockIdx.x, p.heads, h, tile);
#else
  // blockIdx.x = token_tile * heads + head (workgroup-uniform, scalar ALU)
  const int h = blockIdx.x % p.heads;
  const int64_t tile = blockIdx.x / p.heads;
#endif
  const int64_t t0 = tile * (kGroups * kT) + threadIdx.x / G;

  int32_t slot[kT];
  u32x4 w[kT][2][V];
#pragma unroll
  for (int j = 0; j < kT; ++j) {
    const int64_t t = t0 + j * kGroups;
    slot[j] = -1;
    if (t < p.num_tokens) {
      slot[j] = p.slot[t];
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv < p.nkv) {
          const char* src = static_cast<const char*>(p.src[kv]) +
                            (t * p.stride_tok[kv] + (int64_t)h * p.stride_head[kv]) * Tag::kBytes;
#pragma unroll
          for (int i = 0; i < V; ++i)
            w[j][kv][i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(src + (lane + i * G) * 16));
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kT; ++j) {
    int64_t page_row;
    if (!locate_slot(p, slot[j], h, page_row)) continue;  // uniform per lane group
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv < p.nkv) {
        float v[V][kPer];
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          unpack(Tag{}, w[j][kv][i], v[i]);
#pragma unroll
          for (int e = 0; e < kPer; ++e) m = abs_max(m, v[i][e]);
        }
        const float amax = __uint_as_float(group_max_u32<G>(__float_as_uint(m)));
        const RowScale rs = kFp8 ? make_fp8_scale(amax) : make_row_scale(amax);
        int8_t* row = p.cache[kv] + page_row * p.head_dim;
#pragma unroll
        for (int i = 0; i < V; ++i) {
          int8_t* dst = row + (lane + i * G) * kPer;
          uint32_t c[kPer / 4];
          if constexpr (kFp8) {
            encode_fp8_row<kPer>(v[i], rs, c);
          } else {
            encode_row<kPer>(v[i], rs, c);
          }
          if constexpr (kPer == 8) {
            u32x2 c2;
            c2[0] = c[0];
            c2[1] = c[1];
            store_nt(reinterpret_cast<u32x2*>(dst), c2);
          } else {
            store_nt(reinterpret_cast<uint32_t*>(dst), c[0]);
          }
        }
        // A plain store: the 4-byte scales of neighbouring heads share a line, which the L2 of
        // the tile's XCD merges (configs[0]: 2.96 -> 2.69 us per call, larger calls unchanged)
        if (lane == 0) p.scale[kv][page_row] = rs.s;
      }
    }
  }
}

// Generic path (any head_dim / alignment): one wavefront per row, scalar loads, two passes.
template <class Tag, bool kFp8>
__global__ __launch_bounds__(256) void quant_paged_generic(QuantPagedParams p) {
  constexpr int kRows = 256 / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int h = blockIdx.x % p.heads;
  const int64_t tile = blockIdx.x / p.heads;
  const int64_t t = tile * kRows + threadIdx.x / kWave;
  if (t >= p.num_tokens) return;
  int64_t page_row;
  if (!locate_slot(p, p.slot[t], h, page_row)) return;
  for (int kv = 0; kv < p.nkv; ++kv) {
    const void* src = p.src[kv];
    const int64_t base = t * p.stride_tok[kv] + (int64_t)h * p.stride_head[kv];
    float m = 0.0f;
    for (int d = lane; d < p.head_dim; d += kWave) m = abs_max(m, load1(Tag{}, src, base + d));
    const float amax = __uint_as_float(group_max_u32<kWave>(__float_as_uint(m)));
    int8_t* dst = p.cache[kv] + page_row * p.head_dim;
    float s;
    if constexpr (kFp8) {
      s = amax / 448.0f;  // IEEE divide
      for (int d = lane; d < p.head_dim; d += kWave)
        dst[d] = (int8_t)encode1_fp8(load1(Tag{}, src, base + d), s);
    } else {
      const RowScale rs = make_row_scale(amax);
      s = rs.s;
      for (int d = lane; d < p.head_dim; d += kWave) dst[d] = encode1(load1(Tag{}, src, base + d), rs);
    }
    if (lane == 0) p.scale[kv][page_row] = s;
  }
}

// ---------------------------------------------------------------------------- static scales

struct StaticScales {
  const float* chan[2];  // [heads, head_dim] fp32 per-channel scales, or null: per tensor
  float tensor[2];
};
// Read in place of an absent per-channel scale table (at most 64 lanes of at most 8 floats).
__device__ __align__(16) const float kNoScales[512] = {};

struct StaticParams {
  QuantPagedParams q;
  StaticScales sc;
};

// 2 tokens per thread measured fastest on configs[2]'s shape (per channel, int8: 36.5 us vs
// 38.0 with 4 and 40.2 with 1)
#ifndef TMO_STATIC_TOKENS_PER_THREAD
#define TMO_STATIC_TOKENS_PER_THREAD 2
#endif

// Vector path of the static quantiser: one 16-byte vector per lane, G lanes per row (as the
// dynamic kernel with V = 1), a workgroup owns kT * 256/G consecutive tokens of one head.  A
// lane always covers the same kPerVec channels of its head, so it loads their scales once
// and computes the reciprocals once for its kT tokens.  There is no row reduction and no
// scale store.
template <class Tag, int G, bool kFp8>
__global__ __launch_bounds__(256) void quant_paged_static_vec(StaticParams sp) {
  const QuantPagedParams& p = sp.q;
  const StaticScales& sc = sp.sc;
  constexpr int kGroups = 256 / G;
  constexpr int kPer = Tag::kPerVec;
  constexpr int kT = TMO_STATIC_TOKENS_PER_THREAD;
  const int lane = threadIdx.x & (G - 1);
#if TMO_QUANT_XCD
  int h;
  int64_t tile;
  xcd_tile_head(blockIdx.x, p.heads, h, tile);
#else
  const int h = blockIdx.x % p.heads;
  const int64_t tile = blockIdx.x / p.heads;
#endif
  const int64_t t0 = tile * (kGroups * kT) + threadIdx.x / G;

  // Tokens past the end load the last token's row again (an L2 hit) and are skipped below:
  // every load is unconditional, so the waits before the first row count exactly.
  int32_t slot[kT];
  u32x4 w[kT][2];
#pragma unroll
  for (int j = 0; j < kT; ++j) {
    const int64_t t = t0 + j * kGroups;
    const int64_t tc = t < p.num_tokens ? t : p.num_tokens - 1;
    slot[j] = p.slot[tc];
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv < p.nkv) {
        const char* src = static_cast<const char*>(p.src[kv]) +
                          (tc * p.stride_tok[kv] + (int64_t)h * p.stride_head[kv]) * Tag::kBytes;
        w[j][kv] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + lane * 16));
      }
    }
    if (t >= p.num_tokens) slot[j] = -1;
  }
  float s[2][kPer];
  {
    // Both tables' loads go out with the rows, before the first wait: an absent table (a
    // per-tensor scale, or no V) reads kNoScales instead, and the values are chosen
    // afterwards.  Loaded under a per-channel / per-tensor branch, each table was waited for
    // where the branch merged, K's before V's loads were issued (37.2 -> 36.6 us on configs[2]'s
    // shape per channel).
    u32x4 raw[2][kPer / 4];
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      typedef const __attribute__((address_space(1))) float* gptr;
      const gptr base = sc.chan[kv] ? (gptr)(sc.chan[kv] + (int64_t)h * p.head_dim + lane * kPer)
                                    : (gptr)(kNoScales + lane * kPer);
#pragma unroll
      for (int q = 0; q < kPer / 4; ++q)
        raw[kv][q] = reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(base)[q];
    }
#pragma unroll
    for (int kv = 0; kv < 2; ++kv)
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        s[kv][e] = sc.chan[kv] ? __uint_as_float(raw[kv][e / 4][e % 4]) : sc.tensor[kv];
  }
  float y[2][kPer];
  bool fast[2];
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    if (kv < p.nkv) {
      fast[kv] = true;
#pragma unroll
      for (int e = 0; e < kPer; ++e) fast[kv] &= static_scale_fast(s[kv][e]);  // no short circuit
      if (!fast[kv]) {
#pragma unroll
        for (int e = 0; e < kPer; ++e) y[kv][e] = 0.0f;
      } else if (sc.chan[kv]) {
#pragma unroll
        for (int e = 0; e < kPer; ++e) y[kv][e] = recip_rn(s[kv][e]);
      } else {
        const float y0 = recip_rn(s[kv][0]);
#pragma unroll
        for (int e = 0; e < kPer; ++e) y[kv][e] = y0;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kT; ++j) {
    int64_t page_row;
    if (!locate_slot(p, slot[j], h, page_row)) continue;  // uniform per lane group
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv < p.nkv) {
        float v[kPer], q[kPer];
        unpack(Tag{}, w[j][kv], v);
        static_quotients<kPer, kFp8>(v, s[kv], y[kv], fast[kv], q);
        uint32_t c[kPer / 4];
        encode_static<kPer, kFp8>(q, c);
        int8_t* dst = p.cache[kv] + page_row * p.head_dim + lane * kPer;
        if constexpr (kPer == 8) {
          u32x2 c2;
          c2[0] = c[0];
          c2[1] = c[1];
          store_nt(reinterpret_cast<u32x2*>(dst), c2);
        } else {
          store_nt(reinterpret_cast<uint32_t*>(dst), c[0]);
        }
      }
    }
  }
}

// Generic static path (any head_dim / alignment): one wavefront per row, IEEE divides.
template <class Tag, bool kFp8>
__global__ __launch_bounds__(256) void quant_paged_static_generic(StaticParams sp) {
  const QuantPagedParams& p = sp.q;
  const StaticScales& sc = sp.sc;
  constexpr int kRows = 256 / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int h = blockIdx.x % p.heads;
  const int64_t tile = blockIdx.x / p.heads;
  const int64_t t = tile * kRows + threadIdx.x / kWave;
  if (t >= p.num_tokens) return;
  int64_t page_row;
  if (!locate_slot(p, p.slot[t], h, page_row)) return;
  for (int kv = 0; kv < p.nkv; ++kv) {
    const int64_t base = t * p.stride_tok[kv] + (int64_t)h * p.stride_head[kv];
    int8_t* dst = p.cache[kv] + page_row * p.head_dim;
    for (int d = lane; d < p.head_dim; d += kWave) {
      // the per-tensor scale is read as a value: choosing between its kernel-argument address
      // and a global address would make the load a flat load of a selected pointer
      float s = kv == 0 ? sc.tensor[0] : sc.tensor[1];
      if (sc.chan[kv]) s = sc.chan[kv][(int64_t)h * p.head_dim + d];
      const float q = load1(Tag{}, p.src[kv], base + d) / s;  // IEEE divide
      const uint32_t b =
          kFp8 ? fp8e4m3_bits(__builtin_amdgcn_fmed3f(q, -448.0f, 448.0f)) : code_bits(q);
      dst[d] = (int8_t)(uint8_t)(b & 0xffu);
    }
  }
}

template <class Tag, bool kFp8>
int launch_static(const StaticParams& sp, hipStream_t stream) {
  const QuantPagedParams& p = sp.q;
  const StaticScales& sc = sp.sc;
  constexpr int kPer = Tag::kPerVec;
  const int nvec = p.head_dim % kPer == 0 ? p.head_dim / kPer : 0;
  bool vec = nvec >= 1 && nvec <= kWave && (nvec & (nvec - 1)) == 0;
  for (int kv = 0; kv < p.nkv && vec; ++kv) {
    vec = (reinterpret_cast<uintptr_t>(p.src[kv]) % 16 == 0) &&
          ((p.stride_tok[kv] * Tag::kBytes) % 16 == 0) &&
          ((p.stride_head[kv] * Tag::kBytes) % 16 == 0) &&
          (reinterpret_cast<uintptr_t>(p.cache[kv]) % 8 == 0) &&
          (reinterpret_cast<uintptr_t>(sc.chan[kv]) % 16 == 0);  // null passes
  }
  const int G = vec ? nvec : kWave;
  const int rows = vec ? (256 / G) * TMO_STATIC_TOKENS_PER_THREAD : 256 / kWave;
  const int64_t tiles = (p.num_tokens + rows - 1) / rows;
  const int64_t blocks = tiles * p.heads;
  const int64_t vec_blocks = TMO_QUANT_XCD ? xcd_grid_tiles(tiles) * p.heads : blocks;
  if (vec_blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 block(256);
  if (!vec)
    return launch_kernel(quant_paged_static_generic<Tag, kFp8>, dim3((unsigned)blocks), block,
                         stream, sp);
  const dim3 grid((unsigned)vec_blocks);
  switch (G) {
    case 1: return launch_kernel(quant_paged_static_vec<Tag, 1, kFp8>, grid, block, stream, sp);
    case 2: return launch_kernel(quant_paged_static_vec<Tag, 2, kFp8>, grid, block, stream, sp);
    case 4: return launch_kernel(quant_paged_static_vec<Tag, 4, kFp8>, grid, block, stream, sp);
    case 8: return launch_kernel(quant_paged_static_vec<Tag, 8, kFp8>, grid, block, stream, sp);
    case 16: return launch_kernel(quant_paged_static_vec<Tag, 16, kFp8>, grid, block, stream, sp);
    case 32: return launch_kernel(quant_paged_static_vec<Tag, 32, kFp8>, grid, block, stream, sp);
    default: return launch_kernel(quant_paged_static_vec<Tag, 64, kFp8>, grid, block, stream, sp);
  }
}

template <class Tag, int V, bool kFp8>
int launch_vec(const QuantPagedParams& p, int G, dim3 grid, dim3 block, hipStream_t stream) {
  switch (G) {
    case 1: return launch_kernel(quant_paged_vec<Tag, 1, V, kFp8>, grid, block, stream, p);
    case 2: return launch_kernel(quant_paged_vec<Tag, 2, V, kFp8>, grid, block, stream, p);
    case 4: return launch_kernel(quant_paged_vec<Tag, 4, V, kFp8>, grid, block, stream, p);
    case 8: return launch_kernel(quant_paged_vec<Tag, 8, V, kFp8>, grid, block, stream, p);
    case 16: return launch_kernel(quant_paged_vec<Tag, 16, V, kFp8>, grid, block, stream, p);
    case 32: return launch_kernel(quant_paged_vec<Tag, 32, V, kFp8>, grid, block, stream, p);
    default: return launch_kernel(quant_paged_vec<Tag, 64, V, kFp8>, grid, block, stream, p);
  }
}

template <class Tag, bool kFp8>
int launch(const QuantPagedParams& p, hipStream_t stream) {
  constexpr int kPer = Tag::kPerVec;
  bool vec = (p.head_dim % kPer) == 0;
  const int nvec = vec ? p.head_dim / kPer : 0;  // 16-byte vectors per row
  vec = vec && nvec >= 1 && nvec <= 64 * TMO_QUANT_VEC_PER_LANE && (nvec & (nvec - 1)) == 0;
  for (int kv = 0; kv < p.nkv && vec; ++kv) {
    vec = (reinterpret_cast<uintptr_t>(p.src[kv]) % 16 == 0) &&
          ((p.stride_tok[kv] * Tag::kBytes) % 16 == 0) &&
          ((p.stride_head[kv] * Tag::kBytes) % 16 == 0) &&
          (reinterpret_cast<uintptr_t>(p.cache[kv]) % 8 == 0);
  }
  // V vectors per lane when the row has at least 4 * V of them, else one
  const int V = (vec && nvec >= 4 * TMO_QUANT_VEC_PER_LANE) ? TMO_QUANT_VEC_PER_LANE : 1;
  const int G = vec ? nvec / V : kWave;
  // Decode-sized launches (fewer than two 256-thread workgroups per CU of a 256-CU part) use
  // 64-thread workgroups: four times as many workgroups spread the row loads and the
  // scattered page stores over more CUs.  configs[1] (256 tokens x 8 heads, 128 -> 512
  // workgroups) 3.58 -> 3.43 us per call, configs[0] 3.15 -> 2.88 us on MI355X; prefill-sized
  // launches lose with small workgroups (configs[2]: 35.6 -> 38.9 us), so they keep 256.
  int wg = 256;
  if (vec && G <= 64) {
    const int64_t tiles256 = (p.num_tokens + (256 / G) * kTokensPerThread - 1) /
                             ((256 / G) * kTokensPerThread);
    if (tiles256 * p.heads < 512) wg = 64;
  }
  const int rows = vec ? (wg / G) * kTokensPerThread : 256 / kWave;
  const int64_t tiles = (p.num_tokens + rows - 1) / rows;
  const int64_t blocks = tiles * p.heads;
  // the vector kernel's XCD-aware order takes whole groups of 8 tiles (extra tiles have no
  // tokens and write nothing)
  const int64_t vec_blocks = TMO_QUANT_XCD ? xcd_grid_tiles(tiles) * p.heads : blocks;
  if (vec_blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 block(256);
  if (!vec) return launch_kernel(quant_paged_generic<Tag, kFp8>, dim3((unsigned)blocks), block, stream, p);
  const dim3 grid((unsigned)vec_blocks), vblock(wg);
  if (V == 1) return launch_vec<Tag, 1, kFp8>(p, G, grid, vblock, stream);
  return launch_vec<Tag, TMO_QUANT_VEC_PER_LANE, kFp8>(p, G, grid, vblock, stream);
}

}  // namespace
}  // namespace tmo

extern "C" int tmo_hip_quant_to_paged_cache(const void* k, const void* v,
                                            int64_t k_stride_token, int64_t k_stride_head,
                                            int64_t v_stride_token, int64_t v_stride_head,
                                            void* k_cache, void* v_cache,
                                            float* k_cache_scale, float* v_cache_scale,
                                            const int32_t* slot_mapping, int64_t num_tokens,
                                            int64_t num_heads, int64_t head_size,
                                            int64_t num_blocks, int64_t block_size, int dtype,
                                            int cache_dtype, void* stream) {
  using namespace tmo;
  if (dtype != TMO_DTYPE_F32 && dtype != TMO_DTYPE_F16 && dtype != TMO_DTYPE_BF16)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (cache_dtype != TMO_DTYPE_I8 && cache_dtype != TMO_DTYPE_F8E4M3)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (!k || !k_cache || !k_cache_scale || !slot_mapping) return TMO_ERR_INVALID_ARGUMENT;
  const bool has_v = v != nullptr;
  if (has_v != (v_cache != nullptr) || has_v != (v_cache_scale != nullptr))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || num_blocks < 0 || block_size <= 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (k_stride_token < 0 || k_stride_head < 0 || (has_v && (v_stride_token < 0 || v_stride_head < 0)))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_heads > 0x7fffffffLL || head_size > 0x7fffffffLL || block_size > 0x7fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0 || num_blocks == 0) return TMO_OK;

  QuantPagedParams p{};
  p.src[0] = k;
  p.src[1] = v;
  p.stride_tok[0] = k_stride_token;
  p.stride_tok[1] = v_stride_token;
  p.stride_head[0] = k_stride_head;
  p.stride_head[1] = v_stride_head;
  p.cache[0] = static_cast<int8_t*>(k_cache);
  p.cache[1] = static_cast<int8_t*>(v_cache);
  p.scale[0] = k_cache_scale;
  p.scale[1] = v_cache_scale;
  p.slot = slot_mapping;
  p.num_tokens = num_tokens;
  p.num_slots = num_blocks * block_size;
  p.heads = (int32_t)num_heads;
  p.head_dim = (int32_t)head_size;
  p.block_size = (int32_t)block_size;
  p.bs_shift = ilog2_if_pow2(block_size);
  p.nkv = has_v ? 2 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool fp8 = cache_dtype == TMO_DTYPE_F8E4M3;
  switch (dtype) {
    case TMO_DTYPE_F32: return fp8 ? launch<F32, true>(p, s) : launch<F32, false>(p, s);
    case TMO_DTYPE_F16: return fp8 ? launch<F16, true>(p, s) : launch<F16, false>(p, s);
    default: return fp8 ? launch<BF16, true>(p, s) : launch<BF16, false>(p, s);
  }
}

extern "C" int tmo_hip_offline_quant_to_paged_cache(
    const void* k, const void* v, int64_t k_stride_token, int64_t k_stride_head,
    int64_t v_stride_token, int64_t v_stride_head, void* k_cache, void* v_cache,
    const float* k_scale_channel, const float* v_scale_channel, float k_scale_tensor,
    float v_scale_tensor, const int32_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
    int64_t head_size, int64_t num_blocks, int64_t block_size, int dtype, int cache_dtype,
    void* stream) {
  using namespace tmo;
  if (dtype != TMO_DTYPE_F32 && dtype != TMO_DTYPE_F16 && dtype != TMO_DTYPE_BF16)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (cache_dtype != TMO_DTYPE_I8 && cache_dtype != TMO_DTYPE_F8E4M3)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (!k || !k_cache || !slot_mapping) return TMO_ERR_INVALID_ARGUMENT;
  const bool has_v = v != nullptr;
  if (has_v != (v_cache != nullptr) || (!has_v && v_scale_channel))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || num_blocks < 0 || block_size <= 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (k_stride_token < 0 || k_stride_head < 0 || (has_v && (v_stride_token < 0 || v_stride_head < 0)))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_heads > 0x7fffffffLL || head_size > 0x7fffffffLL || block_size > 0x7fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0 || num_blocks == 0) return TMO_OK;

  QuantPagedParams p{};
  p.src[0] = k;
  p.src[1] = v;
  p.stride_tok[0] = k_stride_token;
  p.stride_tok[1] = v_stride_token;
  p.stride_head[0] = k_stride_head;
  p.stride_head[1] = v_stride_head;
  p.cache[0] = static_cast<int8_t*>(k_cache);
  p.cache[1] = static_cast<int8_t*>(v_cache);
  p.slot = slot_mapping;
  p.num_tokens = num_tokens;
  p.num_slots = num_blocks * block_size;
  p.heads = (int32_t)num_heads;
  p.head_dim = (int32_t)head_size;
  p.block_size = (int32_t)block_size;
  p.bs_shift = ilog2_if_pow2(block_size);
  p.nkv = has_v ? 2 : 1;
  StaticParams sp{};
  sp.q = p;
  sp.sc.chan[0] = k_scale_channel;
  sp.sc.chan[1] = v_scale_channel;
  sp.sc.tensor[0] = k_scale_tensor;
  sp.sc.tensor[1] = v_scale_tensor;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool fp8 = cache_dtype == TMO_DTYPE_F8E4M3;
  switch (dtype) {
    case TMO_DTYPE_F32: return fp8 ? launch_static<F32, true>(sp, s) : launch_static<F32, false>(sp, s);
    case TMO_DTYPE_F16: return fp8 ? launch_static<F16, true>(sp, s) : launch_static<F16, false>(sp, s);
    default: return fp8 ? launch_static<BF16, true>(sp, s) : launch_static<BF16, false>(sp, s);
  }
}
