// reshape_paged_cache for gfx950: byte-exact scatter of K/V rows into
// [num_blocks, heads, block_size, head_dim] pages through slot_mapping (direction == 0), or
// the gather of the same rows back (direction != 0).
//
// Semantics: reference _ops.py:1251-1294 (math block :1262-1268).
// Entry point: tmo_hip_reshape_paged_cache (include/tmo_hip.h).
//
// A row is head_dim * elem_size bytes, moved in the widest vector (16/8/4/2/1 bytes) that
// the row length, base pointers and strides allow.  G lanes (the largest power of two <= the
// number of vectors in a row, capped at 64) share a row; a 256-thread workgroup owns 256/G
// consecutive tokens of one head, so consecutive slots produce contiguous page writes.
#include "tmo_device.h"

namespace tmo {
namespace {

struct ReshapeParams {
  char* kv[2];             // [T, H, D] rows
  int64_t stride_tok[2];   // bytes
  int64_t stride_head[2];  // bytes
  char* cache[2];          // [NB, H, BS, D]
  const int32_t* slot;
  int64_t num_tokens;
  int64_t num_slots;
  int64_t row_bytes;
  int32_t heads;
  int32_t block_size;
  int32_t bs_shift;
  int32_t units;       // vectors per row
  int32_t g_shift;     // log2(lanes per row)
  int32_t nkv;
  int32_t gather;      // direction != 0
};

template <int VW>
struct VecOf;
template <>
struct VecOf<16> { using T = u32x4; };
template <>
struct VecOf<8> { using T = u32x2; };
template <>
struct VecOf<4> { using T = uint32_t; };
template <>
struct VecOf<2> { using T = uint16_t; };
template <>
struct VecOf<1> { using T = uint8_t; };

template <int VW>
__global__ __launch_bounds__(256) void reshape_paged_kernel(ReshapeParams p) {
  using V = typename VecOf<VW>::T;
  const int G = 1 << p.g_shift;
  const int lane = threadIdx.x & (G - 1);
  const int rows = 256 >> p.g_shift;
  int h;
  int64_t tile;
  xcd_tile_head(blockIdx.x, p.heads, h, tile);  // the grid holds whole groups of 8 tiles
  const int64_t t = tile * rows + (threadIdx.x >> p.g_shift);
  if (t >= p.num_tokens) return;
  const int32_t slot = p.slot[t];
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  int32_t blk, off;
  if (p.bs_shift >= 0) {
    blk = slot >> p.bs_shift;
    off = slot & (p.block_size - 1);
  } else {
    blk = slot / p.block_size;
    off = slot - blk * p.block_size;
  }
  const int64_t page_off = (((int64_t)blk * p.heads + h) * p.block_size + off) * p.row_bytes;
  for (int kv = 0; kv < p.nkv; ++kv) {
    char* tok = p.kv[kv] + t * p.stride_tok[kv] + (int64_t)h * p.stride_head[kv];
    char* page = p.cache[kv] + page_off;
    const V* src = reinterpret_cast<const V*>(p.gather ? page : tok);
    V* dst = reinterpret_cast<V*>(p.gather ? tok : page);
    for (int u = lane; u < p.units; u += G) __builtin_nontemporal_store(src[u], dst + u);
  }
}

// Rows of exactly G vectors (one per lane), K and V: every load of a lane is issued before the
// first wait.  Scatter: the token rows do not depend on the slot, so the slot and both rows
// are read together (a V row that is absent re-reads K's).  Gather: the slot first, then both
// page rows.  In the general kernel above the rows are moved one after the other, each load
// waited for before its store, and the memory counter is in order: a thread paid the slot's,
// K's and V's round trips in turn, V's behind K's store.
template <int VW>
__global__ __launch_bounds__(256) void reshape_paged_rows(ReshapeParams p) {
  using V = typename VecOf<VW>::T;
  const int G = 1 << p.g_shift;
  const int lane = threadIdx.x & (G - 1);
  const int rows = 256 >> p.g_shift;
  int h;
  int64_t tile;
  xcd_tile_head(blockIdx.x, p.heads, h, tile);
  const int64_t t = tile * rows + (threadIdx.x >> p.g_shift);
  if (t >= p.num_tokens) return;
  const int kv1 = p.nkv > 1 ? 1 : 0;
  char* tk = p.kv[0] + t * p.stride_tok[0] + (int64_t)h * p.stride_head[0];
  char* tv = p.kv[kv1] + t * p.stride_tok[kv1] + (int64_t)h * p.stride_head[kv1];
  const int32_t slot = p.slot[t];
  V a, b;
  if (!p.gather) {
    a = __builtin_nontemporal_load(reinterpret_cast<const V*>(tk) + lane);
    b = __builtin_nontemporal_load(reinterpret_cast<const V*>(tv) + lane);
  }
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  int32_t blk, off;
  if (p.bs_shift >= 0) {
    blk = slot >> p.bs_shift;
    off = slot & (p.block_size - 1);
  } else {
    blk = slot / p.block_size;
    off = slot - blk * p.block_size;
  }
  const int64_t page_off = (((int64_t)blk * p.heads + h) * p.block_size + off) * p.row_bytes;
  char* pk = p.cache[0] + page_off;
  char* pv = p.cache[kv1] + page_off;
  if (p.gather) {
    a = __builtin_nontemporal_load(reinterpret_cast<const V*>(pk) + lane);
    b = __builtin_nontemporal_load(reinterpret_cast<const V*>(pv) + lane);
    __builtin_nontemporal_store(a, reinterpret_cast<V*>(tk) + lane);
    if (p.nkv > 1) __builtin_nontemporal_store(b, reinterpret_cast<V*>(tv) + lane);
  } else {
    __builtin_nontemporal_store(a, reinterpret_cast<V*>(pk) + lane);
    if (p.nkv > 1) __builtin_nontemporal_store(b, reinterpret_cast<V*>(pv) + lane);
  }
}

template <int VW>
int launch(const ReshapeParams& p0, hipStream_t stream) {
  ReshapeParams p = p0;
  p.units = (int32_t)(p.row_bytes / VW);
  int g = 1;
  while (g * 2 <= p.units && g < 64) g *= 2;
  p.g_shift = ilog2_if_pow2(g);
  const int rows = 256 / g;
  const int64_t blocks = xcd_grid_tiles((p.num_tokens + rows - 1) / rows) * p.heads;
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  if (p.units == g)
    return launch_kernel(reshape_paged_rows<VW>, dim3((unsigned)blocks), dim3(256), stream, p);
  return launch_kernel(reshape_paged_kernel<VW>, dim3((unsigned)blocks), dim3(256), stream, p);
}

bool aligned(const ReshapeParams& p, int vw) {
  if (p.row_bytes % vw) return false;
  for (int kv = 0; kv < p.nkv; ++kv) {
    if (reinterpret_cast<uintptr_t>(p.kv[kv]) % vw || reinterpret_cast<uintptr_t>(p.cache[kv]) % vw)
      return false;
    if (p.stride_tok[kv] % vw || p.stride_head[kv] % vw) return false;
  }
  return true;
}

}  // namespace
}  // namespace tmo

extern "C" int tmo_hip_reshape_paged_cache(void* k, void* v, int64_t k_stride_token,
                                           int64_t k_stride_head, int64_t v_stride_token,
                                           int64_t v_stride_head, void* k_cache, void* v_cache,
                                           const int32_t* slot_mapping, int64_t num_tokens,
                                           int64_t num_heads, int64_t head_size,
                                           int64_t num_blocks, int64_t block_size, int dtype,
                                           int direction, void* stream) {
  using namespace tmo;
  int es;
  switch (dtype) {
    case TMO_DTYPE_F32: es = 4; break;
    case TMO_DTYPE_F16:
    case TMO_DTYPE_BF16: es = 2; break;
    case TMO_DTYPE_I8: es = 1; break;
    default: return TMO_ERR_UNSUPPORTED_DTYPE;
  }
  if (!k || !k_cache || !slot_mapping) return TMO_ERR_INVALID_ARGUMENT;
  const bool has_v = v != nullptr;
  if (has_v != (v_cache != nullptr)) return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens < 0 || num_heads <= 0 || head_size <= 0 || num_blocks < 0 || block_size <= 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (k_stride_token < 0 || k_stride_head < 0 || (has_v && (v_stride_token < 0 || v_stride_head < 0)))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_heads > 0x7fffffffLL || block_size > 0x7fffffffLL || head_size > 0x3fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0 || num_blocks == 0) return TMO_OK;

  ReshapeParams p{};
  p.kv[0] = static_cast<char*>(k);
  p.kv[1] = static_cast<char*>(v);
  p.stride_tok[0] = k_stride_token * es;
  p.stride_tok[1] = v_stride_token * es;
  p.stride_head[0] = k_stride_head * es;
  p.stride_head[1] = v_stride_head * es;
  p.cache[0] = static_cast<char*>(k_cache);
  p.cache[1] = static_cast<char*>(v_cache);
  p.slot = slot_mapping;
  p.num_tokens = num_tokens;
  p.num_slots = num_blocks * block_size;
  p.row_bytes = head_size * es;
  p.heads = (int32_t)num_heads;
  p.block_size = (int32_t)block_size;
  p.bs_shift = ilog2_if_pow2(block_size);
  p.nkv = has_v ? 2 : 1;
  p.gather = direction != 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (aligned(p, 16)) return launch<16>(p, s);
  if (aligned(p, 8)) return launch<8>(p, s);
  if (aligned(p, 4)) return launch<4>(p, s);
  if (aligned(p, 2)) return launch<2>(p, s);
  return launch<1>(p, s);
}
