// The linear-cache siblings of the paged path, for gfx950.  A linear cache is
// [max_batch, heads, cache_len, head_dim]: one cache batch per sequence, tokens at
// consecutive positions.  Five reference ops share one addressing model:
//
//   reshape_linear_cache            token rows -> cache, byte copy     _ops.py:1189-1249
//   quant_to_linear_cache           dynamic int8 / fp8 per token/group _ops.py:1708-1806
//   offline_quant_to_linear_cache   static int8 / fp8                  _ops.py:1808-1919
//   dequant_from_linear_cache       int8 cache -> token rows           _ops.py:3642-3732
//   reshape_from_cache              cache -> token rows, byte copy     _ops.py:3898-3969
//
// Sequence i covers len_i = min(context_lengths[i], max_context_len) tokens (with packed
// input context_lengths holds batch + 1 prefix offsets and len_i = cu[i + 1] - cu[i]).  Its
// token j is row start_i + j of the token-major tensor [rows, heads, head_dim]: start_i =
// context_seq_offset[i] if given, else cu[i] (packed input), i * seqlen (padded input) or
// the exclusive prefix sum of the lengths (the outputs of the two read ops).  Its cache
// position is pos = cache_seq_offset[i] + j (else j), in cache batch cache_bs_id[i] (else i;
// negative: the sequence is skipped).  reshape_from_cache's block table [batch, max_blocks]
// generalises this to pages of block_rows positions: position pos lives in row
// pos % block_rows of page block_tables[i, pos / block_rows]; a one-column table is the
// linear layout with the table naming the cache batch.  Tokens whose row, cache batch / page
// or position falls outside its tensor are skipped.
//
// Per-token scales are [max_batch, heads, cache_len] (x groups for group-wise dynamic
// quantisation), static scales per channel [heads, head_dim], per head [heads, cache_len]
// (indexed by cache position) or one number.  The arithmetic is the paged kernels'
// (tmo_device.h): int8 dynamic = RN(amax / 127) + IEEE quotients, fp8 dynamic = RN(amax / 448)
// + IEEE quotients clamped to +-448 and rounded to e4m3fn, static = IEEE quotients,
// dequant = RN(fp32(code) * scale).
//
// Grid: y = sequence, x = (token tile, head) with the head fastest, so the workgroups of one
// token tile read neighbouring parts of the same token rows, and a workgroup's cache rows are
// consecutive.  Copies move 16 bytes per lane (G = row bytes / 16 lanes per row); the
// quantising kernels take 8 elements per lane (G = head_dim / 8).
#include "tmo_device.h"

namespace tmo {
namespace {

struct LinParams {
  void* tok[2];          // token-major tensors: input of the write ops, output of the reads
  void* cache[2];
  int64_t st[2], sh[2];  // token / head strides of the token tensors (elements)
  int64_t rows;          // rows of the token tensors
  int32_t heads, head_dim;
  int32_t nkv;
  int32_t in_dir;        // 1: token rows -> cache
  int64_t blocks;        // cache batches (linear) or pages (block table)
  int64_t block_rows;    // cache_len (linear) or rows per page
  const int32_t* lens;
  int32_t packed;
  int64_t pad_seqlen;
  const int32_t* seq_off;
  const int32_t* bs_id;
  const int32_t* cache_off;
  const int32_t* block_tables;
  int64_t max_blocks;
  int64_t max_len;
  float* scale[2];        // per-token scales: written by the dynamic quantiser, read by dequant
  const float* chan[2];   // static / dequant per-channel [H, D] or static per-head [H, cache_len]
  float tscale[2];        // static per-tensor scales
  int32_t smode;          // 0 channel, 1 head (static) or token (dequant), 2 tensor
  int32_t groups;         // dynamic scale groups per row
  int32_t op;             // generic kernel: 0 copy, 1 dynamic quant, 2 static quant, 3 dequant
  int32_t es;             // copies: bytes per element
  int64_t batch;          // sequences (token-major launches)
};

// Workgroup-uniform addressing of one sequence.
struct Seq {
  int64_t len, start, pos0;
};

// Exclusive prefix sum of the (int32) lengths before sequence i, computed by each wavefront on
// its own (no LDS, no barrier): lane l adds lens[l], lens[l + 64], ... split into a signed high
// and an unsigned low 16-bit half, so that both lane sums and both wavefront totals stay exact
// in 32 bits for any batch the grid allows (<= 65535 sequences); DPP row sums and four lane
// reads combine them.
__device__ __forceinline__ int32_t row_sum_i32(int32_t v) {
  v += (int32_t)dpp<kDppQuadSwap1>((uint32_t)v);
  v += (int32_t)dpp<kDppQuadSwap2>((uint32_t)v);
  v += (int32_t)dpp<kDppRowHalfMirror>((uint32_t)v);
  v += (int32_t)dpp<kDppRowMirror>((uint32_t)v);
  return v;  // every lane: the sum over its 16-lane row
}

__device__ int64_t length_prefix(const LinParams& p, int64_t i) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t lo = 0;
  int32_t hi = 0;
  for (int64_t k0 = 0; k0 < i; k0 += kWave) {
    const int64_t k = k0 + lane;
    const int32_t v = k < i ? p.lens[k] : 0;
    lo += (uint32_t)v & 0xffffu;
    hi += v >> 16;
  }
  const uint32_t lo_r = (uint32_t)row_sum_i32((int32_t)lo);
  const int32_t hi_r = row_sum_i32(hi);
  uint64_t lo_t = 0;
  int64_t hi_t = 0;
#pragma unroll
  for (int r = 0; r < kWave; r += 16) {
    lo_t += (uint32_t)__builtin_amdgcn_readlane((int)lo_r, r);
    hi_t += __builtin_amdgcn_readlane(hi_r, r);
  }
  return hi_t * 65536 + (int64_t)lo_t;
}

// Called by whole wavefronts (the prefix sum reads across lanes).  The four
// per-sequence numbers are loaded from valid addresses whether or not their tensor is given
// (an absent one reads lens[i] and is discarded), so the loads issue together and the
// workgroup waits for memory once before its rows' addresses are known.
__device__ Seq sequence(const LinParams& p, int64_t i, bool defer_prefix = false) {
  Seq s;
  const int32_t* so = p.seq_off ? p.seq_off + i : p.lens + i;
  const int32_t* co = p.cache_off ? p.cache_off + i : p.lens + i;
  const int32_t l0 = p.lens[i];
  const int32_t l1 = p.lens[i + p.packed];
  const int32_t so_v = *so;
  const int32_t co_v = *co;
  const int64_t len = p.packed ? (int64_t)l1 - l0 : (int64_t)l0;
  s.len = len < p.max_len ? len : p.max_len;
  if (p.seq_off) {
    s.start = so_v;
  } else if (p.in_dir) {
    s.start = p.packed ? (int64_t)l0 : i * p.pad_seqlen;
  } else {
    s.start = defer_prefix ? 0 : length_prefix(p, i);
  }
  s.pos0 = p.cache_off ? (int64_t)co_v : 0;
  return s;
}

// Read ops: the cache rows (load addresses) do not depend on where the sequence's output rows
// start, so the kernels issue their loads first and take the prefix sum (when no
// context_seq_offset is given) while the loads are in flight.
__device__ __forceinline__ void finish_start(const LinParams& p, int64_t i, Seq& s) {
  if (!p.seq_off && !p.in_dir) s.start = length_prefix(p, i);
}

// Cache row of the token at cache position `pos` for head h, or -1 when it is skipped.
__device__ __forceinline__ int64_t cache_row(const LinParams& p, int64_t i, int64_t pos, int h) {
  if (pos < 0) return -1;
  int64_t blk, r;
  if (p.block_tables) {
    const int64_t col = pos / p.block_rows;
    if (col >= p.max_blocks) return -1;
    blk = p.block_tables[i * p.max_blocks + col];
    r = pos - col * p.block_rows;
  } else {
    if (pos >= p.block_rows) return -1;
    blk = p.bs_id ? (int64_t)p.bs_id[i] : i;
    r = pos;
  }
  if (blk < 0 || blk >= p.blocks) return -1;
  return (blk * p.heads + h) * p.block_rows + r;
}

// Tokens per thread of the vector kernels: every load of a thread's tokens is issued before
// the first is used, so a workgroup keeps kT rows per lane group in flight and the
// per-workgroup prologue (sequence lengths / offsets) is paid once per kT tokens.
#ifndef TMO_LIN_TOKENS_PER_THREAD
#define TMO_LIN_TOKENS_PER_THREAD 1
#endif
constexpr int kLinT = TMO_LIN_TOKENS_PER_THREAD;

// Input rows are read once: non-temporal loads keep them from displacing the written rows.
#ifndef TMO_LIN_NT_LOAD
#define TMO_LIN_NT_LOAD 1
#endif
template <class T>
__device__ __forceinline__ T stream_load(const T* q) {
  if constexpr (TMO_LIN_NT_LOAD) return __builtin_nontemporal_load(q);
  return *q;
}

// Codes are written once and not read back by the kernel: non-temporal stores.
#ifndef TMO_LIN_NT_STORE
#define TMO_LIN_NT_STORE 1
#endif

// Token j (< len) of thread slot t, its row and its cache row; false when skipped.
__device__ __forceinline__ bool locate(const LinParams& p, const Seq& s, int64_t i, int h,
                                       int64_t j, int64_t& r, int64_t& crow) {
  if (j >= s.len) return false;
  r = s.start + j;
  crow = cache_row(p, i, s.pos0 + j, h);
  return r >= 0 && r < p.rows && crow >= 0;
}

// Token-major write launches (packed input, no context_seq_offset, at most 63 sequences): the
// grid walks the token rows themselves, so a row's load address needs no per-sequence number;
// the sequence is found while the row loads are in flight.  The per-sequence numbers are read
// into lanes first (lane l holds cu[l], cache_seq_offset[l] and cache_bs_id[l]) with
// unconditional loads, then the row loads are issued, also unconditionally: the code between
// them is straight-line, so the only wait in front of the lookup is for the first three loads
// (the memory counter is in order and the compiler counts the row loads issued after them).
// With a branch among these loads the compiler waited for every load there, and the lookup ran
// after the row data had arrived (quant_to_linear_cache, 8 x 4096 tokens: 2.4 us of the
// kernel's 41 us).
struct TmSeqs {
  int32_t cu, off, id;
};
__device__ __forceinline__ TmSeqs tm_prefetch(const LinParams& p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int k = lane <= p.batch ? lane : 0;   // cu has batch + 1 entries
  const int ks = lane < p.batch ? lane : 0;   // the per-sequence arrays have batch
  // an absent array reads cu instead (the value is discarded in tm_locate); the pointers are
  // device pointers, read through the global address space (a selected generic pointer would
  // compile to a flat load, which the compiler waits for together with every other load)
  typedef const __attribute__((address_space(1))) int32_t* gptr;
  const gptr offp = (gptr)(p.cache_off ? p.cache_off : p.lens);
  const gptr idp = (gptr)(p.bs_id ? p.bs_id : p.lens);
  TmSeqs t;
  t.cu = ((gptr)p.lens)[k];
  t.off = offp[ks];
  t.id = idp[ks];
  return t;
}

// Row r (the wavefront's rows are rbase + q, q = lane / G, rbase wave-uniform) -> its cache row
// for head h and its cache position; false when r is no stored token.  The sequence is the
// number of prefix offsets cu[1..batch] at or below r (the offsets are non-decreasing), and r
// must lie in [cu[i], cu[i] + min(cu[i + 1] - cu[i], max_len)): one ballot per row and lane
// shuffles.  With kUniform, when the wavefront's first and last rows count the same offsets
// (all its rows in one sequence, the usual case; the lanes counted only grow with the row, so
// then every row counts the same ones) two ballots give the wave-uniform sequence and
// readlane its numbers: quant_to_linear_cache, 8 x 4096 tokens, 40.9 -> 40.2 us and 39.3 ->
// 39.1 us on two boxes; the bf16 reshape measured slower with it (46.1 -> 47.7 us) and keeps
// the per-row form.  Every lane
// of the wavefront must call it (it holds ballots and lane shuffles).
template <int G, bool kUniform>
__device__ __forceinline__ bool tm_locate(const LinParams& p, const TmSeqs& t, int64_t rbase,
                                          int h, int64_t& crow, int64_t& pos) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = rbase + lane / G;
  const bool seq_lane = lane >= 1 && lane <= p.batch;
  uint64_t first = 0, last = 1;
  if constexpr (kUniform) {
    first = __ballot(seq_lane && (int64_t)t.cu <= rbase);
    last = __ballot(seq_lane && (int64_t)t.cu <= rbase + kWave / G - 1);
  }
  int cnt;
  int64_t c0, c1;
  int32_t off_i, id_i;
  if (kUniform && first == last) {  // wave-uniform
    cnt = __popcll(first);
    c0 = __builtin_amdgcn_readlane(t.cu, cnt);
    c1 = __builtin_amdgcn_readlane(t.cu, cnt + 1 < kWave ? cnt + 1 : cnt);
    off_i = __builtin_amdgcn_readlane(t.off, cnt);
    id_i = __builtin_amdgcn_readlane(t.id, cnt);
  } else {
    cnt = 0;
#pragma unroll
    for (int q = 0; q < kWave / G; ++q) {
      const uint64_t hit = __ballot(seq_lane && (int64_t)t.cu <= rbase + q);
      if (q == lane / G) cnt = __popcll(hit);
    }
    c0 = __shfl(t.cu, cnt, kWave);
    c1 = __shfl(t.cu, cnt + 1 < kWave ? cnt + 1 : cnt, kWave);
    off_i = __shfl(t.off, cnt, kWave);
    id_i = __shfl(t.id, cnt, kWave);
  }
  const int64_t i = cnt;
  if (i >= p.batch) return false;
  const int64_t off = p.cache_off ? (int64_t)off_i : 0;
  const int64_t id = p.bs_id ? (int64_t)id_i : i;
  const int64_t j = r - c0;
  int64_t len = c1 - c0;
  if (len > p.max_len) len = p.max_len;
  if (j < 0 || j >= len) return false;
  pos = off + j;
  if (pos < 0 || pos >= p.block_rows || id < 0 || id >= p.blocks) return false;
  crow = (id * p.heads + h) * p.block_rows + pos;
  return true;
}

// (token tile, head) of this workgroup: head fastest along x (sequence-major launches), or the
// XCD-aware order of the token-major launches (xcd_tile_head: the heads of one token tile run
// on one XCD, so one L2 sees whole token rows; the bf16 reshape of 8 x 4096 tokens measured
// 52.0 -> 49.8 us with it, the quantiser unchanged).
template <bool kXcd>
__device__ __forceinline__ void lin_tile_head(const LinParams& p, int& h, int64_t& tile) {
  if constexpr (kXcd) {
    xcd_tile_head(blockIdx.x, p.heads, h, tile);
  } else {
    h = blockIdx.x % p.heads;
    tile = blockIdx.x / p.heads;
  }
}

// ------------------------------------------------------------------------------ byte copies

// reshape_linear_cache / reshape_from_cache: G lanes x 16 bytes per row, kLinT rows per lane
// group.
template <int G, bool kTM>
__global__ __launch_bounds__(256) void lin_copy(LinParams p) {
  constexpr int kRows = 256 / G;
  const int64_t es = p.es, row_bytes = (int64_t)p.head_dim * p.es;
  const int lane = threadIdx.x & (G - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<kTM>(p, h, tile);
  const int64_t j0 = tile * (kRows * kLinT) + threadIdx.x / G;
  bool ok[kLinT];
  int64_t r[kLinT], crow[kLinT];
  u32x4 v[kLinT][2];
  if constexpr (kTM) {  // token rows -> cache, the grid over the token rows
    const TmSeqs seqs = tm_prefetch(p);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      r[t] = j0 + t * kRows;
      ok[t] = r[t] < p.rows;
      if (!ok[t]) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        const char* tk = static_cast<const char*>(p.tok[kv]) +
                         (r[t] * p.st[kv] + (int64_t)h * p.sh[kv]) * es;
        v[t][kv] = stream_load(reinterpret_cast<const u32x4*>(tk + lane * 16));
      }
    }
    const int64_t wbase = tile * (kRows * kLinT) + (threadIdx.x / kWave) * (kWave / G);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      int64_t pos;
      ok[t] = tm_locate<G, false>(p, seqs, wbase + t * kRows, h, crow[t], pos) && ok[t];
    }
  } else {
  Seq s = sequence(p, i, true);
  if (p.in_dir) {  // token rows -> cache: the loads need the rows
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      ok[t] = locate(p, s, i, h, j0 + t * kRows, r[t], crow[t]);
      if (!ok[t]) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        const char* tk = static_cast<const char*>(p.tok[kv]) +
                         (r[t] * p.st[kv] + (int64_t)h * p.sh[kv]) * es;
        v[t][kv] = stream_load(reinterpret_cast<const u32x4*>(tk + lane * 16));
      }
    }
  } else {  // cache -> token rows: load first, place the rows afterwards
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      const int64_t j = j0 + t * kRows;
      ok[t] = j < s.len;
      crow[t] = ok[t] ? cache_row(p, i, s.pos0 + j, h) : -1;
      ok[t] = crow[t] >= 0;
      if (!ok[t]) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        const char* c = static_cast<const char*>(p.cache[kv]) + crow[t] * row_bytes;
        v[t][kv] = stream_load(reinterpret_cast<const u32x4*>(c + lane * 16));
      }
    }
    finish_start(p, i, s);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      r[t] = s.start + j0 + t * kRows;
      ok[t] = ok[t] && r[t] >= 0 && r[t] < p.rows;
    }
  }
  }
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
    if (!ok[t]) continue;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv >= p.nkv) continue;
      char* tk = static_cast<char*>(p.tok[kv]) + (r[t] * p.st[kv] + (int64_t)h * p.sh[kv]) * es;
      char* c = static_cast<char*>(p.cache[kv]) + crow[t] * row_bytes;
      // rows written once and not read back: non-temporal (bf16 reshape, 8 x 4096 tokens:
      // 47.2 -> 45.9 us against cached stores)
      __builtin_nontemporal_store(
          v[t][kv], reinterpret_cast<u32x4*>((kTM || p.in_dir ? c : tk) + lane * 16));
    }
  }
}

// ------------------------------------------------------------------------------ 8-element I/O

// 8 elements of a token row as raw 16-byte vectors (one for 16-bit types, two for fp32).
template <class Tag>
struct Raw8 {
  u32x4 w[Tag::kBytes == 4 ? 2 : 1];
};

template <class Tag>
__device__ __forceinline__ Raw8<Tag> load8(const void* base, int64_t e) {
  Raw8<Tag> x;
  const u32x4* q = reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + e * Tag::kBytes);
  x.w[0] = stream_load(q);
  if constexpr (Tag::kBytes == 4) x.w[1] = stream_load(q + 1);
  return x;
}

template <class Tag>
__device__ __forceinline__ void unpack8(const Raw8<Tag>& x, float* v) {
  if constexpr (Tag::kBytes == 4) {
    unpack(F32{}, x.w[0], v);
    unpack(F32{}, x.w[1], v + 4);
  } else {
    unpack(Tag{}, x.w[0], v);
  }
}

// 8 elements of an output token row, non-temporal (the read ops write each row once; the
// linear dequant 41.9 -> 37.1 us against cached stores).
template <class Tag>
__device__ __forceinline__ void store8(void* base, int64_t e, const float* v) {
  if constexpr (Tag::kBytes == 4) {
    u32x4 a, b;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[k] = __float_as_uint(v[k]);
      b[k] = __float_as_uint(v[4 + k]);
    }
    u32x4* q = reinterpret_cast<u32x4*>(static_cast<float*>(base) + e);
    __builtin_nontemporal_store(a, q);
    __builtin_nontemporal_store(b, q + 1);
  } else {
    u32x4 w;
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = pack2(Tag{}, v[2 * k], v[2 * k + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + e));
  }
}

// Max over aligned groups of `gl` lanes (a power of two <= G, the same in every lane).
template <int G>
__device__ __forceinline__ uint32_t lane_group_max(uint32_t v, int gl) {
  if (G >= 2 && gl >= 2) v = max(v, dpp<kDppQuadSwap1>(v));
  if (G >= 4 && gl >= 4) v = max(v, dpp<kDppQuadSwap2>(v));
  if (G >= 8 && gl >= 8) v = max(v, dpp<kDppRowHalfMirror>(v));
  if (G >= 16 && gl >= 16) v = max(v, dpp<kDppRowMirror>(v));
  if (G >= 32 && gl >= 32) v = max(v, (uint32_t)__shfl_xor((int)v, 16, kWave));
  if (G >= 64 && gl >= 64) v = max(v, (uint32_t)__shfl_xor((int)v, 32, kWave));
  return v;
}

// ------------------------------------------------------------------------------ quantisers

// quant_to_linear_cache (kStatic false) / offline_quant_to_linear_cache (kStatic true):
// G = head_dim / 8 lanes per row, 8 channels per lane, kLinT rows per lane group.
template <class Tag, int G, bool kFp8, bool kStatic, bool kTM>
__global__ __launch_bounds__(256) void lin_quant(LinParams p) {
  constexpr int kRows = 256 / G;
  const int lane = threadIdx.x & (G - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<kTM>(p, h, tile);
  const int d0 = lane * 8;
  const float tscale0 = p.tscale[0], tscale1 = p.tscale[1];
  // per-channel static scales: the same 8 channels for every token of the thread
  float chan[2][8];
  if constexpr (kStatic) {
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv < p.nkv && p.smode == 0) {
        const u32x4* sp =
            reinterpret_cast<const u32x4*>(p.chan[kv] + (int64_t)h * p.head_dim + d0);
        const u32x4 a = sp[0], b = sp[1];
        unpack(F32{}, a, chan[kv]);
        unpack(F32{}, b, chan[kv] + 4);
      }
    }
  }
  const int64_t j0 = tile * (kRows * kLinT) + threadIdx.x / G;
  bool ok[kLinT];
  int64_t r[kLinT], crow[kLinT], pos[kLinT];
  Raw8<Tag> x[kLinT][2];
  if constexpr (kTM) {  // the grid over the token rows: loads first, the sequence afterwards
    const TmSeqs seqs = tm_prefetch(p);
    // unconditional row loads, as in lin_copy
    const void* vsrc = p.nkv > 1 ? p.tok[1] : p.tok[0];
    const int64_t vst = p.nkv > 1 ? p.st[1] : p.st[0], vsh = p.nkv > 1 ? p.sh[1] : p.sh[0];
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      r[t] = j0 + t * kRows;
      ok[t] = r[t] < p.rows;
      const int64_t rl = ok[t] ? r[t] : 0;
      x[t][0] = load8<Tag>(p.tok[0], rl * p.st[0] + (int64_t)h * p.sh[0] + d0);
      x[t][1] = load8<Tag>(vsrc, rl * vst + (int64_t)h * vsh + d0);
    }
    const int64_t wbase = tile * (kRows * kLinT) + (threadIdx.x / kWave) * (kWave / G);
#pragma unroll
    for (int t = 0; t < kLinT; ++t)
      ok[t] = tm_locate<G, true>(p, seqs, wbase + t * kRows, h, crow[t], pos[t]) && ok[t];
  } else {
    const Seq s = sequence(p, i);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      ok[t] = locate(p, s, i, h, j0 + t * kRows, r[t], crow[t]);  // the same in a row's lanes
      pos[t] = s.pos0 + j0 + t * kRows;
      if (!ok[t]) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv)
        if (kv < p.nkv) x[t][kv] = load8<Tag>(p.tok[kv], r[t] * p.st[kv] + (int64_t)h * p.sh[kv] + d0);
    }
  }

  // Every row is encoded before the first store: the stores count in the same memory counter
  // as the loads, so a row still to be read behind a store would wait for that store too.
  u32x2 code[kLinT][2];
  float rscale[kLinT][2];
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
    if (!ok[t]) continue;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv >= p.nkv) continue;
      float v[8];
      unpack8<Tag>(x[t][kv], v);
      uint32_t c[2];
      if constexpr (kStatic) {
        float sc[8], y[8], q[8];
        if (p.smode == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) sc[e] = chan[kv][e];
        } else {
          // the per-tensor scale as a value: a conditional expression choosing between the
          // address of a kernel-argument field and a global address compiles to a flat load
          // whose address the argument-field path never set (it faulted), so the two are
          // read separately
          float one = kv == 0 ? tscale0 : tscale1;
          if (p.smode == 1) one = p.chan[kv][(int64_t)h * p.block_rows + pos[t]];
#pragma unroll
          for (int e = 0; e < 8; ++e) sc[e] = one;
        }
        bool fast = true;
#pragma unroll
        for (int e = 0; e < 8; ++e) fast &= static_scale_fast(sc[e]);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = fast ? recip_rn(sc[e]) : 0.0f;
        static_quotients<8, kFp8>(v, sc, y, fast, q);
        encode_static<8, kFp8>(q, c);
      } else {
        const int gl = G / p.groups;  // lanes per scale group
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) m = abs_max(m, v[e]);
        // one scale per row (the common case): the full-row reduction without the group
        // width's branches between its steps (quant_to_linear_cache 41.1 -> 40.2 us)
        const float amax = __uint_as_float(p.groups == 1 ? group_max_u32<G>(__float_as_uint(m))
                                                         : lane_group_max<G>(__float_as_uint(m), gl));
        float scale;
        if constexpr (kFp8) {
          const RowScale rs = make_fp8_scale(amax);
          encode_fp8_row<8>(v, rs, c);
          scale = rs.s;
        } else {
          const RowScale rs = make_row_scale(amax);
          encode_row<8>(v, rs, c);
          scale = rs.s;
        }
        rscale[t][kv] = scale;
      }
      code[t][kv][0] = c[0];
      code[t][kv][1] = c[1];
    }
  }
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
    if (!ok[t]) continue;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv >= p.nkv) continue;
      if constexpr (!kStatic) {
        const int gl = G / p.groups;
        if ((lane & (gl - 1)) == 0)
          __builtin_nontemporal_store(rscale[t][kv], p.scale[kv] + crow[t] * p.groups + lane / gl);
      }
      u32x2* dst = reinterpret_cast<u32x2*>(static_cast<int8_t*>(p.cache[kv]) +
                                            crow[t] * p.head_dim + d0);
      if constexpr (TMO_LIN_NT_STORE) {
        store_nt(dst, code[t][kv]);
      } else {
        *dst = code[t][kv];
      }
    }
  }
}

// dequant_from_linear_cache: out = RN(fp32(code) * scale), 8 channels per lane, kLinT rows
// per lane group.
template <class Tag, int G>
__global__ __launch_bounds__(256) void lin_dequant(LinParams p) {
  constexpr int kRows = 256 / G;
  const int lane = threadIdx.x & (G - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<false>(p, h, tile);
  const int d0 = lane * 8;
  float chan[2][8];
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    if (kv < p.nkv && p.smode == 0) {
      const u32x4* sp = reinterpret_cast<const u32x4*>(p.chan[kv] + (int64_t)h * p.head_dim + d0);
      const u32x4 a = sp[0], b = sp[1];
      unpack(F32{}, a, chan[kv]);
      unpack(F32{}, b, chan[kv] + 4);
    }
  }
  const int64_t j0 = tile * (kRows * kLinT) + threadIdx.x / G;
  bool ok[kLinT];
  int64_t r[kLinT], crow[kLinT];
  u32x2 code[kLinT][2];
  float tok_scale[kLinT][2];
  Seq s;
  if (!p.cache_off && !p.block_tables && !p.bs_id && i < p.blocks && p.block_rows > 0) {
    // Cache row (i, h, j) needs no per-sequence number: the row loads go out together with the
    // sequence's numbers, from the row clamped into the cache (a position past the sequence
    // is read and not written), instead of waiting for the length first.
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      const int64_t j = j0 + t * kRows;
      const int64_t row = (i * p.heads + h) * p.block_rows + (j < p.block_rows ? j : p.block_rows - 1);
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        code[t][kv] = stream_load(reinterpret_cast<const u32x2*>(
            static_cast<const int8_t*>(p.cache[kv]) + row * p.head_dim + d0));
        if (p.smode != 0) tok_scale[t][kv] = p.scale[kv][row];
      }
    }
    s = sequence(p, i, true);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      const int64_t j = j0 + t * kRows;
      ok[t] = j < s.len && j < p.block_rows;
    }
  } else {
    s = sequence(p, i, true);
#pragma unroll
    for (int t = 0; t < kLinT; ++t) {
      const int64_t j = j0 + t * kRows;
      crow[t] = j < s.len ? cache_row(p, i, s.pos0 + j, h) : -1;
      ok[t] = crow[t] >= 0;
      if (!ok[t]) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        code[t][kv] = stream_load(reinterpret_cast<const u32x2*>(
            static_cast<const int8_t*>(p.cache[kv]) + crow[t] * p.head_dim + d0));
        if (p.smode != 0) tok_scale[t][kv] = p.scale[kv][crow[t]];
      }
    }
  }
  finish_start(p, i, s);
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
    r[t] = s.start + j0 + t * kRows;
    ok[t] = ok[t] && r[t] >= 0 && r[t] < p.rows;
  }
  // Both rows are converted before the first store: the stores count in the same in-order
  // memory counter as the loads, and a wait for V's codes placed after K's store (the
  // compiler cannot count across the two load paths above) waited for that store as well.
  float out[kLinT][2][8];
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sc = p.smode == 0 ? chan[kv][e] : tok_scale[t][kv];
        out[t][kv][e] = (float)(int8_t)(code[t][kv][e >> 2] >> (8 * (e & 3))) * sc;
      }
      // used here, so the scheduler cannot move the conversion (and its wait) past a store
      asm volatile("" ::"v"(out[t][kv][0]), "v"(out[t][kv][1]), "v"(out[t][kv][2]),
                   "v"(out[t][kv][3]), "v"(out[t][kv][4]), "v"(out[t][kv][5]),
                   "v"(out[t][kv][6]), "v"(out[t][kv][7]));
    }
  }
#pragma unroll
  for (int t = 0; t < kLinT; ++t) {
    if (!ok[t]) continue;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      if (kv >= p.nkv) continue;
      store8<Tag>(p.tok[kv], r[t] * p.st[kv] + (int64_t)h * p.sh[kv] + d0, out[t][kv]);
    }
  }
}

// ------------------------------------------------------------------------------ 4-bit caches

// int8 caches of signed 4-bit pairs (quant_bit 4, _ops.py:1723-1750, 3664-3700): the even element
// of a pair in the high nibble, the odd one in the low nibble (the dequant math's unpack[0::2] =
// byte >> 4, unpack[1::2] = byte << 4 >> 4).  K pairs adjacent channels ([.., cache_len, D / 2]),
// V pairs adjacent cache positions ([.., cache_len / 2, D]).  scale = RN(amax / 7) (one IEEE
// divide per row or group), code = clip(RNE(RN(x / scale)), -8, 7).
struct Scale4 {
  float s;
  double y64;  // recip64(s) for div_recip64
  bool fast;
};
__device__ __forceinline__ Scale4 make_scale4(float amax) {
  Scale4 r;
  r.s = amax / 7.0f;  // IEEE divide, once per row / group
  const bool normal = r.s >= kFastDivMinScale && r.s < __builtin_inff();
  r.fast = normal || r.s == 0.0f;  // y64 = 0 gives quotients +-0 (codes 0) for an all-zero row
  r.y64 = normal ? recip64(r.s) : 0.0;
  return r;
}
// 4-bit code (two's complement nibble) of x.  On the fast path |x| <= amax bounds |q| by 7, so
// the clamp to [-8, 7] of the reference math only acts on the IEEE-divide path.
__device__ __forceinline__ uint32_t nibble4(float x, const Scale4& r) {
  float q;
  if (r.fast) {
    q = div_recip64(x, r.y64);
  } else {
    keep_branch();
    q = x / r.s;
  }
  return rne_bits(__builtin_amdgcn_fmed3f(q, -8.0f, 7.0f)) & 0xFu;
}
__device__ __forceinline__ int32_t sext4(uint32_t n) { return ((int32_t)(n << 28)) >> 28; }

// Floor of v / 2 for any sign.
__device__ __forceinline__ int64_t floor_half(int64_t v) { return v >= 0 ? v / 2 : -((1 - v) / 2); }

// quant_to_linear_cache with quant_bit 4: G lanes per row (a power of two >= head_dim / 8;
// lanes past the row idle), 8 channels per lane, one lane group per pair of cache positions
// (2P, 2P + 1) of one head, so the two tokens that share the V bytes are encoded together and
// every V byte is written by one lane.  A position of the pair outside the sequence's tokens
// keeps its nibble: the lane merges only its own nibbles into the V bytes, with atomics.
template <class Tag, int G>
__global__ __launch_bounds__(256) void lin_quant4(LinParams p) {
  constexpr int kPairs = 256 / G;
  const int lane = threadIdx.x & (G - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<false>(p, h, tile);
  const Seq s = sequence(p, i);
  const int d0 = lane * 8;
  const bool lane_in = d0 < p.head_dim;
  const int64_t P = floor_half(s.pos0) + tile * kPairs + threadIdx.x / G;
  const int64_t L = p.block_rows, D = p.head_dim;
  const int gl = G / p.groups;  // lanes per scale group (power of two)
  bool tin[2];
  int64_t r[2], crow[2];
  Raw8<Tag> x[2][2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int64_t j = 2 * P + e - s.pos0;
    tin[e] = j >= 0 && locate(p, s, i, h, j, r[e], crow[e]);
    if (!tin[e] || !lane_in) continue;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv)
      if (kv < p.nkv) x[e][kv] = load8<Tag>(p.tok[kv], r[e] * p.st[kv] + (int64_t)h * p.sh[kv] + d0);
  }
  if (!tin[0] && !tin[1]) return;  // uniform per lane group; no barrier below
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    if (kv >= p.nkv) continue;
    uint32_t nib[2][8];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float v[8];
      if (tin[e] && lane_in) {
        unpack8<Tag>(x[e][kv], v);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = 0.0f;
      }
      float m = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) m = abs_max(m, v[k]);
      const float amax = __uint_as_float(p.groups == 1 ? group_max_u32<G>(__float_as_uint(m))
                                                       : lane_group_max<G>(__float_as_uint(m), gl));
      const Scale4 sc = make_scale4(amax);
#pragma unroll
      for (int k = 0; k < 8; ++k) nib[e][k] = nibble4(v[k], sc);
      if (tin[e] && lane_in && (lane & (gl - 1)) == 0)
        __builtin_nontemporal_store(sc.s, p.scale[kv] + crow[e] * p.groups + lane / gl);
      if (kv == 0 && tin[e] && lane_in) {  // K: channel pairs, 4 bytes per lane
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w |= ((nib[e][2 * k] << 4) | nib[e][2 * k + 1]) << (8 * k);
        store_nt(reinterpret_cast<uint32_t*>(static_cast<int8_t*>(p.cache[0]) + crow[e] * (D / 2) + d0 / 2), w);
      }
    }
    if (kv == 1 && lane_in) {  // V: position pairs, 8 bytes per lane at byte row P
      const int64_t cr = tin[0] ? crow[0] : crow[1];
      const int64_t pos = tin[0] ? 2 * P : 2 * P + 1;
      const int64_t vrow = (cr - pos) / L * (L / 2) + P;  // (batch * H + h) * (L / 2) + P
      u32x2* dst = reinterpret_cast<u32x2*>(static_cast<int8_t*>(p.cache[1]) + vrow * D + d0);
      u32x2 w;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        uint32_t acc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t hi = tin[0] ? nib[0][4 * q + k] : 0u;
          const uint32_t lo = tin[1] ? nib[1][4 * q + k] : 0u;
          acc |= ((hi << 4) | lo) << (8 * k);
        }
        w[q] = acc;
      }
      if (tin[0] && tin[1]) {
        *dst = w;
      } else {
        // One position of the pair belongs to this call's sequence, the other may belong to
        // another sequence of the same call (the same cache batch, adjacent position ranges
        // meeting at an odd position), written by another workgroup at the same time.  Each
        // side clears and sets only its own nibbles with 32-bit vector atomics, so the two
        // merges commute; a read-modify-write of the whole bytes could lose the other's.
        const uint32_t own = tin[0] ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          atomicAnd(d32 + q, ~own);
          atomicOr(d32 + q, w[q] & own);
        }
      }
    }
  }
}

// dequant_from_linear_cache with quant_bit 4: G lanes per row, 8 channels per lane, kLinT tokens
// per lane group; K reads the row's 4 bytes of the lane's channel pairs, V the 8 bytes of byte
// row pos / 2 and the nibble of the position's parity.
template <class Tag, int G>
__global__ __launch_bounds__(256) void lin_dequant4(LinParams p) {
  constexpr int kRows = 256 / G;
  const int lane = threadIdx.x & (G - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<false>(p, h, tile);
  const int d0 = lane * 8;
  const bool lane_in = d0 < p.head_dim;
  const int64_t L = p.block_rows, D = p.head_dim;
  float chan[2][8];
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    if (kv < p.nkv && p.smode == 0 && lane_in) {
      const u32x4* sp = reinterpret_cast<const u32x4*>(p.chan[kv] + (int64_t)h * D + d0);
      const u32x4 a = sp[0], b = sp[1];
      unpack(F32{}, a, chan[kv]);
      unpack(F32{}, b, chan[kv] + 4);
    }
  }
  // every lane stays until finish_start (its prefix sum reads across the wavefront)
  Seq s = sequence(p, i, true);
  const int64_t j = tile * kRows + threadIdx.x / G;
  const int64_t crow = j < s.len ? cache_row(p, i, s.pos0 + j, h) : -1;
  const bool ok = crow >= 0 && lane_in;
  const int64_t pos = s.pos0 + j;
  uint32_t kw = 0;
  u32x2 vw = {0u, 0u};
  float tsc[2] = {0.0f, 0.0f};
  if (ok) {
    kw = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(
        static_cast<const int8_t*>(p.cache[0]) + crow * (D / 2) + d0 / 2));
    if (p.nkv > 1) {
      const int64_t vrow = (crow - pos) / L * (L / 2) + pos / 2;
      vw = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(
          static_cast<const int8_t*>(p.cache[1]) + vrow * D + d0));
    }
    if (p.smode != 0) {
      tsc[0] = p.scale[0][crow];
      if (p.nkv > 1) tsc[1] = p.scale[1][crow];
    }
  }
  finish_start(p, i, s);
  const int64_t r = s.start + j;
  if (!ok || r < 0 || r >= p.rows) return;
  const int vshift = (pos & 1) ? 0 : 4;
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    if (kv >= p.nkv) continue;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t n;
      if (kv == 0) {
        const uint32_t byte = (kw >> (8 * (e / 2))) & 0xFFu;
        n = (e & 1) ? byte & 0xFu : byte >> 4;
      } else {
        const uint32_t byte = (vw[e / 4] >> (8 * (e % 4))) & 0xFFu;
        n = (byte >> vshift) & 0xFu;
      }
      const float sc = p.smode == 0 ? chan[kv][e] : tsc[kv];
      v[e] = (float)sext4(n) * sc;
    }
    store8<Tag>(p.tok[kv], r * p.st[kv] + (int64_t)h * p.sh[kv] + d0, v);
  }
}

// ------------------------------------------------------------------------------ generic path

// Any head_dim / alignment: one wavefront per (token, head) row, element by element, IEEE
// divides.  p.op: 0 copy (p.es bytes per element), 1 dynamic quant, 2 static quant, 3 dequant.
template <class Tag, bool kFp8>
__global__ __launch_bounds__(256) void lin_generic(LinParams p) {
  const int op = p.op;
  const int64_t es = p.es;
  constexpr int kRows = 256 / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t i = blockIdx.y;
  int h;
  int64_t tile;
  lin_tile_head<false>(p, h, tile);
  const Seq s = sequence(p, i);
  const int64_t j = tile * kRows + threadIdx.x / kWave;
  if (j >= s.len) return;
  const int64_t r = s.start + j;
  const int64_t pos = s.pos0 + j;
  const int64_t crow = cache_row(p, i, pos, h);
  if (r < 0 || r >= p.rows || crow < 0) return;
  const int D = p.head_dim;
  for (int kv = 0; kv < p.nkv; ++kv) {
    const int64_t te = r * p.st[kv] + (int64_t)h * p.sh[kv];
    if (op == 0) {
      char* t = static_cast<char*>(p.tok[kv]) + te * es;
      char* c = static_cast<char*>(p.cache[kv]) + crow * D * es;
      char* to = p.in_dir ? c : t;
      const char* from = p.in_dir ? t : c;
      for (int b = lane; b < D * es; b += kWave) to[b] = from[b];
      continue;
    }
    uint8_t* codes = static_cast<uint8_t*>(p.cache[kv]) + crow * D;
    if (op == 3) {
      for (int d = lane; d < D; d += kWave) {
        const float sc = p.smode == 0 ? p.chan[kv][(int64_t)h * D + d] : p.scale[kv][crow];
        store1(Tag{}, p.tok[kv], te + d, (float)(int8_t)codes[d] * sc);
      }
    } else if (op == 2) {
      const float tsc = kv == 0 ? p.tscale[0] : p.tscale[1];  // a value, not an address
      for (int d = lane; d < D; d += kWave) {
        float sc = tsc;
        if (p.smode == 0) sc = p.chan[kv][(int64_t)h * D + d];
        if (p.smode == 1) sc = p.chan[kv][(int64_t)h * p.block_rows + pos];
        const float q = load1(Tag{}, p.tok[kv], te + d) / sc;  // IEEE divide
        const uint32_t b =
            kFp8 ? fp8e4m3_bits(__builtin_amdgcn_fmed3f(q, -448.0f, 448.0f)) : code_bits(q);
        codes[d] = (uint8_t)(b & 0xffu);
      }
    } else {
      const int gs = D / p.groups;
      for (int g = 0; g < p.groups; ++g) {
        float m = 0.0f;
        for (int d = lane; d < gs; d += kWave)
          m = abs_max(m, load1(Tag{}, p.tok[kv], te + g * gs + d));
        const float amax = __uint_as_float(group_max_u32<kWave>(__float_as_uint(m)));
        const float sc = amax / (kFp8 ? 448.0f : 127.0f);  // IEEE divide
        for (int d = lane; d < gs; d += kWave) {
          const float q = load1(Tag{}, p.tok[kv], te + g * gs + d) / sc;
          uint32_t b;
          if (sc == 0.0f) {
            b = 0u;
          } else if (kFp8) {
            b = fp8e4m3_bits(__builtin_amdgcn_fmed3f(q, -448.0f, 448.0f));
          } else {
            b = code_bits(q);
          }
          codes[g * gs + d] = (uint8_t)(b & 0xffu);
        }
        if (lane == 0) p.scale[kv][crow * p.groups + g] = sc;
      }
    }
  }
}

// ------------------------------------------------------------------------------ launchers

bool aligned(const void* q, int a) { return reinterpret_cast<uintptr_t>(q) % a == 0; }

int grid_for(const LinParams& p, int64_t batch, int rows_per_wg, dim3& grid) {
  const int64_t tiles = (p.max_len + rows_per_wg - 1) / rows_per_wg;
  const int64_t gx = tiles * p.heads;
  if (gx > 0x7fffffffLL || batch > 65535) return TMO_ERR_INVALID_ARGUMENT;
  grid = dim3((unsigned)gx, (unsigned)batch);
  return TMO_OK;
}

// Token-major grid (write ops over packed input without context_seq_offset): the workgroups
// walk the token rows, (row tile, head) with the head fastest.  False when the launch does not
// qualify or the grid would not fit.
#ifndef TMO_LIN_TOKEN_MAJOR
#define TMO_LIN_TOKEN_MAJOR 1
#endif
bool token_major_grid(const LinParams& p, int rows_per_wg, dim3& grid) {
  // packed input only: a padded layout with a length past seqlen would give that sequence
  // rows of the next one, which a row-to-sequence mapping cannot reproduce
  if (!TMO_LIN_TOKEN_MAJOR || !p.in_dir || p.seq_off || p.block_tables || !p.packed ||
      p.batch > kWave - 1)
    return false;
  // whole groups of 8 tiles for the XCD-aware order (tiles past the rows do nothing)
  const int64_t gx = xcd_grid_tiles((p.rows + rows_per_wg - 1) / rows_per_wg) * p.heads;
  if (gx <= 0 || gx > 0x7fffffffLL) return false;
  grid = dim3((unsigned)gx, 1);
  return true;
}

// 16-byte vector access to the token tensors: base, token and head strides aligned.
bool token_vec_ok(const LinParams& p, int es) {
  for (int kv = 0; kv < p.nkv; ++kv)
    if (!aligned(p.tok[kv], 16) || (p.st[kv] * es) % 16 != 0 || (p.sh[kv] * es) % 16 != 0)
      return false;
  return true;
}

template <class Tag>
int launch_generic(const LinParams& p, int64_t batch, int op, int es, bool fp8, hipStream_t st) {
  dim3 grid;
  const int rc = grid_for(p, batch, 256 / kWave, grid);
  if (rc != TMO_OK) return rc;
  LinParams q = p;
  q.op = op;
  q.es = es;
  return fp8 ? launch_kernel(lin_generic<Tag, true>, grid, dim3(256), st, q)
             : launch_kernel(lin_generic<Tag, false>, grid, dim3(256), st, q);
}

int launch_copy(const LinParams& p, int64_t batch, int es, hipStream_t st) {
  const int64_t row_bytes = (int64_t)p.head_dim * es;
  const int G = row_bytes % 16 == 0 && row_bytes / 16 <= kWave ? (int)(row_bytes / 16) : 0;
  bool vec = G >= 1 && (G & (G - 1)) == 0 && token_vec_ok(p, es);
  for (int kv = 0; kv < p.nkv && vec; ++kv) vec = aligned(p.cache[kv], 16);
  if (!vec) return launch_generic<BF16>(p, batch, 0, es, false, st);
  dim3 grid;
  LinParams q = p;
  q.es = es;
  if (token_major_grid(p, (256 / G) * kLinT, grid)) {
    switch (G) {
      case 1: return launch_kernel(lin_copy<1, true>, grid, dim3(256), st, q);
      case 2: return launch_kernel(lin_copy<2, true>, grid, dim3(256), st, q);
      case 4: return launch_kernel(lin_copy<4, true>, grid, dim3(256), st, q);
      case 8: return launch_kernel(lin_copy<8, true>, grid, dim3(256), st, q);
      case 16: return launch_kernel(lin_copy<16, true>, grid, dim3(256), st, q);
      case 32: return launch_kernel(lin_copy<32, true>, grid, dim3(256), st, q);
      default: return launch_kernel(lin_copy<64, true>, grid, dim3(256), st, q);
    }
  }
  const int rc = grid_for(p, batch, (256 / G) * kLinT, grid);
  if (rc != TMO_OK) return rc;
  switch (G) {
    case 1: return launch_kernel(lin_copy<1, false>, grid, dim3(256), st, q);
    case 2: return launch_kernel(lin_copy<2, false>, grid, dim3(256), st, q);
    case 4: return launch_kernel(lin_copy<4, false>, grid, dim3(256), st, q);
    case 8: return launch_kernel(lin_copy<8, false>, grid, dim3(256), st, q);
    case 16: return launch_kernel(lin_copy<16, false>, grid, dim3(256), st, q);
    case 32: return launch_kernel(lin_copy<32, false>, grid, dim3(256), st, q);
    default: return launch_kernel(lin_copy<64, false>, grid, dim3(256), st, q);
  }
}

// Lanes per row of the 8-channels-per-lane kernels, or 0 when the generic path must run.
int lanes8(const LinParams& p, int es) {
  const int G = p.head_dim % 8 == 0 ? p.head_dim / 8 : 0;
  if (G < 1 || G > kWave || (G & (G - 1)) != 0 || !token_vec_ok(p, es)) return 0;
  for (int kv = 0; kv < p.nkv; ++kv) {
    if (!aligned(p.cache[kv], 8)) return 0;
    if (p.smode == 0 && p.chan[kv] && !aligned(p.chan[kv], 16)) return 0;
  }
  return G;
}

template <class Tag, bool kFp8, bool kStatic>
int launch_quant(const LinParams& p, int64_t batch, hipStream_t st) {
  const int G = lanes8(p, Tag::kBytes);
  bool vec = G > 0;
  if (vec && !kStatic) {  // scale groups must be whole, aligned sets of lanes
    const int gl = G % p.groups == 0 ? G / p.groups : 0;
    vec = gl >= 1 && (gl & (gl - 1)) == 0;
  }
  if (!vec) return launch_generic<Tag>(p, batch, kStatic ? 2 : 1, Tag::kBytes, kFp8, st);
  dim3 grid;
  if (token_major_grid(p, (256 / G) * kLinT, grid)) {
    switch (G) {
      case 1: return launch_kernel(lin_quant<Tag, 1, kFp8, kStatic, true>, grid, dim3(256), st, p);
      case 2: return launch_kernel(lin_quant<Tag, 2, kFp8, kStatic, true>, grid, dim3(256), st, p);
      case 4: return launch_kernel(lin_quant<Tag, 4, kFp8, kStatic, true>, grid, dim3(256), st, p);
      case 8: return launch_kernel(lin_quant<Tag, 8, kFp8, kStatic, true>, grid, dim3(256), st, p);
      case 16: return launch_kernel(lin_quant<Tag, 16, kFp8, kStatic, true>, grid, dim3(256), st, p);
      case 32: return launch_kernel(lin_quant<Tag, 32, kFp8, kStatic, true>, grid, dim3(256), st, p);
      default: return launch_kernel(lin_quant<Tag, 64, kFp8, kStatic, true>, grid, dim3(256), st, p);
    }
  }
  const int rc = grid_for(p, batch, (256 / G) * kLinT, grid);
  if (rc != TMO_OK) return rc;
  switch (G) {
    case 1: return launch_kernel(lin_quant<Tag, 1, kFp8, kStatic, false>, grid, dim3(256), st, p);
    case 2: return launch_kernel(lin_quant<Tag, 2, kFp8, kStatic, false>, grid, dim3(256), st, p);
    case 4: return launch_kernel(lin_quant<Tag, 4, kFp8, kStatic, false>, grid, dim3(256), st, p);
    case 8: return launch_kernel(lin_quant<Tag, 8, kFp8, kStatic, false>, grid, dim3(256), st, p);
    case 16: return launch_kernel(lin_quant<Tag, 16, kFp8, kStatic, false>, grid, dim3(256), st, p);
    case 32: return launch_kernel(lin_quant<Tag, 32, kFp8, kStatic, false>, grid, dim3(256), st, p);
    default: return launch_kernel(lin_quant<Tag, 64, kFp8, kStatic, false>, grid, dim3(256), st, p);
  }
}

// 4-bit launches: G = the power of two >= head_dim / 8 lanes per row; 0 when the shape or the
// alignment is outside the 4-bit kernels (head_dim % 8 != 0 or > 512, scale groups that are not
// whole aligned lane groups, unaligned tensors, an odd V cache length).
int lanes4(const LinParams& p, int es) {
  const int D = p.head_dim;
  if (D % 8 != 0 || D > 8 * kWave) return 0;
  int G = 1;
  while (G * 8 < D) G *= 2;
  if (p.groups > 1) {  // each group a whole, aligned, power-of-two set of lanes
    const int gl = G % p.groups == 0 ? G / p.groups : 0;
    if (G * 8 != D || gl < 1 || (gl & (gl - 1)) != 0) return 0;
  }
  if (!token_vec_ok(p, es) || !aligned(p.cache[0], 4)) return 0;
  if (p.nkv > 1 && (!aligned(p.cache[1], 8) || p.block_rows % 2 != 0)) return 0;
  for (int kv = 0; kv < p.nkv; ++kv)
    if (p.smode == 0 && p.chan[kv] && !aligned(p.chan[kv], 16)) return 0;
  return G;
}

template <class Tag>
int launch_quant4(const LinParams& p, int64_t batch, hipStream_t st) {
  const int G = lanes4(p, Tag::kBytes);
  if (G == 0) return TMO_ERR_UNSUPPORTED_MODE;
  // position pairs of a sequence: at most max_len / 2 + 1
  const int64_t pairs = p.max_len / 2 + 1, per_wg = 256 / G;
  const int64_t gx = (pairs + per_wg - 1) / per_wg * p.heads;
  if (gx > 0x7fffffffLL || batch > 65535) return TMO_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)gx, (unsigned)batch), block(256);
  switch (G) {
    case 1: return launch_kernel(lin_quant4<Tag, 1>, grid, block, st, p);
    case 2: return launch_kernel(lin_quant4<Tag, 2>, grid, block, st, p);
    case 4: return launch_kernel(lin_quant4<Tag, 4>, grid, block, st, p);
    case 8: return launch_kernel(lin_quant4<Tag, 8>, grid, block, st, p);
    case 16: return launch_kernel(lin_quant4<Tag, 16>, grid, block, st, p);
    case 32: return launch_kernel(lin_quant4<Tag, 32>, grid, block, st, p);
    default: return launch_kernel(lin_quant4<Tag, 64>, grid, block, st, p);
  }
}

template <class Tag>
int launch_dequant4(const LinParams& p, int64_t batch, hipStream_t st) {
  const int G = lanes4(p, Tag::kBytes);
  if (G == 0) return TMO_ERR_UNSUPPORTED_MODE;
  dim3 grid;
  const int rc = grid_for(p, batch, 256 / G, grid);
  if (rc != TMO_OK) return rc;
  switch (G) {
    case 1: return launch_kernel(lin_dequant4<Tag, 1>, grid, dim3(256), st, p);
    case 2: return launch_kernel(lin_dequant4<Tag, 2>, grid, dim3(256), st, p);
    case 4: return launch_kernel(lin_dequant4<Tag, 4>, grid, dim3(256), st, p);
    case 8: return launch_kernel(lin_dequant4<Tag, 8>, grid, dim3(256), st, p);
    case 16: return launch_kernel(lin_dequant4<Tag, 16>, grid, dim3(256), st, p);
    case 32: return launch_kernel(lin_dequant4<Tag, 32>, grid, dim3(256), st, p);
    default: return launch_kernel(lin_dequant4<Tag, 64>, grid, dim3(256), st, p);
  }
}

template <bool kStatic>
int dispatch_quant(const LinParams& p, int64_t batch, int dtype, bool fp8, hipStream_t st) {
  switch (dtype) {
    case TMO_DTYPE_F16:
      return fp8 ? launch_quant<F16, true, kStatic>(p, batch, st)
                 : launch_quant<F16, false, kStatic>(p, batch, st);
    case TMO_DTYPE_BF16:
      return fp8 ? launch_quant<BF16, true, kStatic>(p, batch, st)
                 : launch_quant<BF16, false, kStatic>(p, batch, st);
    default:
      return fp8 ? launch_quant<F32, true, kStatic>(p, batch, st)
                 : launch_quant<F32, false, kStatic>(p, batch, st);
  }
}

template <class Tag>
int launch_dequant(const LinParams& p, int64_t batch, hipStream_t st) {
  const int G = lanes8(p, Tag::kBytes);
  if (G == 0) return launch_generic<Tag>(p, batch, 3, Tag::kBytes, false, st);
  dim3 grid;
  const int rc = grid_for(p, batch, (256 / G) * kLinT, grid);
  if (rc != TMO_OK) return rc;
  switch (G) {
    case 1: return launch_kernel(lin_dequant<Tag, 1>, grid, dim3(256), st, p);
    case 2: return launch_kernel(lin_dequant<Tag, 2>, grid, dim3(256), st, p);
    case 4: return launch_kernel(lin_dequant<Tag, 4>, grid, dim3(256), st, p);
    case 8: return launch_kernel(lin_dequant<Tag, 8>, grid, dim3(256), st, p);
    case 16: return launch_kernel(lin_dequant<Tag, 16>, grid, dim3(256), st, p);
    case 32: return launch_kernel(lin_dequant<Tag, 32>, grid, dim3(256), st, p);
    default: return launch_kernel(lin_dequant<Tag, 64>, grid, dim3(256), st, p);
  }
}

int elem_bytes(int dtype) {
  switch (dtype) {
    case TMO_DTYPE_F32: return 4;
    case TMO_DTYPE_F16:
    case TMO_DTYPE_BF16: return 2;
    case TMO_DTYPE_I8: return 1;
    default: return 0;
  }
}

bool float_dtype(int dtype) {
  return dtype == TMO_DTYPE_F32 || dtype == TMO_DTYPE_F16 || dtype == TMO_DTYPE_BF16;
}

// Checks shared by the five entry points; fills the addressing part of `p`.
int common_setup(LinParams& p, void* key, void* value, int64_t kst, int64_t ksh, int64_t vst,
                 int64_t vsh, int64_t rows, void* kc, void* vc, int64_t blocks, int64_t heads,
                 int64_t block_rows, int64_t head_size, const int32_t* lens, int64_t batch,
                 int64_t max_len, int packed, int64_t seqlen, const int32_t* seq_off,
                 const int32_t* bs_id, const int32_t* cache_off, bool in_dir) {
  if (!key || !kc || !lens) return TMO_ERR_INVALID_ARGUMENT;
  const bool has_v = value != nullptr;
  if (has_v != (vc != nullptr)) return TMO_ERR_INVALID_ARGUMENT;
  if (rows < 0 || blocks < 0 || heads <= 0 || block_rows < 0 || head_size <= 0 || batch < 0 ||
      max_len < 0 || seqlen < 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (kst < 0 || ksh < 0 || (has_v && (vst < 0 || vsh < 0))) return TMO_ERR_INVALID_ARGUMENT;
  if (heads > 0x7fffffffLL || head_size > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  p.tok[0] = key;
  p.tok[1] = value;
  p.cache[0] = kc;
  p.cache[1] = vc;
  p.st[0] = kst;
  p.sh[0] = ksh;
  p.st[1] = vst;
  p.sh[1] = vsh;
  p.rows = rows;
  p.heads = (int32_t)heads;
  p.head_dim = (int32_t)head_size;
  p.nkv = has_v ? 2 : 1;
  p.in_dir = in_dir ? 1 : 0;
  p.blocks = blocks;
  p.block_rows = block_rows;
  p.lens = lens;
  p.packed = packed ? 1 : 0;
  p.pad_seqlen = seqlen;
  p.batch = batch;
  p.seq_off = seq_off;
  p.bs_id = bs_id;
  p.cache_off = cache_off;
  p.max_len = max_len;
  p.groups = 1;
  return TMO_OK;
}

bool nothing_to_do(const LinParams& p, int64_t batch) {
  return batch == 0 || p.max_len == 0 || p.rows == 0 || p.blocks == 0 || p.block_rows == 0;
}

}  // namespace
}  // namespace tmo

using namespace tmo;

extern "C" int tmo_hip_reshape_linear_cache(
    const void* key, const void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t rows, void* key_cache,
    void* value_cache, int64_t max_batch, int64_t num_heads, int64_t cache_len, int64_t head_size,
    const int32_t* context_lengths, int64_t batch, int64_t max_context_len, int packed,
    int64_t seqlen, const int32_t* context_seq_offset, const int32_t* cache_bs_id,
    const int32_t* cache_seqlen_offset, int dtype, void* stream) {
  const int es = elem_bytes(dtype);
  if (es == 0) return TMO_ERR_UNSUPPORTED_DTYPE;
  LinParams p{};
  const int rc = common_setup(p, const_cast<void*>(key), const_cast<void*>(value),
                              key_stride_token, key_stride_head, value_stride_token,
                              value_stride_head, rows, key_cache, value_cache, max_batch,
                              num_heads, cache_len, head_size, context_lengths, batch,
                              max_context_len, packed, seqlen, context_seq_offset, cache_bs_id,
                              cache_seqlen_offset, true);
  if (rc != TMO_OK) return rc;
  if (nothing_to_do(p, batch)) return TMO_OK;
  return launch_copy(p, batch, es, static_cast<hipStream_t>(stream));
}

extern "C" int tmo_hip_quant_to_linear_cache(
    const void* key, const void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t rows, void* key_cache,
    void* value_cache, float* key_scale, float* value_scale, int64_t max_batch,
    int64_t num_heads, int64_t cache_len, int64_t head_size, int64_t group_num,
    const int32_t* context_lengths, int64_t batch, int64_t max_context_len, int packed,
    int64_t seqlen, const int32_t* context_seq_offset, const int32_t* cache_bs_id,
    const int32_t* cache_seqlen_offset, int quant_bit, int dtype, int cache_dtype, void* stream) {
  if (!float_dtype(dtype) || (cache_dtype != TMO_DTYPE_I8 && cache_dtype != TMO_DTYPE_F8E4M3))
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (quant_bit != 8 && quant_bit != 4) return TMO_ERR_UNSUPPORTED_MODE;
  if (quant_bit == 4 && cache_dtype != TMO_DTYPE_I8) return TMO_ERR_UNSUPPORTED_DTYPE;
  if (group_num <= 0 || head_size % group_num != 0) return TMO_ERR_INVALID_ARGUMENT;
  if (!key_scale || ((value != nullptr) != (value_scale != nullptr)))
    return TMO_ERR_INVALID_ARGUMENT;
  LinParams p{};
  const int rc = common_setup(p, const_cast<void*>(key), const_cast<void*>(value),
                              key_stride_token, key_stride_head, value_stride_token,
                              value_stride_head, rows, key_cache, value_cache, max_batch,
                              num_heads, cache_len, head_size, context_lengths, batch,
                              max_context_len, packed, seqlen, context_seq_offset, cache_bs_id,
                              cache_seqlen_offset, true);
  if (rc != TMO_OK) return rc;
  p.scale[0] = key_scale;
  p.scale[1] = value_scale;
  p.groups = (int32_t)group_num;
  if (quant_bit == 4) {
    if (lanes4(p, dtype == TMO_DTYPE_F32 ? 4 : 2) == 0) return TMO_ERR_UNSUPPORTED_MODE;
    if (nothing_to_do(p, batch)) return TMO_OK;
    hipStream_t s4 = static_cast<hipStream_t>(stream);
    switch (dtype) {
      case TMO_DTYPE_F16: return launch_quant4<F16>(p, batch, s4);
      case TMO_DTYPE_BF16: return launch_quant4<BF16>(p, batch, s4);
      default: return launch_quant4<F32>(p, batch, s4);
    }
  }
  if (nothing_to_do(p, batch)) return TMO_OK;
  return dispatch_quant<false>(p, batch, dtype, cache_dtype == TMO_DTYPE_F8E4M3,
                               static_cast<hipStream_t>(stream));
}

extern "C" int tmo_hip_offline_quant_to_linear_cache(
    const void* key, const void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t rows, void* key_cache,
    void* value_cache, const float* key_scale, const float* value_scale,
    float key_scale_per_tensor, float value_scale_per_tensor, int quant_mode, int64_t max_batch,
    int64_t num_heads, int64_t cache_len, int64_t head_size, const int32_t* context_lengths,
    int64_t batch, int64_t max_context_len, int packed, int64_t seqlen,
    const int32_t* context_seq_offset, const int32_t* cache_bs_id,
    const int32_t* cache_seqlen_offset, int dtype, int cache_dtype, void* stream) {
  if (!float_dtype(dtype) || (cache_dtype != TMO_DTYPE_I8 && cache_dtype != TMO_DTYPE_F8E4M3))
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (quant_mode < 0 || quant_mode > 3) return TMO_ERR_UNSUPPORTED_MODE;
  const int smode = quant_mode >= 2 ? 2 : quant_mode;
  if (smode < 2 && (!key_scale || ((value != nullptr) != (value_scale != nullptr))))
    return TMO_ERR_INVALID_ARGUMENT;
  LinParams p{};
  const int rc = common_setup(p, const_cast<void*>(key), const_cast<void*>(value),
                              key_stride_token, key_stride_head, value_stride_token,
                              value_stride_head, rows, key_cache, value_cache, max_batch,
                              num_heads, cache_len, head_size, context_lengths, batch,
                              max_context_len, packed, seqlen, context_seq_offset, cache_bs_id,
                              cache_seqlen_offset, true);
  if (rc != TMO_OK) return rc;
  p.smode = smode;
  p.chan[0] = smode < 2 ? key_scale : nullptr;
  p.chan[1] = smode < 2 ? value_scale : nullptr;
  p.tscale[0] = key_scale_per_tensor;
  p.tscale[1] = value_scale_per_tensor;
  if (nothing_to_do(p, batch)) return TMO_OK;
  return dispatch_quant<true>(p, batch, dtype, cache_dtype == TMO_DTYPE_F8E4M3,
                              static_cast<hipStream_t>(stream));
}

extern "C" int tmo_hip_dequant_from_linear_cache(
    void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t rows, const int8_t* key_cache,
    const int8_t* value_cache, const float* key_scale, const float* value_scale,
    int64_t max_batch, int64_t num_heads, int64_t cache_len, int64_t head_size,
    const int32_t* context_lengths, int64_t batch, int64_t max_context_len,
    const int32_t* context_seq_offset, const int32_t* cache_bs_id, const int32_t* cache_seq_offset,
    int quant_mode, int quant_bit, int out_dtype, void* stream) {
  if (!float_dtype(out_dtype)) return TMO_ERR_UNSUPPORTED_DTYPE;
  if ((quant_bit != 8 && quant_bit != 4) || (quant_mode != 0 && quant_mode != 1))
    return TMO_ERR_UNSUPPORTED_MODE;
  if (!key_scale || ((value != nullptr) != (value_scale != nullptr)))
    return TMO_ERR_INVALID_ARGUMENT;
  LinParams p{};
  const int rc = common_setup(p, key, value, key_stride_token, key_stride_head,
                              value_stride_token, value_stride_head, rows,
                              const_cast<int8_t*>(key_cache), const_cast<int8_t*>(value_cache),
                              max_batch, num_heads, cache_len, head_size, context_lengths, batch,
                              max_context_len, 0, 0, context_seq_offset, cache_bs_id,
                              cache_seq_offset, false);
  if (rc != TMO_OK) return rc;
  p.smode = quant_mode;
  p.chan[0] = quant_mode == 0 ? key_scale : nullptr;
  p.chan[1] = quant_mode == 0 ? value_scale : nullptr;
  p.scale[0] = quant_mode == 1 ? const_cast<float*>(key_scale) : nullptr;
  p.scale[1] = quant_mode == 1 ? const_cast<float*>(value_scale) : nullptr;
  if (quant_bit == 4 && lanes4(p, out_dtype == TMO_DTYPE_F32 ? 4 : 2) == 0)
    return TMO_ERR_UNSUPPORTED_MODE;
  if (nothing_to_do(p, batch)) return TMO_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (quant_bit == 4) {
    switch (out_dtype) {
      case TMO_DTYPE_F16: return launch_dequant4<F16>(p, batch, s);
      case TMO_DTYPE_BF16: return launch_dequant4<BF16>(p, batch, s);
      default: return launch_dequant4<F32>(p, batch, s);
    }
  }
  switch (out_dtype) {
    case TMO_DTYPE_F16: return launch_dequant<F16>(p, batch, s);
    case TMO_DTYPE_BF16: return launch_dequant<BF16>(p, batch, s);
    default: return launch_dequant<F32>(p, batch, s);
  }
}

extern "C" int tmo_hip_reshape_from_cache(
    void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t rows, const void* key_cache,
    const void* value_cache, int64_t num_blocks, int64_t num_heads, int64_t block_rows,
    int64_t head_size, const int32_t* context_lengths, int64_t batch, int64_t max_context_len,
    const int32_t* context_seq_offset, const int32_t* block_tables, int64_t max_blocks,
    const int32_t* cache_seq_offset, int dtype, void* stream) {
  const int es = elem_bytes(dtype);
  if (es == 0) return TMO_ERR_UNSUPPORTED_DTYPE;
  if (block_tables && max_blocks <= 0) return TMO_ERR_INVALID_ARGUMENT;
  LinParams p{};
  const int rc = common_setup(p, key, value, key_stride_token, key_stride_head,
                              value_stride_token, value_stride_head, rows,
                              const_cast<void*>(key_cache), const_cast<void*>(value_cache),
                              num_blocks, num_heads, block_rows, head_size, context_lengths,
                              batch, max_context_len, 0, 0, context_seq_offset, nullptr,
                              cache_seq_offset, false);
  if (rc != TMO_OK) return rc;
  p.block_tables = block_tables;
  p.max_blocks = block_tables ? max_blocks : 0;
  if (nothing_to_do(p, batch)) return TMO_OK;
  return launch_copy(p, batch, es, static_cast<hipStream_t>(stream));
}
