// dequant_from_paged_cache for gfx950: gathers each sequence's int8 (or float8_e4m3fn) pages
// through its block table and writes RNE(fp32(code) * scale) as bf16 / fp16 into packed
// [sum(ctx), H, D] rows; scales fp32 or bf16.
//
// Semantics: reference _ops.py:3734-3824 (math block :3749-3774; cast order of the linear
// sibling :3677; quant_mode 0 per-channel scale [H, D], 1 per-token scale [NB, H, BS]).
// Entry point: tmo_hip_dequant_from_paged_cache (include/tmo_hip.h).
//
// A page of one head is block_size * head_dim contiguous bytes, and all heads of a block are
// contiguous, so a workgroup streams a whole [H, BS, D] block (K and V) with 16-byte loads,
// every thread holding kIters units of each in flight before it converts and stores 32-byte
// output runs.  The main (persistent) kernel walks a flat list of all pages; the per-page
// kernel covers layouts it does not take (non power-of-two heads, very large batches), and a
// scalar kernel covers head sizes that are not a multiple of 16.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "tmo_device.h"

namespace tmo {
namespace {

struct DequantParams {
  void* out[2];
  int64_t out_st[2];  // elements
  int64_t out_sh[2];  // elements
  int64_t total_rows;
  const int8_t* cache[2];  // int8 codes, or float8_e4m3fn bytes when fp8
  const void* scale[2];    // fp32, or bf16 when s_bf16
  const int32_t* ctx_len;
  const int32_t* seq_off;  // nullable
  const int32_t* block_tables;
  int64_t batch;
  int64_t max_blocks;    // row length of block_tables
  int64_t grid_blocks;   // pages per sequence covered by the grid
  int64_t num_blocks;
  int32_t heads;
  int32_t block_size;
  int32_t head_dim;
  int32_t u_shift;   // log2(head_dim / 16)        (vector paths)
  int32_t bs_shift;  // log2(block_size)           (vector paths)
  int32_t h_shift;   // log2(heads)                (persistent path)
  int32_t part_shift;  // log2(work items per page)  (page-list path)
  int32_t mode;      // 0 per-channel, 1 per-token
  int32_t nkv;
  int32_t fp8;       // float8_e4m3fn caches
  int32_t s_bf16;    // bf16 scales
};

// Code / scale formats of the vector kernels as one template argument: bit 1 set for
// float8_e4m3fn caches (else int8), bit 0 for bf16 scales (else fp32).
constexpr bool cs_fp8(int cs) { return (cs & 2) != 0; }
constexpr bool cs_bf16(int cs) { return (cs & 1) != 0; }

// 16 outputs of one 16-code unit (w) with the per-channel scales of channels d0 .. d0 + 15 of
// head h (in L2: loaded here, next to their use) or one per-token scale s.
template <int kCS>
__device__ __forceinline__ void decode16(const u32x4& w, const void* scale, int64_t chan0,
                                         bool per_token, float s, float* f) {
  if (per_token) {
#pragma unroll
    for (int e = 0; e < 16; ++e) f[e] = code_byte(w[e >> 2], e & 3, cs_fp8(kCS)) * s;
    return;
  }
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    u32x4 sv[2];
    if constexpr (cs_bf16(kCS)) {
      sv[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(scale) + chan0 + 8 * half);
    } else {
      const u32x4* sp = reinterpret_cast<const u32x4*>(static_cast<const float*>(scale) + chan0 + 8 * half);
      sv[0] = sp[0];
      sv[1] = sp[1];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      f[8 * half + e] = code_byte(w[2 * half + e / 4], e & 3, cs_fp8(kCS)) * scale_of8<cs_bf16(kCS)>(sv, e);
  }
}

// The per-token scale of page row srow, read in the scale tensor's own type.
template <int kCS>
__device__ __forceinline__ float token_scale(const void* scale, int64_t srow) {
  return scale_at(scale, srow, cs_bf16(kCS));
}

// Exclusive prefix sum of ctx_len[0..i), computed by the whole workgroup.
__device__ int64_t seq_begin(const DequantParams& p, int64_t i, int64_t* red) {
  if (p.seq_off) return p.seq_off[i];
  int64_t acc = 0;
  for (int64_t k = threadIdx.x; k < i; k += blockDim.x) acc += p.ctx_len[k];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = acc;
  __syncthreads();
  int64_t total = 0;
  for (int w = 0; w < (int)(blockDim.x / kWave); ++w) total += red[w];
  return total;
}

#ifndef TMO_DEQUANT_NT_STORE
#define TMO_DEQUANT_NT_STORE 0
#endif

template <class Tag>
__device__ __forceinline__ void store16(Tag, void* base, int64_t elem, const float* f) {
  u32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = pack2(Tag{}, f[2 * i], f[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = pack2(Tag{}, f[8 + 2 * i], f[8 + 2 * i + 1]);
  u32x4* dst = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + elem);
#if TMO_DEQUANT_NT_STORE
  __builtin_nontemporal_store(a, dst);
  __builtin_nontemporal_store(b, dst + 1);
#else
  dst[0] = a;  // cached stores: L2 merges the two half-sector streams of a wavefront
  dst[1] = b;
#endif
}

__device__ __forceinline__ void store16(F32, void* base, int64_t elem, const float* f) {
  u32x4* dst = reinterpret_cast<u32x4*>(static_cast<float*>(base) + elem);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4 a;
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = __float_as_uint(f[4 * i + j]);
    dst[i] = a;
  }
}

// Vector path: head_dim % 16 == 0 with head_dim/16 and block_size powers of two, 16-byte
// aligned caches and output rows.
template <class Tag, int kIters, int kCS>
__global__ __launch_bounds__(256) void dequant_paged_vec(DequantParams p) {
  __shared__ int64_t red[256 / kWave];
  const int64_t i = blockIdx.x / p.grid_blocks;  // sequence
  const int64_t j = blockIdx.x % p.grid_blocks;  // page of the sequence
  const int64_t len = p.ctx_len[i];
  const int64_t first = j * p.block_size;
  if (first >= len) return;
  const int64_t blk = p.block_tables[i * p.max_blocks + j];
  if (blk < 0 || blk >= p.num_blocks) return;
  const int ntok = (int)min<int64_t>(p.block_size, len - first);
  const int64_t row0 = seq_begin(p, i, red) + first;

  const int units_per_row = 1 << p.u_shift;               // 16-code units
  const int units = p.heads << (p.bs_shift + p.u_shift);  // whole block, all heads
  const int64_t page_base = blk * p.heads * (int64_t)p.block_size * p.head_dim;

  for (int u0 = 0; u0 < units; u0 += 256 * kIters) {
    u32x4 w[2][kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int u = u0 + it * 256 + threadIdx.x;
      const int o = (u >> p.u_shift) & (p.block_size - 1);
      if (u < units && o < ntok) {
#pragma unroll
        for (int kv = 0; kv < 2; ++kv)
          if (kv < p.nkv)
            w[kv][it] = *reinterpret_cast<const u32x4*>(p.cache[kv] + page_base + (int64_t)u * 16);
      }
    }
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int u = u0 + it * 256 + threadIdx.x;
      const int o = (u >> p.u_shift) & (p.block_size - 1);
      if (u >= units || o >= ntok) continue;
      const int h = u >> (p.u_shift + p.bs_shift);
      const int d0 = (u & (units_per_row - 1)) * 16;
      const int64_t row = row0 + o;
      if (row < 0 || row >= p.total_rows) continue;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        if (kv >= p.nkv) continue;
        float f[16];
        const float s = p.mode == 1
                            ? token_scale<kCS>(p.scale[kv], ((blk * p.heads + h) << p.bs_shift) + o)
                            : 0.0f;
        decode16<kCS>(w[kv][it], p.scale[kv], (int64_t)h * p.head_dim + d0, p.mode == 1, s, f);
        store16(Tag{}, p.out[kv], row * p.out_st[kv] + (int64_t)h * p.out_sh[kv] + d0, f);
      }
    }
  }
}

// Workgroups launched per CU by the flat-page kernel.  Far more than can be resident (8 per CU
// at 256 threads): the hardware dispatcher then hands the next workgroup to whichever CU frees
// a slot, which balances the tail that a fixed page-per-workgroup split leaves.  configs[4]
// (~75 K pages over 256 CUs): 8 per CU 1541 us, 64: 1442 us, 192-320: ~1400 us, 512 (one page
// per workgroup) 1476 us.
#ifndef TMO_DEQUANT_WG_PER_CU
#define TMO_DEQUANT_WG_PER_CU 256
#endif
#ifndef TMO_DEQUANT_WRITE_CONTIGUOUS
#define TMO_DEQUANT_WRITE_CONTIGUOUS 0
#endif
#ifndef TMO_DEQUANT_ITERS
#define TMO_DEQUANT_ITERS 8
#endif

// Position of 16-code unit u inside a page: write-contiguous order runs d16, head, token
// (a wavefront covers one token's [H, D] output row); read-contiguous order runs d16, token,
// head (a wavefront covers one head page's rows, the cache layout order).
struct UnitPos {
  int d16, h, o;
};
__device__ __forceinline__ UnitPos unit_pos(int u, int u_shift, int h_shift, int bs_shift) {
  UnitPos r;
  r.d16 = u & ((1 << u_shift) - 1);
  if (TMO_DEQUANT_WRITE_CONTIGUOUS) {
    r.h = (u >> u_shift) & ((1 << h_shift) - 1);
    r.o = u >> (u_shift + h_shift);
  } else {
    r.o = (u >> u_shift) & ((1 << bs_shift) - 1);
    r.h = u >> (u_shift + bs_shift);
  }
  return r;
}
constexpr int kPersistentMaxSeqs = 4096;

// Inclusive scan of v over the 256 threads of the workgroup (4 wavefronts); `tmp` holds
// 4 partials.  Returns the inclusive prefix; `total` receives the workgroup sum.
template <typename T>
__device__ __forceinline__ T block_scan(T v, T* tmp, T& total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const T n = __shfl_up(v, o, kWave);
    if (lane >= o) v += n;
  }
  if (lane == kWave - 1) tmp[wave] = v;
  __syncthreads();
  T before = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const T t = tmp[w];
    if (w < wave) before += t;
    total += t;
  }
  __syncthreads();
  return v + before;
}

// Persistent vector path (heads, head_dim / 16 and block_size powers of two, batch <= 4096).
// All pages of all sequences form one flat list, sequence-major; workgroup b takes pages
// b, b + gridDim.x, ... (about one page each at the launch size used, see
// TMO_DEQUANT_WG_PER_CU).  Each workgroup first scans context_lengths once into LDS: the first
// page and first output row of every sequence.  Inside a page the 16-code units follow the
// cache layout (d16, then token, then head: a wavefront reads 1 KiB of one head page and
// writes 256 B runs of 8 output rows), which measured faster on MI355X than the
// output-row-major order.
template <class Tag, int kIters, int kCS>
__global__ __launch_bounds__(256) void dequant_paged_persistent(DequantParams p) {
  extern __shared__ int64_t lds[];
  int64_t* tok_start = lds;                                           // [batch]
  int32_t* page_start = reinterpret_cast<int32_t*>(lds + p.batch);    // [batch + 1]
  int32_t* ctx = page_start + p.batch + 1;                            // [batch]
  __shared__ int64_t scan64[4];
  __shared__ int32_t scan32[4];

  int64_t tok_run = 0;
  int32_t page_run = 0;
  for (int64_t base = 0; base < p.batch; base += 256) {
    const int64_t i = base + threadIdx.x;
    int32_t n = i < p.batch ? p.ctx_len[i] : 0;
    const int64_t cap = p.grid_blocks * (int64_t)p.block_size;  // tokens the launch covers
    const int32_t covered = n <= 0 ? 0 : (int32_t)min<int64_t>(n, cap);
    const int32_t pages = (covered + p.block_size - 1) >> p.bs_shift;
    int64_t tot_tok;
    int32_t tot_pages;
    // output rows follow the plain running sum of context_lengths (reference _ops.py:3758)
    const int64_t incl_tok = block_scan<int64_t>(n, scan64, tot_tok);
    const int32_t incl_pages = block_scan<int32_t>(pages, scan32, tot_pages);
    if (i < p.batch) {
      tok_start[i] = p.seq_off ? (int64_t)p.seq_off[i] : tok_run + incl_tok - n;
      page_start[i] = page_run + incl_pages - pages;
      ctx[i] = covered;
    }
    tok_run += tot_tok;
    page_run += tot_pages;
  }
  if (threadIdx.x == 0) page_start[p.batch] = page_run;
  __syncthreads();
  const int32_t total_pages = page_run;

  const int d_shift = p.u_shift + 4;                 // log2(head_dim)
  const int units = p.block_size << (p.h_shift + p.u_shift);
  for (int32_t wpage = blockIdx.x; wpage < total_pages; wpage += gridDim.x) {
    // sequence of this page: the last i with page_start[i] <= wpage
    int32_t lo = 0, hi = (int32_t)p.batch;
    while (hi - lo > 1) {
      const int32_t mid = (lo + hi) >> 1;
      if (page_start[mid] <= wpage) lo = mid; else hi = mid;
    }
    const int64_t i = lo;
    const int64_t j = wpage - page_start[i];
    const int64_t blk = p.block_tables[i * p.max_blocks + j];
    if (blk < 0 || blk >= p.num_blocks) continue;  // workgroup-uniform
    const int ntok = min(p.block_size, ctx[i] - (int)(j << p.bs_shift));
    const int64_t row0 = tok_start[i] + (j << p.bs_shift);
    const int64_t page_base = blk << (p.h_shift + p.bs_shift + d_shift);

    for (int u0 = 0; u0 < units; u0 += 256 * kIters) {
      u32x4 w[2][kIters];
      float sc[2][kIters];
#pragma unroll
      for (int it = 0; it < kIters; ++it) {
        const int u = u0 + it * 256 + threadIdx.x;
        const UnitPos q = unit_pos(u, p.u_shift, p.h_shift, p.bs_shift);
        if (u < units && q.o < ntok) {
          const int64_t off =
              page_base + ((int64_t)((q.h << p.bs_shift) + q.o) << d_shift) + q.d16 * 16;
          const int64_t srow = (((blk << p.h_shift) + q.h) << p.bs_shift) + q.o;
#pragma unroll
          for (int kv = 0; kv < 2; ++kv) {
            if (kv < p.nkv) {
              w[kv][it] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.cache[kv] + off));
              if (p.mode == 1) sc[kv][it] = token_scale<kCS>(p.scale[kv], srow);
            }
          }
        }
      }
#pragma unroll
      for (int it = 0; it < kIters; ++it) {
        const int u = u0 + it * 256 + threadIdx.x;
        const UnitPos q = unit_pos(u, p.u_shift, p.h_shift, p.bs_shift);
        if (u >= units || q.o >= ntok) continue;
        const int64_t row = row0 + q.o;
        if (row < 0 || row >= p.total_rows) continue;
        const int d0 = q.d16 * 16;
#pragma unroll
        for (int kv = 0; kv < 2; ++kv) {
          if (kv >= p.nkv) continue;
          float f[16];
          decode16<kCS>(w[kv][it], p.scale[kv], (int64_t)q.h * p.head_dim + d0, p.mode == 1,
                        p.mode == 1 ? sc[kv][it] : 0.0f, f);
          store16(Tag{}, p.out[kv], row * p.out_st[kv] + (int64_t)q.h * p.out_sh[kv] + d0, f);
        }
      }
    }
  }
}

// 8 outputs of one 8-code unit as one contiguous 16-byte (bf16 / fp16) or 32-byte (fp32) run.
// Non-temporal: the rows are not read again by this kernel, and on configs[4] the page-list
// kernel measured 1340 -> 1301 us with them (the single-kernel path keeps cached stores, which
// merge its two half-sector stores per lane in L2).
template <class Tag>
__device__ __forceinline__ void store8(Tag, void* base, int64_t elem, const float* f) {
  u32x4 a;
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = pack2(Tag{}, f[2 * i], f[2 * i + 1]);
  __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + elem));
}
__device__ __forceinline__ void store8(F32, void* base, int64_t elem, const float* f) {
  u32x4* dst = reinterpret_cast<u32x4*>(static_cast<float*>(base) + elem);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    u32x4 a;
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = __float_as_uint(f[4 * i + j]);
    __builtin_nontemporal_store(a, dst + i);
  }
}

// ---------------------------------------------------------------------- page-list path
//
// With a caller-provided workspace the dequant runs as two kernels.  dequant_page_list writes
// the flat page list -- every page of every sequence, sequence-major, as (cache block, tokens
// in the page, first output row) -- and the page count; dequant_paged_list then gives each
// workgroup one item: 256 consecutive 8-code units of one page (for D = 128 and BS = 16 exactly
// one head page of K and of V, 2 KiB each).  A workgroup's only dependent read before its
// code loads is its 16-byte list entry (a scalar load issued together with the page count),
// so it reaches its HBM loads about as early as a kernel with a precomputed table can; small
// items measured ~5% faster than whole-page workgroups on MI355X with random block tables.
// Each thread converts one 8-code unit of K and of V and writes each as one contiguous
// 16-byte (32-byte for fp32) run; a wavefront's loads cover 512 contiguous code bytes and its
// stores 256-byte output-row runs.
struct PageEntry {
  int32_t blk;   // cache block, -1: skip the page (block-table entry outside [0, num_blocks))
  int32_t ntok;  // tokens of the page that are written (1..block_size)
  int64_t row0;  // output row of the page's first token
};
constexpr int64_t kListHeader = 16;  // bytes before the entries: int64 page count + padding

// Grid (ceil(grid_blocks / 256), batch): the workgroup of sequence i sums the page counts and
// context lengths of sequences 0..i-1 (its first page and first output row), then writes the
// entries of pages j = blockIdx.x * 256 + t < pages_i.  The last sequence's first workgroup
// writes the total page count.
__global__ __launch_bounds__(256) void dequant_page_list(DequantParams p, PageEntry* list,
                                                         int64_t* total) {
  __shared__ int64_t red[2][256 / kWave];
  const int64_t i = blockIdx.y;
  const int64_t cap = p.grid_blocks * (int64_t)p.block_size;  // tokens the launch covers
  auto pages_of = [&](int32_t n) -> int64_t {
    const int64_t covered = n <= 0 ? 0 : min<int64_t>(n, cap);
    return (covered + p.block_size - 1) >> p.bs_shift;
  };
  int64_t pg = 0, tok = 0;
  for (int64_t k = threadIdx.x; k < i; k += blockDim.x) {
    const int32_t n = p.ctx_len[k];
    pg += pages_of(n);
    tok += n;  // output rows follow the plain running sum (reference _ops.py:3758)
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    pg += __shfl_xor(pg, o, kWave);
    tok += __shfl_xor(tok, o, kWave);
  }
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    red[0][wave] = pg;
    red[1][wave] = tok;
  }
  __syncthreads();
  int64_t page_start = 0, tok_start = 0;
#pragma unroll
  for (int w = 0; w < 256 / kWave; ++w) {
    page_start += red[0][w];
    tok_start += red[1][w];
  }
  const int32_t n = p.ctx_len[i];
  const int64_t npages = pages_of(n);
  const int64_t covered = n <= 0 ? 0 : min<int64_t>(n, cap);
  if (p.seq_off) tok_start = p.seq_off[i];
  if (i == p.batch - 1 && blockIdx.x == 0 && threadIdx.x == 0) *total = page_start + npages;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= npages) return;
  const int32_t b = p.block_tables[i * p.max_blocks + j];
  PageEntry e;
  e.blk = (b < 0 || b >= p.num_blocks) ? -1 : b;
  e.ntok = (int32_t)min<int64_t>(p.block_size, covered - (j << p.bs_shift));
  e.row0 = tok_start + (j << p.bs_shift);
  list[page_start + j] = e;
}

template <class Tag, int kMode, int kKV, int kCS>
__global__ __launch_bounds__(256) void dequant_paged_list(DequantParams p,
                                                          const PageEntry* __restrict__ list,
                                                          const int64_t* __restrict__ total) {
  // XCD-aware item order: workgroups are dispatched round-robin over the 8 XCDs, so workgroup
  // b runs on XCD b % 8.  All items of one page go to the same XCD (page = 8 * (slot / parts)
  // + b % 8, part = slot % parts, slot = b / 8), where they share its L2 -- one fetch of the
  // page's per-token scale lines instead of one per XCD.  The grid is a multiple of
  // 8 * parts, so the order is a permutation of the grid's items.
  const int part_shift = p.part_shift;
  const int64_t stride = (int64_t)(gridDim.x >> part_shift);  // pages per grid sweep
  const uint32_t slot = blockIdx.x / kXcds;
  int64_t w = (int64_t)(slot >> part_shift) * kXcds + blockIdx.x % kXcds;
  const int u = ((int)(slot & ((1u << part_shift) - 1)) << 8) + threadIdx.x;
  const int u8 = p.u_shift + 1;  // log2(head_dim / 8)
  const int o = (u >> u8) & (p.block_size - 1);
  const int h = u >> (u8 + p.bs_shift);
  const int d0 = (u & ((1 << u8) - 1)) * 8;
  const int64_t page_codes = (int64_t)p.heads * p.block_size * p.head_dim;
  const int64_t page_rows = (int64_t)p.heads * p.block_size;
  // the entry is read before the count (the list holds at least `stride` entries), so the
  // two loads are issued together
  const int64_t first = w;
  PageEntry e = list[w];
  const int64_t pages = *total;
  for (; w < pages; w += stride) {
    if (w != first) e = list[w];
    if (e.blk < 0) continue;  // workgroup-uniform
    const int64_t row = e.row0 + o;
    const bool ok = o < e.ntok && row >= 0 && row < p.total_rows;
    // every unit of a valid page lies inside the caches, so the loads are unconditional (a
    // tail token past the context is read and not written); only the stores are predicated
    u32x2 c[kKV];
    float sc[kKV];
#pragma unroll
    for (int kv = 0; kv < kKV; ++kv) {
      c[kv] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x2*>(p.cache[kv] + e.blk * page_codes + (int64_t)u * 8));
      if constexpr (kMode == 1) sc[kv] = token_scale<kCS>(p.scale[kv], e.blk * page_rows + (u >> u8));
    }
#pragma unroll
    for (int kv = 0; kv < kKV; ++kv) {
      float f[8];
      if constexpr (kMode == 1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] = code_byte(c[kv][k >> 2], k & 3, cs_fp8(kCS)) * sc[kv];
      } else {
        u32x4 sv[2];
        const int64_t c0 = (int64_t)h * p.head_dim + d0;
        if constexpr (cs_bf16(kCS)) {
          sv[0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.scale[kv]) + c0);
        } else {
          const u32x4* sp = reinterpret_cast<const u32x4*>(static_cast<const float*>(p.scale[kv]) + c0);
          sv[0] = sp[0];
          sv[1] = sp[1];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
          f[k] = code_byte(c[kv][k >> 2], k & 3, cs_fp8(kCS)) * scale_of8<cs_bf16(kCS)>(sv, k);
      }
      if (ok) store8(Tag{}, p.out[kv], row * p.out_st[kv] + (int64_t)h * p.out_sh[kv] + d0, f);
    }
  }
}

// Workspace of the page-list path: header + one entry per page the launch can cover.
int64_t list_workspace_bytes(int64_t batch, int64_t grid_blocks) {
  const int64_t entries = (batch * grid_blocks + kXcds - 1) / kXcds * kXcds;
  return kListHeader + entries * (int64_t)sizeof(PageEntry);
}

// Generic path: one wavefront per (token, head) row, scalar loads and stores.
template <class Tag>
__global__ __launch_bounds__(256) void dequant_paged_generic(DequantParams p) {
  __shared__ int64_t red[256 / kWave];
  const int64_t i = blockIdx.x / p.grid_blocks;
  const int64_t j = blockIdx.x % p.grid_blocks;
  const int64_t len = p.ctx_len[i];
  const int64_t first = j * p.block_size;
  if (first >= len) return;
  const int64_t blk = p.block_tables[i * p.max_blocks + j];
  if (blk < 0 || blk >= p.num_blocks) return;
  const int ntok = (int)min<int64_t>(p.block_size, len - first);
  const int64_t row0 = seq_begin(p, i, red) + first;
  const int lane = threadIdx.x & (kWave - 1);
  const int nrows = p.heads * ntok;
  for (int r = threadIdx.x / kWave; r < nrows; r += 256 / kWave) {
    const int h = r / ntok, o = r % ntok;
    const int64_t row = row0 + o;
    if (row < 0 || row >= p.total_rows) continue;
    const int64_t prow = (blk * p.heads + h) * p.block_size + o;
    for (int kv = 0; kv < p.nkv; ++kv) {
      const int8_t* codes = p.cache[kv] + prow * p.head_dim;
      const int64_t obase = row * p.out_st[kv] + (int64_t)h * p.out_sh[kv];
      for (int d = lane; d < p.head_dim; d += kWave) {
        const float s = scale_at(p.scale[kv], p.mode == 1 ? prow : (int64_t)h * p.head_dim + d,
                                 p.s_bf16);
        store1(Tag{}, p.out[kv], obase + d, code_byte((uint8_t)codes[d], 0, p.fp8) * s);
      }
    }
  }
}

template <class Tag, int kCS>
int launch(DequantParams p, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  constexpr int kBytes = Tag::kBytes;
  const int64_t blocks = p.batch * p.grid_blocks;
  if (blocks > 0x7fffffffLL) return TMO_ERR_INVALID_ARGUMENT;
  const int u_shift = (p.head_dim % 16 == 0) ? ilog2_if_pow2(p.head_dim / 16) : -1;
  const int bs_shift = ilog2_if_pow2(p.block_size);
  bool vec = u_shift >= 0 && bs_shift >= 0 &&
             (int64_t)p.heads * p.block_size * (p.head_dim / 16) < (int64_t(1) << 30);
  for (int kv = 0; kv < p.nkv && vec; ++kv) {
    vec = reinterpret_cast<uintptr_t>(p.out[kv]) % 16 == 0 &&
          reinterpret_cast<uintptr_t>(p.cache[kv]) % 16 == 0 &&
          (p.out_st[kv] * kBytes) % 16 == 0 && (p.out_sh[kv] * kBytes) % 16 == 0 &&
          (p.mode == 1 || reinterpret_cast<uintptr_t>(p.scale[kv]) % 16 == 0);
  }
  const dim3 grid((unsigned)blocks), block(256);
  if (!vec) return launch_kernel(dequant_paged_generic<Tag>, grid, block, stream, p);
  p.u_shift = u_shift;
  p.bs_shift = bs_shift;
  p.h_shift = ilog2_if_pow2(p.heads);
  // page-list path: 256-unit items, a power of two of them per page, and a workspace.  Its
  // grid-stride loop covers every page whatever the grid; the grid is sized from the output
  // rows, which gives one item per workgroup: with no context_seq_offset and non-negative
  // context lengths, page w of the flat list starts at output row >= (w - batch) *
  // block_size, so at most ceil(total_rows / BS) + batch pages write anything.
  const int64_t page_units = (int64_t)p.heads * p.block_size * (p.head_dim / 8);
  const int part_shift = page_units % 256 == 0 ? ilog2_if_pow2(page_units / 256) : -1;
  if (workspace != nullptr && part_shift >= 0 && part_shift <= 20 &&
      workspace_bytes >= list_workspace_bytes(p.batch, p.grid_blocks) &&
      reinterpret_cast<uintptr_t>(workspace) % 16 == 0 && p.batch <= 65535) {
    p.part_shift = part_shift;
    int64_t* total = static_cast<int64_t*>(workspace);
    PageEntry* list = reinterpret_cast<PageEntry*>(static_cast<char*>(workspace) + kListHeader);
    const dim3 lgrid((unsigned)((p.grid_blocks + 255) / 256), (unsigned)p.batch);
    int st = launch_kernel(dequant_page_list, lgrid, block, stream, p, list, total);
    if (st != TMO_OK) return st;
    int64_t bound = (p.seq_off ? p.batch * p.grid_blocks
                               : (p.total_rows + p.block_size - 1) / p.block_size + p.batch);
    bound = std::min(bound, p.batch * p.grid_blocks);
    // whole groups of 8 pages (the XCD-aware order); pages past the list are skipped
    bound = (bound + kXcds - 1) / kXcds * kXcds;
    const int64_t cap = (0x7fffffffLL >> (part_shift + 3)) << 3;
    const int64_t want = std::min<int64_t>(bound, cap) << part_shift;
    const dim3 g((unsigned)want);
    if (p.nkv == 2)
      return p.mode == 1
                 ? launch_kernel(dequant_paged_list<Tag, 1, 2, kCS>, g, block, stream, p, list, total)
                 : launch_kernel(dequant_paged_list<Tag, 0, 2, kCS>, g, block, stream, p, list, total);
    return p.mode == 1
               ? launch_kernel(dequant_paged_list<Tag, 1, 1, kCS>, g, block, stream, p, list, total)
               : launch_kernel(dequant_paged_list<Tag, 0, 1, kCS>, g, block, stream, p, list, total);
  }
  if (p.h_shift >= 0 && p.batch <= kPersistentMaxSeqs &&
      ((int64_t)p.heads << (bs_shift + u_shift)) % 256 == 0) {
    int device = 0, cus = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return TMO_ERR_LAUNCH;
    const int64_t want = std::min<int64_t>(blocks, (int64_t)cus * TMO_DEQUANT_WG_PER_CU);
    const unsigned lds = (unsigned)(p.batch * 8 + (2 * p.batch + 1) * 4);
    return launch_kernel(dequant_paged_persistent<Tag, TMO_DEQUANT_ITERS, kCS>, dim3((unsigned)want),
                         block, stream, p, lds);
  }
  return launch_kernel(dequant_paged_vec<Tag, 4, kCS>, grid, block, stream, p);
}

// The kernels for the cache / scale formats of p (int8 or float8_e4m3fn codes, fp32 or bf16
// scales).
template <class Tag>
int launch_cs(const DequantParams& p, void* workspace, int64_t workspace_bytes, hipStream_t s) {
  switch ((p.fp8 ? 2 : 0) | (p.s_bf16 ? 1 : 0)) {
    case 0: return launch<Tag, 0>(p, workspace, workspace_bytes, s);
    case 1: return launch<Tag, 1>(p, workspace, workspace_bytes, s);
    case 2: return launch<Tag, 2>(p, workspace, workspace_bytes, s);
    default: return launch<Tag, 3>(p, workspace, workspace_bytes, s);
  }
}

int dequant_paged(void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
                  int64_t value_stride_token, int64_t value_stride_head, int64_t total_rows,
                  const void* key_cache, const void* value_cache, const void* key_scale,
                  const void* value_scale, const int32_t* context_lengths,
                  const int32_t* context_seq_offset, const int32_t* block_tables, int64_t batch,
                  int64_t max_blocks_per_seq, int64_t max_context_len, int64_t num_blocks,
                  int64_t num_heads, int64_t block_size, int64_t head_size, int quant_mode,
                  int quant_bit, int out_dtype, int cache_dtype, int scale_dtype,
                  void* workspace, int64_t workspace_bytes, void* stream);

}  // namespace
}  // namespace tmo

extern "C" int tmo_hip_dequant_from_paged_cache(
    void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t total_rows,
    const void* key_cache, const void* value_cache, const void* key_scale,
    const void* value_scale, const int32_t* context_lengths, const int32_t* context_seq_offset,
    const int32_t* block_tables, int64_t batch, int64_t max_blocks_per_seq,
    int64_t max_context_len, int64_t num_blocks, int64_t num_heads, int64_t block_size,
    int64_t head_size, int quant_mode, int quant_bit, int out_dtype, int cache_dtype,
    int scale_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return tmo::dequant_paged(key, value, key_stride_token, key_stride_head, value_stride_token,
                            value_stride_head, total_rows, key_cache, value_cache, key_scale,
                            value_scale, context_lengths, context_seq_offset, block_tables, batch,
                            max_blocks_per_seq, max_context_len, num_blocks, num_heads,
                            block_size, head_size, quant_mode, quant_bit, out_dtype, cache_dtype,
                            scale_dtype, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------- allocation-free entry
//
// The page list of tmo_hip_dequant_from_paged_cache_noalloc lives in `scratch`, a file-scope
// device array: each GPU the library runs on holds one (TMO_HIP_DEQUANT_SCRATCH_BYTES) until the
// process ends, and every call on that GPU shares it.  In host code `scratch` names a host-side
// stand-in, not device memory: its device address is taken once per device with
// hipGetSymbolAddress (that device current) and kept in scratch_addr[]; host code passes only
// that address to kernels.  Nothing in it has to start at zero: the pre-pass writes the page
// count and every entry the main kernel uses before that kernel runs (stream order).  Calls
// on one GPU are ordered on it by the entry point itself (order_calls below); calls captured
// into a HIP graph are ordered by that graph.
static __device__ __align__(256) unsigned char scratch[TMO_HIP_DEQUANT_SCRATCH_BYTES];

namespace tmo {
namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> scratch_addr[kMaxScratchDevices];
std::mutex scratch_mu;

// Device address of the current device's `scratch`, looked up on the first call per device.
int scratch_of_current_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return TMO_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxScratchDevices) return TMO_ERR_INVALID_ARGUMENT;
  void* p = scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TMO_ERR_LAUNCH;
      scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return TMO_OK;
}

// Ordering of the calls that share one GPU's scratch.  Host threads enqueue one at a time
// (the device's mutex, held from the wait to the record); a call on a stream other than the
// previous call's first makes its stream wait for the event recorded after the previous
// call's kernels (hipStreamWaitEvent: a queue dependency, no host wait), so the two calls'
// uses of the scratch never overlap; calls on one stream are already in order.  The event is
// created on the first such call on the device and kept until the process ends.  A stream
// under capture takes no event operation: the graph it is recorded into orders the call.
struct CallOrder {
  std::mutex mu;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool any = false;
};
CallOrder call_order[kMaxScratchDevices];

}  // namespace
}  // namespace tmo

extern "C" int tmo_hip_dequant_from_paged_cache_noalloc(
    void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
    int64_t value_stride_token, int64_t value_stride_head, int64_t total_rows,
    const void* key_cache, const void* value_cache, const void* key_scale,
    const void* value_scale, const int32_t* context_lengths, const int32_t* context_seq_offset,
    const int32_t* block_tables, int64_t batch, int64_t max_blocks_per_seq,
    int64_t max_context_len, int64_t num_blocks, int64_t num_heads, int64_t block_size,
    int64_t head_size, int quant_mode, int quant_bit, int out_dtype, int cache_dtype,
    int scale_dtype, void* stream) {
  using namespace tmo;
  if (batch < 0 || max_blocks_per_seq < 0) return TMO_ERR_INVALID_ARGUMENT;
  if (batch > 0 && max_blocks_per_seq > (TMO_HIP_DEQUANT_SCRATCH_BYTES - kListHeader) /
                                             (int64_t)sizeof(PageEntry) / batch)
    return TMO_ERR_SCRATCH_TOO_SMALL;
  const int64_t need = tmo_hip_dequant_workspace_bytes(batch, max_blocks_per_seq,
                                                       max_context_len, block_size);
  if (need > TMO_HIP_DEQUANT_SCRATCH_BYTES) return TMO_ERR_SCRATCH_TOO_SMALL;
  void* ws = nullptr;
  auto run = [&]() {
    return dequant_paged(key, value, key_stride_token, key_stride_head, value_stride_token,
                         value_stride_head, total_rows, key_cache, value_cache, key_scale,
                         value_scale, context_lengths, context_seq_offset, block_tables, batch,
                         max_blocks_per_seq, max_context_len, num_blocks, num_heads, block_size,
                         head_size, quant_mode, quant_bit, out_dtype, cache_dtype, scale_dtype,
                         ws, need > 0 ? (int64_t)TMO_HIP_DEQUANT_SCRATCH_BYTES : 0, stream);
  };
  if (need == 0) return run();  // nothing to do: no scratch, no kernel
  const int st = scratch_of_current_device(&ws);
  if (st != TMO_OK) return st;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return TMO_ERR_LAUNCH;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(hs, &cap) != hipSuccess) return TMO_ERR_LAUNCH;
  if (cap != hipStreamCaptureStatusNone) return run();
  CallOrder& o = call_order[dev];
  std::lock_guard<std::mutex> lock(o.mu);
  if (o.any && o.last != hs && hipStreamWaitEvent(hs, o.done, 0) != hipSuccess)
    return TMO_ERR_LAUNCH;
  const int rc = run();
  if (rc != TMO_OK) return rc;
  if (!o.done && hipEventCreateWithFlags(&o.done, hipEventDisableTiming) != hipSuccess) {
    o.done = nullptr;
    return TMO_ERR_LAUNCH;
  }
  if (hipEventRecord(o.done, hs) != hipSuccess) return TMO_ERR_LAUNCH;
  o.last = hs;
  o.any = true;
  return TMO_OK;
}

namespace tmo {
namespace {

int dequant_paged(void* key, void* value, int64_t key_stride_token, int64_t key_stride_head,
                  int64_t value_stride_token, int64_t value_stride_head, int64_t total_rows,
                  const void* key_cache, const void* value_cache, const void* key_scale,
                  const void* value_scale, const int32_t* context_lengths,
                  const int32_t* context_seq_offset, const int32_t* block_tables, int64_t batch,
                  int64_t max_blocks_per_seq, int64_t max_context_len, int64_t num_blocks,
                  int64_t num_heads, int64_t block_size, int64_t head_size, int quant_mode,
                  int quant_bit, int out_dtype, int cache_dtype, int scale_dtype,
                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0 || (workspace_bytes > 0 && workspace == nullptr))
    return TMO_ERR_INVALID_ARGUMENT;
  if (out_dtype != TMO_DTYPE_F16 && out_dtype != TMO_DTYPE_BF16 && out_dtype != TMO_DTYPE_F32)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if ((cache_dtype != TMO_DTYPE_I8 && cache_dtype != TMO_DTYPE_F8E4M3) ||
      (scale_dtype != TMO_DTYPE_F32 && scale_dtype != TMO_DTYPE_BF16))
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (quant_bit != 8 || (quant_mode != 0 && quant_mode != 1)) return TMO_ERR_UNSUPPORTED_MODE;
  if (!key || !key_cache || !key_scale || !context_lengths || !block_tables)
    return TMO_ERR_INVALID_ARGUMENT;
  const bool has_v = value != nullptr;
  if (has_v != (value_cache != nullptr) || has_v != (value_scale != nullptr))
    return TMO_ERR_INVALID_ARGUMENT;
  // max_context_len is not used: the reference's math (_ops.py:3749-3774) dequantises every
  // context_lengths[i] token its block table holds, whatever the maximum says
  (void)max_context_len;
  if (batch < 0 || max_blocks_per_seq < 0 || num_blocks < 0 ||
      num_heads <= 0 || block_size <= 0 || head_size <= 0 || total_rows < 0)
    return TMO_ERR_INVALID_ARGUMENT;
  if (key_stride_token < 0 || key_stride_head < 0 ||
      (has_v && (value_stride_token < 0 || value_stride_head < 0)))
    return TMO_ERR_INVALID_ARGUMENT;
  if (num_heads > 0x7fffffffLL || block_size > 0x7fffffffLL || head_size > 0x7fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  const int64_t grid_blocks = max_blocks_per_seq;
  if (batch == 0 || grid_blocks == 0 || num_blocks == 0 || total_rows == 0) return TMO_OK;

  DequantParams p{};
  p.out[0] = key;
  p.out[1] = value;
  p.out_st[0] = key_stride_token;
  p.out_st[1] = value_stride_token;
  p.out_sh[0] = key_stride_head;
  p.out_sh[1] = value_stride_head;
  p.total_rows = total_rows;
  p.cache[0] = static_cast<const int8_t*>(key_cache);
  p.cache[1] = static_cast<const int8_t*>(value_cache);
  p.scale[0] = key_scale;
  p.scale[1] = value_scale;
  p.ctx_len = context_lengths;
  p.seq_off = context_seq_offset;
  p.block_tables = block_tables;
  p.batch = batch;
  p.max_blocks = max_blocks_per_seq;
  p.grid_blocks = grid_blocks;
  p.num_blocks = num_blocks;
  p.heads = (int32_t)num_heads;
  p.block_size = (int32_t)block_size;
  p.head_dim = (int32_t)head_size;
  p.mode = quant_mode;
  p.nkv = has_v ? 2 : 1;
  p.fp8 = cache_dtype == TMO_DTYPE_F8E4M3;
  p.s_bf16 = scale_dtype == TMO_DTYPE_BF16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case TMO_DTYPE_F16: return launch_cs<F16>(p, workspace, workspace_bytes, s);
    case TMO_DTYPE_BF16: return launch_cs<BF16>(p, workspace, workspace_bytes, s);
    default: return launch_cs<F32>(p, workspace, workspace_bytes, s);
  }
}

}  // namespace
}  // namespace tmo

extern "C" int64_t tmo_hip_dequant_workspace_bytes(int64_t batch, int64_t max_blocks_per_seq,
                                                   int64_t max_context_len, int64_t block_size) {
  (void)max_context_len;  // the dequant covers every page of the block table (see above)
  if (batch <= 0 || max_blocks_per_seq <= 0 || block_size <= 0) return 0;
  return tmo::list_workspace_bytes(batch, max_blocks_per_seq);
}
