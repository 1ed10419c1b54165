// single_query_cached_kv_attn for gfx950: the query tokens of each sequence against its paged
// KV cache (reference _ops.py:777-900; header include/torch_mlu_ops.h:107-130).
//
//   s_j = softmax_scale * q . k_j (+ alibi_slope * (j - P)),
//   out = sum_j e^(s_j) v_j / (sum_j e^(s_j) (+ e^sink)),  lse = log of that denominator,
//
// for query token s of a sequence with nq tokens and L keys at position P = L - nq + s (one
// token: P = L - 1), over keys j in [max(0, P - window_left), P]; key j at row j % BS of page
// block_tables[i, j / BS] (pages outside [0, NB) are masked): k_j its first D channels, v_j
// the first Dv of the V cache's row, or of the K row when both live in one cache; query head
// hq reads KV head hq / (Hq / Hkv).  Caches are int8 codes, float8_e4m3fn values or int4 pairs
// (K pairing channels, V pairing the rows of a page or channels) with fp32 or bf16 scales (k =
// code * scale) per token [NB, Hkv, BS] (strided in the first two dims), per channel [Hkv, D],
// or per group (K [NB, Hkv, BS, D / 32], V [NB, Hkv, BS / 32, Dv]), or of q's dtype.  A mask
// adds its terms to the logits of each sequence's last mask_len keys.
//
// MFMA path (bf16 or f16 operands, fp32 accumulation; K and V head sizes and cache rows all 64
// / 128 / 256, block_size a multiple of 16, per-token or per-channel scales): the query columns of a (sequence, KV head) are its (token, query head)
// pairs, c = s * g + head-in-group (g = Hq / Hkv), in blocks of 16.  A workgroup of four
// wavefronts owns one (sequence, KV head, split, column block) and its wavefronts take every
// fourth 16-token tile.  Per tile:
//   * S^T = K Q^T with v_mfma_f32_16x16x16 (tokens are the rows, the block's query columns the
//     columns, zero-padded to 16): lane (t = l % 16, c = l / 16) holds token t's channels
//     [c D/4, (c + 1) D/4), so the K tile is read as contiguous row pieces, and MFMA m takes
//     channels c D/4 + 4m .. + 3 of every lane group (a permutation of the reduction order).
//     Int8 codes enter as exact f16 values 1152 + code (two byte permutes per four codes) against
//     a power-of-two scaled f16 q, and 1152 * sum(q) is subtracted from the fp32 result; the
//     per-token scale and softmax_scale * log2(e) then multiply it.  Int4 codes enter as
//     3 + code / 8 (int4_f16), 3 * sum(q) is subtracted and the factor 8 joins the scale.
//   * The result layout (lane holds tokens 4c .. 4c + 3 of query column l % 16) IS the B
//     operand layout of O^T = V^T P^T, so the probabilities feed the second product without a
//     shuffle.  V^T's operand needs four tokens of one channel per lane: lane (n, c) reads
//     D/16 bytes of tokens 4c .. 4c + 3 at channels n D/16 .., and MFMA j uses channel
//     n D/16 + j of them, so lane (q, c) accumulates channels [4c D/16, (4c + 4) D/16) -- one
//     contiguous run of the output row.
//   * p (times the per-token V scale) is split into hi + lo bf16 operands (16 significant
//     bits) and two products accumulate, against V codes converted to bf16 exactly; q gets a
//     lo operand too when it is folded with per-channel key scales.
//   * Online softmax in base 2 per query column, each column masked to its own key range; a
//     lane keeps a partial sum over its own four tokens, summed over the lane groups at the
//     end.  The sink joins the denominator when the output is written.
// The four wavefronts combine through LDS; with more than one split per (sequence, KV head)
// the partials (max, sum, normalised row) go to a caller-provided workspace and a combine
// kernel merges them.  A generic kernel (one wavefront per (query token, query head), VALU)
// serves every other shape, dtype and scale layout.
#include "tmo_device.h"

namespace tmo {
namespace {

typedef short bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;  // log2 headroom of the lazily moved softmax maximum
constexpr float kLn2 = 0.6931471805599453f;

// Query rows: token s of sequence i is at element i * q_sb + (row0_i + s) * q_ss + hq * q_sh,
// row0_i = cu[i] with cu_seq_q (q_sb 0 then) and 0 without; out and lse alike.
struct AttnParams {
  const void* q;
  int64_t q_sb, q_ss, q_sh;      // strides (elements); last dim contiguous
  const int32_t* cu;             // cu_seq_q [B + 1], or null: S tokens per sequence
  int32_t S;                     // tokens per sequence (at most, with cu)
  int32_t ncols;                 // S * g query columns per (sequence, KV head)
  int32_t ncb;                   // column blocks of 16
  int64_t total_q;               // q rows with cu: rows outside [0, total_q) are skipped
  const float* sink;             // [Hq] natural-log logits, or null
  const void* kc;
  const void* vc;                // caches [NB, Hkv, BS, k_row / v_row] contiguous
  int64_t k_row, v_row;          // cache row lengths (elements)
  const void* ks;                // scales: fp32, or bf16 when s_bf16
  const void* vs;
  int32_t s_bf16;
  int32_t smode;                 // 0 plain caches, 1 per token, 2 per channel, 3 per group
  int64_t ks_sb, ks_sh, vs_sb, vs_sh;  // per-token scale strides (page, head)
  const int32_t* bt;
  int64_t max_blocks;
  const int32_t* lens;
  const float* alibi;            // [B, Hq] or null
  int64_t window;                // < 0: unlimited
  float scale_log2;              // softmax_scale * log2(e)
  void* out;
  int64_t o_sb, o_ss, o_sh;
  float* lse;                    // null when not requested
  int64_t lse_sb, lse_ss, lse_sh;
  int32_t B, Hq, Hkv, g, D, Dv, BS;  // D: query / key head size, Dv: value head size
  int32_t bs_shift;              // log2(BS) when BS is a power of two, else -1
  int64_t NB;
  int32_t q_dtype;               // TMO_DTYPE_*: F32 / F16 / BF16, or I8 / F8E4M3 codes (qs)
  int32_t o_dtype;               // output TMO_DTYPE_* (q's for unquantised q)
  const void* qs;                // q scales of I8 / F8E4M3 q: fp32, or bf16 when qs_bf16
  int32_t qs_mode;               // 0 none, 1 per tensor, 2 per (token, head), 3 per channel group
  int32_t qs_bf16;
  int64_t qs_sb, qs_ss, qs_sh;   // q scale strides (sequence, token, head), as q's
  int32_t qs_group;              // mode 3: channels per scale (head_size / scale_num)
  int64_t bt_heads;              // block-table rows per sequence: 0 ([B, MB]), Hkv or Hq
  int32_t q_vec;                 // q rows 16-byte aligned 2-byte values: vector q loads
  int32_t c_dtype;               // cache TMO_DTYPE_*
  int32_t v_ch;                  // int4 caches: V pairs channels (else the rows of a page)
  const void* mask;              // [B, S, mask_len] logit terms of the last keys, or null
  int32_t mask_dtype;            // F32 / F16 / BF16
  int32_t mask_len;
  int64_t m_sb, m_ss;            // mask strides (sequence, token); last dim contiguous
  int32_t splits;
  int64_t split_tokens;          // multiple of 64
  float* ws;                     // [B, Hkv, splits, ncols, Dv + 2] when splits > 1
};

// ------------------------------------------------------------------------------ small helpers


__device__ __forceinline__ uint16_t bf16_bits_rne(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ float bf16_value(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Query element e as stored: a float, or an int8 / float8_e4m3fn code (its scale applies
// separately: q_scale_of below).
__device__ __forceinline__ float load_q(const AttnParams& p, int64_t e) {
  switch (p.q_dtype) {
    case TMO_DTYPE_BF16: return load1(BF16{}, p.q, e);
    case TMO_DTYPE_F16: return load1(F16{}, p.q, e);
    case TMO_DTYPE_I8: return (float)static_cast<const int8_t*>(p.q)[e];
    case TMO_DTYPE_F8E4M3: return fp8_value(static_cast<const uint8_t*>(p.q)[e], 0);
    default: return load1(F32{}, p.q, e);
  }
}

// Scale of quantised q: the whole row's (per tensor, per token and head) -- `base` the row's
// scale element i * qs_sb + row * qs_ss + hq * qs_sh -- or, per channel group, channel d's.
__device__ __forceinline__ float q_row_scale(const AttnParams& p, int64_t base) {
  if (p.qs_mode == 1) return scale_at(p.qs, 0, p.qs_bf16);
  if (p.qs_mode == 2) return scale_at(p.qs, base, p.qs_bf16);
  return 1.0f;
}
__device__ __forceinline__ float q_group_scale(const AttnParams& p, int64_t base, int d) {
  return p.qs_mode == 3 ? scale_at(p.qs, base + d / p.qs_group, p.qs_bf16) : 1.0f;
}

// The block-table row of sequence i for query head hq (KV head hk): sparse-KV tables hold one
// per KV head or per query head.
__device__ __forceinline__ const int32_t* bt_row_of(const AttnParams& p, int64_t i, int hq, int hk) {
  const int64_t r = p.bt_heads == 0 ? i : i * p.bt_heads + (p.bt_heads == p.Hq ? hq : hk);
  return p.bt + r * p.max_blocks;
}

__device__ __forceinline__ void store_out(const AttnParams& p, int64_t e, float v) {
  switch (p.o_dtype) {
    case TMO_DTYPE_BF16: store1(BF16{}, p.out, e, v); break;
    case TMO_DTYPE_F16: store1(F16{}, p.out, e, v); break;
    default: store1(F32{}, p.out, e, v); break;
  }
}

// Mask element e (a logit term, natural-log units) as fp32.
__device__ __forceinline__ float mask_value(const AttnParams& p, int64_t e) {
  switch (p.mask_dtype) {
    case TMO_DTYPE_BF16: return load1(BF16{}, p.mask, e);
    case TMO_DTYPE_F16: return load1(F16{}, p.mask, e);
    default: return load1(F32{}, p.mask, e);
  }
}

// Sequence i: its keys L (clamped to its block table), its query tokens nq (the first
// min(nq, S) are computed) and the row of its token 0.
struct Seq {
  int64_t L, nq, row0;
};

__device__ __forceinline__ Seq seq_of(const AttnParams& p, int64_t i) {
  Seq q;
  int64_t L = p.lens[i];
  const int64_t cap = p.max_blocks * (int64_t)p.BS;
  if (L > cap) L = cap;
  if (L < 0) L = 0;
  q.L = L;
  if (p.cu) {
    q.row0 = p.cu[i];
    q.nq = (int64_t)p.cu[i + 1] - q.row0;
  } else {
    q.row0 = 0;
    q.nq = p.S;
  }
  return q;
}

// Token s of the sequence is computed: within S and nq, and (with cu_seq_q) a row of q.
__device__ __forceinline__ bool token_valid(const AttnParams& p, const Seq& q, int64_t s) {
  return s < p.S && s < q.nq && (!p.cu || (q.row0 + s >= 0 && q.row0 + s < p.total_q));
}

// Key range of the sequence (token 0's window start to L) and of split s within it.
struct Range {
  int64_t begin, end;
};

__device__ __forceinline__ Range token_range(const AttnParams& p, const Seq& q, int s) {
  Range r;
  const int64_t L = q.L;
  int64_t j0 = 0;
  if (p.window >= 0 && L - q.nq - p.window > 0) j0 = L - q.nq - p.window;
  r.begin = j0 + (int64_t)s * p.split_tokens;
  r.end = r.begin + p.split_tokens < L ? r.begin + p.split_tokens : L;
  if (s == p.splits - 1) r.end = L;  // the last split takes any tokens past max_context_len
  if (p.splits == 1) r.begin = j0;
  return r;
}

// Final normalisation with the sink: m, l the column's maximum (base 2) and sum over its keys
// (l = 0: none).  Returns the factor of the unnormalised accumulators and writes the lse.
__device__ __forceinline__ float finish(const AttnParams& p, int hq, float m, float l, float* lse) {
  float inv = l > 0.0f ? 1.0f / l : 0.0f;
  float lg = l > 0.0f ? m + log2f(l) : -__builtin_inff();
  if (p.sink) {
    const float sk = p.sink[hq] * kLog2e;
    if (l > 0.0f) {
      const float mm = fmaxf(m, sk);
      const float lt = l * __builtin_amdgcn_exp2f(m - mm) + __builtin_amdgcn_exp2f(sk - mm);
      inv = __builtin_amdgcn_exp2f(m - mm) / lt;
      lg = mm + log2f(lt);
    } else {
      lg = sk;
    }
  }
  *lse = lg * kLn2;
  return inv;
}

// Max / sum over the four lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48) of a column.
__device__ __forceinline__ float col_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float col_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

// ------------------------------------------------------------------------------ MFMA kernel

template <bool kF16>
struct Mfma;
template <>
struct Mfma<false> {  // bf16 operands
  typedef bf16x4 V4;
  static __device__ __forceinline__ f32x4 run(V4 a, V4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ short bits(float x) { return (short)bf16_bits_rne(x); }
  static __device__ __forceinline__ float value(short b) { return bf16_value((uint16_t)b); }
};
template <>
struct Mfma<true> {  // f16 operands
  typedef f16x4 V4;
  static __device__ __forceinline__ f32x4 run(V4 a, V4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// Four int8 codes (one dword) -> four f16 operands holding 1152 + code exactly: with
// u = code + 128 (the byte with its top bit flipped), the f16 pattern 0x6400 | u is 1024 + u
// (ulp 1 in [1024, 2048)), so two byte permutes build the four values.  The QK product then
// carries 1152 * sum(q), which is subtracted per query column.
constexpr float kCodeBias = 1152.0f;
__device__ __forceinline__ f16x4 codes_f16(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  u32x2 h;
  h[0] = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [u0, 0x64, u1, 0x64]
  h[1] = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [u2, 0x64, u3, 0x64]
  return __builtin_bit_cast(f16x4, h);
}

// Four float8_e4m3fn codes (one dword) -> four f16 operands holding their values exactly:
// v_cvt_pk_f32_fp8 decodes two codes to fp32, v_cvt_pkrtz_f16_f32 packs two fp32 into f16
// (every e4m3fn value -- at most 4 significant bits, 2^-9 .. 448 -- is an f16 value, so the
// conversion's rounding never acts).
__device__ __forceinline__ f16x4 fp8_f16(uint32_t w) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  u32x2 h;
  h[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a[0], a[1]));
  h[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[0], b[1]));
  return __builtin_bit_cast(f16x4, h);
}

// Eight int4 codes (one dword of a K row: byte b holds channels 2b (high nibble) and 2b + 1
// (low nibble)) -> the f16 operands of channels 4h + {0, 2, 1, 3}, h = `half` (bytes 2h and
// 2h + 1), as 2 + u / 8 with u = code + 8 (the nibble with its top bit flipped): the f16
// pattern 0x4000 | u << 6 has exponent 1 and u in the top four mantissa bits, so the value
// 3 + code / 8 is exact.  Each f16 pair is one byte permute (the two high or two low nibbles
// into the pair's low bytes) and one shift-or.  The QK product then carries 3 * sum(q) and a
// factor 1/8; the channel order within the operand is matched by q's.
__device__ __forceinline__ f16x4 int4_f16(uint32_t w, int half) {
  const uint32_t x = w ^ 0x88888888u;
  const uint32_t hi = x & 0xf0f0f0f0u, lo = x & 0x0f0f0f0fu;
  const uint32_t sel = half ? 0x0c030c02u : 0x0c010c00u;  // [byte 2h, 0, byte 2h + 1, 0]
  u32x2 h;
  h[0] = (__builtin_amdgcn_perm(hi, hi, sel) << 2) | 0x40004000u;  // channels 4h, 4h + 2
  h[1] = (__builtin_amdgcn_perm(lo, lo, sel) << 6) | 0x40004000u;  // channels 4h + 1, 4h + 3
  return __builtin_bit_cast(f16x4, h);
}
constexpr float kInt4Bias = 3.0f;
// Channel of operand element e of QK MFMA m within the lane's run: int4 operands hold
// channels 4m + {0, 2, 1, 3}
__host__ __device__ constexpr int qk_channel(bool int4, int m, int e) {
  return 4 * m + (int4 ? (((e & 1) << 1) | (e >> 1)) : e);
}

// kKind: 0 int8 caches (f16 QK, bf16 PV), 1 bf16 caches, 2 f16 caches, 3 float8_e4m3fn caches
// (as int8: f16 QK against the exact code values, no bias; bf16 PV), 4 int4 pairs (K pairing
// channels, V pairing the rows of a page; f16 QK through int4_f16, bf16 PV of the exact
// codes).  kQLo: q needs a lo operand.  kSB: the scale tensors are bf16 (else fp32).  kMask:
// a mask is given (its terms are added in the tiles that reach the last mask_len keys; the
// instances without one carry none of that code and its registers).
// Workgroups per CU the register allocation must allow: three (168 registers per lane) for
// the quantised-cache kernels up to head_size 128, fewer where that would spill.
constexpr bool attn_quant(int kind) { return kind == 0 || kind == 3 || kind == 4; }
constexpr int attn_min_blocks(int d, int kind) {
  return d == 256 ? 1 : (!attn_quant(kind) && d == 128 ? 2 : 3);
}

#ifndef TMO_ATTN_DEPTH
#define TMO_ATTN_DEPTH 2
#endif

template <int kD, int kKind, bool kQLo, bool kSB, bool kMask>
__global__ __launch_bounds__(256, (attn_min_blocks(kD, kKind))) void attn_mfma(AttnParams p) {
  constexpr bool kQuant = attn_quant(kKind);  // codes with per-token / per-channel scales
  // tiles in flight per wavefront: three register sets where they fit the register budget of
  // attn_min_blocks (the quantised-cache kernels up to head_size 128)
  constexpr int kDepth = (kQuant && kD <= 128 && !kQLo) ? TMO_ATTN_DEPTH : 2;
  constexpr bool kF16 = kKind == 2;
  using M = Mfma<kF16>;
  using V4 = typename M::V4;
  constexpr int kDC = kD / 4;       // channels per lane group in the K layout
  constexpr int kDV = kD / 16;      // channels per lane in the V layout
  constexpr int kQK = kD / 16;      // QK MFMAs per tile
  constexpr int kEs = kQuant ? 1 : 2;  // cache element bytes
  constexpr bool kInt4 = kKind == 4;

  const int lane = threadIdx.x & (kWave - 1);
  // wave-uniform (readfirstlane): the tile indices, page numbers and page offsets derived from it
  // stay in scalar registers, and the tile loads take a scalar base plus a per-lane offset
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int col = lane & 15;        // query column within the block / token row
  const int grp = lane >> 4;        // lane group c
  const int64_t i = blockIdx.z;
  const int hk = blockIdx.y;
  const int cb = (int)(blockIdx.x / (unsigned)p.splits);   // column block
  const int split = (int)blockIdx.x - cb * p.splits;
  const Seq sq = seq_of(p, i);
  const Range rg = token_range(p, sq, split);
  // An empty split (past the sequence's keys) writes no partial; the combine skips it.  With
  // one split the (zero) output and lse are still written below.
  if (p.splits > 1 && rg.begin >= rg.end) return;
  // column c = token s * g + head hc: query head hk * g + hc of token s at position P
  const int c = cb * 16 + col;
  const int tok = c / p.g;
  const int hq = hk * p.g + (c - tok * p.g);
  const bool qvalid = c < p.ncols && token_valid(p, sq, tok);
  const int64_t qrow = sq.row0 + tok;

  // ---- Q operand (B of S^T = K Q^T): column `col`, channels grp * kDC + 4m .. + 3.  The QK
  // product runs on f16 operands: int8 codes as 1152 + code (codes_f16), q scaled by a power
  // of two sigma that puts the column's largest |q| in [2^14, 2^15) (an f16 holds every bf16
  // and f16 value of that column exactly down to 2^-29 of the largest), with a second (lo)
  // operand when q is folded with per-channel key scales.  Plain caches use their own type.
  using MQ = Mfma<kQuant ? true : kF16>;
  using VQ = typename MQ::V4;
  VQ qhi[kQK], qlo[kQLo ? kQK : 1];
  float qx[kQK][4];
  float qabs = 0.0f;
  // token positions fit in 32 bits (context lengths are int32).  Column keys: [klo, khi]
  // within the split, khi < klo when the column has none (or is padding).
  const int32_t pos = (int32_t)(sq.L - sq.nq) + tok;                 // the column's P
  int32_t klo = (int32_t)rg.begin, khi = (int32_t)rg.end - 1;
  if (p.window >= 0 && pos - (int32_t)p.window > klo) klo = pos - (int32_t)p.window;
  if (pos < khi) khi = pos;
  if (!qvalid) khi = klo - 1;
  // Tiles inside every valid column's keys need no per-key range test: [t0, t0 + 15] within
  // [wklo, wkhi], the largest klo and the smallest khi over the block's valid columns
  // (wave-uniform; the 16 columns are the lanes of each row, order-preserving u32 maxima).
  // Padding columns then carry scores of keys outside their range, which no output reads.
  int32_t wklo, wkhi;
  {
    const uint32_t lo = qvalid ? ((uint32_t)klo ^ 0x80000000u) : 0u;
    const uint32_t hi = qvalid ? ~((uint32_t)khi ^ 0x80000000u) : 0u;
    wklo = (int32_t)((uint32_t)__builtin_amdgcn_readfirstlane((int)group_max_u32<16>(lo)) ^
                     0x80000000u);
    wkhi = (int32_t)(~(uint32_t)__builtin_amdgcn_readfirstlane((int)group_max_u32<16>(hi)) ^
                     0x80000000u);
  }
  // The block's tiles: from its first valid token's window start to its last token's P
  // (wave-uniform: every lane computes the same numbers)
  int64_t bbeg = rg.begin, bend = rg.end;
  {
    const int64_t ntok = sq.nq < p.S ? sq.nq : p.S;
    const int64_t s_first = (int64_t)cb * 16 / p.g;
    int64_t s_last = ((int64_t)cb * 16 + 15) / p.g;
    if (s_last > ntok - 1) s_last = ntok - 1;
    const int64_t p_first = sq.L - sq.nq + s_first, p_last = sq.L - sq.nq + s_last;
    if (p.window >= 0 && p_first - p.window > bbeg) bbeg = p_first - p.window;
    if (p_last + 1 < bend) bend = p_last + 1;
    if (s_last < s_first || bend <= bbeg) bbeg = bend = 0;   // no key for the block: no tile
  }
  const int32_t first_tile = (int32_t)(bbeg >> 4);
  const int32_t end_tile = (int32_t)((bend + 15) >> 4);
  // the MFMA kernel takes tables of one row per sequence or per KV head
  const int32_t* bt_row = p.bt + (p.bt_heads ? i * p.bt_heads + hk : i) * p.max_blocks;
  auto page_of = [&](int32_t tl) -> int32_t {
    const int32_t t0 = tl * 16;
    return p.bs_shift >= 0 ? t0 >> p.bs_shift : t0 / p.BS;
  };
  // The wave's tiles are first_tile + wave + 4n.  Lane l holds the block of the window's
  // tile n = l (64 tiles per refill), read per tile with v_readlane.
  int32_t lane_blk = -1;
  int32_t win_base = first_tile + wave;
  auto refill = [&]() {
    const int32_t tl = win_base + 4 * lane;
    lane_blk = tl < end_tile ? bt_row[page_of(tl)] : -1;
  };
  // Start-up: the q row (and per-channel key scales) and the first block-table window are
  // independent reads, issued together -- q first, so the q arithmetic waits for q only and
  // the block ids arrive meanwhile; the first tile loads wait for the block ids alone.
  if (p.q_vec) {  // 16-byte aligned q rows of a 2-byte type: kDC / 8 vectors per lane
    constexpr int kQV = kDC / 8;
    u32x4 qraw[kQV];
    const u32x4* qp = reinterpret_cast<const u32x4*>(
        static_cast<const uint16_t*>(p.q) + i * p.q_sb + qrow * p.q_ss + (int64_t)hq * p.q_sh +
        grp * kDC);
#pragma unroll
    for (int v = 0; v < kQV; ++v) qraw[v] = qvalid ? qp[v] : u32x4{0u, 0u, 0u, 0u};
    // per-channel key scales of the lane's channels, raw: fp32 (4 per vector) or bf16 (8)
    constexpr int kCS = kQuant ? (kSB ? kDC / 8 : kDC / 4) : 1;
    u32x4 kcs[kCS];
    if (kQuant && p.smode == 2) {
      const int64_t e0 = (int64_t)hk * kD + grp * kDC;
      const u32x4* sp = kSB ? reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.ks) + e0)
                            : reinterpret_cast<const u32x4*>(static_cast<const float*>(p.ks) + e0);
#pragma unroll
      for (int v = 0; v < kCS; ++v) kcs[v] = sp[v];
    }
    refill();
    const bool bf = p.q_dtype == TMO_DTYPE_BF16;
#pragma unroll
    for (int m = 0; m < kQK; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = qk_channel(kInt4, m, e);  // channel within the lane's run
        const uint32_t w = qraw[c / 8][(c % 8) / 2];
        const uint32_t h = (c & 1) ? (w >> 16) : (w & 0xffffu);
        float x = bf ? __uint_as_float(h << 16) : f16_bits_to_f32(h);
        if (kQuant && p.smode == 2) {
          if constexpr (kSB) {
            const uint32_t sw = kcs[c / 8][(c % 8) / 2];
            x *= __uint_as_float((c & 1) ? (sw & 0xffff0000u) : (sw << 16));
          } else {
            x *= __uint_as_float(kcs[c / 4][c % 4]);
          }
        }
        qx[m][e] = x;
        qabs = fmaxf(qabs, fabsf(x));
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < kQK; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = grp * kDC + qk_channel(kInt4, m, e);
        float x = qvalid ? load_q(p, i * p.q_sb + qrow * p.q_ss + (int64_t)hq * p.q_sh + d) : 0.0f;
        if (kQuant && p.qs_mode == 3 && qvalid)  // group-wise q scales (kQLo holds the rest)
          x *= q_group_scale(p, i * p.qs_sb + qrow * p.qs_ss + (int64_t)hq * p.qs_sh, d);
        if (kQuant && p.smode == 2) x *= scale_at(p.ks, (int64_t)hk * kD + d, kSB);
        qx[m][e] = x;
        qabs = fmaxf(qabs, fabsf(x));
      }
    }
    refill();
  }
  float inv_sigma = 1.0f, qk_off = 0.0f;
  if constexpr (kQuant) {
    qabs = col_max(qabs);
    const int ex = qabs > 0.0f ? __builtin_amdgcn_frexp_expf(qabs) : 1;  // qabs in [2^(ex-1), 2^ex)
    const float sigma = __builtin_ldexpf(1.0f, 15 - ex);
    inv_sigma = __builtin_ldexpf(1.0f, ex - 15);
    float qsum = 0.0f;
#pragma unroll
    for (int m = 0; m < kQK; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y = qx[m][e] * sigma;
        const _Float16 h = (_Float16)y;
        qhi[m][e] = h;
        qsum += (float)h;
        if constexpr (kQLo) {
          const _Float16 l = (_Float16)(y - (float)h);
          qlo[m][e] = l;
          qsum += (float)l;
        }
      }
    }
    if constexpr (kKind == 0) qk_off = kCodeBias * col_sum(qsum);
    if constexpr (kInt4) qk_off = kInt4Bias * col_sum(qsum);
  } else {
#pragma unroll
    for (int m = 0; m < kQK; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (kF16) {
          qhi[m][e] = (_Float16)qx[m][e];
        } else {
          qhi[m][e] = M::bits(qx[m][e]);
        }
      }
    }
  }
  const float alibi = (p.alibi && qvalid) ? p.alibi[i * p.Hq + hq] * kLog2e : 0.0f;
  // inv_sigma: an exact power of two; int4 operands carry the codes / 8; a per-tensor or
  // per-token q scale multiplies the column's scores (its q operand holds the exact codes)
  const float q_rs = (kQuant && qvalid && p.qs_mode)
                         ? q_row_scale(p, i * p.qs_sb + qrow * p.qs_ss + (int64_t)hq * p.qs_sh)
                         : 1.0f;
  const float score_scale = p.scale_log2 * inv_sigma * (kInt4 ? 8.0f : 1.0f) * q_rs;
  // mask: terms for keys [mask_lo, L), element mask_row + m for key mask_lo + m
  const int32_t mask_lo = (int32_t)sq.L - p.mask_len;

  float mrun = -__builtin_inff();   // running max (base 2) of this lane's column
  float lpart = 0.0f;               // this lane's share of the running sum
  f32x4 acc[kDV];
#pragma unroll
  for (int j = 0; j < kDV; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const char* kbase = static_cast<const char*>(p.kc);
  const char* vbase = static_cast<const char*>(p.vc);
  // cache row bytes: K rows of kD elements (int4: kD / 2 bytes of channel pairs); V rows of kD
  // elements (int4: pair rows of kD bytes, each two tokens, so a page is BS / 2 of them and
  // the same bytes as a K page)
  constexpr int kKRow = kInt4 ? kD / 2 : kD * kEs;
  constexpr int kVRow = kInt4 ? kD : kD * kEs;
  constexpr int kVRows = kInt4 ? 2 : 4;                     // V rows per lane: tokens 4 grp .. + 3
  const int64_t page_bytes = (int64_t)p.BS * kKRow;         // one head's page
  // per-lane offsets inside a 16-row piece of a page: K token `col`, channels grp * kDC ..;
  // V tokens 4 grp .. + 3, channels col * kDV ..
  const int32_t k_lane = col * kKRow + grp * (kInt4 ? kDC / 2 : kDC * kEs);
  const int32_t v_lane = kVRows * grp * kVRow + col * kDV * (kInt4 ? 1 : kEs);
  constexpr int kKW = kInt4 ? kDC / 8 : kDC * kEs / 4;      // dwords per lane
  constexpr int kVW = kInt4 ? kDV / 4 : kDV * kEs / 4;

  // Raw tile: this lane's K piece, its V pieces of four tokens, the per-token scales.
  // The per-token scales stay raw until the tile is computed (fp32 words, or bf16 pairs in
  // ks[0..1] / vs[0..1]): widening them at load time would wait for the loads there.
  struct Raw {
    uint32_t kw[kKW];
    uint32_t vw[kVRows][kVW];
    uint32_t ks[4], vs[4];
  };
  auto raw_scale = [](const uint32_t (&w)[4], int e) -> float {
    if constexpr (kSB) return __uint_as_float((e & 1) ? (w[e / 2] & 0xffff0000u) : (w[e / 2] << 16));
    return __uint_as_float(w[e]);
  };
  auto load_tile = [&](Raw& r, int32_t tl, int64_t blk) {
    const int32_t t0 = tl * 16;
    const int32_t row0 = t0 - page_of(tl) * p.BS;
    // the piece's offset in a K page; in an int4 V page (pair rows of kD bytes) row0 / 2 * kD
    // is the same number
    const int64_t piece = (blk * p.Hkv + hk) * page_bytes + (int64_t)row0 * kKRow;
    const char* krow = kbase + piece + k_lane;
    if constexpr (kKW >= 4) {
#pragma unroll
      for (int u = 0; u < kKW / 4; ++u) {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(krow) + u);
#pragma unroll
        for (int e = 0; e < 4; ++e) r.kw[4 * u + e] = w[e];
      }
    } else if constexpr (kKW == 2) {
      const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(krow));
      r.kw[0] = w[0];
      r.kw[1] = w[1];
    } else {
      r.kw[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(krow));
    }
#pragma unroll
    for (int e = 0; e < kVRows; ++e) {
      const char* vrow = vbase + piece + v_lane + e * kVRow;
      if constexpr (kVW == 4) {
        const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vrow));
#pragma unroll
        for (int u = 0; u < 4; ++u) r.vw[e][u] = w[u];
      } else if constexpr (kVW == 2) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vrow));
        r.vw[e][0] = w[0];
        r.vw[e][1] = w[1];
      } else if constexpr (kVW == 1) {
        r.vw[e][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vrow));
      } else {  // 32 bytes
        const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vrow));
        const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vrow) + 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          r.vw[e][u] = a[u];
          r.vw[e][4 + u] = b[u];
        }
      }
    }
    constexpr uint32_t kOne = kSB ? 0x3f803f80u : 0x3f800000u;  // 1.0 (a bf16 pair)
#pragma unroll
    for (int e = 0; e < 4; ++e) r.ks[e] = r.vs[e] = kOne;
    if (kQuant && p.smode == 1) {
      const int32_t so = row0 + 4 * grp;
      const int64_t ka = blk * p.ks_sb + hk * p.ks_sh + so, va = blk * p.vs_sb + hk * p.vs_sh + so;
      if constexpr (kSB) {
        const u32x2 a = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p.ks) + ka);
        const u32x2 b = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p.vs) + va);
        r.ks[0] = a[0];
        r.ks[1] = a[1];
        r.vs[0] = b[0];
        r.vs[1] = b[1];
      } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const float*>(p.ks) + ka);
        const u32x4 b = *reinterpret_cast<const u32x4*>(static_cast<const float*>(p.vs) + va);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r.ks[e] = a[e];
          r.vs[e] = b[e];
        }
      }
    }
  };

  // Arithmetic of one loaded tile (the whole wavefront: the MFMAs need every lane).
  auto compute_tile = [&](const Raw& r, int32_t tile) {
      const int32_t t0 = tile * 16;
      // ---- S^T = K Q^T
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int m = 0; m < kQK; ++m) {
        VQ a;
        if constexpr (kKind == 0) {
          a = codes_f16(r.kw[m]);
        } else if constexpr (kInt4) {
          a = int4_f16(r.kw[m >> 1], m & 1);
        } else if constexpr (kKind == 3) {
          a = fp8_f16(r.kw[m]);
        } else {
          u32x2 w;
          w[0] = r.kw[2 * m];
          w[1] = r.kw[2 * m + 1];
          a = __builtin_bit_cast(VQ, w);
        }
        s = MQ::run(a, qhi[m], s);
        if constexpr (kQLo) s = MQ::run(a, qlo[m], s);
      }

      // ---- scores (base 2), masking, online softmax
      float sc[4];
      float tmax = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = (s[e] - qk_off) * (raw_scale(r.ks, e) * score_scale);
      // ALiBi and the key-range test as wave-uniform branches (if-converted, both ran on
      // every tile: ~36 VALU per tile, a tenth of the int4 kernel's)
      if (p.alibi) {
        keep_branch();
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] += alibi * (float)(t0 + 4 * grp + e - pos);
      }
      if (t0 < wklo || t0 + 15 > wkhi) {
        keep_branch();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t j = t0 + 4 * grp + e;
          if (j < klo || j > khi) sc[e] = -__builtin_inff();
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, sc[e]);
      // mask terms of the last mask_len keys: only the tiles that reach them (wave-uniform)
      if (kMask && t0 + 15 >= mask_lo) {
        // the column's row of terms (recomputed here: nothing stays live across the tiles;
        // a padding column reads token S - 1's row, in bounds, and its scores stay -inf)
        const int ct = (cb * 16 + col) / p.g;
        const int64_t mask_row = i * p.m_sb + (int64_t)(ct < p.S ? ct : p.S - 1) * p.m_ss;
        tmax = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t j = t0 + 4 * grp + e;
          if (j >= mask_lo) sc[e] += mask_value(p, mask_row + (j - mask_lo)) * kLog2e;
          tmax = fmaxf(tmax, sc[e]);
        }
      }
      tmax = col_max(tmax);
      // No branch on the column's state: the MFMAs below need the whole wavefront.  The
      // reference maximum moves only when a score exceeds it by more than kLazy (base 2), so
      // the probabilities stay below 2^kLazy and the accumulators are rarely rescaled; the
      // first finite score sets it.
      const bool was_empty = mrun == -__builtin_inff();
      const bool raise = tmax > mrun + kLazy || (was_empty && tmax != -__builtin_inff());
      const float mnew = raise ? tmax : mrun;
      const bool live = mnew != -__builtin_inff();          // some key of this column so far
      const float corr = raise ? __builtin_amdgcn_exp2f(mrun - mnew) : 1.0f;  // -inf -> 0
      mrun = mnew;
      float pe[4];
      float psum = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pe[e] = live ? __builtin_amdgcn_exp2f(sc[e] - mnew) : 0.0f;  // masked: -inf -> 0
        psum += pe[e];
      }
      lpart = lpart * corr + psum;
      if (__ballot(corr != 1.0f && !was_empty)) {  // an empty column's accumulators are zero
#pragma unroll
        for (int j = 0; j < kDV; ++j) acc[j] *= corr;
      }

      // ---- P^T operands (hi + lo) with the per-token V scale folded in
      V4 phi, plo;
      if constexpr (!kF16) {
        // bf16 pairs: one v_cvt_pk_bf16_f32 rounds two probabilities (hi), the hi values are
        // read back from the packed bits, and one more rounds the two remainders (lo)
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        u32x2 hv, lv;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const f2 a = {pe[2 * k] * raw_scale(r.vs, 2 * k), pe[2 * k + 1] * raw_scale(r.vs, 2 * k + 1)};
          const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(a, bf2));
          const f2 l = {a[0] - __uint_as_float(h << 16), a[1] - __uint_as_float(h & 0xffff0000u)};
          hv[k] = h;
          lv[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(l, bf2));
        }
        phi = __builtin_bit_cast(V4, hv);
        plo = __builtin_bit_cast(V4, lv);
      } else
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pv = pe[e] * raw_scale(r.vs, e);
        if constexpr (kF16) {
          const _Float16 h = (_Float16)pv;
          phi[e] = h;
          plo[e] = (_Float16)(pv - (float)h);
        } else {
          const short hb = M::bits(pv);
          phi[e] = hb;
          plo[e] = M::bits(pv - M::value(hb));
        }
      }

      // int4 V: the nibbles of token 4 grp + e moved into the high half of their bytes, so
      // each byte read as signed is 16 x the code (the low nibble shifted up, the other half
      // cleared; one mask per dword, kept whole in a register -- left to the combiner, the
      // masks were split into per-byte shifts and extractions)
      uint32_t vm[kInt4 ? 4 : 1][kInt4 ? kVW : 1];
      if constexpr (kInt4) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int u = 0; u < kVW; ++u) {
            const uint32_t w = r.vw[e >> 1][u];
            uint32_t m = ((e & 1) ? (w << 4) : w) & 0xF0F0F0F0u;
            asm("" : "+v"(m));
            vm[e][u] = m;
          }
      }

      // ---- O^T += V^T P^T: MFMA j takes channel col * kDV + j of tokens 4 grp .. + 3
#pragma unroll
      for (int j = 0; j < kDV; ++j) {
        typedef short s4 __attribute__((ext_vector_type(4)));
        s4 b4;
        if constexpr (kKind == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int8_t code = (int8_t)(r.vw[e][j >> 2] >> (8 * (j & 3)));
            b4[e] = (short)(__float_as_uint((float)code) >> 16);
          }
        } else if constexpr (kInt4) {
          // channel j's byte of pair row e / 2 holds tokens 4 grp + e (high nibble, e even)
          // and + 1 (low nibble); byte j & 3 of the masked dword is 16 x the code: one
          // sign-extending byte conversion, as for int8 codes, exact as bf16.  The factor 16
          // leaves with the normalisation (exactly: a power of two).
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int8_t c16 = (int8_t)(vm[e][j >> 2] >> (8 * (j & 3)));
            b4[e] = (short)(__float_as_uint((float)c16) >> 16);
          }
        } else if constexpr (kKind == 3) {
          // the e4m3fn value's fp32 pattern truncated to bf16 is exact (<= 4 significant bits)
#pragma unroll
          for (int e = 0; e < 4; ++e) b4[e] = (short)(__float_as_uint(fp8_value(r.vw[e][j >> 2], j & 3)) >> 16);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) b4[e] = (short)(r.vw[e][j >> 1] >> (16 * (j & 1)));
        }
        const V4 a = __builtin_bit_cast(V4, b4);
        acc[j] = M::run(a, phi, acc[j]);
        acc[j] = M::run(a, plo, acc[j]);
      }
  };

  // Register sets rotate: while one tile is computed the loads of the next kDepth - 1 tiles
  // are in flight (no copies between the sets).
  int32_t slot = 0;  // index in the window of the most recently loaded tile
  Raw ra, rb;
  int32_t tile = first_tile + wave;
  // Every call issues a tile's loads: a tile past the wave's range or on a missing page (its
  // keys masked) re-reads the wave's last valid tile (in bounds and just read; page 0 before
  // any) and is not computed.  With the loads under a branch, the register set was assigned
  // on one path only, and the copies that merged it waited for the loads just issued -- the
  // next tile's -- before the current tile was computed.
  int32_t safe_tl = first_tile + wave;
  int64_t safe_blk = 0;
  auto try_load = [&](Raw& r, int32_t tl) -> bool {
    const int64_t blk = __builtin_amdgcn_readlane(lane_blk, slot);
    const bool ok = tl < end_tile && blk >= 0 && blk < p.NB;  // wave-uniform
    if (ok) {
      safe_tl = tl;
      safe_blk = blk;
    }
    load_tile(r, safe_tl, safe_blk);
    return ok;
  };
  auto advance = [&]() {
    if (++slot == kWave) {
      win_base += 4 * kWave;
      refill();
      slot = 0;
    }
  };
  bool ok_a = try_load(ra, tile);
  if constexpr (kDepth == 3) {
    Raw rc;
    advance();
    bool ok_b = try_load(rb, tile + 4);
    while (tile < end_tile) {
      advance();
      const bool ok_c = try_load(rc, tile + 8);
      if (ok_a) compute_tile(ra, tile);
      tile += 4;
      if (tile >= end_tile) break;
      advance();
      ok_a = try_load(ra, tile + 8);
      if (ok_b) compute_tile(rb, tile);
      tile += 4;
      if (tile >= end_tile) break;
      advance();
      ok_b = try_load(rb, tile + 8);
      if (ok_c) compute_tile(rc, tile);
      tile += 4;
    }
  } else {
    while (tile < end_tile) {
      advance();
      const bool ok_b = try_load(rb, tile + 4);
      if (ok_a) compute_tile(ra, tile);
      tile += 4;
      if (tile >= end_tile) break;
      advance();
      ok_a = try_load(ra, tile + 4);
      if (ok_b) compute_tile(rb, tile);
      tile += 4;
    }
  }

  // ---- combine the four wavefronts: waves 1..3 leave (max, sum, accumulators) in LDS in
  // their lane layout, wave 0 merges them into its own registers lane by lane and writes
  const float lsum = col_sum(lpart);
  __shared__ float lds_m[4][16];
  __shared__ float lds_l[4][16];
  // lane-major partial rows, padded by one float: lane l's value k at l * (4 kDV + 1) + k, so
  // the 64 lanes of one store or load hit 64 different banks (a [col][channel] layout put the
  // 16 columns of a wavefront on one bank)
  constexpr int kRow = 4 * kDV + 1;
  __shared__ float lds_o[3][kWave * kRow];
  if (grp == 0) {
    lds_m[wave][col] = mrun;
    lds_l[wave][col] = lsum;
  }
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < kDV; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) lds_o[wave - 1][lane * kRow + e * kDV + j] = acc[j][e];
  }
  __syncthreads();
  if (wave != 0) return;
  float mx = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < 4; ++w) mx = fmaxf(mx, lds_m[w][col]);
  float f[4];
  float lt = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    f[w] = mx == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(lds_m[w][col] - mx);
    lt += lds_l[w][col] * f[w];
  }
  if (!qvalid) return;
  const bool direct = p.splits == 1;
  float lse_v;
  // int4 V operands carry 16 x the codes: the power-of-two factor is exact, so the outputs
  // are those of the codes themselves bit for bit
  const float inv = (direct ? finish(p, hq, mx, lt, &lse_v) : (lt > 0.0f ? 1.0f / lt : 0.0f)) *
                    (kInt4 ? 0.0625f : 1.0f);
  float* ws_row = p.ws + ((((i * p.Hkv + hk) * p.splits + split) * p.ncols + c) * (int64_t)(kD + 2));
  if (!direct && grp == 0) {
    ws_row[0] = mx;
    ws_row[1] = lt;
  }
  const int64_t orow = i * p.o_sb + qrow * p.o_ss + (int64_t)hq * p.o_sh;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int j = 0; j < kDV; ++j) {
      const int d = kDV * (4 * grp + e) + j;
      float o = acc[j][e] * f[0];
#pragma unroll
      for (int w = 1; w < 4; ++w) o += lds_o[w - 1][lane * kRow + e * kDV + j] * f[w];
      o *= inv;
      if (kQuant && p.smode == 2) o *= scale_at(p.vs, (int64_t)hk * kD + d, kSB);  // per-channel V
      if (direct) {
        store_out(p, orow + d, o);
      } else {
        ws_row[2 + d] = o;
      }
    }
  }
  if (direct && grp == 0 && p.lse) p.lse[i * p.lse_sb + qrow * p.lse_ss + (int64_t)hq * p.lse_sh] = lse_v;
}

// Merge the splits of one (query token, query head): one wavefront per row.  Lane s holds
// split s's (max, sum) and turns them into the split's weight sum_s * 2^(max_s - max), once;
// the output channels then read each split's row once, weighted through a lane broadcast.
__global__ __launch_bounds__(256) void attn_combine(AttnParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;  // (i * S + s) * Hq + hq
  if (row >= (int64_t)p.B * p.S * p.Hq) return;
  const int64_t it = row / p.Hq;
  const int hq = (int)(row - it * p.Hq);
  const int64_t i = it / p.S;
  const int tok = (int)(it - i * p.S);
  const Seq sq = seq_of(p, i);
  if (!token_valid(p, sq, tok)) return;
  const int hk = hq / p.g;
  const int c = tok * p.g + (hq - hk * p.g);
  const int64_t stride = (int64_t)p.ncols * (p.Dv + 2);
  const float* base = p.ws + ((i * p.Hkv + hk) * p.splits * (int64_t)p.ncols + c) * (p.Dv + 2);
  // splits past the sequence's keys wrote nothing (the main kernel returned early): the
  // non-empty splits are a prefix, of length `live`
  const Range r0 = token_range(p, sq, 0);
  int live = p.splits;
  if (p.split_tokens > 0) {
    const int64_t n = (sq.L - r0.begin + p.split_tokens - 1) / p.split_tokens;
    live = (int)(n < p.splits ? n : p.splits);
    if (live < 1 && p.splits > 0) live = r0.begin < sq.L ? 1 : 0;
  }
  // Every load is unconditional (split and channel indices clamped into this column's rows of
  // the workspace; an empty split's row is read and given weight 0), so the loads of a batch
  // issue together.  Under the per-split weight test each row load waited for the previous
  // one: up to 2 x live round trips per wavefront.
  const int last = live > 0 ? live - 1 : 0;
  const int64_t qrow = sq.row0 + tok;
  const int64_t orow = i * p.o_sb + qrow * p.o_ss + (int64_t)hq * p.o_sh;
  constexpr int kBatch = 8;
  if (live <= kWave) {  // wave-uniform; every launch of the torch op (at most 63 splits)
    // lane s holds split s's (max, sum), loaded once; the values in batches of kBatch splits
    const int sc = lane < live ? lane : last;
    const float m_raw = base[sc * stride], l_raw = base[sc * stride + 1];
    const float m = lane < live ? m_raw : -__builtin_inff();
    float mx = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    const float wgt = m != -__builtin_inff() ? l_raw * __builtin_amdgcn_exp2f(m - mx) : 0.0f;
    float lt = wgt;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) lt += __shfl_xor(lt, o, kWave);
    float lse_v;
    const float inv = finish(p, hq, mx, lt, &lse_v);
    for (int d0 = 0; d0 < p.Dv; d0 += kWave) {
      const int d = d0 + lane;
      const int dc = d < p.Dv ? d : p.Dv - 1;
      float o = 0.0f;
      for (int k0 = 0; k0 < live; k0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = base[(k0 + k < live ? k0 + k : last) * stride + 2 + dc];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const float wk = __shfl(wgt, k0 + k < live ? k0 + k : 0, kWave);
          if (k0 + k < live && wk != 0.0f) o += v[k] * wk;
        }
      }
      if (d < p.Dv) store_out(p, orow + d, o * inv);
    }
    if (lane == 0 && p.lse) p.lse[i * p.lse_sb + qrow * p.lse_ss + (int64_t)hq * p.lse_sh] = lse_v;
    return;
  }
  float mx = -__builtin_inff();
  for (int s0 = 0; s0 < live; s0 += kWave) {
    const int s = s0 + lane;
    const float m = base[(s < live ? s : last) * stride];
    mx = fmaxf(mx, s < live ? m : -__builtin_inff());
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  float lt = 0.0f;
  for (int s0 = 0; s0 < live; s0 += kWave) {
    const int s = s0 + lane;
    const int sc = s < live ? s : last;
    const float m = s < live ? base[sc * stride] : -__builtin_inff();
    const float l = base[sc * stride + 1];
    lt += m != -__builtin_inff() ? l * __builtin_amdgcn_exp2f(m - mx) : 0.0f;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lt += __shfl_xor(lt, o, kWave);
  float lse_v;
  const float inv = finish(p, hq, mx, lt, &lse_v);
  for (int d0 = 0; d0 < p.Dv; d0 += kWave) {
    const int d = d0 + lane;
    const int dc = d < p.Dv ? d : p.Dv - 1;
    float o = 0.0f;
    for (int s0 = 0; s0 < live; s0 += kWave) {
      const int sl = s0 + lane;
      const int sc = sl < live ? sl : last;
      const float m = sl < live ? base[sc * stride] : -__builtin_inff();
      const float wgt = m != -__builtin_inff() ? base[sc * stride + 1] * __builtin_amdgcn_exp2f(m - mx) : 0.0f;
      const int n = live - s0 < kWave ? live - s0 : kWave;
      for (int k0 = 0; k0 < n; k0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const int s = s0 + (k0 + k < n ? k0 + k : n - 1);
          v[k] = base[s * stride + 2 + dc];
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const float wk = __shfl(wgt, k0 + k < n ? k0 + k : 0, kWave);
          if (k0 + k < n && wk != 0.0f) o += v[k] * wk;
        }
      }
    }
    if (d < p.Dv) store_out(p, orow + d, o * inv);
  }
  if (lane == 0 && p.lse) p.lse[i * p.lse_sb + qrow * p.lse_ss + (int64_t)hq * p.lse_sh] = lse_v;
}

// ------------------------------------------------------------------------------ generic kernel

__device__ __forceinline__ float plain_value(const void* base, int64_t e, int cache_dtype) {
  switch (cache_dtype) {
    case TMO_DTYPE_BF16: return load1(BF16{}, base, e);
    case TMO_DTYPE_F16: return load1(F16{}, base, e);
    default: return load1(F32{}, base, e);
  }
}

// Code e of a quantised cache as fp32: an int8 code, or a float8_e4m3fn value.
__device__ __forceinline__ float code_value(const void* base, int64_t e, int cache_dtype) {
  if (cache_dtype == TMO_DTYPE_I8) return (float)static_cast<const int8_t*>(base)[e];
  return fp8_value(static_cast<const uint8_t*>(base)[e], 0);
}

// Signed 4-bit code `odd` of byte e of an int4-pair cache: the even element of a pair in the
// high nibble, the odd one in the low nibble, sign-extended.
__device__ __forceinline__ float nibble_value(const void* base, int64_t e, int odd) {
  const int32_t b = static_cast<const int8_t*>(base)[e];
  return (float)(odd ? (int32_t)((uint32_t)b << 28) >> 28 : b >> 4);
}

__device__ __forceinline__ bool quant_cache(int cache_dtype) {
  return cache_dtype == TMO_DTYPE_I8 || cache_dtype == TMO_DTYPE_F8E4M3 ||
         cache_dtype == TMO_DTYPE_I4;
}

// Key channel d of row `row` of page blk, KV head hk.
__device__ __forceinline__ float key_value(const AttnParams& p, int64_t blk, int hk, int64_t row,
                                           int d, int cache_dtype) {
  const int64_t r = (blk * p.Hkv + hk) * p.BS + row;
  if (!quant_cache(cache_dtype)) return plain_value(p.kc, r * p.k_row + d, cache_dtype);
  // int4: K pairs adjacent channels, k_row bytes per row
  const float code = cache_dtype == TMO_DTYPE_I4 ? nibble_value(p.kc, r * p.k_row + (d >> 1), d & 1)
                                                 : code_value(p.kc, r * p.k_row + d, cache_dtype);
  switch (p.smode) {
    case 1: return code * scale_at(p.ks, blk * p.ks_sb + hk * p.ks_sh + row, p.s_bf16);
    case 2: return code * scale_at(p.ks, (int64_t)hk * p.D + d, p.s_bf16);
    default: return code * scale_at(p.ks, r * (p.D >> 5) + (d >> 5), p.s_bf16);
  }
}

// Value channel d: per-group V scales hold one number per 32 rows of a page and channel.
__device__ __forceinline__ float value_value(const AttnParams& p, int64_t blk, int hk, int64_t row,
                                             int d, int cache_dtype) {
  const int64_t r = (blk * p.Hkv + hk) * p.BS + row;
  if (!quant_cache(cache_dtype)) return plain_value(p.vc, r * p.v_row + d, cache_dtype);
  float code;
  if (cache_dtype != TMO_DTYPE_I4)
    code = code_value(p.vc, r * p.v_row + d, cache_dtype);
  else if (p.v_ch)  // int4, V pairing channels: as K
    code = nibble_value(p.vc, r * p.v_row + (d >> 1), d & 1);
  else  // int4, V pairing the rows of a page: [NB, Hkv, BS / 2, v_row]
    code = nibble_value(p.vc, ((blk * p.Hkv + hk) * (p.BS >> 1) + (row >> 1)) * p.v_row + d,
                        (int)(row & 1));
  switch (p.smode) {
    case 1: return code * scale_at(p.vs, blk * p.vs_sb + hk * p.vs_sh + row, p.s_bf16);
    case 2: return code * scale_at(p.vs, (int64_t)hk * p.Dv + d, p.s_bf16);
    default:
      return code * scale_at(p.vs, ((blk * p.Hkv + hk) * (p.BS >> 5) + (row >> 5)) * p.Dv + d,
                             p.s_bf16);
  }
}

// One wavefront per (query token, query head): 64 keys at a time, one per lane (a lane
// computes its key's full dot product), then every lane accumulates its channels over the 64
// keys.  Value head sizes up to 512 (8 accumulators per lane); any key head size.
__global__ __launch_bounds__(256) void attn_generic(AttnParams p) {
  const int cache_dtype = p.c_dtype;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;  // (i * S + s) * Hq + hq
  if (row >= (int64_t)p.B * p.S * p.Hq) return;
  const int64_t it = row / p.Hq;
  const int hq = (int)(row - it * p.Hq);
  const int64_t i = it / p.S;
  const int64_t tok = it - i * p.S;
  const Seq sq = seq_of(p, i);
  if (!token_valid(p, sq, tok)) return;
  const int hk = hq / p.g;
  // keys [jb, je) of the token at position P
  const int64_t P = sq.L - sq.nq + tok;
  const int64_t je = P + 1 < sq.L ? P + 1 : sq.L;
  const int64_t jb = p.window >= 0 && P - p.window > 0 ? P - p.window : 0;
  const float alibi = p.alibi ? p.alibi[i * p.Hq + hq] * kLog2e : 0.0f;
  float mrun = -__builtin_inff(), l = 0.0f;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
  const int64_t qrow = sq.row0 + tok;
  const int64_t qe = i * p.q_sb + qrow * p.q_ss + (int64_t)hq * p.q_sh;
  const int64_t qse = i * p.qs_sb + qrow * p.qs_ss + (int64_t)hq * p.qs_sh;  // quantised q
  const float q_rs = p.qs_mode ? q_row_scale(p, qse) : 1.0f;
  const int32_t* btr = bt_row_of(p, i, hq, hk);
  for (int64_t j0 = jb; j0 < je; j0 += kWave) {
    const int64_t j = j0 + lane;
    float s = -__builtin_inff();
    int blk = -1, r = 0;
    if (j < je) {
      blk = btr[j / p.BS];
      r = (int)(j % p.BS);
      if (blk >= 0 && blk < p.NB) {
        float dot = 0.0f;
        for (int d = 0; d < p.D; ++d)
          dot += load_q(p, qe + d) * q_group_scale(p, qse, d) *
                 key_value(p, blk, hk, r, d, cache_dtype);
        s = dot * q_rs * p.scale_log2;
        if (p.alibi) s += alibi * (float)(j - P);
        if (p.mask && j >= sq.L - p.mask_len)
          s += mask_value(p, i * p.m_sb + tok * p.m_ss + (j - (sq.L - p.mask_len))) * kLog2e;
      } else {
        blk = -1;
      }
    }
    float tmax = s;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, kWave));
    const float mnew = fmaxf(mrun, tmax);
    if (mnew == -__builtin_inff()) continue;
    const float corr = __builtin_amdgcn_exp2f(mrun - mnew);
    mrun = mnew;
    const float pj = __builtin_amdgcn_exp2f(s - mnew);
    float ps = pj;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ps += __shfl_xor(ps, o, kWave);
    l = l * corr + ps;
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] *= corr;
    for (int t = 0; t < kWave; ++t) {
      const float pt = __shfl(pj, t, kWave);
      const int bt_ = __shfl(blk, t, kWave);
      const int rt = __shfl(r, t, kWave);
      if (pt == 0.0f || bt_ < 0) continue;  // the same in every lane
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int d = lane + u * kWave;
        if (d < p.Dv) acc[u] += pt * value_value(p, bt_, hk, rt, d, cache_dtype);
      }
    }
  }
  float lse_v;
  const float inv = finish(p, hq, mrun, l, &lse_v);
  const int64_t orow = i * p.o_sb + qrow * p.o_ss + (int64_t)hq * p.o_sh;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int d = lane + u * kWave;
    if (d < p.Dv) store_out(p, orow + d, p.sink ? acc[u] * inv : (l > 0.0f ? acc[u] / l : 0.0f));
  }
  if (lane == 0 && p.lse) p.lse[i * p.lse_sb + qrow * p.lse_ss + (int64_t)hq * p.lse_sh] = lse_v;
}

// ------------------------------------------------------------------------------ launch

template <int kD, int kKind, bool kSB>
int launch_mfma_d(const AttnParams& p, bool qlo, hipStream_t st) {
  const dim3 grid((unsigned)(p.splits * p.ncb), (unsigned)p.Hkv, (unsigned)p.B), block(256);
  int rc;
  if (p.mask)
    rc = qlo ? launch_kernel(attn_mfma<kD, kKind, true, kSB, true>, grid, block, st, p)
             : launch_kernel(attn_mfma<kD, kKind, false, kSB, true>, grid, block, st, p);
  else
    rc = qlo ? launch_kernel(attn_mfma<kD, kKind, true, kSB, false>, grid, block, st, p)
             : launch_kernel(attn_mfma<kD, kKind, false, kSB, false>, grid, block, st, p);
  if (rc != TMO_OK || p.splits == 1) return rc;
  const int64_t rows = (int64_t)p.B * p.S * p.Hq;
  return launch_kernel(attn_combine, dim3((unsigned)((rows + 3) / 4)), block, st, p);
}

template <int kKind, bool kSB>
int launch_mfma(const AttnParams& p, bool qlo, hipStream_t st) {
  switch (p.D) {
    case 64: return launch_mfma_d<64, kKind, kSB>(p, qlo, st);
    case 128: return launch_mfma_d<128, kKind, kSB>(p, qlo, st);
    default: return launch_mfma_d<256, kKind, kSB>(p, qlo, st);
  }
}

}  // namespace
}  // namespace tmo

using namespace tmo;

extern "C" int64_t tmo_hip_cached_kv_attn_workspace_bytes(int64_t batch, int64_t num_kv_heads,
                                                          int64_t num_q_heads,
                                                          int64_t head_size_v, int64_t seq_q,
                                                          int64_t splits) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || head_size_v <= 0 || seq_q <= 0 ||
      splits <= 1)
    return 0;
  return batch * num_kv_heads * splits * seq_q * (num_q_heads / num_kv_heads) *
         (head_size_v + 2) * (int64_t)sizeof(float);
}

extern "C" int64_t tmo_hip_attn_workspace_bytes(int64_t batch, int64_t num_kv_heads,
                                                int64_t num_q_heads, int64_t head_size,
                                                int64_t max_context_len, int64_t splits) {
  (void)max_context_len;
  return tmo_hip_cached_kv_attn_workspace_bytes(batch, num_kv_heads, num_q_heads, head_size, 1,
                                                splits);
}

extern "C" int tmo_hip_cached_kv_attn(
    const void* q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    const void* q_scale, int q_scale_mode, int q_scale_dtype, int64_t q_scale_stride_batch,
    int64_t q_scale_stride_token, int64_t q_scale_stride_head, int64_t q_scale_groups,
    const int32_t* cu_seq_q, int64_t seq_q, int64_t total_q, const void* k_cache,
    const void* v_cache, int64_t k_cache_dim, int64_t v_cache_dim, const void* k_scale,
    const void* v_scale, int scale_mode, int scale_dtype, int64_t k_scale_stride_block,
    int64_t k_scale_stride_head, int64_t v_scale_stride_block, int64_t v_scale_stride_head,
    const int32_t* block_tables, int64_t max_blocks, int64_t block_table_heads,
    const int32_t* context_lens, const float* alibi_slopes, const float* sink, const void* mask,
    int mask_dtype,
    int64_t mask_len, int64_t mask_stride_batch, int64_t mask_stride_token, void* out,
    int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head, float* lse,
    int64_t lse_stride_batch, int64_t lse_stride_token, int64_t lse_stride_head, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
    int64_t num_blocks, int64_t block_size, int64_t max_context_len, int64_t window_left,
    float softmax_scale, int q_dtype, int cache_dtype, int v_pair_channels, int out_dtype,
    int64_t splits, void* workspace, int64_t workspace_bytes, void* stream) {
  // q: floats (the output of q's dtype), or int8 / float8_e4m3fn codes with q_scale (the
  // output of out_dtype) over quantised caches
  const bool qquant = q_dtype == TMO_DTYPE_I8 || q_dtype == TMO_DTYPE_F8E4M3;
  if (q_dtype != TMO_DTYPE_BF16 && q_dtype != TMO_DTYPE_F16 && q_dtype != TMO_DTYPE_F32 && !qquant)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (out_dtype != TMO_DTYPE_BF16 && out_dtype != TMO_DTYPE_F16 && out_dtype != TMO_DTYPE_F32)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (!qquant && out_dtype != q_dtype) return TMO_ERR_UNSUPPORTED_DTYPE;
  if (qquant) {
    if (q_scale_mode < 1 || q_scale_mode > 3) return TMO_ERR_UNSUPPORTED_MODE;
    if (q_scale_dtype != TMO_DTYPE_F32 && q_scale_dtype != TMO_DTYPE_BF16)
      return TMO_ERR_UNSUPPORTED_DTYPE;
    if (!q_scale || q_scale_stride_batch < 0 || q_scale_stride_token < 0 ||
        q_scale_stride_head < 0 ||
        (q_scale_mode == 3 && (q_scale_groups <= 0 || head_size % q_scale_groups != 0)))
      return TMO_ERR_INVALID_ARGUMENT;
  }
  if (block_table_heads != 0 && block_table_heads != num_kv_heads &&
      block_table_heads != num_q_heads)
    return TMO_ERR_INVALID_ARGUMENT;
  // quantised caches: int8 codes, float8_e4m3fn values or int4 pairs, times fp32 or bf16 scales
  const bool int4 = cache_dtype == TMO_DTYPE_I4;
  const bool quant = cache_dtype == TMO_DTYPE_I8 || cache_dtype == TMO_DTYPE_F8E4M3 || int4;
  if (!quant && cache_dtype != q_dtype) return TMO_ERR_UNSUPPORTED_DTYPE;  // quantised q: quantised caches
  if (mask && mask_dtype != TMO_DTYPE_F32 && mask_dtype != TMO_DTYPE_F16 &&
      mask_dtype != TMO_DTYPE_BF16)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (mask && (mask_len <= 0 || mask_len > 0x7fffffffLL || mask_stride_batch < 0 ||
               mask_stride_token < 0))
    return TMO_ERR_INVALID_ARGUMENT;
  if (quant && scale_dtype != TMO_DTYPE_F32 && scale_dtype != TMO_DTYPE_BF16)
    return TMO_ERR_UNSUPPORTED_DTYPE;
  if (quant && (scale_mode < 1 || scale_mode > 3)) return TMO_ERR_UNSUPPORTED_MODE;
  // An empty cache (num_blocks 0: every block-table entry is outside it, so every key is
  // masked) may come with null cache and per-token scale pointers; nothing reads them.
  // Likewise an empty block table (max_blocks 0 caps every context at 0 keys).
  if (!q || !context_lens || !out) return TMO_ERR_INVALID_ARGUMENT;
  if ((num_blocks > 0 && !k_cache) || (max_blocks > 0 && !block_tables))
    return TMO_ERR_INVALID_ARGUMENT;
  if (quant && (!k_scale || !v_scale) && (num_blocks > 0 || scale_mode != 1))
    return TMO_ERR_INVALID_ARGUMENT;
  // v_cache null: the values are the first head_size_v channels of the K cache's rows (not
  // for int4 pairs, whose K and V caches pair different axes: null only with an empty cache)
  const bool v_null = !v_cache;
  if (!v_cache) {
    if (int4 && num_blocks > 0) return TMO_ERR_INVALID_ARGUMENT;
    v_cache = k_cache;
    v_cache_dim = k_cache_dim;
  }
  // max_context_len <= 0: "an uncertain maximum value of context_lens" (reference _ops.py,
  // single_query_cached_kv_attn's max_context_len); it only sizes the splits, so a negative
  // value is taken as 0 (the last split always runs to the sequence's own length)
  if (max_context_len < 0) max_context_len = 0;
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      head_size <= 0 || head_size > 4096 || head_size_v <= 0 || head_size_v > 512 ||
      num_blocks < 0 ||
      block_size <= 0 || max_blocks < 0 || splits < 1 || seq_q < 0 || q_stride_batch < 0 ||
      q_stride_token < 0 || q_stride_head < 0 || out_stride_batch < 0 || out_stride_token < 0 ||
      out_stride_head < 0 || (cu_seq_q && total_q < 0))
    return TMO_ERR_INVALID_ARGUMENT;
  if (quant && scale_mode == 1 &&
      (k_scale_stride_block < 0 || k_scale_stride_head < 0 || v_scale_stride_block < 0 ||
       v_scale_stride_head < 0))
    return TMO_ERR_INVALID_ARGUMENT;
  if (quant && scale_mode == 3 && (head_size % 32 != 0 || block_size % 32 != 0))
    return TMO_ERR_INVALID_ARGUMENT;
  // cache rows: elements, or bytes of int4 pairs (K: head_size / 2 channel pairs; V: pairs of
  // rows -- [num_blocks, Hkv, block_size / 2, v_cache_dim], block_size even -- or of channels)
  if (!int4 ? (k_cache_dim < head_size || v_cache_dim < head_size_v)
            : (2 * k_cache_dim < head_size ||
               (!v_null && (v_pair_channels ? 2 * v_cache_dim < head_size_v
                                            : (v_cache_dim < head_size_v || block_size % 2 != 0)))))
    return TMO_ERR_INVALID_ARGUMENT;
  const int64_t g = num_q_heads / num_kv_heads;
  if (batch > 65535 || num_kv_heads > 65535 || splits > 65535 || num_q_heads > 0x7fffffffLL ||
      seq_q > 0x7fffffffLL / num_q_heads)
    return TMO_ERR_INVALID_ARGUMENT;
  const int64_t ncb = (seq_q * g + 15) / 16;
  if (splits * ncb > 0x7fffffffLL || (batch * seq_q * num_q_heads + 3) / 4 > 0x7fffffffLL)
    return TMO_ERR_INVALID_ARGUMENT;
  if (splits > 1 && (!workspace ||
                     workspace_bytes < tmo_hip_cached_kv_attn_workspace_bytes(
                                           batch, num_kv_heads, num_q_heads, head_size_v, seq_q,
                                           splits)))
    return TMO_ERR_INVALID_ARGUMENT;
  if (batch == 0 || seq_q == 0) return TMO_OK;

  AttnParams p{};
  p.q = q;
  p.q_sb = cu_seq_q ? 0 : q_stride_batch;
  p.q_ss = q_stride_token;
  p.q_sh = q_stride_head;
  p.cu = cu_seq_q;
  p.S = (int32_t)seq_q;
  p.ncols = (int32_t)(seq_q * g);
  p.ncb = (int32_t)ncb;
  p.total_q = cu_seq_q ? total_q : batch * seq_q;
  p.sink = sink;
  p.kc = k_cache;
  p.vc = v_cache;
  p.k_row = k_cache_dim;
  p.v_row = v_cache_dim;
  p.ks = k_scale;
  p.vs = v_scale;
  p.smode = quant ? scale_mode : 0;
  p.s_bf16 = quant && scale_dtype == TMO_DTYPE_BF16;
  p.ks_sb = k_scale_stride_block;
  p.ks_sh = k_scale_stride_head;
  p.vs_sb = v_scale_stride_block;
  p.vs_sh = v_scale_stride_head;
  p.bt = block_tables;
  p.max_blocks = max_blocks;
  p.lens = context_lens;
  p.alibi = alibi_slopes;
  p.window = window_left;
  p.scale_log2 = softmax_scale * kLog2e;
  p.out = out;
  p.o_sb = cu_seq_q ? 0 : out_stride_batch;
  p.o_ss = out_stride_token;
  p.o_sh = out_stride_head;
  p.lse = lse;
  p.lse_sb = cu_seq_q ? 0 : lse_stride_batch;
  p.lse_ss = lse_stride_token;
  p.lse_sh = lse_stride_head;
  p.B = (int32_t)batch;
  p.Hq = (int32_t)num_q_heads;
  p.Hkv = (int32_t)num_kv_heads;
  p.g = (int32_t)g;
  p.D = (int32_t)head_size;
  p.Dv = (int32_t)head_size_v;
  p.BS = (int32_t)block_size;
  p.bs_shift = ilog2_if_pow2(block_size);
  p.NB = num_blocks;
  p.q_dtype = q_dtype;
  p.o_dtype = out_dtype;
  p.qs = qquant ? q_scale : nullptr;
  p.qs_mode = qquant ? q_scale_mode : 0;
  p.qs_bf16 = qquant && q_scale_dtype == TMO_DTYPE_BF16;
  p.qs_sb = cu_seq_q ? 0 : q_scale_stride_batch;
  p.qs_ss = q_scale_stride_token;
  p.qs_sh = q_scale_stride_head;
  p.qs_group = qquant && q_scale_mode == 3 ? (int32_t)(head_size / q_scale_groups) : 1;
  p.bt_heads = block_table_heads;
  p.q_vec = (q_dtype == TMO_DTYPE_BF16 || q_dtype == TMO_DTYPE_F16) &&
            reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
            p.q_sb % 8 == 0 && q_stride_token % 8 == 0 && q_stride_head % 8 == 0 &&
            (!quant || scale_mode != 2 || reinterpret_cast<uintptr_t>(k_scale) % 16 == 0);
  p.ws = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);

  // MFMA path eligibility: one head size for K and V that is also both caches' row length,
  // page rows in whole 16-token tiles, 16-byte aligned rows and scale vectors (per-token scale
  // offsets of a page and head in multiples of four), q's dtype representable by the operands
  // (quantised caches: f16 with a lo part when needed), per-token or per-channel scales.
  auto al = [](const void* x, int a) { return reinterpret_cast<uintptr_t>(x) % a == 0; };
  // The MFMA kernel always issues its tile loads (a wave with no valid page yet reads page 0,
  // see attn_mfma), so an empty cache takes attn_generic, whose loads are all under the page
  // check: every output row is then 0 and its lse -inf (nothing to attend to).
  // int4 pages: K rows of head_size / 2 bytes, V pairing rows (pair rows of head_size bytes)
  bool mfma = num_blocks > 0 && (head_size == 64 || head_size == 128 || head_size == 256) &&
              head_size_v == head_size &&
              k_cache_dim == (int4 ? head_size / 2 : head_size) && v_cache_dim == head_size &&
              !(int4 && v_pair_channels) && block_size % 16 == 0 && al(k_cache, 16) &&
              al(v_cache, 16) && q_dtype != TMO_DTYPE_F32 &&
              (block_table_heads != num_q_heads || num_q_heads == num_kv_heads);
  if (quant)
    mfma = mfma && scale_mode != 3 &&
           (scale_mode != 1 ||
            (al(k_scale, p.s_bf16 ? 8 : 16) && al(v_scale, p.s_bf16 ? 8 : 16) &&
             k_scale_stride_block % 4 == 0 &&
             k_scale_stride_head % 4 == 0 && v_scale_stride_block % 4 == 0 &&
             v_scale_stride_head % 4 == 0));
  p.c_dtype = cache_dtype;
  p.v_ch = int4 && v_pair_channels;
  p.mask = mask;
  p.mask_dtype = mask_dtype;
  p.mask_len = (int32_t)mask_len;
  p.m_sb = mask_stride_batch;
  p.m_ss = mask_stride_token;
  if (!mfma) {
    p.splits = 1;
    p.split_tokens = 1;
    const int64_t rows = batch * seq_q * num_q_heads;
    return launch_kernel(attn_generic, dim3((unsigned)((rows + 3) / 4)), dim3(256), st, p);
  }
  p.splits = (int32_t)splits;
  // tokens per split: the context divided evenly, rounded up to whole 64-token steps (four
  // wavefronts x 16-token tiles)
  int64_t per = (max_context_len + splits - 1) / splits;
  per = (per + 63) / 64 * 64;
  p.split_tokens = per > 0 ? per : 64;
  // quantised caches: bf16 and f16 q, and int8 / float8_e4m3fn q codes, are exact f16 operands
  // after the power-of-two scaling; q folded with per-channel key scales or group-wise q
  // scales needs the lo operand
  const bool qlo = scale_mode == 2 || p.qs_mode == 3;
  if (cache_dtype == TMO_DTYPE_I8)
    return p.s_bf16 ? launch_mfma<0, true>(p, qlo, st) : launch_mfma<0, false>(p, qlo, st);
  if (cache_dtype == TMO_DTYPE_F8E4M3)
    return p.s_bf16 ? launch_mfma<3, true>(p, qlo, st) : launch_mfma<3, false>(p, qlo, st);
  if (int4)
    return p.s_bf16 ? launch_mfma<4, true>(p, qlo, st) : launch_mfma<4, false>(p, qlo, st);
  if (cache_dtype == TMO_DTYPE_BF16) return launch_mfma<1, false>(p, false, st);
  return launch_mfma<2, false>(p, false, st);
}

extern "C" int tmo_hip_single_query_cached_kv_attn(
    const void* q, int64_t q_stride_seq, int64_t q_stride_head, const void* k_cache,
    const void* v_cache, const float* k_scale, const float* v_scale, int scale_mode,
    const int32_t* block_tables, int64_t max_blocks, const int32_t* context_lens,
    const float* alibi_slopes, void* out, int64_t out_stride_seq, int64_t out_stride_head,
    float* lse, int64_t lse_stride_seq, int64_t lse_stride_head, int64_t batch,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_size, int64_t num_blocks,
    int64_t block_size, int64_t max_context_len, int64_t window_left, float softmax_scale,
    int q_dtype, int cache_dtype, int64_t splits, void* workspace, int64_t workspace_bytes,
    void* stream) {
  if ((cache_dtype == TMO_DTYPE_I8 || cache_dtype == TMO_DTYPE_F8E4M3) && scale_mode == 3)
    return TMO_ERR_UNSUPPORTED_MODE;
  if (!v_cache && num_blocks > 0) return TMO_ERR_INVALID_ARGUMENT;
  if (head_size > 512) return TMO_ERR_INVALID_ARGUMENT;
  // contiguous per-token scales [num_blocks, Hkv, block_size]
  const int64_t sb = num_kv_heads * block_size, sh = block_size;
  if (cache_dtype == TMO_DTYPE_I4) return TMO_ERR_UNSUPPORTED_DTYPE;
  if (q_dtype == TMO_DTYPE_I8 || q_dtype == TMO_DTYPE_F8E4M3) return TMO_ERR_UNSUPPORTED_DTYPE;
  return tmo_hip_cached_kv_attn(
      q, q_stride_seq, 0, q_stride_head, nullptr, 0, TMO_DTYPE_F32, 0, 0, 0, 0, nullptr, 1, 0,
      k_cache, v_cache, head_size, head_size, k_scale, v_scale, scale_mode, TMO_DTYPE_F32, sb,
      sh, sb, sh, block_tables, max_blocks, 0, context_lens, alibi_slopes, nullptr, nullptr, 0,
      0, 0, 0, out, out_stride_seq, 0, out_stride_head, lse, lse_stride_seq, 0,
      lse_stride_head, batch, num_q_heads, num_kv_heads, head_size, head_size, num_blocks,
      block_size, max_context_len, window_left, softmax_scale, q_dtype, cache_dtype, 0, q_dtype,
      splits, workspace, workspace_bytes, stream);
}
