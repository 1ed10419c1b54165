/*
 * tmo_oracle.c -- CPU restatement of torch_mlu_ops' quantized paged-KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels and the
 * CPU baseline timed by bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  The product path (domesticated_torch_mlu_ops_amd) never
 * links, loads or calls it, and has no CPU fallback.
 *
 * The reference ships no kernels and no CPU implementation: its arithmetic is specified
 * only by the docstring "Math" blocks of /root/reference/_ops.py, cited per function
 * below.  Where those blocks are ambiguous this file fixes one reading:
 *
 *   D1  arithmetic in fp32: scale = RN(fp32(amax) / 127.0f) (IEEE divide), and
 *       code = RNE(RN(fp32(x) / scale)) with a true IEEE divide per element
 *       (_ops.py:1532-1533, 3171-3172).
 *   D2  codes are clamped to [-128, 127] (_ops.py:1535, 3172).
 *   D3  an all-zero row gives scale 0 and codes 0 (the literal math divides 0/0).
 *   D4  slot < 0 writes neither codes nor scale (_ops.py:1264, 1656, 6400-6401); a slot
 *       >= num_blocks*block_size is treated the same way (undefined in the reference).
 *   D5  NaN / Inf inputs are outside the contract.
 *   D6  dequant = RNE_out(fp32(code) * scale)   (cast order of _ops.py:3677).
 *   D7  smoothed = RN(fp32(x) * smooth), materialised before amax and divide (no FMA).
 *   D8  int8 codes for the dynamic ops.
 *   D10 fused_rope (rmsnorm mode) in fp32 with one final rounding: the sum of squares of a
 *       row is taken over chunks of 8 consecutive elements (each chunk summed in order, every
 *       product and sum rounded), then over the chunk sums as a balanced binary tree in
 *       natural order (padded with zeros to a power of two); inv = RN(1 / RN(sqrt(RN(RN(ss/D)
 *       + eps)))); y = RN(RN(x * inv) * gamma); rope (fold) out = RN(RN(rot * sin) +
 *       RN(y * cos)) with rot = (-y2, y1) over [off, off + rope_dim) (a position outside the
 *       table's rows leaves the row unrotated -- undefined in the reference); K is quantised (or
 *       rounded) from the fp32 result, V from its input values (_ops.py:3493-3520,
 *       6356-6423; rotary math _ops.py:1116-1127).
 *   D13 fused_rope, norm_type "layernorm" (_ops.py:3501-3504): Q and K are rotated (D10's rope
 *       on the raw fp32 row), then K alone is layer-normalised in fp32, two passes over the
 *       D10 chunk order: mean = RN(s1 / D) with s1 the chunked sum of the rotated row;
 *       d = RN(x - mean); var = RN(s2 / D) with s2 the chunked sum of RN(d * d) (biased, as
 *       torch's layer_norm); inv = RN(1 / RN(sqrt(RN(var + eps)))); y = RN(RN(d * inv) *
 *       gamma), then RN(y + beta) when beta is given.  q_gamma is not used.
 *   D14 fused_rope with linear caches [max_batch, kv_heads, cache_len, head_size]
 *       (cache_bs_id_hp / cache_seq_offsets_hp, _ops.py:3469-3601 "reshape_linear_cache"
 *       branch): token s of sequence b is stored at cache batch cache_bs_id[b] (b when absent),
 *       position cache_seq_offsets[b] + s (s when absent), and not at all when the batch or the
 *       position is outside the cache; dynamic scales [max_batch, kv_heads, cache_len].  The
 *       layout equals the paged one with cache_len-row pages, one per cache batch: the Python
 *       wrapper (fused_rope_linear) maps each token to that slot and runs this function.
 *   D11 linear caches [max_batch, H, cache_len, D] (_ops.py:1189-1249, 1708-1919, 3642-3732,
 *       3898-3969): sequence i covers len_i tokens -- cu[i+1] - cu[i] when the input is
 *       packed (context_lengths holds batch + 1 prefix offsets), else context_lengths[i]; its
 *       token j is input row start_i + j (start_i = context_seq_offset[i], else cu[i] when
 *       packed, else i * seqlen for padded [batch, seqlen, H, D] input) or output row
 *       start_i + j (start_i = context_seq_offset[i], else the exclusive prefix sum of the
 *       lengths); it lives in cache batch cache_bs_id[i] (else i; negative: the sequence is
 *       skipped) at position cache_seq_offset[i] + j (else j); reshape_from_cache's block
 *       table [batch, max_blocks] instead maps position p to row p % block_size of block
 *       block_tables[i, p / block_size] (a one-column table is the linear layout with the
 *       table naming the cache batch, _ops.py:3906-3915).  Rows whose cache batch or
 *       position falls outside the cache, or whose input / output row falls outside its
 *       tensor, are skipped, as are tokens j >= max_context_len.  Per-head static scales
 *       [H, cache_len] are indexed by cache position.  The dynamic quantiser works per token
 *       or per group of D / group_num channels (scale [max_batch, H, cache_len, group_num]):
 *       int8 as D1-D3, fp8 e4m3fn with scale = RN(amax / 448), codes e4m3fn_RNE(clip(RN(x /
 *       scale), -448, 448)) and an all-zero group giving scale 0 and codes 0 (_ops.py:1728-1745).
 *   D12 single_query_cached_kv_attn (_ops.py:777-900): the docstring math in double with
 *       k = code * scale exact (code: an int8, or a float8_e4m3fn value, _ops.py:868).  A sequence's nq query tokens (q [batch, seq_q, ...] or rows
 *       cu_seq_q[i] .. cu_seq_q[i+1] - 1 of a [total_q, ...] q, _ops.py:824, 860-861) are its
 *       last nq positions: token s sits at position P = L - nq + s and sees keys j <= P
 *       (causal within the new tokens; one token: P = L - 1), and with a left window keys
 *       j >= P - window_left; alibi adds slope * (j - P) (key position relative to the
 *       query, the usual decode form; create_alibi is not defined in the reference); the
 *       sink (_ops.py:864, one logit per query head) joins the softmax denominator only:
 *       out = sum_j e^(s_j) v_j / (sum_j e^(s_j) + e^sink); lse = log of that denominator
 *       (the docstring writes logsumexp(qk), which equals it without alibi and sink); a key
 *       on a page outside [0, NB) is masked; no key and no sink gives out 0, lse -inf.
 *       Keys are the first head_size_qk channels of a K cache row, values the first
 *       head_size_v of a V cache row -- of the K row itself when v_cache is None
 *       (_ops.py:828-831); per-group scales (_ops.py:841-842) cover 32 channels of one key
 *       (K) or 32 rows of one page and channel (V: block_size // 32 per page).
 *   D15 4-bit linear caches (quant_to_linear_cache / dequant_from_linear_cache with quant_bit
 *       4, _ops.py:1723-1750, 3664-3700): int8 caches hold two signed 4-bit codes per byte.
 *       Codes: scale = RN(amax / 7) (int_max = 2^(4-1) - 1), code = clip(RNE(RN(x / scale)),
 *       -8, 7), an all-zero row or group giving scale 0 and codes 0.  Nibble order: the even
 *       element of a pair in the high nibble, the odd one in the low nibble -- the dequant
 *       math's `unpack[0::2] = byte >> 4; unpack[1::2] = byte << 4 >> 4` (arithmetic shifts
 *       of int8), which the quant math's `(d1 << 4) + (d0 & 0x0f)` also gives when its
 *       repeated `[0::2]` is read as d1 = even, d0 = odd elements.  K pairs adjacent
 *       channels: key_cache [max_batch, H, cache_len, D / 2], byte c of a row = (code[2c],
 *       code[2c + 1]).  V pairs adjacent cache positions (value_cache [max_batch, H,
 *       cache_len / 2, D], the dequant docstring's and fused_rope's v_cache_lp shape): byte
 *       [p / 2, d] = (code of position 2 (p / 2), code of position 2 (p / 2) + 1) at channel
 *       d; writing one position leaves the other nibble of its byte as it was.  Scales stay
 *       one per (position, head) (or per group of D / group_num channels) for K and V.
 *   D16 single_query_cached_kv_attn's int4 caches and mask (_ops.py:826-829, 852, 860, 868,
 *       887).  kv_cache_quant_bit_size 4: int8 caches of signed 4-bit pairs in D15's nibble
 *       order (even element high, odd low, sign-extending reads), k = code * scale as D12.
 *       K pairs adjacent channels (k_cache [NB, Hkv, BS, D / 2], "cache_dim = head_size_qk //
 *       2").  V pairs adjacent positions of a page, v_cache [NB, Hkv, BS / 2, Dv]: byte
 *       [r / 2, d] holds rows 2 (r / 2) and 2 (r / 2) + 1 of channel d -- the layout whose last
 *       dim is head_size_v, which the reference's own output allocation reads
 *       (`head_size_v = v_cache.shape[-1]`, _ops.py:887; also
 *       single_query_mixed_cached_kv_attn's, _ops.py:975, fed fused_rope's v_cache_lp
 *       [.., max_decode_len / 2, head_size], _ops.py:3534); or, when v_cache is
 *       [NB, Hkv, BS, Dv / 2] ("the same as k_cache, except cache_dim", _ops.py:830), pairs of
 *       adjacent channels as K.  mask [batch, seq_q, mask_len] (_ops.py:860): an additive
 *       logit term for the last mask_len keys of the sequence -- key j >= L - mask_len of
 *       query token s gets s_j += mask[i, s, j - (L - mask_len)] after softmax_scale and
 *       alibi (L the sequence's context length as clamped to its block table); -inf removes
 *       the key.  The reference states the shape and limits (seq_q <= 16, mask_len <= 64,
 *       mask_len % seq_q == 0) but not which keys the columns address: the last mask_len
 *       keys -- the newest tokens, the ones a speculative-decoding tree mask covers -- is this
 *       build's reading.
 *   D17 single_query_cached_kv_attn's quantised q and sparse-KV block tables (_ops.py:834,
 *       853-856, 862, 868-875, 887-890).  q of int8 or float8_e4m3fn holds codes: q = code *
 *       q_quant_scale, the scale per tensor ([1]), per token and head ([total_q, heads] or
 *       [batch, seq_q, heads]) or per group of head_size / scale_num channels ([batch, seq_q,
 *       heads, scale_num]), the product taken exactly; the output is out_dtype.  Sparse KV:
 *       block_tables [batch, head_num_kv, max_blocks] or [batch, head_num_q, max_blocks]
 *       give each KV head (or each query head) its own pages; context lengths stay per
 *       sequence.
 *   D9  offline (static-scale) quantisation divides: code = clip(RNE(RN(fp32(x) / s)), -128, 127)
 *       for int8, fp8 = e4m3fn_RNE(clip(RN(fp32(x) / s), -448, 448)), s the fp32 per-channel
 *       scale or the per-tensor scalar rounded to fp32 (_ops.py:1652-1670; the division is
 *       the linear sibling's `key_i /= scale`, _ops.py:1829-1840).
 *
 * Parity pins for every function here live in tests/test_oracle_pins.py (torch-CPU
 * execution of the docstring math, exact rational arithmetic on engineered near-ties,
 * closed forms and invariants).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math, SSE2 fp32 math).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* DT_I4: int8 storage of signed 4-bit pairs (D15 / D16 nibble order) */
enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3, DT_F8E4M3 = 4, DT_I4 = 5 };

/* ------------------------------------------------------------------ conversions */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

static inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));          /* inf / nan */
    if (e == 0) {
        if (m == 0) return u2f(sign);                                    /* +-0 */
        /* subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN) */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* round-to-nearest-even fp32 -> fp16, IEEE overflow to inf, gradual underflow */
static inline uint16_t f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                                     /* normal fp16 */
        uint32_t r = ax - 0x38000000u;                           /* rebias 127 -> 15 */
        r += 0xfffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    if (ax < 0x33000000u) return (uint16_t)sign;                 /* < 2^-25 -> 0 */
    uint32_t e = ax >> 23;                                       /* 102 .. 112 */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;                                   /* 14 .. 24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static inline float load_elem(const void* base, int64_t idx, int dtype) {
    switch (dtype) {
    case DT_F32: return ((const float*)base)[idx];
    case DT_F16: return f16_to_f32(((const uint16_t*)base)[idx]);
    case DT_BF16: return bf16_to_f32(((const uint16_t*)base)[idx]);
    default: return 0.0f;
    }
}

static inline void store_elem(void* base, int64_t idx, int dtype, float v) {
    switch (dtype) {
    case DT_F32: ((float*)base)[idx] = v; break;
    case DT_F16: ((uint16_t*)base)[idx] = f32_to_f16(v); break;
    case DT_BF16: ((uint16_t*)base)[idx] = f32_to_bf16(v); break;
    default: break;
    }
}

static int elem_size(int dtype) {
    switch (dtype) {
    case DT_F32: return 4;
    case DT_F16: case DT_BF16: return 2;
    case DT_I8: return 1;
    default: return 0;
    }
}

/* Exposed for the pins in tests/: element conversions over arrays. */
void oracle_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}
void oracle_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}
void oracle_f16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------ threading */

typedef void (*range_fn)(void* ctx, int64_t lo, int64_t hi);
typedef struct { range_fn fn; void* ctx; int64_t lo, hi; } range_job;

static void* run_range(void* p) {
    range_job* j = (range_job*)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* Split [0, n) into nthreads contiguous ranges and run fn on each (plain pthreads, so the
 * library does not bring its own OpenMP runtime into a process that already has torch's). */
static void parallel_for(int64_t n, int nthreads, range_fn fn, void* ctx) {
    if (nthreads <= 1 || n < 2 * (int64_t)nthreads) { fn(ctx, 0, n); return; }
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    int created[256];
    range_job jobs[256];
    int64_t chunk = (n + nthreads - 1) / nthreads;
    int nt = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t lo = (int64_t)t * chunk, hi = lo + chunk;
        if (lo >= n) break;
        if (hi > n) hi = n;
        jobs[t].fn = fn; jobs[t].ctx = ctx; jobs[t].lo = lo; jobs[t].hi = hi;
        created[t] = pthread_create(&th[t], NULL, run_range, &jobs[t]) == 0;
        if (!created[t]) fn(ctx, lo, hi);
        nt = t + 1;
    }
    for (int t = 0; t < nt; ++t)
        if (created[t]) pthread_join(th[t], NULL);
}

/*
 * fp32 -> float8_e4m3fn (sign, 4 exponent bits with bias 7, 3 fraction bits, no infinities,
 * largest finite 448), round to nearest even; defined for finite |f| <= 448 (the callers clip
 * first, as the reference math does).  Computed in double: the quantum of |f|'s binade
 * (2^(E-3), E clamped to the subnormal binade -6) divides |f| exactly, nearbyint rounds half
 * to even, and the rounded value is re-encoded.
 */
static uint8_t f32_to_e4m3(float f) {
    const uint8_t sign = signbit(f) ? 0x80 : 0;
    const double a = fabs((double)f);
    if (a == 0.0) return sign;
    int e;
    frexp(a, &e);
    int E = e - 1;                           /* 2^E <= a < 2^(E+1) */
    if (E < -6) E = -6;
    const double quantum = ldexp(1.0, E - 3);
    const double n = nearbyint(a / quantum);
    const double r = n * quantum;
    if (r < ldexp(1.0, -6)) return (uint8_t)(sign | (uint8_t)n);   /* subnormal: n * 2^-9 */
    frexp(r, &e);
    const int Er = e - 1;
    const int frac = (int)(r / ldexp(1.0, Er - 3)) - 8;
    return (uint8_t)(sign | (uint8_t)(((Er + 7) << 3) | frac));
}

void oracle_f32_to_e4m3(const float* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_e4m3(in[i]);
}

/*
 * float8_e4m3fn -> its value (the reader of the pages the fp8 branch writes): sign, exponent
 * field e (bias 7) and fraction m; e = 0 is subnormal, m * 2^-9; otherwise (8 + m) * 2^(e-10);
 * S.1111.111 is NaN (the format has no infinities).
 */
static double e4m3_to_f64(uint8_t b) {
    const int e = (b >> 3) & 15, m = b & 7;
    double v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexp((double)m, -9);
    else v = ldexp((double)(8 + m), e - 10);
    return (b & 0x80) ? -v : v;
}

void oracle_e4m3_to_f32(const uint8_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = (float)e4m3_to_f64(in[i]);
}

/* Code byte of a quantised cache as a number: int8, or a float8_e4m3fn value. */
static inline double cache_code(const void* base, int64_t idx, int cache_dtype) {
    if (cache_dtype == DT_F8E4M3) return e4m3_to_f64(((const uint8_t*)base)[idx]);
    return (double)((const int8_t*)base)[idx];
}

/* ------------------------------------------------------------------ row quantiser */

/*
 * One row of `n` fp32 values (already converted / smoothed) -> int8 codes + fp32 scale.
 * _ops.py:1524-1537 (quant_to_paged_cache) and _ops.py:3167-3172 (moe_quantize):
 *   max_value = max(|x|); scale = max_value / 127; codes = clip(round(x / scale), -128, 127)
 */
static float quant_row(const float* x, int64_t n, int8_t* codes) {
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float scale = amax / 127.0f;
    if (scale == 0.0f) {                                   /* D3 */
        memset(codes, 0, (size_t)n);
        return scale;
    }
    for (int64_t i = 0; i < n; ++i) {
        float q = rintf(x[i] / scale);                     /* D1: IEEE divide, RNE */
        if (q < -128.0f) q = -128.0f;                      /* D2 */
        if (q > 127.0f) q = 127.0f;
        codes[i] = (int8_t)q;
    }
    return scale;
}

/* One row / group of n values -> codes (int8 bytes, or e4m3fn bytes with scale = RN(amax / 448)
 * and codes e4m3fn_RNE(clip(RN(x / scale), -448, 448))) + fp32 scale (_ops.py:1524-1537,
 * 1728-1745). */
static float quant_group(const float* x, int64_t n, uint8_t* codes, int cache_dtype) {
    if (cache_dtype == DT_I8) return quant_row(x, n, (int8_t*)codes);
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float scale = amax / 448.0f;                           /* IEEE divide */
    if (scale == 0.0f) {                                   /* as D3 */
        memset(codes, 0, (size_t)n);
        return scale;
    }
    for (int64_t i = 0; i < n; ++i) {
        float q = x[i] / scale;
        if (q < -448.0f) q = -448.0f;                      /* clip(key_i, -448, 448) */
        if (q > 448.0f) q = 448.0f;
        codes[i] = f32_to_e4m3(q);
    }
    return scale;
}

/* D15: one row / group of n values -> signed 4-bit codes (one per int8, -8..7) + fp32 scale:
 * scale = RN(amax / 7), code = clip(RNE(RN(x / scale)), -8, 7) (_ops.py:1736-1742). */
static float quant_group4(const float* x, int64_t n, int8_t* codes) {
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float scale = amax / 7.0f;                             /* IEEE divide */
    if (scale == 0.0f) {                                   /* as D3 */
        memset(codes, 0, (size_t)n);
        return scale;
    }
    for (int64_t i = 0; i < n; ++i) {
        float q = rintf(x[i] / scale);                     /* IEEE divide, RNE */
        if (q < -8.0f) q = -8.0f;
        if (q > 7.0f) q = 7.0f;
        codes[i] = (int8_t)q;
    }
    return scale;
}

/* D15 nibble access: the even element of a pair in the high nibble, the odd one in the low
 * nibble; a read sign-extends (int8 arithmetic shifts). */
static inline void put_nibble(uint8_t* byte, int odd, int8_t code) {
    uint8_t c = (uint8_t)code & 0x0Fu;
    *byte = odd ? (uint8_t)((*byte & 0xF0u) | c) : (uint8_t)((*byte & 0x0Fu) | (c << 4));
}
static inline int8_t get_nibble(uint8_t byte, int odd) {
    int8_t b = (int8_t)byte;
    return odd ? (int8_t)((int8_t)(b << 4) >> 4) : (int8_t)(b >> 4);
}

/* ------------------------------------------------------------------ quant_to_paged_cache */

typedef struct {
    const void* src[2];
    int64_t st[2], sh[2];
    uint8_t* cache[2];
    float* scale[2];
    int nkv;
    const int32_t* slot;
    int64_t T, H, D, NB, BS;
    int dtype, cache_dtype;
} qpc_ctx;

static void qpc_range(void* p, int64_t lo, int64_t hi) {
    qpc_ctx* c = (qpc_ctx*)p;
    float* row = (float*)malloc((size_t)c->D * sizeof(float));
    uint8_t* codes = (uint8_t*)malloc((size_t)c->D);
    for (int64_t t = lo; t < hi; ++t) {
        int64_t slot = c->slot[t];
        if (slot < 0 || slot >= c->NB * c->BS) continue;            /* D4 */
        int64_t blk = slot / c->BS, off = slot % c->BS;              /* _ops.py:1265-1266 */
        for (int kv = 0; kv < c->nkv; ++kv) {
            for (int64_t h = 0; h < c->H; ++h) {
                int64_t base = t * c->st[kv] + h * c->sh[kv];
                for (int64_t d = 0; d < c->D; ++d) row[d] = load_elem(c->src[kv], base + d, c->dtype);
                float s = quant_group(row, c->D, codes, c->cache_dtype);
                int64_t page_row = (blk * c->H + h) * c->BS + off;   /* [NB, H, BS] */
                memcpy(c->cache[kv] + page_row * c->D, codes, (size_t)c->D);
                c->scale[kv][page_row] = s;
            }
        }
    }
    free(row);
    free(codes);
}

/* _ops.py:1511-1565: quant_to_paged_cache(k, v, k_cache, v_cache, k_scale, v_scale, slot_mapping)
 * k/v [T, H, D] with element strides (token, head), last dim contiguous;
 * caches [NB, H, BS, D] int8 or float8_e4m3fn (cache_dtype) contiguous; scales [NB, H, BS] fp32
 * contiguous. v may be NULL. */
int oracle_quant_to_paged_cache(const void* k, const void* v, int dtype,
                                int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
                                void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                                const int32_t* slot_mapping, int64_t T, int64_t H, int64_t D,
                                int64_t NB, int64_t BS, int cache_dtype, int nthreads) {
    if (elem_size(dtype) == 0 || dtype == DT_I8) return -2;
    if (cache_dtype != DT_I8 && cache_dtype != DT_F8E4M3) return -2;
    if (T < 0 || H <= 0 || D <= 0 || NB < 0 || BS <= 0) return -1;
    qpc_ctx c = {{k, v}, {k_st, v_st}, {k_sh, v_sh}, {(uint8_t*)k_cache, (uint8_t*)v_cache},
                 {k_scale, v_scale}, v ? 2 : 1, slot_mapping, T, H, D, NB, BS, dtype, cache_dtype};
    parallel_for(T, nthreads, qpc_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ offline_quant_to_paged_cache */

typedef struct {
    const void* src[2];
    int64_t st[2], sh[2];
    uint8_t* cache[2];
    const float* chan[2];
    float tensor[2];
    int nkv;
    const int32_t* slot;
    int64_t T, H, D, NB, BS;
    int dtype, cache_dtype;
} oqpc_ctx;

/* One element: D9. */
static uint8_t static_code(float x, float s, int cache_dtype) {
    float q = x / s;                                       /* IEEE divide */
    if (cache_dtype == DT_F8E4M3) {
        if (q < -448.0f) q = -448.0f;                      /* clip(key_i, -448, 448) */
        if (q > 448.0f) q = 448.0f;
        return f32_to_e4m3(q);
    }
    q = rintf(q);                                          /* round half to even */
    if (q < -128.0f) q = -128.0f;                          /* clip(-128, 127) */
    if (q > 127.0f) q = 127.0f;
    return (uint8_t)(int8_t)q;
}

static void oqpc_range(void* p, int64_t lo, int64_t hi) {
    oqpc_ctx* c = (oqpc_ctx*)p;
    for (int64_t t = lo; t < hi; ++t) {
        int64_t slot = c->slot[t];
        if (slot < 0 || slot >= c->NB * c->BS) continue;            /* _ops.py:1656, D4 */
        int64_t blk = slot / c->BS, off = slot % c->BS;              /* _ops.py:1659-1660 */
        for (int kv = 0; kv < c->nkv; ++kv) {
            for (int64_t h = 0; h < c->H; ++h) {
                int64_t base = t * c->st[kv] + h * c->sh[kv];
                uint8_t* dst = c->cache[kv] + ((blk * c->H + h) * c->BS + off) * c->D;
                for (int64_t d = 0; d < c->D; ++d) {
                    float s = c->chan[kv] ? c->chan[kv][h * c->D + d] : c->tensor[kv];
                    dst[d] = static_code(load_elem(c->src[kv], base + d, c->dtype), s, c->cache_dtype);
                }
            }
        }
    }
}

/* _ops.py:1639-1706: offline_quant_to_paged_cache(k, v, k_cache_scale, v_cache_scale,
 * slot_mapping, k_cache, v_cache).  k/v [T, H, D] with element strides (token, head);
 * caches [NB, H, BS, D] int8 or float8_e4m3fn (cache_dtype DT_I8 / DT_F8E4M3); each of K and
 * V uses its per-channel scale [H, D] when given, else its per-tensor scalar. */
int oracle_offline_quant_to_paged_cache(const void* k, const void* v, int dtype,
                                        int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
                                        void* k_cache, void* v_cache, int cache_dtype,
                                        const float* k_chan, const float* v_chan,
                                        float k_tensor, float v_tensor,
                                        const int32_t* slot_mapping, int64_t T, int64_t H,
                                        int64_t D, int64_t NB, int64_t BS, int nthreads) {
    if (elem_size(dtype) == 0 || dtype == DT_I8) return -2;
    if (cache_dtype != DT_I8 && cache_dtype != DT_F8E4M3) return -2;
    if (T < 0 || H <= 0 || D <= 0 || NB < 0 || BS <= 0) return -1;
    oqpc_ctx c = {{k, v}, {k_st, v_st}, {k_sh, v_sh}, {(uint8_t*)k_cache, (uint8_t*)v_cache},
                  {k_chan, v_chan}, {k_tensor, v_tensor}, v ? 2 : 1, slot_mapping,
                  T, H, D, NB, BS, dtype, cache_dtype};
    parallel_for(T, nthreads, oqpc_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ fused_rope (rmsnorm, paged) */

typedef struct {
    void* qkv;
    int dtype;
    int64_t T, S, Hq, Hk, D;
    const void* sin_t;
    const void* cos_t;
    int64_t rope_dim, rope_off, table_stride, table_rows;
    const int32_t* position;
    const void* k_gamma;
    const void* q_gamma;
    float eps;
    const void* k_beta;             /* layernorm only, nullable */
    int norm;                       /* 0 rmsnorm, 1 layernorm */
    void* cache[2];
    int cache_dtype;
    float* scale[2];
    int scale_mode;                 /* 0 none, 1 dynamic per token [NB, Hk, BS], 2 static [Hk, D] */
    const int32_t* slot;
    int64_t NB, BS;
} frope_ctx;

/* D10: sum of squares in 8-element chunks, then a balanced tree over the chunk sums. */
static float rms_sum_squares(const float* x, int64_t n) {
    float part[64];
    int64_t nchunks = (n + 7) / 8, width = 1;
    while (width < nchunks) width *= 2;
    for (int64_t c = 0; c < width; ++c) {
        float acc = 0.0f;
        if (c < nchunks) {
            int64_t e0 = 8 * c, e1 = e0 + 8 < n ? e0 + 8 : n;
            acc = x[e0] * x[e0];
            for (int64_t e = e0 + 1; e < e1; ++e) {
                float sq = x[e] * x[e];
                acc = acc + sq;
            }
        }
        part[c] = acc;
    }
    for (int64_t w = width; w > 1; w /= 2)
        for (int64_t c = 0; c < w / 2; ++c) part[c] = part[2 * c] + part[2 * c + 1];
    return part[0];
}

/* D13: the chunked sum (D10 order) of the values themselves. */
static float chunk_sum(const float* x, int64_t n) {
    float part[64];
    int64_t nchunks = (n + 7) / 8, width = 1;
    while (width < nchunks) width *= 2;
    for (int64_t c = 0; c < width; ++c) {
        float acc = 0.0f;
        if (c < nchunks) {
            int64_t e0 = 8 * c, e1 = e0 + 8 < n ? e0 + 8 : n;
            acc = x[e0];
            for (int64_t e = e0 + 1; e < e1; ++e) acc = acc + x[e];
        }
        part[c] = acc;
    }
    for (int64_t w = width; w > 1; w /= 2)
        for (int64_t c = 0; c < w / 2; ++c) part[c] = part[2 * c] + part[2 * c + 1];
    return part[0];
}

/* D13 layernorm with gamma and optional beta (in place on fp32 row; tmp: D floats) */
static void layernorm_row(float* x, float* tmp, int64_t D, const void* gamma, const void* beta,
                          int dtype, float eps) {
    float mean = chunk_sum(x, D) / (float)D;
    for (int64_t d = 0; d < D; ++d) tmp[d] = x[d] - mean;
    float var = rms_sum_squares(tmp, D) / (float)D;
    float r = sqrtf(var + eps);
    float inv = 1.0f / r;
    for (int64_t d = 0; d < D; ++d) {
        float t = tmp[d] * inv;
        float y = t * load_elem(gamma, d, dtype);
        if (beta) y = y + load_elem(beta, d, dtype);
        x[d] = y;
    }
}

/* rmsnorm with gamma (in place on fp32 row) */
static void rmsnorm_row(float* x, int64_t D, const void* gamma, int dtype, float eps) {
    float ss = rms_sum_squares(x, D);
    float mean = ss / (float)D;
    float r = sqrtf(mean + eps);
    float inv = 1.0f / r;
    for (int64_t d = 0; d < D; ++d) {
        float t = x[d] * inv;
        x[d] = t * load_elem(gamma, d, dtype);
    }
}

/* fold rope over [off, off + rope_dim) of the row (_ops.py:1120-1127, interleaved False) */
static void rope_row(float* y, float* tmp, const frope_ctx* c, int64_t pos) {
    int64_t half = c->rope_dim / 2;
    if (pos < 0 || pos >= c->table_rows) return;   /* D10: no table row, no rotation */
    for (int64_t d = 0; d < c->D; ++d) tmp[d] = y[d];
    for (int64_t j = 0; j < c->rope_dim; ++j) {
        float rot = j < half ? -tmp[c->rope_off + j + half] : tmp[c->rope_off + j - half];
        float sn = load_elem(c->sin_t, pos * c->table_stride + j, c->dtype);
        float cs = load_elem(c->cos_t, pos * c->table_stride + j, c->dtype);
        float a = rot * sn;
        float b = tmp[c->rope_off + j] * cs;
        y[c->rope_off + j] = a + b;
    }
}

static void frope_store(const frope_ctx* c, int kv, const float* row, int64_t page_row, int64_t h) {
    int64_t D = c->D;
    if (c->scale_mode == 0) {
        for (int64_t d = 0; d < D; ++d) store_elem(c->cache[kv], page_row * D + d, c->dtype, row[d]);
        return;
    }
    int8_t* dst = (int8_t*)c->cache[kv] + page_row * D;
    if (c->scale_mode == 1) {
        c->scale[kv][page_row] = quant_row(row, D, dst);
        return;
    }
    for (int64_t d = 0; d < D; ++d) {
        float q = row[d] / c->scale[kv][h * D + d];
        q = rintf(q);
        if (q < -128.0f) q = -128.0f;
        if (q > 127.0f) q = 127.0f;
        dst[d] = (int8_t)q;
    }
}

static void frope_range(void* p, int64_t lo, int64_t hi) {
    frope_ctx* c = (frope_ctx*)p;
    int64_t D = c->D, H = c->Hq + 2 * c->Hk;
    float* row = (float*)malloc((size_t)D * sizeof(float));
    float* tmp = (float*)malloc((size_t)D * sizeof(float));
    for (int64_t t = lo; t < hi; ++t) {
        int64_t pos = (int64_t)c->position[t / c->S] + t % c->S;
        int64_t slot = c->slot[t];
        int valid = slot >= 0 && slot < c->NB * c->BS;
        int64_t blk = valid ? slot / c->BS : 0, off = valid ? slot % c->BS : 0;
        for (int64_t hh = 0; hh < H; ++hh) {
            int64_t base = (t * H + hh) * D;
            for (int64_t d = 0; d < D; ++d) row[d] = load_elem(c->qkv, base + d, c->dtype);
            if (hh < c->Hq) {                     /* q: rmsnorm (if q_gamma, rmsnorm only), rope */
                if (c->norm == 0 && c->q_gamma) rmsnorm_row(row, D, c->q_gamma, c->dtype, c->eps);
                rope_row(row, tmp, c, pos);
                for (int64_t d = 0; d < D; ++d) store_elem(c->qkv, base + d, c->dtype, row[d]);
            } else if (hh < c->Hq + c->Hk) {     /* k: rmsnorm + rope, or rope + layernorm; store */
                if (!valid) continue;
                int64_t h = hh - c->Hq;
                if (c->norm == 0) {
                    rmsnorm_row(row, D, c->k_gamma, c->dtype, c->eps);
                    rope_row(row, tmp, c, pos);
                } else {
                    rope_row(row, tmp, c, pos);
                    layernorm_row(row, tmp, D, c->k_gamma, c->k_beta, c->dtype, c->eps);
                }
                frope_store(c, 0, row, (blk * c->Hk + h) * c->BS + off, h);
            } else {                                             /* v: store */
                if (!valid) continue;
                int64_t h = hh - c->Hq - c->Hk;
                frope_store(c, 1, row, (blk * c->Hk + h) * c->BS + off, h);
            }
        }
    }
    free(row);
    free(tmp);
}

/* _ops.py:3469-3601 fused_rope / 6356-6423 fused_rmsnorm_rope_store_paged_cache, norm_type
 * "rmsnorm" (norm 0, D10) or "layernorm" (norm 1, D13), paged high-precision caches.  qkv [T, Hq + 2 Hk, D] contiguous (T = batch * S,
 * token t at position position[t / S] + t % S); sin/cos [rows, table_stride] of qkv's dtype;
 * caches [NB, Hk, BS, D] of qkv's dtype (scale_mode 0) or int8 (1: dynamic per-token scales
 * written to [NB, Hk, BS]; 2: static per-channel scales read from [Hk, D]). */
int oracle_fused_rope_paged(void* qkv, int dtype, int64_t T, int64_t S, int64_t Hq, int64_t Hk,
                            int64_t D, const void* sin_t, const void* cos_t, int64_t rope_dim,
                            int64_t rope_off, int64_t table_stride, int64_t table_rows,
                            const int32_t* position,
                            const void* k_gamma, const void* q_gamma, float eps,
                            const void* k_beta, int norm,
                            void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                            int scale_mode, const int32_t* slot, int64_t NB, int64_t BS,
                            int nthreads) {
    if (dtype != DT_F16 && dtype != DT_BF16 && dtype != DT_F32) return -2;
    if (T < 0 || S <= 0 || Hq < 0 || Hk <= 0 || D <= 0 || D > 512 || NB < 0 || BS <= 0) return -1;
    if (rope_dim < 0 || rope_dim % 2 || rope_off < 0 || rope_off + rope_dim > D) return -1;
    if (norm != 0 && norm != 1) return -3;
    frope_ctx c = {qkv, dtype, T, S, Hq, Hk, D, sin_t, cos_t, rope_dim, rope_off, table_stride,
                   table_rows, position, k_gamma, q_gamma, eps, k_beta, norm, {k_cache, v_cache},
                   DT_I8, {k_scale, v_scale}, scale_mode, slot, NB, BS};
    parallel_for(T, nthreads, frope_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ linear caches (D11) */

typedef struct {
    int64_t batch, H, D, cache_batch, cache_len, rows;   /* rows: input / output tensor rows */
    const int32_t* lens;       /* [batch] or [batch + 1] when packed */
    int packed;
    int64_t pad_seqlen;        /* padded input: rows per sequence */
    const int32_t* seq_off;    /* nullable */
    const int32_t* bs_id;      /* nullable */
    const int32_t* cache_off;  /* nullable */
    const int32_t* bt;         /* nullable: block table [batch, max_blocks] of cache_len-row blocks */
    int64_t max_blocks;
} lin_addr;

static int64_t lin_len(const lin_addr* a, int64_t i) {
    return a->packed ? (int64_t)a->lens[i + 1] - a->lens[i] : a->lens[i];
}

/* first row of sequence i in the token-major tensor; in_dir: it is the input of a cache write */
static int64_t lin_start(const lin_addr* a, int64_t i, int in_dir) {
    if (a->seq_off) return a->seq_off[i];
    if (in_dir && a->packed) return a->lens[i];
    if (in_dir) return i * a->pad_seqlen;
    int64_t s = 0;
    for (int64_t k = 0; k < i; ++k) s += lin_len(a, k);
    return s;
}

/* cache row (b * H + h) * cache_len + pos % cache_len of token j of sequence i, or -1 when
 * skipped.  pos = cache_offset[i] + j; without a block table b = cache_bs_id[i] (else i) and
 * pos must lie in [0, cache_len); with one, b = bt[i, pos / cache_len] (a paged cache of
 * cache_len-row blocks; a one-column table is the linear layout, _ops.py:3906-3909). */
static int64_t lin_cache_row(const lin_addr* a, int64_t i, int64_t j, int64_t h) {
    int64_t pos = (a->cache_off ? a->cache_off[i] : 0) + j;
    if (pos < 0 || a->cache_len <= 0) return -1;
    int64_t bi = pos / a->cache_len, b;
    if (a->bt) {
        if (bi >= a->max_blocks) return -1;
        b = a->bt[i * a->max_blocks + bi];
    } else {
        if (bi != 0) return -1;
        b = a->bs_id ? a->bs_id[i] : i;
    }
    if (b < 0 || b >= a->cache_batch) return -1;
    return (b * a->H + h) * a->cache_len + pos % a->cache_len;
}

typedef struct {
    lin_addr a;
    int op;                   /* 0 copy in, 1 dynamic quant in, 2 static quant in, 3 dequant out, 4 copy out */
    const void* src[2];
    void* dst[2];
    int64_t st[2], sh[2];     /* token-major tensor strides (elements) */
    int dtype;                /* token-major tensor dtype */
    float* scale[2];          /* dynamic: [cache_batch, H, cache_len] */
    const float* chan[2];     /* static mode 0 [H, D]; mode 1 [H, cache_len] */
    float tensor_scale[2];    /* static modes 2/3 */
    int smode;                /* static / dequant scale mode: 0 channel, 1 head (static) or token (dequant), 2 tensor */
    int nkv;
    int cache_dtype;          /* quantising ops: DT_I8 or DT_F8E4M3 */
    int64_t groups;           /* dynamic: scale groups per (token, head) */
    int64_t max_len;          /* tokens j >= max_len are skipped */
    int bits;                 /* ops 1 and 3: 8, or 4 (D15: packed int4 pairs) */
} lin_ctx;

static void lin_range(void* p, int64_t lo, int64_t hi) {
    lin_ctx* c = (lin_ctx*)p;
    const lin_addr* a = &c->a;
    int64_t D = a->D;
    int in_dir = c->op <= 2;
    float* row = (float*)malloc((size_t)D * sizeof(float));
    uint8_t* codes = (uint8_t*)malloc((size_t)D);
    for (int64_t i = lo; i < hi; ++i) {
        int64_t len = lin_len(a, i), start = lin_start(a, i, in_dir);
        if (len > c->max_len) len = c->max_len;
        for (int64_t j = 0; j < len; ++j) {
            int64_t r = start + j;
            if (r < 0 || r >= a->rows) continue;
            for (int kv = 0; kv < c->nkv; ++kv) {
                for (int64_t h = 0; h < a->H; ++h) {
                    int64_t cr = lin_cache_row(a, i, j, h);
                    if (cr < 0) continue;
                    int64_t tok = r * c->st[kv] + h * c->sh[kv];
                    int64_t pos = cr % a->cache_len;
                    if (c->op == 0 || c->op == 4) {                 /* byte copy */
                        int es = elem_size(c->dtype);
                        const char* from = c->op == 0 ? (const char*)c->src[kv] + tok * es
                                                      : (const char*)c->src[kv] + cr * D * es;
                        char* to = c->op == 0 ? (char*)c->dst[kv] + cr * D * es
                                              : (char*)c->dst[kv] + tok * es;
                        memcpy(to, from, (size_t)(D * es));
                    } else if (c->op == 1 && c->bits == 4) {        /* D15: int4 pairs */
                        int64_t gs = D / c->groups;
                        for (int64_t d = 0; d < D; ++d) row[d] = load_elem(c->src[kv], tok + d, c->dtype);
                        for (int64_t g = 0; g < c->groups; ++g)
                            c->scale[kv][cr * c->groups + g] =
                                quant_group4(row + g * gs, gs, (int8_t*)codes + g * gs);
                        if (kv == 0) {                              /* K: channel pairs */
                            uint8_t* out = (uint8_t*)c->dst[kv] + cr * (D / 2);
                            for (int64_t d = 0; d < D; ++d) put_nibble(out + d / 2, (int)(d & 1), (int8_t)codes[d]);
                        } else {                                    /* V: position pairs */
                            int64_t bh = (cr - pos) / a->cache_len;
                            uint8_t* out = (uint8_t*)c->dst[kv] + (bh * (a->cache_len / 2) + pos / 2) * D;
                            for (int64_t d = 0; d < D; ++d) put_nibble(out + d, (int)(pos & 1), (int8_t)codes[d]);
                        }
                    } else if (c->op == 1) {                        /* dynamic per token / group */
                        int64_t gs = D / c->groups;
                        for (int64_t d = 0; d < D; ++d) row[d] = load_elem(c->src[kv], tok + d, c->dtype);
                        for (int64_t g = 0; g < c->groups; ++g)
                            c->scale[kv][cr * c->groups + g] =
                                quant_group(row + g * gs, gs, codes + g * gs, c->cache_dtype);
                        memcpy((uint8_t*)c->dst[kv] + cr * D, codes, (size_t)D);
                    } else if (c->op == 2) {                        /* static */
                        uint8_t* out = (uint8_t*)c->dst[kv] + cr * D;
                        for (int64_t d = 0; d < D; ++d) {
                            float s = c->smode == 0 ? c->chan[kv][h * D + d]
                                    : c->smode == 1 ? c->chan[kv][h * a->cache_len + pos]
                                                    : c->tensor_scale[kv];
                            out[d] = static_code(load_elem(c->src[kv], tok + d, c->dtype), s, c->cache_dtype);
                        }
                    } else if (c->bits == 4) {                      /* dequant, D15 int4 pairs */
                        for (int64_t d = 0; d < D; ++d) {
                            int8_t code;
                            if (kv == 0) {
                                code = get_nibble(((const uint8_t*)c->src[kv])[cr * (D / 2) + d / 2], (int)(d & 1));
                            } else {
                                int64_t bh = (cr - pos) / a->cache_len;
                                code = get_nibble(((const uint8_t*)c->src[kv])[(bh * (a->cache_len / 2) + pos / 2) * D + d],
                                                  (int)(pos & 1));
                            }
                            float s = c->smode == 0 ? c->chan[kv][h * D + d] : c->scale[kv][cr];
                            store_elem(c->dst[kv], tok + d, c->dtype, (float)code * s);
                        }
                    } else {                                        /* dequant */
                        const int8_t* in = (const int8_t*)c->src[kv] + cr * D;
                        for (int64_t d = 0; d < D; ++d) {
                            float s = c->smode == 0 ? c->chan[kv][h * D + d] : c->scale[kv][cr];
                            store_elem(c->dst[kv], tok + d, c->dtype, (float)in[d] * s);
                        }
                    }
                }
            }
        }
    }
    free(row);
    free(codes);
}

/* One entry for the five linear-cache ops (the op code selects the direction and arithmetic):
 *   op 0 reshape_linear_cache (_ops.py:1189-1249), 1 quant_to_linear_cache (:1708-1806),
 *   2 offline_quant_to_linear_cache (:1808-1919), 3 dequant_from_linear_cache (:3642-3732),
 *   4 reshape_from_cache, linear mode (:3898-3969).
 * tok[2] / tok_st / tok_sh: the token-major tensors (input for ops 0-2, output for 3-4).
 * cache_dtype: the cache's element type for ops 1-2 (DT_I8 or DT_F8E4M3; op 3 reads int8);
 * groups: scale groups per (token, head) for op 1.  block_tables [batch, max_blocks] (nullable)
 * turns the cache into pages of cache_len rows: op 4 with it is reshape_from_cache's paged mode,
 * op 3 with it reads per-token scales [num_blocks, H, cache_len]. */
int oracle_linear_cache_bits(int op, void* tok_k, void* tok_v, int dtype, int64_t k_st, int64_t k_sh,
                             int64_t v_st, int64_t v_sh, int64_t rows, void* cache_k, void* cache_v,
                             int cache_dtype, int64_t cache_batch, int64_t H, int64_t cache_len, int64_t D,
                             float* k_scale, float* v_scale, const float* k_chan, const float* v_chan,
                             float k_tensor, float v_tensor, int smode, int64_t groups,
                             const int32_t* lens, int64_t batch, int64_t max_len, int packed,
                             int64_t pad_seqlen, const int32_t* seq_off, const int32_t* bs_id,
                             const int32_t* cache_off, const int32_t* block_tables,
                             int64_t max_blocks, int bits, int nthreads);

int oracle_linear_cache(int op, void* tok_k, void* tok_v, int dtype, int64_t k_st, int64_t k_sh,
                        int64_t v_st, int64_t v_sh, int64_t rows, void* cache_k, void* cache_v,
                        int cache_dtype, int64_t cache_batch, int64_t H, int64_t cache_len, int64_t D,
                        float* k_scale, float* v_scale, const float* k_chan, const float* v_chan,
                        float k_tensor, float v_tensor, int smode, int64_t groups,
                        const int32_t* lens, int64_t batch, int64_t max_len, int packed,
                        int64_t pad_seqlen, const int32_t* seq_off, const int32_t* bs_id,
                        const int32_t* cache_off, const int32_t* block_tables,
                        int64_t max_blocks, int nthreads) {
    return oracle_linear_cache_bits(op, tok_k, tok_v, dtype, k_st, k_sh, v_st, v_sh, rows, cache_k,
                                    cache_v, cache_dtype, cache_batch, H, cache_len, D, k_scale,
                                    v_scale, k_chan, v_chan, k_tensor, v_tensor, smode, groups, lens,
                                    batch, max_len, packed, pad_seqlen, seq_off, bs_id, cache_off,
                                    block_tables, max_blocks, 8, nthreads);
}

/* The same with quant_bit `bits` for ops 1 and 3: 8, or 4 (D15: int8 caches of int4 pairs, K
 * [cache_batch, H, cache_len, D / 2], V [cache_batch, H, cache_len / 2, D] with cache_len
 * even; no block table, int8 caches only). */
int oracle_linear_cache_bits(int op, void* tok_k, void* tok_v, int dtype, int64_t k_st, int64_t k_sh,
                             int64_t v_st, int64_t v_sh, int64_t rows, void* cache_k, void* cache_v,
                             int cache_dtype, int64_t cache_batch, int64_t H, int64_t cache_len, int64_t D,
                             float* k_scale, float* v_scale, const float* k_chan, const float* v_chan,
                             float k_tensor, float v_tensor, int smode, int64_t groups,
                             const int32_t* lens, int64_t batch, int64_t max_len, int packed,
                             int64_t pad_seqlen, const int32_t* seq_off, const int32_t* bs_id,
                             const int32_t* cache_off, const int32_t* block_tables,
                             int64_t max_blocks, int bits, int nthreads) {
    if (bits != 8 && bits != 4) return -3;
    if (bits == 4 && ((op != 1 && op != 3) || (op == 1 && cache_dtype != DT_I8) || D % 2 != 0 ||
                      (tok_v && cache_len % 2 != 0) || block_tables)) return -3;
    if (op < 0 || op > 4 || elem_size(dtype) == 0) return -2;
    if ((op == 1 || op == 2 || op == 3) && dtype == DT_I8) return -2;
    if ((op == 1 || op == 2) && cache_dtype != DT_I8 && cache_dtype != DT_F8E4M3) return -2;
    if (op == 1 && (groups <= 0 || D % groups != 0)) return -1;
    if (batch < 0 || H <= 0 || D <= 0 || cache_batch < 0 || cache_len < 0 || rows < 0) return -1;
    lin_ctx c;
    memset(&c, 0, sizeof c);
    c.a.batch = batch; c.a.H = H; c.a.D = D; c.a.cache_batch = cache_batch; c.a.cache_len = cache_len;
    c.a.rows = rows; c.a.lens = lens; c.a.packed = packed; c.a.pad_seqlen = pad_seqlen;
    c.a.seq_off = seq_off; c.a.bs_id = bs_id; c.a.cache_off = cache_off;
    c.a.bt = block_tables; c.a.max_blocks = max_blocks;
    c.op = op; c.dtype = dtype; c.nkv = tok_v ? 2 : 1;
    c.st[0] = k_st; c.st[1] = v_st; c.sh[0] = k_sh; c.sh[1] = v_sh;
    c.scale[0] = k_scale; c.scale[1] = v_scale; c.chan[0] = k_chan; c.chan[1] = v_chan;
    c.tensor_scale[0] = k_tensor; c.tensor_scale[1] = v_tensor; c.smode = smode;
    c.cache_dtype = cache_dtype; c.groups = groups > 0 ? groups : 1; c.max_len = max_len;
    c.bits = bits;
    if (op <= 2) { c.src[0] = tok_k; c.src[1] = tok_v; c.dst[0] = cache_k; c.dst[1] = cache_v; }
    else { c.src[0] = cache_k; c.src[1] = cache_v; c.dst[0] = tok_k; c.dst[1] = tok_v; }
    parallel_for(batch, nthreads, lin_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ reshape_paged_cache */

typedef struct {
    char* kv[2];
    int64_t st[2], sh[2];
    char* cache[2];
    int nkv;
    const int32_t* slot;
    int64_t T, H, D, NB, BS, es;
    int direction;
} rpc_ctx;

static void rpc_range(void* p, int64_t lo, int64_t hi) {
    rpc_ctx* c = (rpc_ctx*)p;
    int64_t row_bytes = c->D * c->es;
    for (int64_t t = lo; t < hi; ++t) {
        int64_t slot = c->slot[t];
        if (slot < 0 || slot >= c->NB * c->BS) continue;             /* _ops.py:1264 */
        int64_t blk = slot / c->BS, off = slot % c->BS;
        for (int kv = 0; kv < c->nkv; ++kv) {
            for (int64_t h = 0; h < c->H; ++h) {
                char* tok = c->kv[kv] + (t * c->st[kv] + h * c->sh[kv]) * c->es;
                char* page = c->cache[kv] + ((blk * c->H + h) * c->BS + off) * row_bytes;
                if (c->direction) memcpy(tok, page, (size_t)row_bytes);   /* gather */
                else memcpy(page, tok, (size_t)row_bytes);               /* scatter */
            }
        }
    }
}

/* _ops.py:1251-1294: reshape_paged_cache(k, v, k_cache, v_cache, slot_mapping, direction).
 * direction == 0 scatters k/v into the caches, direction != 0 gathers them back. */
int oracle_reshape_paged_cache(void* k, void* v, int dtype, int64_t k_st, int64_t k_sh,
                               int64_t v_st, int64_t v_sh, void* k_cache, void* v_cache,
                               const int32_t* slot_mapping, int64_t T, int64_t H, int64_t D,
                               int64_t NB, int64_t BS, int direction, int nthreads) {
    int es = elem_size(dtype);
    if (es == 0) return -2;
    if (T < 0 || H <= 0 || D <= 0 || NB < 0 || BS <= 0) return -1;
    rpc_ctx c = {{(char*)k, (char*)v}, {k_st, v_st}, {k_sh, v_sh},
                 {(char*)k_cache, (char*)v_cache}, (v && v_cache) ? 2 : 1, slot_mapping,
                 T, H, D, NB, BS, es, direction};
    parallel_for(T, nthreads, rpc_range, &c);
    return 0;
}

/* ------------------------------------------------------------------ dequant_from_paged_cache */

typedef struct {
    void* out[2];
    int64_t st[2], sh[2];
    const int8_t* cache[2];
    const float* scale[2];
    int nkv;
    int cache_dtype;          /* DT_I8 or DT_F8E4M3 */
    const int32_t* ctx_len;
    const int64_t* seq_off;
    const int32_t* bt;
    int64_t B, MB, NB, H, BS, D, total;
    int mode, dtype;
} dpc_ctx;

static void dpc_range(void* p, int64_t lo, int64_t hi) {
    dpc_ctx* c = (dpc_ctx*)p;
    for (int64_t i = lo; i < hi; ++i) {
        int64_t len = c->ctx_len[i];
        int64_t begin = c->seq_off[i];
        for (int64_t t = 0; t < len; ++t) {
            int64_t j = t / c->BS, o = t % c->BS;                  /* _ops.py:3750-3751 */
            if (j >= c->MB) break;
            int64_t blk = c->bt[i * c->MB + j];
            if (blk < 0 || blk >= c->NB) continue;
            int64_t row = begin + t;
            if (row < 0 || row >= c->total) continue;
            for (int kv = 0; kv < c->nkv; ++kv) {
                for (int64_t h = 0; h < c->H; ++h) {
                    const int64_t cbase = ((blk * c->H + h) * c->BS + o) * c->D;
                    int64_t obase = row * c->st[kv] + h * c->sh[kv];
                    for (int64_t d = 0; d < c->D; ++d) {
                        float s = c->mode == 0 ? c->scale[kv][h * c->D + d]          /* [H, D] */
                                               : c->scale[kv][(blk * c->H + h) * c->BS + o];
                        /* D6: the code (an int8, or an e4m3fn value) is exact in fp32 */
                        const float code = (float)cache_code(c->cache[kv], cbase + d, c->cache_dtype);
                        store_elem(c->out[kv], obase + d, c->dtype, code * s);
                    }
                }
            }
        }
    }
}

/* _ops.py:3734-3824: dequant_from_paged_cache(key, value, key_cache, value_cache, key_scale,
 * value_scale, context_lengths, max_context_len, context_seq_offset, block_tables, quant_mode,
 * quant_bit).  quant_mode 0: scale [H, D]; 1: scale [NB, H, BS] (_ops.py:3765-3771).
 * context_seq_offset NULL -> exclusive cumsum of context_lengths (_ops.py:3758).  Caches of
 * int8 codes (DT_I8, the reference's type) or float8_e4m3fn values (DT_F8E4M3, the pages the
 * fp8 branch of quant_to_paged_cache writes).  fp32 scales (a bf16 scale tensor widens to
 * fp32 exactly, so callers pass it widened). */
int oracle_dequant_from_paged_cache(void* key, void* value, int out_dtype, int cache_dtype,
                                    int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh,
                                    int64_t total_rows, const void* key_cache,
                                    const void* value_cache, const float* key_scale,
                                    const float* value_scale, const int32_t* context_lengths,
                                    const int32_t* context_seq_offset, const int32_t* block_tables,
                                    int64_t B, int64_t max_blocks, int64_t NB, int64_t H,
                                    int64_t BS, int64_t D, int quant_mode, int nthreads) {
    if (out_dtype != DT_F16 && out_dtype != DT_BF16 && out_dtype != DT_F32) return -2;
    if (cache_dtype != DT_I8 && cache_dtype != DT_F8E4M3) return -2;
    if (quant_mode != 0 && quant_mode != 1) return -3;
    if (B < 0 || H <= 0 || D <= 0 || BS <= 0 || max_blocks < 0) return -1;
    int64_t* off = (int64_t*)malloc((size_t)(B > 0 ? B : 1) * sizeof(int64_t));
    int64_t acc = 0;
    for (int64_t i = 0; i < B; ++i) {
        off[i] = context_seq_offset ? (int64_t)context_seq_offset[i] : acc;
        acc += context_lengths[i];
    }
    dpc_ctx c = {{key, value}, {k_st, v_st}, {k_sh, v_sh},
                 {(const int8_t*)key_cache, (const int8_t*)value_cache},
                 {key_scale, value_scale}, (value && value_cache) ? 2 : 1, cache_dtype,
                 context_lengths, off,
                 block_tables, B, max_blocks, NB, H, BS, D, total_rows, quant_mode, out_dtype};
    parallel_for(B, nthreads, dpc_range, &c);
    free(off);
    return 0;
}

/* ------------------------------------------------------------------ scaled_quantize (dynamic per token) */

typedef struct {
    const void* x;
    int dtype;
    int64_t n0, inner, C, row_stride;
    int8_t* out;
    float* out_scale;
    const float* smooth;
    int64_t smooth_len;
    const int64_t* group_end;   /* inclusive prefix of token_count, or NULL */
    int64_t ngroups;
    const int32_t* gidx;
    int64_t gstart, glen;
    int64_t rows, valid_rows;
} sq_ctx;

static void sq_range(void* p, int64_t lo, int64_t hi) {
    sq_ctx* c = (sq_ctx*)p;
    float* row = (float*)malloc((size_t)c->C * sizeof(float));
    for (int64_t r = lo; r < hi; ++r) {
        if (r >= c->valid_rows) continue;
        int64_t src = r;
        if (c->gidx) {                                                 /* _ops.py:3150-3154 */
            int64_t gi = c->gstart + r;
            if (gi < 0 || gi >= c->glen) continue;
            src = c->gidx[gi];
        }
        if (src < 0 || src >= c->n0) continue;
        const float* sm = c->smooth;
        if (c->group_end) {                                            /* _ops.py:3156-3162 */
            int64_t g = 0;
            while (g < c->ngroups && c->group_end[g] <= r) ++g;
            if (g >= c->ngroups) continue;   /* r >= sum(token_count): not produced */
            if (sm) sm += g * c->smooth_len;
        }
        for (int64_t j = 0; j < c->inner; ++j) {
            int64_t ibase = (src * c->inner + j) * c->row_stride;
            int64_t orow = r * c->inner + j;
            for (int64_t d = 0; d < c->C; ++d) {
                float xv = load_elem(c->x, ibase + d, c->dtype);
                if (sm) xv = xv * sm[c->smooth_len == 1 ? 0 : d];          /* D7 */
                row[d] = xv;
            }
            c->out_scale[orow] = quant_row(row, c->C, c->out + orow * c->C);
        }
    }
    free(row);
}

/* _ops.py:3126-3253 (moe_quantize) / 4407-4492 (scaled_quantize), quant_mode "dynamic_per_token":
 *   x [n0, inner..., C] viewed as n0*inner rows of C (row stride `row_stride` elements);
 *   smooth NULL, [1], [C] or [groups, C] fp32 (smooth_len = 1 or C); token_count [groups] (NULL: no grouping);
 *   gather_index [gather_len] (NULL: identity); gather_start NULL or [1]; rows whose
 *   gather position falls outside gather_index are not produced.
 *   Output rows = `rows` (gather_index.size(0) or n0) x inner; codes [rows*inner, C] int8,
 *   scales [rows*inner] fp32.  With gather_start given only the first sum(token_count) rows
 *   are produced (_ops.py:3150-3152); with token_count given, rows at or past
 *   sum(token_count) are never produced. */
int oracle_scaled_quantize_per_token(const void* x, int dtype, int64_t n0, int64_t inner,
                                     int64_t C, int64_t row_stride, int8_t* out, float* out_scale,
                                     const float* smooth, int64_t smooth_len,
                                     const int32_t* token_count,
                                     int64_t ngroups, const int32_t* gather_index,
                                     int64_t gather_len, const int32_t* gather_start,
                                     int64_t rows, int nthreads) {
    if (dtype != DT_F32 && dtype != DT_F16 && dtype != DT_BF16) return -2;
    if (n0 < 0 || inner <= 0 || C <= 0 || rows < 0) return -1;
    if (smooth && smooth_len != 1 && smooth_len != C) return -1;
    int64_t* gend = NULL;
    int64_t total = rows;
    if (token_count) {
        gend = (int64_t*)malloc((size_t)(ngroups > 0 ? ngroups : 1) * sizeof(int64_t));
        int64_t acc = 0;
        for (int64_t g = 0; g < ngroups; ++g) { acc += token_count[g]; gend[g] = acc; }
        if (gather_start) total = acc < rows ? acc : rows;
    }
    sq_ctx c = {x, dtype, n0, inner, C, row_stride, out, out_scale, smooth, smooth_len,
                gend, ngroups, gather_index,
                gather_start ? (int64_t)gather_start[0] : 0, gather_len, rows, total};
    parallel_for(rows, nthreads, sq_range, &c);
    free(gend);
    return 0;
}

/* ------------------------------------------------------------------ single_query_cached_kv_attn (D12) */

typedef struct {
    const void* q; int q_dtype; int64_t q_st, q_sh;      /* q rows [T, Hq, D], element strides */
    const float* qs; int qs_mode; int64_t qs_st, qs_sh, qs_groups;  /* D17 q scales */
    const int32_t* cu; int64_t S, T;                     /* cu_seq_q [B + 1], or S tokens each */
    const void* kc; const void* vc; int c_dtype;         /* caches [NB, Hkv, BS, krow / vrow] */
    int v_ch;                                            /* DT_I4: V pairs channels (else rows) */
    int64_t NB, Hkv, BS, D, Dv, krow, vrow, Hq, MB, B;
    int64_t bt_heads;                                    /* D17: 0, Hkv or Hq block-table rows */
    const float* ks; const float* vs; int smode;         /* 0 none, 1 token, 2 channel, 3 group */
    int64_t ks_sb, ks_sh, vs_sb, vs_sh;                  /* per-token scale strides */
    const int32_t* bt; const int32_t* lens;
    const float* alibi; const float* sink; int64_t window; double scale;
    const void* mask; int mask_dtype; int64_t mask_len, m_sb, m_ss;  /* D16, or mask NULL */
    double* out; double* lse;                            /* [T, Hq, Dv], [T, Hq] */
} sqa_ctx;

/* Key channel d (< D) of row `row` of page blk, KV head hk: the first D of the row's krow. */
static double key_val(const sqa_ctx* c, int64_t blk, int64_t hk, int64_t row, int64_t d) {
    const int64_t r = (blk * c->Hkv + hk) * c->BS + row;
    if (c->c_dtype == DT_I8 || c->c_dtype == DT_F8E4M3 || c->c_dtype == DT_I4) {
        double code = c->c_dtype == DT_I4
                          ? (double)get_nibble(((const uint8_t*)c->kc)[r * c->krow + d / 2], (int)(d & 1))
                          : cache_code(c->kc, r * c->krow + d, c->c_dtype);
        if (c->smode == 1) return code * (double)c->ks[blk * c->ks_sb + hk * c->ks_sh + row];
        if (c->smode == 2) return code * (double)c->ks[hk * c->D + d];
        if (c->smode == 3) return code * (double)c->ks[r * (c->D / 32) + d / 32];
        return code;
    }
    return (double)load_elem(c->kc, r * c->krow + d, c->c_dtype);
}

/* Value channel d (< Dv): per-group V scales hold one number per 32 rows of a page and channel. */
static double value_val(const sqa_ctx* c, int64_t blk, int64_t hk, int64_t row, int64_t d) {
    const int64_t r = (blk * c->Hkv + hk) * c->BS + row;
    if (c->c_dtype == DT_I8 || c->c_dtype == DT_F8E4M3 || c->c_dtype == DT_I4) {
        double code;
        if (c->c_dtype != DT_I4)
            code = cache_code(c->vc, r * c->vrow + d, c->c_dtype);
        else if (c->v_ch)  /* D16: channel pairs */
            code = get_nibble(((const uint8_t*)c->vc)[r * c->vrow + d / 2], (int)(d & 1));
        else               /* D16: row pairs [NB, Hkv, BS / 2, vrow] */
            code = get_nibble(((const uint8_t*)c->vc)[((blk * c->Hkv + hk) * (c->BS / 2) + row / 2) * c->vrow + d],
                              (int)(row & 1));
        if (c->smode == 1) return code * (double)c->vs[blk * c->vs_sb + hk * c->vs_sh + row];
        if (c->smode == 2) return code * (double)c->vs[hk * c->Dv + d];
        if (c->smode == 3)
            return code * (double)c->vs[((blk * c->Hkv + hk) * (c->BS / 32) + row / 32) * c->Dv + d];
        return code;
    }
    return (double)load_elem(c->vc, r * c->vrow + d, c->c_dtype);
}

/* Query element d of row t, head hq (D17): the stored value, or for int8 / float8_e4m3fn q
 * the code times its scale -- per tensor (qs[0]), per (row, head) (qs[t * qs_st + hq * qs_sh])
 * or per group of D / qs_groups channels (qs[(t * Hq + hq) * qs_groups + d / (D / qs_groups)]);
 * the product is exact in double. */
static double q_val(const sqa_ctx* c, int64_t t, int64_t hq, int64_t d) {
    const int64_t e = t * c->q_st + hq * c->q_sh + d;
    if (c->q_dtype != DT_I8 && c->q_dtype != DT_F8E4M3) return (double)load_elem(c->q, e, c->q_dtype);
    double x = cache_code(c->q, e, c->q_dtype);
    if (c->qs_mode == 1) x *= (double)c->qs[0];
    else if (c->qs_mode == 2) x *= (double)c->qs[t * c->qs_st + hq * c->qs_sh];
    else if (c->qs_mode == 3) x *= (double)c->qs[(t * c->Hq + hq) * c->qs_groups + d / (c->D / c->qs_groups)];
    return x;
}

/* The sequence of query row t and the row's token index in it; -1 when no sequence holds t. */
static int64_t sqa_seq(const sqa_ctx* c, int64_t t, int64_t* s, int64_t* nq) {
    if (!c->cu) {
        *s = t % c->S;
        *nq = c->S;
        return t / c->S;
    }
    for (int64_t i = 0; i < c->B; ++i)
        if (c->cu[i] <= t && t < c->cu[i + 1]) {
            *s = t - c->cu[i];
            *nq = c->cu[i + 1] - c->cu[i];
            return i;
        }
    return -1;
}

static void sqa_range(void* p, int64_t lo, int64_t hi) {
    sqa_ctx* c = (sqa_ctx*)p;
    int64_t g = c->Hq / c->Hkv;
    double* s = (double*)malloc((size_t)(c->MB * c->BS > 0 ? c->MB * c->BS : 1) * sizeof(double));
    for (int64_t w = lo; w < hi; ++w) {             /* w = t * Hq + hq */
        int64_t t = w / c->Hq, hq = w % c->Hq, hk = hq / g, tok, nq;
        int64_t i = sqa_seq(c, t, &tok, &nq);
        if (i < 0) continue;                        /* a row no sequence holds: untouched */
        /* D17: the sequence's block table, or its KV head's / query head's row of it */
        const int32_t* btr = c->bt + (c->bt_heads == 0 ? i : i * c->bt_heads + (c->bt_heads == c->Hq ? hq : hk)) * c->MB;
        int64_t L = c->lens[i];
        if (L > c->MB * c->BS) L = c->MB * c->BS;
        const int64_t P = L - nq + tok;             /* the token's position: keys j <= P */
        const int64_t jend = P + 1 < L ? P + 1 : L;
        int64_t j0 = c->window >= 0 && P - c->window > 0 ? P - c->window : 0;
        double* o = c->out + w * c->Dv;
        for (int64_t d = 0; d < c->Dv; ++d) o[d] = 0.0;
        double m = c->sink ? (double)c->sink[hq] : -INFINITY;
        for (int64_t j = j0; j < jend; ++j) {
            int64_t blk = btr[j / c->BS], row = j % c->BS;
            if (blk < 0 || blk >= c->NB) { s[j] = -INFINITY; continue; }   /* missing page: masked */
            double acc = 0.0;
            for (int64_t d = 0; d < c->D; ++d)
                acc += q_val(c, t, hq, d) *
                       key_val(c, blk, hk, row, d);
            s[j] = c->scale * acc;
            if (c->alibi) s[j] += (double)c->alibi[i * c->Hq + hq] * (double)(j - P);
            if (c->mask && j >= L - c->mask_len)   /* D16: the last mask_len keys */
                s[j] += (double)load_elem(c->mask, i * c->m_sb + tok * c->m_ss + (j - (L - c->mask_len)),
                                          c->mask_dtype);
            if (s[j] > m) m = s[j];
        }
        double l = 0.0;
        if (m > -INFINITY) {
            if (c->sink) l = exp((double)c->sink[hq] - m);
            for (int64_t j = j0; j < jend; ++j) {
                if (s[j] == -INFINITY) continue;
                double pj = exp(s[j] - m);
                l += pj;
                int64_t blk = btr[j / c->BS], row = j % c->BS;
                for (int64_t d = 0; d < c->Dv; ++d) o[d] += pj * value_val(c, blk, hk, row, d);
            }
            for (int64_t d = 0; d < c->Dv; ++d) o[d] /= l;
        }
        if (c->lse) c->lse[w] = m > -INFINITY ? m + log(l) : -INFINITY;
    }
    free(s);
}

/* _ops.py:777-900, single_query_cached_kv_attn in double (D12):
 *   s_j = softmax_scale * sum_d q_d k_jd (+ alibi_slope[i, hq] * (j - P)),
 *   out = sum_j e^(s_j) v_j / (sum_j e^(s_j) (+ e^sink[hq])),  lse = log of that denominator,
 * for query token s of sequence i at position P = L - nq + s (L = context_lens[i], nq its
 * query tokens) over keys j in [max(0, P - window_left), min(P, L - 1)] (all of [0, P] when
 * window_left < 0), key j at row j % BS of page block_tables[i, j / BS]: its first D channels
 * are k_j, the first Dv of the V cache's row (or of the same K row, _ops.py:828-831, when the
 * caller passes the K cache as V) v_j.  Int8 caches (and float8_e4m3fn caches, _ops.py:868,
 * their code the e4m3fn value) hold code * scale exactly, scale_mode 1:
 * per token, [NB, Hkv, BS] at blk * s_sb + hk * s_sh + row; 2: per channel [Hkv, D] / [Hkv,
 * Dv]; 3: per group (_ops.py:841-842), K [NB, Hkv, BS, D / 32] (one per token and 32
 * channels), V [NB, Hkv, BS / 32, Dv] (one per 32 rows of a page and channel); other caches
 * the stored value.  Query head hq reads KV head hq / (Hq / Hkv).  Query rows: q [T, Hq, D] with row t
 * at t * q_st; cu_seq_q null: S tokens per sequence, sequence i's at rows i S .. i S + S - 1
 * (T = B S); else rows cu_seq_q[i] .. cu_seq_q[i + 1] - 1 (rows of no sequence untouched).
 * No key: out 0, lse = sink or -inf.  out [T, Hq, Dv], lse [T, Hq].
 * DT_I4 caches (D16): k_row / v_row count bytes; K pairs channels, V pairs the rows of a page
 * ([NB, Hkv, BS / 2, v_row], v_ch 0) or channels (v_ch 1).  mask (D16, nullable): element
 * i * mask_sb + s * mask_ss + m of mask_dtype (F32 / F16 / BF16) is added to the logit of key
 * L - mask_len + m of query token s of sequence i.
 * D17: q of DT_I8 / DT_F8E4M3 holds codes with q_scale (q_scale_mode 1 per tensor, 2 per
 * (row, head) at t * qs_st + hq * qs_sh, 3 per group of D / qs_groups channels, contiguous
 * [T, Hq, qs_groups]); bt_heads 0: block_tables [B, max_blocks]; Hkv or Hq: [B, bt_heads,
 * max_blocks], the row of the query head's KV head or of the query head itself. */
int oracle_cached_kv_attn(const void* q, int q_dtype, int64_t q_st, int64_t q_sh,
                          const float* q_scale, int q_scale_mode, int64_t qs_st, int64_t qs_sh,
                          int64_t qs_groups, const int32_t* cu_seq_q, int64_t S, int64_t T,
                          const void* k_cache, const void* v_cache, int cache_dtype, int v_ch,
                          int64_t NB, int64_t Hkv, int64_t BS, int64_t D, int64_t Dv,
                          int64_t k_row, int64_t v_row,
                          const float* k_scale, const float* v_scale, int scale_mode,
                          int64_t ks_sb, int64_t ks_sh, int64_t vs_sb, int64_t vs_sh,
                          const int32_t* block_tables, int64_t max_blocks, int64_t bt_heads,
                          const int32_t* context_lens, int64_t B, int64_t Hq,
                          const float* alibi, const float* sink, const void* mask,
                          int mask_dtype, int64_t mask_len, int64_t mask_sb, int64_t mask_ss,
                          int64_t window_left, double softmax_scale, double* out, double* lse,
                          int nthreads) {
    const int quant = cache_dtype == DT_I8 || cache_dtype == DT_F8E4M3 || cache_dtype == DT_I4;
    const int qquant = q_dtype == DT_I8 || q_dtype == DT_F8E4M3;
    if (qquant && (q_scale_mode < 1 || q_scale_mode > 3 || !q_scale ||
                   (q_scale_mode == 3 && (qs_groups <= 0 || D % qs_groups != 0))))
        return -3;
    if (bt_heads != 0 && bt_heads != Hkv && bt_heads != Hq) return -1;
    if ((!qquant && elem_size(q_dtype) == 0) || (!quant && elem_size(cache_dtype) == 0))
        return -2;
    if (quant && (scale_mode < 1 || scale_mode > 3)) return -3;
    if (B < 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || BS <= 0 || D <= 0 || Dv <= 0 ||
        (cache_dtype != DT_I4 && (k_row < D || v_row < Dv)) || max_blocks < 0 || T < 0 ||
        (!cu_seq_q && (S <= 0 || T != B * S)))
        return -1;
    if (quant && scale_mode == 3 && (D % 32 != 0 || BS % 32 != 0)) return -1;
    if (cache_dtype == DT_I4 && (k_row * 2 < D || (v_ch ? v_row * 2 < Dv : (v_row < Dv || BS % 2 != 0))))
        return -1;
    if (mask && (mask_len < 0 || (mask_dtype != DT_F32 && mask_dtype != DT_F16 && mask_dtype != DT_BF16)))
        return -1;
    sqa_ctx c = {q, q_dtype, q_st, q_sh, q_scale, qquant ? q_scale_mode : 0, qs_st, qs_sh, qs_groups,
                 cu_seq_q, S, T, k_cache, v_cache, cache_dtype,
                 cache_dtype == DT_I4 && v_ch, NB, Hkv,
                 BS, D, Dv, k_row, v_row, Hq, max_blocks, B, bt_heads, k_scale, v_scale,
                 quant ? scale_mode : 0, ks_sb, ks_sh, vs_sb, vs_sh,
                 block_tables, context_lens, alibi, sink, window_left, softmax_scale,
                 mask, mask_dtype, mask_len, mask_sb, mask_ss, out, lse};
    parallel_for(T * Hq, nthreads, sqa_range, &c);
    return 0;
}

/* One query token per sequence (q [B, Hq, D], row i at i * q_sb): oracle_cached_kv_attn with
 * S = 1 and no sink.  out [B, Hq, D], lse [B, Hq]. */
int oracle_single_query_attn(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                             const void* k_cache, const void* v_cache, int cache_dtype,
                             int64_t NB, int64_t Hkv, int64_t BS, int64_t D,
                             const float* k_scale, const float* v_scale, int scale_mode,
                             const int32_t* block_tables, int64_t max_blocks,
                             const int32_t* context_lens, int64_t B, int64_t Hq,
                             const float* alibi, int64_t window_left, double softmax_scale,
                             double* out, double* lse, int nthreads) {
    if (scale_mode == 3) return -3;
    if (cache_dtype == DT_I4 || q_dtype == DT_I8 || q_dtype == DT_F8E4M3) return -2;
    return oracle_cached_kv_attn(q, q_dtype, q_sb, q_sh, NULL, 0, 0, 0, 0, NULL, 1, B < 0 ? 0 : B,
                                 k_cache, v_cache, cache_dtype, 0, NB, Hkv, BS, D, D, D, D,
                                 k_scale, v_scale, scale_mode, Hkv * BS, BS, Hkv * BS, BS,
                                 block_tables, max_blocks, 0, context_lens, B, Hq, alibi, NULL,
                                 NULL, 0, 0, 0, 0, window_left, softmax_scale, out, lse, nthreads);
}
