/*
 * tmo_hip.h -- plain C ABI of the MI355X (gfx950) quantized paged-KV-cache library
 * (libtmo_hip.so).
 *
 * These entry points replace the device side of torch_mlu_ops' hot path: the closed
 * MLU kernels that the unshipped native extension `_TMOC` dispatches to behind the
 * C++ prototypes of reference include/torch_mlu_ops.h.  Each function cites the
 * prototype and the Python wrapper it stands behind.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HBM).  Tensors laid out [T, H, D] are addressed with
 *     element strides for the token and head dims; the last dim is contiguous.
 *     Paged caches are contiguous [num_blocks, num_heads, block_size, head_size]
 *     (reference KVFormat.NB_HN_BS_HS, _ops.py:1301-1310); per-token scales are
 *     contiguous [num_blocks, num_heads, block_size] fp32.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Work is enqueued on it;
 *     nothing synchronises, nothing allocates, no global mutable state: calls are
 *     reentrant and thread-safe across streams.
 *   - The return value is TMO_OK (0) or a negative tmo_status.  Arguments are validated
 *     before anything is enqueued; a failed call writes no device memory.
 *   - slot < 0 in slot_mapping means "skip this token" (_ops.py:1264); a slot at or past
 *     num_blocks*block_size is skipped the same way rather than written out of bounds.
 */
#ifndef TMO_HIP_H_
#define TMO_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMO_HIP_ABI_VERSION 17

/* element types */
enum tmo_dtype {
    TMO_DTYPE_F32 = 0,
    TMO_DTYPE_F16 = 1,
    TMO_DTYPE_BF16 = 2,
    TMO_DTYPE_I8 = 3,
    TMO_DTYPE_F8E4M3 = 4, /* float8_e4m3fn: 1-4-3, bias 7, no infinities, max 448 */
    TMO_DTYPE_I4 = 5      /* int8 storage of signed 4-bit pairs: the even element of a pair in
                           * the high nibble, the odd one in the low nibble */
};

/* return codes */
enum tmo_status {
    TMO_OK = 0,
    TMO_ERR_INVALID_ARGUMENT = -1, /* null pointer, negative/zero size, bad stride */
    TMO_ERR_UNSUPPORTED_DTYPE = -2,
    TMO_ERR_UNSUPPORTED_MODE = -3, /* quant_mode / quant_bit outside the int8 path */
    TMO_ERR_LAUNCH = -4,           /* the HIP launch itself failed */
    TMO_ERR_SCRATCH_TOO_SMALL = -5 /* the call needs more than the library's static scratch */
};

/* ABI version of the loaded library (TMO_HIP_ABI_VERSION at build time). */
int tmo_hip_abi_version(void);

/* Static, human-readable text for a tmo_status value. */
const char* tmo_hip_status_string(int status);

/*
 * reshape_paged_cache -- byte-exact scatter (direction == 0) of k/v[T, H, D] rows into the
 * paged caches at slot_mapping, or gather (direction != 0) of the same rows back.
 * Replaces tmo::torch_api::reshape_paged_cache (reference include/torch_mlu_ops.h:143-148),
 * called by torch_mlu_ops.reshape_paged_cache (reference _ops.py:1251-1294).
 * dtype: any tmo_dtype (caches have the dtype of k/v).  v and v_cache are both NULL or
 * both non-NULL.
 */
int tmo_hip_reshape_paged_cache(void* k, void* v,
                                int64_t k_stride_token, int64_t k_stride_head,
                                int64_t v_stride_token, int64_t v_stride_head,
                                void* k_cache, void* v_cache,
                                const int32_t* slot_mapping,
                                int64_t num_tokens, int64_t num_heads, int64_t head_size,
                                int64_t num_blocks, int64_t block_size,
                                int dtype, int direction, void* stream);

/*
 * quant_to_paged_cache -- dynamic per-(token, head) quantisation of k/v[T, H, D] into the
 * paged caches.  cache_dtype I8: scale = fp32(max|row|) / 127 (IEEE), code = RNE(row / scale)
 * clamped to [-128, 127]; cache_dtype F8E4M3: scale = fp32(max|row|) / 448, code =
 * e4m3fn_RNE(clip(row / scale, -448, 448)); an all-zero row gives scale 0 and codes 0.
 * Codes go to cache[slot / block_size, h, slot % block_size, :] and the scale to the same
 * [.., h, ..] position of the scale pages.
 * Replaces tmo::torch_api::quant_to_paged_cache (reference include/torch_mlu_ops.h:176-182),
 * called by torch_mlu_ops.quant_to_paged_cache (reference _ops.py:1511-1565).
 * dtype: F32, F16 or BF16 (of k and v).  v, v_cache, v_cache_scale: all NULL or all set.
 */
int tmo_hip_quant_to_paged_cache(const void* k, const void* v,
                                 int64_t k_stride_token, int64_t k_stride_head,
                                 int64_t v_stride_token, int64_t v_stride_head,
                                 void* k_cache, void* v_cache,
                                 float* k_cache_scale, float* v_cache_scale,
                                 const int32_t* slot_mapping,
                                 int64_t num_tokens, int64_t num_heads, int64_t head_size,
                                 int64_t num_blocks, int64_t block_size,
                                 int dtype, int cache_dtype, void* stream);

/*
 * offline_quant_to_paged_cache -- static quantisation of k/v[T, H, D] into the paged caches
 * with caller-given scales: q = RN(fp32(x) / s) (IEEE divide), stored as
 * clip(RNE(q), -128, 127) in an int8 cache or as float8_e4m3fn(clip(q, -448, 448)) (round to
 * nearest even) in an fp8 cache, at cache[slot / block_size, h, slot % block_size, :].
 * s = k_scale_channel[h * head_size + d] when k_scale_channel is set (per channel, [H, D] fp32
 * contiguous), else k_scale_tensor (per tensor); likewise for v.  No scales are written.
 * Scales must be finite and non-zero (other values give unspecified codes, never a fault).
 * Replaces tmo::torch_api::offline_quant_to_paged_cache (reference
 * include/torch_mlu_ops.h:184-192), called by torch_mlu_ops.offline_quant_to_paged_cache
 * (reference _ops.py:1639-1706).
 * dtype: F32, F16 or BF16 (of k and v); cache_dtype: I8 or F8E4M3 (both caches).  v and
 * v_cache: both NULL or both set; v_scale_channel must be NULL without v.
 */
int tmo_hip_offline_quant_to_paged_cache(const void* k, const void* v,
                                         int64_t k_stride_token, int64_t k_stride_head,
                                         int64_t v_stride_token, int64_t v_stride_head,
                                         void* k_cache, void* v_cache,
                                         const float* k_scale_channel,
                                         const float* v_scale_channel,
                                         float k_scale_tensor, float v_scale_tensor,
                                         const int32_t* slot_mapping,
                                         int64_t num_tokens, int64_t num_heads, int64_t head_size,
                                         int64_t num_blocks, int64_t block_size,
                                         int dtype, int cache_dtype, void* stream);

/*
 * fused_rope_paged -- one pass over qkv [num_tokens, q_heads + 2 kv_heads, head_size]
 * (contiguous, token t = b * seq_len + s at rotary position position_ids[b] + s).  norm_type 0
 * (rmsnorm): RMS-normalise Q (when q_gamma is set) and K per head with eps and gamma
 * [head_size], then rotate; norm_type 1 (layernorm): rotate, then layer-normalise K with
 * k_gamma and an optional k_beta (two-pass mean / variance over the same chunk order, see
 * below; q_gamma is ignored).  The rotation is the fold rotary
 * embedding over [rope_offset, rope_offset + rope_dim) with rows of sin_table / cos_table
 * [table_rows, table_stride] (a position outside the table leaves the row unrotated), write Q
 * back into qkv, and store K and V rows at slot_mapping into [num_blocks, kv_heads, block_size,
 * head_size] pages: scale_mode 0 stores them in qkv's dtype; 1 quantises to int8 with a
 * dynamic per-(token, head) scale written to k_scale / v_scale [num_blocks, kv_heads,
 * block_size]; 2 quantises to int8 with static per-channel scales read from [kv_heads,
 * head_size].  fp32 arithmetic, one final rounding; the sum of squares is taken over
 * 8-element chunks in order, then a balanced tree over the chunks; 1/rms = RN(1 / RN(sqrt(
 * RN(RN(ss / head_size) + eps)))).
 * Layernorm: mean = RN(s1 / head_size) over the chunked sum s1 of the rotated row, var =
 * RN(s2 / head_size) over the chunked sum of RN(d * d), d = RN(x - mean), out = RN(RN(d *
 * RN(1 / RN(sqrt(RN(var + eps))))) * gamma) (+ beta, rounded).
 * Replaces tmo::torch_api::fused_rope (reference include/torch_mlu_ops.h:562-585) with
 * paged high-precision caches, called by torch_mlu_ops.fused_rope
 * (reference _ops.py:3469-3601) and torch_mlu_ops.fused_rmsnorm_rope_store_paged_cache
 * (reference _ops.py:6356-6423).
 * dtype: F16 or BF16 (qkv, tables, gammas); head_size <= 512; num_tokens <= batch * seq_len.
 */
int tmo_hip_fused_rope_paged(void* qkv, int64_t num_tokens, int64_t seq_len,
                             int64_t q_heads, int64_t kv_heads, int64_t head_size,
                             const void* sin_table, const void* cos_table,
                             int64_t table_rows, int64_t table_stride,
                             int64_t rope_dim, int64_t rope_offset,
                             const int32_t* position_ids, int64_t batch,
                             const void* k_gamma, const void* k_beta, const void* q_gamma,
                             float eps, int norm_type,
                             void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                             int scale_mode, const int32_t* slot_mapping,
                             int64_t num_blocks, int64_t block_size, int dtype, void* stream);

/*
 * fused_rope_linear -- fused_rope_paged's arithmetic with linear high-precision caches
 * k_cache / v_cache [max_batch, kv_heads, cache_len, head_size] as the target: token s of
 * sequence b (token t = b * seq_len + s) is stored at cache batch cb = cache_bs_id[b] (b when
 * cache_bs_id is NULL), position cache_seq_offsets[b] + s (s when cache_seq_offsets is NULL);
 * rows whose cb is outside [0, max_batch) or whose position is outside [0, cache_len) are not
 * stored (Q is still written back).  Dynamic scales (scale_mode 1) are [max_batch, kv_heads,
 * cache_len]; static ones (2) [kv_heads, head_size].  max_batch * cache_len must fit an int32.
 * Replaces tmo::torch_api::fused_rope (reference include/torch_mlu_ops.h:562-585) with
 * cache_bs_id_hp / cache_seq_offsets_hp, called by torch_mlu_ops.fused_rope (reference
 * _ops.py:3469-3601, "reshape_linear_cache" branch of its Math).
 */
int tmo_hip_fused_rope_linear(void* qkv, int64_t num_tokens, int64_t seq_len,
                              int64_t q_heads, int64_t kv_heads, int64_t head_size,
                              const void* sin_table, const void* cos_table,
                              int64_t table_rows, int64_t table_stride,
                              int64_t rope_dim, int64_t rope_offset,
                              const int32_t* position_ids, int64_t batch,
                              const void* k_gamma, const void* k_beta, const void* q_gamma,
                              float eps, int norm_type,
                              void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                              int scale_mode, const int32_t* cache_bs_id,
                              const int32_t* cache_seq_offsets, int64_t max_batch,
                              int64_t cache_len, int dtype, void* stream);

/*
 * dequant_from_paged_cache -- gathers each sequence's pages through block_tables and writes
 * out[begin_i + t, h, :] = RNE_out(fp32(code) * scale) for t < context_lengths[i], where
 * begin_i = context_seq_offset[i], or the exclusive prefix sum of context_lengths when
 * context_seq_offset is NULL.  quant_mode 0: scale [H, D] (per channel);
 * quant_mode 1: scale [num_blocks, H, block_size] (per token).  quant_bit must be 8.
 * Tokens at or past max_blocks_per_seq * block_size are not written; block-table entries
 * outside [0, num_blocks) and output rows outside [0, total_rows) are skipped.
 * max_context_len is accepted for the reference signature and not used: the reference math
 * (_ops.py:3749-3774) reads context_lengths only.
 * Replaces tmo::torch_api::dequant_from_paged_cache (reference include/torch_mlu_ops.h:650-661),
 * called by torch_mlu_ops.dequant_from_paged_cache (reference _ops.py:3734-3824).
 * out_dtype: F16, BF16 (or F32).  value, value_cache, value_scale: all NULL or all set.
 * cache_dtype: TMO_DTYPE_I8 (int8 codes, the reference's type, _ops.py:3803-3804) or
 * TMO_DTYPE_F8E4M3 (float8_e4m3fn values, as quant_to_paged_cache writes them; an extension:
 * out = RNE_out(fp32(e4m3 value) * scale)).  scale_dtype: TMO_DTYPE_F32 or TMO_DTYPE_BF16
 * (_ops.py:3805-3806; a bf16 scale widens to fp32 exactly, so the product is the same).
 * `workspace`: NULL (workspace_bytes 0), or device memory of at least
 * tmo_hip_dequant_workspace_bytes(...) bytes, 16-byte aligned, used by this call only (calls
 * that share one workspace must be ordered on a stream).  With it the call runs as a small
 * page-list kernel followed by the main kernel, which is the faster layout on MI355X; without
 * it (or with a smaller one) a single kernel runs.  The results are identical.
 */
int tmo_hip_dequant_from_paged_cache(void* key, void* value,
                                     int64_t key_stride_token, int64_t key_stride_head,
                                     int64_t value_stride_token, int64_t value_stride_head,
                                     int64_t total_rows,
                                     const void* key_cache, const void* value_cache,
                                     const void* key_scale, const void* value_scale,
                                     const int32_t* context_lengths,
                                     const int32_t* context_seq_offset,
                                     const int32_t* block_tables,
                                     int64_t batch, int64_t max_blocks_per_seq,
                                     int64_t max_context_len,
                                     int64_t num_blocks, int64_t num_heads,
                                     int64_t block_size, int64_t head_size,
                                     int quant_mode, int quant_bit, int out_dtype,
                                     int cache_dtype, int scale_dtype,
                                     void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes for tmo_hip_dequant_from_paged_cache's page-list path: 16 + 16 per page the
 * call can cover (batch * max_blocks_per_seq, rounded up to a multiple of 8); 0 when there is
 * nothing to do.  max_context_len is not used.  No reference counterpart (the MLU kernels take
 * none). */
int64_t tmo_hip_dequant_workspace_bytes(int64_t batch, int64_t max_blocks_per_seq,
                                        int64_t max_context_len, int64_t block_size);

/* Bytes of the static device scratch of tmo_hip_dequant_from_paged_cache_noalloc (per GPU). */
#define TMO_HIP_DEQUANT_SCRATCH_BYTES 4194304

/*
 * dequant_from_paged_cache_noalloc -- tmo_hip_dequant_from_paged_cache (same arguments and
 * results, the page-list path's workspace left out) for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference.  It allocates nothing: the page list lives in a static
 * device array of TMO_HIP_DEQUANT_SCRATCH_BYTES (4 MiB) that each GPU the library runs on holds
 * until the process ends, so batch * max_blocks_per_seq may be at most 262136 pages; a larger
 * call returns TMO_ERR_SCRATCH_TOO_SMALL before enqueueing anything (use the entry point above
 * with a workspace).  `stream` must belong to the current device.  Every call on one GPU
 * shares that array, and the entry point orders the calls on it: host threads enqueue one at
 * a time, and a call on a stream other than the previous call's makes its stream wait (on the
 * GPU, hipStreamWaitEvent) for the previous call's kernels.  A call made while its stream is
 * being captured into a HIP graph takes no event operation: the graph orders it, and two
 * graphs holding such calls must not be replayed at the same time on one GPU.
 */
int tmo_hip_dequant_from_paged_cache_noalloc(void* key, void* value,
                                             int64_t key_stride_token, int64_t key_stride_head,
                                             int64_t value_stride_token, int64_t value_stride_head,
                                             int64_t total_rows,
                                             const void* key_cache, const void* value_cache,
                                             const void* key_scale, const void* value_scale,
                                             const int32_t* context_lengths,
                                             const int32_t* context_seq_offset,
                                             const int32_t* block_tables,
                                             int64_t batch, int64_t max_blocks_per_seq,
                                             int64_t max_context_len,
                                             int64_t num_blocks, int64_t num_heads,
                                             int64_t block_size, int64_t head_size,
                                             int quant_mode, int quant_bit, int out_dtype,
                                             int cache_dtype, int scale_dtype, void* stream);

/*
 * scaled_quantize_per_token -- "dynamic_per_token" int8 quantisation with an optional smooth
 * vector, optional row gather and optional per-group (per-expert) smooth rows:
 *   src row r   = gather_index[start + r] (start = *gather_start or 0), or r without gather;
 *   smoothed    = RN(fp32(x[src, j, :]) * smooth_g)   (smooth_g = smooth row of r's group);
 *   scale[r, j] = fp32(max|smoothed|) / 127;  out[r, j, :] = RNE(smoothed / scale) clamped.
 * x is [n0, inner, C] (rows of C elements, `x_row_stride` elements apart, row (s, j) at
 * (s * inner + j) * x_row_stride).  smooth: NULL, length 1 (broadcast), length C, or
 * [num_groups, C] when token_count is given.  token_count [num_groups]: row r belongs to the
 * group g with prefix(g) <= r < prefix(g + 1); rows at or past sum(token_count) are not
 * written (with gather_start given, only sum(token_count) rows are produced).
 * out [out_rows, inner, C] int8 contiguous, out_scale [out_rows, inner] fp32.
 * Replaces tmo::torch_api::scaled_quantize (reference include/torch_mlu_ops.h:334-350) in
 * quant_mode "dynamic_per_token", act_mode "none", int8 output, called by
 * torch_mlu_ops.moe_quantize (reference _ops.py:3126-3253) and torch_mlu_ops.scaled_quantize
 * (reference _ops.py:4407-4492).
 * dtype: F32, F16 or BF16 (of x).
 */
int tmo_hip_scaled_quantize_per_token(const void* x, int64_t n0, int64_t inner,
                                      int64_t channels, int64_t x_row_stride,
                                      int8_t* out, float* out_scale,
                                      const float* smooth, int64_t smooth_len,
                                      const int32_t* token_count, int64_t num_groups,
                                      const int32_t* gather_index, int64_t gather_len,
                                      const int32_t* gather_start,
                                      int64_t out_rows, int dtype, void* stream);

/*
 * Linear caches [max_batch, num_heads, cache_len, head_size] (contiguous), one cache batch per
 * sequence.  Shared addressing of the five entry points below, for sequence i < batch:
 *   len_i  = min(context_lengths[i], max_context_len); with packed input context_lengths holds
 *            batch + 1 prefix offsets cu and len_i = min(cu[i + 1] - cu[i], max_context_len);
 *   token j < len_i is row start_i + j of the token-major tensor (rows x [num_heads,
 *            head_size] with the given element strides): start_i = context_seq_offset[i] if
 *            non-NULL, else cu[i] (packed input), i * seqlen (padded [batch, seqlen, H, D]
 *            input flattened to rows), or sum(len_k, k < i) for the outputs of the read ops;
 *   its cache position is cache_seq_offset[i] + j (0 + j when NULL) in cache batch
 *            cache_bs_id[i] (i when NULL; a negative id skips the sequence).
 * A token whose row, cache batch or position lies outside its tensor is skipped.  Different
 * sequences must not map to the same cache rows (write ops) or token rows (read ops), and
 * packed prefix offsets are non-decreasing.
 * Per-token scales are contiguous [max_batch, num_heads, cache_len] fp32.
 */

/*
 * reshape_linear_cache -- byte copy of key/value token rows into the linear caches.
 * Replaces tmo::torch_api::reshape_linear_cache (reference include/torch_mlu_ops.h:132-141),
 * called by torch_mlu_ops.reshape_linear_cache (reference _ops.py:1189-1249).
 * dtype: F32, F16, BF16 or I8 (caches have the dtype of key).  value and value_cache are
 * both NULL or both set.
 */
int tmo_hip_reshape_linear_cache(const void* key, const void* value,
                                 int64_t key_stride_token, int64_t key_stride_head,
                                 int64_t value_stride_token, int64_t value_stride_head,
                                 int64_t rows, void* key_cache, void* value_cache,
                                 int64_t max_batch, int64_t num_heads, int64_t cache_len,
                                 int64_t head_size, const int32_t* context_lengths,
                                 int64_t batch, int64_t max_context_len, int packed,
                                 int64_t seqlen, const int32_t* context_seq_offset,
                                 const int32_t* cache_bs_id, const int32_t* cache_seqlen_offset,
                                 int dtype, void* stream);

/*
 * quant_to_linear_cache -- dynamic quantisation of key/value token rows into the linear
 * caches, per (token, head) or per group of head_size / group_num channels: int8 as
 * quant_to_paged_cache (scale = fp32(amax) / 127), or float8_e4m3fn with scale =
 * fp32(amax) / 448 and code = e4m3fn_RNE(clip(x / scale, -448, 448)) (all-zero group: scale 0,
 * codes +0).  Scales go to key_scale[b, h, pos, g] ([max_batch, H, cache_len, group_num]).
 * Replaces tmo::torch_api::quant_to_linear_cache (reference include/torch_mlu_ops.h:194-206),
 * called by torch_mlu_ops.quant_to_linear_cache (reference _ops.py:1708-1806).
 * dtype: F32, F16 or BF16; cache_dtype: I8 or F8E4M3; quant_bit: 8, or 4 with an I8 cache:
 * scale = RN(fp32(amax) / 7), code = clip(RNE(x / scale), -8, 7), two codes per byte with the
 * even element of a pair in the high nibble; key_cache [max_batch, H, cache_len, head_size / 2]
 * pairs channels, value_cache [max_batch, H, cache_len / 2, head_size] pairs cache positions
 * (cache_len even; a position written without its partner keeps the partner's nibble, so two
 * sequences of one call must not write the two positions of one pair).  4-bit needs head_size
 * % 8 == 0 and <= 512, 16-byte aligned token rows, a 4-byte aligned key_cache, an 8-byte aligned
 * value_cache and, for group_num > 1, head_size / 8 a power of two that group_num divides into
 * powers of two; otherwise TMO_ERR_UNSUPPORTED_MODE.
 */
int tmo_hip_quant_to_linear_cache(const void* key, const void* value,
                                  int64_t key_stride_token, int64_t key_stride_head,
                                  int64_t value_stride_token, int64_t value_stride_head,
                                  int64_t rows, void* key_cache, void* value_cache,
                                  float* key_scale, float* value_scale, int64_t max_batch,
                                  int64_t num_heads, int64_t cache_len, int64_t head_size,
                                  int64_t group_num, const int32_t* context_lengths,
                                  int64_t batch, int64_t max_context_len, int packed,
                                  int64_t seqlen, const int32_t* context_seq_offset,
                                  const int32_t* cache_bs_id,
                                  const int32_t* cache_seqlen_offset, int quant_bit, int dtype,
                                  int cache_dtype, void* stream);

/*
 * offline_quant_to_linear_cache -- static quantisation (code = clip(RNE(fp32(x) / s), -128,
 * 127), or e4m3fn_RNE(clip(fp32(x) / s, -448, 448)), IEEE quotients) into the linear caches.
 * quant_mode 0: key_scale [num_heads, head_size] per channel; 1: [num_heads, cache_len] per
 * head and cache position; 2 or 3: the per-tensor scalars (key_scale may be NULL).
 * Replaces tmo::torch_api::offline_quant_to_linear_cache (reference
 * include/torch_mlu_ops.h:208-222), called by torch_mlu_ops.offline_quant_to_linear_cache
 * (reference _ops.py:1808-1919).  dtype: F32, F16 or BF16; cache_dtype: I8 or F8E4M3.
 */
int tmo_hip_offline_quant_to_linear_cache(const void* key, const void* value,
                                          int64_t key_stride_token, int64_t key_stride_head,
                                          int64_t value_stride_token, int64_t value_stride_head,
                                          int64_t rows, void* key_cache, void* value_cache,
                                          const float* key_scale, const float* value_scale,
                                          float key_scale_per_tensor,
                                          float value_scale_per_tensor, int quant_mode,
                                          int64_t max_batch, int64_t num_heads,
                                          int64_t cache_len, int64_t head_size,
                                          const int32_t* context_lengths, int64_t batch,
                                          int64_t max_context_len, int packed, int64_t seqlen,
                                          const int32_t* context_seq_offset,
                                          const int32_t* cache_bs_id,
                                          const int32_t* cache_seqlen_offset, int dtype,
                                          int cache_dtype, void* stream);

/*
 * dequant_from_linear_cache -- out[row, h, :] = RN_out(fp32(code) * scale) from the int8
 * linear caches; quant_mode 0: key_scale [num_heads, head_size]; 1: per-token
 * [max_batch, num_heads, cache_len].  context_lengths holds [batch] lengths.
 * Replaces tmo::torch_api::dequant_from_linear_cache (reference
 * include/torch_mlu_ops.h:636-648), called by torch_mlu_ops.dequant_from_linear_cache
 * (reference _ops.py:3642-3732).  out_dtype: F16, BF16 (or F32); quant_bit: 8, or 4 for the
 * caches quant_to_linear_cache writes with quant_bit 4 (key_cache [max_batch, H, cache_len,
 * head_size / 2], value_cache [max_batch, H, cache_len / 2, head_size]; nibbles sign-extended,
 * the even element in the high nibble), with the same shape limits.
 */
int tmo_hip_dequant_from_linear_cache(void* key, void* value,
                                      int64_t key_stride_token, int64_t key_stride_head,
                                      int64_t value_stride_token, int64_t value_stride_head,
                                      int64_t rows, const int8_t* key_cache,
                                      const int8_t* value_cache, const float* key_scale,
                                      const float* value_scale, int64_t max_batch,
                                      int64_t num_heads, int64_t cache_len, int64_t head_size,
                                      const int32_t* context_lengths, int64_t batch,
                                      int64_t max_context_len,
                                      const int32_t* context_seq_offset,
                                      const int32_t* cache_bs_id,
                                      const int32_t* cache_seq_offset, int quant_mode,
                                      int quant_bit, int out_dtype, void* stream);

/*
 * reshape_from_cache -- byte copy of cache rows back to token-major key/value rows.
 * Without block_tables the cache is linear [num_blocks = max_batch, H, block_rows = cache_len,
 * D] and sequence i reads cache batch i; with block_tables [batch, max_blocks] position pos of
 * sequence i is row pos % block_rows of page block_tables[i, pos / block_rows] (paged mode;
 * a [batch, 1] table is the linear mode with the table naming the cache batch).  Position =
 * cache_seq_offset[i] + j.  context_lengths holds [batch] lengths.
 * Replaces tmo::torch_api::reshape_from_cache (reference include/torch_mlu_ops.h:663-671),
 * called by torch_mlu_ops.reshape_from_cache (reference _ops.py:3898-3969).
 * dtype: F32, F16, BF16 or I8.
 */
int tmo_hip_reshape_from_cache(void* key, void* value,
                               int64_t key_stride_token, int64_t key_stride_head,
                               int64_t value_stride_token, int64_t value_stride_head,
                               int64_t rows, const void* key_cache, const void* value_cache,
                               int64_t num_blocks, int64_t num_heads, int64_t block_rows,
                               int64_t head_size, const int32_t* context_lengths, int64_t batch,
                               int64_t max_context_len, const int32_t* context_seq_offset,
                               const int32_t* block_tables, int64_t max_blocks,
                               const int32_t* cache_seq_offset, int dtype, void* stream);

/*
 * cached_kv_attn -- single_query_cached_kv_attn for the query tokens of each sequence over its
 * paged KV cache.  Sequence i has nq_i query tokens, the last nq_i of its L = context_lens[i]
 * positions: token s sits at P = L - nq_i + s.  For query head hq of token s (KV head
 * hk = hq / (Hq / Hkv)),
 *   s_j = softmax_scale * q . k_j (+ alibi_slopes[i, hq] * (j - P)),
 *   out = sum_j e^(s_j) v_j / (sum_j e^(s_j) (+ e^sink[hq])),  lse = ln of that denominator,
 * over keys j in [max(0, P - window_left), P] (from 0 when window_left < 0): causal within
 * the new tokens.  Key j sits at row j % block_size of page block_tables[i, j / block_size];
 * pages outside [0, num_blocks) are masked.  A token with no key: out 0, lse = sink or -inf.
 * Query rows, two forms:
 *   cu_seq_q null: seq_q tokens per sequence; token s of sequence i at element
 *     i * q_stride_batch + s * q_stride_token + hq * q_stride_head (q [batch, seq_q, Hq, D]);
 *   cu_seq_q [batch + 1] int32: sequence i's tokens are rows cu_seq_q[i] .. cu_seq_q[i+1] - 1
 *     of a [total_q, Hq, D] q, row t at t * q_stride_token (q_stride_batch unused); seq_q is
 *     an upper bound of the counts (tokens past it are not computed) and rows outside
 *     [0, total_q) are skipped.
 * out (out_dtype, head_size_v channels) and lse (nullable, fp32) are addressed the same way
 * with their own strides.  q of F32 / F16 / BF16 takes out_dtype = q_dtype.  q of
 * TMO_DTYPE_I8 / TMO_DTYPE_F8E4M3 holds codes (_ops.py:853-856, 868; quantised caches only):
 * q = code * q_scale, with q_scale (fp32 or bf16, q_scale_dtype) by q_scale_mode 1 per tensor
 * (one value), 2 per token and head (element i * q_scale_stride_batch + token row *
 * q_scale_stride_token + hq * q_scale_stride_head, addressed like q), 3 per group of
 * head_size / q_scale_groups channels (that element plus d / group, the strides counting
 * groups); out_dtype F32, F16 or BF16.
 * block_tables: [batch, max_blocks] (block_table_heads 0), or sparse-KV tables [batch,
 * block_table_heads, max_blocks] with block_table_heads = Hkv (each KV head its own pages) or
 * Hq (each query head its own; _ops.py:834).
 * Caches [num_blocks, Hkv, block_size, k_cache_dim / v_cache_dim] contiguous: k_j is the first
 * head_size channels of its K row, v_j the first head_size_v of its V row -- of its K row when
 * v_cache is null (K and V in one cache, reference _ops.py:828-831; v_cache_dim unused).
 * Quantised caches -- int8 codes (cache_dtype TMO_DTYPE_I8) or float8_e4m3fn values
 * (TMO_DTYPE_F8E4M3; _ops.py:868, kv_cache_quant_bit_size 8 "int8/float8_e4m3fn") -- hold
 * k = code * scale, with fp32 or bf16 scales (scale_dtype TMO_DTYPE_F32 / TMO_DTYPE_BF16,
 * _ops.py:872; ignored for other caches) by scale_mode:
 *   1 per token: [num_blocks, Hkv, block_size] with element strides (scale_stride_block,
 *     scale_stride_head, 1) -- any strides in the first two dims (_ops.py:838);
 *   2 per channel: [Hkv, head_size] (K) and [Hkv, head_size_v] (V), contiguous;
 *   3 per group (_ops.py:841-842): K [num_blocks, Hkv, block_size, head_size / 32] (one per
 *     token and 32 channels), V [num_blocks, Hkv, block_size / 32, head_size_v] (one per 32 rows
 *     of a page and channel), contiguous; head_size and block_size multiples of 32.
 * int4 caches (cache_dtype TMO_DTYPE_I4; _ops.py:826-829, 852, "int8(pairwise-int4)" :868)
 * hold two signed 4-bit codes per byte -- the even element of a pair in the high nibble, the
 * odd one in the low nibble (the reference's unpack `byte >> 4`, `byte << 4 >> 4`,
 * _ops.py:3681-3682) -- with the same scale modes.  Row lengths then count bytes: K
 * [num_blocks, Hkv, block_size, k_cache_dim >= head_size / 2] pairs adjacent channels; V
 * pairs adjacent rows of a page, [num_blocks, Hkv, block_size / 2, v_cache_dim >=
 * head_size_v] with block_size even (v_pair_channels 0: the layout whose last dim is
 * head_size_v, as the reference's own output allocation reads it, _ops.py:887, and
 * fused_rope's v_cache_lp, _ops.py:3534), or adjacent channels, [num_blocks, Hkv, block_size,
 * v_cache_dim >= head_size_v / 2] (v_pair_channels 1).  v_cache must not be null.
 * Other caches are of q's dtype (F32, F16 or BF16).  sink (nullable): [Hq] fp32 natural-log
 * logits.  mask (nullable; _ops.py:860): logit terms of mask_dtype (F32, F16 or BF16) for the
 * last mask_len keys of each sequence -- key j >= L - mask_len of query token s of sequence i
 * gets s_j += mask[i * mask_stride_batch + s * mask_stride_token + j - (L - mask_len)] after
 * softmax_scale and ALiBi (L clamped to the block table; -inf removes the key).  Head sizes:
 * head_size up to 4096, head_size_v up to 512; the MFMA kernels take K and V head sizes of 64,
 * 128 or 256 (equal, with cache rows of that many elements -- int4: K rows of head_size / 2
 * bytes, V pairing rows) and per-token or per-channel scales, a VALU kernel the rest (int4
 * V pairing channels and per-query-head tables with grouped heads included).
 * Arithmetic: fp32 accumulation (MFMA with bf16/f16 operands: int8 codes and e4m3fn values are
 * exact; q and the probabilities are split into two operands when one is not exact), softmax
 * in fp32.
 * splits > 1 divides each sequence's keys over that many workgroups per KV head; it needs
 * `workspace` of at least tmo_hip_cached_kv_attn_workspace_bytes(...) bytes (device memory).
 * max_context_len <= 0 (negative included) means an unknown maximum: one split per sequence
 * unless `splits` says otherwise; it never limits the keys read.
 * Replaces tmo::torch_api::single_query_cached_kv_attn (reference
 * include/torch_mlu_ops.h:107-130) without out quantisation (out_quant_scale is reserved
 * there), called by
 * torch_mlu_ops.single_query_cached_kv_attn (reference _ops.py:777-900; q forms :824,
 * cu_seq_q / max_seq_q :860-861, sink :864).
 */
int tmo_hip_cached_kv_attn(const void* q, int64_t q_stride_batch, int64_t q_stride_token,
                           int64_t q_stride_head, const void* q_scale, int q_scale_mode,
                           int q_scale_dtype, int64_t q_scale_stride_batch,
                           int64_t q_scale_stride_token, int64_t q_scale_stride_head,
                           int64_t q_scale_groups, const int32_t* cu_seq_q, int64_t seq_q,
                           int64_t total_q, const void* k_cache, const void* v_cache,
                           int64_t k_cache_dim, int64_t v_cache_dim, const void* k_scale,
                           const void* v_scale, int scale_mode, int scale_dtype,
                           int64_t k_scale_stride_block,
                           int64_t k_scale_stride_head, int64_t v_scale_stride_block,
                           int64_t v_scale_stride_head, const int32_t* block_tables,
                           int64_t max_blocks, int64_t block_table_heads,
                           const int32_t* context_lens,
                           const float* alibi_slopes, const float* sink, const void* mask,
                           int mask_dtype, int64_t mask_len, int64_t mask_stride_batch,
                           int64_t mask_stride_token, void* out,
                           int64_t out_stride_batch, int64_t out_stride_token,
                           int64_t out_stride_head, float* lse, int64_t lse_stride_batch,
                           int64_t lse_stride_token, int64_t lse_stride_head, int64_t batch,
                           int64_t num_q_heads, int64_t num_kv_heads, int64_t head_size,
                           int64_t head_size_v, int64_t num_blocks, int64_t block_size,
                           int64_t max_context_len, int64_t window_left, float softmax_scale,
                           int q_dtype, int cache_dtype, int v_pair_channels, int out_dtype,
                           int64_t splits, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* Workspace bytes tmo_hip_cached_kv_attn needs for `splits` with up to seq_q tokens per
 * sequence (0 when splits <= 1). */
int64_t tmo_hip_cached_kv_attn_workspace_bytes(int64_t batch, int64_t num_kv_heads,
                                               int64_t num_q_heads, int64_t head_size_v,
                                               int64_t seq_q, int64_t splits);

/*
 * single_query_cached_kv_attn -- tmo_hip_cached_kv_attn with one query token per sequence
 * (seq_q 1, no cu_seq_q, no sink), separate K and V caches [num_blocks, Hkv, block_size,
 * head_size], fp32 scales, scale_mode 1 (contiguous per-token scales) or 2: q / out [batch, Hq, head_size]
 * rows with the given strides, lse (nullable) at i * lse_stride_seq + hq * lse_stride_head;
 * head_size up to 512.  Replaces the same reference interface for the decode step (reference
 * include/torch_mlu_ops.h:107-130, _ops.py:777-900).
 */
int tmo_hip_single_query_cached_kv_attn(const void* q, int64_t q_stride_seq, int64_t q_stride_head,
                                        const void* k_cache, const void* v_cache,
                                        const float* k_scale, const float* v_scale,
                                        int scale_mode, const int32_t* block_tables,
                                        int64_t max_blocks, const int32_t* context_lens,
                                        const float* alibi_slopes, void* out,
                                        int64_t out_stride_seq, int64_t out_stride_head,
                                        float* lse, int64_t lse_stride_seq,
                                        int64_t lse_stride_head, int64_t batch,
                                        int64_t num_q_heads, int64_t num_kv_heads,
                                        int64_t head_size, int64_t num_blocks,
                                        int64_t block_size, int64_t max_context_len,
                                        int64_t window_left, float softmax_scale, int q_dtype,
                                        int cache_dtype, int64_t splits, void* workspace,
                                        int64_t workspace_bytes, void* stream);

/* Workspace bytes tmo_hip_single_query_cached_kv_attn needs for `splits` (0 when splits <= 1);
 * max_context_len is not used. */
int64_t tmo_hip_attn_workspace_bytes(int64_t batch, int64_t num_kv_heads, int64_t num_q_heads,
                                     int64_t head_size, int64_t max_context_len, int64_t splits);

#ifdef __cplusplus
}
#endif

#endif /* TMO_HIP_H_ */
