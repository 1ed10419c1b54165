/*
 * torch_mlu_ops.h -- C++ torch API of the quantized paged-KV-cache path, MI355X build.
 *
 * Same namespace, names and parameter lists as the reference's prototypes
 * (reference include/torch_mlu_ops.h:21-22 namespace tmo::torch_api), restricted to the
 * ops of this path.  The implementations (domesticated_torch_mlu_ops_amd/csrc/
 * torch_api.cpp) validate shapes/dtypes, take the current HIP stream of the tensors' device
 * and call the plain C ABI of tmo_hip.h; they are registered as the CUDA-key (HIP on ROCm)
 * kernels of the torch_mlu_ops::* ops.  All tensors are caller-owned and written in place;
 * nothing here allocates.
 */
#ifndef CSRC_TORCH_API_TORCH_MLU_OPS_H_
#define CSRC_TORCH_API_TORCH_MLU_OPS_H_

#include <cstdint>
#include <optional>
#include <string>

#include "torch/extension.h"

namespace tmo {
namespace torch_api {

/* reference include/torch_mlu_ops.h:143-148 */
void reshape_paged_cache(torch::Tensor &k,
                         const c10::optional<torch::Tensor> &v,
                         torch::Tensor &k_cache,
                         const c10::optional<torch::Tensor> &v_cache,
                         const torch::Tensor &slot_mapping,
                         bool direction);

/* reference include/torch_mlu_ops.h:176-182 */
void quant_to_paged_cache(const torch::Tensor &k,
                          const c10::optional<torch::Tensor> &v,
                          torch::Tensor &k_cache,
                          const c10::optional<torch::Tensor> &v_cache,
                          torch::Tensor &k_cache_scale,
                          const c10::optional<torch::Tensor> &v_cache_scale,
                          const torch::Tensor &slot_mapping);

/* reference include/torch_mlu_ops.h:184-192 (int8 and float8_e4m3fn caches) */
void offline_quant_to_paged_cache(const torch::Tensor &k,
                                  const c10::optional<torch::Tensor> &v,
                                  const c10::optional<torch::Tensor> &k_cache_scale_per_channel,
                                  const c10::optional<torch::Tensor> &v_cache_scale_per_channel,
                                  const torch::Tensor &slot_mapping,
                                  torch::Tensor &k_cache,
                                  const c10::optional<torch::Tensor> &v_cache,
                                  double k_cache_scale_per_tensor,
                                  double v_cache_scale_per_tensor);

/* reference include/torch_mlu_ops.h:562-585 (norm_type "rmsnorm", paged high-precision
 * caches: unquantised, or int8 with dynamic per-token / static per-channel scales) */
void fused_rope(at::Tensor &qkv,
                at::Tensor &key_cache_hp,
                at::Tensor &value_cache_hp,
                const c10::optional<at::Tensor> &key_cache_lp,
                const c10::optional<at::Tensor> &value_cache_lp,
                const at::Tensor &sin_table,
                const at::Tensor &cos_table,
                const at::Tensor &position_ids,
                const at::Tensor &gamma,
                const c10::optional<at::Tensor> &k_beta,
                const c10::optional<at::Tensor> &key_scale_hp,
                const c10::optional<at::Tensor> &value_scale_hp,
                const c10::optional<at::Tensor> &key_scale_lp,
                const c10::optional<at::Tensor> &value_scale_lp,
                const c10::optional<at::Tensor> &cache_bs_id_hp,
                const c10::optional<at::Tensor> &cache_seq_offsets_hp,
                const c10::optional<at::Tensor> &cache_bs_id_lp,
                const c10::optional<at::Tensor> &cache_seq_offsets_lp,
                const c10::optional<at::Tensor> &slot_mapping_hp,
                const c10::optional<at::Tensor> &slot_mapping_lp,
                const std::string &norm_type,
                c10::SymInt rope_dim_offset,
                const double eps,
                const c10::optional<at::Tensor> &q_gamma = c10::nullopt);

/* reference include/torch_mlu_ops.h:334-350 (int8 "dynamic_per_token", act_mode "none") */
void scaled_quantize(const at::Tensor &x,
                     const at::Tensor &output,
                     const c10::optional<at::Tensor> &output_scale,
                     const c10::optional<at::Tensor> &x_scale,
                     const c10::optional<at::Tensor> &x_zero,
                     const c10::optional<at::Tensor> &m_list,
                     const c10::optional<at::Tensor> &gather_index,
                     const c10::optional<at::Tensor> &gather_index_start_position,
                     const c10::optional<at::Tensor> &scale_upper_bound,
                     const std::string &quant_mode,
                     const std::string &act_mode,
                     double active_coef,
                     bool is_gated,
                     int64_t quant_bit_size = 8,
                     bool need_output_scale_trans = false,
                     const c10::optional<at::Tensor> &output_reduced = c10::nullopt,
                     int64_t group_size = 1);

/* reference include/torch_mlu_ops.h:650-661 (quant_mode 0 and 1, quant_bit 8) */
void dequant_from_paged_cache(at::Tensor &key,
                              const c10::optional<at::Tensor> &value,
                              const at::Tensor &key_cache,
                              const c10::optional<at::Tensor> &value_cache,
                              const at::Tensor &key_cache_quant_scale,
                              const c10::optional<at::Tensor> &value_cache_quant_scale,
                              const at::Tensor &context_lengths,
                              const c10::SymInt max_context_len,
                              const c10::optional<at::Tensor> &context_seq_offset,
                              const at::Tensor &block_tables,
                              const int64_t quant_mode,
                              const int64_t quant_bit);

/* reference include/torch_mlu_ops.h:132-141 */
void reshape_linear_cache(const at::Tensor &key,
                          const c10::optional<at::Tensor> &value,
                          at::Tensor &key_cache,
                          const c10::optional<at::Tensor> &value_cache,
                          const at::Tensor &context_lengths,
                          const c10::SymInt max_context_len,
                          bool packed,
                          const c10::optional<at::Tensor> &context_seq_offset,
                          const c10::optional<at::Tensor> &cache_bs_id,
                          const c10::optional<at::Tensor> &cache_seqlen_offset);

/* reference include/torch_mlu_ops.h:194-206 */
void quant_to_linear_cache(const at::Tensor &key,
                           const c10::optional<at::Tensor> &value,
                           at::Tensor &key_cache,
                           const c10::optional<at::Tensor> &value_cache,
                           at::Tensor &key_cache_scale,
                           const c10::optional<at::Tensor> &value_cache_scale,
                           const at::Tensor &context_lengths,
                           const c10::SymInt max_context_len,
                           bool packed,
                           const c10::optional<at::Tensor> &context_seq_offset,
                           const c10::optional<at::Tensor> &cache_bs_id,
                           const c10::optional<at::Tensor> &cache_seqlen_offset,
                           const int64_t quant_bit);

/* reference include/torch_mlu_ops.h:208-222 */
void offline_quant_to_linear_cache(const at::Tensor &key,
                                   const c10::optional<at::Tensor> &value,
                                   at::Tensor &key_cache,
                                   const c10::optional<at::Tensor> &value_cache,
                                   const c10::optional<at::Tensor> &key_cache_scale,
                                   const c10::optional<at::Tensor> &value_cache_scale,
                                   const at::Tensor &context_lengths,
                                   const c10::SymInt max_context_len,
                                   const int64_t quant_mode,
                                   const bool packed,
                                   const c10::optional<at::Tensor> &context_seq_offset,
                                   const c10::optional<at::Tensor> &cache_bs_id,
                                   const c10::optional<at::Tensor> &cache_seqlen_offset,
                                   double key_cache_scale_per_tensor,
                                   double value_cache_scale_per_tensor);

/* reference include/torch_mlu_ops.h:636-648 */
void dequant_from_linear_cache(at::Tensor &key,
                               const c10::optional<at::Tensor> &value,
                               const at::Tensor &key_cache,
                               const c10::optional<at::Tensor> &value_cache,
                               const at::Tensor &key_quant_scale,
                               const c10::optional<at::Tensor> &value_quant_scale,
                               const at::Tensor &context_lengths,
                               const c10::SymInt max_context_len,
                               const c10::optional<at::Tensor> &context_seq_offset,
                               const c10::optional<at::Tensor> &cache_bs_id,
                               const c10::optional<at::Tensor> &cache_seq_offset,
                               const int64_t quant_mode,
                               const int64_t quant_bit);

/* reference include/torch_mlu_ops.h:663-671 */
void reshape_from_cache(at::Tensor &key,
                        const c10::optional<at::Tensor> &value,
                        const at::Tensor &key_cache,
                        const c10::optional<at::Tensor> &value_cache,
                        const at::Tensor &context_lengths,
                        c10::SymInt max_context_len,
                        const c10::optional<at::Tensor> &context_seq_offset,
                        const c10::optional<at::Tensor> &block_tables,
                        const c10::optional<at::Tensor> &cache_seq_offset);

/* reference include/torch_mlu_ops.h:107-130 */
void single_query_cached_kv_attn(const torch::Tensor &q_ori,
                                 const torch::Tensor &k_cache,
                                 const torch::Tensor &output,
                                 const torch::Tensor &block_tables,
                                 const torch::Tensor &context_lens,
                                 const c10::optional<torch::Tensor> &v_cache,
                                 const c10::optional<torch::Tensor> &output_lse,
                                 const c10::optional<torch::Tensor> &q_quant_scale,
                                 const c10::optional<torch::Tensor> &k_cache_quant_scale,
                                 const c10::optional<torch::Tensor> &v_cache_quant_scale,
                                 const c10::optional<torch::Tensor> &out_quant_scale,
                                 const c10::optional<torch::Tensor> &alibi_slopes,
                                 const c10::optional<torch::Tensor> &mask,
                                 const std::string &compute_dtype,
                                 c10::SymInt max_context_len,
                                 c10::SymInt windows_size_left,
                                 c10::SymInt windows_size_right,
                                 double softmax_scale,
                                 bool return_lse,
                                 int64_t kv_cache_quant_bit_size,
                                 const c10::optional<torch::Tensor> &cu_seq_q = c10::nullopt,
                                 c10::SymInt max_seq_q = -1,
                                 const c10::optional<torch::Tensor> &sink = c10::nullopt);

}  // namespace torch_api
}  // namespace tmo

#endif  // CSRC_TORCH_API_TORCH_MLU_OPS_H_
