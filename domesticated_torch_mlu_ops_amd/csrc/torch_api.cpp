// Thin PyTorch-ROCm glue: tmo::torch_api (include/torch_mlu_ops.h) over the plain C ABI of
// include/tmo_hip.h, and the torch_mlu_ops::* schemas with their HIP (CUDA-key) kernels.
//
// Each function validates everything on the host (shapes, dtypes, devices, contiguity),
// takes the current HIP stream of the tensors' device, and calls exactly one C-ABI entry
// point.  Errors surface as c10::Error (Python RuntimeError) before anything is enqueued.
// The schemas carry the alias/mutation annotations the reference's unshipped extension must
// have had (its Python wrappers return the written tensors in place: reference
// _ops.py:1290-1294, 1562-1565, 3821-3824, 3249-3253), so torch.compile functionalisation
// keeps the cache writes.
#include <algorithm>
#include <cmath>

#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include "tmo_hip.h"
#include "torch_mlu_ops.h"

namespace tmo {
namespace torch_api {
namespace {

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return TMO_DTYPE_F32;
    case at::kHalf: return TMO_DTYPE_F16;
    case at::kBFloat16: return TMO_DTYPE_BF16;
    case at::kChar: return TMO_DTYPE_I8;
    case at::kFloat8_e4m3fn: return TMO_DTYPE_F8E4M3;
    default: return -1;
  }
}

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

void check_status(int status, const char* op) {
  TORCH_CHECK(status == TMO_OK, "torch_mlu_ops::", op, ": ", tmo_hip_status_string(status),
              " (status ", status, ")");
}

void check_device(const at::Tensor& t, const at::Tensor& ref, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU (HIP) tensor, got ", t.device());
  TORCH_CHECK(t.device() == ref.device(), name, " is on ", t.device(), " but expected ",
              ref.device());
}

// [T, H, D] token-major rows with a contiguous last dim (k/v may be views into a fused qkv).
void check_rows(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.dim() == 3, name, " must be 3-D [tokens, heads, head_size], got ", t.sizes());
  TORCH_CHECK(t.size(2) <= 1 || t.stride(2) == 1, name, " must have a contiguous last dim");
  TORCH_CHECK(t.stride(0) >= 0 && t.stride(1) >= 0, name, " has negative strides");
}

void check_cache(const at::Tensor& c, const char* name) {
  TORCH_CHECK(c.dim() == 4, name, " must be 4-D [num_blocks, heads, block_size, head_size], got ",
              c.sizes());
  TORCH_CHECK(c.is_contiguous(), name, " must be contiguous");
}

}  // namespace

void reshape_paged_cache(torch::Tensor& k, const c10::optional<torch::Tensor>& v,
                         torch::Tensor& k_cache, const c10::optional<torch::Tensor>& v_cache,
                         const torch::Tensor& slot_mapping, bool direction) {
  check_rows(k, "k");
  check_cache(k_cache, "k_cache");
  check_device(k, k, "k");
  check_device(k_cache, k, "k_cache");
  check_device(slot_mapping, k, "slot_mapping");
  TORCH_CHECK(v.has_value() == v_cache.has_value(), "v and v_cache must both be given or both be None");
  const int dt = dtype_code(k.scalar_type());
  TORCH_CHECK(dt >= 0, "reshape_paged_cache: unsupported dtype ", k.scalar_type());
  TORCH_CHECK(k_cache.scalar_type() == k.scalar_type(), "k_cache dtype ", k_cache.scalar_type(),
              " must match k dtype ", k.scalar_type());
  const int64_t T = k.size(0), H = k.size(1), D = k.size(2);
  TORCH_CHECK(k_cache.size(1) == H && k_cache.size(3) == D, "k_cache ", k_cache.sizes(),
              " does not match k ", k.sizes());
  TORCH_CHECK(slot_mapping.scalar_type() == at::kInt && slot_mapping.dim() == 1 &&
                  slot_mapping.size(0) == T && slot_mapping.is_contiguous(),
              "slot_mapping must be a contiguous int32 [num_tokens] tensor");
  if (v.has_value()) {
    check_rows(*v, "v");
    check_cache(*v_cache, "v_cache");
    check_device(*v, k, "v");
    check_device(*v_cache, k, "v_cache");
    TORCH_CHECK(v->sizes() == k.sizes() && v->scalar_type() == k.scalar_type(), "v must match k");
    TORCH_CHECK(v_cache->sizes() == k_cache.sizes() && v_cache->scalar_type() == k.scalar_type(),
                "v_cache must match k_cache");
  }
  if (T == 0) return;
  c10::DeviceGuard guard(k.device());
  const int st = tmo_hip_reshape_paged_cache(
      k.data_ptr(), v ? v->data_ptr() : nullptr, k.stride(0), k.stride(1),
      v ? v->stride(0) : 0, v ? v->stride(1) : 0, k_cache.data_ptr(),
      v_cache ? v_cache->data_ptr() : nullptr, slot_mapping.data_ptr<int32_t>(), T, H, D,
      k_cache.size(0), k_cache.size(2), dt, direction ? 1 : 0, stream_of(k));
  check_status(st, "reshape_paged_cache");
}

void quant_to_paged_cache(const torch::Tensor& k, const c10::optional<torch::Tensor>& v,
                          torch::Tensor& k_cache, const c10::optional<torch::Tensor>& v_cache,
                          torch::Tensor& k_cache_scale,
                          const c10::optional<torch::Tensor>& v_cache_scale,
                          const torch::Tensor& slot_mapping) {
  check_rows(k, "k");
  check_cache(k_cache, "k_cache");
  check_device(k, k, "k");
  check_device(k_cache, k, "k_cache");
  check_device(k_cache_scale, k, "k_cache_scale");
  check_device(slot_mapping, k, "slot_mapping");
  const int dt = dtype_code(k.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F32 || dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "quant_to_paged_cache: k must be float, half or bfloat16, got ", k.scalar_type());
  const int cdt = dtype_code(k_cache.scalar_type());
  TORCH_CHECK(cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3,
              "quant_to_paged_cache: caches must be int8 or float8_e4m3fn, got ",
              k_cache.scalar_type());
  const int64_t T = k.size(0), H = k.size(1), D = k.size(2);
  const int64_t NB = k_cache.size(0), BS = k_cache.size(2);
  TORCH_CHECK(k_cache.size(1) == H && k_cache.size(3) == D, "k_cache ", k_cache.sizes(),
              " does not match k ", k.sizes());
  TORCH_CHECK(k_cache_scale.scalar_type() == at::kFloat && k_cache_scale.is_contiguous() &&
                  k_cache_scale.dim() == 3 && k_cache_scale.size(0) == NB &&
                  k_cache_scale.size(1) == H && k_cache_scale.size(2) == BS,
              "k_cache_scale must be a contiguous float32 [num_blocks, heads, block_size] tensor");
  TORCH_CHECK(slot_mapping.scalar_type() == at::kInt && slot_mapping.dim() == 1 &&
                  slot_mapping.size(0) == T && slot_mapping.is_contiguous(),
              "slot_mapping must be a contiguous int32 [num_tokens] tensor");
  const bool has_v = v.has_value();
  TORCH_CHECK(has_v == v_cache.has_value() && has_v == v_cache_scale.has_value(),
              "v, v_cache and v_cache_scale must all be given or all be None");
  if (has_v) {
    check_rows(*v, "v");
    check_cache(*v_cache, "v_cache");
    check_device(*v, k, "v");
    check_device(*v_cache, k, "v_cache");
    check_device(*v_cache_scale, k, "v_cache_scale");
    TORCH_CHECK(v->sizes() == k.sizes() && v->scalar_type() == k.scalar_type(), "v must match k");
    TORCH_CHECK(v_cache->sizes() == k_cache.sizes() &&
                    v_cache->scalar_type() == k_cache.scalar_type(),
                "v_cache must match k_cache");
    TORCH_CHECK(v_cache_scale->sizes() == k_cache_scale.sizes() &&
                    v_cache_scale->scalar_type() == at::kFloat && v_cache_scale->is_contiguous(),
                "v_cache_scale must match k_cache_scale");
  }
  if (T == 0) return;
  c10::DeviceGuard guard(k.device());
  const int st = tmo_hip_quant_to_paged_cache(
      k.data_ptr(), has_v ? v->data_ptr() : nullptr, k.stride(0), k.stride(1),
      has_v ? v->stride(0) : 0, has_v ? v->stride(1) : 0, k_cache.data_ptr(),
      has_v ? v_cache->data_ptr() : nullptr, k_cache_scale.data_ptr<float>(),
      has_v ? v_cache_scale->data_ptr<float>() : nullptr, slot_mapping.data_ptr<int32_t>(), T, H,
      D, NB, BS, dt, cdt, stream_of(k));
  check_status(st, "quant_to_paged_cache");
}

void offline_quant_to_paged_cache(const torch::Tensor& k, const c10::optional<torch::Tensor>& v,
                                  const c10::optional<torch::Tensor>& k_cache_scale_per_channel,
                                  const c10::optional<torch::Tensor>& v_cache_scale_per_channel,
                                  const torch::Tensor& slot_mapping, torch::Tensor& k_cache,
                                  const c10::optional<torch::Tensor>& v_cache,
                                  double k_cache_scale_per_tensor,
                                  double v_cache_scale_per_tensor) {
  check_rows(k, "k");
  check_cache(k_cache, "k_cache");
  check_device(k, k, "k");
  check_device(k_cache, k, "k_cache");
  check_device(slot_mapping, k, "slot_mapping");
  const int dt = dtype_code(k.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F32 || dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "offline_quant_to_paged_cache: k must be float, half or bfloat16, got ",
              k.scalar_type());
  const int cdt = dtype_code(k_cache.scalar_type());
  TORCH_CHECK(cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3,
              "offline_quant_to_paged_cache: caches must be int8 or float8_e4m3fn, got ",
              k_cache.scalar_type());
  const int64_t T = k.size(0), H = k.size(1), D = k.size(2);
  TORCH_CHECK(k_cache.size(1) == H && k_cache.size(3) == D, "k_cache ", k_cache.sizes(),
              " does not match k ", k.sizes());
  TORCH_CHECK(slot_mapping.scalar_type() == at::kInt && slot_mapping.dim() == 1 &&
                  slot_mapping.size(0) == T && slot_mapping.is_contiguous(),
              "slot_mapping must be a contiguous int32 [num_tokens] tensor");
  const bool has_v = v.has_value();
  TORCH_CHECK(has_v == v_cache.has_value(), "v and v_cache must both be given or both be None");
  TORCH_CHECK(has_v || !v_cache_scale_per_channel.has_value(),
              "v_cache_scale given without v");
  if (has_v) {
    check_rows(*v, "v");
    check_cache(*v_cache, "v_cache");
    check_device(*v, k, "v");
    check_device(*v_cache, k, "v_cache");
    TORCH_CHECK(v->sizes() == k.sizes() && v->scalar_type() == k.scalar_type(), "v must match k");
    TORCH_CHECK(v_cache->sizes() == k_cache.sizes() &&
                    v_cache->scalar_type() == k_cache.scalar_type(),
                "v_cache must match k_cache");
  }
  // per channel: a float32 [heads, head_size] tensor; per tensor: a finite non-zero number
  auto channel = [&](const c10::optional<torch::Tensor>& sc, const char* name) -> const float* {
    if (!sc.has_value()) return nullptr;
    check_device(*sc, k, name);
    TORCH_CHECK(sc->scalar_type() == at::kFloat && sc->is_contiguous() && sc->dim() == 2 &&
                    sc->size(0) == H && sc->size(1) == D,
                name, " must be a contiguous float32 [heads, head_size] tensor, got ",
                sc->scalar_type(), " ", sc->sizes());
    return sc->data_ptr<float>();
  };
  const float* kch = channel(k_cache_scale_per_channel, "k_cache_scale");
  const float* vch = channel(v_cache_scale_per_channel, "v_cache_scale");
  const float kt = static_cast<float>(k_cache_scale_per_tensor);
  const float vt = static_cast<float>(v_cache_scale_per_tensor);
  TORCH_CHECK(kch || (std::isfinite(kt) && kt != 0.0f),
              "k_cache_scale must be finite and non-zero, got ", k_cache_scale_per_tensor);
  TORCH_CHECK(!has_v || vch || (std::isfinite(vt) && vt != 0.0f),
              "v_cache_scale must be finite and non-zero, got ", v_cache_scale_per_tensor);
  if (T == 0) return;
  c10::DeviceGuard guard(k.device());
  const int st = tmo_hip_offline_quant_to_paged_cache(
      k.data_ptr(), has_v ? v->data_ptr() : nullptr, k.stride(0), k.stride(1),
      has_v ? v->stride(0) : 0, has_v ? v->stride(1) : 0, k_cache.data_ptr(),
      has_v ? v_cache->data_ptr() : nullptr, kch, vch, kt, vt, slot_mapping.data_ptr<int32_t>(),
      T, H, D, k_cache.size(0), k_cache.size(2), dt, cdt, stream_of(k));
  check_status(st, "offline_quant_to_paged_cache");
}

void fused_rope(at::Tensor& qkv, at::Tensor& key_cache_hp, at::Tensor& value_cache_hp,
                const c10::optional<at::Tensor>& key_cache_lp,
                const c10::optional<at::Tensor>& value_cache_lp, const at::Tensor& sin_table,
                const at::Tensor& cos_table, const at::Tensor& position_ids,
                const at::Tensor& gamma, const c10::optional<at::Tensor>& k_beta,
                const c10::optional<at::Tensor>& key_scale_hp,
                const c10::optional<at::Tensor>& value_scale_hp,
                const c10::optional<at::Tensor>& key_scale_lp,
                const c10::optional<at::Tensor>& value_scale_lp,
                const c10::optional<at::Tensor>& cache_bs_id_hp,
                const c10::optional<at::Tensor>& cache_seq_offsets_hp,
                const c10::optional<at::Tensor>& cache_bs_id_lp,
                const c10::optional<at::Tensor>& cache_seq_offsets_lp,
                const c10::optional<at::Tensor>& slot_mapping_hp,
                const c10::optional<at::Tensor>& slot_mapping_lp, const std::string& norm_type,
                c10::SymInt rope_dim_offset, const double eps,
                const c10::optional<at::Tensor>& q_gamma) {
  TORCH_CHECK(norm_type == "rmsnorm" || norm_type == "layernorm",
              "fused_rope: norm_type must be \"rmsnorm\" or \"layernorm\", got \"", norm_type,
              "\"");
  const bool layernorm = norm_type == "layernorm";
  TORCH_CHECK(!key_cache_lp && !value_cache_lp && !key_scale_lp && !value_scale_lp &&
                  !slot_mapping_lp && !cache_bs_id_lp && !cache_seq_offsets_lp,
              "fused_rope: low-precision (int4) caches are not supported by this build");
  // the target: paged caches through slot_mapping_hp, else linear caches [max_batch, kv_heads,
  // cache_len, head_size] through cache_bs_id_hp / cache_seq_offsets_hp (either may be None)
  const bool linear = !slot_mapping_hp.has_value();
  TORCH_CHECK(linear || (!cache_bs_id_hp && !cache_seq_offsets_hp),
              "fused_rope: pass slot_mapping_hp (paged caches) or cache_bs_id_hp / "
              "cache_seq_offsets_hp (linear caches), not both");
  TORCH_CHECK(layernorm || !k_beta.has_value(), "fused_rope: k_beta applies to layernorm only");
  check_device(qkv, qkv, "qkv");
  TORCH_CHECK(qkv.dim() == 4 && qkv.is_contiguous(),
              "qkv must be a contiguous [batch, seq_len, heads, head_size] tensor, got ",
              qkv.sizes());
  const int dt = dtype_code(qkv.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "fused_rope: qkv must be half or bfloat16, got ", qkv.scalar_type());
  const int64_t B = qkv.size(0), S = qkv.size(1), H = qkv.size(2), D = qkv.size(3);
  check_cache(key_cache_hp, "key_cache_hp");
  check_cache(value_cache_hp, "value_cache_hp");
  check_device(key_cache_hp, qkv, "key_cache_hp");
  check_device(value_cache_hp, qkv, "value_cache_hp");
  const int64_t NB = key_cache_hp.size(0), Hk = key_cache_hp.size(1), BS = key_cache_hp.size(2);
  TORCH_CHECK(key_cache_hp.size(3) == D && value_cache_hp.sizes() == key_cache_hp.sizes() &&
                  value_cache_hp.scalar_type() == key_cache_hp.scalar_type(),
              "key/value caches must be [num_blocks, kv_heads, block_size, head_size] (or "
              "[max_batch, kv_heads, cache_len, head_size]) alike");
  TORCH_CHECK(H > 2 * Hk, "qkv has ", H, " heads, fewer than 2 * kv_heads + 1");
  const int64_t Hq = H - 2 * Hk;
  int mode = 0;
  float* ks = nullptr;
  float* vs = nullptr;
  if (key_scale_hp.has_value() || value_scale_hp.has_value()) {
    TORCH_CHECK(key_scale_hp.has_value() && value_scale_hp.has_value(),
                "key_scale and value_scale must both be given or both be None");
    TORCH_CHECK(key_cache_hp.scalar_type() == at::kChar,
                "fused_rope: quantised caches must be int8, got ", key_cache_hp.scalar_type());
    for (const at::Tensor* sc : {&*key_scale_hp, &*value_scale_hp}) {
      check_device(*sc, qkv, "scale");
      TORCH_CHECK(sc->scalar_type() == at::kFloat && sc->is_contiguous(),
                  "fused_rope: scales must be contiguous float32");
    }
    if (key_scale_hp->dim() == 3) {
      mode = 1;  // dynamic per (token, head): written
      TORCH_CHECK(key_scale_hp->size(0) == NB && key_scale_hp->size(1) == Hk &&
                      key_scale_hp->size(2) == BS &&
                      value_scale_hp->sizes() == key_scale_hp->sizes(),
                  "dynamic scales must be [num_blocks, kv_heads, block_size] ([max_batch, kv_heads, cache_len] for linear caches)");
    } else {
      mode = 2;  // static per channel: read
      TORCH_CHECK(key_scale_hp->dim() == 2 && key_scale_hp->size(0) == Hk &&
                      key_scale_hp->size(1) == D && value_scale_hp->sizes() == key_scale_hp->sizes(),
                  "static scales must be [kv_heads, head_size]");
    }
    ks = key_scale_hp->data_ptr<float>();
    vs = value_scale_hp->data_ptr<float>();
  } else {
    TORCH_CHECK(key_cache_hp.scalar_type() == qkv.scalar_type(),
                "fused_rope: unquantised caches must have qkv's dtype");
  }
  for (const at::Tensor* tb : {&sin_table, &cos_table}) {
    check_device(*tb, qkv, "sin/cos table");
    TORCH_CHECK(tb->dim() == 2 && tb->scalar_type() == qkv.scalar_type() &&
                    (tb->size(1) <= 1 || tb->stride(1) == 1),
                "sin/cos tables must be [rotary_seq, rope_dim] of qkv's dtype, last dim contiguous");
  }
  TORCH_CHECK(sin_table.sizes() == cos_table.sizes() && sin_table.stride(0) == cos_table.stride(0),
              "sin and cos tables must have the same shape and row stride");
  const int64_t rope_dim = sin_table.size(1);
  const int64_t off = rope_dim_offset.expect_int();
  TORCH_CHECK(rope_dim % 2 == 0 && off >= 0 && off + rope_dim <= D,
              "rope_dim (", rope_dim, ") must be even and rope_dim + rope_dim_offset <= head_size");
  check_device(position_ids, qkv, "position_ids");
  TORCH_CHECK(position_ids.scalar_type() == at::kInt && position_ids.dim() == 1 &&
                  position_ids.size(0) == B && position_ids.is_contiguous(),
              "position_ids must be a contiguous int32 [batch] tensor");
  // layernorm normalises K only (after its rotation); q_gamma belongs to the rmsnorm branch
  // (reference _ops.py:3501-3509) and is not read there
  const at::Tensor* qg = (!layernorm && q_gamma) ? &*q_gamma : nullptr;
  const at::Tensor* kb = (layernorm && k_beta) ? &*k_beta : nullptr;
  for (const at::Tensor* g : {&gamma, qg, kb}) {
    if (!g) continue;
    check_device(*g, qkv, "gamma");
    TORCH_CHECK(g->dim() == 1 && g->size(0) == D && g->scalar_type() == qkv.scalar_type() &&
                    g->is_contiguous(),
                "gammas and k_beta must be contiguous [head_size] tensors of qkv's dtype");
  }
  TORCH_CHECK(D <= 512, "fused_rope: head_size must be <= 512");
  if (linear) {
    for (const c10::optional<at::Tensor>* t : {&cache_bs_id_hp, &cache_seq_offsets_hp}) {
      if (!t->has_value()) continue;
      check_device(**t, qkv, "cache_bs_id / cache_seq_offsets");
      TORCH_CHECK((*t)->scalar_type() == at::kInt && (*t)->dim() == 1 && (*t)->size(0) == B &&
                      (*t)->is_contiguous(),
                  "cache_bs_id_hp / cache_seq_offsets_hp must be contiguous int32 [batch] tensors");
    }
    TORCH_CHECK(NB * BS <= 0x7fffffffLL,
                "fused_rope: linear caches of more than 2^31 - 1 rows per head are not supported");
  } else {
    const at::Tensor& slot = *slot_mapping_hp;
    check_device(slot, qkv, "slot_mapping");
    TORCH_CHECK(slot.scalar_type() == at::kInt && slot.numel() == B * S && slot.is_contiguous(),
                "slot_mapping must be a contiguous int32 tensor of batch * seq_len entries");
  }
  if (B * S == 0) return;
  c10::DeviceGuard guard(qkv.device());
  auto i32 = [](const c10::optional<at::Tensor>& t) -> const int32_t* {
    return t.has_value() ? t->data_ptr<int32_t>() : nullptr;
  };
  const int st =
      linear ? tmo_hip_fused_rope_linear(
                   qkv.data_ptr(), B * S, S, Hq, Hk, D, sin_table.data_ptr(), cos_table.data_ptr(),
                   sin_table.size(0), sin_table.stride(0), rope_dim, off,
                   position_ids.data_ptr<int32_t>(), B, gamma.data_ptr(),
                   kb ? kb->data_ptr() : nullptr, qg ? qg->data_ptr() : nullptr,
                   static_cast<float>(eps), layernorm ? 1 : 0, key_cache_hp.data_ptr(),
                   value_cache_hp.data_ptr(), ks, vs, mode, i32(cache_bs_id_hp),
                   i32(cache_seq_offsets_hp), NB, BS, dt, stream_of(qkv))
             : tmo_hip_fused_rope_paged(
                   qkv.data_ptr(), B * S, S, Hq, Hk, D, sin_table.data_ptr(), cos_table.data_ptr(),
                   sin_table.size(0), sin_table.stride(0), rope_dim, off,
                   position_ids.data_ptr<int32_t>(), B, gamma.data_ptr(),
                   kb ? kb->data_ptr() : nullptr, qg ? qg->data_ptr() : nullptr,
                   static_cast<float>(eps), layernorm ? 1 : 0, key_cache_hp.data_ptr(),
                   value_cache_hp.data_ptr(), ks, vs, mode, slot_mapping_hp->data_ptr<int32_t>(),
                   NB, BS, dt, stream_of(qkv));
  check_status(st, "fused_rope");
}

void dequant_from_paged_cache(at::Tensor& key, const c10::optional<at::Tensor>& value,
                              const at::Tensor& key_cache,
                              const c10::optional<at::Tensor>& value_cache,
                              const at::Tensor& key_cache_quant_scale,
                              const c10::optional<at::Tensor>& value_cache_quant_scale,
                              const at::Tensor& context_lengths, const c10::SymInt max_context_len,
                              const c10::optional<at::Tensor>& context_seq_offset,
                              const at::Tensor& block_tables, const int64_t quant_mode,
                              const int64_t quant_bit) {
  TORCH_CHECK(quant_mode == 0 || quant_mode == 1,
              "dequant_from_paged_cache: quant_mode must be 0 (per-channel) or 1 (per-token), got ",
              quant_mode);
  TORCH_CHECK(quant_bit == 8, "dequant_from_paged_cache: only quant_bit 8 is supported, got ",
              quant_bit);
  check_rows(key, "key");
  check_cache(key_cache, "key_cache");
  check_device(key, key, "key");
  check_device(key_cache, key, "key_cache");
  check_device(key_cache_quant_scale, key, "key_cache_quant_scale");
  check_device(context_lengths, key, "context_lengths");
  check_device(block_tables, key, "block_tables");
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16 || dt == TMO_DTYPE_F32,
              "dequant_from_paged_cache: key must be half, bfloat16 or float, got ",
              key.scalar_type());
  // int8 codes (the reference's type, _ops.py:3803-3804), or the float8_e4m3fn pages that
  // quant_to_paged_cache / offline_quant_to_paged_cache write
  const int cdt = dtype_code(key_cache.scalar_type());
  TORCH_CHECK(cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3,
              "key_cache must be int8 or float8_e4m3fn, got ", key_cache.scalar_type());
  const int64_t NB = key_cache.size(0), H = key_cache.size(1), BS = key_cache.size(2),
                D = key_cache.size(3);
  TORCH_CHECK(key.size(1) == H && key.size(2) == D, "key ", key.sizes(), " does not match key_cache ",
              key_cache.sizes());
  // scales: float32 or bfloat16 (_ops.py:3805-3806), both tensors of one type
  const at::ScalarType sdt = key_cache_quant_scale.scalar_type();
  auto check_scale = [&](const at::Tensor& s, const char* name) {
    TORCH_CHECK((s.scalar_type() == at::kFloat || s.scalar_type() == at::kBFloat16) &&
                    s.scalar_type() == sdt && s.is_contiguous(),
                name, " must be a contiguous float32 or bfloat16 tensor (K and V scales of one type)");
    if (quant_mode == 0) {
      TORCH_CHECK(s.dim() == 2 && s.size(0) == H && s.size(1) == D, name,
                  " must be [heads, head_size] for quant_mode 0, got ", s.sizes());
    } else {
      TORCH_CHECK(s.dim() == 3 && s.size(0) == NB && s.size(1) == H && s.size(2) == BS, name,
                  " must be [num_blocks, heads, block_size] for quant_mode 1, got ", s.sizes());
    }
  };
  check_scale(key_cache_quant_scale, "key_cache_quant_scale");
  TORCH_CHECK(context_lengths.scalar_type() == at::kInt && context_lengths.dim() == 1 &&
                  context_lengths.is_contiguous(),
              "context_lengths must be a contiguous int32 [batch] tensor");
  const int64_t B = context_lengths.size(0);
  TORCH_CHECK(block_tables.scalar_type() == at::kInt && block_tables.dim() == 2 &&
                  block_tables.size(0) == B && block_tables.is_contiguous(),
              "block_tables must be a contiguous int32 [batch, max_blocks] tensor");
  if (context_seq_offset.has_value()) {
    check_device(*context_seq_offset, key, "context_seq_offset");
    TORCH_CHECK(context_seq_offset->scalar_type() == at::kInt && context_seq_offset->dim() == 1 &&
                    context_seq_offset->size(0) == B && context_seq_offset->is_contiguous(),
                "context_seq_offset must be a contiguous int32 [batch] tensor");
  }
  const bool has_v = value.has_value();
  TORCH_CHECK(has_v == value_cache.has_value() && has_v == value_cache_quant_scale.has_value(),
              "value, value_cache and value_cache_quant_scale must all be given or all be None");
  if (has_v) {
    check_rows(*value, "value");
    check_cache(*value_cache, "value_cache");
    check_device(*value, key, "value");
    check_device(*value_cache, key, "value_cache");
    check_device(*value_cache_quant_scale, key, "value_cache_quant_scale");
    TORCH_CHECK(value->sizes() == key.sizes() && value->scalar_type() == key.scalar_type(),
                "value must match key");
    TORCH_CHECK(value_cache->sizes() == key_cache.sizes() &&
                    value_cache->scalar_type() == key_cache.scalar_type(),
                "value_cache must match key_cache");
    check_scale(*value_cache_quant_scale, "value_cache_quant_scale");
  }
  // max_context_len is not used by the dequant (the reference math reads context_lengths)
  const int64_t max_ctx = max_context_len.expect_int();
  if (B == 0 || key.size(0) == 0) return;
  c10::DeviceGuard guard(key.device());
  const int64_t ws_bytes =
      tmo_hip_dequant_workspace_bytes(B, block_tables.size(1), max_ctx, BS);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes}, key.options().dtype(at::kByte));
  const int st = tmo_hip_dequant_from_paged_cache(
      key.data_ptr(), has_v ? value->data_ptr() : nullptr, key.stride(0), key.stride(1),
      has_v ? value->stride(0) : 0, has_v ? value->stride(1) : 0, key.size(0),
      key_cache.data_ptr(), has_v ? value_cache->data_ptr() : nullptr,
      key_cache_quant_scale.data_ptr(), has_v ? value_cache_quant_scale->data_ptr() : nullptr,
      context_lengths.data_ptr<int32_t>(),
      context_seq_offset ? context_seq_offset->data_ptr<int32_t>() : nullptr,
      block_tables.data_ptr<int32_t>(), B, block_tables.size(1), max_ctx, NB, H, BS, D,
      (int)quant_mode, (int)quant_bit, dt, cdt,
      sdt == at::kBFloat16 ? TMO_DTYPE_BF16 : TMO_DTYPE_F32,
      ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(key));
  check_status(st, "dequant_from_paged_cache");
}

void scaled_quantize(const at::Tensor& x, const at::Tensor& output,
                     const c10::optional<at::Tensor>& output_scale,
                     const c10::optional<at::Tensor>& x_scale,
                     const c10::optional<at::Tensor>& x_zero,
                     const c10::optional<at::Tensor>& m_list,
                     const c10::optional<at::Tensor>& gather_index,
                     const c10::optional<at::Tensor>& gather_index_start_position,
                     const c10::optional<at::Tensor>& scale_upper_bound,
                     const std::string& quant_mode, const std::string& act_mode,
                     double active_coef, bool is_gated, int64_t quant_bit_size,
                     bool need_output_scale_trans,
                     const c10::optional<at::Tensor>& output_reduced, int64_t group_size) {
  (void)active_coef;
  (void)group_size;
  (void)scale_upper_bound;  // only meaningful for fp8 outputs (reference _ops.py:4426-4427)
  TORCH_CHECK(quant_mode == "dynamic_per_token",
              "scaled_quantize: only quant_mode 'dynamic_per_token' is implemented, got '",
              quant_mode, "'");
  TORCH_CHECK(act_mode == "none", "scaled_quantize: only act_mode 'none' is implemented, got '",
              act_mode, "'");
  TORCH_CHECK(!is_gated, "scaled_quantize: is_gated requires an activation (not implemented)");
  TORCH_CHECK(quant_bit_size == 8, "scaled_quantize: only quant_bit_size 8 is implemented");
  TORCH_CHECK(!need_output_scale_trans, "scaled_quantize: need_output_scale_trans (mx) is not implemented");
  TORCH_CHECK(!output_reduced.has_value(), "scaled_quantize: output_reduced is not implemented");
  TORCH_CHECK(!x_zero.has_value(), "scaled_quantize: zero is not supported, must pass None");
  TORCH_CHECK(output_scale.has_value(), "scaled_quantize: dynamic_per_token needs output_scale");
  check_device(x, x, "x");
  check_device(output, x, "output");
  check_device(*output_scale, x, "output_scale");
  const int dt = dtype_code(x.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F32 || dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "scaled_quantize: x must be float, half or bfloat16, got ", x.scalar_type());
  TORCH_CHECK(output.scalar_type() == at::kChar, "scaled_quantize: only int8 output is implemented, got ",
              output.scalar_type());
  TORCH_CHECK(output_scale->scalar_type() == at::kFloat && output_scale->is_contiguous(),
              "output_scale must be a contiguous float32 tensor");
  TORCH_CHECK(output.is_contiguous(), "output must be contiguous");
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dim");
  const int64_t C = x.size(-1);
  TORCH_CHECK(x.dim() == 1 || x.size(-1) <= 1 || x.stride(-1) == 1, "x must have a contiguous last dim");
  // Rows: x is [n0, inner..., C]; dims 0..-2 must collapse into one row index with a uniform
  // row stride ("continuous between 0 and -2 dimensions", reference _ops.py:3179).
  const int64_t n0 = x.dim() >= 2 ? x.size(0) : 1;
  int64_t inner = 1;
  for (int64_t d = 1; d + 1 < x.dim(); ++d) inner *= x.size(d);
  int64_t row_stride = -1, span = 1;
  for (int64_t d = x.dim() - 2; d >= 0; --d) {
    if (x.size(d) != 1) {
      if (row_stride < 0) row_stride = x.stride(d);
      TORCH_CHECK(x.stride(d) == row_stride * span, "x must be contiguous between dims 0 and -2");
    }
    span *= x.size(d);
  }
  if (row_stride < 0) row_stride = C;  // a single row
  TORCH_CHECK(row_stride >= C, "x rows overlap (row stride ", row_stride, " < ", C, ")");
  const float* smooth = nullptr;
  int64_t smooth_len = 0;
  if (x_scale.has_value()) {
    check_device(*x_scale, x, "smooth");
    TORCH_CHECK(x_scale->scalar_type() == at::kFloat && x_scale->is_contiguous(),
                "smooth must be a contiguous float32 tensor");
    smooth = x_scale->data_ptr<float>();
    if (m_list.has_value()) {
      TORCH_CHECK(x_scale->dim() == 2 && x_scale->size(0) == m_list->size(0) && x_scale->size(1) == C,
                  "smooth must be [groups, C] when token_count is given, got ", x_scale->sizes());
      smooth_len = C;
    } else {
      TORCH_CHECK(x_scale->numel() == C || x_scale->numel() == 1,
                  "smooth must have C or 1 elements, got ", x_scale->sizes());
      smooth_len = x_scale->numel();
    }
  }
  int64_t groups = 0;
  if (m_list.has_value()) {
    check_device(*m_list, x, "token_count");
    TORCH_CHECK(m_list->scalar_type() == at::kInt && m_list->dim() == 1 && m_list->is_contiguous() &&
                    m_list->size(0) > 0,
                "token_count must be a non-empty contiguous int32 [groups] tensor");
    groups = m_list->size(0);
  }
  int64_t rows = n0;
  int64_t gather_len = 0;
  if (gather_index.has_value()) {
    check_device(*gather_index, x, "gather_index");
    TORCH_CHECK(gather_index->scalar_type() == at::kInt && gather_index->dim() == 1 &&
                    gather_index->is_contiguous(),
                "gather_index must be a contiguous int32 [rows] tensor");
    gather_len = gather_index->size(0);
    rows = gather_len;
  }
  if (gather_index_start_position.has_value()) {
    TORCH_CHECK(gather_index.has_value(), "gather_index_start_position needs gather_index");
    check_device(*gather_index_start_position, x, "gather_index_start_position");
    TORCH_CHECK(gather_index_start_position->scalar_type() == at::kInt &&
                    gather_index_start_position->numel() == 1,
                "gather_index_start_position must be an int32 [1] tensor");
  }
  TORCH_CHECK(output.numel() == rows * inner * C, "output has ", output.numel(),
              " elements, expected ", rows * inner * C);
  TORCH_CHECK(output_scale->numel() == rows * inner, "output_scale has ", output_scale->numel(),
              " elements, expected ", rows * inner);
  if (rows == 0 || n0 == 0 || C == 0) return;
  c10::DeviceGuard guard(x.device());
  const int st = tmo_hip_scaled_quantize_per_token(
      x.data_ptr(), n0, inner, C, row_stride, output.data_ptr<int8_t>(),
      output_scale->data_ptr<float>(), smooth, smooth_len,
      m_list ? m_list->data_ptr<int32_t>() : nullptr, groups,
      gather_index ? gather_index->data_ptr<int32_t>() : nullptr, gather_len,
      gather_index_start_position ? gather_index_start_position->data_ptr<int32_t>() : nullptr, rows,
      dt, stream_of(x));
  check_status(st, "scaled_quantize");
}

// ------------------------------------------------------------------------------ linear caches

namespace {

// Token-major tensor of a linear-cache op as rows of [heads, head_size]: [T, H, D], or padded
// [B, S, H, D] (write ops) flattened to B * S rows.  A padded tensor whose batch stride is not
// S row strides is copied first (it is an input).
struct TokenRows {
  at::Tensor t;
  int64_t rows, st, sh, seqlen, H, D;
};

TokenRows token_rows(const at::Tensor& x, bool allow_padded, const char* name) {
  TokenRows r;
  if (x.dim() == 4 && allow_padded) {
    at::Tensor t = x;
    if (t.size(3) > 1 && t.stride(3) != 1) t = t.contiguous();
    if (t.stride(0) != t.size(1) * t.stride(1) || t.stride(1) < 0 || t.stride(2) < 0)
      t = t.contiguous();
    r.t = t;
    r.rows = t.size(0) * t.size(1);
    r.st = t.stride(1);
    r.sh = t.stride(2);
    r.seqlen = t.size(1);
    r.H = t.size(2);
    r.D = t.size(3);
    return r;
  }
  TORCH_CHECK(x.dim() == 3, name, " must be 3-D [tokens, heads, head_size]",
              allow_padded ? " or 4-D [batch, seqlen, heads, head_size]" : "", ", got ",
              x.sizes());
  check_rows(x, name);
  r.t = x;
  r.rows = x.size(0);
  r.st = x.stride(0);
  r.sh = x.stride(1);
  r.seqlen = 0;
  r.H = x.size(1);
  r.D = x.size(2);
  return r;
}

void check_linear_cache(const at::Tensor& c, const at::Tensor& ref, int64_t H, int64_t D,
                        const char* name) {
  check_device(c, ref, name);
  TORCH_CHECK(c.dim() == 4 && c.is_contiguous(), name,
              " must be a contiguous 4-D [max_batch, heads, cache_len, head_size] tensor, got ",
              c.sizes());
  TORCH_CHECK(c.size(1) == H && c.size(3) == D, name, " ", c.sizes(),
              " does not match the token rows' [heads, head_size] = [", H, ", ", D, "]");
}

// Optional int32 [n] tensor -> device pointer (NULL when absent).
const int32_t* i32_vec(const c10::optional<at::Tensor>& t, const at::Tensor& ref, int64_t n,
                       const char* name) {
  if (!t.has_value()) return nullptr;
  check_device(*t, ref, name);
  TORCH_CHECK(t->scalar_type() == at::kInt && t->dim() == 1 && t->size(0) == n &&
                  t->is_contiguous(),
              name, " must be a contiguous int32 [", n, "] tensor, got ", t->scalar_type(), " ",
              t->sizes());
  return t->data_ptr<int32_t>();
}

int64_t check_lengths(const at::Tensor& lens, const at::Tensor& ref, bool packed) {
  check_device(lens, ref, "context_lengths");
  TORCH_CHECK(lens.scalar_type() == at::kInt && lens.dim() == 1 && lens.is_contiguous(),
              "context_lengths must be a contiguous int32 1-D tensor");
  TORCH_CHECK(!packed || lens.size(0) >= 1,
              "context_lengths must hold batch + 1 offsets in packed mode");
  return packed ? lens.size(0) - 1 : lens.size(0);
}

// The K/V pair of a write op (value and value_cache both given or both None).
struct KvPair {
  TokenRows k, v;
  bool has_v;
};

// 4-bit linear caches (int8 holding int4 pairs): key_cache [max_batch, heads, cache_len,
// head_size / 2] (channel pairs), value_cache [max_batch, heads, cache_len / 2, head_size]
// (position pairs), both int8 (reference _ops.py:3690-3697).
void check_linear_cache4(const at::Tensor& kc, const c10::optional<at::Tensor>& vc,
                         const at::Tensor& ref, int64_t H, int64_t D) {
  check_device(kc, ref, "key_cache");
  TORCH_CHECK(D % 2 == 0, "quant_bit 4 needs an even head_size, got ", D);
  TORCH_CHECK(kc.dim() == 4 && kc.is_contiguous() && kc.scalar_type() == at::kChar,
              "key_cache must be a contiguous int8 [max_batch, heads, cache_len, head_size / 2] "
              "tensor for quant_bit 4, got ", kc.sizes(), " ", kc.scalar_type());
  TORCH_CHECK(kc.size(1) == H && kc.size(3) * 2 == D, "key_cache ", kc.sizes(),
              " does not match [heads, head_size / 2] = [", H, ", ", D / 2, "] for quant_bit 4");
  if (vc.has_value()) {
    check_device(*vc, ref, "value_cache");
    TORCH_CHECK(vc->dim() == 4 && vc->is_contiguous() && vc->scalar_type() == at::kChar,
                "value_cache must be a contiguous int8 [max_batch, heads, cache_len / 2, "
                "head_size] tensor for quant_bit 4, got ", vc->sizes(), " ", vc->scalar_type());
    TORCH_CHECK(vc->size(0) == kc.size(0) && vc->size(1) == H && vc->size(2) * 2 == kc.size(2) &&
                    vc->size(3) == D,
                "value_cache ", vc->sizes(), " must be [max_batch, heads, cache_len / 2, "
                "head_size] = [", kc.size(0), ", ", H, ", ", kc.size(2) / 2, ", ", D,
                "] for quant_bit 4 (cache_len even)");
  }
}

KvPair write_rows(const at::Tensor& key, const c10::optional<at::Tensor>& value,
                  const at::Tensor& key_cache, const c10::optional<at::Tensor>& value_cache,
                  int64_t bits = 8) {
  KvPair kv;
  check_device(key, key, "key");
  kv.k = token_rows(key, true, "key");
  kv.has_v = value.has_value();
  TORCH_CHECK(kv.has_v == value_cache.has_value(),
              "value and value_cache must both be given or both be None");
  if (bits == 4) {
    check_linear_cache4(key_cache, value_cache, key, kv.k.H, kv.k.D);
  } else {
    check_linear_cache(key_cache, key, kv.k.H, kv.k.D, "key_cache");
  }
  if (kv.has_v) {
    check_device(*value, key, "value");
    TORCH_CHECK(value->sizes() == key.sizes() && value->scalar_type() == key.scalar_type(),
                "value must match key");
    kv.v = token_rows(*value, true, "value");
    if (bits != 4) {
      check_linear_cache(*value_cache, key, kv.k.H, kv.k.D, "value_cache");
      TORCH_CHECK(value_cache->sizes() == key_cache.sizes() &&
                      value_cache->scalar_type() == key_cache.scalar_type(),
                  "value_cache must match key_cache");
    }
  }
  return kv;
}

}  // namespace

void reshape_linear_cache(const at::Tensor& key, const c10::optional<at::Tensor>& value,
                          at::Tensor& key_cache, const c10::optional<at::Tensor>& value_cache,
                          const at::Tensor& context_lengths, const c10::SymInt max_context_len,
                          bool packed, const c10::optional<at::Tensor>& context_seq_offset,
                          const c10::optional<at::Tensor>& cache_bs_id,
                          const c10::optional<at::Tensor>& cache_seqlen_offset) {
  const KvPair kv = write_rows(key, value, key_cache, value_cache);
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt >= 0 && dt != TMO_DTYPE_F8E4M3, "reshape_linear_cache: unsupported dtype ",
              key.scalar_type());
  TORCH_CHECK(key_cache.scalar_type() == key.scalar_type(), "key_cache dtype ",
              key_cache.scalar_type(), " must match key dtype ", key.scalar_type());
  TORCH_CHECK(packed || key.dim() == 4, "padded (packed=False) key must be 4-D");
  const int64_t B = check_lengths(context_lengths, key, packed);
  const int32_t* cso = i32_vec(context_seq_offset, key, B, "context_seq_offset");
  const int32_t* bsi = i32_vec(cache_bs_id, key, B, "cache_bs_id");
  const int32_t* coff = i32_vec(cache_seqlen_offset, key, B, "cache_seqlen_offset");
  const int64_t max_ctx = max_context_len.expect_int();
  TORCH_CHECK(max_ctx >= 0, "max_context_len must be >= 0");
  c10::DeviceGuard guard(key.device());
  const int st = tmo_hip_reshape_linear_cache(
      kv.k.t.data_ptr(), kv.has_v ? kv.v.t.data_ptr() : nullptr, kv.k.st, kv.k.sh,
      kv.has_v ? kv.v.st : 0, kv.has_v ? kv.v.sh : 0, kv.k.rows, key_cache.data_ptr(),
      kv.has_v ? value_cache->data_ptr() : nullptr, key_cache.size(0), kv.k.H,
      key_cache.size(2), kv.k.D, context_lengths.data_ptr<int32_t>(), B, max_ctx, packed ? 1 : 0,
      kv.k.seqlen, cso, bsi, coff, dt, stream_of(key));
  check_status(st, "reshape_linear_cache");
}

void quant_to_linear_cache(const at::Tensor& key, const c10::optional<at::Tensor>& value,
                           at::Tensor& key_cache, const c10::optional<at::Tensor>& value_cache,
                           at::Tensor& key_cache_scale,
                           const c10::optional<at::Tensor>& value_cache_scale,
                           const at::Tensor& context_lengths, const c10::SymInt max_context_len,
                           bool packed, const c10::optional<at::Tensor>& context_seq_offset,
                           const c10::optional<at::Tensor>& cache_bs_id,
                           const c10::optional<at::Tensor>& cache_seqlen_offset,
                           const int64_t quant_bit) {
  TORCH_CHECK(quant_bit == 8 || quant_bit == 4,
              "quant_to_linear_cache: quant_bit must be 8 or 4, got ", quant_bit);
  const KvPair kv = write_rows(key, value, key_cache, value_cache, quant_bit);
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F32 || dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "quant_to_linear_cache: key must be float, half or bfloat16, got ",
              key.scalar_type());
  const int cdt = dtype_code(key_cache.scalar_type());
  TORCH_CHECK(cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3,
              "quant_to_linear_cache: caches must be int8 or float8_e4m3fn, got ",
              key_cache.scalar_type());
  TORCH_CHECK(packed || key.dim() == 4, "padded (packed=False) key must be 4-D");
  TORCH_CHECK(kv.has_v == value_cache_scale.has_value(),
              "value_cache_scale must be given exactly when value is");
  const int64_t MB = key_cache.size(0), L = key_cache.size(2);
  auto check_scale = [&](const at::Tensor& s, const char* name) -> int64_t {
    check_device(s, key, name);
    TORCH_CHECK(s.scalar_type() == at::kFloat && s.is_contiguous(), name,
                " must be a contiguous float32 tensor");
    TORCH_CHECK((s.dim() == 3 || s.dim() == 4) && s.size(0) == MB && s.size(1) == kv.k.H &&
                    s.size(2) == L,
                name, " must be [max_batch, heads, cache_len] or [max_batch, heads, cache_len, "
                "group_num], got ", s.sizes());
    const int64_t g = s.dim() == 4 ? s.size(3) : 1;
    TORCH_CHECK(g >= 1 && kv.k.D % g == 0, name, ": head_size ", kv.k.D,
                " is not a multiple of group_num ", g);
    return g;
  };
  const int64_t groups = check_scale(key_cache_scale, "key_cache_scale");
  if (kv.has_v) {
    TORCH_CHECK(check_scale(*value_cache_scale, "value_cache_scale") == groups &&
                    value_cache_scale->sizes() == key_cache_scale.sizes(),
                "value_cache_scale must match key_cache_scale");
  }
  const int64_t B = check_lengths(context_lengths, key, packed);
  const int32_t* cso = i32_vec(context_seq_offset, key, B, "context_seq_offset");
  const int32_t* bsi = i32_vec(cache_bs_id, key, B, "cache_bs_id");
  const int32_t* coff = i32_vec(cache_seqlen_offset, key, B, "cache_seqlen_offset");
  const int64_t max_ctx = max_context_len.expect_int();
  TORCH_CHECK(max_ctx >= 0, "max_context_len must be >= 0");
  c10::DeviceGuard guard(key.device());
  const int st = tmo_hip_quant_to_linear_cache(
      kv.k.t.data_ptr(), kv.has_v ? kv.v.t.data_ptr() : nullptr, kv.k.st, kv.k.sh,
      kv.has_v ? kv.v.st : 0, kv.has_v ? kv.v.sh : 0, kv.k.rows, key_cache.data_ptr(),
      kv.has_v ? value_cache->data_ptr() : nullptr, key_cache_scale.data_ptr<float>(),
      kv.has_v ? value_cache_scale->data_ptr<float>() : nullptr, MB, kv.k.H, L, kv.k.D, groups,
      context_lengths.data_ptr<int32_t>(), B, max_ctx, packed ? 1 : 0, kv.k.seqlen, cso, bsi,
      coff, (int)quant_bit, dt, cdt, stream_of(key));
  check_status(st, "quant_to_linear_cache");
}

void offline_quant_to_linear_cache(const at::Tensor& key, const c10::optional<at::Tensor>& value,
                                   at::Tensor& key_cache,
                                   const c10::optional<at::Tensor>& value_cache,
                                   const c10::optional<at::Tensor>& key_cache_scale,
                                   const c10::optional<at::Tensor>& value_cache_scale,
                                   const at::Tensor& context_lengths,
                                   const c10::SymInt max_context_len, const int64_t quant_mode,
                                   const bool packed,
                                   const c10::optional<at::Tensor>& context_seq_offset,
                                   const c10::optional<at::Tensor>& cache_bs_id,
                                   const c10::optional<at::Tensor>& cache_seqlen_offset,
                                   double key_cache_scale_per_tensor,
                                   double value_cache_scale_per_tensor) {
  TORCH_CHECK(quant_mode >= 0 && quant_mode <= 3,
              "offline_quant_to_linear_cache: quant_mode must be 0 (per channel), 1 (per head) "
              "or 2/3 (per tensor), got ", quant_mode);
  const KvPair kv = write_rows(key, value, key_cache, value_cache);
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F32 || dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16,
              "offline_quant_to_linear_cache: key must be float, half or bfloat16, got ",
              key.scalar_type());
  const int cdt = dtype_code(key_cache.scalar_type());
  TORCH_CHECK(cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3,
              "offline_quant_to_linear_cache: caches must be int8 or float8_e4m3fn, got ",
              key_cache.scalar_type());
  TORCH_CHECK(packed || key.dim() == 4, "padded (packed=False) key must be 4-D");
  const int64_t H = kv.k.H, D = kv.k.D, L = key_cache.size(2);
  const float* ks = nullptr;
  const float* vs = nullptr;
  const float kt = static_cast<float>(key_cache_scale_per_tensor);
  const float vt = static_cast<float>(value_cache_scale_per_tensor);
  if (quant_mode < 2) {
    const int64_t cols = quant_mode == 0 ? D : L;
    auto check_scale = [&](const c10::optional<at::Tensor>& s, const char* name) {
      TORCH_CHECK(s.has_value(), name, " is required for quant_mode ", quant_mode);
      check_device(*s, key, name);
      TORCH_CHECK(s->scalar_type() == at::kFloat && s->is_contiguous() && s->dim() == 2 &&
                      s->size(0) == H && s->size(1) == cols,
                  name, " must be a contiguous float32 [heads, ",
                  quant_mode == 0 ? "head_size" : "cache_len", "] tensor, got ",
                  s->scalar_type(), " ", s->sizes());
      return s->data_ptr<float>();
    };
    ks = check_scale(key_cache_scale, "key_cache_scale");
    if (kv.has_v) vs = check_scale(value_cache_scale, "value_cache_scale");
  } else {
    TORCH_CHECK(!key_cache_scale.has_value() && !value_cache_scale.has_value(),
                "offline_quant_to_linear_cache: per-tensor quant_mode ", quant_mode,
                " takes the scales as numbers");
    TORCH_CHECK(std::isfinite(kt) && kt != 0.0f, "key_cache_scale must be finite and non-zero, got ",
                key_cache_scale_per_tensor);
    TORCH_CHECK(!kv.has_v || (std::isfinite(vt) && vt != 0.0f),
                "value_cache_scale must be finite and non-zero, got ",
                value_cache_scale_per_tensor);
  }
  const int64_t B = check_lengths(context_lengths, key, packed);
  const int32_t* cso = i32_vec(context_seq_offset, key, B, "context_seq_offset");
  const int32_t* bsi = i32_vec(cache_bs_id, key, B, "cache_bs_id");
  const int32_t* coff = i32_vec(cache_seqlen_offset, key, B, "cache_seqlen_offset");
  const int64_t max_ctx = max_context_len.expect_int();
  TORCH_CHECK(max_ctx >= 0, "max_context_len must be >= 0");
  c10::DeviceGuard guard(key.device());
  const int st = tmo_hip_offline_quant_to_linear_cache(
      kv.k.t.data_ptr(), kv.has_v ? kv.v.t.data_ptr() : nullptr, kv.k.st, kv.k.sh,
      kv.has_v ? kv.v.st : 0, kv.has_v ? kv.v.sh : 0, kv.k.rows, key_cache.data_ptr(),
      kv.has_v ? value_cache->data_ptr() : nullptr, ks, vs, kt, vt, (int)quant_mode,
      key_cache.size(0), H, L, D, context_lengths.data_ptr<int32_t>(), B, max_ctx,
      packed ? 1 : 0, kv.k.seqlen, cso, bsi, coff, dt, cdt, stream_of(key));
  check_status(st, "offline_quant_to_linear_cache");
}

void dequant_from_linear_cache(at::Tensor& key, const c10::optional<at::Tensor>& value,
                               const at::Tensor& key_cache,
                               const c10::optional<at::Tensor>& value_cache,
                               const at::Tensor& key_quant_scale,
                               const c10::optional<at::Tensor>& value_quant_scale,
                               const at::Tensor& context_lengths,
                               const c10::SymInt max_context_len,
                               const c10::optional<at::Tensor>& context_seq_offset,
                               const c10::optional<at::Tensor>& cache_bs_id,
                               const c10::optional<at::Tensor>& cache_seq_offset,
                               const int64_t quant_mode, const int64_t quant_bit) {
  TORCH_CHECK(quant_mode == 0 || quant_mode == 1,
              "dequant_from_linear_cache: quant_mode must be 0 (per-channel) or 1 (per-token), "
              "got ", quant_mode);
  TORCH_CHECK(quant_bit == 8 || quant_bit == 4,
              "dequant_from_linear_cache: quant_bit must be 8 or 4, got ", quant_bit);
  check_device(key, key, "key");
  const TokenRows k = token_rows(key, false, "key");
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt == TMO_DTYPE_F16 || dt == TMO_DTYPE_BF16 || dt == TMO_DTYPE_F32,
              "dequant_from_linear_cache: key must be half, bfloat16 or float, got ",
              key.scalar_type());
  if (quant_bit == 4) {
    check_linear_cache4(key_cache, value_cache, key, k.H, k.D);
  } else {
    check_linear_cache(key_cache, key, k.H, k.D, "key_cache");
  }
  TORCH_CHECK(key_cache.scalar_type() == at::kChar, "key_cache must be int8");
  const int64_t MB = key_cache.size(0), L = key_cache.size(2);
  auto check_scale = [&](const at::Tensor& s, const char* name) {
    check_device(s, key, name);
    TORCH_CHECK(s.scalar_type() == at::kFloat && s.is_contiguous(), name,
                " must be a contiguous float32 tensor");
    if (quant_mode == 0) {
      TORCH_CHECK(s.dim() == 2 && s.size(0) == k.H && s.size(1) == k.D, name,
                  " must be [heads, head_size] for quant_mode 0, got ", s.sizes());
    } else {
      TORCH_CHECK(s.dim() == 3 && s.size(0) == MB && s.size(1) == k.H && s.size(2) == L, name,
                  " must be [max_batch, heads, cache_len] for quant_mode 1, got ", s.sizes());
    }
  };
  check_scale(key_quant_scale, "key_cache_quant_scale");
  const bool has_v = value.has_value();
  TORCH_CHECK(has_v == value_cache.has_value() && has_v == value_quant_scale.has_value(),
              "value, value_cache and value_cache_quant_scale must all be given or all be None");
  TokenRows v{};
  if (has_v) {
    check_device(*value, key, "value");
    TORCH_CHECK(value->sizes() == key.sizes() && value->scalar_type() == key.scalar_type(),
                "value must match key");
    v = token_rows(*value, false, "value");
    if (quant_bit != 4) {
      check_linear_cache(*value_cache, key, k.H, k.D, "value_cache");
      TORCH_CHECK(value_cache->sizes() == key_cache.sizes() &&
                      value_cache->scalar_type() == at::kChar,
                  "value_cache must match key_cache");
    }
    check_scale(*value_quant_scale, "value_cache_quant_scale");
  }
  const int64_t B = check_lengths(context_lengths, key, false);
  const int32_t* cso = i32_vec(context_seq_offset, key, B, "context_seq_offset");
  const int32_t* bsi = i32_vec(cache_bs_id, key, B, "cache_bs_id");
  const int32_t* coff = i32_vec(cache_seq_offset, key, B, "cache_seq_offset");
  const int64_t max_ctx = max_context_len.expect_int();
  TORCH_CHECK(max_ctx >= 0, "max_context_len must be >= 0");
  c10::DeviceGuard guard(key.device());
  const int st = tmo_hip_dequant_from_linear_cache(
      key.data_ptr(), has_v ? value->data_ptr() : nullptr, k.st, k.sh, has_v ? v.st : 0,
      has_v ? v.sh : 0, k.rows, key_cache.data_ptr<int8_t>(),
      has_v ? value_cache->data_ptr<int8_t>() : nullptr, key_quant_scale.data_ptr<float>(),
      has_v ? value_quant_scale->data_ptr<float>() : nullptr, MB, k.H, L, k.D,
      context_lengths.data_ptr<int32_t>(), B, max_ctx, cso, bsi, coff, (int)quant_mode,
      (int)quant_bit, dt, stream_of(key));
  check_status(st, "dequant_from_linear_cache");
}

void reshape_from_cache(at::Tensor& key, const c10::optional<at::Tensor>& value,
                        const at::Tensor& key_cache, const c10::optional<at::Tensor>& value_cache,
                        const at::Tensor& context_lengths, c10::SymInt max_context_len,
                        const c10::optional<at::Tensor>& context_seq_offset,
                        const c10::optional<at::Tensor>& block_tables,
                        const c10::optional<at::Tensor>& cache_seq_offset) {
  check_device(key, key, "key");
  const TokenRows k = token_rows(key, false, "key");
  const int dt = dtype_code(key.scalar_type());
  TORCH_CHECK(dt >= 0 && dt != TMO_DTYPE_F8E4M3, "reshape_from_cache: unsupported dtype ",
              key.scalar_type());
  check_linear_cache(key_cache, key, k.H, k.D, "key_cache");
  TORCH_CHECK(key_cache.scalar_type() == key.scalar_type(), "key_cache dtype ",
              key_cache.scalar_type(), " must match key dtype ", key.scalar_type());
  const bool has_v = value.has_value();
  TORCH_CHECK(has_v == value_cache.has_value(),
              "value and value_cache must both be given or both be None");
  TokenRows v{};
  if (has_v) {
    check_device(*value, key, "value");
    TORCH_CHECK(value->sizes() == key.sizes() && value->scalar_type() == key.scalar_type(),
                "value must match key");
    v = token_rows(*value, false, "value");
    check_linear_cache(*value_cache, key, k.H, k.D, "value_cache");
    TORCH_CHECK(value_cache->sizes() == key_cache.sizes() &&
                    value_cache->scalar_type() == key_cache.scalar_type(),
                "value_cache must match key_cache");
  }
  const int64_t B = check_lengths(context_lengths, key, false);
  const int32_t* cso = i32_vec(context_seq_offset, key, B, "context_seq_offset");
  const int32_t* coff = i32_vec(cache_seq_offset, key, B, "cache_seq_offset");
  const int32_t* bt = nullptr;
  int64_t max_blocks = 0;
  if (block_tables.has_value()) {
    check_device(*block_tables, key, "block_tables");
    TORCH_CHECK(block_tables->scalar_type() == at::kInt && block_tables->dim() == 2 &&
                    block_tables->size(0) == B && block_tables->size(1) >= 1 &&
                    block_tables->is_contiguous(),
                "block_tables must be a contiguous int32 [batch, max_blocks] tensor, got ",
                block_tables->sizes());
    bt = block_tables->data_ptr<int32_t>();
    max_blocks = block_tables->size(1);
  }
  const int64_t max_ctx = max_context_len.expect_int();
  TORCH_CHECK(max_ctx >= 0, "max_context_len must be >= 0");
  c10::DeviceGuard guard(key.device());
  const int st = tmo_hip_reshape_from_cache(
      key.data_ptr(), has_v ? value->data_ptr() : nullptr, k.st, k.sh, has_v ? v.st : 0,
      has_v ? v.sh : 0, k.rows, key_cache.data_ptr(), has_v ? value_cache->data_ptr() : nullptr,
      key_cache.size(0), k.H, key_cache.size(2), k.D, context_lengths.data_ptr<int32_t>(), B,
      max_ctx, cso, bt, max_blocks, coff, dt, stream_of(key));
  check_status(st, "reshape_from_cache");
}

// ------------------------------------------------------------------------------ decode attention

void single_query_cached_kv_attn(const torch::Tensor& q_ori, const torch::Tensor& k_cache,
                                 const torch::Tensor& output, const torch::Tensor& block_tables,
                                 const torch::Tensor& context_lens,
                                 const c10::optional<torch::Tensor>& v_cache,
                                 const c10::optional<torch::Tensor>& output_lse,
                                 const c10::optional<torch::Tensor>& q_quant_scale,
                                 const c10::optional<torch::Tensor>& k_cache_quant_scale,
                                 const c10::optional<torch::Tensor>& v_cache_quant_scale,
                                 const c10::optional<torch::Tensor>& out_quant_scale,
                                 const c10::optional<torch::Tensor>& alibi_slopes,
                                 const c10::optional<torch::Tensor>& mask,
                                 const std::string& compute_dtype, c10::SymInt max_context_len,
                                 c10::SymInt windows_size_left, c10::SymInt windows_size_right,
                                 double softmax_scale, bool return_lse,
                                 int64_t kv_cache_quant_bit_size,
                                 const c10::optional<torch::Tensor>& cu_seq_q,
                                 c10::SymInt max_seq_q, const c10::optional<torch::Tensor>& sink) {
  const char* op = "single_query_cached_kv_attn";
  TORCH_CHECK(!out_quant_scale.has_value(), op,
              ": out_quant_scale is a reserved parameter and must be None (_ops.py:857)");
  TORCH_CHECK(compute_dtype == "float" || compute_dtype == "half" || compute_dtype == "bfloat16",
              op, ": compute_dtype must be float, half or bfloat16 (the softmax runs in fp32)");
  TORCH_CHECK(windows_size_right.expect_int() == -1, op, ": windows_size_right must be -1");
  TORCH_CHECK(kv_cache_quant_bit_size == -1 || kv_cache_quant_bit_size == 8 ||
                  kv_cache_quant_bit_size == 4,
              op, ": kv_cache_quant_bit_size must be -1, 8 (int8 / float8_e4m3fn) or 4 (int4 ",
              "pairs in int8), got ", kv_cache_quant_bit_size);
  const bool int4 = kv_cache_quant_bit_size == 4;
  check_device(q_ori, q_ori, "q");
  // q forms (reference _ops.py:824): [batch, seq_q, heads, head_size] (seq_q tokens for every
  // sequence), [total_q, heads, head_size] with cu_seq_q [batch + 1], or [batch, heads,
  // head_size] (one token each).  Token s of a sequence with nq tokens sits at position
  // L - nq + s and sees the keys up to it.
  const bool four = q_ori.dim() == 4;
  TORCH_CHECK(four || q_ori.dim() == 3, op,
              ": q must be [batch, seq_q, heads, head_size] or [total_q, heads, head_size], got ",
              q_ori.sizes());
  TORCH_CHECK(!(four && cu_seq_q.has_value()), op, ": cu_seq_q goes with a 3-D q");
  const at::Tensor& q = q_ori;
  TORCH_CHECK(q.size(-1) <= 1 || q.stride(-1) == 1, "q must have a contiguous last dim");
  // q: float, half, bfloat16, or int8 / float8_e4m3fn codes with q_quant_scale (_ops.py:853-856,
  // 868); the output then has its own dtype (float8_e4m3fn q: half, _ops.py:858)
  const bool qquant = q.scalar_type() == at::kChar || q.scalar_type() == at::kFloat8_e4m3fn;
  const int qdt = q.scalar_type() == at::kChar ? TMO_DTYPE_I8
                  : q.scalar_type() == at::kFloat8_e4m3fn ? TMO_DTYPE_F8E4M3
                                                          : dtype_code(q.scalar_type());
  TORCH_CHECK(qdt == TMO_DTYPE_F32 || qdt == TMO_DTYPE_F16 || qdt == TMO_DTYPE_BF16 || qquant, op,
              ": q must be float, half, bfloat16, int8 or float8_e4m3fn, got ", q.scalar_type());
  TORCH_CHECK(qquant == q_quant_scale.has_value(), op,
              ": q_quant_scale goes with (and only with) an int8 or float8_e4m3fn q");
  const int64_t Hq = q.size(-2), D = q.size(-1);
  check_device(context_lens, q_ori, "context_lens");
  TORCH_CHECK(context_lens.scalar_type() == at::kInt && context_lens.dim() == 1 &&
                  context_lens.is_contiguous(),
              op, ": context_lens must be a contiguous int32 [batch] tensor");
  const int64_t B = context_lens.size(0);
  const int32_t* cu = nullptr;
  int64_t seq_q = 1, total_q = 0;
  if (four) {
    TORCH_CHECK(q.size(0) == B, op, ": q's batch ", q.size(0), " != context_lens' ", B);
    seq_q = q.size(1);
  } else if (cu_seq_q.has_value()) {
    const at::Tensor& c = *cu_seq_q;
    check_device(c, q_ori, "cu_seq_q");
    TORCH_CHECK(c.scalar_type() == at::kInt && c.dim() == 1 && c.size(0) == B + 1 &&
                    c.is_contiguous(),
                op, ": cu_seq_q must be a contiguous int32 [batch + 1] tensor, got ", c.sizes());
    cu = c.data_ptr<int32_t>();
    total_q = q.size(0);
    // max_seq_q <= 0: unknown, read from cu_seq_q (one device-to-host copy).  A positive
    // max_seq_q is trusted, as the reference trusts max_context_len ("if 0 < max_context_len <
    // max(context_lens), the correctness is not guaranteed", _ops.py:847): query tokens of a
    // sequence at or past it are not computed and their output rows are left as they were.
    seq_q = max_seq_q.expect_int();
    if (seq_q <= 0)
      seq_q = B == 0 ? 0 : std::max<int64_t>(0, (c.slice(0, 1) - c.slice(0, 0, B)).max().item<int64_t>());
  } else {
    TORCH_CHECK(q.size(0) == B, op, ": q's rows ", q.size(0), " != context_lens' batch ", B,
                " (pass cu_seq_q for several tokens per sequence)");
  }
  const float* sink_p = nullptr;
  if (sink.has_value()) {
    check_device(*sink, q_ori, "sink");
    TORCH_CHECK(sink->scalar_type() == at::kFloat && sink->is_contiguous() &&
                    sink->numel() == Hq,
                op, ": sink must be a contiguous float32 [heads] tensor");
    sink_p = sink->data_ptr<float>();
  }
  // caches [num_blocks, kv_heads, block_size, cache_dim]: keys are the first head_size
  // channels of a K row, values the first head_size_v (out's last dim) of a V row, or of the
  // K row when v_cache is None (cache_dim = max(head_size_qk, head_size_v), _ops.py:828-831)
  check_device(k_cache, q_ori, "k_cache");
  TORCH_CHECK(k_cache.dim() == 4 && k_cache.is_contiguous(), op,
              ": k_cache must be a contiguous [num_blocks, kv_heads, block_size, cache_dim] ",
              "tensor, got ", k_cache.sizes());
  const int64_t NB = k_cache.size(0), Hkv = k_cache.size(1), BS = k_cache.size(2);
  const int64_t kdim = k_cache.size(3);
  check_device(output, q_ori, "output");
  TORCH_CHECK(output.dim() == q_ori.dim() &&
                  output.sizes().slice(0, q_ori.dim() - 1) == q_ori.sizes().slice(0, q_ori.dim() - 1),
              op, ": output must be q's shape with head_size_v channels");
  const int odt = dtype_code(output.scalar_type());
  if (qquant) {
    TORCH_CHECK(odt == TMO_DTYPE_F32 || odt == TMO_DTYPE_F16 || odt == TMO_DTYPE_BF16, op,
                ": the output of a quantised q must be float, half or bfloat16");
    TORCH_CHECK(q.scalar_type() != at::kFloat8_e4m3fn || odt == TMO_DTYPE_F16, op,
                ": the output must be half when q is float8_e4m3fn (_ops.py:858)");
  } else {
    TORCH_CHECK(output.scalar_type() == q.scalar_type(), op, ": output must have q's dtype");
  }
  const int64_t Dv = output.size(-1);
  int64_t vdim = kdim;
  int v_pair_channels = 0;
  if (int4) {
    // int4 pairs (_ops.py:826-829, 852, 868): K [NB, Hkv, BS, D / 2] pairing channels; V
    // pairing the rows of a page, [NB, Hkv, BS / 2, Dv] (the layout the reference's output
    // allocation reads head_size_v from, _ops.py:887), or channels, [NB, Hkv, BS, Dv / 2]
    TORCH_CHECK(k_cache.scalar_type() == at::kChar, op,
                ": kv_cache_quant_bit_size 4 needs int8 caches of int4 pairs");
    TORCH_CHECK(v_cache.has_value(), op, ": int4 caches need a separate v_cache");
    const at::Tensor& vc = *v_cache;
    check_device(vc, q_ori, "v_cache");
    TORCH_CHECK(vc.dim() == 4 && vc.is_contiguous() && vc.size(0) == NB && vc.size(1) == Hkv &&
                    vc.scalar_type() == at::kChar,
                op, ": v_cache must be a contiguous int8 [num_blocks, kv_heads, ...] tensor");
    TORCH_CHECK(2 * kdim == D, op, ": int4 k_cache's last dim must be head_size / 2 = ", D / 2,
                ", got ", kdim);
    vdim = vc.size(3);
    if (2 * vc.size(2) == BS && vdim == Dv) {
      v_pair_channels = 0;
    } else if (vc.size(2) == BS && 2 * vdim == Dv) {
      v_pair_channels = 1;
    } else {
      TORCH_CHECK(false, op, ": int4 v_cache must be [num_blocks, kv_heads, block_size / 2, ",
                  "head_size_v] (row pairs) or [num_blocks, kv_heads, block_size, head_size_v / 2] ",
                  "(channel pairs), got ", vc.sizes(), " with block_size ", BS, ", head_size_v ", Dv);
    }
  } else if (v_cache.has_value()) {
    const at::Tensor& vc = *v_cache;
    check_device(vc, q_ori, "v_cache");
    TORCH_CHECK(vc.dim() == 4 && vc.is_contiguous() && vc.size(0) == NB && vc.size(1) == Hkv &&
                    vc.size(2) == BS && vc.scalar_type() == k_cache.scalar_type(),
                op, ": v_cache must be a contiguous [num_blocks, kv_heads, block_size, ",
                "head_size_v] tensor of k_cache's dtype, got ", vc.sizes());
    vdim = vc.size(3);
    TORCH_CHECK(kdim == D, op, ": k_cache head_size ", kdim, " != q's ", D);
    TORCH_CHECK(vdim == Dv, op, ": v_cache head_size ", vdim, " != output's ", Dv);
  } else {
    TORCH_CHECK(kdim == std::max(D, Dv), op, ": with v_cache None, k_cache's last dim must be ",
                "max(head_size_qk, head_size_v) = ", std::max(D, Dv), ", got ", kdim);
  }
  TORCH_CHECK(Hkv > 0 && Hq % Hkv == 0, op, ": query heads ", Hq,
              " must be a multiple of the KV heads ", Hkv);
  TORCH_CHECK(D <= 4096 && Dv <= 512, op, ": head sizes up to 4096 (keys) and 512 (values)");
  const int cdt = int4 ? TMO_DTYPE_I4 : dtype_code(k_cache.scalar_type());
  // quantised caches: int8 codes or float8_e4m3fn values (_ops.py:868; bit size 8 covers both,
  // _ops.py:1061), or int4 pairs (bit size 4), with per-token / per-channel / per-group scales
  const bool int8 = cdt == TMO_DTYPE_I8 || cdt == TMO_DTYPE_F8E4M3 || int4;
  // caches "the same as q" (kv_cache_quant_bit_size -1, _ops.py:852) under an int8 /
  // float8_e4m3fn q: codes read as they are, i.e. with unit scales
  const bool same_as_q = qquant && kv_cache_quant_bit_size == -1 && cdt == qdt;
  TORCH_CHECK(int4 || same_as_q || int8 == (kv_cache_quant_bit_size == 8), op,
              ": kv_cache_quant_bit_size 8 goes with int8 or float8_e4m3fn caches, -1 with caches ",
              "of q's dtype");
  TORCH_CHECK(int8 || cdt == qdt, op, ": unquantised caches must have q's dtype");
  // scales: per token [NB, Hkv, BS] (or [..., 1]; any strides in the first two dims), per
  // channel [Hkv, D] / [Hkv, Dv], per tensor [1], per group K [NB, Hkv, BS, D / 32] with
  // V [NB, Hkv, BS / 32, Dv] (_ops.py:838-842)
  int smode = 0;
  at::Tensor ks, vs;
  int64_t ks_sb = 0, ks_sh = 0, vs_sb = 0, vs_sh = 0;
  if (same_as_q) {
    TORCH_CHECK(!k_cache_quant_scale.has_value() && !v_cache_quant_scale.has_value(), op,
                ": caches of q's dtype take no scales");
    smode = 2;
    ks = at::ones({Hkv, D}, q_ori.options().dtype(at::kFloat));
    vs = at::ones({Hkv, Dv}, q_ori.options().dtype(at::kFloat));
  } else if (int8) {
    TORCH_CHECK(k_cache_quant_scale.has_value() && v_cache_quant_scale.has_value(), op,
                ": int8 caches need k_cache_quant_scale and v_cache_quant_scale");
    const at::Tensor& ksc = *k_cache_quant_scale;
    const at::Tensor& vsc = *v_cache_quant_scale;
    check_device(ksc, q_ori, "k_cache_quant_scale");
    check_device(vsc, q_ori, "v_cache_quant_scale");
    // float32 or bfloat16 (_ops.py:872), both of one type
    TORCH_CHECK((ksc.scalar_type() == at::kFloat || ksc.scalar_type() == at::kBFloat16) &&
                    vsc.scalar_type() == ksc.scalar_type(),
                op, ": cache scales must be float32 or bfloat16 (K and V of one type)");
    const bool group = ksc.dim() == 4 && vsc.dim() == 4 && D % 32 == 0 && BS % 32 == 0 &&
                       ksc.sizes() == at::IntArrayRef({NB, Hkv, BS, D / 32}) &&
                       vsc.sizes() == at::IntArrayRef({NB, Hkv, BS / 32, Dv});
    if (group) {
      TORCH_CHECK(ksc.is_contiguous() && vsc.is_contiguous(), op,
                  ": per-group scales must be contiguous");
      smode = 3;
      ks = ksc;
      vs = vsc;
    } else {
      auto norm = [&](const at::Tensor& sc, int64_t dims, int64_t& sb, int64_t& sh,
                      const char* name) -> at::Tensor {
        if ((sc.dim() == 3 || (sc.dim() == 4 && sc.size(3) == 1)) && sc.size(0) == NB &&
            sc.size(1) == Hkv && sc.size(2) == BS) {
          TORCH_CHECK(smode == 0 || smode == 1, op, ": K and V scales must use one mode");
          smode = 1;
          at::Tensor t = sc.dim() == 4 ? sc.select(3, 0) : sc;
          if (BS > 1 && t.stride(2) != 1) t = t.contiguous();
          sb = t.stride(0);
          sh = t.stride(1);
          return t;
        }
        if (sc.dim() == 2 && sc.size(0) == Hkv && sc.size(1) == dims) {
          TORCH_CHECK(smode == 0 || smode == 2, op, ": K and V scales must use one mode");
          smode = 2;
          return sc.contiguous();
        }
        if (sc.numel() == 1) {  // per tensor: one number for every channel
          TORCH_CHECK(smode == 0 || smode == 2, op, ": K and V scales must use one mode");
          smode = 2;
          return sc.reshape({1, 1}).expand({Hkv, dims}).contiguous();
        }
        TORCH_CHECK(false, name, ": expected [num_blocks, kv_heads, block_size], [kv_heads, ",
                    "head_size], [1] or per-group K [num_blocks, kv_heads, block_size, ",
                    "head_size / 32] with V [num_blocks, kv_heads, block_size / 32, ",
                    "head_size_v], got ", sc.sizes());
        return sc;
      };
      ks = norm(ksc, D, ks_sb, ks_sh, "k_cache_quant_scale");
      vs = norm(vsc, Dv, vs_sb, vs_sh, "v_cache_quant_scale");
    }
  }
  // block tables [batch, max_blocks], or sparse-KV [batch, kv_heads or heads, max_blocks]
  // (_ops.py:834): each KV head's (query head's) own pages
  check_device(block_tables, q_ori, "block_tables");
  TORCH_CHECK(block_tables.scalar_type() == at::kInt && block_tables.is_contiguous() &&
                  block_tables.size(0) == B &&
                  (block_tables.dim() == 2 ||
                   (block_tables.dim() == 3 &&
                    (block_tables.size(1) == Hkv || block_tables.size(1) == Hq))),
              op, ": block_tables must be a contiguous int32 [batch, max_blocks] or [batch, ",
              "kv_heads or heads, max_blocks] tensor, got ", block_tables.sizes());
  const int64_t bt_heads = block_tables.dim() == 3 ? block_tables.size(1) : 0;
  // q_quant_scale (_ops.py:853-856): [1] per tensor, q's leading shape per token and head, or
  // that shape plus scale_num per channel group; float32 or bfloat16 (_ops.py:871)
  int qs_mode = 0, qs_dt = TMO_DTYPE_F32;
  int64_t qs_sb = 0, qs_ss = 0, qs_sh = 0, qs_groups = 0;
  at::Tensor qst;
  if (qquant) {
    qst = *q_quant_scale;
    check_device(qst, q_ori, "q_quant_scale");
    TORCH_CHECK(qst.scalar_type() == at::kFloat || qst.scalar_type() == at::kBFloat16, op,
                ": q_quant_scale must be float32 or bfloat16");
    qs_dt = qst.scalar_type() == at::kBFloat16 ? TMO_DTYPE_BF16 : TMO_DTYPE_F32;
    const auto lead = q.sizes().slice(0, q.dim() - 1);
    if (qst.numel() == 1) {
      qs_mode = 1;
      qst = qst.reshape({1}).contiguous();
    } else if (qst.sizes() == lead) {
      qs_mode = 2;
      if (four) {
        qs_sb = qst.stride(0), qs_ss = qst.stride(1), qs_sh = qst.stride(2);
      } else {
        (cu ? qs_ss : qs_sb) = qst.stride(0);
        qs_sh = qst.stride(1);
      }
    } else {
      TORCH_CHECK(qst.dim() == q.dim() && qst.sizes().slice(0, q.dim() - 1) == lead &&
                      qst.size(-1) > 0 && D % qst.size(-1) == 0,
                  op, ": q_quant_scale must be [1], q's shape without head_size, or that with ",
                  "a last dim dividing head_size, got ", qst.sizes());
      qs_mode = 3;
      qst = qst.contiguous();
      qs_groups = qst.size(-1);
      if (four) {
        qs_sb = qst.stride(0), qs_ss = qst.stride(1), qs_sh = qst.stride(2);
      } else {
        (cu ? qs_ss : qs_sb) = qst.stride(0);
        qs_sh = qst.stride(1);
      }
    }
  }
  const float* alibi = nullptr;
  if (alibi_slopes.has_value()) {
    check_device(*alibi_slopes, q_ori, "alibi_slopes");
    TORCH_CHECK(alibi_slopes->scalar_type() == at::kFloat && alibi_slopes->is_contiguous() &&
                    alibi_slopes->numel() == B * Hq,
                op, ": alibi_slopes must be a contiguous float32 [batch, heads] tensor");
    alibi = alibi_slopes->data_ptr<float>();
  }
  const at::Tensor& out = output;
  TORCH_CHECK(out.size(-1) <= 1 || out.stride(-1) == 1, "output must have a contiguous last dim");
  // element strides (batch, token, head) of q, out and lse
  const int64_t q_sb = four || !cu ? q.stride(0) : 0, q_ss = four ? q.stride(1) : (cu ? q.stride(0) : 0);
  const int64_t o_sb = four || !cu ? out.stride(0) : 0, o_ss = four ? out.stride(1) : (cu ? out.stride(0) : 0);
  float* lse = nullptr;
  int64_t lse_sb = 0, lse_ss = 0, lse_sh = 0;
  if (return_lse) {
    TORCH_CHECK(output_lse.has_value(), op, ": return_lse needs output_lse");
    const at::Tensor& l = *output_lse;
    check_device(l, q_ori, "output_lse");
    TORCH_CHECK(l.scalar_type() == at::kFloat, "output_lse must be float32");
    if (four) {  // [batch, heads, seq_q]
      TORCH_CHECK(l.dim() == 3 && l.size(0) == B && l.size(1) == Hq && l.size(2) == seq_q, op,
                  ": output_lse must be [batch, heads, seq_q], got ", l.sizes());
      lse_sb = l.stride(0);
      lse_sh = l.stride(1);
      lse_ss = l.stride(2);
    } else {  // [heads, total_q]
      TORCH_CHECK(l.dim() == 2 && l.size(0) == Hq && l.size(1) == q.size(0), op,
                  ": output_lse must be [heads, total_q], got ", l.sizes());
      lse_sh = l.stride(0);
      (cu ? lse_ss : lse_sb) = l.stride(1);
    }
    lse = l.data_ptr<float>();
  }
  // mask [batch, seq_q, mask_len] (_ops.py:860): logit terms for each sequence's last
  // mask_len keys, in compute_dtype, within the reference's stated limits (seq_q <= 16,
  // mask_len <= 64, mask_len % seq_q == 0, not with float32 q)
  const void* mask_p = nullptr;
  int mask_dt = TMO_DTYPE_F32;
  int64_t mask_len = 0, m_sb = 0, m_ss = 0;
  at::Tensor mk;
  if (mask.has_value()) {
    mk = *mask;
    check_device(mk, q_ori, "mask");
    const at::ScalarType want = compute_dtype == "float" ? at::kFloat
                                : compute_dtype == "half" ? at::kHalf : at::kBFloat16;
    TORCH_CHECK(mk.scalar_type() == want, op, ": mask must be of compute_dtype (", compute_dtype,
                "), got ", mk.scalar_type());
    TORCH_CHECK(qdt != TMO_DTYPE_F32, op, ": mask is not supported with float32 q");
    TORCH_CHECK(mk.dim() == 3 && mk.size(0) == B && mk.size(1) == seq_q, op,
                ": mask must be [batch, seq_q, mask_len] = [", B, ", ", seq_q, ", mask_len], got ",
                mk.sizes());
    mask_len = mk.size(2);
    TORCH_CHECK(seq_q <= 16 && mask_len >= 1 && mask_len <= 64 && mask_len % seq_q == 0, op,
                ": mask needs seq_q <= 16, 1 <= mask_len <= 64 and mask_len % seq_q == 0, got ",
                "seq_q ", seq_q, ", mask_len ", mask_len);
    if (mask_len > 1 && mk.stride(2) != 1) mk = mk.contiguous();
    mask_p = mk.data_ptr();
    mask_dt = dtype_code(mk.scalar_type());
    m_sb = mk.stride(0);
    m_ss = mk.stride(1);
  }
  // max_context_len <= 0: an uncertain maximum (reference docstring); negative counts as 0
  const int64_t max_ctx = std::max<int64_t>(0, max_context_len.expect_int());
  const int64_t window = windows_size_left.expect_int();
  if (B == 0 || seq_q == 0) return;
  // Splits: about twelve workgroups per CU (3072) when the batch alone does not give them, at
  // least 256 keys per split, at most 63 splits -- and an odd count.  The kernel's grid runs
  // the splits of one (sequence, KV head) on consecutive workgroups, which the dispatcher deals
  // round-robin to the 8 XCDs: with 8 (or 4) splits every first chunk lands on one XCD (or
  // two) and the mostly empty last chunks of short contexts on another, while a count coprime
  // with 8 spreads them.  configs[4]'s 512 (sequence, KV head) pairs, splits 1..10: 681, 726,
  // 595, 673, 556, 571, 550, 713, 561, 590 us (5 vs 7 repeated on one box: 560 vs 545).
  int64_t splits = 1;
  const int64_t pairs = B * Hkv * ((seq_q * (Hq / Hkv) + 15) / 16);  // x column blocks
  if (max_ctx > 0 && pairs < 3072) {
    const int64_t want = (3072 + pairs - 1) / pairs;
    const int64_t cap = (max_ctx + 255) / 256;
    splits = std::max<int64_t>(1, std::min<int64_t>({want, cap, 63}));
    if (splits > 1 && splits % 2 == 0) splits += splits + 1 <= cap ? 1 : -1;
  }
  c10::DeviceGuard guard(q_ori.device());
  at::Tensor ws;
  const int64_t ws_bytes = tmo_hip_cached_kv_attn_workspace_bytes(B, Hkv, Hq, Dv, seq_q, splits);
  if (ws_bytes > 0)
    ws = at::empty({(ws_bytes + 3) / 4}, q_ori.options().dtype(at::kFloat));
  const bool scaled = int8 || same_as_q;
  const int st = tmo_hip_cached_kv_attn(
      q.data_ptr(), q_sb, q_ss, q.stride(-2), qquant ? qst.data_ptr() : nullptr, qs_mode, qs_dt,
      qs_sb, qs_ss, qs_sh, qs_groups, cu, seq_q, total_q, k_cache.data_ptr(),
      v_cache.has_value() ? v_cache->data_ptr() : nullptr, kdim, vdim,
      scaled ? ks.data_ptr() : nullptr, scaled ? vs.data_ptr() : nullptr, smode,
      scaled && ks.scalar_type() == at::kBFloat16 ? TMO_DTYPE_BF16 : TMO_DTYPE_F32,
      ks_sb, ks_sh, vs_sb, vs_sh, block_tables.data_ptr<int32_t>(), block_tables.size(-1),
      bt_heads, context_lens.data_ptr<int32_t>(), alibi, sink_p, mask_p, mask_dt, mask_len, m_sb,
      m_ss, out.data_ptr(), o_sb, o_ss, out.stride(-2), lse, lse_sb, lse_ss, lse_sh, B, Hq, Hkv,
      D, Dv, NB, BS, max_ctx, window, static_cast<float>(softmax_scale), qdt, cdt,
      v_pair_channels, odt, splits, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
      stream_of(q_ori));
  check_status(st, op);
}

}  // namespace torch_api
}  // namespace tmo

TORCH_LIBRARY(torch_mlu_ops, m) {
  m.def(
      "reshape_paged_cache(Tensor(a!) k, Tensor(b!)? v, Tensor(c!) k_cache, Tensor(d!)? v_cache, "
      "Tensor slot_mapping, bool direction) -> ()");
  m.def(
      "quant_to_paged_cache(Tensor k, Tensor? v, Tensor(a!) k_cache, Tensor(b!)? v_cache, "
      "Tensor(c!) k_cache_scale, Tensor(d!)? v_cache_scale, Tensor slot_mapping) -> ()");
  m.def(
      "offline_quant_to_paged_cache(Tensor k, Tensor? v, Tensor? k_cache_scale_per_channel, "
      "Tensor? v_cache_scale_per_channel, Tensor slot_mapping, Tensor(a!) k_cache, "
      "Tensor(b!)? v_cache, float k_cache_scale_per_tensor, float v_cache_scale_per_tensor) -> ()");
  m.def(
      "fused_rope(Tensor(a!) qkv, Tensor(b!) key_cache_hp, Tensor(c!) value_cache_hp, "
      "Tensor(d!)? key_cache_lp, Tensor(e!)? value_cache_lp, Tensor sin_table, Tensor cos_table, "
      "Tensor position_ids, Tensor gamma, Tensor? k_beta, Tensor(f!)? key_scale_hp, "
      "Tensor(g!)? value_scale_hp, Tensor(h!)? key_scale_lp, Tensor(i!)? value_scale_lp, "
      "Tensor? cache_bs_id_hp, Tensor? cache_seq_offsets_hp, Tensor? cache_bs_id_lp, "
      "Tensor? cache_seq_offsets_lp, Tensor? slot_mapping_hp, Tensor? slot_mapping_lp, "
      "str norm_type, SymInt rope_dim_offset, float eps, Tensor? q_gamma=None) -> ()");
  m.def(
      "dequant_from_paged_cache(Tensor(a!) key, Tensor(b!)? value, Tensor key_cache, "
      "Tensor? value_cache, Tensor key_cache_quant_scale, Tensor? value_cache_quant_scale, "
      "Tensor context_lengths, SymInt max_context_len, Tensor? context_seq_offset, "
      "Tensor block_tables, int quant_mode, int quant_bit) -> ()");
  m.def(
      "scaled_quantize(Tensor x, Tensor(a!) output, Tensor(b!)? output_scale, Tensor? x_scale, "
      "Tensor? x_zero, Tensor? m_list, Tensor? gather_index, Tensor? gather_index_start_position, "
      "Tensor? scale_upper_bound, str quant_mode, str act_mode, float active_coef, bool is_gated, "
      "int quant_bit_size=8, bool need_output_scale_trans=False, Tensor(c!)? output_reduced=None, "
      "int group_size=1) -> ()");
  m.def(
      "reshape_linear_cache(Tensor key, Tensor? value, Tensor(a!) key_cache, "
      "Tensor(b!)? value_cache, Tensor context_lengths, SymInt max_context_len, bool packed, "
      "Tensor? context_seq_offset, Tensor? cache_bs_id, Tensor? cache_seqlen_offset) -> ()");
  m.def(
      "quant_to_linear_cache(Tensor key, Tensor? value, Tensor(a!) key_cache, "
      "Tensor(b!)? value_cache, Tensor(c!) key_cache_scale, Tensor(d!)? value_cache_scale, "
      "Tensor context_lengths, SymInt max_context_len, bool packed, Tensor? context_seq_offset, "
      "Tensor? cache_bs_id, Tensor? cache_seqlen_offset, int quant_bit=8) -> ()");
  m.def(
      "offline_quant_to_linear_cache(Tensor key, Tensor? value, Tensor(a!) key_cache, "
      "Tensor(b!)? value_cache, Tensor? key_cache_scale, Tensor? value_cache_scale, "
      "Tensor context_lengths, SymInt max_context_len, int quant_mode, bool packed, "
      "Tensor? context_seq_offset, Tensor? cache_bs_id, Tensor? cache_seqlen_offset, "
      "float key_cache_scale_per_tensor, float value_cache_scale_per_tensor) -> ()");
  m.def(
      "dequant_from_linear_cache(Tensor(a!) key, Tensor(b!)? value, Tensor key_cache, "
      "Tensor? value_cache, Tensor key_cache_quant_scale, Tensor? value_cache_quant_scale, "
      "Tensor context_lengths, SymInt max_context_len, Tensor? context_seq_offset, "
      "Tensor? cache_bs_id, Tensor? cache_seq_offset, int quant_mode=0, int quant_bit=8) -> ()");
  m.def(
      "single_query_cached_kv_attn(Tensor q_ori, Tensor k_cache, Tensor(a!) output, "
      "Tensor block_tables, Tensor context_lens, Tensor? v_cache, Tensor(b!)? output_lse, "
      "Tensor? q_quant_scale, Tensor? k_cache_quant_scale, Tensor? v_cache_quant_scale, "
      "Tensor? out_quant_scale, Tensor? alibi_slopes, Tensor? mask, str compute_dtype, "
      "SymInt max_context_len, SymInt windows_size_left, SymInt windows_size_right, "
      "float softmax_scale, bool return_lse, int kv_cache_quant_bit_size, "
      "Tensor? cu_seq_q=None, SymInt max_seq_q=-1, Tensor? sink=None) -> ()");
  m.def(
      "reshape_from_cache(Tensor(a!) key, Tensor(b!)? value, Tensor key_cache, "
      "Tensor? value_cache, Tensor context_lengths, SymInt max_context_len, "
      "Tensor? context_seq_offset=None, Tensor? block_tables=None, "
      "Tensor? cache_seq_offset=None) -> ()");
}

TORCH_LIBRARY_IMPL(torch_mlu_ops, CUDA, m) {
  m.impl("reshape_paged_cache", &tmo::torch_api::reshape_paged_cache);
  m.impl("quant_to_paged_cache", &tmo::torch_api::quant_to_paged_cache);
  m.impl("offline_quant_to_paged_cache", &tmo::torch_api::offline_quant_to_paged_cache);
  m.impl("dequant_from_paged_cache", &tmo::torch_api::dequant_from_paged_cache);
  m.impl("fused_rope", &tmo::torch_api::fused_rope);
  m.impl("scaled_quantize", &tmo::torch_api::scaled_quantize);
  m.impl("reshape_linear_cache", &tmo::torch_api::reshape_linear_cache);
  m.impl("quant_to_linear_cache", &tmo::torch_api::quant_to_linear_cache);
  m.impl("offline_quant_to_linear_cache", &tmo::torch_api::offline_quant_to_linear_cache);
  m.impl("dequant_from_linear_cache", &tmo::torch_api::dequant_from_linear_cache);
  m.impl("reshape_from_cache", &tmo::torch_api::reshape_from_cache);
  m.impl("single_query_cached_kv_attn", &tmo::torch_api::single_query_cached_kv_attn);
}
