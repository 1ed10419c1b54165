"""Fake (meta) kernels of the path's ops, registered unconditionally.

The reference registers its fakes only when ``torch.__version__ >= '2.3.0'`` holds as a
*string* comparison (reference ``__init__.py:3``), which is False for torch 2.10, so on
current torch it registers none.  Here they are always registered.  Every op writes its
outputs in place and returns nothing (reference ``abstract.py:148-152``, ``172-182``,
``746-761``, ``811-832``); the fake of ``scaled_quantize`` follows the C++ parameter order
(reference ``include/torch_mlu_ops.h:334-350``), without the extra ``quant_type`` parameter
of reference ``abstract.py:822``.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

__all__: list = []


@torch.library.register_fake("torch_mlu_ops::reshape_paged_cache")
def reshape_paged_cache_abstract(k: Tensor, v: Optional[Tensor], k_cache: Tensor,
                                 v_cache: Optional[Tensor], slot_mapping: Tensor,
                                 direction: bool) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::quant_to_paged_cache")
def quant_to_paged_cache_abstract(k: Tensor, v: Optional[Tensor], k_cache: Tensor,
                                  v_cache: Optional[Tensor], k_cache_scale: Tensor,
                                  v_cache_scale: Optional[Tensor], slot_mapping: Tensor) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::offline_quant_to_paged_cache")
def offline_quant_to_paged_cache_abstract(k: Tensor, v: Optional[Tensor],
                                          k_cache_scale_per_channel: Optional[Tensor],
                                          v_cache_scale_per_channel: Optional[Tensor],
                                          slot_mapping: Tensor, k_cache: Tensor,
                                          v_cache: Optional[Tensor],
                                          k_cache_scale_per_tensor: float,
                                          v_cache_scale_per_tensor: float) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::fused_rope")
def fused_rope_abstract(qkv: Tensor, key_cache_hp: Tensor, value_cache_hp: Tensor,
                        key_cache_lp: Optional[Tensor], value_cache_lp: Optional[Tensor],
                        sin_table: Tensor, cos_table: Tensor, position_ids: Tensor,
                        gamma: Tensor, k_beta: Optional[Tensor], key_scale_hp: Optional[Tensor],
                        value_scale_hp: Optional[Tensor], key_scale_lp: Optional[Tensor],
                        value_scale_lp: Optional[Tensor], cache_bs_id_hp: Optional[Tensor],
                        cache_seq_offsets_hp: Optional[Tensor], cache_bs_id_lp: Optional[Tensor],
                        cache_seq_offsets_lp: Optional[Tensor], slot_mapping_hp: Optional[Tensor],
                        slot_mapping_lp: Optional[Tensor], norm_type: str, rope_dim_offset: int,
                        eps: float, q_gamma: Optional[Tensor] = None) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::dequant_from_paged_cache")
def dequant_from_paged_cache_abstract(key: Tensor, value: Optional[Tensor], key_cache: Tensor,
                                      value_cache: Optional[Tensor],
                                      key_cache_quant_scale: Tensor,
                                      value_cache_quant_scale: Optional[Tensor],
                                      context_lengths: Tensor, max_context_len: int,
                                      context_seq_offset: Optional[Tensor], block_tables: Tensor,
                                      quant_mode: int = 0, quant_bit: int = 8) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::scaled_quantize")
def scaled_quantize_abstract(x: Tensor, output: Tensor, output_scale: Optional[Tensor],
                             x_scale: Optional[Tensor] = None, x_zero: Optional[Tensor] = None,
                             m_list: Optional[Tensor] = None,
                             gather_index: Optional[Tensor] = None,
                             gather_index_start_position: Optional[Tensor] = None,
                             scale_upper_bound: Optional[Tensor] = None,
                             quant_mode: str = "dynamic_per_token", act_mode: str = "none",
                             active_coef: float = 1.0, is_gated: bool = False,
                             quant_bit_size: int = 8, need_output_scale_trans: bool = False,
                             output_reduced: Optional[Tensor] = None,
                             group_size: int = 1) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::reshape_linear_cache")
def reshape_linear_cache_abstract(key: Tensor, value: Optional[Tensor], key_cache: Tensor,
                                  value_cache: Optional[Tensor], context_lengths: Tensor,
                                  max_context_len: int, packed: bool,
                                  context_seq_offset: Optional[Tensor],
                                  cache_bs_id: Optional[Tensor],
                                  cache_seqlen_offset: Optional[Tensor]) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::quant_to_linear_cache")
def quant_to_linear_cache_abstract(key: Tensor, value: Optional[Tensor], key_cache: Tensor,
                                   value_cache: Optional[Tensor], key_cache_scale: Tensor,
                                   value_cache_scale: Optional[Tensor], context_lengths: Tensor,
                                   max_context_len: int, packed: bool,
                                   context_seq_offset: Optional[Tensor],
                                   cache_bs_id: Optional[Tensor],
                                   cache_seqlen_offset: Optional[Tensor],
                                   quant_bit: int = 8) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::offline_quant_to_linear_cache")
def offline_quant_to_linear_cache_abstract(key: Tensor, value: Optional[Tensor],
                                           key_cache: Tensor, value_cache: Optional[Tensor],
                                           key_cache_scale: Optional[Tensor],
                                           value_cache_scale: Optional[Tensor],
                                           context_lengths: Tensor, max_context_len: int,
                                           quant_mode: int, packed: bool,
                                           context_seq_offset: Optional[Tensor],
                                           cache_bs_id: Optional[Tensor],
                                           cache_seqlen_offset: Optional[Tensor],
                                           key_cache_scale_per_tensor: float,
                                           value_cache_scale_per_tensor: float) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::dequant_from_linear_cache")
def dequant_from_linear_cache_abstract(key: Tensor, value: Optional[Tensor], key_cache: Tensor,
                                       value_cache: Optional[Tensor],
                                       key_cache_quant_scale: Tensor,
                                       value_cache_quant_scale: Optional[Tensor],
                                       context_lengths: Tensor, max_context_len: int,
                                       context_seq_offset: Optional[Tensor],
                                       cache_bs_id: Optional[Tensor],
                                       cache_seq_offset: Optional[Tensor],
                                       quant_mode: int = 0, quant_bit: int = 8) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::reshape_from_cache")
def reshape_from_cache_abstract(key: Tensor, value: Optional[Tensor], key_cache: Tensor,
                                value_cache: Optional[Tensor], context_lengths: Tensor,
                                max_context_len: int, context_seq_offset: Optional[Tensor] = None,
                                block_tables: Optional[Tensor] = None,
                                cache_seq_offset: Optional[Tensor] = None) -> None:
    return None


@torch.library.register_fake("torch_mlu_ops::single_query_cached_kv_attn")
def single_query_cached_kv_attn_abstract(q_ori: Tensor, k_cache: Tensor, output: Tensor,
                                         block_tables: Tensor, context_lens: Tensor,
                                         v_cache: Optional[Tensor], output_lse: Optional[Tensor],
                                         q_quant_scale: Optional[Tensor],
                                         k_cache_quant_scale: Optional[Tensor],
                                         v_cache_quant_scale: Optional[Tensor],
                                         out_quant_scale: Optional[Tensor],
                                         alibi_slopes: Optional[Tensor], mask: Optional[Tensor],
                                         compute_dtype: str, max_context_len: int,
                                         windows_size_left: int, windows_size_right: int,
                                         softmax_scale: float, return_lse: bool,
                                         kv_cache_quant_bit_size: int,
                                         cu_seq_q: Optional[Tensor] = None, max_seq_q: int = -1,
                                         sink: Optional[Tensor] = None) -> None:
    return None

