"""Python op surface of the quantized paged-KV-cache path.

Signatures, argument meaning and return conventions are those of the reference wrappers
(cited per function); each wrapper is a call of the ``torch_mlu_ops::*`` op registered by
``_lib/_tmo_torch.so``, whose HIP kernel calls the C ABI of ``include/tmo_hip.h``.  Outputs are
written in place; the wrappers allocate only where the reference wrappers do.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

__all__ = [
    "reshape_paged_cache",
    "quant_to_paged_cache",
    "offline_quant_to_paged_cache",
    "fused_rope",
    "fused_rmsnorm_rope_store_paged_cache",
    "dequant_from_paged_cache",
    "moe_quantize",
    "scaled_quantize",
    "per_token_smooth_quantize",
    "reshape_linear_cache",
    "quant_to_linear_cache",
    "offline_quant_to_linear_cache",
    "dequant_from_linear_cache",
    "reshape_from_cache",
    "single_query_cached_kv_attn",
]


def reshape_paged_cache(
    k: torch.Tensor,
    v: Optional[torch.Tensor],
    k_cache: torch.Tensor,
    v_cache: Optional[torch.Tensor],
    slot_mapping: torch.Tensor,
    direction: bool = False,
) -> Union[Tuple[torch.Tensor], torch.Tensor]:
    """Scatter k/v ``[num_tokens, heads, head_size]`` rows into the paged caches
    ``[num_blocks, heads, block_size, head_size]`` at ``slot_mapping`` (``direction=False``),
    or gather them back into k/v (``direction=True``).  Tokens whose slot is negative are
    skipped.  Byte-exact for float, half, bfloat16 and int8.

    Reference: ``_ops.py:1251-1294`` (math ``:1262-1268``).  Returns k (and v) when
    ``direction`` is True, else k_cache (and v_cache), as the reference does.
    """
    torch.ops.torch_mlu_ops.reshape_paged_cache(k, v, k_cache, v_cache, slot_mapping, direction)
    if direction:
        return (k, v) if v is not None else k
    return (k_cache, v_cache) if v_cache is not None else k_cache


def quant_to_paged_cache(
    k: torch.Tensor,
    v: Optional[torch.Tensor],
    k_cache: torch.Tensor,
    v_cache: Optional[torch.Tensor],
    k_cache_quant_scale: torch.Tensor,
    v_cache_quant_scale: Optional[torch.Tensor],
    slot_mapping: torch.Tensor,
) -> Tuple[torch.Tensor]:
    """Dynamic per-(token, head) quantisation of k/v into the paged caches.

    For each token ``i`` with ``slot_mapping[i] >= 0`` and each head ``h``: int8 caches
    ``scale = fp32(max|k[i, h]|) / 127``, ``code = clip(round_half_even(k[i, h] / scale),
    -128, 127)``; ``torch.float8_e4m3fn`` caches ``scale = fp32(max|k[i, h]|) / 448``,
    ``code = clip(k[i, h] / scale, -448, 448)`` rounded to nearest even.  Codes go to
    ``k_cache[slot // bs, h, slot % bs]`` and the scale to ``k_cache_quant_scale[slot // bs,
    h, slot % bs]`` (same for v).  An all-zero row stores scale 0 and codes 0.  k/v: float,
    half or bfloat16 (may be strided views).

    Reference: ``_ops.py:1511-1565`` (math ``:1524-1537``).  Returns
    ``(k_cache, v_cache, k_scale, v_scale)`` or ``(k_cache, k_scale)``.
    """
    torch.ops.torch_mlu_ops.quant_to_paged_cache(
        k, v, k_cache, v_cache, k_cache_quant_scale, v_cache_quant_scale, slot_mapping)
    if v_cache is not None:
        return (k_cache, v_cache, k_cache_quant_scale, v_cache_quant_scale)
    return (k_cache, k_cache_quant_scale)


def offline_quant_to_paged_cache(
    k: torch.Tensor,
    v: Optional[torch.Tensor],
    k_cache_scale: Union[torch.Tensor, float],
    v_cache_scale: Optional[Union[torch.Tensor, float]],
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: Optional[torch.Tensor],
) -> Union[Tuple[torch.Tensor], torch.Tensor]:
    """Static quantisation of k/v into the paged caches with calibrated scales.

    For each token ``i`` with ``slot_mapping[i] >= 0``: ``q = fp32(k[i]) / k_cache_scale``
    (IEEE divide; a ``[heads, head_size]`` float32 tensor scales per channel, a number per
    tensor); an int8 cache stores ``clip(round_half_even(q), -128, 127)``, a
    ``torch.float8_e4m3fn`` cache stores ``clip(q, -448, 448)`` rounded to nearest even, at
    ``k_cache[slot // bs, :, slot % bs, :]`` (same for v).  No scales are written.

    Reference: ``_ops.py:1639-1706`` (math ``:1652-1670``; the division is the linear
    sibling's ``key_i /= scale``, ``:1829-1840``).  Returns ``(k_cache, v_cache)`` or
    ``k_cache``.
    """
    if torch.is_tensor(k_cache_scale):
        torch.ops.torch_mlu_ops.offline_quant_to_paged_cache(
            k, v, k_cache_scale, v_cache_scale, slot_mapping, k_cache, v_cache, 1.0, 1.0)
    else:
        torch.ops.torch_mlu_ops.offline_quant_to_paged_cache(
            k, v, None, None, slot_mapping, k_cache, v_cache, k_cache_scale,
            v_cache_scale if v_cache_scale is not None else 1.0)
    return (k_cache, v_cache) if v_cache is not None else k_cache


def fused_rope(
    qkv: torch.Tensor,
    k_cache_hp: torch.Tensor,
    v_cache_hp: torch.Tensor,
    sin_cache: torch.Tensor,
    cos_cache: torch.Tensor,
    position_id: torch.Tensor,
    k_gamma: torch.Tensor,
    k_beta: Optional[torch.Tensor],
    k_cache_lp: Optional[torch.Tensor] = None,
    v_cache_lp: Optional[torch.Tensor] = None,
    cache_bs_id_hp: Optional[torch.Tensor] = None,
    cache_seq_offsets_hp: Optional[torch.Tensor] = None,
    cache_bs_id_lp: Optional[torch.Tensor] = None,
    cache_seq_offsets_lp: Optional[torch.Tensor] = None,
    k_scale_hp: Optional[torch.Tensor] = None,
    v_scale_hp: Optional[torch.Tensor] = None,
    k_scale_lp: Optional[torch.Tensor] = None,
    v_scale_lp: Optional[torch.Tensor] = None,
    slot_mapping_hp: Optional[torch.Tensor] = None,
    slot_mapping_lp: Optional[torch.Tensor] = None,
    norm_type: str = "layernorm",
    rope_dim_offset: int = 0,
    eps: float = 1e-5,
    q_gamma: Optional[torch.Tensor] = None,
):
    """Fold rotary embedding + a norm + store of K and V into paged caches, in one pass over
    ``qkv [batch, seq_len, q_heads + 2 kv_heads, head_size]``.  ``norm_type="rmsnorm"``: RMSNorm
    of Q (with ``q_gamma`` unless None) and of K (``k_gamma``), then the rotation.
    ``norm_type="layernorm"``: Q and K rotated, then K layer-normalised (biased variance) with
    ``k_gamma`` and ``k_beta`` (None: no shift); ``q_gamma`` is not used.  V is stored as it is.

    Token ``(b, s)`` is rotated at position ``position_id[b] + s`` with rows of
    ``sin_cache`` / ``cos_cache [rotary_seq, rope_dim]`` over head dims
    ``[rope_dim_offset, rope_dim_offset + rope_dim)``; Q is written back into ``qkv``; K and V
    go to ``k_cache_hp`` / ``v_cache_hp [num_blocks, kv_heads, block_size, head_size]`` at
    ``slot_mapping_hp`` (negative slots skipped): in qkv's dtype, or int8 with ``k_scale_hp`` /
    ``v_scale_hp`` either ``[num_blocks, kv_heads, block_size]`` (dynamic per-token scales,
    written) or ``[kv_heads, head_size]`` (static per-channel scales, read).  fp32 arithmetic
    with one final rounding.  Without ``slot_mapping_hp`` the caches are linear ``[max_batch,
    kv_heads, cache_len, head_size]``: sequence b goes to cache batch ``cache_bs_id_hp[b]``
    (default b) from position ``cache_seq_offsets_hp[b]`` (default 0), rows outside the cache
    skipped, dynamic scales ``[max_batch, kv_heads, cache_len]``.  The low-precision (int4)
    caches raise ``RuntimeError``.

    Reference: ``_ops.py:3469-3601`` (math ``:3496-3520``, rotary math ``:1116-1127``).
    Returns ``(qkv, k_cache_hp, v_cache_hp)`` (plus the low-precision tensors when given).
    """
    torch.ops.torch_mlu_ops.fused_rope(qkv, k_cache_hp, v_cache_hp, k_cache_lp, v_cache_lp,
            sin_cache, cos_cache, position_id, k_gamma, k_beta, k_scale_hp, v_scale_hp,
            k_scale_lp, v_scale_lp, cache_bs_id_hp, cache_seq_offsets_hp,
            cache_bs_id_lp, cache_seq_offsets_lp, slot_mapping_hp, slot_mapping_lp,
            norm_type, rope_dim_offset, eps, q_gamma)
    out = (qkv, k_cache_hp, v_cache_hp)
    if k_cache_lp is not None:
        out += (k_cache_lp, v_cache_lp)
        if k_scale_lp is not None:
            out += (k_scale_lp, v_scale_lp)
    return out


def fused_rmsnorm_rope_store_paged_cache(
    qkv: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    sin_cache: torch.Tensor,
    cos_cache: torch.Tensor,
    position_id: torch.Tensor,
    k_gamma: torch.Tensor,
    q_gamma: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    eps: float = 1e-5,
):
    """RMSNorm (Q with ``q_gamma`` unless None, K with ``k_gamma``) + RoPE + store of K and V
    into the paged caches, one kernel; see ``fused_rope`` for the layouts and the quantised
    cache forms.

    Reference: ``_ops.py:6356-6423``.  Returns ``(qkv, k_cache, v_cache)`` plus
    ``(k_scale, v_scale)`` when quantising.
    """
    torch.ops.torch_mlu_ops.fused_rope(qkv, k_cache, v_cache, None, None,
        sin_cache, cos_cache, position_id, k_gamma, None, k_scale, v_scale,
        None, None, None, None, None, None, slot_mapping, None, "rmsnorm", 0, eps, q_gamma)
    out = (qkv, k_cache, v_cache)
    if k_scale is not None:
        out += (k_scale, v_scale)
    return out


def dequant_from_paged_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    key_cache_quant_scale: torch.Tensor,
    value_cache_quant_scale: Optional[torch.Tensor],
    context_lengths: torch.Tensor,
    max_context_len: int,
    context_seq_offset: Optional[torch.Tensor],
    block_tables: torch.Tensor,
    quant_mode: int = 0,
    quant_bit: int = 8,
) -> None:
    """Gather each sequence's pages through ``block_tables`` and write
    ``key[begin_i + t] = (fp32(code) * scale).to(key.dtype)`` for ``t < context_lengths[i]``;
    ``begin_i`` is ``context_seq_offset[i]`` or the running sum of ``context_lengths``.
    ``quant_mode`` 0: per-channel scale ``[heads, head_size]``; 1: per-token scale
    ``[num_blocks, heads, block_size]``; scales float32 or bfloat16.  The caches are int8, or
    the ``torch.float8_e4m3fn`` pages ``quant_to_paged_cache`` writes (code = the e4m3fn
    value).  ``quant_bit`` must be 8 (the mx-fp6 mode 2 is not part of this build).

    Reference: ``_ops.py:3734-3824`` (math ``:3749-3774``).  Returns None.
    """
    torch.ops.torch_mlu_ops.dequant_from_paged_cache(
        key, value, key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale,
        context_lengths, max_context_len, context_seq_offset, block_tables, quant_mode, quant_bit)


def moe_quantize(
    x: torch.Tensor,
    smooth: torch.Tensor,
    zero: Optional[torch.Tensor] = None,
    token_count: Optional[torch.Tensor] = None,
    gather_index: Optional[torch.Tensor] = None,
    gather_index_start_position: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
    output_scale: Optional[torch.Tensor] = None,
    dynamic_quant: bool = True,
    act_mode: str = "none",
    active_coef: float = 1.0,
    is_gated: bool = False,
    quant_type: torch.dtype = torch.int8,
    quant_bit_size=8,
    scale_type=torch.float32,
    need_output_scale_trans: bool = False,
    output_reduced: Optional[torch.Tensor] = None,
    group_size: int = 1,
) -> Tuple[torch.Tensor]:
    """Smooth + dynamic per-token int8 quantisation, optionally over gathered rows
    (``x[gather_index]``) with per-group smooth rows (``token_count`` splits the rows into
    groups, group ``g`` uses ``smooth[g]``):
    ``smoothed = fp32(x) * smooth``; ``scale = max|smoothed| / 127``;
    ``output = clip(round_half_even(smoothed / scale), -128, 127)``.

    Reference: ``_ops.py:3126-3253`` (math ``:3147-3176``, shapes ``:3220-3248``).  This build
    implements ``dynamic_quant=True``, ``act_mode="none"``, int8 output and fp32 scales; the
    other modes raise RuntimeError from the op.  Returns ``(output, output_scale)``.
    """
    tokens, ci = x.shape[0], x.shape[-1]
    if gather_index is not None:
        tokens = gather_index.size(0)
    if quant_type == torch.int8 and quant_bit_size == 4:
        ci = ci // 2 // (1 + is_gated)
    else:
        ci = ci // (1 + is_gated)
    output_shape = ((tokens,) + tuple(x.shape[1:-1]) + (ci,))[: x.dim()]
    scale_shape = ((tokens,) + tuple(x.shape[1:-1]))[: x.dim() - 1]
    if output is None:
        output = torch.empty(output_shape, dtype=quant_type, device=x.device)
    if output_scale is None and dynamic_quant:
        output_scale = torch.empty(scale_shape, dtype=scale_type, device=x.device)
    torch.ops.torch_mlu_ops.scaled_quantize(
        x, output, output_scale, smooth, zero, token_count, gather_index,
        gather_index_start_position, None,
        "dynamic_per_token" if dynamic_quant else "static_per_channel",
        act_mode, active_coef, is_gated, quant_bit_size, need_output_scale_trans,
        output_reduced, group_size)
    return (output, output_scale) if dynamic_quant else (output,)


def scaled_quantize(
    x: torch.Tensor,
    scale: Optional[torch.Tensor] = None,
    zero: Optional[torch.Tensor] = None,
    scale_ub: Optional[torch.Tensor] = None,
    quant_type=torch.int8,
    quant_mode: str = "dynamic_per_token",
    act_mode: str = "none",
    active_coef: float = 1.0,
    is_gated: bool = False,
    quant_bit_size: int = 8,
    scale_type=torch.float32,
    need_output_scale_trans: bool = False,
    output_reduced: Optional[torch.Tensor] = None,
    group_size: int = 1,
) -> Tuple[torch.Tensor]:
    """Per-token int8 quantisation of ``x [..., C]`` with an optional smooth vector
    ``scale`` (shape ``[C]`` or ``[1]``).

    Reference: ``_ops.py:4407-4492``.  This build implements ``quant_mode="dynamic_per_token"``
    with int8 output and fp32 scales (``act_mode="none"``).  Returns ``(output, output_scale)``.
    """
    is_dynamic = quant_mode in ("dynamic_per_token", "dynamic_per_tensor")
    cols = x.size(-1) // (1 + is_gated)
    if quant_type == torch.int8 and quant_bit_size == 4:
        cols = x.size(-1) // 2 // (1 + is_gated)
    output = torch.empty(x.size()[:-1] + (cols,), dtype=quant_type, device=x.device)
    output_scale = None
    if quant_mode == "dynamic_per_tensor":
        output_scale = torch.empty(1, dtype=torch.float32, device=x.device)
    elif quant_mode == "dynamic_per_token":
        output_scale = torch.empty(x.size()[:-1], dtype=scale_type, device=x.device)
    torch.ops.torch_mlu_ops.scaled_quantize(
        x, output, output_scale, scale, zero, None, None, None, scale_ub, quant_mode, act_mode,
        active_coef, is_gated, quant_bit_size, need_output_scale_trans, output_reduced,
        group_size)
    return (output, output_scale) if is_dynamic else output


def per_token_smooth_quantize(
    x: torch.Tensor,
    smooth: torch.Tensor,
    zero: Optional[torch.Tensor] = None,
    token_count: Optional[torch.Tensor] = None,
    gather_index: Optional[torch.Tensor] = None,
    gather_index_start_position: Optional[torch.Tensor] = None,
    output: Optional[torch.Tensor] = None,
    output_scale: Optional[torch.Tensor] = None,
    dynamic_quant: bool = True,
) -> Tuple[torch.Tensor]:
    """Alias of :func:`moe_quantize` restricted to its smooth-quant arguments.

    Not a reference API: the reference exposes this operation as ``moe_quantize``
    (``_ops.py:3126-3253``) and ``scaled_quantize`` (``_ops.py:4407-4492``), both lowering to
    the op ``scaled_quantize`` in mode ``'dynamic_per_token'``.  Returns
    ``(output, output_scale)``.
    """
    return moe_quantize(x, smooth, zero, token_count, gather_index, gather_index_start_position,
                        output, output_scale, dynamic_quant)


# ---------------------------------------------------------------------------- linear caches
#
# Linear caches are [max_batch, heads, cache_len, head_size], one cache batch per sequence.
# Sequence i covers min(len_i, max_context_len) tokens; token j is row start_i + j of the
# token-major tensor (start_i = context_seq_offset[i], else the packed prefix offset / i *
# seqlen for padded input / the running sum of the lengths for outputs) and sits at cache
# position cache_seq_offset[i] + j of cache batch cache_bs_id[i] (default i; negative: skip).
# Tokens outside the cache or the token tensor are skipped.


def reshape_linear_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    context_lengths: torch.Tensor,
    max_context_len: int,
    packed: bool,
    context_seq_offset: Optional[torch.Tensor],
    cache_bs_id: Optional[torch.Tensor],
    cache_seqlen_offset: Optional[torch.Tensor],
) -> Union[Tuple[torch.Tensor], torch.Tensor]:
    """Copy key/value token rows (packed ``[total, heads, head_size]`` with ``context_lengths``
    holding batch + 1 offsets, or padded ``[batch, seqlen, heads, head_size]`` with lengths)
    into the linear caches, byte for byte (float, half, bfloat16, int8).

    Reference: ``_ops.py:1189-1249``.  Returns ``(key_cache, value_cache)`` or ``key_cache``.
    """
    torch.ops.torch_mlu_ops.reshape_linear_cache(
        key, value, key_cache, value_cache, context_lengths, max_context_len, packed,
        context_seq_offset, cache_bs_id, cache_seqlen_offset)
    return (key_cache, value_cache) if value_cache is not None else key_cache


def quant_to_linear_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    key_cache_quant_scale: torch.Tensor,
    value_cache_quant_scale: Optional[torch.Tensor],
    context_lengths: torch.Tensor,
    max_context_len: int,
    packed: bool,
    context_seq_offset: Optional[torch.Tensor],
    cache_bs_id: Optional[torch.Tensor],
    cache_seqlen_offset: Optional[torch.Tensor],
    quant_bit: int = 8,
) -> Tuple[torch.Tensor]:
    """Dynamic quantisation of key/value into the linear caches, per (token, head) (scale
    ``[max_batch, heads, cache_len]``) or per group of ``head_size / group_num`` channels (scale
    ``[..., group_num]``).  int8 caches: ``scale = fp32(amax) / 127``, ``code =
    clip(round_half_even(x / scale), -128, 127)``; float8_e4m3fn caches: ``scale = fp32(amax) /
    448``, ``code = clip(x / scale, -448, 448)`` rounded to nearest even.  An all-zero group
    stores scale 0 and codes 0.  ``quant_bit`` 4 (int8 caches of int4 pairs): ``scale =
    fp32(amax) / 7``, ``code = clip(round_half_even(x / scale), -8, 7)``, two codes per byte with
    the even element in the high nibble; ``key_cache`` ``[max_batch, heads, cache_len,
    head_size / 2]`` pairs channels, ``value_cache`` ``[max_batch, heads, cache_len / 2,
    head_size]`` pairs cache positions (a position written alone keeps its partner's nibble);
    ``head_size`` a multiple of 8, at most 512.

    Reference: ``_ops.py:1708-1806`` (math ``:1725-1750``).  Returns
    ``(key_cache, value_cache, key_scale, value_scale)`` or ``(key_cache, key_scale)``.
    """
    torch.ops.torch_mlu_ops.quant_to_linear_cache(
        key, value, key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale,
        context_lengths, max_context_len, packed, context_seq_offset, cache_bs_id,
        cache_seqlen_offset, quant_bit)
    if value_cache is not None:
        return (key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale)
    return (key_cache, key_cache_quant_scale)


def offline_quant_to_linear_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    key_cache_quant_scale: Union[torch.Tensor, float],
    value_cache_quant_scale: Optional[Union[torch.Tensor, float]],
    context_lengths: torch.Tensor,
    max_context_len: int,
    quant_mode: int,
    packed: bool,
    context_seq_offset: Optional[torch.Tensor],
    cache_bs_id: Optional[torch.Tensor],
    cache_seqlen_offset: Optional[torch.Tensor],
) -> Tuple[torch.Tensor]:
    """Static quantisation of key/value into the linear caches: ``q = fp32(x) / scale`` (IEEE
    divide) with ``quant_mode`` 0: a ``[heads, head_size]`` scale per channel, 1: a
    ``[heads, cache_len]`` scale per head and cache position, 2/3: a number; int8 caches store
    ``clip(round_half_even(q), -128, 127)``, float8_e4m3fn caches ``clip(q, -448, 448)``
    rounded to nearest even.  No scales are written.

    Reference: ``_ops.py:1808-1919`` (math ``:1829-1840``).  Returns
    ``(key_cache, value_cache, key_scale, value_scale)`` or ``(key_cache, key_scale)``.
    """
    if torch.is_tensor(key_cache_quant_scale):
        torch.ops.torch_mlu_ops.offline_quant_to_linear_cache(
            key, value, key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale,
            context_lengths, max_context_len, quant_mode, packed, context_seq_offset,
            cache_bs_id, cache_seqlen_offset, 1.0, 1.0)
    else:
        torch.ops.torch_mlu_ops.offline_quant_to_linear_cache(
            key, value, key_cache, value_cache, None, None, context_lengths, max_context_len,
            quant_mode, packed, context_seq_offset, cache_bs_id, cache_seqlen_offset,
            key_cache_quant_scale,
            value_cache_quant_scale if value_cache_quant_scale is not None else 1.0)
    if value_cache is not None:
        return (key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale)
    return (key_cache, key_cache_quant_scale)


def dequant_from_linear_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    key_cache_quant_scale: torch.Tensor,
    value_cache_quant_scale: Optional[torch.Tensor],
    context_lengths: torch.Tensor,
    max_context_len: int,
    context_seq_offset: Optional[torch.Tensor],
    cache_bs_id: Optional[torch.Tensor],
    cache_seq_offset: Optional[torch.Tensor],
    quant_mode: int = 0,
    quant_bit: int = 8,
) -> None:
    """``key[start_i + j] = (fp32(code) * scale).to(key.dtype)`` from the int8 linear caches,
    ``quant_mode`` 0: scale ``[heads, head_size]``; 1: per-token ``[max_batch, heads,
    cache_len]``.  ``context_lengths`` holds ``[batch]`` lengths.  ``quant_bit`` 4 reads int4
    pairs (even element in the high nibble, sign-extended): ``key_cache`` ``[max_batch, heads,
    cache_len, head_size / 2]`` (channel pairs), ``value_cache`` ``[max_batch, heads, cache_len
    / 2, head_size]`` (position pairs).

    Reference: ``_ops.py:3642-3732`` (math ``:3663-3683``).  Returns None.
    """
    torch.ops.torch_mlu_ops.dequant_from_linear_cache(
        key, value, key_cache, value_cache, key_cache_quant_scale, value_cache_quant_scale,
        context_lengths, max_context_len, context_seq_offset, cache_bs_id, cache_seq_offset,
        quant_mode, quant_bit)


def reshape_from_cache(
    key: torch.Tensor,
    value: Optional[torch.Tensor],
    key_cache: torch.Tensor,
    value_cache: Optional[torch.Tensor],
    context_lengths: torch.Tensor,
    max_context_len: int,
    context_seq_offset: Optional[torch.Tensor] = None,
    block_tables: Optional[torch.Tensor] = None,
    cache_seq_offset: Optional[torch.Tensor] = None,
) -> None:
    """Copy cache rows back to token-major ``key [total, heads, head_size]`` (and value).
    Linear mode (no ``block_tables``, or a ``[batch, 1]`` table naming each sequence's cache
    batch): sequence i reads positions ``cache_seq_offset[i] + j``.  Paged mode (``[batch,
    max_blocks]`` table over ``[num_blocks, heads, block_size, head_size]`` caches): position p
    is row ``p % block_size`` of page ``block_tables[i, p // block_size]``.

    Reference: ``_ops.py:3898-3969`` (math ``:3905-3926``).  Returns None.
    """
    torch.ops.torch_mlu_ops.reshape_from_cache(
        key, value, key_cache, value_cache, context_lengths, max_context_len,
        context_seq_offset, block_tables, cache_seq_offset)


# ---------------------------------------------------------------------------- decode attention

_DTYPE_STR = {torch.half: "half", torch.float: "float", torch.bfloat16: "bfloat16"}


def single_query_cached_kv_attn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: Optional[torch.Tensor],
    out: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    k_cache_quant_scale: Optional[torch.Tensor],
    v_cache_quant_scale: Optional[torch.Tensor],
    alibi_slopes: Optional[torch.Tensor],
    max_context_len: int,
    windows_size_left: int,
    windows_size_right: int,
    softmax_scale: float,
    return_lse: bool = False,
    kv_cache_quant_bit_size=-1,
    q_quant_scale: Optional[torch.Tensor] = None,
    out_quant_scale: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.half,
    compute_dtype: torch.dtype = torch.float,
    head_size_v: int = -1,
    mask: Optional[torch.Tensor] = None,
    cu_seq_q: Optional[torch.Tensor] = None,
    max_seq_q: int = -1,
    sink: Optional[torch.Tensor] = None,
):
    """Attention of each sequence's query tokens over its paged KV cache:
    ``softmax(softmax_scale * q K^T (+ alibi)) V`` per query head, keys gathered through
    ``block_tables`` from ``[num_blocks, kv_heads, block_size, head_size]`` caches -- int8 or
    ``torch.float8_e4m3fn`` (``kv_cache_quant_bit_size=8``) with per-token, per-channel,
    per-group or per-tensor float32 / bfloat16 scales, or of q's dtype (``-1``); query head h
    reads KV head ``h // (heads / kv_heads)``.  q is ``[batch,
    seq_q, heads, head_size]``, ``[total_q, heads, head_size]`` with ``cu_seq_q`` (``[batch +
    1]``, ``max_seq_q`` an upper bound of the counts or <= 0 for unknown) or ``[batch, heads,
    head_size]``.  A sequence's nq tokens are its last nq positions: token s (position
    ``P = L - nq + s``) sees keys ``[max(0, P - windows_size_left), P]``, ALiBi adds
    ``slope * (j - P)``, and ``sink`` (``[heads]`` float logits) joins the softmax
    denominator only.  ``kv_cache_quant_bit_size=4``: int8 caches of signed int4 pairs (even
    element in the high nibble), K ``[num_blocks, kv_heads, block_size, head_size // 2]``, V
    ``[num_blocks, kv_heads, block_size // 2, head_size_v]`` (rows paired) or ``[...,
    block_size, head_size_v // 2]`` (channels paired), scales as for int8.  ``mask``
    (``[batch, seq_q, mask_len]`` in ``compute_dtype``; seq_q <= 16, mask_len <= 64, a
    multiple of seq_q; not with float32 q) is added to the logits of each sequence's last
    ``mask_len`` keys.  Computed in fp32 (MFMA with exact bf16/f16 operands).  With
    ``return_lse`` also returns ``ln`` of the softmax denominator, ``[batch, heads, seq_q]``
    (or ``[heads, total_q]`` for 3-D q).  An int8 or ``torch.float8_e4m3fn`` q holds codes
    times ``q_quant_scale`` (``[1]``, q's shape without head_size, or that with a last dim of
    scale_num channel groups; float32 or bfloat16) and the output is ``out_dtype`` (half for
    a float8 q); such a q reads quantised caches, or caches of its own dtype
    (``kv_cache_quant_bit_size=-1``) as codes with unit scales.  ``block_tables`` may be
    ``[batch, kv_heads or heads, max_blocks]`` (sparse KV: each head its own pages).
    ``out_quant_scale`` must be None.  A positive ``max_seq_q`` is trusted: query tokens past
    it are not computed (as the reference says of an understated ``max_context_len``).

    Reference: ``_ops.py:777-900`` (math ``:800-817``; int4 ``:826-829``, ``:852``; mask
    ``:860``; quantised q ``:853-858``; sparse KV ``:834``).  Returns ``out`` or ``(out, lse)``.
    """
    tmo_out = out
    if out is None:
        if v_cache is not None:
            head_size_v = v_cache.shape[-1]
        if q.dtype not in {torch.float8_e4m3fn, torch.int8}:
            out_dtype = q.dtype
        tmo_out = torch.empty(q.size()[:-1] + (head_size_v,), dtype=out_dtype, device=q.device)
    out_lse = None
    if return_lse:
        lse_shape = q.shape[:-3] + (q.shape[-2],) + (q.shape[-3],)
        out_lse = torch.empty(lse_shape, dtype=torch.float, device=q.device)
    torch.ops.torch_mlu_ops.single_query_cached_kv_attn(
        q, k_cache, tmo_out, block_tables, context_lens, v_cache, out_lse, q_quant_scale,
        k_cache_quant_scale, v_cache_quant_scale, out_quant_scale, alibi_slopes, mask,
        _DTYPE_STR.get(compute_dtype, str(compute_dtype)), max_context_len, windows_size_left,
        windows_size_right, softmax_scale, return_lse, kv_cache_quant_bit_size, cu_seq_q,
        max_seq_q, sink)
    return (tmo_out, out_lse) if return_lse else tmo_out

