"""CPU oracle of the quantized paged-KV-cache path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker / CPU baseline; the product package
(``domesticated_torch_mlu_ops_amd``) never touches it.

The arithmetic lives in ``tmo_oracle.c`` (a restatement of the reference's docstring math,
cited per function there, built by ``Makefile`` into ``_build/libtmo_oracle.so``).  This module
wraps it for CPU torch tensors with the argument conventions of the reference ops: outputs
are written in place.  ``nthreads`` defaults to the CPUs this process may run on.

Parity pins: tests/test_oracle_pins.py.  The reference itself cannot be imported or built
here (it needs torch_mlu and the unshipped _TMOC extension), so ``oracle/_ref`` does not exist.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Optional

import torch

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "libtmo_oracle.so"

_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.int8: 3}
_lib: Optional[ctypes.CDLL] = None

c_void_p, c_int64, c_int, c_float = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_quant_to_paged_cache.argtypes = [c_void_p, c_void_p, c_int] + [c_int64] * 4 + \
            [c_void_p] * 5 + [c_int64] * 5 + [c_int, c_int]
        L.oracle_reshape_paged_cache.argtypes = [c_void_p, c_void_p, c_int] + [c_int64] * 4 + \
            [c_void_p] * 3 + [c_int64] * 5 + [c_int, c_int]
        L.oracle_dequant_from_paged_cache.argtypes = [c_void_p, c_void_p, c_int, c_int] + [c_int64] * 5 + \
            [c_void_p] * 7 + [c_int64] * 6 + [c_int, c_int]
        L.oracle_scaled_quantize_per_token.argtypes = [c_void_p, c_int] + [c_int64] * 4 + \
            [c_void_p] * 3 + [c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                              c_int]
        L.oracle_fused_rope_paged.argtypes = [c_void_p, c_int] + [c_int64] * 5 + \
            [c_void_p, c_void_p] + [c_int64] * 4 + [c_void_p] * 3 + [c_float, c_void_p, c_int] + \
            [c_void_p] * 4 + [c_int, c_void_p, c_int64, c_int64, c_int]
        L.oracle_fused_rope_paged.restype = c_int
        L.oracle_offline_quant_to_paged_cache.argtypes = [c_void_p, c_void_p, c_int] + \
            [c_int64] * 4 + [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_float, c_float,
                             c_void_p] + [c_int64] * 5 + [c_int]
        L.oracle_linear_cache.argtypes = [c_int, c_void_p, c_void_p, c_int] + [c_int64] * 5 + \
            [c_void_p, c_void_p, c_int] + [c_int64] * 4 + [c_void_p] * 4 + \
            [c_float, c_float, c_int, c_int64, c_void_p, c_int64, c_int64, c_int, c_int64] + \
            [c_void_p] * 4 + [c_int64, c_int]
        L.oracle_linear_cache.restype = c_int
        L.oracle_linear_cache_bits.argtypes = L.oracle_linear_cache.argtypes[:-1] + [c_int, c_int]
        L.oracle_linear_cache_bits.restype = c_int
        c_double = ctypes.c_double
        L.oracle_single_query_attn.argtypes = [c_void_p, c_int, c_int64, c_int64, c_void_p,
                                               c_void_p, c_int] + [c_int64] * 4 + \
            [c_void_p, c_void_p, c_int, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p,
             c_int64, c_double, c_void_p, c_void_p, c_int]
        L.oracle_single_query_attn.restype = c_int
        L.oracle_cached_kv_attn.argtypes = [c_void_p, c_int, c_int64, c_int64,
                                            c_void_p, c_int, c_int64, c_int64, c_int64,
                                            c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int,
                                            c_int] + \
            [c_int64] * 7 + [c_void_p, c_void_p, c_int] + [c_int64] * 4 + \
            [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
             c_void_p, c_int, c_int64, c_int64, c_int64, c_int64,
             c_double, c_void_p, c_void_p, c_int]
        L.oracle_cached_kv_attn.restype = c_int
        for name in ("oracle_f32_to_bf16", "oracle_f32_to_f16", "oracle_f16_to_f32",
                     "oracle_f32_to_e4m3", "oracle_e4m3_to_f32"):
            getattr(L, name).argtypes = [c_void_p, c_void_p, c_int64]
        for name in ("oracle_quant_to_paged_cache", "oracle_reshape_paged_cache",
                     "oracle_dequant_from_paged_cache", "oracle_scaled_quantize_per_token",
                     "oracle_offline_quant_to_paged_cache"):
            getattr(L, name).restype = c_int
        _lib = L
    return _lib


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return max(1, os.cpu_count() or 1)


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    assert t.device.type == "cpu", "oracle works on CPU tensors"
    return t.data_ptr()


def _check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {name} rejected its arguments (rc={rc})")


def quant_to_paged_cache(k, v, k_cache, v_cache, k_scale, v_scale, slot_mapping,
                         nthreads: Optional[int] = None) -> None:
    """reference _ops.py:1511-1565 (see tmo_oracle.c); in place on CPU tensors; int8 or
    torch.float8_e4m3fn caches."""
    assert k.stride(2) == 1 and k_cache.is_contiguous() and k_scale.is_contiguous()
    T, H, D = k.shape
    NB, _, BS, _ = k_cache.shape
    slots = slot_mapping.to(torch.int32).contiguous()  # kept alive across the call
    rc = lib().oracle_quant_to_paged_cache(
        _ptr(k), _ptr(v), _DT[k.dtype], k.stride(0), k.stride(1),
        v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0,
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        _ptr(slots), T, H, D, NB, BS, {torch.int8: 3, torch.float8_e4m3fn: 4}[k_cache.dtype],
        nthreads or default_threads())
    _check(rc, "quant_to_paged_cache")


def offline_quant_to_paged_cache(k, v, k_cache_scale, v_cache_scale, slot_mapping, k_cache,
                                 v_cache, nthreads: Optional[int] = None) -> None:
    """reference _ops.py:1639-1706 (decision D9 in tmo_oracle.c); in place on CPU tensors.
    Each scale is a [H, D] fp32 tensor (per channel) or a Python number (per tensor); the
    caches are int8 or torch.float8_e4m3fn."""
    assert k.stride(2) == 1 and k_cache.is_contiguous()
    T, H, D = k.shape
    NB, _, BS, _ = k_cache.shape
    cdt = {torch.int8: 3, torch.float8_e4m3fn: 4}[k_cache.dtype]
    slots = slot_mapping.to(torch.int32).contiguous()  # kept alive across the call

    def split(sc):
        if torch.is_tensor(sc):
            return sc.to(torch.float32).contiguous(), 1.0
        return None, float(1.0 if sc is None else sc)

    kch, kt = split(k_cache_scale)
    vch, vt = split(v_cache_scale)
    rc = lib().oracle_offline_quant_to_paged_cache(
        _ptr(k), _ptr(v), _DT[k.dtype], k.stride(0), k.stride(1),
        v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0,
        _ptr(k_cache), _ptr(v_cache), cdt, _ptr(kch), _ptr(vch), kt, vt,
        _ptr(slots), T, H, D, NB, BS, nthreads or default_threads())
    _check(rc, "offline_quant_to_paged_cache")


def fused_rope_paged(qkv, k_cache, v_cache, sin_cache, cos_cache, position_id, k_gamma, k_scale,
                     v_scale, slot_mapping, eps: float = 1e-5, q_gamma=None, rope_dim_offset: int = 0,
                     nthreads: Optional[int] = None, norm_type: str = "rmsnorm",
                     k_beta=None) -> None:
    """reference _ops.py:3469-3601 (fused_rope, paged hp caches) under decisions D10
    (norm_type "rmsnorm") and D13 ("layernorm": rope, then layernorm of K with k_gamma and
    k_beta) of tmo_oracle.c; in place on CPU tensors (q back into qkv, K/V into the pages).
    qkv [B, S, Hq + 2 Hk, D] (or [T, Hq + 2 Hk, D] with S = T); caches [NB, Hk, BS, D] of qkv's
    dtype (no scales) or int8 with k_scale/v_scale [NB, Hk, BS] (dynamic, written) or [Hk, D]
    (static, read)."""
    assert qkv.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous()
    S = qkv.shape[1] if qkv.dim() == 4 else qkv.shape[0]
    T = qkv.shape[0] * S if qkv.dim() == 4 else qkv.shape[0]
    H, D = qkv.shape[-2], qkv.shape[-1]
    NB, Hk, BS, _ = k_cache.shape
    Hq = H - 2 * Hk
    if k_scale is None:
        mode = 0
    else:
        mode = 1 if k_scale.dim() == 3 else 2
    assert sin_cache.stride(-1) == 1 and cos_cache.stride(-1) == 1
    assert sin_cache.stride(0) == cos_cache.stride(0)
    pos = position_id.to(torch.int32).contiguous()
    slots = slot_mapping.to(torch.int32).contiguous()
    rc = lib().oracle_fused_rope_paged(
        _ptr(qkv), _DT[qkv.dtype], T, S, Hq, Hk, D, _ptr(sin_cache), _ptr(cos_cache),
        sin_cache.shape[-1], rope_dim_offset, sin_cache.stride(0), sin_cache.shape[0],
        _ptr(pos), _ptr(k_gamma),
        _ptr(q_gamma), float(eps), _ptr(k_beta), {"rmsnorm": 0, "layernorm": 1}[norm_type],
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        mode, _ptr(slots), NB, BS, nthreads or default_threads())
    _check(rc, "fused_rope_paged")


def fused_rope_linear(qkv, k_cache, v_cache, sin_cache, cos_cache, position_id, k_gamma, k_scale,
                      v_scale, cache_bs_id, cache_seq_offsets, eps: float = 1e-5, q_gamma=None,
                      rope_dim_offset: int = 0, nthreads: Optional[int] = None,
                      norm_type: str = "rmsnorm", k_beta=None) -> None:
    """reference _ops.py:3469-3601 with linear hp caches [max_batch, kv_heads, cache_len,
    head_size] (decision D14 of tmo_oracle.c): token s of sequence b goes to cache batch
    cache_bs_id[b] (default b) at position cache_seq_offsets[b] + s (default s), and nowhere
    when either falls outside the cache.  That layout is the paged one with one page of
    cache_len rows per cache batch, so the rows are mapped to those slots and stored by
    fused_rope_paged."""
    B, S = qkv.shape[:2]
    MB, _, L, _ = k_cache.shape
    cb = (cache_bs_id.long() if cache_bs_id is not None else torch.arange(B))[:, None].expand(B, S)
    pos = torch.arange(S)[None, :] + (cache_seq_offsets.long()[:, None]
                                      if cache_seq_offsets is not None else 0)
    ok = (cb >= 0) & (cb < MB) & (pos >= 0) & (pos < L)
    slot = torch.where(ok, cb * L + pos, torch.full_like(pos, -1)).to(torch.int32)
    fused_rope_paged(qkv, k_cache, v_cache, sin_cache, cos_cache, position_id, k_gamma, k_scale,
                     v_scale, slot, eps, q_gamma, rope_dim_offset, nthreads, norm_type, k_beta)


def e4m3_to_f32(bits: torch.Tensor) -> torch.Tensor:
    """The values (fp32) of float8_e4m3fn bit patterns (uint8); S.1111.111 is NaN."""
    bits = bits.to(torch.uint8).contiguous()
    out = torch.empty(bits.shape, dtype=torch.float32)
    lib().oracle_e4m3_to_f32(_ptr(bits), _ptr(out), bits.numel())
    return out


def f32_to_e4m3(x: torch.Tensor) -> torch.Tensor:
    """float8_e4m3fn bit patterns (uint8) of fp32 values |x| <= 448, round to nearest even."""
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8)
    lib().oracle_f32_to_e4m3(_ptr(x), _ptr(out), x.numel())
    return out


_CACHE_DT = {torch.int8: 3, torch.float8_e4m3fn: 4}
_ATTN_CACHE_DT = {**_DT, torch.float8_e4m3fn: 4}


def _rows_view(t: Optional[torch.Tensor]):
    """[B, S, H, D] (padded) or [T, H, D] token tensor -> its [rows, H, D] view."""
    if t is None or t.dim() == 3:
        return t
    assert t.dim() == 4 and t.stride(0) == t.shape[1] * t.stride(1), "padded tensor must flatten"
    return t.reshape(-1, t.shape[2], t.shape[3])


def _i32(t: Optional[torch.Tensor]):
    return t.to(torch.int32).contiguous() if t is not None else None


def linear_cache(op: int, key, value, key_cache, value_cache, context_lengths, max_context_len,
                 packed: bool = False, context_seq_offset=None, cache_bs_id=None,
                 cache_seq_offset=None, key_scale=None, value_scale=None, key_chan=None,
                 value_chan=None, key_tensor: float = 1.0, value_tensor: float = 1.0,
                 smode: int = 0, groups: int = 1, block_tables=None,
                 nthreads: Optional[int] = None, bits: int = 8) -> None:
    """The five linear-cache ops of tmo_oracle.c (decision D11), in place on CPU tensors.

    op 0 reshape_linear_cache, 1 quant_to_linear_cache, 2 offline_quant_to_linear_cache,
    3 dequant_from_linear_cache, 4 reshape_from_cache.  ``key``/``value`` are the token-major
    tensors ([T, H, D], or [B, S, H, D] padded input for ops 0-2); caches [NB, H, L, D];
    ``key_scale`` per-token scales (op 1 written, op 3 mode 1 read), ``key_chan`` static /
    per-channel scales, ``key_tensor`` a per-tensor scale.  ``bits`` 4 (ops 1 and 3, decision
    D15): int8 caches of int4 pairs, key_cache [NB, H, L, D / 2], value_cache [NB, H, L / 2, D]."""
    k, v = _rows_view(key), _rows_view(value)
    assert k.stride(2) == 1 and key_cache.is_contiguous()
    pad = key.shape[1] if key.dim() == 4 else 0
    NB, H, L, D = key_cache.shape
    if bits == 4:
        D = k.shape[2]
        assert key_cache.shape[3] * 2 == D, "4-bit key cache is [NB, H, L, D / 2]"
        assert value_cache is None or tuple(value_cache.shape) == (NB, H, L // 2, D)
    ctx = _i32(context_lengths)
    B = ctx.numel() - 1 if packed else ctx.numel()
    cso, bsi, coff, bt = _i32(context_seq_offset), _i32(cache_bs_id), _i32(cache_seq_offset), \
        _i32(block_tables)
    kch = key_chan.to(torch.float32).contiguous() if key_chan is not None else None
    vch = value_chan.to(torch.float32).contiguous() if value_chan is not None else None
    rc = lib().oracle_linear_cache_bits(
        op, _ptr(k), _ptr(v), _DT[k.dtype], k.stride(0), k.stride(1),
        v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0, k.shape[0],
        _ptr(key_cache), _ptr(value_cache), _CACHE_DT.get(key_cache.dtype, 3), NB, H, L, D,
        _ptr(key_scale), _ptr(value_scale), _ptr(kch), _ptr(vch), float(key_tensor),
        float(value_tensor), int(smode), int(groups), _ptr(ctx), B, int(max_context_len),
        int(bool(packed)), pad, _ptr(cso), _ptr(bsi), _ptr(coff), _ptr(bt),
        bt.shape[1] if bt is not None else 0, int(bits), nthreads or default_threads())
    _check(rc, "linear_cache")


def single_query_attn(q, k_cache, v_cache, block_tables, context_lens, softmax_scale: float,
                      k_scale=None, v_scale=None, alibi_slopes=None, window_left: int = -1,
                      nthreads: Optional[int] = None):
    """reference _ops.py:777-900 for one query token per sequence (decision D12 of
    tmo_oracle.c), in float64.  q [B, Hq, D] or [B, 1, Hq, D]; caches [NB, Hkv, BS, D] (int8 or
    float8_e4m3fn with k_scale/v_scale [NB, Hkv, BS] per token or [Hkv, D] per channel, fp32
    or bf16, or float);
    block_tables [B, max_blocks]; returns (out [B, Hq, D] float64, lse [B, Hq] float64)."""
    if q.dim() == 4:
        assert q.shape[1] == 1
        q = q[:, 0]
    assert q.stride(-1) == 1 and k_cache.is_contiguous() and v_cache.is_contiguous()
    B, Hq, D = q.shape
    NB, Hkv, BS, _ = k_cache.shape
    cdt = _ATTN_CACHE_DT[k_cache.dtype]
    mode = 0
    ks = vs = None
    if k_cache.dtype in (torch.int8, torch.float8_e4m3fn):
        ks = k_scale.to(torch.float32).contiguous()
        vs = v_scale.to(torch.float32).contiguous()
        mode = 2 if ks.dim() == 2 else 1
    bt = block_tables.to(torch.int32).contiguous()
    lens = context_lens.to(torch.int32).contiguous()
    al = alibi_slopes.to(torch.float32).contiguous() if alibi_slopes is not None else None
    out = torch.empty((B, Hq, D), dtype=torch.float64)
    lse = torch.empty((B, Hq), dtype=torch.float64)
    rc = lib().oracle_single_query_attn(
        _ptr(q), _DT[q.dtype], q.stride(0), q.stride(1), _ptr(k_cache), _ptr(v_cache), cdt,
        NB, Hkv, BS, D, _ptr(ks), _ptr(vs), mode, _ptr(bt), bt.shape[1], _ptr(lens), B, Hq,
        _ptr(al), int(window_left), float(softmax_scale), _ptr(out), _ptr(lse),
        nthreads or default_threads())
    _check(rc, "single_query_attn")
    return out, lse


def cached_kv_attn(q, k_cache, v_cache, block_tables, context_lens, softmax_scale: float,
                   k_scale=None, v_scale=None, alibi_slopes=None, window_left: int = -1,
                   cu_seq_q=None, sink=None, head_size_v: Optional[int] = None,
                   int4: bool = False, mask=None, q_scale=None,
                   nthreads: Optional[int] = None):
    """reference _ops.py:777-900 with several query tokens per sequence (decision D12 of
    tmo_oracle.c), in float64.  q [B, S, Hq, D] (S tokens per sequence), or [T, Hq, D] with
    cu_seq_q [B + 1] (rows cu_seq_q[i] .. cu_seq_q[i + 1] - 1 are sequence i's), or [B, Hq, D]
    (one token each); token s of a sequence with nq tokens and L keys sits at position
    L - nq + s.  Keys are the first D channels of k_cache's rows; values the first
    head_size_v (default: v_cache's last dim, or D) of v_cache's, or of k_cache's when v_cache
    is None.  Int8 scales: [NB, Hkv, BS] (or [..., 1]; any strides in the first two dims) per
    token, [Hkv, D or Dv] per channel, or per group K [NB, Hkv, BS, D / 32] and V [NB, Hkv,
    BS / 32, Dv].  sink [Hq] or None.  Returns (out, lse) float64 of q's leading shape:
    [B, S, Hq, Dv] / [B, S, Hq] for 4-D q, [T, Hq, Dv] / [T, Hq] otherwise; rows that no
    sequence of cu_seq_q holds are NaN.  int4 (kv_cache_quant_bit_size 4, decision D16): int8
    caches of 4-bit pairs, K [NB, Hkv, BS, D / 2] pairing channels, V [NB, Hkv, BS / 2, Dv]
    pairing rows or [NB, Hkv, BS, Dv / 2] pairing channels.  mask [B, S, mask_len] (float32 /
    float16 / bfloat16, D16) is added to the logits of each sequence's last mask_len keys.
    q of int8 / float8_e4m3fn (D17) holds codes times q_scale: [1] per tensor, q's leading
    shape per token and head, or that shape plus scale_num per channel group.  block_tables
    [B, Hkv or Hq, max_blocks] (D17): each KV head's (or query head's) own pages."""
    four = q.dim() == 4
    qs, qs_mode, qs_st, qs_sh, qs_groups = None, 0, 0, 0, 0
    if q.dtype in (torch.int8, torch.float8_e4m3fn):
        assert q_scale is not None
        qsc = q_scale.to(torch.float32)
        if qsc.numel() == 1:
            qs, qs_mode = qsc.reshape(1).contiguous(), 1
        elif tuple(qsc.shape) == tuple(q.shape[:-1]):
            qs, qs_mode = qsc.reshape(-1, q.shape[-2]).contiguous(), 2
            qs_st, qs_sh = q.shape[-2], 1
        else:
            assert qsc.dim() == q.dim() and tuple(qsc.shape[:-1]) == tuple(q.shape[:-2]) + (q.shape[-2],)
            qs, qs_mode, qs_groups = qsc.contiguous(), 3, qsc.shape[-1]
    if four:
        B, S = q.shape[:2]
        q = q.reshape(B * S, q.shape[2], q.shape[3])
    else:
        B = context_lens.shape[0]
        S = 1
    vc = k_cache if v_cache is None else v_cache
    assert q.stride(-1) == 1 and k_cache.is_contiguous() and vc.is_contiguous()
    T, Hq, D = q.shape
    NB, Hkv, BS, krow = k_cache.shape
    vrow = vc.shape[3]
    v_ch = 0
    if int4:
        assert k_cache.dtype == torch.int8 and v_cache is not None
        v_ch = int(vc.shape[2] == BS)    # else [NB, Hkv, BS / 2, Dv]: row pairs
        assert v_ch or 2 * vc.shape[2] == BS
        cdt = 5
        Dv = head_size_v if head_size_v is not None else (2 * vrow if v_ch else vrow)
    else:
        Dv = head_size_v if head_size_v is not None else (vrow if v_cache is not None else D)
        cdt = _ATTN_CACHE_DT[k_cache.dtype]
    mode = 0
    ks = vs = None
    strides = [0, 0, 0, 0]
    if k_cache.dtype in (torch.int8, torch.float8_e4m3fn):
        def one(sc):  # noqa: E306
            sc = sc.to(torch.float32)
            if sc.dim() == 4 and sc.shape[3] == 1:
                sc = sc[..., 0]
            if sc.dim() == 3:
                assert sc.stride(2) == 1
                return sc, 1, (sc.stride(0), sc.stride(1))
            return sc.contiguous(), (2 if sc.dim() == 2 else 3), (0, 0)
        ks, mode, strides[0:2] = one(k_scale)
        vs, vmode, strides[2:4] = one(v_scale)
        assert vmode == mode
    bt = block_tables.to(torch.int32).contiguous()
    bt_heads = bt.shape[1] if bt.dim() == 3 else 0
    lens = context_lens.to(torch.int32).contiguous()
    cu = cu_seq_q.to(torch.int32).contiguous() if cu_seq_q is not None else None
    assert cu is None or (not four and cu.numel() == B + 1)
    al = alibi_slopes.to(torch.float32).contiguous() if alibi_slopes is not None else None
    sk = sink.to(torch.float32).contiguous() if sink is not None else None
    mk, mdt, mlen, msb, mss = None, 0, 0, 0, 0
    if mask is not None:
        mk = mask.contiguous()
        assert mk.dim() == 3 and mk.shape[0] == B
        mdt, mlen, msb, mss = _DT[mk.dtype], mk.shape[2], mk.stride(0), mk.stride(1)
    out = torch.full((T, Hq, Dv), float("nan"), dtype=torch.float64)
    lse = torch.full((T, Hq), float("nan"), dtype=torch.float64)
    rc = lib().oracle_cached_kv_attn(
        _ptr(q), _ATTN_CACHE_DT[q.dtype], q.stride(0), q.stride(1), _ptr(qs), qs_mode, qs_st,
        qs_sh, qs_groups, _ptr(cu), S, T, _ptr(k_cache),
        _ptr(vc), cdt, v_ch, NB, Hkv, BS, D, Dv, krow, vrow, _ptr(ks), _ptr(vs), mode, *strides,
        _ptr(bt), bt.shape[-1], bt_heads, _ptr(lens), B, Hq, _ptr(al), _ptr(sk), _ptr(mk), mdt, mlen, msb,
        mss, int(window_left),
        float(softmax_scale), _ptr(out), _ptr(lse), nthreads or default_threads())
    _check(rc, "cached_kv_attn")
    if four:
        return out.reshape(B, S, Hq, Dv), lse.reshape(B, S, Hq)
    return out, lse


def reshape_paged_cache(k, v, k_cache, v_cache, slot_mapping, direction: bool = False,
                        nthreads: Optional[int] = None) -> None:
    """reference _ops.py:1251-1294; byte copy in place on CPU tensors."""
    assert k.stride(2) == 1 and k_cache.is_contiguous()
    T, H, D = k.shape
    NB, _, BS, _ = k_cache.shape
    slots = slot_mapping.to(torch.int32).contiguous()  # kept alive across the call
    rc = lib().oracle_reshape_paged_cache(
        _ptr(k), _ptr(v), _DT[k.dtype], k.stride(0), k.stride(1),
        v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0,
        _ptr(k_cache), _ptr(v_cache), _ptr(slots),
        T, H, D, NB, BS, int(bool(direction)), nthreads or default_threads())
    _check(rc, "reshape_paged_cache")


def dequant_from_paged_cache(key, value, key_cache, value_cache, key_scale, value_scale,
                             context_lengths, context_seq_offset, block_tables,
                             quant_mode: int, nthreads: Optional[int] = None) -> None:
    """reference _ops.py:3734-3824 (quant_mode 0/1, 8-bit); in place on CPU tensors.  Caches
    int8 or float8_e4m3fn; scales fp32 or bf16 (widened to fp32, exactly)."""
    assert key.stride(2) == 1 and key_cache.is_contiguous() and block_tables.is_contiguous()
    NB, H, BS, D = key_cache.shape
    B, MB = block_tables.shape
    # converted copies are kept alive across the call
    cso = context_seq_offset.to(torch.int32).contiguous() if context_seq_offset is not None else None
    ctx = context_lengths.to(torch.int32).contiguous()
    bt = block_tables.to(torch.int32).contiguous()
    key_scale = key_scale.to(torch.float32).contiguous()
    value_scale = value_scale.to(torch.float32).contiguous() if value_scale is not None else None
    rc = lib().oracle_dequant_from_paged_cache(
        _ptr(key), _ptr(value), _DT[key.dtype], _CACHE_DT[key_cache.dtype], key.stride(0),
        key.stride(1),
        value.stride(0) if value is not None else 0, value.stride(1) if value is not None else 0,
        key.shape[0], _ptr(key_cache), _ptr(value_cache), _ptr(key_scale), _ptr(value_scale),
        _ptr(ctx), _ptr(cso), _ptr(bt), B, MB, NB, H, BS, D, int(quant_mode),
        nthreads or default_threads())
    _check(rc, "dequant_from_paged_cache")


def scaled_quantize_per_token(x, out, out_scale, smooth=None, token_count=None,
                              gather_index=None, gather_start=None,
                              nthreads: Optional[int] = None) -> None:
    """reference _ops.py:3126-3253 / 4407-4492, mode dynamic_per_token; in place.

    ``x`` is [n0, ..., C] with a contiguous row layout; ``out`` [rows, ..., C] int8 and
    ``out_scale`` [rows, ...] fp32, rows = gather_index.numel() or n0."""
    x = x.contiguous()
    C = x.shape[-1]
    n0 = x.shape[0] if x.dim() >= 2 else 1
    inner = 1
    for s in x.shape[1:-1]:
        inner *= s
    rows = gather_index.numel() if gather_index is not None else n0
    sm = smooth.to(torch.float32).contiguous() if smooth is not None else None
    smooth_len = 0 if sm is None else (C if (token_count is not None or sm.numel() != 1) else 1)
    tc = token_count.to(torch.int32).contiguous() if token_count is not None else None
    gi = gather_index.to(torch.int32).contiguous() if gather_index is not None else None
    gs = gather_start.to(torch.int32).contiguous() if gather_start is not None else None
    rc = lib().oracle_scaled_quantize_per_token(
        _ptr(x), _DT[x.dtype], n0, inner, C, C, _ptr(out), _ptr(out_scale), _ptr(sm),
        smooth_len, _ptr(tc), tc.numel() if tc is not None else 0, _ptr(gi),
        gi.numel() if gi is not None else 0, _ptr(gs), rows, nthreads or default_threads())
    _check(rc, "scaled_quantize_per_token")


def f32_to_bf16_bits(x: torch.Tensor) -> torch.Tensor:
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.int16)
    lib().oracle_f32_to_bf16(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def f32_to_f16_bits(x: torch.Tensor) -> torch.Tensor:
    x = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.int16)
    lib().oracle_f32_to_f16(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def f16_bits_to_f32(bits: torch.Tensor) -> torch.Tensor:
    bits = bits.to(torch.int16).contiguous()
    out = torch.empty(bits.shape, dtype=torch.float32)
    lib().oracle_f16_to_f32(bits.data_ptr(), out.data_ptr(), bits.numel())
    return out
