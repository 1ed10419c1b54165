"""Loaders for the golden fixtures of tests/golden (written by tests/golden/make_fixtures.py):
each case rebuilds its input tensors, runs one op through a caller-given implementation (the
CPU oracle or the HIP ops) and returns (name, got, want) triples to compare bit for bit."""
import hashlib
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
DT = {"torch.bfloat16": torch.bfloat16, "torch.float16": torch.float16,
      "torch.float32": torch.float32}


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def manifest() -> dict:
    out = {}
    for line in (GOLDEN / "MANIFEST.sha256").read_text().splitlines():
        digest, fname = line.split()
        out[fname] = digest
    return out


def sha256(fname: str) -> str:
    return hashlib.sha256((GOLDEN / fname).read_bytes()).hexdigest()


def t16(a: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(dtype)


def t32f(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.float32).copy())


def t8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.copy()).view(torch.int8)


def tensor_of(a: np.ndarray, dtype) -> torch.Tensor:
    if dtype in (torch.bfloat16, torch.float16):
        return t16(a, dtype)
    return t32f(a)


def bits(t: torch.Tensor) -> torch.Tensor:
    t = t.cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


QUANT_PAGED = ["quant_paged_cfg1", "quant_paged_special_bf16", "quant_paged_special_f16",
               "quant_paged_special_f32"]


def run_quant_paged(name, quant_to_paged_cache, device="cpu"):
    z = load(name)
    dt = DT[str(z["dtype"])]
    k, v = tensor_of(z["k"], dt), tensor_of(z["v"], dt)
    slot = torch.from_numpy(z["slot_mapping"].copy())
    want = [t8(z["k_cache"]), t8(z["v_cache"]), t32f(z["k_scale"]), t32f(z["v_scale"])]
    from tests import workloads as W
    kc = torch.full(want[0].shape, W.CACHE_SENTINEL, dtype=torch.int8, device=device)
    vc = kc.clone()
    ks = torch.full(want[2].shape, W.SCALE_SENTINEL, device=device)
    vs = ks.clone()
    quant_to_paged_cache(k.to(device), v.to(device), kc, vc, ks, vs, slot.to(device))
    return [(n, g, w) for n, g, w in zip(("k_cache", "v_cache", "k_scale", "v_scale"),
                                         (kc, vc, ks, vs), want)]


def run_smooth_quant(fn, device="cpu"):
    """fn(x, out, out_scale, smooth, token_count, gather_index)"""
    z = load("smooth_quant_moe")
    x = t16(z["x"], torch.bfloat16)
    smooth = t32f(z["smooth"])
    tc = torch.from_numpy(z["token_count"].copy())
    gi = torch.from_numpy(z["gather_index"].copy())
    out = torch.zeros(gi.numel(), x.shape[1], dtype=torch.int8, device=device)
    osc = torch.zeros(gi.numel(), device=device)
    fn(x.to(device), out, osc, smooth.to(device), tc.to(device), gi.to(device))
    return [("out", out, t8(z["out"])), ("out_scale", osc, t32f(z["out_scale"]))]


def run_dequant_paged(fn, device="cpu"):
    """fn(key, value, k_cache, v_cache, k_scale, v_scale, context_lengths, block_tables)"""
    z = load("dequant_paged")
    want_k, want_v = t16(z["key"], torch.bfloat16), t16(z["value"], torch.bfloat16)
    key = torch.zeros(want_k.shape, dtype=torch.bfloat16, device=device)
    val = torch.zeros_like(key)
    fn(key, val, t8(z["k_cache"]).to(device), t8(z["v_cache"]).to(device),
       t32f(z["k_scale"]).to(device), t32f(z["v_scale"]).to(device),
       torch.from_numpy(z["context_lengths"].copy()).to(device),
       torch.from_numpy(z["block_tables"].copy()).to(device))
    return [("key", key, want_k), ("value", val, want_v)]


def run_linear_int4(fn, device="cpu", name="linear_int4"):
    """fn(key, value, k_cache, v_cache, k_scale, v_scale, context_lengths, max_context_len,
    context_seq_offset, cache_bs_id, cache_seq_offset); `name` = "linear_int8" for the 8-bit
    fixture"""
    z = load(name)
    key, value = t16(z["key"], torch.bfloat16), t16(z["value"], torch.bfloat16)
    want = [t8(z["k_cache"]), t8(z["v_cache"]), t32f(z["k_scale"]), t32f(z["v_scale"])]
    kc = torch.full(want[0].shape, 0x5A, dtype=torch.uint8, device=device).view(torch.int8)
    vc = torch.full(want[1].shape, 0x5A, dtype=torch.uint8, device=device).view(torch.int8)
    from tests import workloads as W
    ks = torch.full(want[2].shape, W.SCALE_SENTINEL, device=device)
    vs = ks.clone()
    i32 = lambda n: torch.from_numpy(z[n].copy()).to(device)
    fn(key.to(device), value.to(device), kc, vc, ks, vs, i32("context_lengths"),
       int(z["max_context_len"]), i32("context_seq_offset"), i32("cache_bs_id"),
       i32("cache_seq_offset"))
    return [(n, g, w) for n, g, w in zip(("k_cache", "v_cache", "k_scale", "v_scale"),
                                         (kc, vc, ks, vs), want)]


FUSED_ROPE = ["fused_rope_rmsnorm", "fused_rope_layernorm"]


def run_fused_rope(name, fn, device="cpu"):
    """fn(qkv, k_cache, v_cache, sin, cos, position_id, k_gamma, q_gamma, k_beta, k_scale,
    v_scale, slot_mapping, norm_type): Q written back into qkv, K / V into the pages."""
    z = load(name)
    bf = torch.bfloat16
    want = [t16(z["qkv_out"], bf), t8(z["k_cache"]), t8(z["v_cache"]), t32f(z["k_scale"]),
            t32f(z["v_scale"])]
    from tests import workloads as W
    qkv = t16(z["qkv"], bf).to(device)
    kc = torch.full(want[1].shape, 0x5A, dtype=torch.uint8, device=device).view(torch.int8)
    vc = kc.clone()
    ks = torch.full(want[3].shape, W.SCALE_SENTINEL, device=device)
    vs = ks.clone()
    d = lambda a: t16(a, bf).to(device)
    fn(qkv, kc, vc, d(z["sin"]), d(z["cos"]), torch.from_numpy(z["position_id"].copy()).to(device),
       d(z["k_gamma"]), d(z["q_gamma"]), d(z["k_beta"]), ks, vs,
       torch.from_numpy(z["slot_mapping"].copy()).to(device), str(z["norm_type"]))
    return [(n, g, w) for n, g, w in zip(("qkv", "k_cache", "v_cache", "k_scale", "v_scale"),
                                         (qkv, kc, vc, ks, vs), want)]


OFFLINE = ["offline_int8", "offline_fp8"]
CDT = {"torch.int8": torch.int8, "torch.float8_e4m3fn": torch.float8_e4m3fn}


def run_offline(name, fn, device="cpu"):
    """fn(k, v, k_scale, v_scale, slot_mapping, k_cache, v_cache)"""
    z = load(name)
    cdt = CDT[str(z["cache_dtype"])]
    want = [torch.from_numpy(z["k_cache"].copy()).view(cdt), torch.from_numpy(z["v_cache"].copy()).view(cdt)]
    kc = torch.full(want[0].shape, 0x5A, dtype=torch.uint8, device=device).view(cdt)
    vc = kc.clone()
    d = lambda a: t16(a, torch.bfloat16).to(device)
    fn(d(z["k"]), d(z["v"]), t32f(z["k_scale"]).to(device), t32f(z["v_scale"]).to(device),
       torch.from_numpy(z["slot_mapping"].copy()).to(device), kc, vc)
    return [("k_cache", kc, want[0]), ("v_cache", vc, want[1])]
