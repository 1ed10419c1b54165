"""Writes the golden fixtures of this directory: small inputs of the hot path with the outputs
the CPU oracle (oracle/tmo_oracle.c, pinned by tests/test_oracle_pins.py) gives for them, and
MANIFEST.sha256.  The fixtures freeze those pinned results as data, so that a change to the
oracle or to a kernel that alters any code, scale or output bit fails tests/test_golden.py
(oracle) or tests/test_gpu_golden.py (HIP kernels) even when both change together;
tests/test_golden_torch.py checks every stored output against the torch restatements of the
reference math, independently of the oracle.

    python tests/golden/make_fixtures.py        # from the repository root; CPU only

The reference ships no golden vectors of its own (its tests are not in the repository), so
these are the build's.  Inputs are seeded; bf16 / fp16 tensors are stored as their uint16 bit
patterns, float8 / int8 as bytes.
"""
import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

import oracle  # noqa: E402
from tests import workloads as W  # noqa: E402

BITS = {torch.bfloat16: np.uint16, torch.float16: np.uint16, torch.float32: np.uint32}


def as_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.contiguous().view(torch.int32).numpy().view(np.uint32)
    if t.dtype in (torch.int8, torch.float8_e4m3fn):
        return t.contiguous().view(torch.uint8).numpy()
    return t.contiguous().numpy()


def special_rows(dtype, seed: int) -> torch.Tensor:
    """Rows of 128: near-ties (x / scale within a few input ulps of k + 0.5), an all-zero row,
    one non-zero element, a constant row, tiny values (bf16 / fp16 subnormals), a row with a
    single outlier."""
    g = torch.Generator().manual_seed(seed)
    D = 128
    rows = []
    for _ in range(4):
        amax = float(torch.rand(1, generator=g)) * 8 + 0.05
        s = np.float32(np.float32(amax) / np.float32(127.0))
        r = [amax]
        for kk in torch.randint(-126, 126, (D - 1,), generator=g).tolist():
            t = torch.tensor([(kk + 0.5) * float(s)], dtype=torch.float32).to(dtype)
            bits = t.view(torch.int16 if dtype != torch.float32 else torch.int32).clone()
            bits += int(torch.randint(-2, 3, (1,), generator=g))
            r.append(float(bits.view(dtype)[0]))
        x = torch.tensor(r, dtype=torch.float32).to(dtype)
        x = torch.where(x.float().abs() <= abs(amax), x, torch.zeros_like(x))
        rows.append(x)
    rows.append(torch.zeros(D, dtype=dtype))
    one = torch.zeros(D, dtype=dtype)
    one[37] = -3.25
    rows.append(one)
    rows.append(torch.full((D,), 0.7, dtype=dtype))
    tiny = (torch.randn(D, generator=g) * 1e-39).to(dtype) if dtype == torch.bfloat16 else \
        (torch.randn(D, generator=g) * 1e-6).to(dtype)
    rows.append(tiny)
    out = (torch.randn(D, generator=g)).to(dtype)
    out[5] = 300.0
    rows.append(out)
    return torch.stack(rows)


def quant_paged(name, k, v, slot, NB, BS=16):
    kc = torch.full((NB, k.shape[1], BS, k.shape[2]), W.CACHE_SENTINEL, dtype=torch.int8)
    vc = kc.clone()
    ks = torch.full((NB, k.shape[1], BS), W.SCALE_SENTINEL)
    vs = ks.clone()
    oracle.quant_to_paged_cache(k, v, kc, vc, ks, vs, slot)
    return {"k": as_np(k), "v": as_np(v), "slot_mapping": slot.numpy(), "num_blocks": np.int64(NB),
            "block_size": np.int64(BS), "dtype": np.array(str(k.dtype)),
            "k_cache": as_np(kc), "v_cache": as_np(vc), "k_scale": as_np(ks), "v_scale": as_np(vs)}


def main() -> None:
    fixtures = {}
    case = W.cfg1()
    fixtures["quant_paged_cfg1"] = quant_paged("cfg1", case.k, case.v, case.slot_mapping, 64)
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float16, "f16"), (torch.float32, "f32")):
        rows = special_rows(dt, seed=7 + len(tag))
        R = rows.shape[0]
        k = rows.reshape(R, 1, 128)
        v = torch.flip(rows, dims=[0]).reshape(R, 1, 128).contiguous()
        slot = torch.arange(R, dtype=torch.int32) * 3
        slot[2] = -1
        fixtures[f"quant_paged_special_{tag}"] = quant_paged(tag, k, v, slot, (3 * R + 15) // 16)

    # smooth quant, gathered and grouped rows (moe_quantize)
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(40, 256, generator=g) * torch.logspace(-2, 1, 256)).to(torch.bfloat16)
    smooth = 0.5 + 1.5 * torch.rand(4, 256, generator=g)
    token_count = torch.tensor([20, 0, 27, 17], dtype=torch.int32)
    gather = torch.randint(0, 40, (64,), generator=g).to(torch.int32)
    out = torch.zeros(64, 256, dtype=torch.int8)
    osc = torch.zeros(64)
    oracle.scaled_quantize_per_token(x, out, osc, smooth, token_count, gather)
    fixtures["smooth_quant_moe"] = {"x": as_np(x), "smooth": as_np(smooth), "token_count": token_count.numpy(),
                                    "gather_index": gather.numpy(), "out": as_np(out), "out_scale": as_np(osc)}

    # paged dequant (per-token scales) of three sequences, one with a partial last page
    NB, H, BS, D = 12, 2, 16, 64
    kc = torch.randint(-127, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    ks = torch.rand(NB, H, BS, generator=g) * 0.05
    vs = torch.rand(NB, H, BS, generator=g) * 0.05
    ctx = torch.tensor([37, 16, 5], dtype=torch.int32)
    bt = torch.tensor([[3, 7, 0], [11, -1, -1], [5, -1, -1]], dtype=torch.int32)
    key = torch.zeros(int(ctx.sum()), H, D, dtype=torch.bfloat16)
    val = torch.zeros_like(key)
    oracle.dequant_from_paged_cache(key, val, kc, vc, ks, vs, ctx, None, bt, 1)
    fixtures["dequant_paged"] = {"k_cache": as_np(kc), "v_cache": as_np(vc), "k_scale": as_np(ks),
                                 "v_scale": as_np(vs), "context_lengths": ctx.numpy(),
                                 "block_tables": bt.numpy(), "key": as_np(key), "value": as_np(val)}

    # 4-bit linear caches (D15): packed input, odd cache offsets
    lc = W.linear_case(torch.bfloat16, 41, packed=True, offsets=True, D=64)
    Hl = lc.key.shape[-2]
    k4 = torch.full((lc.cache_batch, Hl, lc.cache_len, 32), 0x5A, dtype=torch.uint8).view(torch.int8)
    v4 = torch.full((lc.cache_batch, Hl, lc.cache_len // 2, 64), 0x5A, dtype=torch.uint8).view(torch.int8)
    k4s, v4s = lc.scales()
    oracle.linear_cache(1, lc.key, lc.value, k4, v4, lc.context_lengths, lc.max_context_len,
                        packed=True, context_seq_offset=lc.context_seq_offset,
                        cache_bs_id=lc.cache_bs_id, cache_seq_offset=lc.cache_seq_offset,
                        key_scale=k4s, value_scale=v4s, bits=4)
    fixtures["linear_int4"] = {"key": as_np(lc.key), "value": as_np(lc.value),
                               "context_lengths": lc.context_lengths.numpy(),
                               "max_context_len": np.int64(lc.max_context_len),
                               "context_seq_offset": lc.context_seq_offset.numpy(),
                               "cache_bs_id": lc.cache_bs_id.numpy(),
                               "cache_seq_offset": lc.cache_seq_offset.numpy(),
                               "k_cache": as_np(k4), "v_cache": as_np(v4),
                               "k_scale": as_np(k4s), "v_scale": as_np(v4s)}

    # fused rope into dynamic int8 pages, rmsnorm (Q and K normalised) and layernorm (K, with
    # beta): -1 slots, a zero K row, the second sequence running past the sin/cos table
    for name, norm, seed in (("fused_rope_rmsnorm", "rmsnorm", 29),
                             ("fused_rope_layernorm", "layernorm", 31)):
        ln = norm == "layernorm"
        qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = W.fused_rope_case(
            torch.bfloat16, "dynamic", seed, B=2, S=12, Hq=4, Hk=2, NB=4, positions=(0, 120))
        kb = (torch.rand(128, generator=torch.Generator().manual_seed(seed)) - 0.5).to(
            torch.bfloat16)
        kc.view(torch.uint8).fill_(0x5A)
        vc.view(torch.uint8).fill_(0x5A)
        ks.fill_(W.SCALE_SENTINEL)
        vs.fill_(W.SCALE_SENTINEL)
        out = qkv.clone()
        oracle.fused_rope_paged(out, kc, vc, sin, cos, pid, kg, ks, vs, slot, 1e-5,
                                None if ln else qg, 0, norm_type=norm, k_beta=kb if ln else None)
        fixtures[name] = {"qkv": as_np(qkv), "sin": as_np(sin), "cos": as_np(cos),
                          "position_id": pid.numpy(), "k_gamma": as_np(kg),
                          "q_gamma": as_np(qg), "k_beta": as_np(kb), "slot_mapping": slot.numpy(),
                          "norm_type": np.array(norm), "qkv_out": as_np(out),
                          "k_cache": as_np(kc), "v_cache": as_np(vc), "k_scale": as_np(ks),
                          "v_scale": as_np(vs)}

    # 8-bit linear caches: packed input, cache offsets and batch ids
    lc8 = W.linear_case(torch.bfloat16, 53, packed=True, offsets=True, D=64)
    H8 = lc8.key.shape[-2]
    k8 = torch.full((lc8.cache_batch, H8, lc8.cache_len, 64), 0x5A, dtype=torch.uint8).view(torch.int8)
    v8 = k8.clone()
    k8s, v8s = lc8.scales()
    oracle.linear_cache(1, lc8.key, lc8.value, k8, v8, lc8.context_lengths, lc8.max_context_len,
                        packed=True, context_seq_offset=lc8.context_seq_offset,
                        cache_bs_id=lc8.cache_bs_id, cache_seq_offset=lc8.cache_seq_offset,
                        key_scale=k8s, value_scale=v8s, bits=8)
    fixtures["linear_int8"] = {"key": as_np(lc8.key), "value": as_np(lc8.value),
                               "context_lengths": lc8.context_lengths.numpy(),
                               "max_context_len": np.int64(lc8.max_context_len),
                               "context_seq_offset": lc8.context_seq_offset.numpy(),
                               "cache_bs_id": lc8.cache_bs_id.numpy(),
                               "cache_seq_offset": lc8.cache_seq_offset.numpy(),
                               "k_cache": as_np(k8), "v_cache": as_np(v8),
                               "k_scale": as_np(k8s), "v_scale": as_np(v8s)}

    # offline (static per-channel) quant into int8 and fp8 e4m3 pages: special rows, scales of
    # both signs (a negative scale flips the codes and the sign of zero quotients), a -1 slot
    for name, cdt, seed in (("offline_int8", torch.int8, 43), ("offline_fp8", torch.float8_e4m3fn, 47)):
        gs = torch.Generator().manual_seed(seed)
        rk, rv = special_rows(torch.bfloat16, seed), special_rows(torch.bfloat16, seed + 1)
        k = torch.stack((rk, torch.flip(rk, dims=[0])), dim=1).contiguous()   # [9, 2, 128]
        v = torch.stack((rv, torch.flip(rv, dims=[0])), dim=1).contiguous()
        ks = 0.005 + 0.05 * torch.rand(2, 128, generator=gs)
        vs = 0.005 + 0.05 * torch.rand(2, 128, generator=gs)
        ks[:, ::17] = -ks[:, ::17]
        vs[:, 5::23] = -vs[:, 5::23]
        T = k.shape[0]
        slot = torch.arange(T, dtype=torch.int32) * 2 + 1
        slot[4] = -1
        NB = (2 * T + 16) // 16
        kc = torch.full((NB, 2, 16, 128), 0x5A, dtype=torch.uint8).view(cdt)
        vc = kc.clone()
        oracle.offline_quant_to_paged_cache(k, v, ks, vs, slot, kc, vc)
        fixtures[name] = {"k": as_np(k), "v": as_np(v), "k_scale": as_np(ks), "v_scale": as_np(vs),
                          "slot_mapping": slot.numpy(), "cache_dtype": np.array(str(cdt)),
                          "k_cache": as_np(kc), "v_cache": as_np(vc)}

    lines = []
    for name, arrays in fixtures.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        lines.append(f"{hashlib.sha256(path.read_bytes()).hexdigest()}  {path.name}")
        print(f"{path.name}: {path.stat().st_size} bytes")
    (HERE / "MANIFEST.sha256").write_text("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
