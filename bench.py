#!/usr/bin/env python3
"""Benchmark of the quantized paged-KV-cache path on one MI355X.

Prints ONE JSON line (rank 0) with BASELINE.json's metric -- achieved HBM GB/s of the
headline workload, its fraction of the 8 TB/s peak and tokens/s -- plus the ``roofline``,
``cpu_baseline`` and ``per_config`` objects.

* A step is one call of the op over one batch of the workload's synthetic input, with the
  inputs resident in HBM.  Calls rotate over enough independent buffer sets that each
  launch's working set has been evicted from the 256 MB MALL since its last use; the
  calls are captured in a HIP graph (so the latency-bound configs measure the GPU, not the
  Python launch path) and the timed region is bracketed by HIP events recorded on the stream
  the kernels run on, with device synchronisation on both sides.  Before the W warm-up
  steps the graph is replayed untimed for SETTLE_S seconds so the timed steps run at the
  GPU's steady clocks (they ramp up over ~10 ms of load after idle).
* GB/s counts ALGORITHMIC bytes (rows actually read, codes + scales written, index tensors,
  the smooth vector once), per BASELINE.md section 2.
* ``cpu_baseline`` times the CPU oracle (a C restatement of the reference math, pthreads)
  on a bounded sample of the headline workload, on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg3]
       [--configs all|headline] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "achieved HBM GB/s (% of MI355X peak) + tokens/s quantized into paged KV cache"
PEAK_GBS = 8000.0          # MI355X HBM3E
MALL_EVICT_BYTES = 1 << 30  # rotate buffer sets until one pass touches >= 1 GiB
SETTLE_S = 0.1              # untimed replays before the warm-up steps (clock ramp-up)

WORKLOADS = {
    "cfg1": "configs[0]: quant_to_paged_cache, 16 tokens x 8 KV heads x 128, bf16 -> int8 pages (64 blocks x 16)",
    "cfg2": "configs[1]: quant_to_paged_cache decode step, 256 seqs x 1 token x 8 KV heads x 128, bf16 -> int8 pages (16384 blocks x 16), 10% slots -1",
    "cfg3": "configs[2]: quant_to_paged_cache prefill chunk, 32768 tokens x 8 KV heads x 128, bf16 -> int8 pages (65536 blocks x 16)",
    "cfg4": "configs[3]: per_token_smooth_quantize 8192 x 4096 bf16 -> int8 + fp32 per-token scale",
    "cfg4_moe": "configs[3] MoE: per_token_smooth_quantize over 16384 gathered rows (top-2 of 64 experts), per-expert smooth",
    "cfg5": "configs[4]: dequant_from_paged_cache, 64 seqs ctx ~U[1024,32768], 8 KV heads x 128, int8 pages -> bf16",
    "offline_i8": "offline_quant_to_paged_cache on configs[2]'s shape (32768 tokens x 8 KV heads x 128 bf16), static per-channel scales -> int8 pages",
    "offline_f8": "offline_quant_to_paged_cache on configs[2]'s shape (32768 tokens x 8 KV heads x 128 bf16), static per-channel scales -> float8_e4m3fn pages",
    "fused_rope": "fused_rmsnorm_rope_store_paged_cache, Llama-3-8B prefill chunk: 8 x 4096 tokens, 32 Q + 8 KV heads x 128 bf16, Q written back, K/V -> int8 pages with dynamic per-token scales (65536 blocks x 16)",
    "fused_rope_70b": "fused_rmsnorm_rope_store_paged_cache, Llama-3-70B prefill chunk: 8 x 4096 tokens, 64 Q + 8 KV heads x 128 bf16, Q written back, K/V -> int8 pages with dynamic per-token scales (65536 blocks x 16)",
    "fused_rope_ln": "fused_rope, norm_type layernorm (rotate, then layer_norm of K with gamma and beta) on the fused_rope workload's shape: 8 x 4096 tokens, 32 Q + 8 KV heads x 128 bf16 -> int8 pages with dynamic per-token scales",
    "linear_quant": "quant_to_linear_cache on configs[2]'s volume: 8 packed sequences x 4096 tokens x 8 KV heads x 128 bf16 -> int8 linear cache [8, 8, 8192, 128] + fp32 per-token scales",
    "linear_dequant": "dequant_from_linear_cache (per-token scales), 8 sequences x 4096 tokens x 8 KV heads x 128: int8 linear cache [8, 8, 8192, 128] -> bf16",
    "linear_reshape": "reshape_linear_cache, 8 packed sequences x 4096 tokens x 8 KV heads x 128 bf16 -> bf16 linear cache [8, 8, 8192, 128]",
    "decode_attn": "single_query_cached_kv_attn, one bf16 query token x 32 heads per sequence over configs[4]'s int8 pages (64 seqs, ctx ~U[1024,32768], 8 KV heads x 128, per-token scales)",
    "reshape_paged": "reshape_paged_cache on configs[2]'s shape: 32768 tokens x 8 KV heads x 128 bf16 K/V scattered into bf16 pages (65536 blocks x 16)",
    "decode_attn_int4": "single_query_cached_kv_attn (kv_cache_quant_bit_size 4), one bf16 query token x 32 heads per sequence over configs[4]'s layout as int4 pages (K pairing channels [NB, 8, 16, 64], V pairing rows [NB, 8, 8, 128], per-token fp32 scales)",
}
KERNELS = {"cfg1": "quant_paged_vec<BF16,16,1,false>", "cfg2": "quant_paged_vec<BF16,16,1,false>",
           "cfg3": "quant_paged_vec<BF16,16,1,false>", "cfg4": "sq_dense_wg<BF16,2,false,true>",
           "cfg4_moe": "sq_grp<BF16,8,4,true,true>", "cfg5": "dequant_paged_list<BF16,1,2,0>",
           "offline_i8": "quant_paged_static_vec<BF16,16,false>",
           "offline_f8": "quant_paged_static_vec<BF16,16,true>",
           "fused_rope": "fused_rope_tok<BF16,16,3,0,256>",
           "fused_rope_ln": "fused_rope_tok<BF16,16,3,1,256>",
           "fused_rope_70b": "fused_rope_tok<BF16,16,3,0,512>",
           "linear_quant": "lin_quant<BF16,16,false,false,true>", "linear_dequant": "lin_dequant<BF16,16>",
           "linear_reshape": "lin_copy<16,true>", "decode_attn": "attn_mfma<128,0,false,false,false>",
           "reshape_paged": "reshape_paged_rows<16>", "decode_attn_int4": "attn_mfma<128,4,false,false,false>"}


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1200)
    ap.add_argument("--warmup", type=int, default=60)
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--configs", default="all", choices=["all", "headline"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-pass", type=int, default=0, metavar="N",
                    help="for rocprofv3 counter runs: call the selected configs' ops N times "
                         "eagerly, then a 1 GiB elementwise copy (counter calibration), and exit")
    return ap.parse_args()


# ---------------------------------------------------------------------------- GPU timing

def time_graph(torch, calls, steps: int, warmup: int) -> float:
    """Median ms per call: `calls` (one closure per buffer set) captured once into a HIP graph,
    replayed until `steps` calls have run; HIP events on the capture stream bracket each timed
    replay (at least 20 of them), and the median replay's time per call is returned (the mean
    over all timed replays is kept in LAST_MEAN_MS)."""
    n = len(calls)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for c in calls:  # eager warm-up of every set (also loads the code object)
            c()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for c in calls:
            c()
    reps = max(20, math.ceil(steps / n))
    wreps = max(1, math.ceil(warmup / n))
    with torch.cuda.stream(stream):
        # Clock settling: after idle the GPU takes ~10 ms of load to reach its steady clocks
        # (measured: the first ~240 configs[2] calls run up to 15% slower), so replay untimed
        # for SETTLE_S of wall time before the W warm-up steps and the timed K steps.
        t_end = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_end:
            graph.replay()
            torch.cuda.synchronize()
        for _ in range(wreps):
            graph.replay()
        torch.cuda.synchronize()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        evs[0].record(stream)
        for i in range(reps):
            graph.replay()
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) / n for i in range(reps)]
    global LAST_MEAN_MS
    LAST_MEAN_MS = evs[0].elapsed_time(evs[reps]) / (reps * n)
    del graph
    return statistics.median(per)


LAST_MEAN_MS = None


def n_sets(bytes_per_call: int, cap: int = 512) -> int:
    return max(1, min(cap, math.ceil(MALL_EVICT_BYTES / max(1, bytes_per_call))))


def bench_paged_quant(torch, tmo, W, case, dev, steps, warmup):
    """quant_to_paged_cache: per set its own K/V rows, slot mapping and caches."""
    alg = case.algorithmic_bytes()
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(7)
    base_k, base_v = case.k.to(dev), case.v.to(dev)
    slots0 = case.slot_mapping.to(dev)
    nslots = case.num_blocks * case.block_size
    # caches: one per set when small, else shared caches with per-set disjoint slot ranges
    cache_bytes = nslots * case.k.shape[1] * (case.k.shape[2] + 4) * 2
    calls = []
    shared = None
    if cache_bytes * sets > (8 << 30):
        shared = case.empty_caches(device=dev)
    for s in range(sets):
        if s == 0:
            k, v, slots = base_k, base_v, slots0
        else:
            k = torch.randn(base_k.shape, generator=g, device=dev).to(base_k.dtype)
            v = torch.randn(base_v.shape, generator=g, device=dev).to(base_v.dtype)
            # same structure (contiguity, -1 entries) at a different page offset
            shift = (s * 9973 * case.block_size) % nslots
            slots = torch.where(slots0 >= 0, (slots0 + shift) % nslots, slots0)
        kc, vc, ks, vs = shared if shared is not None else case.empty_caches(device=dev)
        calls.append(lambda k=k, v=v, kc=kc, vc=vc, ks=ks, vs=vs, sl=slots:
                     tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, sl))
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, case.valid_tokens(), sets


def bench_reshape(torch, tmo, W, case, dev, steps, warmup):
    """reshape_paged_cache (scatter, direction False) of configs[2]'s K/V as bf16 into bf16
    pages: per set its own K/V rows; shared caches with per-set shifted slots."""
    T, H, D = case.k.shape
    alg = 2 * 2 * case.valid_tokens() * H * D * case.k.element_size() + 4 * T
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(19)
    nslots = case.num_blocks * case.block_size
    slots0 = case.slot_mapping.to(dev)
    kc = torch.zeros((case.num_blocks, H, case.block_size, D), dtype=case.k.dtype, device=dev)
    vc = torch.zeros_like(kc)
    calls = []
    for s in range(sets):
        k = torch.randn((T, H, D), generator=g, device=dev).to(case.k.dtype)
        v = torch.randn((T, H, D), generator=g, device=dev).to(case.k.dtype)
        shift = (s * 9973 * case.block_size) % nslots
        slots = torch.where(slots0 >= 0, (slots0 + shift) % nslots, slots0)
        calls.append(lambda k=k, v=v, sl=slots: tmo.reshape_paged_cache(k, v, kc, vc, sl, False))
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, case.valid_tokens(), sets


def offline_bytes(case) -> int:
    """Algorithmic bytes of offline_quant_to_paged_cache: the valid tokens' K/V rows read,
    their codes written (no scales), the slot mapping, and the two [H, D] fp32 scale tables."""
    T, H, D = case.k.shape
    es = case.k.element_size()
    return case.valid_tokens() * 2 * H * D * (es + 1) + 4 * T + 2 * H * D * 4


def bench_offline(torch, tmo, W, case, cache_dtype, dev, steps, warmup):
    """offline_quant_to_paged_cache with per-channel scales: per set its own K/V rows and slot
    mapping, shared caches with per-set disjoint page ranges."""
    alg = offline_bytes(case)
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(9)
    T, H, D = case.k.shape
    nslots = case.num_blocks * case.block_size
    slots0 = case.slot_mapping.to(dev)
    shape = (case.num_blocks, H, case.block_size, D)
    kc = torch.zeros(shape, dtype=torch.uint8, device=dev).view(cache_dtype)
    vc = torch.zeros(shape, dtype=torch.uint8, device=dev).view(cache_dtype)
    gs = torch.Generator().manual_seed(2024)
    ks = (0.005 + 0.05 * torch.rand(H, D, generator=gs)).to(dev)
    vs = (0.005 + 0.05 * torch.rand(H, D, generator=gs)).to(dev)
    calls = []
    for s in range(sets):
        if s == 0:
            k, v, slots = case.k.to(dev), case.v.to(dev), slots0
        else:
            k = torch.randn((T, H, D), generator=g, device=dev).to(case.k.dtype)
            v = torch.randn((T, H, D), generator=g, device=dev).to(case.v.dtype)
            shift = (s * 9973 * case.block_size) % nslots
            slots = torch.where(slots0 >= 0, (slots0 + shift) % nslots, slots0)
        calls.append(lambda k=k, v=v, sl=slots:
                     tmo.offline_quant_to_paged_cache(k, v, ks, vs, sl, kc, vc))
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, case.valid_tokens(), sets


FR_B, FR_S, FR_HQ, FR_HK = 8, 4096, 32, 8
FR_HQ_70B = 64  # Llama-3-70B: 64 query heads, 8 KV heads


def fr_q_heads(name: str) -> int:
    return FR_HQ_70B if name == "fused_rope_70b" else FR_HQ


def fused_rope_bytes(T: int, rope: int = 128, hq: int = FR_HQ) -> int:
    """Algorithmic bytes of the fused_rope workload: qkv read once, Q written back, K/V codes
    and scales written, the slot mapping, one sin and one cos row per token, the gammas."""
    D, H = W_D, hq + 2 * FR_HK
    return (T * H * D * 2 + T * hq * D * 2 + 2 * T * FR_HK * (D + 4) + 4 * T
            + 2 * T * rope * 2 + 2 * D * 2 + 4 * FR_B)


W_D = 128


def bench_fused_rope(torch, tmo, W, dev, steps, warmup, layernorm=False, hq=FR_HQ):
    """fused_rmsnorm_rope_store_paged_cache (or fused_rope with norm_type "layernorm") on a
    Llama-3-8B-shaped prefill chunk (hq = 64: Llama-3-70B): per set its own qkv; shared int8
    caches and scales, configs[2]-style slots shifted per set."""
    T = FR_B * FR_S
    alg = fused_rope_bytes(T, hq=hq)
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(11)
    case3 = W.cfg3()
    nslots = case3.num_blocks * case3.block_size
    slots0 = case3.slot_mapping.to(dev)
    shape = (case3.num_blocks, FR_HK, case3.block_size, W_D)
    kc = torch.zeros(shape, dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(shape[:3], dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    maxpos = 8192
    ang = torch.arange(maxpos, device=dev)[:, None] * \
        (1e4 ** (-torch.arange(64, device=dev) / 64.0))[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    sin, cos = torch.sin(ang).to(torch.bfloat16), torch.cos(ang).to(torch.bfloat16)
    pid = torch.arange(FR_B, dtype=torch.int32, device=dev) * 512
    kg = (0.5 + torch.rand(W_D, generator=g, device=dev)).to(torch.bfloat16)
    qg = (0.5 + torch.rand(W_D, generator=g, device=dev)).to(torch.bfloat16)
    calls = []
    for s in range(sets):
        qkv = torch.randn((FR_B, FR_S, hq + 2 * FR_HK, W_D), generator=g, device=dev).to(torch.bfloat16)
        shift = (s * 9973 * case3.block_size) % nslots
        slots = (slots0 + shift) % nslots
        if layernorm:  # qg serves as k_beta
            calls.append(lambda qkv=qkv, sl=slots: tmo.fused_rope(
                qkv, kc, vc, sin, cos, pid, kg, qg, k_scale_hp=ks, v_scale_hp=vs,
                slot_mapping_hp=sl, norm_type="layernorm", eps=1e-5))
        else:
            calls.append(lambda qkv=qkv, sl=slots: tmo.fused_rmsnorm_rope_store_paged_cache(
                qkv, kc, vc, sin, cos, pid, kg, qg, sl, ks, vs, 1e-5))
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, T, sets


LIN_B, LIN_S, LIN_L = 8, 4096, 8192


def linear_bytes(op: str, B: int = LIN_B, S: int = LIN_S, H: int = 8, D: int = W_D) -> int:
    """Algorithmic bytes of a linear-cache workload (K and V): quant reads the bf16 rows and
    writes codes + per-token scales; dequant reads codes + scales and writes bf16 rows; reshape
    reads and writes bf16 rows; plus the context lengths."""
    T = B * S
    per_row = {"linear_quant": D * 2 + D + 4, "linear_dequant": D + 4 + D * 2,
               "linear_reshape": 2 * D * 2}[op]
    return 2 * T * H * per_row + 4 * (B + 1)


def linear_call(torch, tmo, op: str, dev, g, B: int = LIN_B, S: int = LIN_S, L: int = LIN_L,
                H: int = 8, D: int = W_D):
    """One buffer set of a linear-cache workload and the closure that runs it."""
    T = B * S
    lens = torch.full((B,), S, dtype=torch.int32, device=dev)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev) * S
    if op == "linear_dequant":
        kc = torch.randint(-127, 128, (B, H, L, D), generator=g, device=dev, dtype=torch.int8)
        vc = torch.randint(-127, 128, (B, H, L, D), generator=g, device=dev, dtype=torch.int8)
        ks = torch.rand((B, H, L), generator=g, device=dev) * 0.05
        vs = torch.rand((B, H, L), generator=g, device=dev) * 0.05
        key = torch.empty((T, H, D), dtype=torch.bfloat16, device=dev)
        value = torch.empty_like(key)
        return lambda: tmo.dequant_from_linear_cache(key, value, kc, vc, ks, vs, lens, S, None,
                                                     None, None, 1, 8)
    key = torch.randn((T, H, D), generator=g, device=dev).to(torch.bfloat16)
    value = torch.randn((T, H, D), generator=g, device=dev).to(torch.bfloat16)
    if op == "linear_reshape":
        kc = torch.zeros((B, H, L, D), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        return lambda: tmo.reshape_linear_cache(key, value, kc, vc, cu, S, True, None, None, None)
    kc = torch.zeros((B, H, L, D), dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((B, H, L), device=dev)
    vs = torch.zeros_like(ks)
    return lambda: tmo.quant_to_linear_cache(key, value, kc, vc, ks, vs, cu, S, True, None, None,
                                             None)


def bench_linear(torch, tmo, op: str, dev, steps, warmup):
    """A linear-cache op over 8 x 4096 packed tokens: per set its own rows and caches."""
    alg = linear_bytes(op)
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(13)
    calls = [linear_call(torch, tmo, op, dev, g) for _ in range(sets)]
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, LIN_B * LIN_S, sets


ATTN_HQ = 32


def attn_bytes(layout, hq: int = ATTN_HQ, heads: int = 8, dim: int = W_D,
               int4: bool = False) -> int:
    """Algorithmic bytes of decode attention over `layout`: every key's K and V codes (dim
    bytes each, dim / 2 for int4 pairs) and scales once per KV head, q read and out written,
    block-table entries and lengths."""
    pages = int(((layout.context_lengths + layout.block_size - 1) // layout.block_size).sum())
    B = layout.context_lengths.numel()
    code = dim // 2 if int4 else dim
    return (layout.total_tokens * heads * 2 * (code + 4) + 2 * B * hq * dim * 2 + 4 * pages
            + 4 * B)


def int4_pages(torch, W, layout, dev, seed: int = 1009):
    """int4 pages over configs[4]'s layout: random codes in [-8, 7] packed K pairing channels
    [NB, 8, 16, 64] and V pairing rows [NB, 8, 8, 128], per-token fp32 scales."""
    NB, bs = layout.num_blocks, layout.block_size
    g = torch.Generator(device=dev).manual_seed(seed)
    def codes():
        return torch.randint(-8, 8, (NB, W.H, bs, W.D), generator=g, device=dev,
                             dtype=torch.int8)
    kc = W.pack_int4(codes(), 3)
    vc = W.pack_int4(codes(), 2)
    ks = 0.05 + 0.25 * torch.rand((NB, W.H, bs), generator=g, device=dev)
    vs = 0.05 + 0.25 * torch.rand((NB, W.H, bs), generator=g, device=dev)
    return kc, vc, ks, vs


def bench_decode_attn(torch, tmo, W, layout, dev, steps, warmup, int4: bool = False):
    """single_query_cached_kv_attn over configs[4]'s filled pages: one call per step (the pages
    are ~2.4 GB -- 1.2 GB as int4 -- far beyond the MALL)."""
    alg = attn_bytes(layout, int4=int4)
    kc, vc, ks, vs = int4_pages(torch, W, layout, dev) if int4 else W.cfg5_fill(layout, dev)
    B = layout.context_lengths.numel()
    g = torch.Generator(device=dev).manual_seed(17)
    q = torch.randn((B, 1, ATTN_HQ, W_D), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    ctx = layout.context_lengths.to(dev)
    bt = layout.block_tables.to(dev)
    mctx = layout.max_context_len
    calls = [lambda: tmo.single_query_cached_kv_attn(q, kc, vc, out, bt, ctx, ks, vs, None, mctx,
                                                     -1, -1, W_D ** -0.5, False,
                                                     4 if int4 else 8)]
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, layout.total_tokens, 1


def bench_smooth_quant(torch, tmo, W, case, dev, steps, warmup):
    alg = case.algorithmic_bytes()
    sets = n_sets(alg)
    g = torch.Generator(device=dev).manual_seed(8)
    calls = []
    for s in range(sets):
        x = case.x.to(dev) if s == 0 else \
            torch.randn(case.x.shape, generator=g, device=dev).to(case.x.dtype)
        sm = case.smooth.to(dev)
        tc = case.token_count.to(dev) if case.token_count is not None else None
        gi = case.gather_index.to(dev) if case.gather_index is not None else None
        out = torch.empty((case.rows, x.shape[-1]), dtype=torch.int8, device=dev)
        sc = torch.empty((case.rows,), dtype=torch.float32, device=dev)
        calls.append(lambda x=x, sm=sm, tc=tc, gi=gi, out=out, sc=sc:
                     tmo.moe_quantize(x, sm, None, tc, gi, None, out, sc))
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, case.rows, sets


def bench_dequant(torch, tmo, W, layout, dev, steps, warmup):
    alg = layout.algorithmic_bytes()
    kc, vc, ks, vs = W.cfg5_fill(layout, dev)
    total = layout.total_tokens
    key = torch.empty((total, kc.shape[1], kc.shape[3]), dtype=torch.bfloat16, device=dev)
    value = torch.empty_like(key)
    ctx = layout.context_lengths.to(dev)
    bt = layout.block_tables.to(dev)
    mctx = layout.max_context_len
    calls = [lambda: tmo.dequant_from_paged_cache(key, value, kc, vc, ks, vs, ctx, mctx, None,
                                                  bt, 1, 8)]
    ms = time_graph(torch, calls, steps, warmup)
    return ms, alg, total, 1


def profile_pass(torch, tmo, W, names, dev, n: int) -> None:
    """Eager calls of each config's op (no graph, no timing) for counter collection, then a
    plain copy kernel of known size: torch.neg over 1 GiB of fp32 reads 1 GiB and writes 1 GiB,
    so FETCH_SIZE / WRITE_SIZE of that dispatch calibrate the counters' units."""
    for name in names:
        if name in ("cfg1", "cfg2", "cfg3"):
            case = getattr(W, name)()
            k, v, sl = case.k.to(dev), case.v.to(dev), case.slot_mapping.to(dev)
            kc, vc, ks, vs = case.empty_caches(device=dev)
            fn = lambda: tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, sl)
        elif name == "reshape_paged":
            case = W.cfg3()
            k, v, sl = case.k.to(dev), case.v.to(dev), case.slot_mapping.to(dev)
            shape = (case.num_blocks, k.shape[1], case.block_size, k.shape[2])
            kc = torch.zeros(shape, dtype=k.dtype, device=dev)
            vc = torch.zeros_like(kc)
            fn = lambda: tmo.reshape_paged_cache(k, v, kc, vc, sl, False)
        elif name.startswith("offline"):
            case = W.cfg3()
            k, v, sl = case.k.to(dev), case.v.to(dev), case.slot_mapping.to(dev)
            cdt = torch.int8 if name == "offline_i8" else torch.float8_e4m3fn
            kc, vc, _, _ = case.empty_caches(device=dev)
            kc, vc = kc.view(cdt), vc.view(cdt)
            ks = torch.full((k.shape[1], k.shape[2]), 0.02, device=dev)
            fn = lambda: tmo.offline_quant_to_paged_cache(k, v, ks, ks, sl, kc, vc)
        elif name.startswith("fused_rope"):
            case3 = W.cfg3()
            qkv = torch.randn((FR_B, FR_S, fr_q_heads(name) + 2 * FR_HK, W_D),
                              device=dev).to(torch.bfloat16)
            kc = torch.zeros((case3.num_blocks, FR_HK, 16, W_D), dtype=torch.int8, device=dev)
            vc = torch.zeros_like(kc)
            ks = torch.zeros(kc.shape[:3], device=dev)
            vs = torch.zeros_like(ks)
            tab = torch.rand((8192, W_D), device=dev).to(torch.bfloat16)
            pid = torch.arange(FR_B, dtype=torch.int32, device=dev) * 512
            gm = torch.ones(W_D, device=dev).to(torch.bfloat16)
            sl = case3.slot_mapping.to(dev)
            if name == "fused_rope_ln":
                fn = lambda: tmo.fused_rope(qkv, kc, vc, tab, tab, pid, gm, gm, k_scale_hp=ks,
                                            v_scale_hp=vs, slot_mapping_hp=sl,
                                            norm_type="layernorm")
            else:
                fn = lambda: tmo.fused_rmsnorm_rope_store_paged_cache(qkv, kc, vc, tab, tab, pid,
                                                                      gm, gm, sl, ks, vs)
        elif name.startswith("linear"):
            fn = linear_call(torch, tmo, name, dev, torch.Generator(device=dev).manual_seed(13))
        elif name in ("decode_attn", "decode_attn_int4"):
            layout = W.cfg5()
            i4 = name == "decode_attn_int4"
            kc, vc, ks, vs = int4_pages(torch, W, layout, dev) if i4 else W.cfg5_fill(layout, dev)
            q = torch.randn((64, 1, ATTN_HQ, W_D), device=dev).to(torch.bfloat16)
            out = torch.empty_like(q)
            ctx, bt = layout.context_lengths.to(dev), layout.block_tables.to(dev)
            mctx = layout.max_context_len
            fn = lambda: tmo.single_query_cached_kv_attn(q, kc, vc, out, bt, ctx, ks, vs, None,
                                                         mctx, -1, -1, W_D ** -0.5, False,
                                                         4 if i4 else 8)
        elif name.startswith("cfg4"):
            case = getattr(W, name)()
            x, sm = case.x.to(dev), case.smooth.to(dev)
            tc = case.token_count.to(dev) if case.token_count is not None else None
            gi = case.gather_index.to(dev) if case.gather_index is not None else None
            fn = lambda: tmo.moe_quantize(x, sm, None, tc, gi)
        else:
            layout = W.cfg5()
            kc, vc, ks, vs = W.cfg5_fill(layout, dev)
            key = torch.empty((layout.total_tokens, W.H, W.D), dtype=torch.bfloat16, device=dev)
            val = torch.empty_like(key)
            ctx, bt = layout.context_lengths.to(dev), layout.block_tables.to(dev)
            mctx = layout.max_context_len
            fn = lambda: tmo.dequant_from_paged_cache(key, val, kc, vc, ks, vs, ctx, mctx, None,
                                                      bt, 1, 8)
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        print(f"# profile pass: {name} x{n}", file=sys.stderr, flush=True)
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(n):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"# profile pass: calibration copy (neg) of {src.numel() * 4} bytes x{n}",
          file=sys.stderr, flush=True)


def copy_ceiling_gbs(torch, dev) -> float:
    """A plain torch copy-class kernel (neg over 1 GiB fp32: 1 GiB read + 1 GiB written) on the
    same device: the practical streaming rate the path's kernels can be compared against."""
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    ms = time_graph(torch, [lambda: torch.neg(src, out=dst)], 20, 4)
    return 2 * src.numel() * 4 / (ms * 1e-3) / 1e9


def stream_ceilings() -> dict | None:
    """Practical HBM ceilings for the workloads' traffic shapes, from the minimal streaming
    kernels of tests/native/stream_ceiling.hip (built by __graft_entry__.build()); None when
    that program is not built."""
    exe = REPO / "tests" / "native" / "_build" / "stream_ceiling"
    if not exe.exists():
        return None
    import subprocess
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    if res.returncode != 0:
        return {"error": (res.stdout + res.stderr).strip()[-200:]}
    return json.loads(res.stdout.strip().splitlines()[-1])


def launch_floor_us(torch, tmo, dev) -> float:
    """Duration of the smallest quant_to_paged_cache launch (1 token, 1 head) -- the per-call
    floor that bounds the latency-bound configs."""
    k = torch.randn(1, 1, 128, device=dev).to(torch.bfloat16)
    kc = torch.zeros(1, 1, 16, 128, dtype=torch.int8, device=dev)
    ks = torch.zeros(1, 1, 16, device=dev)
    sl = torch.zeros(1, dtype=torch.int32, device=dev)
    calls = [lambda: tmo.quant_to_paged_cache(k, None, kc, None, ks, None, sl)] * 64
    return 1000.0 * time_graph(torch, calls, 640, 64)


# ---------------------------------------------------------------------------- CPU baseline

def cpu_baseline(torch, W, workload: str, seconds: float) -> dict:
    """The CPU oracle on a bounded sample of the headline workload, on this host's cores."""
    import oracle
    nthreads = oracle.default_threads()
    if workload in ("cfg1", "cfg2", "cfg3"):
        case = getattr(W, workload)()
        n = min(case.tokens, 4096)
        sub = W.PagedQuantCase(case.name, case.k[:n].contiguous(), case.v[:n].contiguous(),
                               case.slot_mapping[:n].contiguous(), case.num_blocks)
        kc, vc, ks, vs = sub.empty_caches()
        fn = lambda: oracle.quant_to_paged_cache(sub.k, sub.v, kc, vc, ks, vs, sub.slot_mapping,
                                                 nthreads=nthreads)
        alg, units, desc = sub.algorithmic_bytes(), sub.valid_tokens(), \
            f"quant_to_paged_cache on the first {n} tokens of {workload}"
    elif workload == "reshape_paged":
        case = W.cfg3()
        n = 4096
        sub = W.PagedQuantCase(case.name, case.k[:n].contiguous(), case.v[:n].contiguous(),
                               case.slot_mapping[:n].contiguous(), case.num_blocks)
        shape = (case.num_blocks, W.H, case.block_size, W.D)
        kc = torch.zeros(shape, dtype=case.k.dtype)
        vc = torch.zeros_like(kc)
        fn = lambda: oracle.reshape_paged_cache(sub.k, sub.v, kc, vc, sub.slot_mapping,
                                                nthreads=nthreads)
        alg = 2 * 2 * n * W.H * W.D * case.k.element_size() + 4 * n
        units, desc = n, f"reshape_paged_cache on the first {n} tokens of cfg3"
    elif workload.startswith("offline"):
        case = W.cfg3()
        n = 4096
        sub = W.PagedQuantCase(case.name, case.k[:n].contiguous(), case.v[:n].contiguous(),
                               case.slot_mapping[:n].contiguous(), case.num_blocks)
        cdt = torch.int8 if workload == "offline_i8" else torch.float8_e4m3fn
        kc, vc = (c.view(cdt) for c in sub.empty_caches()[:2])
        gs = torch.Generator().manual_seed(2024)
        ks = 0.005 + 0.05 * torch.rand(W.H, W.D, generator=gs)
        fn = lambda: oracle.offline_quant_to_paged_cache(sub.k, sub.v, ks, ks, sub.slot_mapping,
                                                         kc, vc, nthreads=nthreads)
        alg, units, desc = offline_bytes(sub), sub.valid_tokens(), \
            f"offline_quant_to_paged_cache on the first {n} tokens of cfg3"
    elif workload.startswith("fused_rope"):
        ln = workload == "fused_rope_ln"
        n = 512
        g = torch.Generator().manual_seed(3)
        hq = fr_q_heads(workload)
        qkv = torch.randn((1, n, hq + 2 * FR_HK, W_D), generator=g).to(torch.bfloat16)
        kc = torch.zeros((n // 16, FR_HK, 16, W_D), dtype=torch.int8)
        vc = torch.zeros_like(kc)
        ks = torch.zeros(kc.shape[:3])
        vs = torch.zeros_like(ks)
        tab = torch.rand((n, W_D), generator=g).to(torch.bfloat16)
        pid = torch.zeros(1, dtype=torch.int32)
        gm = torch.ones(W_D).to(torch.bfloat16)
        sl = torch.arange(n, dtype=torch.int32)
        fn = lambda: oracle.fused_rope_paged(qkv, kc, vc, tab, tab, pid, gm, ks, vs, sl, 1e-5,
                                             None if ln else gm, nthreads=nthreads,
                                             norm_type="layernorm" if ln else "rmsnorm",
                                             k_beta=gm if ln else None)
        alg, units, desc = fused_rope_bytes(n, hq=hq), n, f"fused rope of one {n}-token sequence"
    elif workload in ("decode_attn", "decode_attn_int4"):
        i4 = workload == "decode_attn_int4"
        layout = W.cfg5()
        nseq = 2
        ctx = layout.context_lengths[:nseq].contiguous()
        pages = [(int(c) + W.BS - 1) // W.BS for c in ctx.tolist()]
        bt = torch.zeros(nseq, max(pages), dtype=torch.int32)
        p0 = 0
        for i, pn in enumerate(pages):  # the sample's pages renumbered into a compact cache
            bt[i, :pn] = torch.arange(p0, p0 + pn, dtype=torch.int32)
            p0 += pn
        sub = W.DequantLayout("cfg5-sample", ctx, bt, p0)
        g = torch.Generator().manual_seed(5)
        lo, hi = (-8, 8) if i4 else (-127, 128)
        kc = torch.randint(lo, hi, (p0, W.H, W.BS, W.D), generator=g, dtype=torch.int8)
        vc = torch.randint(lo, hi, (p0, W.H, W.BS, W.D), generator=g, dtype=torch.int8)
        ks = torch.rand(p0, W.H, W.BS, generator=g) * 0.05
        vs = torch.rand(p0, W.H, W.BS, generator=g) * 0.05
        q = torch.randn(nseq, ATTN_HQ, W.D, generator=g).to(torch.bfloat16)
        if i4:
            kc, vc = W.pack_int4(kc, 3), W.pack_int4(vc, 2)
            fn = lambda: oracle.cached_kv_attn(q, kc, vc, bt, ctx, W.D ** -0.5, ks, vs,
                                               int4=True, nthreads=nthreads)
        else:
            fn = lambda: oracle.single_query_attn(q, kc, vc, bt, ctx, W.D ** -0.5, ks, vs,
                                                  nthreads=nthreads)
        alg, units = attn_bytes(sub, int4=i4), sub.total_tokens
        desc = (f"float64 decode attention of the first {nseq} sequences of cfg5 ({units} keys, "
                f"{ATTN_HQ} query heads{', int4 pages' if i4 else ''})")
    elif workload.startswith("linear"):
        nb, S, H = LIN_B, 1024, W.H   # every sequence (the oracle threads over sequences)
        op = {"linear_reshape": 0, "linear_quant": 1, "linear_dequant": 3}[workload]
        g = torch.Generator().manual_seed(13)
        lens = torch.full((nb,), S, dtype=torch.int32)
        cu = torch.arange(nb + 1, dtype=torch.int32) * S
        key = torch.randn((nb * S, H, W.D), generator=g).to(torch.bfloat16)
        value = torch.randn((nb * S, H, W.D), generator=g).to(torch.bfloat16)
        cdt = torch.bfloat16 if op == 0 else torch.int8
        kc = torch.zeros((nb, H, LIN_L, W.D), dtype=cdt)
        vc = torch.zeros_like(kc)
        ks = torch.rand((nb, H, LIN_L), generator=g) * 0.05
        vs = torch.rand((nb, H, LIN_L), generator=g) * 0.05
        if op == 3:
            kc.random_(-127, 128, generator=g)
            vc.random_(-127, 128, generator=g)
        fn = lambda: oracle.linear_cache(op, key, value, kc, vc, lens if op == 3 else cu, S,
                                         packed=op != 3, key_scale=ks, value_scale=vs, smode=1,
                                         nthreads=nthreads)
        alg, units = linear_bytes(workload, B=nb, S=S), nb * S
        desc = f"{workload} on the first {S} tokens of each of the {nb} sequences"
    elif workload.startswith("cfg4"):
        case = getattr(W, workload)()
        n = min(case.rows, 2048)
        gi = case.gather_index[:n].contiguous() if case.gather_index is not None else None
        x = case.x if gi is not None else case.x[:n].contiguous()
        tc = None
        if case.token_count is not None:  # the first n rows keep their expert grouping
            ends = torch.cumsum(case.token_count.to(torch.int64), 0).clamp(max=n)
            tc = torch.diff(ends, prepend=torch.zeros(1, dtype=torch.int64)).to(torch.int32)
        sub = W.SmoothQuantCase(case.name, x, case.smooth, tc, gi)
        out = torch.empty((n, x.shape[-1]), dtype=torch.int8)
        sc = torch.empty((n,), dtype=torch.float32)
        fn = lambda: oracle.scaled_quantize_per_token(sub.x, out, sc, sub.smooth, sub.token_count,
                                                      sub.gather_index, nthreads=nthreads)
        alg, units, desc = sub.algorithmic_bytes(), n, f"smooth quant of the first {n} rows of {workload}"
    else:
        layout = W.cfg5()
        nseq = 2
        ctx = layout.context_lengths[:nseq].contiguous()
        pages = [(int(c) + W.BS - 1) // W.BS for c in ctx.tolist()]
        bt = torch.zeros(nseq, max(pages), dtype=torch.int32)
        p0 = 0
        for i, p in enumerate(pages):  # the sample's pages renumbered into a compact cache
            bt[i, :p] = torch.arange(p0, p0 + p, dtype=torch.int32)
            p0 += p
        sub = W.DequantLayout("cfg5-sample", ctx, bt, p0)
        g = torch.Generator().manual_seed(5)
        kc = torch.randint(-127, 128, (p0, W.H, W.BS, W.D), generator=g, dtype=torch.int8)
        vc = torch.randint(-127, 128, (p0, W.H, W.BS, W.D), generator=g, dtype=torch.int8)
        ks = torch.rand(p0, W.H, W.BS, generator=g) * 0.05
        vs = torch.rand(p0, W.H, W.BS, generator=g) * 0.05
        key = torch.empty(sub.total_tokens, W.H, W.D, dtype=torch.bfloat16)
        value = torch.empty_like(key)
        fn = lambda: oracle.dequant_from_paged_cache(key, value, kc, vc, ks, vs, ctx, None, bt, 1,
                                                     nthreads=nthreads)
        alg, units = sub.algorithmic_bytes(), sub.total_tokens
        desc = f"dequant of the first {nseq} sequences of cfg5 ({units} tokens)"
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(alg / t / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": f"{desc}; median of {len(times)} runs, {t * 1e3:.3f} ms each",
            "tokens_per_s": round(units / t, 1), "cpu_model": cpu_model()}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), as the baseline's hardware."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------------- main

def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards by KV heads or sequences with no exchange between GPUs)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import domesticated_torch_mlu_ops_amd as tmo
    from tests import workloads as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    todo = [args.workload] if args.configs == "headline" else \
        ["cfg1", "cfg2", "cfg3", "cfg4", "cfg4_moe", "cfg5", "offline_i8", "offline_f8",
         "fused_rope", "fused_rope_ln", "fused_rope_70b", "linear_quant", "linear_dequant",
         "linear_reshape", "decode_attn", "reshape_paged", "decode_attn_int4"]
    if args.workload not in todo:
        todo.append(args.workload)
    if args.profile_pass:
        profile_pass(torch, tmo, W, todo, dev, args.profile_pass)
        return
    # rocprofv3 per-dispatch mean duration of each workload's kernel, from the committed
    # profile summary: graph replays overlap consecutive small calls, so for the decode-sized
    # configs the per-call figure and the per-dispatch figure differ
    tfile = REPO / "profiles" / "traffic.json"
    tjson = json.loads(tfile.read_text()) if tfile.exists() else {}
    profiled = {k: v["dispatch_us"] for k, v in tjson.items()
                if isinstance(v, dict) and "dispatch_us" in v}
    # where roofline.traffic and us_per_dispatch_rocprof come from: the committed profile, not
    # this run (rocprofv3 cannot run inside the timed process)
    src = tjson.get("_source", {})
    profile_source = (f"profiles/traffic.json: rocprofv3 kernel trace and FETCH_SIZE / WRITE_SIZE "
                      f"counters of commit {src.get('commit', 'unknown')} ({src.get('date', '?')}), "
                      f"not this run")
    per = {}
    for name in todo:
        t0 = time.perf_counter()
        if name in ("cfg1", "cfg2", "cfg3"):
            ms, alg, units, sets = bench_paged_quant(torch, tmo, W, getattr(W, name)(), dev,
                                                     args.steps, args.warmup)
        elif name == "reshape_paged":
            ms, alg, units, sets = bench_reshape(torch, tmo, W, W.cfg3(), dev,
                                                 max(20, args.steps // 4), max(4, args.warmup // 4))
        elif name.startswith("cfg4"):
            ms, alg, units, sets = bench_smooth_quant(torch, tmo, W, getattr(W, name)(), dev,
                                                      args.steps, args.warmup)
        elif name.startswith("offline"):
            cdt = torch.int8 if name == "offline_i8" else torch.float8_e4m3fn
            ms, alg, units, sets = bench_offline(torch, tmo, W, W.cfg3(), cdt, dev, args.steps,
                                                 args.warmup)
        elif name.startswith("fused_rope"):
            ms, alg, units, sets = bench_fused_rope(torch, tmo, W, dev, max(20, args.steps // 4),
                                                    args.warmup // 4, name == "fused_rope_ln",
                                                    fr_q_heads(name))
        elif name.startswith("linear"):
            ms, alg, units, sets = bench_linear(torch, tmo, name, dev, max(20, args.steps // 4),
                                                max(4, args.warmup // 4))
        elif name in ("decode_attn", "decode_attn_int4"):
            ms, alg, units, sets = bench_decode_attn(torch, tmo, W, W.cfg5(), dev,
                                                     max(10, args.steps // 40),
                                                     max(2, args.warmup // 10),
                                                     int4=name == "decode_attn_int4")
        else:
            ms, alg, units, sets = bench_dequant(torch, tmo, W, W.cfg5(), dev,
                                                 max(10, args.steps // 40), max(2, args.warmup // 10))
        gbs = alg / (ms * 1e-3) / 1e9
        per[name] = {"kernel": KERNELS[name], "us_per_call": round(ms * 1e3, 3),
                     "us_per_call_mean": round(LAST_MEAN_MS * 1e3, 3),
                     "algorithmic_bytes": alg, "GB_s": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_GBS, 4),
                     "units_per_s": round(units / (ms * 1e-3), 1), "buffer_sets": sets}
        if name in profiled:  # per-dispatch duration of the same kernel in the committed profile
            per[name]["us_per_dispatch_rocprof"] = profiled[name]
        if name == "cfg4_moe":  # every gathered row counted as read (top-2 reads a token twice)
            rb = W.cfg4_moe().algorithmic_bytes(per_row_reads=True)
            per[name]["per_row_read_bytes"] = rb
            per[name]["per_row_read_GB_s"] = round(rb / (ms * 1e-3) / 1e9, 1)
        print(f"# {name}: {ms * 1e3:.2f} us/call  {gbs:.1f} GB/s  ({100 * gbs / PEAK_GBS:.1f}% of "
              f"peak)  [{time.perf_counter() - t0:.1f} s]", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    floor = launch_floor_us(torch, tmo, dev) if args.configs == "all" else None
    ceiling = copy_ceiling_gbs(torch, dev) if args.configs == "all" else None
    streams = stream_ceilings() if args.configs == "all" else None

    head = per[args.workload]
    traffic = tjson.get(args.workload, {}).get("hbm_bytes_per_launch")
    cpu = cpu_baseline(torch, W, args.workload, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": head["GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, BASELINE.md section 3)",
        "config": {"workload": WORKLOADS[args.workload],
                   "io": {"cfg5": "int8 codes + fp32 scales in; bf16 out",
                          "offline_i8": "bf16 in; int8 codes out (static per-channel scales)",
                          "offline_f8": "bf16 in; float8_e4m3fn codes out (static per-channel scales)",
                          "fused_rope": "bf16 qkv in; bf16 Q written back; int8 K/V codes + fp32 scales out",
                          "fused_rope_ln": "bf16 qkv in; bf16 Q written back; int8 K/V codes + fp32 scales out",
                          "fused_rope_70b": "bf16 qkv in; bf16 Q written back; int8 K/V codes + fp32 scales out",
                          "linear_dequant": "int8 codes + fp32 scales in; bf16 out",
                          "linear_reshape": "bf16 in; bf16 out",
                          "reshape_paged": "bf16 K/V rows in; bf16 pages out",
                          "decode_attn": "bf16 q, int8 K/V pages + fp32 scales in; bf16 out; fp32 softmax",
                          "decode_attn_int4": "bf16 q, int4 K/V pages + fp32 scales in; bf16 out; fp32 softmax"}
                   .get(args.workload, "bf16 in; int8 codes + fp32 scales out"),
                   "tokens_per_s": head["units_per_s"],
                   "frac_of_peak": head["frac_of_peak"]},
        "roofline": {"bound": "hbm", "achieved": head["GB_s"], "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": head["frac_of_peak"], "traffic": traffic,
                     "traffic_source": profile_source, "kernel": head["kernel"]},
        "cpu_baseline": cpu,
        "per_config": per,
        "us_per_dispatch_rocprof_source": profile_source,
        "settle_s": SETTLE_S,
        "launch_floor_us": round(floor, 3) if floor is not None else None,
        "copy_ceiling_GB_s": round(ceiling, 1) if ceiling is not None else None,
        "stream_ceilings": streams,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
