"""Seeded sweep of random shapes for the paged-cache ops and the smooth quantiser, GPU against
the oracle, bit-exact (the same bar as tests/test_gpu_parity.py, whose helpers run each case).

Each case draws its shape from a fixed seed: dtypes f32 / f16 / bf16, head sizes that take the
vector paths (powers of two times 8) and the generic ones, block sizes that are and are not
powers of two, int8 and float8_e4m3fn pages, -1 and out-of-range slots, per-token and
per-channel dequant scales with and without context_seq_offset, empty sequences, K only, and
smooth-quant rows with and without gather / groups / a smooth vector.  Sizes stay small so the
oracle finishes in well under a second per case.
"""
import pytest
import torch

from tests import workloads as W
from tests.test_gpu_parity import _dequant_both, _sq_both, check_offline, check_quant

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
HEAD_SIZES = [8, 16, 32, 64, 128, 256, 24, 40, 72, 96]
BLOCK_SIZES = [16, 32, 8, 1, 5, 12]


def _rng(seed):
    return torch.Generator().manual_seed(seed)


def _pick(g, seq):
    return seq[int(torch.randint(0, len(seq), (1,), generator=g))]


def _int(g, lo, hi):
    return int(torch.randint(lo, hi + 1, (1,), generator=g))


@pytest.mark.parametrize("seed", range(24))
def test_sweep_quant_to_paged_cache(tmo, ref, dev, seed):
    g = _rng(1000 + seed)
    dtype, D, BS = _pick(g, DTYPES), _pick(g, HEAD_SIZES), _pick(g, BLOCK_SIZES)
    H, T = _int(g, 1, 9), _int(g, 1, 300)
    NB = max(1, (T + BS - 1) // BS + _int(g, 0, 8))
    k = (torch.randn(T, H, D, generator=g) * torch.logspace(-2, 2, T)[:, None, None]).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32) if T <= NB * BS else \
        torch.randint(0, NB * BS, (T,), generator=g).to(torch.int32)
    slot[torch.rand(T, generator=g) < 0.1] = -1
    slot[torch.rand(T, generator=g) < 0.03] = NB * BS + 3
    case = W.PagedQuantCase(f"sweep{seed} {dtype} D={D} BS={BS} H={H} T={T}", k, v, slot, NB, BS)
    cdt = torch.float8_e4m3fn if seed % 3 == 0 else torch.int8
    print(f"[sweep quant] {case.name} {cdt}", flush=True)
    if T <= NB * BS:  # unique slots: the result does not depend on write order
        check_quant(tmo, ref, dev, case, cache_dtype=cdt)
        check_quant(tmo, ref, dev, case, with_v=False, cache_dtype=cdt)


@pytest.mark.parametrize("seed", range(16))
def test_sweep_offline_quant(tmo, ref, dev, seed):
    g = _rng(2000 + seed)
    dtype, D, BS = _pick(g, DTYPES), _pick(g, HEAD_SIZES), _pick(g, BLOCK_SIZES)
    H, T = _int(g, 1, 9), _int(g, 1, 200)
    NB = (T + BS - 1) // BS + _int(g, 0, 4)
    k = (torch.randn(T, H, D, generator=g) * 4).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[torch.rand(T, generator=g) < 0.1] = -1
    if seed % 2:
        ks = 0.01 + 0.1 * torch.rand(H, D, generator=g)
        vs = 0.02 + 0.1 * torch.rand(H, D, generator=g)
    else:
        ks, vs = 0.0313, 0.047
    cdt = torch.float8_e4m3fn if seed % 4 < 2 else torch.int8
    name = f"sweep{seed} {dtype} D={D} BS={BS} H={H} T={T} {cdt}"
    print(f"[sweep offline] {name}", flush=True)
    check_offline(tmo, ref, dev, name, k, v, ks, vs, slot, NB, BS, cdt)


@pytest.mark.parametrize("seed", range(20))
def test_sweep_dequant(tmo, ref, dev, seed):
    g = _rng(3000 + seed)
    out_dtype = _pick(g, DTYPES)
    D = _pick(g, [16, 32, 64, 128, 256, 48, 80])
    BS = _pick(g, [16, 32, 8, 12])
    H, B = _int(g, 1, 8), _int(g, 1, 70)
    max_ctx = _int(g, 1, 120)
    ctx = torch.randint(0, max_ctx + 1, (B,), generator=g).to(torch.int32)
    MB = (max_ctx + BS - 1) // BS
    NB = B * MB + _int(g, 0, 8)
    bt = torch.randperm(NB, generator=g)[: B * MB].reshape(B, MB).to(torch.int32)
    if seed % 5 == 0:
        bt[0, 0] = -1  # a missing page: its rows keep the sentinel
    kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    mode = seed % 2
    if mode == 1:
        ks, vs = torch.rand(NB, H, BS, generator=g) * 0.1, torch.rand(NB, H, BS, generator=g) * 0.1
    else:
        ks, vs = torch.rand(H, D, generator=g) * 0.05, torch.rand(H, D, generator=g) * 0.05
    layout = W.DequantLayout(f"sweep{seed} D={D} BS={BS} H={H} B={B}", ctx, bt, NB, BS)
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    print(f"[sweep dequant] {layout.name} mode={mode} {out_dtype}", flush=True)
    _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode, with_v=seed % 3 != 0)
    if seed % 4 == 1:  # explicit start rows, shifted, with spare rows at the end
        off = (torch.cumsum(ctx, 0) - ctx + 2).to(torch.int32)
        _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode, seq_offset=off,
                      total=layout.total_tokens + 6)


@pytest.mark.parametrize("seed", range(16))
def test_sweep_smooth_quant(tmo, ref, dev, seed):
    g = _rng(4000 + seed)
    dtype = _pick(g, DTYPES)
    C = _pick(g, [64, 128, 512, 1024, 4096, 96, 200, 8192])
    n0 = _int(g, 1, 200)
    x = (torch.randn(n0, C, generator=g) * torch.logspace(-2, 2, n0)[:, None]).to(dtype)
    kind = seed % 4
    if kind == 0:    # dense rows, per-channel smooth
        case = W.SmoothQuantCase(f"sweep{seed}", x, 0.5 + torch.rand(C, generator=g))
    elif kind == 1:  # dense rows, scalar smooth
        case = W.SmoothQuantCase(f"sweep{seed}", x, torch.tensor([1.3]))
    else:            # gathered rows in groups (MoE), per-group smooth rows
        E = _int(g, 1, 12)
        topk = _int(g, 1, 3)
        experts = torch.randint(0, E, (n0 * topk,), generator=g)
        order = torch.sort(experts, stable=True).indices
        gi = (order // topk).to(torch.int32)
        tc = torch.bincount(experts, minlength=E).to(torch.int32)
        sm = 0.5 + torch.rand(E, C, generator=g)
        case = W.SmoothQuantCase(f"sweep{seed} E={E} top{topk}", x, sm, tc, gi)
    print(f"[sweep smooth] {case.name} {dtype} C={C} n0={n0} kind={kind}", flush=True)
    _sq_both(tmo, ref, dev, case)
