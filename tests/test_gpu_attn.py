"""GPU parity of single_query_cached_kv_attn (one query token per sequence over paged KV
caches) against the float64 CPU oracle (decision D12 of oracle/tmo_oracle.c).

Floating point, so the bar is a stated tolerance per output dtype: with r the oracle's float64
result and vmax the largest |V| entry the sequence can read,
    |out - r| <= rtol * |r| + atol * vmax,
    rtol = 2^-7 (bf16: one unit in the last place), 2^-10 (fp16), 2^-16 (fp32);
    atol = 2^-14 (bf16, fp16), 2^-16 (fp32)
-- the kernel accumulates in fp32 with exact int8 operands and 16-bit-split probabilities, so
its own error is far inside one output ulp; the tolerance is the output rounding.  The
log-sum-exp: |lse - r| <= 2^-14 * max(1, |r|).  Cases: the three q dtypes, int8 caches with
per-token / per-channel / per-tensor scales and unquantised caches, head sizes 64 / 128 / 256
and off-grid ones (generic kernel), query-head groups 1..16 and 20, block sizes 16 / 32 / 8,
windows, ALiBi, missing pages, long contexts over several splits, 3-D q, and configs[4]'s
pages with 32 query heads.  Several query tokens per sequence (the 4-D q [batch, seq_q, heads,
D] and the 3-D q with cu_seq_q, causal within the new tokens) and the sink are held to the
same bar against the oracle's cached_kv_attn, with rows of no sequence left untouched.
"""
import math

import pytest
import torch

from tests import workloads as W

pytestmark = pytest.mark.gpu

RTOL = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -16}
ATOL = {torch.bfloat16: 2.0 ** -14, torch.float16: 2.0 ** -14, torch.float32: 2.0 ** -16}


def _vmax(case, vs):
    v = case.v_cache.double()
    if vs is not None:
        if vs.dim() == 3:
            v = v * vs.double()[..., None]
        elif vs.dim() == 2:
            v = v * vs.double()[None, :, None, :]
        else:
            v = v * float(vs)
    return float(v.abs().max())


def run_attn(tmo, ref, dev, case, scale=0.0883883, window=-1, four_d=True, with_lse=True,
             bit=None, per_tensor=False, max_ctx=None):
    q = case.q
    kbit = 8 if case.k_cache.dtype == torch.int8 else -1
    ks, vs = case.k_scale, case.v_scale
    if per_tensor:
        ks, vs = torch.tensor([0.0137]), torch.tensor([0.0211])
    want, wlse = ref.single_query_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                       case.context_lens, scale,
                                       ks.expand(case.k_cache.shape[1], q.shape[-1])
                                       if per_tensor else ks,
                                       vs.expand(case.k_cache.shape[1], q.shape[-1])
                                       if per_tensor else vs,
                                       case.alibi, window)
    qd = (q[:, None] if four_d else q).to(dev)
    res = tmo.single_query_cached_kv_attn(
        qd, case.k_cache.to(dev), case.v_cache.to(dev), None, case.block_tables.to(dev),
        case.context_lens.to(dev), ks.to(dev) if ks is not None else None,
        vs.to(dev) if vs is not None else None,
        case.alibi.to(dev) if case.alibi is not None else None,
        case.max_context_len if max_ctx is None else max_ctx, window, -1, scale,
        return_lse=with_lse, kv_cache_quant_bit_size=kbit if bit is None else bit)
    out, lse = res if with_lse else (res, None)
    torch.cuda.synchronize()
    out = out.cpu()
    got = (out[:, 0] if four_d else out).double()
    vmax = _vmax(case, vs)
    err = (got - want).abs()
    lim = RTOL[q.dtype] * want.abs() + ATOL[q.dtype] * vmax
    bad = err > lim
    assert not bad.any(), (f"{int(bad.sum())} outputs off; worst {float((err / lim).max()):.3g}x "
                           f"the tolerance at {tuple(bad.nonzero()[0].tolist())}")
    if with_lse:
        lse = lse.cpu().double()
        lse = lse[..., 0] if four_d else lse.transpose(0, 1)
        fin = torch.isfinite(wlse)
        assert torch.equal(torch.isfinite(lse), fin)
        assert ((lse[fin] - wlse[fin]).abs() <= 2.0 ** -14 * wlse[fin].abs().clamp(min=1)).all()
    return got, want


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_attn_dtypes_and_cache_kinds(tmo, ref, dev, dtype, kv):
    case = W.attn_case(dtype, 11, kv=kv, B=6, Hq=8, Hkv=2, D=128, BS=16, NB=96, max_ctx=250)
    run_attn(tmo, ref, dev, case)


def test_attn_per_tensor_scales(tmo, ref, dev):
    case = W.attn_case(torch.bfloat16, 12, kv="int8_token", B=4, Hq=4, Hkv=4, D=128, max_ctx=90)
    run_attn(tmo, ref, dev, case, per_tensor=True)


@pytest.mark.parametrize("D", [64, 128, 256, 96, 40])
@pytest.mark.parametrize("kv", ["int8_token", "plain"])
def test_attn_head_sizes(tmo, ref, dev, D, kv):
    case = W.attn_case(torch.bfloat16, 13 + D, kv=kv, B=4, Hq=8, Hkv=4, D=D, BS=16, NB=64,
                       max_ctx=150)
    run_attn(tmo, ref, dev, case, scale=1.0 / math.sqrt(D))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 8), (64, 8), (16, 1), (40, 2)])
def test_attn_query_head_groups(tmo, ref, dev, Hq, Hkv):
    case = W.attn_case(torch.bfloat16, 14 + Hq, kv="int8_token", B=3, Hq=Hq, Hkv=Hkv, D=128,
                       NB=48, max_ctx=120)
    run_attn(tmo, ref, dev, case)


@pytest.mark.parametrize("BS", [16, 32, 64, 8, 1])
def test_attn_block_sizes(tmo, ref, dev, BS):
    case = W.attn_case(torch.float16, 15 + BS, kv="int8_token", B=4, Hq=8, Hkv=2, D=128, BS=BS,
                       NB=max(64, 4 * ((100 + BS - 1) // BS)), max_ctx=100)
    run_attn(tmo, ref, dev, case)


def test_attn_windows_alibi_missing_pages_and_layouts(tmo, ref, dev):
    case = W.attn_case(torch.bfloat16, 16, kv="int8_token", B=5, Hq=8, Hkv=2, D=128, NB=80,
                       max_ctx=200, alibi=True)
    case.block_tables[0, 3] = -1                   # a missing page: its keys are masked
    case.block_tables[2, 0] = 10 ** 6              # outside the cache: masked too
    for window in (-1, 0, 1, 17, 150, 10 ** 6):
        run_attn(tmo, ref, dev, case, window=window)
    case.alibi = None
    run_attn(tmo, ref, dev, case, four_d=False)
    run_attn(tmo, ref, dev, case, with_lse=False)
    run_attn(tmo, ref, dev, case, max_ctx=0)       # "uncertain maximum": one split
    run_attn(tmo, ref, dev, case, max_ctx=-1)      # negative counts as unknown, like 0


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain"])
def test_attn_long_contexts_over_splits(tmo, ref, dev, kv):
    """Few sequences with long contexts: the keys of each (sequence, KV head) are spread over
    several workgroups and merged by the combine kernel."""
    case = W.attn_case(torch.bfloat16, 17, kv=kv, B=2, Hq=8, Hkv=2, D=128, BS=16, NB=1100,
                       max_ctx=8000)
    case.context_lens[1] = 4097
    run_attn(tmo, ref, dev, case)
    run_attn(tmo, ref, dev, case, window=3000)
    run_attn(tmo, ref, dev, case, max_ctx=1000)    # an understated maximum: the last split takes the rest


def test_attn_decode_on_configs4_pages(tmo, ref, dev):
    """configs[4]'s page layout (64 sequences, contexts 1024..32768, 8 KV heads x 128, int8
    pages with per-token scales) with 32 query heads, on a sample of 6 sequences checked
    against the oracle (the full batch would take the float64 oracle minutes)."""
    layout = W.cfg5()
    sel = torch.tensor([0, 1, 7, 20, 41, 63])
    ctx = layout.context_lengths[sel].contiguous()
    bt = layout.block_tables[sel].contiguous()
    used = [bt[i, :(c + 15) // 16] for i, c in enumerate(ctx.tolist())]
    pages = torch.unique(torch.cat(used))                  # sorted page ids the sample reads
    bt2 = torch.full_like(bt, -1)
    for i, u in enumerate(used):                           # renumber into a compact cache
        bt2[i, :u.numel()] = torch.searchsorted(pages, u).to(torch.int32)
    g = torch.Generator().manual_seed(5)
    NB = pages.numel()
    kc = torch.randint(-127, 128, (NB, 8, 16, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (NB, 8, 16, 128), generator=g, dtype=torch.int8)
    ks = 0.005 + 0.02 * torch.rand(NB, 8, 16, generator=g)
    vs = 0.005 + 0.02 * torch.rand(NB, 8, 16, generator=g)
    q = torch.randn(len(sel), 32, 128, generator=g).to(torch.bfloat16)
    case = W.AttnCase(q, kc, vc, ks, vs, bt2, ctx)
    run_attn(tmo, ref, dev, case)


def run_attn_mq(tmo, ref, dev, case, q, cu=None, sink=None, scale=0.0883883, window=-1,
                max_seq_q=-1, max_ctx=None, with_lse=True):
    """Several query tokens per sequence: q [B, S, Hq, D] or [T, Hq, D] with cu.  The output
    starts as a sentinel, which rows of no sequence must keep."""
    kbit = 8 if case.k_cache.dtype == torch.int8 else -1
    want, wlse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                    case.context_lens, scale, case.k_scale, case.v_scale,
                                    case.alibi, window, cu_seq_q=cu, sink=sink)
    out = torch.full(q.shape, 7.0, dtype=q.dtype, device=dev)
    res = tmo.single_query_cached_kv_attn(
        q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev), out, case.block_tables.to(dev),
        case.context_lens.to(dev), case.k_scale.to(dev) if case.k_scale is not None else None,
        case.v_scale.to(dev) if case.v_scale is not None else None,
        case.alibi.to(dev) if case.alibi is not None else None,
        case.max_context_len if max_ctx is None else max_ctx, window, -1, scale,
        return_lse=with_lse, kv_cache_quant_bit_size=kbit,
        cu_seq_q=cu.to(dev) if cu is not None else None, max_seq_q=max_seq_q,
        sink=sink.to(dev) if sink is not None else None)
    torch.cuda.synchronize()
    got = out.cpu().double()
    held = ~want.isnan()
    assert (got[~held] == 7.0).all(), "a row of no sequence was written"
    vmax = _vmax(case, case.v_scale)
    err = (got - want).abs()
    lim = RTOL[q.dtype] * want.abs() + ATOL[q.dtype] * vmax
    bad = (err > lim) & held
    assert not bad.any(), (f"{int(bad.sum())} outputs off; worst {float((err / lim)[held].max()):.3g}x "
                           f"the tolerance at {tuple(bad.nonzero()[0].tolist())}")
    if with_lse:
        lse = res[1].cpu().double()
        lse = lse.transpose(1, 2) if q.dim() == 4 else lse.transpose(0, 1)   # like wlse
        rows = ~wlse.isnan()
        fin = torch.isfinite(wlse) & rows
        assert torch.equal(torch.isfinite(lse) & rows, fin)
        assert ((lse[fin] - wlse[fin]).abs() <= 2.0 ** -14 * wlse[fin].abs().clamp(min=1)).all()
    return got, want


SINK8 = torch.tensor([0.5, -1.0, 3.0, 0.0, -20.0, 1.5, 2.0, -0.25])


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_attn_multi_token_dtypes_and_cache_kinds(tmo, ref, dev, dtype, kv):
    """4-D q with 2, 4 (16 query columns of 4 heads x 4 tokens) and 5 (two column blocks)
    tokens per sequence, with and without a sink; sequence 1 holds one key, so its first
    tokens see none."""
    case = W.attn_case(dtype, 31, kv=kv, B=6, Hq=8, Hkv=2, D=128, BS=16, NB=96, max_ctx=250)
    for S in (2, 4, 5):
        q = W.attn_queries(dtype, 32 + S, B=6, Hq=8, D=128, S=S)
        run_attn_mq(tmo, ref, dev, case, q)
        run_attn_mq(tmo, ref, dev, case, q, sink=SINK8)


def test_attn_multi_token_windows_alibi_and_pages(tmo, ref, dev):
    case = W.attn_case(torch.bfloat16, 33, kv="int8_token", B=5, Hq=8, Hkv=2, D=128, NB=80,
                       max_ctx=200, alibi=True)
    case.block_tables[0, 3] = -1
    case.block_tables[2, 0] = 10 ** 6
    q = W.attn_queries(torch.bfloat16, 34, B=5, Hq=8, D=128, S=4)
    for window in (-1, 0, 1, 17, 150):
        run_attn_mq(tmo, ref, dev, case, q, window=window, sink=SINK8 if window == 17 else None)
    case.alibi = None
    run_attn_mq(tmo, ref, dev, case, q, with_lse=False)
    run_attn_mq(tmo, ref, dev, case, q, max_ctx=0)


@pytest.mark.parametrize("max_seq_q", [-1, 16, 40])
def test_attn_multi_token_cu_seq_q(tmo, ref, dev, max_seq_q):
    """3-D q with cu_seq_q: ragged counts (an empty sequence, one of 16 tokens), max_seq_q
    unknown, exact or loose, two trailing rows of no sequence."""
    counts = [3, 0, 7, 1, 16, 2]
    case = W.attn_case(torch.bfloat16, 35, kv="int8_token", B=6, Hq=8, Hkv=2, D=128, NB=96,
                       max_ctx=230, alibi=True)
    q, cu = W.attn_queries(torch.bfloat16, 36, B=6, Hq=8, D=128, counts=counts)
    q = torch.cat([q, q[:2]])
    run_attn_mq(tmo, ref, dev, case, q, cu=cu, max_seq_q=max_seq_q, sink=SINK8)
    run_attn_mq(tmo, ref, dev, case, q, cu=cu, max_seq_q=max_seq_q, window=20)


@pytest.mark.parametrize("Hq,Hkv,D,S", [(16, 1, 128, 3), (40, 2, 128, 2), (8, 8, 64, 6),
                                        (8, 2, 96, 3), (8, 2, 256, 4)])
def test_attn_multi_token_groups_and_head_sizes(tmo, ref, dev, Hq, Hkv, D, S):
    """Query columns over several blocks (16 x 3 = 48, 20 x 2 = 40), one head per group,
    the generic kernel (head size 96) and head size 256."""
    case = W.attn_case(torch.bfloat16, 37 + Hq + D, kv="int8_token", B=3, Hq=Hq, Hkv=Hkv, D=D,
                       NB=48, max_ctx=120)
    q = W.attn_queries(torch.bfloat16, 38 + S, B=3, Hq=Hq, D=D, S=S)
    sink = torch.linspace(-2.0, 2.0, Hq)
    run_attn_mq(tmo, ref, dev, case, q, scale=1.0 / math.sqrt(D), sink=sink)


@pytest.mark.parametrize("kv", ["int8_token", "plain"])
def test_attn_multi_token_long_contexts_over_splits(tmo, ref, dev, kv):
    case = W.attn_case(torch.bfloat16, 39, kv=kv, B=2, Hq=8, Hkv=2, D=128, BS=16, NB=1100,
                       max_ctx=8000)
    case.context_lens[1] = 4097
    q = W.attn_queries(torch.bfloat16, 40, B=2, Hq=8, D=128, S=4)
    run_attn_mq(tmo, ref, dev, case, q, sink=SINK8)
    run_attn_mq(tmo, ref, dev, case, q, window=3000)
    q3, cu = W.attn_queries(torch.bfloat16, 41, B=2, Hq=8, D=128, counts=[5, 2])
    run_attn_mq(tmo, ref, dev, case, q3, cu=cu, max_ctx=1000)


def test_attn_multi_token_on_configs4_pages(tmo, ref, dev):
    """configs[4]'s page layout with 32 query heads and 4 query tokens per sequence (a
    speculative-decode verification step), with a sink, on the same 6-sequence sample as the
    decode test."""
    layout = W.cfg5()
    sel = torch.tensor([0, 1, 7, 20, 41, 63])
    ctx = layout.context_lengths[sel].contiguous()
    bt = layout.block_tables[sel].contiguous()
    used = [bt[i, :(c + 15) // 16] for i, c in enumerate(ctx.tolist())]
    pages = torch.unique(torch.cat(used))
    bt2 = torch.full_like(bt, -1)
    for i, u in enumerate(used):
        bt2[i, :u.numel()] = torch.searchsorted(pages, u).to(torch.int32)
    g = torch.Generator().manual_seed(6)
    NB = pages.numel()
    kc = torch.randint(-127, 128, (NB, 8, 16, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (NB, 8, 16, 128), generator=g, dtype=torch.int8)
    ks = 0.005 + 0.02 * torch.rand(NB, 8, 16, generator=g)
    vs = 0.005 + 0.02 * torch.rand(NB, 8, 16, generator=g)
    q = torch.randn(len(sel), 4, 32, 128, generator=g).to(torch.bfloat16)
    case = W.AttnCase(q[:, 0], kc, vc, ks, vs, bt2, ctx)
    run_attn_mq(tmo, ref, dev, case, q, sink=torch.linspace(-1.0, 3.0, 32))
