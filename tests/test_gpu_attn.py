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
same bar against the oracle's cached_kv_attn, with rows of no sequence left untouched; so are
the other cache forms: K and V in one cache (v_cache None, value head size below, equal to or
above the key's, a 576 / 512 latent-cache shape), value head sizes other than the key's,
per-group scales and per-token scales with strides in their first two dims; and so are int4
pair caches (V pairing rows or channels) and masks (terms for the last mask_len keys, decision
D16 of oracle/tmo_oracle.c) on the MFMA and generic kernels, over splits.
"""
import math

import pytest
import torch

from tests import workloads as W

pytestmark = pytest.mark.gpu

RTOL = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -16}
ATOL = {torch.bfloat16: 2.0 ** -14, torch.float16: 2.0 ** -14, torch.float32: 2.0 ** -16}


def _vmax(case, vs, Dv=None):
    """The largest |v| entry: the first Dv channels of the V cache (of the K cache when the
    case has none), dequantised (int4 pairs unpacked first)."""
    v = (case.k_cache if case.v_cache is None else case.v_cache)
    if case.int4:
        v = W.unpack_int4(v, 2 if 2 * v.shape[2] == case.k_cache.shape[2] else 3)
    v = v.double()
    if Dv is not None:
        v = v[..., :Dv]
    if vs is not None:
        if vs.dim() == 4 and vs.shape[3] == 1:
            vs = vs[..., 0]
        if vs.dim() == 3:
            v = v * vs.double()[..., None]
        elif vs.dim() == 2:
            v = v * vs.double()[None, :, None, :]
        elif vs.dim() == 4:                           # per group of 32 rows
            v = v * vs.double().repeat_interleave(32, dim=2)
        else:
            v = v * float(vs)
    return float(v.abs().max())


def run_attn(tmo, ref, dev, case, scale=0.0883883, window=-1, four_d=True, with_lse=True,
             bit=None, per_tensor=False, max_ctx=None):
    q = case.q
    kbit = 8 if case.k_cache.dtype in (torch.int8, torch.float8_e4m3fn) else -1
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


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kv", ["fp8_token", "fp8_channel", "fp8_group", "int8_token",
                                "int8_channel"])
@pytest.mark.parametrize("D", [64, 128, 256, 96])
def test_attn_fp8_pages_and_bf16_scales(tmo, ref, dev, D, kv, scale_dtype):
    """float8_e4m3fn pages (_ops.py:868; kv_cache_quant_bit_size 8) and bf16 scale tensors
    (_ops.py:872), on the MFMA kernels (head sizes 64 / 128 / 256, per-token and per-channel
    scales) and the VALU kernel (per-group scales, head size 96), against the float64 oracle
    at the stated tolerance."""
    if kv.endswith("group") and D % 32:
        pytest.skip("per-group scales need head_size % 32 == 0")
    case = W.attn_case(torch.bfloat16, 41 + D, kv=kv, B=5, Hq=8, Hkv=2, D=D, BS=32, NB=64,
                       max_ctx=300, scale_dtype=scale_dtype)
    case.block_tables[3, 2] = -1                          # a missing page
    # the oracle's general entry (per-group scales included), one query token per sequence
    run_attn_mq(tmo, ref, dev, case, case.q, scale=1.0 / math.sqrt(D))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attn_fp8_pages_multi_token_and_splits(tmo, ref, dev, dtype):
    """fp8 pages with several query tokens per sequence (cu_seq_q), a sink and contexts long
    enough for several splits."""
    case = W.attn_case(dtype, 45, kv="fp8_token", B=4, Hq=16, Hkv=2, D=128, BS=16, NB=700,
                       max_ctx=2500, scale_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(46)
    nq = torch.tensor([1, 3, 4, 2], dtype=torch.int32)
    cu = torch.cat((torch.zeros(1, dtype=torch.int32), nq.cumsum(0).to(torch.int32)))
    q = torch.randn(int(nq.sum()), 16, 128, generator=g).to(dtype)
    sink = torch.randn(16, generator=g)
    run_attn_mq(tmo, ref, dev, case, q, cu=cu, sink=sink)


def test_attn_decode_on_configs4_fp8_pages(tmo, ref, dev):
    """configs[4]'s page layout with float8_e4m3fn pages written by this build's own
    quant_to_paged_cache (fp8 branch: scale = amax / 448 per token and head) from bf16 K/V,
    read by the attention with 32 query heads, on a sample of 6 sequences against the oracle."""
    layout = W.cfg5()
    sel = torch.tensor([0, 1, 7, 20, 41, 63])
    ctx = layout.context_lengths[sel].contiguous()
    bt = layout.block_tables[sel].contiguous()
    used = [bt[i, :(c + 15) // 16] for i, c in enumerate(ctx.tolist())]
    pages = torch.unique(torch.cat(used))
    bt2 = torch.full_like(bt, -1)
    for i, u in enumerate(used):
        bt2[i, :u.numel()] = torch.searchsorted(pages, u).to(torch.int32)
    NB = pages.numel()
    sub = W.DequantLayout("cfg5_sample", ctx, bt2, NB, 16)
    kc, vc, ks, vs = W.cfg5_fill(sub, dev, seed=77, cache_dtype=torch.float8_e4m3fn)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(len(sel), 32, 128, generator=g).to(torch.bfloat16)
    case = W.AttnCase(q, kc.cpu(), vc.cpu(), ks.cpu(), vs.cpu(), bt2, ctx)
    run_attn(tmo, ref, dev, case)


@pytest.mark.parametrize("kv", ["int8_token", "plain"])
def test_attn_empty_cache(tmo, dev, kv):
    """num_blocks 0 with positive context lengths: every block-table entry lies outside the
    (zero-size) cache, so every key is masked -- D12's empty window, output 0 and lse -inf.
    The shape is one the MFMA kernel takes for a non-empty cache; it must not read the cache."""
    B, Hq, Hkv, D, BS = 3, 8, 2, 128, 16
    int8 = kv == "int8_token"
    cdt = torch.int8 if int8 else torch.bfloat16
    q = torch.randn(B, 1, Hq, D, device=dev).to(torch.bfloat16)
    kc = torch.empty(0, Hkv, BS, D, dtype=cdt, device=dev)
    vc = torch.empty(0, Hkv, BS, D, dtype=cdt, device=dev)
    ks = torch.empty(0, Hkv, BS, device=dev) if int8 else None
    vs = torch.empty(0, Hkv, BS, device=dev) if int8 else None
    bt = torch.tensor([[0, 1, 2, 3], [5, -1, 0, 2], [1, 1, 1, 1]], dtype=torch.int32, device=dev)
    lens = torch.tensor([50, 17, 64], dtype=torch.int32, device=dev)
    out = torch.full_like(q, 7.0)
    res, lse = tmo.single_query_cached_kv_attn(q, kc, vc, out, bt, lens, ks, vs, None, 64, -1,
                                               -1, 0.088, return_lse=True,
                                               kv_cache_quant_bit_size=8 if int8 else -1)
    torch.cuda.synchronize()
    assert res is out
    assert bool((out == 0).all())
    assert bool(torch.isneginf(lse).all())


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
                max_seq_q=-1, max_ctx=None, with_lse=True, Dv=None, mask=None,
                compute_dtype=torch.float32, q_scale=None, out_dtype=None, kbit=None,
                ref_scales=None):
    """Several query tokens per sequence: q [B, S, Hq, D] or [T, Hq, D] with cu.  The output
    ([..., Dv], Dv the V cache's head size or q's by default) starts as a sentinel, which rows
    of no sequence must keep.  case.v_cache None: K and V in one cache.  case.int4: int4-pair
    caches (kv_cache_quant_bit_size 4).  mask [B, S, mask_len] in compute_dtype.  q_scale:
    int8 / float8_e4m3fn q codes' scales, the output in out_dtype (half by default).  kbit
    overrides the cache bit size (-1 with code caches of q's dtype: ref_scales are the unit
    scales the oracle reads them with).  case.block_tables may be [B, heads, max_blocks]."""
    kb = kbit
    kbit = 8 if case.k_cache.dtype in (torch.int8, torch.float8_e4m3fn) else -1
    if kb is not None:
        kbit = kb
    odt = out_dtype or (torch.float16 if q_scale is not None else q.dtype)
    if case.int4:
        kbit = 4
        v_ch = case.v_cache.shape[2] == case.k_cache.shape[2]
        Dv = Dv or case.v_cache.shape[-1] * (2 if v_ch else 1)
    Dv = Dv or (case.v_cache.shape[-1] if case.v_cache is not None else q.shape[-1])
    cpu = lambda t: t.cpu() if t is not None else None            # noqa: E731
    on_dev = lambda t: t if t is None or t.is_cuda else t.to(dev)  # noqa: E731  (views kept)
    ks, vs = cpu(case.k_scale), cpu(case.v_scale)
    rks, rvs = ref_scales if ref_scales is not None else (ks, vs)
    want, wlse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                    case.context_lens, scale, rks, rvs, case.alibi, window,
                                    cu_seq_q=cu, sink=sink, head_size_v=Dv, int4=case.int4,
                                    mask=mask, q_scale=q_scale)
    out = torch.full(q.shape[:-1] + (Dv,), 7.0, dtype=odt, device=dev)
    res = tmo.single_query_cached_kv_attn(
        q.to(dev), case.k_cache.to(dev),
        case.v_cache.to(dev) if case.v_cache is not None else None, out,
        case.block_tables.to(dev), case.context_lens.to(dev), on_dev(case.k_scale),
        on_dev(case.v_scale),
        case.alibi.to(dev) if case.alibi is not None else None,
        case.max_context_len if max_ctx is None else max_ctx, window, -1, scale,
        return_lse=with_lse, kv_cache_quant_bit_size=kbit, compute_dtype=compute_dtype,
        mask=mask.to(dev) if mask is not None else None,
        cu_seq_q=cu.to(dev) if cu is not None else None, max_seq_q=max_seq_q,
        sink=sink.to(dev) if sink is not None else None,
        q_quant_scale=q_scale.to(dev) if q_scale is not None else None, out_dtype=odt)
    torch.cuda.synchronize()
    got = out.cpu().double()
    held = ~want.isnan()
    assert (got[~held] == 7.0).all(), "a row of no sequence was written"
    vmax = _vmax(case, rvs, Dv)
    err = (got - want).abs()
    lim = RTOL[odt] * want.abs() + ATOL[odt] * vmax
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


def _one_cache(case, D, Dv, seed):
    """K and V in one cache of max(D, Dv) channels (_ops.py:828-831): the case's K cache widened
    with random channels; values are the first Dv channels of each row."""
    g = torch.Generator().manual_seed(seed)
    NB, Hkv, BS, Dk = case.k_cache.shape
    Wd = max(D, Dv)
    if case.k_cache.dtype == torch.int8:
        extra = torch.randint(-127, 128, (NB, Hkv, BS, Wd - Dk), generator=g, dtype=torch.int8)
    else:
        extra = torch.randn(NB, Hkv, BS, Wd - Dk, generator=g).to(case.k_cache.dtype)
    kc = torch.cat([case.k_cache, extra], dim=-1) if Wd > Dk else case.k_cache
    return W.AttnCase(case.q, kc, None, case.k_scale, case.v_scale, case.block_tables,
                      case.context_lens, case.alibi)


@pytest.mark.parametrize("kv", ["int8_token", "plain"])
@pytest.mark.parametrize("Dv", [128, 64, 192])
def test_attn_one_kv_cache(tmo, ref, dev, kv, Dv):
    """v_cache None: equal head sizes run the MFMA kernel on the one cache, others the VALU
    kernel."""
    case = W.attn_case(torch.bfloat16, 61, kv=kv, B=4, Hq=8, Hkv=2, D=128, NB=64, max_ctx=200)
    one = _one_cache(case, 128, Dv, 62)
    q = W.attn_queries(torch.bfloat16, 63, B=4, Hq=8, D=128, S=2)
    run_attn_mq(tmo, ref, dev, one, q, Dv=Dv, sink=SINK8)
    run_attn_mq(tmo, ref, dev, one, q[:, :1], Dv=Dv)


def test_attn_latent_cache_shape(tmo, ref, dev):
    """A latent-cache shape: one KV head of 576 channels holding 512-channel values, 16 query
    heads, two query tokens (VALU kernel)."""
    case = W.attn_case(torch.bfloat16, 64, kv="plain", B=2, Hq=16, Hkv=1, D=576, NB=24,
                       max_ctx=150)
    one = W.AttnCase(case.q, case.k_cache, None, None, None, case.block_tables,
                     case.context_lens)
    q = W.attn_queries(torch.bfloat16, 65, B=2, Hq=16, D=576, S=2)
    run_attn_mq(tmo, ref, dev, one, q, scale=576 ** -0.5, Dv=512)


def test_attn_value_head_size(tmo, ref, dev):
    case = W.attn_case(torch.float16, 66, kv="int8_token", B=3, Hq=8, Hkv=2, D=128, NB=48,
                       max_ctx=150)
    case.v_cache = case.v_cache[..., :64].contiguous()
    q = W.attn_queries(torch.float16, 67, B=3, Hq=8, D=128, S=3)
    run_attn_mq(tmo, ref, dev, case, q)


@pytest.mark.parametrize("S", [1, 3])
def test_attn_group_scales(tmo, ref, dev, S):
    """Per-group scales: K one per token and 32 channels, V one per 32 rows and channel."""
    case = W.attn_case(torch.bfloat16, 68, kv="int8_group", B=3, Hq=8, Hkv=2, D=128, BS=32,
                       NB=32, max_ctx=200, alibi=True)
    q = W.attn_queries(torch.bfloat16, 69, B=3, Hq=8, D=128, S=S)
    run_attn_mq(tmo, ref, dev, case, q, sink=SINK8)


@pytest.mark.parametrize("pad", [4, 3])
def test_attn_strided_token_scales(tmo, ref, dev, pad):
    """Per-token scales as a view with strides in the first two dims (pages padded by `pad`
    scales, heads outermost): strides in multiples of four keep the MFMA kernel's vector
    loads, others take the VALU kernel; no copy either way."""
    case = W.attn_case(torch.bfloat16, 70, kv="int8_token", B=4, Hq=8, Hkv=2, D=128, NB=64,
                       max_ctx=200)
    NB, Hkv, BS = case.k_scale.shape
    views = []
    for sc in (case.k_scale, case.v_scale):
        big = torch.rand(Hkv, NB, BS + pad)
        big[:, :, :BS] = sc.transpose(0, 1)
        # the view is built on the device (a copy of a view to the device would be contiguous)
        views.append(big.to(dev).transpose(0, 1)[:, :, :BS])
    assert views[0].stride() == (BS + pad, NB * (BS + pad), 1)
    assert torch.equal(views[0].cpu(), case.k_scale)
    q = W.attn_queries(torch.bfloat16, 71, B=4, Hq=8, D=128, S=2)
    strided = W.AttnCase(case.q, case.k_cache, case.v_cache, *views, case.block_tables,
                         case.context_lens)
    run_attn_mq(tmo, ref, dev, strided, q)


# ---------------------------------------------------------------------------- int4 caches, mask

@pytest.mark.parametrize("v_pairs", ["rows", "channels"])
@pytest.mark.parametrize("kv", ["int4_token", "int4_channel", "int4_group"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attn_int4_caches(tmo, ref, dev, dtype, kv, v_pairs):
    """kv_cache_quant_bit_size 4: int8 caches of int4 pairs, K pairing channels, V pairing the
    rows of a page or channels; per-token / per-channel / per-group scales; one and several
    query tokens (4-D and cu_seq_q), a sink, a window, ALiBi and a missing page."""
    BS = 32 if kv == "int4_group" else 16
    case = W.attn_case(dtype, 91, kv=kv, B=5, Hq=8, Hkv=2, D=128, BS=BS, NB=64, max_ctx=180,
                       v_pairs=v_pairs)
    case.block_tables[2, 1] = -1
    for S in (1, 3):
        q = W.attn_queries(dtype, 92 + S, B=5, Hq=8, D=128, S=S)
        run_attn_mq(tmo, ref, dev, case, q, sink=SINK8 if S == 3 else None)
    q3, cu = W.attn_queries(dtype, 96, B=5, Hq=8, D=128, counts=[4, 1, 0, 2, 6])
    case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1)
    run_attn_mq(tmo, ref, dev, case, q3, cu=cu, window=40)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("kv,sdt", [("int4_token", torch.float32), ("int4_channel", torch.bfloat16),
                                    ("int4_token", torch.bfloat16)])
def test_attn_int4_mfma_head_sizes(tmo, ref, dev, D, kv, sdt):
    """int4 pages (V pairing rows) of head sizes 64 and 256 on the MFMA kernel, per-token or
    per-channel scales in float32 or bfloat16, one and three query tokens."""
    case = W.attn_case(torch.bfloat16, 120 + D, kv=kv, B=4, Hq=8, Hkv=2, D=D, NB=64,
                       max_ctx=150, scale_dtype=sdt)
    for S in (1, 3):
        q = W.attn_queries(torch.bfloat16, 121 + S, B=4, Hq=8, D=D, S=S)
        run_attn_mq(tmo, ref, dev, case, q, sink=SINK8 if S == 3 else None)


def test_attn_decode_on_configs4_int4_pages(tmo, ref, dev):
    """configs[4]'s page layout with int4 pages (K pairing channels, V pairing rows, per-token
    fp32 scales), 32 query heads, on a sample of 6 sequences against the oracle."""
    layout = W.cfg5()
    sel = torch.tensor([0, 1, 7, 20, 41, 63])
    ctx = layout.context_lengths[sel].contiguous()
    bt = layout.block_tables[sel].contiguous()
    used = [bt[i, :(c + 15) // 16] for i, c in enumerate(ctx.tolist())]
    pages = torch.unique(torch.cat(used))
    bt2 = torch.full_like(bt, -1)
    for i, u in enumerate(used):
        bt2[i, :u.numel()] = torch.searchsorted(pages, u).to(torch.int32)
    g = torch.Generator().manual_seed(8)
    NB = pages.numel()
    kc = W.pack_int4(torch.randint(-8, 8, (NB, 8, 16, 128), generator=g, dtype=torch.int8), 3)
    vc = W.pack_int4(torch.randint(-8, 8, (NB, 8, 16, 128), generator=g, dtype=torch.int8), 2)
    ks = 0.05 + 0.25 * torch.rand(NB, 8, 16, generator=g)
    vs = 0.05 + 0.25 * torch.rand(NB, 8, 16, generator=g)
    q = torch.randn(len(sel), 1, 32, 128, generator=g).to(torch.bfloat16)
    case = W.AttnCase(q[:, 0], kc, vc, ks, vs, bt2, ctx, int4=True)
    run_attn_mq(tmo, ref, dev, case, q)


def test_attn_int4_long_contexts(tmo, ref, dev):
    """int4 pages over a few thousand keys, 32 query heads over 8 KV heads, with splits."""
    case = W.attn_case(torch.bfloat16, 97, kv="int4_token", B=3, Hq=32, Hkv=8, D=128, BS=16,
                       NB=800, max_ctx=4000)
    q = W.attn_queries(torch.bfloat16, 98, B=3, Hq=32, D=128, S=1)
    run_attn_mq(tmo, ref, dev, case, q)


def _mask(seed, B, S, ml, dtype, neg_inf_every=7):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, ml, generator=g) * 2
    m.view(-1)[::neg_inf_every] = float("-inf")
    return m.to(dtype)


@pytest.mark.parametrize("D", [128, 64, 96])
@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain", "fp8_token"])
def test_attn_mask(tmo, ref, dev, kv, D):
    """mask [batch, seq_q, mask_len] in compute_dtype: float32, bfloat16 and float16 terms for
    the last mask_len keys, -inf entries removing keys; the MFMA kernels (D 64 / 128) and the
    generic one (D 96); 4-D q and cu_seq_q, with a sink, a window and ALiBi."""
    dtype = torch.bfloat16
    case = W.attn_case(dtype, 101, kv=kv, B=5, Hq=8, Hkv=2, D=D, NB=64, max_ctx=180)
    case.block_tables[3, 0] = -1
    q4 = W.attn_queries(dtype, 102, B=5, Hq=8, D=D, S=4)
    for ml, cdt in ((4, torch.float32), (16, torch.bfloat16), (64, torch.float16)):
        mask = _mask(103 + ml, 5, 4, ml, cdt)
        run_attn_mq(tmo, ref, dev, case, q4, mask=mask, compute_dtype=cdt,
                    sink=SINK8 if ml == 16 else None)
    q3, cu = W.attn_queries(dtype, 104, B=5, Hq=8, D=D, counts=[2, 1, 0, 2, 2])
    case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1)
    mask = _mask(105, 5, 2, 8, torch.float32)
    run_attn_mq(tmo, ref, dev, case, q3, cu=cu, max_seq_q=2, mask=mask, window=30)


def test_attn_mask_over_splits_and_int4(tmo, ref, dev):
    """A mask over the last 64 keys of contexts long enough to be split over several
    workgroups (the mask terms land in the last split), and a mask on int4 pages."""
    case = W.attn_case(torch.float16, 106, kv="int8_token", B=3, Hq=32, Hkv=8, D=128, BS=16,
                       NB=800, max_ctx=4000)
    q = W.attn_queries(torch.float16, 107, B=3, Hq=32, D=128, S=2)
    run_attn_mq(tmo, ref, dev, case, q, mask=_mask(108, 3, 2, 64, torch.float16),
                compute_dtype=torch.float16)
    c4 = W.attn_case(torch.bfloat16, 109, kv="int4_channel", B=4, Hq=8, Hkv=2, D=128,
                     max_ctx=100)
    q = W.attn_queries(torch.bfloat16, 110, B=4, Hq=8, D=128, S=2)
    run_attn_mq(tmo, ref, dev, c4, q, mask=_mask(111, 4, 2, 32, torch.float32))


def test_attn_mask_and_int4_rejections(tmo, dev):
    """The reference's stated limits raise: mask_len above 64 or not a multiple of seq_q, a
    mask dtype other than compute_dtype, float32 q with a mask; int4 caches of the wrong
    shapes."""
    case = W.attn_case(torch.bfloat16, 112, kv="int8_token", B=2, Hq=4, Hkv=2, D=64, max_ctx=40)
    q = W.attn_queries(torch.bfloat16, 113, B=2, Hq=4, D=64, S=2).to(dev)
    args = lambda c: (c.k_cache.to(dev), c.v_cache.to(dev), None, c.block_tables.to(dev),  # noqa: E731
                      c.context_lens.to(dev), c.k_scale.to(dev), c.v_scale.to(dev), None, 40,
                      -1, -1, 0.1)
    for m, cdt in ((torch.zeros(2, 2, 66), torch.float32), (torch.zeros(2, 2, 3), torch.float32),
                   (torch.zeros(2, 2, 8), torch.bfloat16), (torch.zeros(2, 3, 8), torch.float32)):
        with pytest.raises(RuntimeError):
            tmo.single_query_cached_kv_attn(q, *args(case), kv_cache_quant_bit_size=8,
                                            mask=m.to(dev), compute_dtype=cdt)
    with pytest.raises(RuntimeError):
        tmo.single_query_cached_kv_attn(q.float(), *args(case), kv_cache_quant_bit_size=8,
                                        mask=torch.zeros(2, 2, 8, device=dev))
    c4 = W.attn_case(torch.bfloat16, 114, kv="int4_token", B=2, Hq=4, Hkv=2, D=64, max_ctx=40)
    with pytest.raises(RuntimeError):                # int8-shaped pages read as int4
        tmo.single_query_cached_kv_attn(q, *args(case), kv_cache_quant_bit_size=4)
    bad = W.AttnCase(c4.q, c4.k_cache, c4.v_cache[:, :, :4].contiguous(), c4.k_scale,
                     c4.v_scale, c4.block_tables, c4.context_lens, int4=True)
    with pytest.raises(RuntimeError):                # V neither row nor channel pairs
        tmo.single_query_cached_kv_attn(q, *args(bad), kv_cache_quant_bit_size=4)


# ---------------------------------------------------------------------------- quantised q, sparse-KV tables

def _q_codes(dtype, shape, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.int8:
        return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)
    return W.fp8_codes(shape, g)


def _q_scale(form, lead, seed, dtype=torch.float32, groups=4):
    g = torch.Generator().manual_seed(seed)
    if form == "tensor":
        return torch.tensor([0.0123]).to(dtype)
    if form == "token":
        return (0.002 + 0.02 * torch.rand(lead, generator=g)).to(dtype)
    return (0.002 + 0.02 * torch.rand(tuple(lead) + (groups,), generator=g)).to(dtype)


@pytest.mark.parametrize("kv,D", [("int8_token", 128), ("int8_token", 96), ("int8_channel", 128),
                                  ("int8_channel", 96), ("fp8_token", 128), ("fp8_token", 96),
                                  ("int4_token", 128)])
@pytest.mark.parametrize("form", ["tensor", "token", "group"])
@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_attn_quantised_q(tmo, ref, dev, qdt, form, kv, D):
    """int8 / float8_e4m3fn q with q_quant_scale per tensor, per token and head, or per channel
    group (float32 and bfloat16 scales), over int8 / fp8 / int4 pages, on the MFMA (128) and
    generic (96) kernels; 4-D q and cu_seq_q; the output in half (bfloat16 too for int8 q)."""
    case = W.attn_case(torch.bfloat16, 140, kv=kv, B=5, Hq=8, Hkv=2, D=D, NB=64, max_ctx=150)
    q4 = _q_codes(qdt, (5, 2, 8, D), 141)
    qs4 = _q_scale(form, (5, 2, 8), 142, torch.bfloat16 if form == "token" else torch.float32)
    run_attn_mq(tmo, ref, dev, case, q4, q_scale=qs4, sink=SINK8)
    q3 = _q_codes(qdt, (9, 8, D), 143)
    cu = torch.tensor([0, 3, 4, 4, 8, 9], dtype=torch.int32)
    qs3 = _q_scale(form, (9, 8), 144)
    odt = torch.bfloat16 if qdt == torch.int8 else torch.float16
    run_attn_mq(tmo, ref, dev, case, q3, cu=cu, q_scale=qs3, out_dtype=odt, window=50)


def test_attn_quantised_q_long_contexts(tmo, ref, dev):
    """int8 q with per-token scales over a few thousand int8 keys, split over workgroups."""
    case = W.attn_case(torch.bfloat16, 145, kv="int8_token", B=3, Hq=32, Hkv=8, D=128, BS=16,
                       NB=800, max_ctx=4000)
    q = _q_codes(torch.int8, (3, 1, 32, 128), 146)
    run_attn_mq(tmo, ref, dev, case, q, q_scale=_q_scale("token", (3, 1, 32), 147))


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
def test_attn_quantised_q_same_as_q_caches(tmo, ref, dev, qdt):
    """kv_cache_quant_bit_size -1 with caches of q's dtype (int8 / float8_e4m3fn codes, no cache
    scales): the codes read as they are, i.e. with unit scales."""
    case = W.attn_case(torch.bfloat16, 148, kv="int8_token" if qdt == torch.int8 else "fp8_token",
                       B=4, Hq=8, Hkv=2, D=128, NB=64, max_ctx=120)
    if qdt == torch.int8:   # small codes keep the unit-scale logits in range
        case.k_cache = (case.k_cache // 16).contiguous()
    ones = (torch.ones(2, 128), torch.ones(2, 128))
    case.k_scale = case.v_scale = None
    q = _q_codes(qdt, (4, 1, 8, 128), 149)
    run_attn_mq(tmo, ref, dev, case, q, q_scale=torch.tensor([0.002]), kbit=-1, ref_scales=ones)


def _sparse_tables(case, per, seed):
    g = torch.Generator().manual_seed(seed)
    bt = case.block_tables
    rows = [bt]
    for _ in range(per - 1):
        rows.append(bt.reshape(-1)[torch.randperm(bt.numel(), generator=g)].reshape(bt.shape))
    return torch.stack(rows, dim=1).contiguous()


@pytest.mark.parametrize("kv,D", [("int8_token", 128), ("int8_token", 96), ("plain", 128),
                                  ("plain", 96), ("int4_token", 128)])
@pytest.mark.parametrize("per", ["kv", "q"])
def test_attn_sparse_tables(tmo, ref, dev, kv, per, D):
    """block_tables [batch, kv_heads or heads, max_blocks]: each KV head's (or query head's)
    own pages; per-KV-head tables on the MFMA kernel, per-query-head tables with grouped heads
    and head size 96 on the generic one; a missing page; 4-D q and cu_seq_q."""
    case = W.attn_case(torch.bfloat16, 150, kv=kv, B=5, Hq=8, Hkv=2, D=D, NB=64, max_ctx=150)
    case.block_tables = _sparse_tables(case, 2 if per == "kv" else 8, 151)
    case.block_tables[2, 1, 1] = -1
    q = W.attn_queries(torch.bfloat16, 152, B=5, Hq=8, D=D, S=2)
    run_attn_mq(tmo, ref, dev, case, q, sink=SINK8)
    q3, cu = W.attn_queries(torch.bfloat16, 153, B=5, Hq=8, D=D, counts=[3, 1, 0, 2, 4])
    run_attn_mq(tmo, ref, dev, case, q3, cu=cu)


def test_attn_sparse_tables_over_splits(tmo, ref, dev):
    """Per-KV-head tables over a few thousand keys, 32 query heads, split over workgroups."""
    case = W.attn_case(torch.bfloat16, 154, kv="int8_token", B=3, Hq=32, Hkv=8, D=128, BS=16,
                       NB=800, max_ctx=4000)
    case.block_tables = _sparse_tables(case, 8, 155)
    q = W.attn_queries(torch.bfloat16, 156, B=3, Hq=32, D=128, S=1)
    run_attn_mq(tmo, ref, dev, case, q)


def test_attn_quantised_q_rejections(tmo, dev):
    """q_quant_scale needs an int8 / float8_e4m3fn q and the reverse; float8_e4m3fn q takes a
    half output; a float output needs a float dtype; block tables of another head count."""
    case = W.attn_case(torch.bfloat16, 157, kv="int8_token", B=2, Hq=4, Hkv=2, D=64, max_ctx=40)
    kc, vc = case.k_cache.to(dev), case.v_cache.to(dev)
    bt, lens = case.block_tables.to(dev), case.context_lens.to(dev)
    ks, vs = case.k_scale.to(dev), case.v_scale.to(dev)
    qb = torch.randn(2, 1, 4, 64, device=dev).to(torch.bfloat16)
    qi = torch.randint(-5, 5, (2, 1, 4, 64), device=dev, dtype=torch.int8)
    qf = qi.to(torch.float8_e4m3fn)
    s1 = torch.tensor([0.01], device=dev)
    def call(q, out_dtype, qs, bt_=bt):
        out = torch.empty(q.shape, dtype=out_dtype, device=dev)
        return tmo.single_query_cached_kv_attn(q, kc, vc, out, bt_, lens, ks, vs, None, 40, -1, -1,
                                               0.1, kv_cache_quant_bit_size=8, q_quant_scale=qs)
    call(qi, torch.float16, s1)                                      # accepted
    for q, odt, qs in ((qb, torch.bfloat16, s1), (qi, torch.float16, None),
                       (qf, torch.bfloat16, s1), (qi, torch.int8, s1)):
        with pytest.raises(RuntimeError):
            call(q, odt, qs)
    with pytest.raises(RuntimeError):
        call(qb, torch.bfloat16, None, bt[:, None].expand(2, 3, -1).contiguous())
