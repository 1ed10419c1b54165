"""GPU parity of the linear-cache siblings (reshape_linear_cache, quant_to_linear_cache,
offline_quant_to_linear_cache, dequant_from_linear_cache, reshape_from_cache) against the CPU
oracle, through the public wrappers -> torch_mlu_ops ops -> C ABI.

Bar: bit-exact on whole tensors (codes, fp8 bytes, fp32 scales, copied bytes, dequantised
outputs), including the sentinel bytes a call must not write.  Cases: packed and padded input,
sequence / cache offsets with a negative cache batch id and a sequence running past the cache
end, empty sequences, max_context_len truncation, every vector lane-group width, the generic
(unaligned / odd head_size) kernels, strided K/V views, group-wise scales, and a prefill-sized
shape checked by round-trip properties.
"""
import pytest
import torch

from tests import workloads as W
from tests.test_gpu_parity import assert_bits_equal

pytestmark = pytest.mark.gpu

FLOATS = [torch.bfloat16, torch.float16, torch.float32]


def _d(t, dev):
    return None if t is None else t.to(dev)


def _cmp(got, want, what):
    if want.dtype == torch.float8_e4m3fn:
        got, want = got.view(torch.uint8), want.view(torch.uint8)
    assert_bits_equal(got, want, what)


# ---------------------------------------------------------------------------- reshape_linear_cache

def _reshape_both(tmo, ref, dev, case, dtype, max_len=None, with_v=True):
    max_len = case.max_context_len if max_len is None else max_len
    kc, vc = case.caches(dtype)
    v = case.value if with_v else None
    if not with_v:
        vc = None
    ref.linear_cache(0, case.key, v, kc, vc, case.context_lengths, max_len, packed=case.packed,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset)
    gk, gv = (t.to(dev) for t in case.caches(dtype))
    if not with_v:
        gv = None
    out = tmo.reshape_linear_cache(case.key.to(dev), _d(v, dev), gk, gv,
                                   case.context_lengths.to(dev), max_len, case.packed,
                                   _d(case.context_seq_offset, dev), _d(case.cache_bs_id, dev),
                                   _d(case.cache_seq_offset, dev))
    assert (out[0] if with_v else out) is gk
    torch.cuda.synchronize()
    _cmp(gk, kc, "key_cache")
    if with_v:
        _cmp(gv, vc, "value_cache")


def _typed(case, dtype):
    if dtype == torch.int8:
        case.key = case.key.to(torch.float32).mul(40).clamp(-127, 127).to(torch.int8)
        case.value = case.value.to(torch.float32).mul(40).clamp(-127, 127).to(torch.int8)
    else:
        case.key, case.value = case.key.to(dtype), case.value.to(dtype)
    return case


@pytest.mark.parametrize("packed,offsets", [(True, False), (True, True), (False, False),
                                            (False, True)])
@pytest.mark.parametrize("dtype", FLOATS + [torch.int8])
def test_reshape_linear_cache(tmo, ref, dev, dtype, packed, offsets):
    case = _typed(W.linear_case(torch.float32, 31, packed=packed, offsets=offsets), dtype)
    _reshape_both(tmo, ref, dev, case, dtype)


@pytest.mark.parametrize("D", [8, 16, 32, 64, 256, 512, 72, 20, 3])
def test_reshape_linear_cache_head_sizes(tmo, ref, dev, D):
    """Every copy lane-group width (16 bytes per lane) and the generic byte path."""
    case = W.linear_case(torch.bfloat16, 32, packed=True, offsets=True, D=D)
    _reshape_both(tmo, ref, dev, case, torch.bfloat16)
    _reshape_both(tmo, ref, dev, case, torch.bfloat16, with_v=False)


def test_reshape_linear_cache_truncation_and_views(tmo, ref, dev):
    case = W.linear_case(torch.float16, 33, packed=True, offsets=True, H=4)
    _reshape_both(tmo, ref, dev, case, torch.float16, max_len=7)
    # K/V as strided views of a fused [T, 3H, D] tensor (head stride D, token stride 3HD)
    T, H, D = case.key.shape
    qkv = torch.randn(T, 3 * H, D, generator=torch.Generator().manual_seed(4)).to(torch.float16)
    case.key, case.value = qkv[:, H:2 * H], qkv[:, 2 * H:]
    _reshape_both(tmo, ref, dev, case, torch.float16)


# ---------------------------------------------------------------------------- token-major launches

@pytest.mark.parametrize("B", [5, 70])
def test_linear_write_ops_token_major_targets(tmo, ref, dev, B):
    """The write ops' token-major launches (packed input without context_seq_offset: rows found
    from the prefix offsets) with cache batch ids (one negative), cache position offsets (one
    running past the cache's end), a max_context_len shorter than some sequences, and more
    sequences than one wavefront holds (the lookup's second path)."""
    case = W.linear_case(torch.bfloat16, 61 + B, packed=True, offsets=True, B=B,
                         cache_batch=B + 3)
    case.context_seq_offset = None  # rows at the prefix offsets of the lengths
    print(f"[linear token-major] B={B}", flush=True)
    _reshape_both(tmo, ref, dev, case, torch.bfloat16)
    _reshape_both(tmo, ref, dev, case, torch.bfloat16, max_len=7)
    for cdt in (torch.int8, torch.float8_e4m3fn):
        _quant_both(tmo, ref, dev, case, cdt)
    _quant_both(tmo, ref, dev, case, torch.int8, groups=4)


# ---------------------------------------------------------------------------- quant_to_linear_cache

def _quant_both(tmo, ref, dev, case, cache_dtype, groups=0, with_v=True):
    kc, vc = case.caches(cache_dtype)
    ks, vs = case.scales(groups)
    v = case.value if with_v else None
    if not with_v:
        vc = vs = None
    ref.linear_cache(1, case.key, v, kc, vc, case.context_lengths, case.max_context_len,
                     packed=case.packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks, value_scale=vs, groups=max(groups, 1))
    gk, gv = (t.to(dev) for t in case.caches(cache_dtype))
    gks, gvs = (t.to(dev) for t in case.scales(groups))
    if not with_v:
        gv = gvs = None
    out = tmo.quant_to_linear_cache(case.key.to(dev), _d(v, dev), gk, gv, gks, gvs,
                                    case.context_lengths.to(dev), case.max_context_len,
                                    case.packed, _d(case.context_seq_offset, dev),
                                    _d(case.cache_bs_id, dev), _d(case.cache_seq_offset, dev))
    assert out[0] is gk
    torch.cuda.synchronize()
    _cmp(gk, kc, "key_cache")
    _cmp(gks, ks, "key_scale")
    if with_v:
        _cmp(gv, vc, "value_cache")
        _cmp(gvs, vs, "value_scale")


@pytest.mark.parametrize("packed,offsets", [(True, False), (True, True), (False, True)])
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("dtype", FLOATS)
def test_quant_to_linear_cache(tmo, ref, dev, dtype, cache_dtype, packed, offsets):
    case = W.linear_case(dtype, 41, packed=packed, offsets=offsets)
    _quant_both(tmo, ref, dev, case, cache_dtype)


@pytest.mark.parametrize("D,groups", [(128, 1), (128, 4), (128, 16), (64, 8), (512, 2),
                                      (256, 32), (8, 1), (72, 3), (72, 1), (20, 4), (96, 3)])
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
def test_quant_to_linear_cache_groups_and_widths(tmo, ref, dev, cache_dtype, D, groups):
    """Lane widths 1..64, group-wise scales (4-D scale tensor) down to one lane per group, and
    the generic kernel (head sizes that are not 8 x a power of two, groups that do not align
    with the lanes)."""
    case = W.linear_case(torch.bfloat16, 42 + D, packed=True, offsets=True, D=D)
    _quant_both(tmo, ref, dev, case, cache_dtype, groups=groups if groups > 1 else 0)
    _quant_both(tmo, ref, dev, case, cache_dtype, groups=groups, with_v=False)


def test_quant_to_linear_cache_extreme_rows(tmo, ref, dev):
    """Zero rows, tiny rows (scale below the reciprocal range: IEEE divides), huge rows."""
    for dtype in (torch.float32, torch.bfloat16):
        case = W.linear_case(dtype, 43, packed=True, offsets=False, S=12)
        k = case.key.to(torch.float32)
        k[0] = 0
        k[1] *= 1e-38
        k[3] = k[3] * 3e-44 if dtype == torch.float32 else k[3] * 1e-30
        k[4] *= 1e30
        case.key = k.to(dtype)
        for cdt in (torch.int8, torch.float8_e4m3fn):
            _quant_both(tmo, ref, dev, case, cdt)


def _with_signed_zeros(case):
    """Rows of both signs of zero among ordinary values: the IEEE quotient -0 / s is -0, the
    float8_e4m3fn byte 0x80 (int8 codes are 0 either way)."""
    k = case.key.clone()
    k[0::3, ..., ::2] = -0.0
    k[1::3, ..., 1::3] = 0.0
    k[2::7] = -0.0
    case.key = k
    return case


@pytest.mark.parametrize("dtype", FLOATS)
def test_linear_signed_zeros(tmo, ref, dev, dtype):
    case = _with_signed_zeros(W.linear_case(dtype, 44, packed=True, offsets=True, S=12))
    for cdt in (torch.int8, torch.float8_e4m3fn):
        _quant_both(tmo, ref, dev, case, cdt)
        _quant_both(tmo, ref, dev, case, cdt, groups=4)
    for mode in (0, 1, 2):
        _offline_both(tmo, ref, dev, case, torch.float8_e4m3fn, mode)


# ---------------------------------------------------------------------------- offline (static)

def _static_scales(H, D, L, smode, g):
    if smode == 0:
        return 0.005 + 0.2 * torch.rand(H, D, generator=g), 0.01 + 0.1 * torch.rand(H, D, generator=g)
    if smode == 1:
        return 0.005 + 0.2 * torch.rand(H, L, generator=g), 0.01 + 0.1 * torch.rand(H, L, generator=g)
    return 0.0371, 0.0523


def _offline_both(tmo, ref, dev, case, cache_dtype, quant_mode, with_v=True):
    g = torch.Generator().manual_seed(7)
    H, D = case.key.shape[-2:]
    smode = min(quant_mode, 2)
    ks, vs = _static_scales(H, D, case.cache_len, smode, g)
    kc, vc = case.caches(cache_dtype)
    v = case.value if with_v else None
    if not with_v:
        vc = None
    tensor = torch.is_tensor(ks)
    ref.linear_cache(2, case.key, v, kc, vc, case.context_lengths, case.max_context_len,
                     packed=case.packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_chan=ks if tensor else None, value_chan=vs if tensor else None,
                     key_tensor=1.0 if tensor else ks, value_tensor=1.0 if tensor else vs,
                     smode=smode)
    gk, gv = (t.to(dev) for t in case.caches(cache_dtype))
    if not with_v:
        gv = None
    gks = ks.to(dev) if tensor else ks
    gvs = (vs.to(dev) if tensor else vs) if with_v else None
    out = tmo.offline_quant_to_linear_cache(case.key.to(dev), _d(v, dev), gk, gv, gks, gvs,
                                            case.context_lengths.to(dev), case.max_context_len,
                                            quant_mode, case.packed,
                                            _d(case.context_seq_offset, dev),
                                            _d(case.cache_bs_id, dev),
                                            _d(case.cache_seq_offset, dev))
    assert out[0] is gk
    torch.cuda.synchronize()
    _cmp(gk, kc, "key_cache")
    if with_v:
        _cmp(gv, vc, "value_cache")


@pytest.mark.parametrize("quant_mode", [0, 1, 2, 3])
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("dtype", FLOATS)
def test_offline_quant_to_linear_cache(tmo, ref, dev, dtype, cache_dtype, quant_mode):
    case = W.linear_case(dtype, 51, packed=True, offsets=True)
    _offline_both(tmo, ref, dev, case, cache_dtype, quant_mode)


@pytest.mark.parametrize("D", [8, 64, 512, 72, 20])
@pytest.mark.parametrize("packed", [True, False])
def test_offline_quant_to_linear_cache_widths(tmo, ref, dev, D, packed):
    case = W.linear_case(torch.float16, 52 + D, packed=packed, offsets=True, D=D)
    for mode in (0, 1, 2):
        _offline_both(tmo, ref, dev, case, torch.int8, mode)
    _offline_both(tmo, ref, dev, case, torch.float8_e4m3fn, 0, with_v=False)


# ---------------------------------------------------------------------------- dequant / copy out

def _filled(case, seed=61):
    g = torch.Generator().manual_seed(seed)
    H, D = case.key.shape[-2:]
    shape = (case.cache_batch, H, case.cache_len, D)
    kc = torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
    kt = torch.rand(shape[:3], generator=g) * 0.05
    vt = torch.rand(shape[:3], generator=g) * 0.05
    kt[0, 0, :3] = torch.tensor([0.0, 1e-38, 3e30])   # zero, subnormal-range and huge scales
    kch = torch.rand(H, D, generator=g) * 0.05
    vch = torch.rand(H, D, generator=g) * 0.05
    return kc, vc, kt, vt, kch, vch


def _dequant_both(tmo, ref, dev, case, dtype, mode, with_v=True, rows=None):
    kc, vc, kt, vt, kch, vch = _filled(case)
    ks, vs = (kch, vch) if mode == 0 else (kt, vt)
    H, D = case.key.shape[-2:]
    T = int(case.lens.sum()) + 3 if rows is None else rows
    if case.context_seq_offset is not None:
        T = max(T, int((case.context_seq_offset + case.lens).max()) + 1)
    key = torch.full((T, H, D), -3.0, dtype=dtype)
    value = key.clone() if with_v else None
    if not with_v:
        vc = vs = None
    ref.linear_cache(3, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks if mode == 1 else None, value_scale=vs if mode == 1 else None,
                     key_chan=ks if mode == 0 else None, value_chan=vs if mode == 0 else None,
                     smode=mode)
    gkey = torch.full((T, H, D), -3.0, dtype=dtype, device=dev)
    gval = gkey.clone() if with_v else None
    assert tmo.dequant_from_linear_cache(gkey, gval, kc.to(dev), _d(vc, dev), ks.to(dev),
                                         _d(vs, dev), case.lens.to(dev), case.max_context_len,
                                         _d(case.context_seq_offset, dev),
                                         _d(case.cache_bs_id, dev),
                                         _d(case.cache_seq_offset, dev), mode, 8) is None
    torch.cuda.synchronize()
    _cmp(gkey, key, "key")
    if with_v:
        _cmp(gval, value, "value")


@pytest.mark.parametrize("offsets", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", FLOATS)
def test_dequant_from_linear_cache(tmo, ref, dev, dtype, mode, offsets):
    case = W.linear_case(dtype, 62, packed=True, offsets=offsets)
    _dequant_both(tmo, ref, dev, case, dtype, mode)


@pytest.mark.parametrize("mode", [0, 1])
def test_dequant_from_linear_cache_direct_rows_edges(tmo, ref, dev, mode):
    """No cache offsets, batch ids or block tables (cache row (i, h, j) read before the length
    arrives): sequences longer than cache_len (positions past it are not written) and more
    sequences than cache batches (the extra ones write nothing)."""
    case = W.linear_case(torch.bfloat16, 405, packed=True, offsets=False, B=6, S=24)
    case.cache_len = 16
    case.cache_batch = 4
    assert int(case.lens.max()) > case.cache_len
    _dequant_both(tmo, ref, dev, case, torch.bfloat16, mode)
    _dequant_both(tmo, ref, dev, case, torch.float16, mode, with_v=False)


@pytest.mark.parametrize("D", [8, 16, 64, 256, 512, 72, 20])
def test_dequant_from_linear_cache_widths(tmo, ref, dev, D):
    case = W.linear_case(torch.bfloat16, 63 + D, packed=True, offsets=True, D=D)
    _dequant_both(tmo, ref, dev, case, torch.bfloat16, 1)
    _dequant_both(tmo, ref, dev, case, torch.float16, 0, with_v=False)


def _paged_view(case, NB_per=4):
    """Re-cut the case's cache geometry into pages: block_rows = cache_len // NB_per."""
    case.cache_len //= NB_per
    case.cache_batch *= NB_per
    return case


@pytest.mark.parametrize("mode", ["linear", "linear_table", "paged"])
@pytest.mark.parametrize("dtype", FLOATS + [torch.int8])
def test_reshape_from_cache(tmo, ref, dev, dtype, mode):
    case = W.linear_case(torch.float32, 71, packed=True, offsets=mode != "paged")
    bt = None
    if mode == "linear":
        case.cache_bs_id = None                       # sequence i reads cache batch i
    elif mode == "paged":
        case = _paged_view(case)
        g = torch.Generator().manual_seed(3)
        MB = (case.max_context_len + case.cache_len - 1) // case.cache_len
        bt = torch.randperm(case.cache_batch, generator=g)[:case.lens.numel() * MB]
        bt = bt.reshape(-1, MB).to(torch.int32)
        bt[0, -1] = -1                                # a missing page
        bt[2, 0] = case.cache_batch + 5               # an out-of-range page
    elif mode == "linear_table":
        bt = case.cache_bs_id.clone().reshape(-1, 1)  # [batch, 1] naming the cache batch
        case.cache_bs_id = None
    kc8, vc8 = _filled(case)[:2]
    kc, vc = (kc8, vc8) if dtype == torch.int8 else (kc8.to(dtype) / 7, vc8.to(dtype) / 3)
    H, D = case.key.shape[-2:]
    T = int(case.lens.sum()) + 2
    if case.context_seq_offset is not None:
        T = max(T, int((case.context_seq_offset + case.lens).max()) + 1)
    key = torch.full((T, H, D), -3, dtype=dtype)
    value = key.clone()
    ref.linear_cache(4, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset, block_tables=bt)
    gkey = torch.full((T, H, D), -3, dtype=dtype, device=dev)
    gval = gkey.clone()
    tmo.reshape_from_cache(gkey, gval, kc.to(dev), vc.to(dev), case.lens.to(dev),
                           case.max_context_len, _d(case.context_seq_offset, dev), _d(bt, dev),
                           _d(case.cache_seq_offset, dev))
    torch.cuda.synchronize()
    _cmp(gkey, key, "key")
    _cmp(gval, value, "value")


# ---------------------------------------------------------------------------- prefill-sized shape

def test_linear_prefill_roundtrips(tmo, ref, dev):
    """16 sequences of up to 2048 tokens, 8 heads x 128, bf16: quant -> dequant within scale/2
    of the input (and bit-exact against the oracle on a sample), reshape -> reshape_from_cache
    is the identity."""
    g = torch.Generator().manual_seed(81)
    B, H, D, L = 16, 8, 128, 2048
    lens = torch.randint(1, L + 1, (B,), generator=g).to(torch.int32)
    lens[0] = L
    cu = torch.cat((torch.zeros(1, dtype=torch.int32), lens.cumsum(0).to(torch.int32)))
    T = int(cu[-1])
    key = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev)
    cud, lensd = cu.to(dev), lens.to(dev)
    kc = torch.full((B, H, L, D), W.CACHE_SENTINEL, dtype=torch.int8, device=dev)
    vc = torch.full_like(kc, W.CACHE_SENTINEL)
    ks = torch.full((B, H, L), W.SCALE_SENTINEL, device=dev)
    vs = torch.full_like(ks, W.SCALE_SENTINEL)
    tmo.quant_to_linear_cache(key, value, kc, vc, ks, vs, cud, L, True, None, None, None)
    back = torch.empty_like(key, dtype=torch.float32)
    tmo.dequant_from_linear_cache(back, None, kc, None, ks, None, lensd, L, None, None, None, 1, 8)
    torch.cuda.synchronize()
    err = (back - key.float()).abs()
    for i in range(B):
        s0, n = int(cu[i]), int(lens[i])
        sc = ks[i, :, :n].transpose(0, 1)[..., None]
        assert (err[s0:s0 + n] <= sc * (0.5 + 2.0 ** -15)).all(), i
    # bit-exact against the oracle on the first two sequences
    n2 = int(cu[2])
    sub = W.LinearCase(key[:n2].cpu(), value[:n2].cpu(), lens[:2], True, None, None, None, 2, L)
    okc, ovc = sub.caches(torch.int8)
    oks, ovs = sub.scales()
    ref.linear_cache(1, sub.key, sub.value, okc, ovc, sub.context_lengths, L, packed=True,
                     key_scale=oks, value_scale=ovs)
    _cmp(kc[:2], okc, "key_cache[:2]")
    _cmp(vs[:2], ovs, "value_scale[:2]")
    # copy in and out
    bc = torch.zeros(B, H, L, D, dtype=torch.bfloat16, device=dev)
    tmo.reshape_linear_cache(key, None, bc, None, cud, L, True, None, None, None)
    out = torch.zeros_like(key)
    tmo.reshape_from_cache(out, None, bc, None, lensd, L)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), key.view(torch.int16))


@pytest.mark.parametrize("B", [1, 63, 64, 65, 150, 700])
def test_output_rows_follow_the_length_prefix(tmo, ref, dev, B):
    """Reads without context_seq_offset place sequence i at the sum of the lengths before it
    (per-wavefront prefix over 64-length chunks: 1, 2 and 11 chunks), zero lengths included."""
    g = torch.Generator().manual_seed(90 + B)
    lens = torch.randint(0, 9, (B,), generator=g).to(torch.int32)
    case = W.LinearCase(torch.zeros(1, 2, 64), torch.zeros(1, 2, 64), lens, False, None, None,
                        None, B, 8)
    kc, vc, kt, vt, _, _ = _filled(case, seed=B)
    T = int(lens.sum()) + 5
    key = torch.full((T, 2, 64), -3.0, dtype=torch.bfloat16)
    ref.linear_cache(3, key, None, kc, None, lens, 8, key_scale=kt, smode=1)
    gkey = torch.full((T, 2, 64), -3.0, dtype=torch.bfloat16, device=dev)
    tmo.dequant_from_linear_cache(gkey, None, kc.to(dev), None, kt.to(dev), None, lens.to(dev), 8,
                                  None, None, None, 1, 8)
    torch.cuda.synchronize()
    _cmp(gkey, key, "key")
    out = torch.full((T, 2, 64), 7, dtype=torch.int8)
    ref.linear_cache(4, out, None, kc, None, lens, 8)
    gout = torch.full((T, 2, 64), 7, dtype=torch.int8, device=dev)
    tmo.reshape_from_cache(gout, None, kc.to(dev), None, lens.to(dev), 8)
    torch.cuda.synchronize()
    _cmp(gout, out, "reshape_from_cache key")


# ---------------------------------------------------------------------------- 4-bit linear caches

def _int4_caches(case, D, device="cpu", fill=0x5A):
    H = case.key.shape[-2]
    kc = torch.full((case.cache_batch, H, case.cache_len, D // 2), fill, dtype=torch.uint8,
                    device=device).view(torch.int8)
    vc = torch.full((case.cache_batch, H, case.cache_len // 2, D), fill, dtype=torch.uint8,
                    device=device).view(torch.int8)
    return kc, vc


def _quant4_both(tmo, ref, dev, case, groups=1, with_v=True):
    H, D = case.key.shape[-2:]
    kc, vc = _int4_caches(case, D)
    ks, vs = case.scales(groups if groups > 1 else 0)
    v = case.value if with_v else None
    if not with_v:
        vc = vs = None
    ref.linear_cache(1, case.key, v, kc, vc, case.context_lengths, case.max_context_len,
                     packed=case.packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks, value_scale=vs, groups=groups, bits=4)
    gk, gv = _int4_caches(case, D, dev)
    gks, gvs = (t.to(dev) for t in case.scales(groups if groups > 1 else 0))
    if not with_v:
        gv = gvs = None
    tmo.quant_to_linear_cache(case.key.to(dev), _d(v, dev), gk, gv, gks, gvs,
                              case.context_lengths.to(dev), case.max_context_len, case.packed,
                              _d(case.context_seq_offset, dev), _d(case.cache_bs_id, dev),
                              _d(case.cache_seq_offset, dev), 4)
    torch.cuda.synchronize()
    _cmp(gk, kc, "key_cache (int4)")
    _cmp(gks, ks, "key_scale (int4)")
    if with_v:
        _cmp(gv, vc, "value_cache (int4)")
        _cmp(gvs, vs, "value_scale (int4)")


@pytest.mark.parametrize("packed,offsets", [(True, False), (True, True), (False, True)])
@pytest.mark.parametrize("dtype", FLOATS)
def test_quant_to_linear_cache_int4(tmo, ref, dev, dtype, packed, offsets):
    """Codes, nibble order, V position pairs (odd cache offsets keep the partner nibble), scales."""
    case = W.linear_case(dtype, 81, packed=packed, offsets=offsets)
    _quant4_both(tmo, ref, dev, case)
    _quant4_both(tmo, ref, dev, case, with_v=False)


@pytest.mark.parametrize("D,groups", [(128, 1), (128, 4), (128, 16), (64, 8), (512, 2),
                                      (8, 1), (16, 2), (80, 1), (24, 1)])
def test_quant_to_linear_cache_int4_groups_and_widths(tmo, ref, dev, D, groups):
    case = W.linear_case(torch.bfloat16, 82 + D, packed=True, offsets=True, D=D)
    _quant4_both(tmo, ref, dev, case, groups)


def test_quant_to_linear_cache_int4_odd_offsets_and_shapes_rejected(tmo, ref, dev):
    """Every cache offset parity; shapes outside the 4-bit kernels raise instead of writing."""
    case = W.linear_case(torch.float16, 83, packed=True, offsets=False, B=4, S=9, cache_len=24)
    for off in ([1, 0, 3, 2], [0, 1, 2, 3], [5, 7, 1, 1]):
        case.cache_seq_offset = torch.tensor(off, dtype=torch.int32)
        _quant4_both(tmo, ref, dev, case)
    bad = W.linear_case(torch.float16, 84, packed=True, D=20)          # head_size % 8 != 0
    H = bad.key.shape[-2]
    kc = torch.zeros(bad.cache_batch, H, bad.cache_len, 10, dtype=torch.int8, device=dev)
    ks = torch.zeros(bad.cache_batch, H, bad.cache_len, device=dev)
    with pytest.raises(RuntimeError):
        tmo.quant_to_linear_cache(bad.key.to(dev), None, kc, None, ks, None,
                                  bad.context_lengths.to(dev), bad.max_context_len, True, None,
                                  None, None, 4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_to_linear_cache_int4_shared_batch_odd_boundaries(tmo, ref, dev, dtype):
    """Many sequences written into ONE cache batch, back to back, with odd lengths: every
    boundary between two sequences falls inside a V position pair, so two workgroups write
    the two nibbles of the same V bytes in the same call.  Each must keep the other's nibble
    (the reference writes every sequence's positions independently)."""
    g = torch.Generator().manual_seed(87)
    B, H, D = 48, 2, 128
    lens = (2 * torch.randint(0, 5, (B,), generator=g) + 1).to(torch.int32)   # 1, 3, ..., 9
    starts = torch.cat((torch.zeros(1, dtype=torch.int64), lens.cumsum(0)[:-1].long()))
    T = int(lens.sum())
    key = (torch.randn(T, H, D, generator=g) * 2).to(dtype)
    value = (torch.randn(T, H, D, generator=g) * 3).to(dtype)
    case = W.LinearCase(key, value, lens, True, None,
                        torch.zeros(B, dtype=torch.int32),           # one cache batch for all
                        (starts + 1).to(torch.int32),                # odd first position
                        cache_batch=2, cache_len=T + 4)
    for _ in range(3):
        _quant4_both(tmo, ref, dev, case)


def _dequant4_both(tmo, ref, dev, case, dtype, mode, with_v=True):
    g = torch.Generator().manual_seed(85)
    H, D = case.key.shape[-2:]
    L = case.cache_len
    kc = torch.randint(-128, 128, (case.cache_batch, H, L, D // 2), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (case.cache_batch, H, L // 2, D), generator=g, dtype=torch.int8)
    kt = torch.rand(case.cache_batch, H, L, generator=g) * 0.05
    vt = torch.rand(case.cache_batch, H, L, generator=g) * 0.05
    kch, vch = torch.rand(H, D, generator=g) * 0.05, torch.rand(H, D, generator=g) * 0.05
    ks, vs = (kch, vch) if mode == 0 else (kt, vt)
    T = int(case.lens.sum()) + 3
    if case.context_seq_offset is not None:
        T = max(T, int((case.context_seq_offset + case.lens).max()) + 1)
    key = torch.full((T, H, D), -3.0, dtype=dtype)
    value = key.clone() if with_v else None
    if not with_v:
        vc = vs = None
    ref.linear_cache(3, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks if mode == 1 else None, value_scale=vs if mode == 1 else None,
                     key_chan=ks if mode == 0 else None, value_chan=vs if mode == 0 else None,
                     smode=mode, bits=4)
    gkey = torch.full((T, H, D), -3.0, dtype=dtype, device=dev)
    gval = gkey.clone() if with_v else None
    tmo.dequant_from_linear_cache(gkey, gval, kc.to(dev), _d(vc, dev), ks.to(dev), _d(vs, dev),
                                  case.lens.to(dev), case.max_context_len,
                                  _d(case.context_seq_offset, dev), _d(case.cache_bs_id, dev),
                                  _d(case.cache_seq_offset, dev), mode, 4)
    torch.cuda.synchronize()
    _cmp(gkey, key, "key (int4)")
    if with_v:
        _cmp(gval, value, "value (int4)")


@pytest.mark.parametrize("offsets", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", FLOATS)
def test_dequant_from_linear_cache_int4(tmo, ref, dev, dtype, mode, offsets):
    case = W.linear_case(dtype, 86, packed=True, offsets=offsets)
    _dequant4_both(tmo, ref, dev, case, dtype, mode)
    _dequant4_both(tmo, ref, dev, case, dtype, mode, with_v=False)


@pytest.mark.parametrize("D", [8, 16, 80, 128, 512])
def test_dequant_from_linear_cache_int4_widths(tmo, ref, dev, D):
    case = W.linear_case(torch.bfloat16, 87 + D, packed=True, offsets=True, D=D)
    _dequant4_both(tmo, ref, dev, case, torch.bfloat16, 1)


def test_int4_round_trip_prefill(tmo, ref, dev):
    """8 x 512 packed tokens, 8 heads x 128, bf16: quant (4 bit) then dequant is within scale / 2
    per element, and bit-exact against the oracle."""
    B, S, H, D, L = 8, 512, 8, 128, 1024
    g = torch.Generator().manual_seed(88)
    key = torch.randn(B * S, H, D, generator=g).to(torch.bfloat16)
    value = torch.randn(B * S, H, D, generator=g).to(torch.bfloat16)
    cu = torch.arange(B + 1, dtype=torch.int32) * S
    case = W.LinearCase(key, value, torch.full((B,), S, dtype=torch.int32), True, None, None,
                        None, B, L)
    _quant4_both(tmo, ref, dev, case)
    kc, vc = _int4_caches(case, D, dev)
    ks = torch.zeros(B, H, L, device=dev)
    vs = torch.zeros_like(ks)
    tmo.quant_to_linear_cache(key.to(dev), value.to(dev), kc, vc, ks, vs, cu.to(dev), S, True,
                              None, None, None, 4)
    bk = torch.empty(B * S, H, D, device=dev)
    bv = torch.empty_like(bk)
    lens = torch.full((B,), S, dtype=torch.int32, device=dev)
    tmo.dequant_from_linear_cache(bk, bv, kc, vc, ks, vs, lens, S, None, None, None, 1, 4)
    torch.cuda.synchronize()
    for x, back, sc in ((key, bk, ks), (value, bv, vs)):
        err = (back.cpu() - x.float()).abs().reshape(B, S, H, D)
        s = sc[:, :, :S].cpu().permute(0, 2, 1)[..., None]
        assert (err <= s * (0.5 + 2.0 ** -15)).all()
