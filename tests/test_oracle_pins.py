"""Pins of the CPU oracle (oracle/tmo_oracle.c) -- CPU only.

The reference ships no golden vectors, fixtures or runnable implementation, so each oracle
function is pinned by checks independent of its C code:

* torch-CPU execution of the reference's docstring "Math" block (library routines: abs/amax,
  IEEE true division, round-half-even, clamp, int8 cast, advanced indexing, bf16/fp16 casts);
* exact rational arithmetic (fractions.Fraction) on rows engineered so that x/scale lands
  within a few ulps of a half-integer -- this fixes "IEEE-divide then round-half-even" apart
  from every cheaper rule (reciprocal multiply, round-half-away, bf16 scale, double rounding);
* closed forms and invariants: hand-computed ties, zero rows, odd symmetry, power-of-two
  scaling, the +-127 argmax code, the scale/2 error bound, sentinel bytes of skipped slots;
* numpy's IEEE float16 casts for the oracle's fp16 conversion.

A plausible mistake in the oracle (divide vs reciprocal, block/offset transposed, wrong
rounding, smooth applied to the wrong group, off-by-one page) fails at least one of these.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from tests import workloads as W

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


# ---------------------------------------------------------------------------- torch restatements

def torch_row_quant(x: torch.Tensor):
    """reference _ops.py:1524-1537 / 3167-3172 executed by torch on the CPU, fp32 (D1),
    all-zero rows -> scale 0 / codes 0 (D3)."""
    amax = x.abs().amax(-1)                      # max in the input dtype (exact)
    scale = amax.to(torch.float32) / 127.0
    q = (x.to(torch.float32) / scale[..., None]).round().clamp(-128, 127)
    q = torch.where(scale[..., None] == 0, torch.zeros_like(q), q)
    return q.to(torch.int8), scale


def torch_quant_to_paged(k, v, kc, vc, ks, vs, slot):
    NB, H, BS, D = kc.shape
    valid = (slot >= 0) & (slot < NB * BS)
    s = slot[valid].long()
    blk, off = s // BS, s % BS
    for x, c, sc in ((k, kc, ks), (v, vc, vs)):
        if x is None:
            continue
        codes, scale = torch_row_quant(x[valid])
        c.permute(0, 2, 1, 3)[blk, off] = codes        # [NB, BS, H, D] view of the pages
        sc.permute(0, 2, 1)[blk, off] = scale


def bits(t):
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16)
    return t


# ---------------------------------------------------------------------------- quant_to_paged_cache

def _rand_case(dtype, T=64, H=4, D=128, NB=40, BS=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, H, D, generator=g) * torch.logspace(-4, 4, T)[:, None, None]).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    k[3] = 0  # zero rows
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[::7] = -1
    slot[5] = NB * BS + 1
    return W.PagedQuantCase("rand", k, v, slot, NB, BS)


@pytest.mark.parametrize("dtype", DTYPES)
def test_quant_matches_torch_docstring_math(ref, dtype):
    for seed in range(4):
        case = _rand_case(dtype, seed=seed)
        kc, vc, ks, vs = case.empty_caches()
        ref.quant_to_paged_cache(case.k, case.v, kc, vc, ks, vs, case.slot_mapping)
        tk, tv, tks, tvs = case.empty_caches()
        torch_quant_to_paged(case.k, case.v, tk, tv, tks, tvs, case.slot_mapping)
        for a, b in ((kc, tk), (vc, tv), (ks, tks), (vs, tvs)):
            assert torch.equal(bits(a), bits(b))


def torch_quant_to_paged_fp8(k, v, kc, vc, ks, vs, slot):
    """The fp8 branch of _ops.py:1524-1537 by torch: scale = fp32(amax) / 448, codes =
    float8_e4m3fn(clip(x / scale, -448, 448)) (the clip of the linear sibling, _ops.py:1741);
    all-zero rows: scale 0, codes 0."""
    NB, H, BS, D = kc.shape
    valid = (slot >= 0) & (slot < NB * BS)
    s = slot[valid].long()
    blk, off = s // BS, s % BS
    for x, c, sc in ((k, kc, ks), (v, vc, vs)):
        if x is None:
            continue
        xv = x[valid]
        scale = xv.abs().amax(-1).to(torch.float32) / 448.0
        q = (xv.to(torch.float32) / scale[..., None]).clamp(-448, 448)
        q = torch.where(scale[..., None] == 0, torch.zeros_like(q), q)
        c.view(torch.uint8).permute(0, 2, 1, 3)[blk, off] = q.to(torch.float8_e4m3fn).view(torch.uint8)
        sc.permute(0, 2, 1)[blk, off] = scale


@pytest.mark.parametrize("dtype", DTYPES)
def test_quant_fp8_matches_torch_docstring_math(ref, dtype):
    for seed in range(3):
        case = _rand_case(dtype, seed=seed)
        kc, vc, ks, vs = case.empty_caches()
        kc, vc = kc.view(torch.float8_e4m3fn), vc.view(torch.float8_e4m3fn)
        ref.quant_to_paged_cache(case.k, case.v, kc, vc, ks, vs, case.slot_mapping)
        tk, tv, tks, tvs = case.empty_caches()
        tk, tv = tk.view(torch.float8_e4m3fn), tv.view(torch.float8_e4m3fn)
        torch_quant_to_paged_fp8(case.k, case.v, tk, tv, tks, tvs, case.slot_mapping)
        for a, b in ((kc, tk), (vc, tv)):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
        for a, b in ((ks, tks), (vs, tvs)):
            assert torch.equal(bits(a), bits(b))


def test_quant_cfg1_and_cfg2_match_torch(ref):
    for case in (W.cfg1(), W.cfg2()):
        kc, vc, ks, vs = case.empty_caches()
        ref.quant_to_paged_cache(case.k, case.v, kc, vc, ks, vs, case.slot_mapping)
        tk, tv, tks, tvs = case.empty_caches()
        torch_quant_to_paged(case.k, case.v, tk, tv, tks, tvs, case.slot_mapping)
        for a, b in ((kc, tk), (vc, tv), (ks, tks), (vs, tvs)):
            assert torch.equal(bits(a), bits(b))
        assert int((ks != W.SCALE_SENTINEL).sum()) == case.valid_tokens() * case.k.shape[1]


def _f32_round(q: Fraction) -> Fraction:
    """Exact round-to-nearest-even of a rational to binary32 (no overflow in this use)."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum_exp = max(e - 23, -149)
    scaled = a / Fraction(2) ** quantum_exp
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * Fraction(2) ** quantum_exp


def _rne_int(q: Fraction) -> int:
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n


def _exact_code(x: float, s: float) -> int:
    return max(-128, min(127, _rne_int(_f32_round(Fraction(x) / Fraction(s)))))


def _near_tie_rows(dtype, seed):
    """Rows (amax first) whose other entries sit within a few ulps of (k + 0.5) * scale."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for _ in range(6):
        amax = torch.tensor([float(torch.rand(1, generator=g)) * 8 + 0.01]).to(dtype)
        s = float(_f32_round(Fraction(float(amax)) / 127))
        xs = [float(amax)]
        for kk in torch.randint(-127, 127, (40,), generator=g).tolist():
            t = torch.tensor([(kk + 0.5) * s], dtype=torch.float32).to(dtype)
            for d in (-2, -1, 0, 1, 2):
                # neighbours of t in the input format
                bitsv = bits(t.clone()).clone()
                bitsv += d
                xs.append(float(bitsv.view(dtype)[0]))
        x = torch.tensor(xs, dtype=torch.float32).to(dtype)
        x = x[x.abs() <= amax.abs()[0].to(dtype)]
        rows.append(x)
    n = max(r.numel() for r in rows)
    out = torch.zeros(len(rows), n, dtype=dtype)
    for i, r in enumerate(rows):
        out[i, : r.numel()] = r
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_quant_near_ties_exact_rational(ref, dtype):
    rows = _near_tie_rows(dtype, seed=DTYPES.index(dtype) + 17)
    R, D = rows.shape
    k = rows.reshape(R, 1, D).contiguous()
    slot = torch.arange(R, dtype=torch.int32)
    case = W.PagedQuantCase("ties", k, k, slot, (R + 15) // 16, 16)
    kc, _, ks, _ = case.empty_caches()
    ref.quant_to_paged_cache(k, None, kc, None, ks, None, slot)
    n_checked = 0
    for r in range(R):
        x = rows[r].to(torch.float32).tolist()
        s = float(ks[r // 16, 0, r % 16])
        amax = max(abs(v) for v in x)
        assert Fraction(s) == _f32_round(Fraction(amax) / 127)
        for d, xv in enumerate(x):
            assert int(kc[r // 16, 0, r % 16, d]) == _exact_code(xv, s), (r, d, xv, s)
            n_checked += 1
    assert n_checked > 1000


def test_quant_closed_forms(ref):
    row = torch.zeros(1, 2, 16)
    row[0, 0, :8] = torch.tensor([127.0, 2.5, 3.5, -0.5, 1.5, -2.5, -3.5, 0.25])
    row[0, 1, :] = 0.0                                         # all-zero row (D3)
    for dtype in DTYPES:
        k = row.to(dtype)
        slot = torch.tensor([5], dtype=torch.int32)
        case = W.PagedQuantCase("closed", k, k, slot, 1, 8)
        kc, _, ks, _ = case.empty_caches()
        ref.quant_to_paged_cache(k, None, kc, None, ks, None, slot)
        assert kc[0, 0, 5, :8].tolist() == [127, 2, 4, 0, 2, -2, -4, 0]
        assert float(ks[0, 0, 5]) == 1.0
        assert kc[0, 1, 5].tolist() == [0] * 16 and float(ks[0, 1, 5]) == 0.0
        # untouched slots keep the sentinel
        assert int((kc[0, :, :5] != W.CACHE_SENTINEL).sum()) == 0
        assert int((ks[0, :, 6:] != W.SCALE_SENTINEL).sum()) == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_quant_invariants(ref, dtype):
    g = torch.Generator().manual_seed(3)
    T, H, D = 256, 2, 96
    x = (torch.randn(T, H, D, generator=g) * torch.logspace(-3, 3, T)[:, None, None]).to(dtype)
    slot = torch.arange(T, dtype=torch.int32)
    case = W.PagedQuantCase("inv", x, x, slot, T // 16, 16)

    def quant(inp):
        kc, _, ks, _ = case.empty_caches()
        ref.quant_to_paged_cache(inp, None, kc, None, ks, None, slot)
        codes = kc.permute(0, 2, 1, 3).reshape(T, H, D)
        scale = ks.permute(0, 2, 1).reshape(T, H)
        return codes, scale

    codes, scale = quant(x)
    xf = x.to(torch.float64)
    s = scale.to(torch.float64)
    # |x - code * s| <= s/2 (+ the fp32 rounding of x/s)
    err = (xf - codes.to(torch.float64) * s[..., None]).abs()
    assert torch.all(err <= s[..., None] * (0.5 + 2.0 ** -15))
    # the argmax element encodes to +-127; codes never exceed the symmetric range
    am = xf.abs().argmax(-1, keepdim=True)
    assert torch.all(codes.gather(-1, am).abs() == 127)
    assert int(codes.min()) >= -127
    # sign agreement
    assert torch.all((codes.sign() == xf.sign()) | (codes == 0))
    # odd symmetry (RNE is symmetric) and power-of-two scaling (exact in every format here)
    c_neg, s_neg = quant(-x)
    assert torch.equal(c_neg, -codes) and torch.equal(s_neg, scale)
    c2, s2 = quant(x * 2)
    assert torch.equal(c2, codes) and torch.equal(s2, scale * 2)


def test_quant_threads_do_not_change_results(ref):
    case = W.cfg2()
    a = case.empty_caches()
    b = case.empty_caches()
    ref.quant_to_paged_cache(case.k, case.v, *a, case.slot_mapping, nthreads=1)
    ref.quant_to_paged_cache(case.k, case.v, *b, case.slot_mapping, nthreads=8)
    for x, y in zip(a, b):
        assert torch.equal(bits(x), bits(y))


# ---------------------------------------------------------------------------- reshape_paged_cache

@pytest.mark.parametrize("dtype", DTYPES + [torch.int8])
def test_reshape_matches_torch_indexing(ref, dtype):
    g = torch.Generator().manual_seed(1)
    T, H, D, NB, BS = 50, 3, 20, 12, 8
    src = torch.randint(-100, 100, (T, 2 * H, D), generator=g).to(dtype)
    k, v = src[:, :H], src[:, H:]                                  # strided views
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[::5] = -1
    slot[2] = NB * BS
    kc = torch.full((NB, H, BS, D), 9, dtype=dtype)
    vc = kc.clone()
    ref.reshape_paged_cache(k, v, kc, vc, slot, False)
    tk, tv = torch.full_like(kc, 9), torch.full_like(vc, 9)
    valid = (slot >= 0) & (slot < NB * BS)
    s = slot[valid].long()
    tk.permute(0, 2, 1, 3)[s // BS, s % BS] = k[valid]
    tv.permute(0, 2, 1, 3)[s // BS, s % BS] = v[valid]
    assert torch.equal(bits(kc), bits(tk)) and torch.equal(bits(vc), bits(tv))
    kb = torch.zeros_like(k)
    ref.reshape_paged_cache(kb, None, kc, None, slot, True)
    assert torch.equal(bits(kb)[valid], bits(k.contiguous())[valid])      # gather o scatter = id
    assert torch.all(bits(kb)[~valid] == 0)


# ---------------------------------------------------------------------------- dequant_from_paged_cache

def torch_dequant(kc, ks, ctx, bt, mode, out_dtype, offsets):
    """reference _ops.py:3749-3774 executed by torch (cast order of _ops.py:3677)."""
    NB, H, BS, D = kc.shape
    out = {}
    for i, n in enumerate(ctx.tolist()):
        nblk = (n + BS - 1) // BS
        pages = bt[i, :nblk].long()
        codes = kc[pages].permute(0, 2, 1, 3).reshape(nblk * BS, H, D)[:n]
        if mode == 1:
            sc = ks[pages].permute(0, 2, 1).reshape(nblk * BS, H)[:n, :, None]
        else:
            sc = ks[None]
        out[int(offsets[i])] = (codes.to(torch.float32) * sc).to(out_dtype)
    return out


@pytest.mark.parametrize("out_dtype", DTYPES)
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("cache", ["int8", "fp8"])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_dequant_fp8_pages_and_bf16_scales_match_torch(ref, out_dtype, mode, cache, scale_dtype):
    """The reference math with bf16 scale tensors (_ops.py:3805-3806) and with the
    float8_e4m3fn pages quant_to_paged_cache writes: (code.to(float32) * scale).to(out_dtype)
    executed by torch, whose float8_e4m3fn and bfloat16 casts to float32 are exact -- bit for
    bit against the oracle, which widens a bf16 scale itself."""
    g = torch.Generator().manual_seed(11 + mode)
    B, NB, H, BS, D = 4, 40, 2, 16, 32
    ctx = torch.tensor([16, 3, 45, 31], dtype=torch.int32)
    bt = torch.randperm(NB, generator=g)[: B * 3].reshape(B, 3).to(torch.int32)
    if cache == "int8":
        kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    else:
        kc = W.fp8_codes((NB, H, BS, D), g)
    ks = (torch.rand(NB, H, BS, generator=g) * 0.1) if mode == 1 else \
        (torch.rand(H, D, generator=g) * 0.1)
    ks.view(-1)[0] = 3e36 if scale_dtype == torch.float32 else 1e30   # beyond fp16 / bf16
    ks = ks.to(scale_dtype)
    total = int(ctx.sum())
    got = torch.full((total, H, D), -1.0).to(out_dtype)
    ref.dequant_from_paged_cache(got, None, kc, None, ks, None, ctx, None, bt, mode)
    offsets = (torch.cumsum(ctx, 0) - ctx).to(torch.int32)
    want = torch_dequant(kc, ks.to(torch.float32), ctx, bt, mode, out_dtype, offsets)
    for start, rows in want.items():
        assert torch.equal(bits(got[start:start + rows.shape[0]]), bits(rows))
    if cache == "fp8":  # the fp8 codes decode to their e4m3fn values: |out| <= 448 * scale
        assert (got.float().abs() <= 448 * ks.float().max() * 1.01).all() or out_dtype != torch.float32


@pytest.mark.parametrize("out_dtype", DTYPES)
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("with_offsets", [False, True])
def test_dequant_matches_torch_docstring_math(ref, out_dtype, mode, with_offsets):
    g = torch.Generator().manual_seed(mode * 7 + int(with_offsets))
    B, NB, H, BS, D = 5, 48, 3, 16, 32
    ctx = torch.tensor([16, 1, 37, 80, 15], dtype=torch.int32)
    bt = torch.randperm(NB, generator=g)[: B * 8].reshape(B, 8).to(torch.int32)
    kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    ks = (torch.rand(NB, H, BS, generator=g) * 0.1) if mode == 1 else \
        (torch.rand(H, D, generator=g) * 0.1)
    ks.view(-1)[0] = 3e36                   # products beyond fp16 / bf16 range
    cum = torch.cumsum(ctx, 0) - ctx
    offsets = (cum.flip(0) if with_offsets else cum).to(torch.int32)
    if with_offsets:  # non-overlapping, shuffled starting rows
        order = torch.tensor([4, 2, 0, 3, 1])
        start = torch.zeros(B, dtype=torch.int64)
        acc = 0
        for i in order.tolist():
            start[i] = acc
            acc += int(ctx[i])
        offsets = start.to(torch.int32)
    total = int(ctx.sum())
    got = torch.full((total, H, D), -1.0).to(out_dtype)
    ref.dequant_from_paged_cache(got, None, kc, None, ks, None, ctx,
                                 offsets if with_offsets else None, bt, mode)
    want = torch_dequant(kc, ks, ctx, bt, mode, out_dtype, offsets)
    for start, rows in want.items():
        assert torch.equal(bits(got[start:start + rows.shape[0]]), bits(rows))


def test_dequant_roundtrip_error_bound(ref):
    """dequant(quant(x)) is within scale/2 (+ bf16 rounding) of x."""
    case = W.cfg1()
    kc, vc, ks, vs = case.empty_caches()
    ref.quant_to_paged_cache(case.k, case.v, kc, vc, ks, vs, case.slot_mapping)
    ctx = torch.tensor([kc.shape[0] * kc.shape[2]], dtype=torch.int32)
    bt = torch.arange(kc.shape[0], dtype=torch.int32)[None]
    out = torch.zeros(int(ctx), 8, 128, dtype=torch.float32)
    ref.dequant_from_paged_cache(out, None, kc, None, ks, None, ctx, None, bt, 1)
    s = case.slot_mapping.long()
    scale = ks.permute(0, 2, 1).reshape(-1, 8)[s]
    err = (out[s] - case.k.float()).abs()
    assert torch.all(err <= scale[..., None] * (0.5 + 2.0 ** -15))


# ---------------------------------------------------------------------------- scaled_quantize

def torch_moe_quantize(x, smooth, token_count=None, gather_index=None, start=None):
    """reference _ops.py:3147-3172 executed by torch (dynamic_quant=True, act_mode none)."""
    inp = x
    if gather_index is not None and start is not None:
        inp = x[gather_index[start: start + int(token_count.sum())].long()]
    elif gather_index is not None:
        inp = x[gather_index.long()]
    if token_count is not None:
        parts = inp.split(token_count.tolist())
        smoothed = torch.cat([parts[i] * smooth[i] for i in range(len(parts))], 0)
    elif smooth is not None:
        smoothed = inp * smooth
    else:
        smoothed = inp
    codes, scale = torch_row_quant(smoothed.to(torch.float32))
    return codes, scale


@pytest.mark.parametrize("dtype", DTYPES)
def test_smooth_quant_matches_torch_docstring_math(ref, dtype):
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(40, 3, 64, generator=g) * 5).to(dtype)
    x[7] = 0
    sm = 0.5 + 1.5 * torch.rand(64, generator=g)
    for smooth in (sm, None, torch.tensor([1.25])):
        out = torch.full((40, 3, 64), 9, dtype=torch.int8)
        sc = torch.full((40, 3), -1.0)
        ref.scaled_quantize_per_token(x, out, sc, smooth)
        w_out, w_sc = torch_moe_quantize(x, smooth)
        assert torch.equal(out, w_out) and torch.equal(bits(sc), bits(w_sc))


def test_smooth_quant_moe_gather_matches_torch(ref):
    case = W.cfg4_moe()
    x = case.x[:512]
    keep = case.gather_index < 512
    gi = case.gather_index[keep]
    experts = torch.repeat_interleave(torch.arange(64), case.token_count.long())[keep]
    tc = torch.bincount(experts, minlength=64).to(torch.int32)
    out = torch.empty(gi.numel(), 4096, dtype=torch.int8)
    sc = torch.empty(gi.numel())
    ref.scaled_quantize_per_token(x, out, sc, case.smooth, tc, gi)
    w_out, w_sc = torch_moe_quantize(x, case.smooth, tc, gi)
    assert torch.equal(out, w_out) and torch.equal(bits(sc), bits(w_sc))
    # gather_index_start_position: rows gather_index[start : start + sum(token_count)]
    tc2 = tc.clone()
    tc2[30:] = 0
    n = int(tc2.sum())
    out2 = torch.full((gi.numel(), 4096), 9, dtype=torch.int8)
    sc2 = torch.full((gi.numel(),), -1.0)
    ref.scaled_quantize_per_token(x, out2, sc2, case.smooth, tc2, gi,
                                  torch.tensor([11], dtype=torch.int32))
    w_out2, w_sc2 = torch_moe_quantize(x, case.smooth, tc2, gi, 11)
    assert torch.equal(out2[:n], w_out2) and torch.equal(bits(sc2[:n]), bits(w_sc2))
    assert torch.all(out2[n:] == 9) and torch.all(sc2[n:] == -1.0)


# ---------------------------------------------------------------------------- conversions

def test_bf16_conversion_matches_torch(ref):
    g = torch.Generator().manual_seed(0)
    raw = torch.randint(-2**31, 2**31 - 1, (2_000_000,), generator=g, dtype=torch.int64)
    f = raw.to(torch.int32).view(torch.float32)
    f = f[~torch.isnan(f)]
    specials = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 3.3895314e38, 1e-45,
                             1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9])
    f = torch.cat([f, specials])
    assert torch.equal(ref.f32_to_bf16_bits(f), f.to(torch.bfloat16).view(torch.int16))


def test_f16_conversions_match_numpy(ref):
    g = torch.Generator().manual_seed(1)
    raw = torch.randint(-2**31, 2**31 - 1, (2_000_000,), generator=g, dtype=torch.int64)
    f = raw.to(torch.int32).view(torch.float32)
    f = f[~torch.isnan(f)]
    # every fp16 value, the midpoints between neighbours and their fp32 neighbours
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mid = (h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2
    mids = mid.astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(0)), mids, h, [65520.0, 65519.996]])
    f = torch.cat([f, torch.from_numpy(near.astype(np.float32)),
                   -torch.from_numpy(near.astype(np.float32))])
    want = torch.from_numpy(f.numpy().astype(np.float16).view(np.int16))
    assert torch.equal(ref.f32_to_f16_bits(f), want)
    allh = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    fin = (allh.to(torch.int32) & 0x7c00) != 0x7c00
    got = ref.f16_bits_to_f32(allh)[fin]
    want32 = torch.from_numpy(allh.numpy().view(np.float16).astype(np.float32))[fin]
    assert torch.equal(got.view(torch.int32), want32.view(torch.int32))


# ---------------------------------------------------------------------------- offline (static) quant

def torch_offline_quant_to_paged(k, v, k_scale, v_scale, slot, kc, vc):
    """reference _ops.py:1652-1670 executed by torch on the CPU, with quant2int8 / quant2fp8
    as the linear sibling spells them out (_ops.py:1829-1840): fp32 x / scale (IEEE), then
    int8 round half even + clip(-128, 127), or clip(-448, 448) + the float8_e4m3fn cast."""
    NB, H, BS, D = kc.shape
    valid = (slot >= 0) & (slot < NB * BS)
    s = slot[valid].long()
    blk, off = s // BS, s % BS
    for x, c, sc in ((k, kc, k_scale), (v, vc, v_scale)):
        if x is None:
            continue
        scale = sc.to(torch.float32) if torch.is_tensor(sc) else \
            torch.tensor(1.0 if sc is None else float(sc), dtype=torch.float32)
        q = x[valid].to(torch.float32) / scale
        if c.dtype == torch.int8:
            codes = q.round().clamp(-128, 127).to(torch.int8).view(torch.uint8)
        else:
            codes = q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        c.view(torch.uint8).permute(0, 2, 1, 3)[blk, off] = codes


def _offline_case(dtype, cache_dtype, per_channel, seed, T=80, H=4, D=64, NB=30, BS=16):
    g = torch.Generator().manual_seed(seed)
    # magnitudes spread so that some quotients saturate and some round to zero
    k = (torch.randn(T, H, D, generator=g) * torch.logspace(-3, 2, T)[:, None, None]).to(dtype)
    v = (torch.randn(T, H, D, generator=g) * 7).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[::9] = -1
    slot[4] = NB * BS + 3
    if per_channel:
        ks = 0.01 + torch.rand(H, D, generator=g) * 0.2
        vs = 0.02 + torch.rand(H, D, generator=g) * 0.1
    else:
        ks, vs = 0.0371, 0.0523
    kc = torch.full((NB, H, BS, D), 0x5A, dtype=torch.uint8).view(cache_dtype)
    return k, v, ks, vs, slot, kc


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("per_channel", [True, False])
def test_offline_quant_matches_torch_docstring_math(ref, dtype, cache_dtype, per_channel):
    for seed in range(3):
        k, v, ks, vs, slot, kc = _offline_case(dtype, cache_dtype, per_channel, seed)
        vc = kc.clone()
        ref.offline_quant_to_paged_cache(k, v, ks, vs, slot, kc, vc)
        tk = torch.full_like(kc.view(torch.uint8), 0x5A).view(cache_dtype)
        tv = tk.clone()
        torch_offline_quant_to_paged(k, v, ks, vs, slot, tk, tv)
        assert torch.equal(kc.view(torch.uint8), tk.view(torch.uint8))
        assert torch.equal(vc.view(torch.uint8), tv.view(torch.uint8))
    # K only, and a strided k (a column view of a fused qkv)
    qkv = torch.randn(32, 12, 64).to(dtype)
    kk = qkv[:, 4:8]
    slot = torch.arange(32, dtype=torch.int32) * 3
    kc = torch.full((8, 4, 16, 64), 0x5A, dtype=torch.uint8).view(cache_dtype)
    tk = kc.clone()
    sc = torch.rand(4, 64) * 0.05 + 0.01 if per_channel else 0.02
    ref.offline_quant_to_paged_cache(kk, None, sc, None, slot, kc, None)
    torch_offline_quant_to_paged(kk, None, sc, None, slot, tk, None)
    assert torch.equal(kc.view(torch.uint8), tk.view(torch.uint8))


def _e4m3_value(c: int) -> Fraction:
    e, m = c >> 3, c & 7
    return Fraction(m, 512) if e == 0 else Fraction(8 + m, 8) * Fraction(2) ** (e - 7)


def test_e4m3_reader_matches_torch_and_closed_form(ref):
    """The oracle's float8_e4m3fn reader (the pages' consumers: attention and dequant) on all
    256 codes: equal to torch's float8_e4m3fn -> float32 cast, and to the closed form
    (-1)^s (8 + m) 2^(e - 10) (m 2^-9 for e = 0); S.1111.111 is NaN and nothing else is."""
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    mine = ref.e4m3_to_f32(b)
    want = b.view(torch.float8_e4m3fn).to(torch.float32)
    nan = torch.isnan(want)
    assert nan.nonzero().flatten().tolist() == [0x7F, 0xFF]
    assert torch.equal(torch.isnan(mine), nan)
    assert torch.equal(bits(mine[~nan]), bits(want[~nan]))
    for c in range(256):
        if c & 0x7F == 0x7F:
            continue
        v = _e4m3_value(c & 0x7F) * (-1 if c & 0x80 else 1)
        assert Fraction(float(mine[c])) == v, c
    assert float(mine[0x08]) == 2.0 ** -6 and float(mine[0x01]) == 2.0 ** -9
    assert float(mine[0x7E]) == 448.0 and float(mine[0x80]) == 0.0 and str(float(mine[0x80])) == "-0.0"


def _exact_e4m3(q: Fraction) -> int:
    """float8_e4m3fn code of a rational (clip to +-448, nearest, ties to the even code)."""
    sign = 0x80 if q < 0 else 0
    a = min(abs(q), Fraction(448))
    best, bd = 0, a
    for c in range(1, 127):
        d = abs(a - _e4m3_value(c))
        if d < bd or (d == bd and c % 2 == 0 and best % 2 == 1):
            best, bd = c, d
    return sign | best


def test_offline_quant_near_ties_exact_rational(ref):
    """x within +-2 ulps of (k + 0.5) * s (int8) and of e4m3 midpoints * s (fp8), per channel:
    the oracle must round the IEEE quotient, not a reciprocal product."""
    g = torch.Generator().manual_seed(99)
    H, D, T = 2, 64, 10
    scales = (0.003 + torch.rand(H, D, generator=g) * 0.5).to(torch.float32)

    def nudge(val: float) -> float:
        t = torch.tensor([val], dtype=torch.float32)
        t = (t.view(torch.int32) + int(torch.randint(-2, 3, (1,), generator=g))).view(torch.float32)
        return float(t)

    xi = torch.empty(T, H, D)
    xf = torch.empty(T, H, D)
    for t in range(T):
        for h in range(H):
            for d in range(D):
                s = float(scales[h, d])
                xi[t, h, d] = nudge((int(torch.randint(-130, 130, (1,), generator=g)) + 0.5) * s)
                c = int(torch.randint(1, 126, (1,), generator=g))
                mid = (_e4m3_value(c) + _e4m3_value(c + 1)) / 2
                xf[t, h, d] = nudge(float(mid) * s * (1 if c % 3 else -1))
    slot = torch.arange(T, dtype=torch.int32)
    for k, cdt in ((xi, torch.int8), (xf, torch.float8_e4m3fn)):
        kc = torch.zeros(1, H, 16, D, dtype=torch.uint8).view(cdt)
        ref.offline_quant_to_paged_cache(k, None, scales, None, slot, kc, None)
        got = kc.view(torch.uint8)
        for t in range(T):
            for h in range(H):
                for d in range(D):
                    q = _f32_round(Fraction(float(k[t, h, d])) / Fraction(float(scales[h, d])))
                    want = (max(-128, min(127, _rne_int(q))) & 0xFF) if cdt == torch.int8 \
                        else _exact_e4m3(q)
                    assert int(got[0, h, t, d]) == want, (cdt, t, h, d)


def test_fp8_conversion_matches_torch(ref):
    """The oracle's fp32 -> float8_e4m3fn against torch's cast: every bf16 value in
    [-448, 448], every midpoint between adjacent e4m3 values and its fp32 neighbours, and 2 M
    random fp32 values in range."""
    b = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    b = b[torch.isfinite(b) & (b.abs() <= 448)]
    vals = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = ((vals[:-1].double() + vals[1:].double()) / 2).float()
    near = torch.cat([mids, torch.nextafter(mids, torch.full_like(mids, 1e9)),
                      torch.nextafter(mids, torch.zeros_like(mids)), vals])
    g = torch.Generator().manual_seed(3)
    r = (torch.rand(2_000_000, generator=g) * 2 - 1) * 448 * torch.rand(2_000_000, generator=g) ** 6
    f = torch.cat([b, near, -near, r, torch.tensor([0.0, -0.0, 448.0, -448.0, 1e-30, -1e-30])])
    assert torch.equal(ref.f32_to_e4m3(f), f.to(torch.float8_e4m3fn).view(torch.uint8))


# ---------------------------------------------------------------------------- fused rope (rmsnorm)

def _sum_squares_chunked(x: torch.Tensor, square: bool = True) -> torch.Tensor:
    """D10's order with elementwise torch ops: 8-element chunks summed in order, then a
    balanced tree over the chunk sums (every product and sum a separate IEEE operation).
    square=False sums the values themselves (D13's mean)."""
    D = x.shape[-1]
    n = (D + 7) // 8
    width = 1 << (n - 1).bit_length()
    term = (lambda e: x[..., e] * x[..., e]) if square else (lambda e: x[..., e])
    parts = []
    for c in range(width):
        if c < n:
            e0, e1 = 8 * c, min(8 * c + 8, D)
            acc = term(e0)
            for e in range(e0 + 1, e1):
                acc = acc + term(e)
        else:
            acc = torch.zeros_like(x[..., 0])
        parts.append(acc)
    while len(parts) > 1:
        parts = [parts[2 * i] + parts[2 * i + 1] for i in range(len(parts) // 2)]
    return parts[0]


def torch_fused_rope(qkv, k_cache, v_cache, sin, cos, position_id, k_gamma, k_scale, v_scale,
                     slot, eps, q_gamma, off, exact=True, wide=torch.float32, norm_type="rmsnorm",
                     k_beta=None, linear=None):
    """reference _ops.py:3493-3520 (rmsnorm branch; layernorm branch: rotate, then layer_norm
    of K, _ops.py:3501-3504) with apply_rotary's fold math (_ops.py:1116-1127), executed by
    torch on the CPU in `wide` precision.  exact=True uses D10's / D13's summation order (then
    the result must equal the oracle bit for bit); exact=False uses torch's own mean of
    squares and torch.nn.functional.layer_norm (the docstring literally)."""
    B, S, H, D = qkv.shape
    NB, Hk, BS, _ = k_cache.shape
    Hq = H - 2 * Hk
    x = qkv.to(wide)
    rope = sin.shape[-1]
    half = rope // 2
    pos = (position_id.long()[:, None] + torch.arange(S)[None, :])          # [B, S]
    inside = ((pos >= 0) & (pos < sin.shape[0]))[:, :, None, None]           # else: no rotation
    pc = pos.clamp(0, sin.shape[0] - 1)
    sn, cs = sin[pc].to(wide)[:, :, None, :], cos[pc].to(wide)[:, :, None, :]

    def rmsnorm(t, gamma):
        ss = _sum_squares_chunked(t) if exact else (t * t).sum(-1)
        mean = ss / D
        # sqrt and 1/r through float64, rounded once: the correctly rounded fp32 results
        # (binary64 has more than twice binary32's precision).  torch's own fp32 sqrt is not
        # always correctly rounded on the CPU (59.49298858642578 -> 7.713169574737549, the
        # nearest float being 7.713170051574707).
        r = torch.sqrt((mean + eps).double()).to(wide)
        inv = (1.0 / r.double()).to(wide)
        return (t * inv[..., None]) * gamma.to(wide)

    def layernorm(t):
        if not exact:
            b = None if k_beta is None else k_beta.to(wide)
            return torch.nn.functional.layer_norm(t, (D,), k_gamma.to(wide), b, eps)
        mean = _sum_squares_chunked(t, square=False) / D
        d = t - mean[..., None]
        var = _sum_squares_chunked(d) / D
        r = torch.sqrt((var + eps).double()).to(wide)
        inv = (1.0 / r.double()).to(wide)
        y = (d * inv[..., None]) * k_gamma.to(wide)
        return y if k_beta is None else y + k_beta.to(wide)

    def rotary(y):
        y = y.clone()
        seg = y[..., off:off + rope].clone()
        rot = torch.cat((-seg[..., half:], seg[..., :half]), dim=-1)
        y[..., off:off + rope] = torch.where(inside, rot * sn + seg * cs, seg)
        return y

    q = x[:, :, :Hq]
    if norm_type == "layernorm":
        q = rotary(q)
        k = layernorm(rotary(x[:, :, Hq:Hq + Hk]))
    else:
        if q_gamma is not None:
            q = rmsnorm(q, q_gamma)
        q = rotary(q)
        k = rotary(rmsnorm(x[:, :, Hq:Hq + Hk], k_gamma))
    v = x[:, :, Hq + Hk:]
    q_out = qkv.clone()
    q_out[:, :, :Hq] = q.to(qkv.dtype)
    if linear is not None:  # linear caches [max_batch, Hk, cache_len, D], indexed directly
        bs_id, offs = linear
        for b in range(B):
            cb = int(bs_id[b]) if bs_id is not None else b
            for s_ in range(S):
                p = (int(offs[b]) if offs is not None else 0) + s_
                if not (0 <= cb < NB and 0 <= p < BS):
                    continue
                for t, c, sc in ((k, k_cache, k_scale), (v, v_cache, v_scale)):
                    row = t[b, s_]
                    if sc is None:
                        c[cb, :, p] = row.to(c.dtype)
                    elif sc.dim() == 3:
                        c[cb, :, p], sc[cb, :, p] = torch_row_quant(row.to(torch.float32))
                    else:
                        c[cb, :, p] = (row.to(torch.float32) / sc).round().clamp(-128, 127).to(torch.int8)
        return q_out
    flat = slot.reshape(-1)
    valid = (flat >= 0) & (flat < NB * BS)
    s_ = flat[valid].long()
    blk, o = s_ // BS, s_ % BS
    for t, c, sc in ((k, k_cache, k_scale), (v, v_cache, v_scale)):
        rows = t.reshape(B * S, Hk, D)[valid]
        if sc is None:
            c.permute(0, 2, 1, 3)[blk, o] = rows.to(c.dtype)
        elif sc.dim() == 3:
            codes, scale = torch_row_quant(rows.to(torch.float32))
            c.permute(0, 2, 1, 3)[blk, o] = codes
            sc.permute(0, 2, 1)[blk, o] = scale
        else:
            c.permute(0, 2, 1, 3)[blk, o] = (rows.to(torch.float32) / sc).round().clamp(-128, 127).to(torch.int8)
    return q_out


_frope_case = W.fused_rope_case


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("with_q_gamma", [True, False])
def test_fused_rope_matches_torch_bitwise(ref, dtype, mode, with_q_gamma):
    """The oracle against the torch-CPU restatement that uses D10's summation order: equal
    bit for bit (q written back, K/V pages, dynamic scales)."""
    for rope, off, D in ((128, 0, 128), (64, 32, 128), (32, 0, 64)):
        # B = 4 on the last shape: its fourth sequence runs past the sin/cos table
        qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = _frope_case(dtype, mode, 3, D=D, rope=rope,
                                                                       B=4 if D == 64 else 3)
        qg = qg if with_q_gamma else None
        want_kc, want_vc = kc.clone(), vc.clone()
        want_ks = ks.clone() if mode == "dynamic" else ks
        want_vs = vs.clone() if mode == "dynamic" else vs
        want_q = torch_fused_rope(qkv, want_kc, want_vc, sin, cos, pid, kg, want_ks, want_vs, slot,
                                  1e-5, qg, off)
        got = qkv.clone()
        ref.fused_rope_paged(got, kc, vc, sin, cos, pid, kg, ks, vs, slot, 1e-5, qg, off)
        assert torch.equal(bits(got), bits(want_q)), (rope, off)
        assert torch.equal(bits(kc), bits(want_kc)) and torch.equal(bits(vc), bits(want_vc))
        if mode == "dynamic":
            assert torch.equal(bits(ks), bits(want_ks)) and torch.equal(bits(vs), bits(want_vs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_rope_within_one_ulp_of_float64(ref, dtype):
    """Against the docstring computed in float64 (torch's own sum of squares): q and K differ
    by at most one ulp of the output type, and only rarely."""
    qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = _frope_case(dtype, "none", 9, B=3, S=30)
    want_kc, want_vc = kc.clone(), vc.clone()
    want_q = torch_fused_rope(qkv, want_kc, want_vc, sin, cos, pid, kg, None, None, slot, 1e-5, qg,
                              0, exact=False, wide=torch.float64)
    got = qkv.clone()
    ref.fused_rope_paged(got, kc, vc, sin, cos, pid, kg, None, None, slot, 1e-5, qg)
    for a, b in ((got, want_q), (kc, want_kc)):
        d = (bits(a).to(torch.int32) - bits(b).to(torch.int32)).abs()
        assert int(d.max()) <= 1
        assert float((d > 0).float().mean()) < 0.05


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("with_beta", [True, False])
def test_fused_rope_layernorm_matches_torch_bitwise(ref, dtype, mode, with_beta):
    """norm_type "layernorm" (D13): the oracle against the torch-CPU restatement in D13's
    summation order, bit for bit; q is rotated only (q_gamma is not used), a zero K row
    becomes beta (or zeros), V is stored unchanged."""
    for rope, off, D in ((128, 0, 128), (64, 32, 128), (32, 0, 64), (32, 8, 72)):
        qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = _frope_case(dtype, mode, 5, D=D, rope=rope,
                                                                       B=4 if D == 64 else 3)
        kb = (torch.rand(D, generator=torch.Generator().manual_seed(D)) - 0.5).to(dtype) \
            if with_beta else None
        want_kc, want_vc = kc.clone(), vc.clone()
        want_ks = ks.clone() if mode == "dynamic" else ks
        want_vs = vs.clone() if mode == "dynamic" else vs
        want_q = torch_fused_rope(qkv, want_kc, want_vc, sin, cos, pid, kg, want_ks, want_vs, slot,
                                  1e-5, None, off, norm_type="layernorm", k_beta=kb)
        got = qkv.clone()
        ref.fused_rope_paged(got, kc, vc, sin, cos, pid, kg, ks, vs, slot, 1e-5, None, off,
                             norm_type="layernorm", k_beta=kb)
        assert torch.equal(bits(got), bits(want_q)), (rope, off)
        assert torch.equal(bits(kc), bits(want_kc)) and torch.equal(bits(vc), bits(want_vc))
        if mode == "dynamic":
            assert torch.equal(bits(ks), bits(want_ks)) and torch.equal(bits(vs), bits(want_vs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_rope_layernorm_within_one_ulp_of_float64(ref, dtype):
    """norm_type "layernorm" against rotation + torch.nn.functional.layer_norm in float64: q
    and K at most one ulp of the output type apart, and rarely; for every stored K row of
    input scale >= 0.3 (eps then below 1e-3 of the variance), (y - beta) / gamma has mean ~0
    and variance ~1."""
    qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = _frope_case(dtype, "none", 11, B=3, S=30)
    kb = (torch.rand(128, generator=torch.Generator().manual_seed(3)) - 0.5).to(dtype)
    want_kc, want_vc = kc.clone(), vc.clone()
    want_q = torch_fused_rope(qkv, want_kc, want_vc, sin, cos, pid, kg, None, None, slot, 1e-5, None,
                              0, exact=False, wide=torch.float64, norm_type="layernorm", k_beta=kb)
    got = qkv.clone()
    ref.fused_rope_paged(got, kc, vc, sin, cos, pid, kg, None, None, slot, 1e-5, None,
                         norm_type="layernorm", k_beta=kb)
    for a, b in ((got, want_q), (kc, want_kc)):
        d = (bits(a).to(torch.int32) - bits(b).to(torch.int32)).abs()
        assert int(d.max()) <= 1
        assert float((d > 0).float().mean()) < 0.05
    flat = slot.reshape(-1)
    keep = (flat >= 0) & (torch.arange(flat.numel()) % 30 >= 15)   # torch.logspace(-2, 1, 30)[15] ~ 0.32
    rows = kc.permute(0, 2, 1, 3).reshape(-1, 2, 128)[flat[keep].long()].double()
    z = (rows - kb.double()) / kg.double()
    assert float(z.mean(-1).abs().max()) < 0.02
    assert float((z.var(-1, unbiased=False) - 1).abs().max()) < 0.03


@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("norm_type", ["rmsnorm", "layernorm"])
@pytest.mark.parametrize("ids", ["given", "default"])
def test_fused_rope_linear_matches_torch_indexing(ref, mode, norm_type, ids):
    """D14: linear caches through cache_bs_id / cache_seq_offsets.  The oracle's slot mapping
    against the torch restatement that indexes cache[cache_bs_id[b], :, offset[b] + s]
    directly: caches and scales equal bit for bit, rows of a -1 cache batch, a batch id past
    the cache and positions past cache_len not stored (their sentinel survives)."""
    qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, _ = _frope_case(torch.bfloat16, mode, 13, B=4, S=12)
    MB, L = 5, 30
    kc = torch.full((MB, 2, L, 128), 7, dtype=kc.dtype)
    vc = torch.full_like(kc, 9)
    if mode == "dynamic":
        ks, vs = torch.full((MB, 2, L), -1.0), torch.full((MB, 2, L), -1.0)
    if ids == "given":
        bs_id = torch.tensor([3, -1, 0, 7], dtype=torch.int32)   # 7: past the cache's 5 batches
        offs = torch.tensor([0, 4, 25, 10], dtype=torch.int32)   # 25 + 11 runs past cache_len
    else:
        bs_id = offs = None
    kb = torch.rand(128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16) \
        if norm_type == "layernorm" else None
    qg = qg if norm_type == "rmsnorm" else None
    want_kc, want_vc = kc.clone(), vc.clone()
    want_ks = ks.clone() if mode == "dynamic" else ks
    want_vs = vs.clone() if mode == "dynamic" else vs
    want_q = torch_fused_rope(qkv, want_kc, want_vc, sin, cos, pid, kg, want_ks, want_vs, None,
                              1e-5, qg, 0, norm_type=norm_type, k_beta=kb, linear=(bs_id, offs))
    got = qkv.clone()
    ref.fused_rope_linear(got, kc, vc, sin, cos, pid, kg, ks, vs, bs_id, offs, 1e-5, qg,
                          norm_type=norm_type, k_beta=kb)
    assert torch.equal(bits(got), bits(want_q))
    assert torch.equal(bits(kc), bits(want_kc)) and torch.equal(bits(vc), bits(want_vc))
    if mode == "dynamic":
        assert torch.equal(bits(ks), bits(want_ks)) and torch.equal(bits(vs), bits(want_vs))
    if ids == "given":
        assert bool((kc[1] == 7).all()) and bool((kc[4] == 7).all())  # no sequence maps there


# ---------------------------------------------------------------------------- linear caches (D11)

def _lin_segments(case, max_len, out_dir, block_tables=None, lens=None):
    """Per sequence: (token rows, cache batch / block per token, cache positions) of the tokens
    that are written, by the docstring math of _ops.py:1203-1206, 3663-3668, 3906-3909."""
    lens = case.lens if lens is None else lens
    rows = case.key.shape[0] * (case.key.shape[1] if case.key.dim() == 4 else 1)
    if out_dir:
        rows = case.key.shape[0] if case.key.dim() == 3 else rows
    starts = torch.cumsum(lens, 0) - lens            # exclusive prefix sums
    out = []
    for i in range(lens.numel()):
        n = min(int(lens[i]), max_len)
        if case.context_seq_offset is not None:
            start = int(case.context_seq_offset[i])
        elif out_dir or case.packed:
            start = int(starts[i])
        else:
            start = i * case.key.shape[1]
        j = torch.arange(n)
        r = start + j
        pos = j + (int(case.cache_seq_offset[i]) if case.cache_seq_offset is not None else 0)
        if block_tables is not None:
            L = case.cache_len
            col = pos // L
            ok = col < block_tables.shape[1]
            b = torch.where(ok, block_tables[i, col.clamp(max=block_tables.shape[1] - 1)].long(),
                            torch.full_like(col, -1))
            pos = pos % L
        else:
            b = torch.full_like(j, int(case.cache_bs_id[i]) if case.cache_bs_id is not None else i)
            b = torch.where(pos < case.cache_len, b, torch.full_like(b, -1))
        keep = (r >= 0) & (r < rows) & (b >= 0) & (b < case.cache_batch) & (pos >= 0)
        out.append((r[keep], b[keep], pos[keep]))
    return out


def torch_linear_write(case, op, kc, vc, ks=None, vs=None, kchan=None, vchan=None, smode=0,
                       groups=1, max_len=None):
    """Ops 0-2 (reshape / dynamic quant / static quant into the linear cache) by torch."""
    max_len = case.max_context_len if max_len is None else max_len
    segs = _lin_segments(case, max_len, out_dir=False)
    for x, c, sc, ch in ((case.key, kc, ks, kchan), (case.value, vc, vs, vchan)):
        x = x.reshape(-1, x.shape[-2], x.shape[-1])
        for r, b, pos in segs:
            if r.numel() == 0:
                continue
            rows = x[r]                                          # [n, H, D]
            if op == 0:
                c[b, :, pos] = rows
                continue
            xf = rows.to(torch.float32)
            if op == 1:
                n, H, D = rows.shape
                grp = xf.reshape(n, H, groups, D // groups)
                amax = rows.reshape(n, H, groups, D // groups).abs().amax(-1).to(torch.float32)
                if c.dtype == torch.int8:
                    scale = amax / 127.0
                    q = (grp / scale[..., None]).round().clamp(-128, 127)
                    q = torch.where(scale[..., None] == 0, torch.zeros_like(q), q)
                    codes = q.to(torch.int8).view(torch.uint8)
                else:
                    scale = amax / 448.0
                    q = (grp / scale[..., None]).clamp(-448, 448)
                    q = torch.where(scale[..., None] == 0, torch.zeros_like(q), q)
                    codes = q.to(torch.float8_e4m3fn).view(torch.uint8)
                c.view(torch.uint8)[b, :, pos] = codes.reshape(n, H, D)
                if sc.dim() == 4:
                    sc[b, :, pos] = scale
                else:
                    sc[b, :, pos] = scale[..., 0]
                continue
            if smode == 0:
                s = ch.to(torch.float32)[None]                          # [1, H, D]
            elif smode == 1:
                s = ch.to(torch.float32)[:, pos].transpose(0, 1)[..., None]  # [n, H, 1]
            else:
                s = torch.tensor(float(ch), dtype=torch.float32)
            q = xf / s
            if c.dtype == torch.int8:
                codes = q.round().clamp(-128, 127).to(torch.int8).view(torch.uint8)
            else:
                codes = q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
            c.view(torch.uint8)[b, :, pos] = codes


def torch_linear_read(case, op, key, value, kc, vc, ks=None, vs=None, smode=0, lens=None,
                      block_tables=None, max_len=None):
    """Ops 3-4 (dequant / copy out of the cache into token-major [T, H, D]) by torch."""
    lens = case.lens if lens is None else lens
    max_len = int(lens.max()) if max_len is None else max_len
    segs = _lin_segments(case, max_len, out_dir=True, block_tables=block_tables, lens=lens)
    for out, c, sc in ((key, kc, ks), (value, vc, vs)):
        if out is None:
            continue
        for r, b, pos in segs:
            if r.numel() == 0:
                continue
            rows = c[b, :, pos]                                   # [n, H, D]
            if op == 4:
                out[r] = rows
            else:
                s = sc[None] if smode == 0 else sc[b, :, pos][..., None]
                out[r] = (rows.to(torch.float32) * s).to(out.dtype)


def _lin_bits(t):
    return t.view(torch.uint8) if t.dtype in (torch.int8, torch.float8_e4m3fn) else bits(t)


LIN_CASES = [(p, o) for p in (True, False) for o in (False, True)]


@pytest.mark.parametrize("packed,offsets", LIN_CASES)
@pytest.mark.parametrize("dtype", DTYPES + [torch.int8])
def test_linear_reshape_matches_torch(ref, dtype, packed, offsets):
    case = W.linear_case(torch.float32, 11, packed=packed, offsets=offsets)
    if dtype == torch.int8:
        case.key = (case.key.clamp(-100, 100)).to(torch.int8)
        case.value = (case.value * 10).clamp(-100, 100).to(torch.int8)
    else:
        case.key, case.value = case.key.to(dtype), case.value.to(dtype)
    kc, vc = case.caches(dtype)
    want_k, want_v = kc.clone(), vc.clone()
    torch_linear_write(case, 0, want_k, want_v)
    ref.linear_cache(0, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset)
    assert torch.equal(_lin_bits(kc), _lin_bits(want_k)) and torch.equal(_lin_bits(vc), _lin_bits(want_v))
    # some rows were written and, with offsets, some were skipped
    assert not torch.equal(_lin_bits(kc), _lin_bits(case.caches(dtype)[0]))


@pytest.mark.parametrize("packed,offsets", LIN_CASES)
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("groups", [1, 4, 0])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_dynamic_quant_matches_torch(ref, dtype, groups, cache_dtype, packed, offsets):
    case = W.linear_case(dtype, 12, packed=packed, offsets=offsets)
    kc, vc = case.caches(cache_dtype)
    ks, vs = case.scales(groups)
    wk, wv, wks, wvs = kc.clone(), vc.clone(), ks.clone(), vs.clone()
    torch_linear_write(case, 1, wk, wv, wks, wvs, groups=max(groups, 1))
    ref.linear_cache(1, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks, value_scale=vs, groups=max(groups, 1))
    assert torch.equal(_lin_bits(kc), _lin_bits(wk)) and torch.equal(_lin_bits(vc), _lin_bits(wv))
    assert torch.equal(ks.view(torch.int32), wks.view(torch.int32))
    assert torch.equal(vs.view(torch.int32), wvs.view(torch.int32))


@pytest.mark.parametrize("smode", [0, 1, 2])
@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_static_quant_matches_torch(ref, dtype, cache_dtype, smode):
    case = W.linear_case(dtype, 13, packed=True, offsets=True)
    g = torch.Generator().manual_seed(5)
    H, D = case.key.shape[-2:]
    if smode == 0:
        kch, vch = 0.01 + 0.2 * torch.rand(H, D, generator=g), 0.02 + 0.1 * torch.rand(H, D, generator=g)
        kt = vt = 1.0
    elif smode == 1:
        kch = 0.01 + 0.2 * torch.rand(H, case.cache_len, generator=g)
        vch = 0.02 + 0.1 * torch.rand(H, case.cache_len, generator=g)
        kt = vt = 1.0
    else:
        kch, vch, kt, vt = None, None, 0.0371, 0.0523
    kc, vc = case.caches(cache_dtype)
    wk, wv = kc.clone(), vc.clone()
    torch_linear_write(case, 2, wk, wv, kchan=kch if smode < 2 else kt,
                       vchan=vch if smode < 2 else vt, smode=smode)
    ref.linear_cache(2, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=True, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_chan=kch, value_chan=vch, key_tensor=kt, value_tensor=vt, smode=smode)
    assert torch.equal(_lin_bits(kc), _lin_bits(wk)) and torch.equal(_lin_bits(vc), _lin_bits(wv))


def _filled_linear_cache(case, seed=21):
    g = torch.Generator().manual_seed(seed)
    H, D = case.key.shape[-2:]
    kc = torch.randint(-128, 128, (case.cache_batch, H, case.cache_len, D), generator=g,
                       dtype=torch.int8)
    vc = torch.randint(-128, 128, kc.shape, generator=g, dtype=torch.int8)
    kt = torch.rand(case.cache_batch, H, case.cache_len, generator=g) * 0.05
    vt = torch.rand(case.cache_batch, H, case.cache_len, generator=g) * 0.05
    kch = torch.rand(H, D, generator=g) * 0.05
    vch = torch.rand(H, D, generator=g) * 0.05
    return kc, vc, kt, vt, kch, vch


@pytest.mark.parametrize("offsets", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_dequant_matches_torch(ref, dtype, mode, offsets):
    case = W.linear_case(dtype, 14, packed=True, offsets=offsets)
    kc, vc, kt, vt, kch, vch = _filled_linear_cache(case)
    T = case.key.shape[0]
    H, D = case.key.shape[-2:]
    key = torch.full((T, H, D), -3.0, dtype=dtype)
    value = key.clone()
    wk, wv = key.clone(), value.clone()
    ks, vs = (kch, vch) if mode == 0 else (kt, vt)
    torch_linear_read(case, 3, wk, wv, kc, vc, ks, vs, smode=mode)
    ref.linear_cache(3, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset,
                     key_scale=kt if mode == 1 else None, value_scale=vt if mode == 1 else None,
                     key_chan=kch if mode == 0 else None, value_chan=vch if mode == 0 else None,
                     smode=mode)
    assert torch.equal(bits(key), bits(wk)) and torch.equal(bits(value), bits(wv))


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("dtype", DTYPES + [torch.int8])
def test_reshape_from_cache_matches_torch(ref, dtype, paged):
    case = W.linear_case(torch.float32, 15, packed=True, offsets=not paged)
    kc8, vc8 = _filled_linear_cache(case)[:2]
    kc, vc = (kc8, vc8) if dtype == torch.int8 else (kc8.to(dtype) / 7, vc8.to(dtype) / 3)
    T = case.key.shape[0]
    H, D = case.key.shape[-2:]
    key = torch.full((T, H, D), -3, dtype=dtype)
    value = key.clone()
    bt = None
    if paged:  # pages of cache_len rows: sequence i uses a column of shuffled pages (-1: unused)
        g = torch.Generator().manual_seed(3)
        L, MB = case.cache_len, 2
        case.cache_len = L // 4                                  # block_size 10
        kc = kc.reshape(case.cache_batch * 4, H, L // 4, D) if False else \
            kc[:, :, :L // 4 * 4].reshape(case.cache_batch, H, 4, L // 4, D).permute(0, 2, 1, 3, 4) \
            .reshape(case.cache_batch * 4, H, L // 4, D).contiguous()
        vc = vc[:, :, :L // 4 * 4].reshape(case.cache_batch, H, 4, L // 4, D).permute(0, 2, 1, 3, 4) \
            .reshape(case.cache_batch * 4, H, L // 4, D).contiguous()
        case.cache_batch *= 4
        MB = 3
        bt = torch.randperm(case.cache_batch, generator=g)[:case.lens.numel() * MB] \
            .reshape(-1, MB).to(torch.int32)
        bt[0, 2] = -1                                            # a missing page
    wk, wv = key.clone(), value.clone()
    torch_linear_read(case, 4, wk, wv, kc, vc, block_tables=bt)
    ref.linear_cache(4, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset, block_tables=bt)
    assert torch.equal(bits(key), bits(wk)) and torch.equal(bits(value), bits(wv))


def test_linear_round_trips(ref):
    """reshape_linear_cache then reshape_from_cache is the identity on the tokens it wrote;
    quant then dequant is within scale / 2 per element (closed forms, not restatements)."""
    case = W.linear_case(torch.bfloat16, 16, packed=True, offsets=False)
    kc, vc = case.caches(torch.bfloat16)
    ref.linear_cache(0, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=True)
    back_k = torch.zeros_like(case.key)
    back_v = torch.zeros_like(case.value)
    ref.linear_cache(4, back_k, back_v, kc, vc, case.lens, case.max_context_len)
    n = int(case.lens.sum())
    assert torch.equal(bits(back_k[:n]), bits(case.key[:n]))
    assert torch.equal(bits(back_v[:n]), bits(case.value[:n]))
    qk, qv = case.caches(torch.int8)
    ks, vs = case.scales()
    ref.linear_cache(1, case.key, case.value, qk, qv, case.context_lengths, case.max_context_len,
                     packed=True, key_scale=ks, value_scale=vs)
    deq = torch.zeros(case.key.shape, dtype=torch.float32)
    ref.linear_cache(3, deq, None, qk, None, case.lens, case.max_context_len, key_scale=ks, smode=1)
    starts = torch.cumsum(case.lens, 0) - case.lens
    for i, (s0, n_i) in enumerate(zip(starts.tolist(), case.lens.tolist())):
        x = case.key[s0:s0 + n_i].to(torch.float32)
        sc = ks[i, :, :n_i].transpose(0, 1)[..., None]
        # |x - code * s| <= s / 2 (1 + 2^-23), plus RN(code * s)'s half ulp <= 127 s 2^-24
        assert ((deq[s0:s0 + n_i] - x).abs() <= sc * (0.5 + 2.0 ** -15)).all()


def test_linear_max_context_len_truncates(ref):
    case = W.linear_case(torch.float16, 17, packed=True, offsets=True)
    kc, vc = case.caches(torch.float16)
    wk, wv = kc.clone(), vc.clone()
    torch_linear_write(case, 0, wk, wv, max_len=7)
    ref.linear_cache(0, case.key, case.value, kc, vc, case.context_lengths, 7, packed=True,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset)
    assert torch.equal(bits(kc), bits(wk)) and torch.equal(bits(vc), bits(wv))


# ---------------------------------------------------------------------------- 4-bit linear caches (D15)

def unpack_docstring(flat_bytes: torch.Tensor) -> torch.Tensor:
    """dequant_from_linear_cache's int4 unpack, as written in its Math block (_ops.py:3680-3682):
    unpack[0::2] = flat >> 4; unpack[1::2] = flat << 4 >> 4, on int8 tensors."""
    flat = flat_bytes.reshape(-1).view(torch.int8)
    out = torch.empty(flat.numel() * 2, dtype=torch.int8)
    out[0::2] = flat >> 4
    out[1::2] = flat << 4 >> 4
    return out


def torch_int4_codes(rows: torch.Tensor, groups: int = 1):
    """quant_to_linear_cache's math with quant_bit 4 (_ops.py:1728-1742) by torch: int_max =
    2^(4-1) - 1 = 7, scale = amax / 7, code = clip(round(x / scale), -8, 7); [n, H, D] ->
    (int8 codes [n, H, D], scales [n, H, groups])."""
    n, H, D = rows.shape
    xf = rows.to(torch.float32).reshape(n, H, groups, D // groups)
    amax = rows.reshape(n, H, groups, D // groups).abs().amax(-1).to(torch.float32)
    scale = amax / 7.0
    q = (xf / scale[..., None]).round().clamp(-8, 7)
    q = torch.where(scale[..., None] == 0, torch.zeros_like(q), q)
    return q.to(torch.int8).reshape(n, H, D), scale


def pack_pairs(codes: torch.Tensor) -> torch.Tensor:
    """Pairs along the last dim into bytes, the inverse of unpack_docstring: (even << 4) | (odd
    & 0xF)."""
    hi = codes[..., 0::2].to(torch.int16) << 4
    lo = codes[..., 1::2].to(torch.int16) & 0xF
    return ((hi | lo) & 0xFF).to(torch.uint8)


def torch_linear_write4(case, kc, vc, ks, vs, groups=1):
    """D15 write by torch: K rows packed along channels; V codes placed by cache position into
    the nibble of byte [pos // 2, d] (even position: high nibble), the other nibble kept."""
    segs = _lin_segments(case, case.max_context_len, out_dir=False)
    k = case.key.reshape(-1, *case.key.shape[-2:])
    v = case.value.reshape(-1, *case.value.shape[-2:])
    kb, vb = kc.view(torch.uint8), vc.view(torch.uint8)
    for r, b, pos in segs:
        if r.numel() == 0:
            continue
        codes, scale = torch_int4_codes(k[r], groups)
        kb[b, :, pos] = pack_pairs(codes)
        ks[b, :, pos] = scale if ks.dim() == 4 else scale[..., 0]
        codes, scale = torch_int4_codes(v[r], groups)
        vs[b, :, pos] = scale if vs.dim() == 4 else scale[..., 0]
        for t in range(r.numel()):
            bt, pt = int(b[t]), int(pos[t])
            old = vb[bt, :, pt // 2].to(torch.int16)
            c = codes[t].to(torch.int16) & 0xF
            new = (old & 0xF0) | c if pt % 2 else (old & 0x0F) | (c << 4)
            vb[bt, :, pt // 2] = new.to(torch.uint8)


@pytest.mark.parametrize("packed,offsets", LIN_CASES)
@pytest.mark.parametrize("groups", [1, 4])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_int4_quant_matches_torch(ref, dtype, groups, packed, offsets):
    case = W.linear_case(dtype, 31, packed=packed, offsets=offsets)
    H, D = case.key.shape[-2:]
    kc = torch.full((case.cache_batch, H, case.cache_len, D // 2), 0x5A, dtype=torch.uint8).view(torch.int8)
    vc = torch.full((case.cache_batch, H, case.cache_len // 2, D), 0x5A, dtype=torch.uint8).view(torch.int8)
    ks, vs = case.scales(groups if groups > 1 else 0)
    wk, wv, wks, wvs = kc.clone(), vc.clone(), ks.clone(), vs.clone()
    torch_linear_write4(case, wk, wv, wks, wvs, groups)
    ref.linear_cache(1, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=packed, context_seq_offset=case.context_seq_offset,
                     cache_bs_id=case.cache_bs_id, cache_seq_offset=case.cache_seq_offset,
                     key_scale=ks, value_scale=vs, groups=groups, bits=4)
    assert torch.equal(kc, wk) and torch.equal(vc, wv)
    assert torch.equal(ks.view(torch.int32), wks.view(torch.int32))
    assert torch.equal(vs.view(torch.int32), wvs.view(torch.int32))
    assert not torch.equal(kc, torch.full_like(kc, 0x5A))


@pytest.mark.parametrize("offsets", [False, True])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_int4_dequant_matches_docstring(ref, dtype, mode, offsets):
    """The K side executes the reference's own unpack expression on each cache row; V applies
    the same unpack along its packed dimension (position pairs of one channel)."""
    case = W.linear_case(dtype, 32, packed=True, offsets=offsets)
    g = torch.Generator().manual_seed(33)
    H, D = case.key.shape[-2:]
    L = case.cache_len
    kc = torch.randint(-128, 128, (case.cache_batch, H, L, D // 2), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (case.cache_batch, H, L // 2, D), generator=g, dtype=torch.int8)
    kt = torch.rand(case.cache_batch, H, L, generator=g) * 0.05
    vt = torch.rand(case.cache_batch, H, L, generator=g) * 0.05
    kch, vch = torch.rand(H, D, generator=g) * 0.05, torch.rand(H, D, generator=g) * 0.05
    T = case.key.shape[0]
    key = torch.full((T, H, D), -3.0, dtype=dtype)
    value = key.clone()
    wk, wv = key.clone(), value.clone()
    # unpacked caches by the docstring's expression: K per row, V along positions per channel
    ku = unpack_docstring(kc).reshape(case.cache_batch, H, L, D)
    vu = unpack_docstring(vc.permute(0, 1, 3, 2).contiguous()) \
        .reshape(case.cache_batch, H, D, L).permute(0, 1, 3, 2)
    torch_linear_read(case, 3, wk, wv, ku, vu, kch if mode == 0 else kt, vch if mode == 0 else vt,
                      smode=mode)
    ref.linear_cache(3, key, value, kc, vc, case.lens, case.max_context_len,
                     context_seq_offset=case.context_seq_offset, cache_bs_id=case.cache_bs_id,
                     cache_seq_offset=case.cache_seq_offset,
                     key_scale=kt if mode == 1 else None, value_scale=vt if mode == 1 else None,
                     key_chan=kch if mode == 0 else None, value_chan=vch if mode == 0 else None,
                     smode=mode, bits=4)
    assert torch.equal(bits(key), bits(wk)) and torch.equal(bits(value), bits(wv))


def test_linear_int4_round_trip_and_closed_forms(ref):
    """quant (4 bit) then dequant: |x - deq| <= scale / 2 per element; codes stay in [-7, 7]
    (|x| <= amax bounds |x / scale| by 7) and the largest element of a row reaches +-7; writing
    from an odd cache position keeps the other nibble of the first V byte."""
    case = W.linear_case(torch.bfloat16, 34, packed=True, offsets=False)
    H, D = case.key.shape[-2:]
    L = case.cache_len
    kc = torch.zeros((case.cache_batch, H, L, D // 2), dtype=torch.int8)
    vc = torch.full((case.cache_batch, H, L // 2, D), 0x5A, dtype=torch.uint8).view(torch.int8)
    ks, vs = case.scales()
    case.cache_seq_offset = torch.ones(case.lens.numel(), dtype=torch.int32)   # odd first position
    ref.linear_cache(1, case.key, case.value, kc, vc, case.context_lengths, case.max_context_len,
                     packed=True, cache_seq_offset=case.cache_seq_offset, key_scale=ks,
                     value_scale=vs, bits=4)
    # byte 0 of every written sequence's V rows: its high nibble (position 0) untouched
    for i, n in enumerate(case.lens.tolist()):
        if n:
            assert torch.equal((vc[i, :, 0].view(torch.uint8) >> 4), torch.full((H, D), 5, dtype=torch.uint8))
    ku = unpack_docstring(kc).reshape(case.cache_batch, H, L, D)
    assert int(ku.min()) >= -7 and int(ku.max()) <= 7
    deq_k = torch.zeros(case.key.shape, dtype=torch.float32)
    deq_v = torch.zeros(case.key.shape, dtype=torch.float32)
    ref.linear_cache(3, deq_k, deq_v, kc, vc, case.lens, case.max_context_len,
                     cache_seq_offset=case.cache_seq_offset, key_scale=ks, value_scale=vs,
                     smode=1, bits=4)
    starts = torch.cumsum(case.lens, 0) - case.lens
    for i, (s0, n_i) in enumerate(zip(starts.tolist(), case.lens.tolist())):
        for x, deq, sc in ((case.key, deq_k, ks), (case.value, deq_v, vs)):
            xs = x[s0:s0 + n_i].to(torch.float32)
            s = sc[i, :, 1:1 + n_i].transpose(0, 1)[..., None]
            assert ((deq[s0:s0 + n_i] - xs).abs() <= s * (0.5 + 2.0 ** -15)).all()
            # the row maximum maps to +-7 exactly: |deq| == 7 * scale there
            top = xs.abs().argmax(-1, keepdim=True)
            got = deq[s0:s0 + n_i].gather(-1, top).abs()
            assert torch.equal(got, (7 * s).to(torch.float32)) or (s == 0).all()


# ---------------------------------------------------------------------------- decode attention (D12)

def torch_attn(case, scale, window=-1):
    """_ops.py:786-800 in float64 by torch: gather each sequence's keys through its block table,
    dequantise (code * scale), repeat KV heads over their query-head group, softmax, @ V."""
    q, kc, vc = case.q.double(), case.k_cache, case.v_cache
    B, Hq, D = q.shape
    NB, Hkv, BS, _ = kc.shape
    g = Hq // Hkv
    out = torch.zeros(B, Hq, D, dtype=torch.float64)
    lse = torch.full((B, Hq), float("-inf"), dtype=torch.float64)
    for i in range(B):
        L = int(case.context_lens[i])
        j = torch.arange(L)
        if window >= 0:
            j = j[j >= L - 1 - window]
        blk = case.block_tables[i, j // BS].long()
        row = j % BS
        keep = (blk >= 0) & (blk < NB)
        j, blk, row = j[keep], blk[keep], row[keep]
        if j.numel() == 0:
            continue
        K, V = kc[blk, :, row].double(), vc[blk, :, row].double()        # [n, Hkv, D]
        if case.k_scale is not None:
            if case.k_scale.dim() == 3:
                K = K * case.k_scale[blk, :, row].double()[..., None]
                V = V * case.v_scale[blk, :, row].double()[..., None]
            else:
                K = K * case.k_scale.double()[None]
                V = V * case.v_scale.double()[None]
        K, V = K.repeat_interleave(g, dim=1), V.repeat_interleave(g, dim=1)  # [n, Hq, D]
        s = (K * q[i][None]).sum(-1).transpose(0, 1) * scale                 # [Hq, n]
        if case.alibi is not None:
            s = s + case.alibi[i].double()[:, None] * (j - (L - 1)).double()[None, :]
        p = torch.softmax(s, dim=-1)
        out[i] = (p[:, :, None] * V.transpose(0, 1)).sum(1)
        lse[i] = torch.logsumexp(s, dim=-1)
    return out, lse


@pytest.mark.parametrize("kv", ["fp8_token", "fp8_channel", "int8_token", "int8_channel"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attn_fp8_pages_and_bf16_scales_match_torch_float64(ref, dtype, kv):
    """float8_e4m3fn caches (_ops.py:868) and bf16 scales (_ops.py:872): the docstring math in
    float64 by torch -- the e4m3fn value (torch's exact cast) times the widened bf16 scale --
    against the oracle, with a missing page, a window and ALiBi."""
    case = W.attn_case(dtype, 31, kv=kv, Hq=8, Hkv=2, D=64, max_ctx=70,
                       scale_dtype=torch.bfloat16)
    case.block_tables[2, 1] = -1
    for window, alibi in ((-1, False), (9, False), (-1, True)):
        case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1) if alibi else None
        out, lse = ref.single_query_attn(case.q, case.k_cache, case.v_cache, case.block_tables,
                                         case.context_lens, 0.125, case.k_scale, case.v_scale,
                                         case.alibi, window)
        want, wlse = torch_attn(case, 0.125, window)
        assert torch.allclose(out, want, rtol=1e-12, atol=1e-12)
        assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12)
    # the fp8 pages are read as their values: an fp8 cache holding x and an fp32 one holding
    # the same numbers give the same result
    if kv.startswith("fp8"):
        plain = W.AttnCase(case.q, case.k_cache.to(torch.float32), case.v_cache.to(torch.float32),
                           None, None, case.block_tables, case.context_lens)
        fold = (lambda c, s: c * (s.float()[..., None] if s.dim() == 3 else s.float()[None, :, None, :]))
        plain.k_cache = fold(plain.k_cache, case.k_scale)
        plain.v_cache = fold(plain.v_cache, case.v_scale)
        case.alibi = None
        out, _ = ref.single_query_attn(case.q, case.k_cache, case.v_cache, case.block_tables,
                                       case.context_lens, 0.125, case.k_scale, case.v_scale)
        want, _ = torch_attn(plain, 0.125)
        assert torch.allclose(out, want, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_attn_matches_torch_float64(ref, dtype, kv):
    case = W.attn_case(dtype, 3, kv=kv, Hq=8, Hkv=2, D=64, max_ctx=70)
    case.block_tables[2, 1] = -1                     # a missing page: its keys are masked
    for window, alibi in ((-1, False), (9, False), (-1, True)):
        case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1) if alibi else None
        out, lse = ref.single_query_attn(case.q, case.k_cache, case.v_cache, case.block_tables,
                                         case.context_lens, 0.125, case.k_scale, case.v_scale,
                                         case.alibi, window)
        want, wlse = torch_attn(case, 0.125, window)
        assert torch.allclose(out, want, rtol=1e-12, atol=1e-12)
        assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12)


def test_attn_closed_forms(ref):
    """One key: out = that key's value row exactly, lse = its logit.  A window of 0: the last
    key's value.  Identical keys: the mean of the value rows.  A dominant ALiBi slope: the last
    value row."""
    case = W.attn_case(torch.bfloat16, 4, kv="int8_token", B=3, Hq=4, Hkv=4, D=32, max_ctx=40)
    NB, Hkv, BS, D = case.k_cache.shape
    out, lse = ref.single_query_attn(case.q, case.k_cache, case.v_cache, case.block_tables,
                                     case.context_lens, 0.3, case.k_scale, case.v_scale)
    blk = int(case.block_tables[1, 0])                               # sequence 1 has one key
    v0 = case.v_cache[blk, :, 0].double() * case.v_scale[blk, :, 0].double()[:, None]
    assert torch.equal(out[1], v0)
    k0 = case.k_cache[blk, :, 0].double() * case.k_scale[blk, :, 0].double()[:, None]
    assert torch.allclose(lse[1], 0.3 * (case.q[1].double() * k0).sum(-1), rtol=1e-14)
    out, _ = ref.single_query_attn(case.q, case.k_cache, case.v_cache, case.block_tables,
                                   case.context_lens, 0.3, case.k_scale, case.v_scale,
                                   window_left=0)
    L = int(case.context_lens[0])
    blk, row = int(case.block_tables[0, (L - 1) // BS]), (L - 1) % BS
    vl = case.v_cache[blk, :, row].double() * case.v_scale[blk, :, row].double()[:, None]
    assert torch.equal(out[0], vl)
    same = W.attn_case(torch.float32, 5, kv="plain", B=1, Hq=2, Hkv=1, D=16, max_ctx=33)
    same.k_cache[:] = same.k_cache[0, :, 0][None, :, None, :]
    out, _ = ref.single_query_attn(same.q, same.k_cache, same.v_cache, same.block_tables,
                                   same.context_lens, 1.0)
    bt = same.block_tables[0]
    j = torch.arange(33)
    V = same.v_cache[bt[j // 16].long(), :, j % 16].double()          # [33, 1, 16]
    assert torch.allclose(out[0], V.mean(0).expand(2, 16), rtol=1e-13, atol=1e-15)
    al = torch.full((1, 2), 1e4)
    out, _ = ref.single_query_attn(same.q, same.k_cache, same.v_cache, same.block_tables,
                                   same.context_lens, 1.0, alibi_slopes=al)
    assert torch.allclose(out[0], V[-1].expand(2, 16), rtol=0, atol=1e-300)


def torch_attn_mq(case, q, scale, window=-1, cu=None, sink=None, Dv=None, mask=None):
    """_ops.py:786-800 for several query tokens per sequence, in float64 by torch: every
    sequence's keys dequantised through its block table, a [heads, tokens, keys] logit matrix
    with query token s of nq at position P = L - nq + s seeing keys j in [P - window, P], ALiBi
    slope * (j - P), the sink as an extra logit column whose value row is zero.  q [B, S, Hq,
    D], or [T, Hq, D] with cu [B + 1]; keys the first D channels of k_cache rows, values the
    first Dv of v_cache rows (k_cache's when v_cache is None); mask [B, S, mask_len] adds
    mask[i, s, m] to key L - mask_len + m of token s (decision D16); returns out / lse shaped
    like q's leading dims (rows of no sequence NaN)."""
    kc, bt = case.k_cache, case.block_tables
    vc = kc if case.v_cache is None else case.v_cache
    NB, Hkv, BS, _ = kc.shape
    D = q.shape[-1]
    Dv = Dv or (D if case.v_cache is None else vc.shape[3])
    B = case.context_lens.shape[0]
    Hq = q.shape[-2]
    g = Hq // Hkv
    qf = q.reshape(-1, Hq, D).double()
    T = qf.shape[0]
    out = torch.full((T, Hq, Dv), float("nan"), dtype=torch.float64)
    lse = torch.full((T, Hq), float("nan"), dtype=torch.float64)
    for i in range(B):
        r0, nq = (i * q.shape[1], q.shape[1]) if cu is None else (int(cu[i]), int(cu[i + 1] - cu[i]))
        if nq <= 0:
            continue
        L = min(int(case.context_lens[i]), bt.shape[1] * BS)
        j = torch.arange(max(L, 0))
        blk, row = bt[i, j // BS].long(), j % BS
        keep = (blk >= 0) & (blk < NB)
        K = torch.zeros(j.numel(), Hkv, D, dtype=torch.float64)
        V = torch.zeros(j.numel(), Hkv, Dv, dtype=torch.float64)
        b, r = blk[keep], row[keep]
        K[keep], V[keep] = kc[b, :, r, :D].double(), vc[b, :, r, :Dv].double()
        ks, vs = case.k_scale, case.v_scale
        if ks is not None:
            if ks.dim() == 4 and ks.shape[3] == 1:
                ks, vs = ks[..., 0], vs[..., 0]
            if ks.dim() == 3:                                   # per token
                K[keep] *= ks[b, :, r].double()[..., None]
                V[keep] *= vs[b, :, r].double()[..., None]
            elif ks.dim() == 2:                                 # per channel
                K[keep] *= ks.double()[None]
                V[keep] *= vs.double()[None]
            else:                                               # per group of 32
                K[keep] *= ks[b, :, r].double().repeat_interleave(32, dim=-1)
                V[keep] *= vs[b, :, r // 32].double()
        K, V = K.repeat_interleave(g, dim=1), V.repeat_interleave(g, dim=1)   # [L, Hq, D]
        s = torch.einsum("thd,jhd->htj", qf[r0:r0 + nq], K) * scale             # [Hq, nq, L]
        P = L - nq + torch.arange(nq)
        if case.alibi is not None:
            s = s + case.alibi[i].double()[:, None, None] * (j[None, :] - P[:, None]).double()[None]
        if mask is not None:
            col = j - (L - mask.shape[2])
            sel = col >= 0
            add = torch.zeros(nq, j.numel(), dtype=torch.float64)
            add[:, sel] = mask[i, :nq][:, col[sel]].double()
            s = s + add[None]
        ok = (j[None, :] <= P[:, None]) & keep[None, :]
        if window >= 0:
            ok &= j[None, :] >= P[:, None] - window
        s = s.masked_fill(~ok[None], float("-inf"))
        if sink is not None:
            s = torch.cat([s, sink.double()[:, None, None].expand(Hq, nq, 1)], dim=-1)
            V = torch.cat([V, torch.zeros(1, Hq, Dv, dtype=torch.float64)], dim=0)
        l = torch.logsumexp(s, dim=-1)                                           # [Hq, nq]
        p = torch.exp(s - l[..., None]).nan_to_num(0.0)
        out[r0:r0 + nq] = torch.einsum("htj,jhd->thd", p, V)
        lse[r0:r0 + nq] = l.transpose(0, 1)
    if cu is None:
        return out.reshape(q.shape[:2] + (Hq, Dv)), lse.reshape(q.shape[:2] + (Hq,))
    return out, lse


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "plain"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_attn_multi_token_matches_torch_float64(ref, dtype, kv):
    """Several query tokens per sequence (4-D q, and 3-D q with cu_seq_q, ragged with an empty
    sequence), with windows, ALiBi, a sink and a missing page, against torch in float64."""
    case = W.attn_case(dtype, 11, kv=kv, Hq=8, Hkv=2, D=64, max_ctx=70)
    case.block_tables[2, 1] = -1
    q4 = W.attn_queries(dtype, 12, B=5, Hq=8, D=64, S=3)
    q3, cu = W.attn_queries(dtype, 13, B=5, Hq=8, D=64, counts=[4, 2, 0, 7, 1])
    sink = torch.tensor([0.5, -1.0, 3.0, 0.0, -20.0, 1.5, 2.0, -0.25])
    for window, alibi, sk in ((-1, False, None), (9, False, sink), (-1, True, sink), (0, True, None)):
        case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1) if alibi else None
        for q, c in ((q4, None), (q3, cu)):
            out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                          case.context_lens, 0.125, case.k_scale, case.v_scale,
                                          case.alibi, window, cu_seq_q=c, sink=sk)
            want, wlse = torch_attn_mq(case, q, 0.125, window, c, sk)
            assert torch.allclose(out, want, rtol=1e-12, atol=1e-12)
            assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12)


def test_attn_multi_token_forms(ref):
    """Token s of nq equals one query token against the first L - nq + s + 1 keys (the causal
    rule), bit for bit; ragged cu_seq_q rows equal the per-sequence 4-D calls; the sink scales
    the output by Z / (Z + e^sink) and adds e^sink under the lse's log; a token with no key
    gives out 0 and lse = sink; rows of no sequence stay untouched."""
    case = W.attn_case(torch.bfloat16, 21, kv="int8_token", B=4, Hq=8, Hkv=2, D=32, max_ctx=50,
                       alibi=True)
    S = 4
    q4 = W.attn_queries(torch.bfloat16, 22, B=4, Hq=8, D=32, S=S)
    for window in (-1, 5):
        out, lse = ref.cached_kv_attn(q4, case.k_cache, case.v_cache, case.block_tables,
                                      case.context_lens, 0.2, case.k_scale, case.v_scale,
                                      case.alibi, window)
        for s in range(S):
            lens_s = (case.context_lens - S + s + 1).clamp(min=0)
            o1, l1 = ref.single_query_attn(q4[:, s], case.k_cache, case.v_cache,
                                           case.block_tables, lens_s, 0.2, case.k_scale,
                                           case.v_scale, case.alibi, window)
            assert torch.equal(out[:, s], o1) and torch.equal(lse[:, s], l1)
    # sequence 1 holds one key: its first three tokens see none
    assert (out[1, :3] == 0).all() and (lse[1, :3] == float("-inf")).all()
    sink = torch.linspace(-3.0, 4.0, 8)
    o_s, l_s = ref.cached_kv_attn(q4, case.k_cache, case.v_cache, case.block_tables,
                                  case.context_lens, 0.2, case.k_scale, case.v_scale, case.alibi,
                                  sink=sink)
    o_0, l_0 = ref.cached_kv_attn(q4, case.k_cache, case.v_cache, case.block_tables,
                                  case.context_lens, 0.2, case.k_scale, case.v_scale, case.alibi)
    live = l_0 > float("-inf")
    sk = sink.double().expand_as(l_0)
    assert torch.allclose(l_s[live], torch.logaddexp(l_0, sk)[live], rtol=1e-14)
    assert torch.allclose(o_s[live], (o_0 * torch.exp(l_0 - l_s)[..., None])[live], rtol=1e-13,
                          atol=1e-15)
    assert (o_s[~live] == 0).all() and torch.equal(l_s[~live], sk[~live])
    counts = [3, 0, 5, 1]
    q3, cu = W.attn_queries(torch.bfloat16, 23, B=4, Hq=8, D=32, counts=counts)
    q3 = torch.cat([q3, q3[:2]])                                  # two rows of no sequence
    out, lse = ref.cached_kv_attn(q3, case.k_cache, case.v_cache, case.block_tables,
                                  case.context_lens, 0.2, case.k_scale, case.v_scale,
                                  case.alibi, 7, cu_seq_q=cu, sink=sink)
    for i, n in enumerate(counts):
        if n == 0:
            continue
        a, b = int(cu[i]), int(cu[i + 1])
        o1, l1 = ref.cached_kv_attn(q3[a:b][None], case.k_cache, case.v_cache,
                                    case.block_tables[i:i + 1], case.context_lens[i:i + 1], 0.2,
                                    case.k_scale, case.v_scale, case.alibi[i:i + 1], 7,
                                    sink=sink)
        assert torch.equal(out[a:b], o1[0]) and torch.equal(lse[a:b], l1[0])
    assert out[-2:].isnan().all() and lse[-2:].isnan().all()


def _shared_cache(case, D, Dv, seed):
    """The case's K cache widened to max(D, Dv) channels (new channels random), V dropped: the
    value is the first Dv channels of each K row (_ops.py:828-831)."""
    g = torch.Generator().manual_seed(seed)
    NB, Hkv, BS, Dk = case.k_cache.shape
    W_ = max(D, Dv)
    if case.k_cache.dtype == torch.int8:
        extra = torch.randint(-127, 128, (NB, Hkv, BS, W_ - Dk), generator=g, dtype=torch.int8)
    else:
        extra = torch.randn(NB, Hkv, BS, W_ - Dk, generator=g).to(case.k_cache.dtype)
    return W.AttnCase(case.q, torch.cat([case.k_cache, extra], dim=-1), None, case.k_scale,
                      case.v_scale, case.block_tables, case.context_lens, case.alibi)


@pytest.mark.parametrize("kv", ["int8_token", "int8_channel", "int8_group", "plain"])
def test_attn_cache_forms_match_torch_float64(ref, kv):
    """K and V in one cache (v_cache None, value head size below, equal to or above the key's),
    separate caches of different head sizes, per-group scales, per-token scales with strides
    in the first two dims -- against torch in float64."""
    D = 64
    case = W.attn_case(torch.bfloat16, 51, kv=kv, B=4, Hq=8, Hkv=2, D=D, BS=32, NB=24,
                       max_ctx=150)
    q = W.attn_queries(torch.bfloat16, 52, B=4, Hq=8, D=D, S=2)
    sink = torch.linspace(-1.0, 2.0, 8)
    for Dv in (32, 64, 96):
        if kv == "int8_channel" and Dv != D:
            continue                       # per-channel V scales are [Hkv, Dv]: built below
        if kv == "int8_group" and Dv > D:
            continue
        sh = _shared_cache(case, D, Dv, 53)
        if kv == "int8_group":
            sh.v_scale = case.v_scale[..., :Dv].contiguous()
        out, lse = ref.cached_kv_attn(q, sh.k_cache, None, sh.block_tables, sh.context_lens,
                                      0.125, sh.k_scale, sh.v_scale, None, -1, sink=sink,
                                      head_size_v=Dv)
        want, wlse = torch_attn_mq(sh, q, 0.125, sink=sink, Dv=Dv)
        assert torch.allclose(out, want, rtol=1e-12, atol=1e-12)
        assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12)
    if kv in ("int8_token", "plain"):      # separate V cache of 40 channels
        vc = case.v_cache[..., :40].contiguous()
        c2 = W.AttnCase(case.q, case.k_cache, vc, case.k_scale, case.v_scale, case.block_tables,
                        case.context_lens)
        out, _ = ref.cached_kv_attn(q, c2.k_cache, vc, c2.block_tables, c2.context_lens, 0.125,
                                    c2.k_scale, c2.v_scale)
        want, _ = torch_attn_mq(c2, q, 0.125)
        assert out.shape[-1] == 40 and torch.allclose(out, want, rtol=1e-12, atol=1e-12)
    if kv == "int8_token":                 # strided per-token scales
        NB, Hkv, BS = case.k_scale.shape
        big = torch.rand(Hkv, NB, BS + 7, generator=torch.Generator().manual_seed(54))
        big[:, :, :BS] = case.k_scale.transpose(0, 1)
        ks = big.transpose(0, 1)[:, :, :BS]                  # strides (BS + 7, NB (BS + 7), 1)
        assert not ks.is_contiguous()
        out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                      case.context_lens, 0.125, ks, case.v_scale[..., None])
        o0, l0 = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                    case.context_lens, 0.125, case.k_scale, case.v_scale)
        assert torch.equal(out, o0) and torch.equal(lse, l0)


def test_attn_cache_form_identities(ref):
    """v_cache None with equal head sizes is v_cache = k_cache; per-group scales equal across
    a token's groups (K) and across a 32-row group's channels (V) give the per-token result bit
    for bit."""
    case = W.attn_case(torch.float16, 55, kv="int8_token", B=3, Hq=8, Hkv=2, D=64, BS=32,
                       NB=16, max_ctx=120)
    q = W.attn_queries(torch.float16, 56, B=3, Hq=8, D=64, S=3)
    a = ref.cached_kv_attn(q, case.k_cache, None, case.block_tables, case.context_lens, 0.1,
                           case.k_scale, case.v_scale)
    b = ref.cached_kv_attn(q, case.k_cache, case.k_cache, case.block_tables, case.context_lens,
                           0.1, case.k_scale, case.v_scale)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    NB, Hkv, BS = case.k_scale.shape
    vs_tok = case.v_scale.reshape(NB, Hkv, BS // 32, 32)[..., :1].expand(NB, Hkv, BS // 32, 32)
    vs_tok = vs_tok.reshape(NB, Hkv, BS).contiguous()          # constant over 32-row groups
    ks_grp = case.k_scale[..., None].expand(NB, Hkv, BS, 2).contiguous()
    vs_grp = vs_tok.reshape(NB, Hkv, BS // 32, 32)[..., 0:1].expand(NB, Hkv, BS // 32, 64).contiguous()
    a = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                           0.1, ks_grp, vs_grp)
    b = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                           0.1, case.k_scale, vs_tok)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------- int4 caches, mask (D16)

def _unpack_ref(b: torch.Tensor, dim: int) -> torch.Tensor:
    """The reference's own unpack expression on int8 bytes (_ops.py:3681-3682:
    `unpack[0::2] = byte >> 4; unpack[1::2] = byte << 4 >> 4`), pairs along `dim`."""
    b = b.movedim(dim, -1)
    out = torch.empty(b.shape[:-1] + (2 * b.shape[-1],), dtype=torch.int8)
    out[..., 0::2] = b >> 4
    out[..., 1::2] = b << 4 >> 4
    return out.movedim(-1, dim).contiguous()


def _int4_codes(case, v_pairs):
    """The case with its int4 pages unpacked by the reference's expression: int8 codes."""
    kc = _unpack_ref(case.k_cache, 3)
    vc = _unpack_ref(case.v_cache, 2 if v_pairs == "rows" else 3)
    return W.AttnCase(case.q, kc, vc, case.k_scale, case.v_scale, case.block_tables,
                      case.context_lens, case.alibi)


@pytest.mark.parametrize("v_pairs", ["rows", "channels"])
@pytest.mark.parametrize("kv", ["int4_token", "int4_channel", "int4_group"])
def test_attn_int4_matches_torch_float64(ref, kv, v_pairs):
    """int4 caches (kv_cache_quant_bit_size 4, _ops.py:826-829, 852): the pages unpacked by the
    reference's own expression, dequantised and attended in float64 by torch, against the
    oracle reading the packed pages -- V pairing rows ([NB, Hkv, BS / 2, Dv]) and channels
    ([NB, Hkv, BS, Dv / 2]); several query tokens, windows, ALiBi, a sink, a missing page."""
    BS = 32 if kv == "int4_group" else 16
    case = W.attn_case(torch.bfloat16, 61, kv=kv, Hq=8, Hkv=2, D=64, BS=BS, max_ctx=70,
                       v_pairs=v_pairs)
    case.block_tables[2, 1] = -1
    codes = _int4_codes(case, v_pairs)
    q4 = W.attn_queries(torch.bfloat16, 62, B=5, Hq=8, D=64, S=3)
    q3, cu = W.attn_queries(torch.bfloat16, 63, B=5, Hq=8, D=64, counts=[4, 2, 0, 7, 1])
    sink = torch.linspace(-2.0, 1.0, 8)
    for window, alibi, sk in ((-1, False, None), (9, False, sink), (-1, True, sink)):
        al = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1) if alibi else None
        case.alibi = codes.alibi = al
        for q, c in ((q4, None), (q3, cu)):
            out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                          case.context_lens, 0.125, case.k_scale, case.v_scale,
                                          al, window, cu_seq_q=c, sink=sk, int4=True)
            want, wlse = torch_attn_mq(codes, q, 0.125, window, c, sk)
            assert out.shape == want.shape
            assert torch.allclose(out, want, rtol=1e-12, atol=1e-12, equal_nan=True)
            assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12, equal_nan=True)


def test_attn_int4_identities(ref):
    """An int4 cache equals the int8 cache of its unpacked codes bit for bit (the codes are
    read, nothing else changes); the two V layouts of the same codes agree bit for bit."""
    rows = W.attn_case(torch.float16, 64, kv="int4_token", B=4, Hq=4, Hkv=2, D=32, max_ctx=60)
    codes = _int4_codes(rows, "rows")
    vch = W.pack_int4(codes.v_cache, 3)
    q = W.attn_queries(torch.float16, 65, B=4, Hq=4, D=32, S=2)
    a = ref.cached_kv_attn(q, rows.k_cache, rows.v_cache, rows.block_tables, rows.context_lens,
                           0.2, rows.k_scale, rows.v_scale, int4=True)
    b = ref.cached_kv_attn(q, codes.k_cache, codes.v_cache, rows.block_tables,
                           rows.context_lens, 0.2, rows.k_scale, rows.v_scale)
    c = ref.cached_kv_attn(q, rows.k_cache, vch, rows.block_tables, rows.context_lens, 0.2,
                           rows.k_scale, rows.v_scale, int4=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(a[0], c[0]) and torch.equal(a[1], c[1])
    assert int(codes.k_cache.min()) == -8 and int(codes.k_cache.max()) == 7


def _mask(seed, B, S, ml, dtype=torch.float32, neg_inf_every=0):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(B, S, ml, generator=g) * 2
    if neg_inf_every:
        m.view(-1)[::neg_inf_every] = float("-inf")
    return m.to(dtype)


@pytest.mark.parametrize("kv", ["int8_token", "plain", "int4_channel"])
def test_attn_mask_matches_torch_float64(ref, kv):
    """mask [batch, seq_q, mask_len] (_ops.py:860; D16): added to the logits of the last
    mask_len keys, -inf entries removing keys; 4-D and cu_seq_q query forms, with windows,
    ALiBi and a sink, in float32 / float16 / bfloat16, against torch in float64."""
    dtype = torch.bfloat16
    case = W.attn_case(dtype, 71, kv=kv, Hq=8, Hkv=2, D=64, max_ctx=90)
    case.block_tables[3, 0] = -1
    codes = _int4_codes(case, "rows") if case.int4 else case
    q4 = W.attn_queries(dtype, 72, B=5, Hq=8, D=64, S=4)
    q3, cu = W.attn_queries(dtype, 73, B=5, Hq=8, D=64, counts=[4, 1, 0, 3, 2])
    sink = torch.linspace(-1.0, 1.0, 8)
    for ml, mdt, window, alibi, sk in ((4, torch.float32, -1, False, None),
                                       (16, torch.bfloat16, 9, False, sink),
                                       (64, torch.float16, -1, True, sink),
                                       (8, torch.float32, 2, True, None)):
        al = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1) if alibi else None
        case.alibi = codes.alibi = al
        mask = _mask(74 + ml, 5, 4, ml, mdt, neg_inf_every=7)
        for q, c in ((q4, None), (q3, cu)):
            out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                          case.context_lens, 0.125, case.k_scale, case.v_scale,
                                          al, window, cu_seq_q=c, sink=sk, int4=case.int4,
                                          mask=mask)
            want, wlse = torch_attn_mq(codes, q, 0.125, window, c, sk, mask=mask)
            assert torch.allclose(out, want, rtol=1e-12, atol=1e-12, equal_nan=True)
            assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12, equal_nan=True)


def test_attn_mask_identities(ref):
    """A zero mask is no mask, bit for bit.  A constant c over every key of a sequence (mask_len
    >= L) leaves out unchanged and adds c to the lse.  -inf over a token's last m keys equals
    the same token seeing only the keys before them (a shorter context, with the token moved
    back): the mask removes keys exactly.  A bfloat16 mask equals the float32 mask of the same
    values."""
    case = W.attn_case(torch.float16, 81, kv="int8_token", B=4, Hq=4, Hkv=2, D=32, max_ctx=40)
    q = W.attn_queries(torch.float16, 82, B=4, Hq=4, D=32, S=1)
    args = (case.k_cache, case.v_cache, case.block_tables, case.context_lens, 0.3,
            case.k_scale, case.v_scale)
    base = ref.cached_kv_attn(q, *args)
    zero = ref.cached_kv_attn(q, *args, mask=torch.zeros(4, 1, 8))
    assert torch.equal(base[0], zero[0]) and torch.equal(base[1], zero[1])
    c = 1.75
    const = ref.cached_kv_attn(q, *args, mask=torch.full((4, 1, 64), c))   # every L <= 40
    assert torch.allclose(const[0], base[0], rtol=1e-13, atol=1e-15)
    assert torch.allclose(const[1], base[1] + c, rtol=1e-13, atol=1e-13)
    m = 3
    cut = torch.zeros(4, 1, m)
    cut[:] = float("-inf")
    masked = ref.cached_kv_attn(q, *args, mask=cut)
    shorter = case.context_lens - m
    for i in range(4):
        if int(case.context_lens[i]) <= m:
            assert torch.all(masked[0][i] == 0) and torch.all(masked[1][i] == float("-inf"))
            continue
        lens = case.context_lens.clone()
        lens[i] = shorter[i]
        o, l = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables, lens, 0.3,
                                  case.k_scale, case.v_scale)
        assert torch.equal(masked[0][i], o[i]) and torch.equal(masked[1][i], l[i])
    vals = _mask(83, 4, 1, 16, torch.bfloat16)
    a = ref.cached_kv_attn(q, *args, mask=vals)
    b = ref.cached_kv_attn(q, *args, mask=vals.float())
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------- quantised q, sparse-KV tables (D17)

def _q_codes(dtype, shape, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.int8:
        return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)
    return W.fp8_codes(shape, g)


def _q_real(q, qs):
    """q codes times q_quant_scale in float64: per tensor, per (token, head), per channel group."""
    x = q.double()
    s = qs.double()
    if s.numel() == 1:
        return x * s.reshape(())
    if tuple(s.shape) == tuple(q.shape[:-1]):
        return x * s[..., None]
    G = s.shape[-1]
    return x * s.repeat_interleave(q.shape[-1] // G, dim=-1)


@pytest.mark.parametrize("qdt", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("form", ["tensor", "token", "group"])
def test_attn_quantised_q_matches_torch_float64(ref, qdt, form):
    """int8 / float8_e4m3fn q with q_quant_scale (_ops.py:853-856, 868): the codes times their
    scale in float64, attended by torch, against the oracle reading the codes -- 4-D q and
    cu_seq_q, int8 pages, a sink, ALiBi."""
    case = W.attn_case(torch.bfloat16, 131, kv="int8_token", Hq=8, Hkv=2, D=64, max_ctx=70)
    q4 = _q_codes(qdt, (5, 3, 8, 64), 132)
    q3 = _q_codes(qdt, (14, 8, 64), 133)
    cu = torch.tensor([0, 4, 6, 6, 13, 14], dtype=torch.int32)
    g = torch.Generator().manual_seed(134)
    for q, c in ((q4, None), (q3, cu)):
        lead = q.shape[:-1]
        qs = {"tensor": torch.tensor([0.0123]),
              "token": 0.002 + 0.02 * torch.rand(lead, generator=g),
              "group": 0.002 + 0.02 * torch.rand(lead + (4,), generator=g)}[form]
        case.alibi = (0.5 ** torch.arange(1, 9, dtype=torch.float32)).repeat(5, 1)
        out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables,
                                      case.context_lens, 0.125, case.k_scale, case.v_scale,
                                      case.alibi, -1, cu_seq_q=c, sink=torch.linspace(-1, 1, 8),
                                      q_scale=qs)
        want, wlse = torch_attn_mq(case, _q_real(q, qs), 0.125, -1, c, torch.linspace(-1, 1, 8))
        assert torch.allclose(out, want, rtol=1e-12, atol=1e-12, equal_nan=True)
        assert torch.allclose(lse, wlse, rtol=1e-12, atol=1e-12, equal_nan=True)


def test_attn_quantised_q_identities(ref):
    """float8_e4m3fn q codes with a unit per-tensor scale equal a bfloat16 q holding the same
    values (every e4m3fn value is a bfloat16 value) bit for bit; a per-token scale s equals
    the per-tensor scale s when every token and head carries s."""
    case = W.attn_case(torch.float16, 135, kv="int8_token", B=4, Hq=4, Hkv=2, D=32, max_ctx=50)
    q = _q_codes(torch.float8_e4m3fn, (4, 2, 4, 32), 136)
    args = (case.k_cache, case.v_cache, case.block_tables, case.context_lens, 0.2, case.k_scale,
            case.v_scale)
    a = ref.cached_kv_attn(q, *args, q_scale=torch.tensor([1.0]))
    b = ref.cached_kv_attn(q.to(torch.bfloat16), *args)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    s = 0.0371
    a = ref.cached_kv_attn(q, *args, q_scale=torch.full((4, 2, 4), s))
    b = ref.cached_kv_attn(q, *args, q_scale=torch.tensor([s]))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _sparse_tables(case, per, seed):
    """[B, per, max_blocks] tables: each head a different permutation of the case's pages (the
    same pages, so every head reads valid blocks), head 0 the case's own table."""
    g = torch.Generator().manual_seed(seed)
    bt = case.block_tables
    rows = [bt]
    for _ in range(per - 1):
        perm = torch.randperm(bt.numel(), generator=g)
        rows.append(bt.reshape(-1)[perm].reshape(bt.shape))
    return torch.stack(rows, dim=1).contiguous()


@pytest.mark.parametrize("per", ["kv", "q"])
def test_attn_sparse_tables_match_torch_float64(ref, per):
    """block_tables [batch, head_num_kv or head_num_q, max_blocks] (_ops.py:834): each head
    reads its own pages -- torch float64 over one head at a time with its row as the table,
    against the oracle over all heads; with every row equal to the 2-D table, the 2-D result
    bit for bit."""
    case = W.attn_case(torch.bfloat16, 137, kv="int8_token", Hq=8, Hkv=2, D=32, max_ctx=60)
    n = 2 if per == "kv" else 8
    bt3 = _sparse_tables(case, n, 138)
    q = W.attn_queries(torch.bfloat16, 139, B=5, Hq=8, D=32, S=2)
    out, lse = ref.cached_kv_attn(q, case.k_cache, case.v_cache, bt3, case.context_lens, 0.3,
                                  case.k_scale, case.v_scale)
    g = 8 // 2
    for hq in range(8):
        hk = hq // g
        row = bt3[:, hk if per == "kv" else hq]
        sub = W.AttnCase(case.q, case.k_cache[:, hk:hk + 1].contiguous(),
                         case.v_cache[:, hk:hk + 1].contiguous(),
                         case.k_scale[:, hk:hk + 1].contiguous(), case.v_scale[:, hk:hk + 1].contiguous(),
                         row.contiguous(), case.context_lens)
        want, wlse = torch_attn_mq(sub, q[:, :, hq:hq + 1], 0.3)
        assert torch.allclose(out[:, :, hq:hq + 1], want, rtol=1e-12, atol=1e-12)
        assert torch.allclose(lse[:, :, hq:hq + 1], wlse, rtol=1e-12, atol=1e-12)
    same = case.block_tables[:, None].expand(5, n, -1).contiguous()
    a = ref.cached_kv_attn(q, case.k_cache, case.v_cache, same, case.context_lens, 0.3,
                           case.k_scale, case.v_scale)
    b = ref.cached_kv_attn(q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                           0.3, case.k_scale, case.v_scale)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
