"""GPU parity: the HIP kernels (through the torch_mlu_ops ops -> C ABI) against the CPU oracle.

Bar: bit-exact for everything -- int8 codes, fp32 scales, gathered/scattered bytes and the
dequantised bf16/fp16/fp32 outputs -- including the bytes a call must NOT write (caches and
outputs start from a sentinel pattern and are compared whole).  All five BASELINE configs run
at full size; the edge-case tests cover the other kernel paths (generic layouts, strided
views, every lane-group width, skipped slots, zero / tiny / huge rows).
"""
import pytest
import torch

from tests import workloads as W

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16)
    return t


def assert_bits_equal(got: torch.Tensor, want: torch.Tensor, what: str) -> None:
    a, b = _bits(got), _bits(want)
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} != {tuple(b.shape)}"
    if torch.equal(a, b):
        return
    diff = (a != b).nonzero()
    first = tuple(diff[0].tolist())
    raise AssertionError(f"{what}: {diff.shape[0]} mismatching elements, first at {first}: "
                         f"gpu={got.detach().cpu()[first]!r} oracle={want[first]!r}")


# ---------------------------------------------------------------------------- quant_to_paged_cache

def run_quant(tmo, ref, dev, case: W.PagedQuantCase, with_v=True, k=None, v=None,
              cache_dtype=torch.int8):
    """GPU op and oracle on the same inputs; returns (gpu caches, oracle caches).  fp8 caches
    start from the same sentinel bytes as int8 ones."""
    k = case.k if k is None else k
    v = (case.v if v is None else v) if with_v else None
    kc, vc, ks, vs = case.empty_caches()
    kc, vc = kc.view(cache_dtype), vc.view(cache_dtype)
    if not with_v:
        vc = vs = None
    ref.quant_to_paged_cache(k, v, kc, vc, ks, vs, case.slot_mapping)
    gk, gv, gks, gvs = case.empty_caches(device=dev)
    gk, gv = gk.view(cache_dtype), gv.view(cache_dtype)
    kd = k.to(dev)
    vd = v.to(dev) if v is not None else None
    if not with_v:
        gv = gvs = None
    out = tmo.quant_to_paged_cache(kd, vd, gk, gv, gks, gvs, case.slot_mapping.to(dev))
    assert out[0] is gk
    torch.cuda.synchronize()
    return (gk, gv, gks, gvs), (kc, vc, ks, vs)


def check_quant(tmo, ref, dev, case, with_v=True, k=None, v=None, cache_dtype=torch.int8):
    got, want = run_quant(tmo, ref, dev, case, with_v, k, v, cache_dtype)
    for g, w, n in zip(got, want, ("k_cache", "v_cache", "k_scale", "v_scale")):
        if w is not None:
            assert_bits_equal(g, w, f"{case.name} {n}")
    return got, want


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_quant_to_paged_cache_configs(tmo, ref, dev, cfg):
    case = getattr(W, cfg)()
    print(f"[quant_to_paged_cache] {cfg} T={case.tokens}", flush=True)
    got, want = check_quant(tmo, ref, dev, case)
    # every valid token wrote its codes; skipped slots kept the sentinel
    written = (want[2] != W.SCALE_SENTINEL).sum().item()
    assert written == case.valid_tokens() * case.k.shape[1]


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3"])
def test_quant_to_paged_cache_fp8_configs(tmo, ref, dev, cfg):
    """The float8_e4m3fn cache branch of the same op (scale = amax / 448) on every config."""
    case = getattr(W, cfg)()
    print(f"[quant_to_paged_cache fp8] {cfg} T={case.tokens}", flush=True)
    check_quant(tmo, ref, dev, case, cache_dtype=torch.float8_e4m3fn)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D,BS", [(8, 16), (64, 16), (128, 16), (512, 16), (128, 7), (72, 5)])
def test_quant_fp8_widths_and_generic(tmo, ref, dev, dtype, D, BS):
    case = _case(f"fp8 D={D} BS={BS}", 61, 3, D, 40, BS, dtype, seed=3 * D + BS, neg_frac=0.1,
                 oob=2)
    k = case.k.to(torch.float32)
    k[0] = 0                                                                # zero row
    k[1] *= 1e-25 if dtype != torch.float16 else 1e-6                       # tiny scales
    k[2] *= 1e25 if dtype != torch.float16 else 1e3                         # huge (finite)
    k[3, :, ::3] = -0.0                                                     # signed zeros:
    k[4, :, 1::2] = 0.0                                                     # fp8 0x80 / 0x00
    k = k.to(dtype)
    check_quant(tmo, ref, dev, case, k=k, cache_dtype=torch.float8_e4m3fn)
    check_quant(tmo, ref, dev, case, k=k, with_v=False, cache_dtype=torch.float8_e4m3fn)


def _case(name, T, H, D, NB, BS, dtype, seed, neg_frac=0.0, oob=0):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(T, H, D, generator=g).to(dtype)
    v = (3.0 * torch.randn(T, H, D, generator=g)).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    if neg_frac:
        slot[torch.randperm(T, generator=g)[: int(neg_frac * T)]] = -1
    if oob:
        slot[torch.randperm(T, generator=g)[:oob]] = NB * BS + 5
    return W.PagedQuantCase(name, k, v, slot, NB, BS)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [8, 16, 32, 64, 128, 256, 512])
def test_quant_lane_group_widths(tmo, ref, dev, dtype, D):
    """Every lane-group width G = D / (16 B / elem) of the vector kernel (1..64 lanes; the
    f32 D=512 row takes the generic one-wave path), the row maximum placed in every lane."""
    T, H = 70, 3
    case = _case(f"G D={D} {dtype}", T, H, D, 40, 16, dtype, seed=D)
    k = case.k.clone()
    for t in range(T):  # put the row max at element t % D (so in lane (t % D) / per_vec)
        k[t, :, t % D] = 50.0 * (1 if t % 2 else -1)
    check_quant(tmo, ref, dev, case, k=k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D,BS", [(128, 16), (128, 7), (80, 16), (96, 32), (72, 5), (1, 16)])
def test_quant_shapes_and_block_sizes(tmo, ref, dev, dtype, D, BS):
    """Power-of-two and odd block sizes; head sizes outside the vector path (generic)."""
    case = _case(f"D={D} BS={BS}", 53, 5, D, 23, BS, dtype, seed=7 * D + BS, neg_frac=0.2, oob=3)
    check_quant(tmo, ref, dev, case)


def test_quant_k_only_and_strided_views(tmo, ref, dev):
    """v=None, and k/v as column views of a fused [T, 3H, D] qkv tensor."""
    T, H, D = 64, 4, 128
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(T, 3 * H, D, generator=g).to(torch.bfloat16)
    k, v = qkv[:, H:2 * H], qkv[:, 2 * H:]
    slot = torch.randperm(32 * 16, generator=g)[:T].to(torch.int32)
    case = W.PagedQuantCase("qkv-view", k, v, slot, 32, 16)
    check_quant(tmo, ref, dev, case)  # vector path with token stride 3*H*D
    check_quant(tmo, ref, dev, case, with_v=False)
    # misaligned by one element: falls back to the generic path
    flat = torch.randn(T * H * D + 1, generator=g).to(torch.bfloat16)
    km = flat[1:].view(T, H, D)
    check_quant(tmo, ref, dev, W.PagedQuantCase("misaligned", km, km, slot, 32, 16))


def test_quant_special_rows(tmo, ref, dev):
    """Zero rows (scale 0, codes 0), exact .5 ties, rows whose scale is below the fast-divide
    range (IEEE path), huge and subnormal magnitudes, single non-zero rows."""
    T, H, D = 16, 2, 128
    k = torch.zeros(T, H, D)
    k[1, 0, :5] = torch.tensor([127.0, 2.5, 3.5, -0.5, 1.5])               # ties, scale 1
    k[2, 1, 7] = -3.0                                                        # single non-zero
    k[3, :, :] = torch.linspace(-1, 1, D) * 1e-20                            # scale < 2^-60
    k[4, :, :] = torch.linspace(-1, 1, D) * 3e38                             # near bf16 max
    k[5, :, :] = torch.linspace(-1, 1, D) * 1e-39                            # bf16 subnormals
    k[6, 0, :] = 5.0                                                         # constant row
    g = torch.Generator().manual_seed(5)
    k[7:] = torch.randn(T - 7, H, D, generator=g) * torch.logspace(-30, 30, T - 7)[:, None, None]
    slot = torch.arange(T, dtype=torch.int32) * 3
    for dtype in (torch.bfloat16, torch.float32):
        kk = k.to(dtype)
        case = W.PagedQuantCase(f"special {dtype}", kk, kk.flip(0).contiguous(), slot, 4, 16)
        got, _ = check_quant(tmo, ref, dev, case)
        kc = got[0].cpu()
        assert torch.all(kc[0, :, 0, :] == 0)                     # token 0 (all zeros)
        assert kc[0, 0, 3, :5].tolist() == [127, 2, 4, 0, 2]      # token 1 at slot 3


# ---------------------------------------------------------------------------- offline_quant_to_paged_cache

def check_offline(tmo, ref, dev, name, k, v, ks, vs, slot, NB, BS, cdt):
    """GPU offline_quant_to_paged_cache vs the oracle, caches compared whole (sentinel start)."""
    H, D = k.shape[1], k.shape[2]

    def fresh():
        return torch.full((NB, H, BS, D), 0x5A, dtype=torch.uint8).view(cdt)

    kc, vc = fresh(), (fresh() if v is not None else None)
    ref.offline_quant_to_paged_cache(k, v, ks, vs, slot, kc, vc)
    gk = fresh().to(dev)
    gv = fresh().to(dev) if v is not None else None
    d = (lambda t: t.to(dev) if torch.is_tensor(t) else t)
    out = tmo.offline_quant_to_paged_cache(d(k), d(v), d(ks), d(vs), slot.to(dev), gk, gv)
    assert (out[0] if v is not None else out) is gk
    assert_bits_equal(gk.view(torch.uint8), kc.view(torch.uint8), f"{name} k_cache")
    if v is not None:
        assert_bits_equal(gv.view(torch.uint8), vc.view(torch.uint8), f"{name} v_cache")


def _offline_inputs(T, H, D, NB, BS, dtype, seed, per_channel):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(T, H, D, generator=g) * torch.logspace(-3, 2, T)[:, None, None]).to(dtype)
    v = (torch.randn(T, H, D, generator=g) * 5).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    if T > 8:
        slot[::11] = -1
        slot[3] = NB * BS + 7
    if per_channel:
        ks = 0.01 + 0.2 * torch.rand(H, D, generator=g)
        vs = 0.02 + 0.1 * torch.rand(H, D, generator=g)
    else:
        ks, vs = 0.0371, 0.0523
    return k, v, ks, vs, slot


CACHE_DTYPES = [torch.int8, torch.float8_e4m3fn]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cdt", CACHE_DTYPES)
@pytest.mark.parametrize("per_channel", [True, False])
def test_offline_quant_modes(tmo, ref, dev, dtype, cdt, per_channel):
    """Per-channel and per-tensor scales, int8 and fp8 caches, every input dtype; magnitudes
    from 1e-3 to 1e2 so that codes underflow to 0 and saturate; -1 and out-of-range slots."""
    k, v, ks, vs, slot = _offline_inputs(300, 8, 128, 64, 16, dtype, 31, per_channel)
    check_offline(tmo, ref, dev, f"offline {dtype} {cdt}", k, v, ks, vs, slot, 64, 16, cdt)
    check_offline(tmo, ref, dev, "k only", k, None, ks, None, slot, 64, 16, cdt)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D,BS", [(8, 16), (16, 16), (32, 16), (64, 16), (256, 16), (512, 16),
                                  (80, 16), (3, 16), (128, 7)])
def test_offline_quant_head_sizes(tmo, ref, dev, dtype, D, BS):
    """Every lane-group width of the vector kernel (1..64 lanes), the generic kernel (head size
    not a vector multiple, or more than 64 vectors), and an odd block size."""
    k, v, ks, vs, slot = _offline_inputs(70, 3, D, 20, BS, dtype, D + BS, True)
    for cdt in CACHE_DTYPES:
        check_offline(tmo, ref, dev, f"D={D} BS={BS} {cdt}", k, v, ks, vs, slot, 20, BS, cdt)


@pytest.mark.parametrize("T", [1, 63, 64, 65, 1000])
def test_offline_quant_token_tails(tmo, ref, dev, T):
    """Token counts around the kernel's tokens-per-workgroup (the last tile re-reads a valid
    row and must not write it)."""
    k, v, ks, vs, slot = _offline_inputs(T, 8, 128, 80, 16, torch.bfloat16, T, True)
    check_offline(tmo, ref, dev, f"T={T}", k, v, ks, vs, slot, 80, 16, torch.int8)


def test_offline_quant_scale_ranges(tmo, ref, dev):
    """Scales outside the reciprocal path's range (tiny, huge) and negative ones, and rows
    whose quotients exceed 2^22 (IEEE-divide branch of the lane); per channel and per tensor."""
    T, H, D = 40, 4, 128
    g = torch.Generator().manual_seed(5)
    k = torch.randn(T, H, D, generator=g) * 3
    k[5, 1, 17] = 3.0e10            # |x / s| > 2^22 in one lane
    k[9, 2, :] = 1e-30              # tiny quotients
    slot = torch.arange(T, dtype=torch.int32)
    ks = 0.05 + 0.1 * torch.rand(H, D, generator=g)
    ks[0, :8] = 1e-20               # below 2^-60
    ks[1, 8:16] = 3e33              # above 2^100
    ks[2, 16:24] *= -1              # negative
    k[11, :, ::2] = -0.0            # signed zeros (fp8 codes 0x80 / 0x00, by the scale's sign)
    k[12, :, 1::2] = 0.0
    for cdt in CACHE_DTYPES:
        for dtype in (torch.float32, torch.bfloat16):
            kk = k.to(dtype)
            check_offline(tmo, ref, dev, f"ranges {cdt} {dtype}", kk, kk.flip(0).contiguous(),
                          ks, ks.flip(0).contiguous(), slot, 3, 16, cdt)
            for st in (1e-25, 2.5e34, -0.03):
                check_offline(tmo, ref, dev, f"tensor {st}", kk, None, st, None, slot, 3, 16, cdt)


def test_offline_quant_strided_views(tmo, ref, dev):
    T, H, D = 64, 4, 128
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn(T, 3 * H, D, generator=g).to(torch.bfloat16)
    k, v = qkv[:, H:2 * H], qkv[:, 2 * H:]
    slot = torch.randperm(32 * 16, generator=g)[:T].to(torch.int32)
    ks = 0.01 + 0.02 * torch.rand(H, D, generator=g)
    for cdt in CACHE_DTYPES:
        check_offline(tmo, ref, dev, "qkv view", k, v, ks, ks, slot, 32, 16, cdt)
        flat = torch.randn(T * H * D + 1, generator=g).to(torch.bfloat16)
        km = flat[1:].view(T, H, D)
        check_offline(tmo, ref, dev, "misaligned", km, km, 0.02, 0.03, slot, 32, 16, cdt)


def test_offline_quant_cfg3_shape(tmo, ref, dev):
    """configs[2]'s shape (32768 tokens x 8 heads x 128, bf16, 65536 pages) with per-channel
    scales, both cache types, at full size."""
    case = W.cfg3()
    g = torch.Generator().manual_seed(2024)
    ks = 0.005 + 0.05 * torch.rand(8, 128, generator=g)
    vs = 0.005 + 0.05 * torch.rand(8, 128, generator=g)
    for cdt in CACHE_DTYPES:
        check_offline(tmo, ref, dev, f"cfg3 {cdt}", case.k, case.v, ks, vs, case.slot_mapping,
                      case.num_blocks, case.block_size, cdt)


# ---------------------------------------------------------------------------- fused rope (rmsnorm)

def check_fused_rope(tmo, ref, dev, name, case, with_q_gamma=True, off=0, api="rmsnorm_store",
                     norm_type="rmsnorm", k_beta=None):
    """GPU fused rope vs the oracle on the same inputs: qkv (Q written back), both caches and
    the dynamic scales compared whole, from a sentinel start.  norm_type "layernorm" goes
    through fused_rope with k_beta; q_gamma is passed but not used there."""
    qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = case
    qg = qg if with_q_gamma else None
    layernorm = norm_type == "layernorm"
    assert not layernorm or api == "fused_rope"
    kc = kc.view(torch.uint8).fill_(0x5A).view(kc.dtype)
    vc = vc.view(torch.uint8).fill_(0x5A).view(vc.dtype)
    if ks is not None and ks.dim() == 3:
        ks.fill_(W.SCALE_SENTINEL)
        vs.fill_(W.SCALE_SENTINEL)
    want = [qkv.clone(), kc.clone(), vc.clone(),
            ks.clone() if ks is not None else None, vs.clone() if vs is not None else None]
    ref.fused_rope_paged(want[0], want[1], want[2], sin, cos, pid, kg, want[3], want[4], slot,
                         1e-5, None if layernorm else qg, off, norm_type=norm_type, k_beta=k_beta)
    d = (lambda t: t.to(dev) if t is not None else None)
    got = [d(qkv), d(kc), d(vc), d(ks), d(vs)]
    if api == "rmsnorm_store":
        assert off == 0
        out = tmo.fused_rmsnorm_rope_store_paged_cache(got[0], got[1], got[2], d(sin), d(cos), d(pid),
                                                       d(kg), d(qg), d(slot), got[3], got[4], 1e-5)
        assert out[0] is got[0] and out[1] is got[1]
    else:
        out = tmo.fused_rope(got[0], got[1], got[2], d(sin), d(cos), d(pid), d(kg), d(k_beta),
                             k_scale_hp=got[3], v_scale_hp=got[4], slot_mapping_hp=d(slot),
                             norm_type=norm_type, rope_dim_offset=off, eps=1e-5, q_gamma=d(qg))
        assert len(out) == 3 and out[0] is got[0]
    for g, w, n in zip(got, want, ("qkv", "k_cache", "v_cache", "k_scale", "v_scale")):
        if w is not None:
            assert_bits_equal(g.view(torch.int8) if g.dtype == torch.int8 else g, w,
                              f"{name} {n}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("with_q_gamma", [True, False])
def test_fused_rope_modes(tmo, ref, dev, dtype, mode, with_q_gamma):
    """Unquantised, dynamic and static int8 caches; Q with and without its RMSNorm; four
    sequences, the last running past the sin/cos table (unrotated); -1 slots; a zero K row."""
    case = W.fused_rope_case(dtype, mode, 21, B=4, S=24, Hq=8, Hk=2, NB=16)
    check_fused_rope(tmo, ref, dev, f"{dtype} {mode}", case, with_q_gamma)


@pytest.mark.parametrize("D,rope,off", [(128, 64, 32), (64, 32, 0), (256, 256, 0), (512, 128, 64),
                                        (16, 16, 0), (8, 8, 0), (96, 64, 16), (100, 40, 6),
                                        (128, 24, 8), (128, 2, 126)])
def test_fused_rope_head_sizes_and_windows(tmo, ref, dev, D, rope, off):
    """Vector path widths (8..512 channels, windows on 8-element chunks) and the generic path
    (head sizes not a power-of-two multiple of 8, windows not on chunk boundaries)."""
    for mode in ("none", "dynamic"):
        case = W.fused_rope_case(torch.bfloat16, mode, D + rope + off, B=2, S=9, Hq=3, Hk=1, D=D,
                                 rope=rope, NB=4)
        check_fused_rope(tmo, ref, dev, f"D={D} rope={rope}+{off} {mode}", case, True, off,
                         api="fused_rope")


@pytest.mark.parametrize("D,Hq,Hk", [(128, 64, 8), (128, 96, 16), (512, 16, 2), (64, 120, 8),
                                    (128, 136, 8), (512, 32, 4), (64, 248, 8), (128, 240, 8),
                                    (128, 264, 8), (512, 64, 4), (64, 512, 8), (256, 40, 4),
                                    (16, 1000, 12), (32, 300, 10)])
def test_fused_rope_many_heads(tmo, ref, dev, D, Hq, Hk):
    """Many heads: the token-major kernel in 512-thread workgroups with 3 to 8 rows per lane
    group (80, 128, 152 and 256 heads at D = 128; 20 and 40 at D = 512; 136 and 264 at D = 64;
    48 at D = 256, 1024 at D = 16, 320 at D = 32), and more heads than those cover in eight
    rows each (280 at D = 128, 72 at D = 512, 528 at D = 64): the row-major kernel, one lane
    group per (token, head) row."""
    for mode in ("dynamic", "static"):
        case = W.fused_rope_case(torch.bfloat16, mode, D + Hq, B=2, S=11, Hq=Hq, Hk=Hk, D=D,
                                 rope=min(D, 128), NB=4)
        check_fused_rope(tmo, ref, dev, f"D={D} Hq={Hq} Hk={Hk} {mode}", case, True)


def test_fused_rope_llama_prefill_shape(tmo, ref, dev):
    """A Llama-3-8B-shaped prefill chunk: 8 x 512 tokens, 32 Q + 8 KV heads x 128, bf16,
    dynamic int8 caches, table of 4096 positions."""
    case = W.fused_rope_case(torch.bfloat16, "dynamic", 5, B=8, S=512, Hq=32, Hk=8, NB=512,
                             maxpos=4096, positions=(0, 512, 1024, 1536, 2048, 2560, 3072, 3584))
    check_fused_rope(tmo, ref, dev, "llama prefill", case, True)


def _beta(D, dtype, seed):
    return (torch.rand(D, generator=torch.Generator().manual_seed(seed)) - 0.5).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("with_beta", [True, False])
def test_fused_rope_layernorm_modes(tmo, ref, dev, dtype, mode, with_beta):
    """norm_type "layernorm" (the reference's default): Q and K rotated, then K layer-normalised
    with k_gamma and k_beta; unquantised, dynamic and static int8 caches; a sequence past the
    sin/cos table; -1 slots; a zero K row (stored as beta)."""
    case = W.fused_rope_case(dtype, mode, 23, B=4, S=24, Hq=8, Hk=2, NB=16)
    check_fused_rope(tmo, ref, dev, f"layernorm {dtype} {mode} beta={with_beta}", case, True,
                     api="fused_rope", norm_type="layernorm",
                     k_beta=_beta(128, dtype, 7) if with_beta else None)


@pytest.mark.parametrize("D,rope,off", [(128, 64, 32), (64, 32, 0), (256, 256, 0), (512, 128, 64),
                                        (16, 16, 0), (8, 8, 0), (96, 64, 16), (100, 40, 6),
                                        (128, 2, 126), (40, 40, 0)])
def test_fused_rope_layernorm_head_sizes_and_windows(tmo, ref, dev, D, rope, off):
    """Layernorm through the vector path (head sizes 8..512) and the generic path (head sizes
    not a power-of-two multiple of 8, windows off chunk boundaries)."""
    for mode in ("none", "dynamic"):
        case = W.fused_rope_case(torch.bfloat16, mode, 3 * D + rope + off, B=2, S=9, Hq=3, Hk=1, D=D,
                                 rope=rope, NB=4)
        check_fused_rope(tmo, ref, dev, f"layernorm D={D} rope={rope}+{off} {mode}", case, True,
                         off, api="fused_rope", norm_type="layernorm",
                         k_beta=_beta(D, torch.bfloat16, D))


@pytest.mark.parametrize("D,Hq,Hk", [(128, 64, 8), (64, 120, 8), (128, 136, 8), (512, 32, 4),
                                    (128, 264, 8), (512, 64, 4)])
def test_fused_rope_layernorm_many_heads(tmo, ref, dev, D, Hq, Hk):
    """Layernorm with many heads: the token-major kernel in 512-thread workgroups (80 and 152
    heads at D = 128, 136 at D = 64, 40 at D = 512) and the row-major kernel (280 heads at
    D = 128, 72 at D = 512)."""
    case = W.fused_rope_case(torch.bfloat16, "dynamic", D + Hq + 1, B=2, S=11, Hq=Hq, Hk=Hk, D=D,
                             rope=min(D, 128), NB=4)
    check_fused_rope(tmo, ref, dev, f"layernorm D={D} Hq={Hq} Hk={Hk}", case, True,
                     api="fused_rope", norm_type="layernorm", k_beta=_beta(D, torch.bfloat16, 1))


@pytest.mark.parametrize("mode", ["none", "dynamic", "static"])
@pytest.mark.parametrize("norm_type", ["rmsnorm", "layernorm"])
@pytest.mark.parametrize("D,Hq,ids", [(128, 8, "given"), (128, 8, "default"), (64, 200, "given"),
                                      (96, 4, "given")])
def test_fused_rope_linear_caches(tmo, ref, dev, mode, norm_type, D, Hq, ids):
    """fused_rope into linear caches [max_batch, kv_heads, cache_len, head_size] through
    cache_bs_id_hp / cache_seq_offsets_hp (token-major, row-major and generic kernels): a -1
    cache batch, a batch id past the cache, positions past cache_len; from sentinel caches."""
    qkv, _, _, sin, cos, pid, kg, qg, ks, vs, _ = W.fused_rope_case(
        torch.bfloat16, mode, D + Hq, B=4, S=13, Hq=Hq, Hk=2, D=D, rope=min(D, 64))
    MB, L = 6, 40
    cdt = torch.bfloat16 if mode == "none" else torch.int8
    kc = torch.zeros(MB, 2, L, D, dtype=cdt).view(torch.uint8).fill_(0x5A).view(cdt)
    vc = kc.clone()
    if mode == "dynamic":
        ks = torch.full((MB, 2, L), W.SCALE_SENTINEL)
        vs = ks.clone()
    if ids == "given":
        bs_id = torch.tensor([5, -1, 0, 9], dtype=torch.int32)
        offs = torch.tensor([0, 4, 33, 20], dtype=torch.int32)
    else:
        bs_id = offs = None
    kb = (torch.rand(D, generator=torch.Generator().manual_seed(4)) - 0.5).to(torch.bfloat16) \
        if norm_type == "layernorm" else None
    qg = qg if norm_type == "rmsnorm" else None
    want = [qkv.clone(), kc.clone(), vc.clone(),
            ks.clone() if ks is not None else None, vs.clone() if vs is not None else None]
    ref.fused_rope_linear(want[0], want[1], want[2], sin, cos, pid, kg, want[3], want[4], bs_id,
                          offs, 1e-5, qg, norm_type=norm_type, k_beta=kb)
    d = (lambda t: t.to(dev) if t is not None else None)
    got = [d(qkv), d(kc), d(vc), d(ks), d(vs)]
    name = f"linear {mode} {norm_type} D={D} Hq={Hq} ids={ids}"
    print(f"[fused_rope linear] {name}", flush=True)
    out = tmo.fused_rope(got[0], got[1], got[2], d(sin), d(cos), d(pid), d(kg), d(kb),
                         cache_bs_id_hp=d(bs_id), cache_seq_offsets_hp=d(offs),
                         k_scale_hp=got[3], v_scale_hp=got[4], norm_type=norm_type, eps=1e-5,
                         q_gamma=d(qg))
    assert len(out) == 3 and out[0] is got[0]
    for g, w, n in zip(got, want, ("qkv", "k_cache", "v_cache", "k_scale", "v_scale")):
        if w is not None:
            assert_bits_equal(g, w, f"{name} {n}")


def test_fused_rope_rejects_both_targets(tmo, dev):
    qkv, kc, vc, sin, cos, pid, kg, qg, ks, vs, slot = W.fused_rope_case(torch.bfloat16, "none", 1)
    d = (lambda t: t.to(dev))
    with pytest.raises(RuntimeError, match="not both"):
        tmo.fused_rope(d(qkv), d(kc), d(vc), d(sin), d(cos), d(pid), d(kg), None,
                       slot_mapping_hp=d(slot), cache_bs_id_hp=d(torch.zeros(3, dtype=torch.int32)),
                       norm_type="rmsnorm")


# ---------------------------------------------------------------------------- reshape_paged_cache

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.int8])
@pytest.mark.parametrize("D", [128, 64, 3, 20])
def test_reshape_paged_cache_roundtrip(tmo, ref, dev, dtype, D):
    T, H, NB, BS = 100, 4, 30, 16
    g = torch.Generator().manual_seed(D)
    if dtype == torch.int8:
        k = torch.randint(-128, 128, (T, H, D), generator=g, dtype=torch.int8)
        v = torch.randint(-128, 128, (T, H, D), generator=g, dtype=torch.int8)
    else:
        k = torch.randn(T, H, D, generator=g).to(dtype)
        v = torch.randn(T, H, D, generator=g).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[::9] = -1
    slot[5] = NB * BS  # out of range: skipped
    case = W.PagedQuantCase("reshape", k, v, slot, NB, BS)
    kc, vc, _, _ = case.empty_caches(dtype=dtype)
    ref.reshape_paged_cache(k, v, kc, vc, slot, False)
    gk, gv, _, _ = case.empty_caches(device=dev, dtype=dtype)
    out = tmo.reshape_paged_cache(k.to(dev), v.to(dev), gk, gv, slot.to(dev), False)
    assert out[0] is gk and out[1] is gv
    assert_bits_equal(gk, kc, "scatter k_cache")
    assert_bits_equal(gv, vc, "scatter v_cache")
    # gather back into fresh rows
    kb = torch.zeros_like(k)
    vb = torch.zeros_like(v)
    ref.reshape_paged_cache(kb, vb, kc, vc, slot, True)
    gkb, gvb = torch.zeros_like(k, device=dev), torch.zeros_like(v, device=dev)
    tmo.reshape_paged_cache(gkb, gvb, gk, gv, slot.to(dev), True)
    assert_bits_equal(gkb, kb, "gather k")
    assert_bits_equal(gvb, vb, "gather v")
    valid = (slot >= 0) & (slot < NB * BS)
    assert torch.equal(_bits(gkb)[valid], _bits(k)[valid])  # gather(scatter(x)) == x


@pytest.mark.parametrize("with_v", [True, False])
def test_reshape_paged_cache_views_and_k_only(tmo, ref, dev, with_v):
    """K and V as strided views into a fused [T, 3H, D] qkv tensor (one 16-byte vector per
    lane: the rows kernel), with and without V, scatter and then gather, against the oracle."""
    T, H, NB, BS, D = 70, 4, 20, 16, 128
    g = torch.Generator().manual_seed(404)
    qkv = torch.randn(T, 3 * H, D, generator=g).to(torch.bfloat16)
    slot = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slot[::7] = -1
    slot[3] = NB * BS
    k, v = qkv[:, H:2 * H], qkv[:, 2 * H:]
    case = W.PagedQuantCase("reshape", k.contiguous(), v.contiguous(), slot, NB, BS)
    kc, vc, _, _ = case.empty_caches(dtype=torch.bfloat16)
    ref.reshape_paged_cache(k, v if with_v else None, kc, vc if with_v else None, slot, False)
    gq = qkv.to(dev)
    gk, gv, _, _ = case.empty_caches(device=dev, dtype=torch.bfloat16)
    gvv = gq[:, 2 * H:] if with_v else None
    tmo.reshape_paged_cache(gq[:, H:2 * H], gvv, gk, gv if with_v else None, slot.to(dev), False)
    torch.cuda.synchronize()
    assert_bits_equal(gk, kc, "scatter k_cache (view)")
    if with_v:
        assert_bits_equal(gv, vc, "scatter v_cache (view)")
    else:
        assert_bits_equal(gv, vc, "v_cache untouched")  # both still the sentinel fill
    # gather back into the views of a fresh qkv: the Q slice and the skipped rows keep their bytes
    back = torch.full_like(qkv, -7.0)
    ref.reshape_paged_cache(back[:, H:2 * H], back[:, 2 * H:] if with_v else None, kc,
                            vc if with_v else None, slot, True)
    gback = torch.full_like(gq, -7.0)
    tmo.reshape_paged_cache(gback[:, H:2 * H], gback[:, 2 * H:] if with_v else None, gk,
                            gv if with_v else None, slot.to(dev), True)
    torch.cuda.synchronize()
    assert_bits_equal(gback, back, "gather into qkv views")


def test_reshape_paged_cache_cfg3(tmo, ref, dev):
    case = W.cfg3()
    kc, vc, _, _ = case.empty_caches(dtype=torch.bfloat16)
    ref.reshape_paged_cache(case.k, case.v, kc, vc, case.slot_mapping, False)
    gk, gv, _, _ = case.empty_caches(device=dev, dtype=torch.bfloat16)
    tmo.reshape_paged_cache(case.k.to(dev), case.v.to(dev), gk, gv, case.slot_mapping.to(dev))
    assert_bits_equal(gk, kc, "cfg3 reshape k_cache")
    assert_bits_equal(gv, vc, "cfg3 reshape v_cache")


# ---------------------------------------------------------------------------- dequant_from_paged_cache

def _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode, seq_offset=None, total=None,
                  with_v=True, max_ctx=None):
    kc, vc, ks, vs = caches
    H, D = kc.shape[1], kc.shape[3]
    total = layout.total_tokens if total is None else total
    kc_h, vc_h, ks_h, vs_h = (t.cpu() if t is not None else None for t in caches)
    want_k = torch.full((total, H, D), -3.0).to(out_dtype)
    want_v = want_k.clone() if with_v else None
    ref.dequant_from_paged_cache(want_k, want_v, kc_h, vc_h if with_v else None, ks_h,
                                 vs_h if with_v else None, layout.context_lengths, seq_offset,
                                 layout.block_tables, mode)
    got_k = torch.full((total, H, D), -3.0, device=dev).to(out_dtype)
    got_v = got_k.clone() if with_v else None
    tmo.dequant_from_paged_cache(
        got_k, got_v, kc, vc if with_v else None, ks, vs if with_v else None,
        layout.context_lengths.to(dev), layout.max_context_len if max_ctx is None else max_ctx,
        seq_offset.to(dev) if seq_offset is not None else None, layout.block_tables.to(dev), mode, 8)
    assert_bits_equal(got_k, want_k, f"{layout.name} key")
    if with_v:
        assert_bits_equal(got_v, want_v, f"{layout.name} value")
    return got_k, want_k


def test_dequant_cfg5_full(tmo, ref, dev):
    layout = W.cfg5()
    print(f"[dequant] cfg5 sum(ctx)={layout.total_tokens}", flush=True)
    caches = W.cfg5_fill(layout, dev)
    _dequant_both(tmo, ref, dev, layout, caches, torch.bfloat16, 1)


def test_dequant_cfg5_full_fp8_pages_bf16_scales(tmo, ref, dev):
    """configs[4] at full size with float8_e4m3fn pages written by this build's
    quant_to_paged_cache (fp8 branch), their fp32 scales read once as written and once
    rounded to bf16 (_ops.py:3805-3806): bit-exact against the oracle."""
    layout = W.cfg5()
    print(f"[dequant fp8] cfg5 sum(ctx)={layout.total_tokens}", flush=True)
    kc, vc, ks, vs = W.cfg5_fill(layout, dev, cache_dtype=torch.float8_e4m3fn)
    _dequant_both(tmo, ref, dev, layout, (kc, vc, ks, vs), torch.bfloat16, 1)
    _dequant_both(tmo, ref, dev, layout, (kc, vc, ks.to(torch.bfloat16), vs.to(torch.bfloat16)),
                  torch.bfloat16, 1)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("cache,scale_dtype", [("fp8", torch.float32), ("fp8", torch.bfloat16),
                                               ("int8", torch.bfloat16)])
@pytest.mark.parametrize("D,BS,H", [(128, 16, 4), (128, 16, 3), (80, 16, 4)])
def test_dequant_fp8_pages_and_bf16_scales(tmo, ref, dev, out_dtype, mode, cache, scale_dtype,
                                           D, BS, H):
    """float8_e4m3fn pages and bf16 scales on the page-list kernels, the per-page kernel and
    the scalar kernel, both modes, every output type, with and without V."""
    layout, (kc, vc, ks, vs) = _small_layout(seed=D + H + mode + 3, D=D, BS=BS, NB=64, H=H)
    if cache == "fp8":
        g = torch.Generator().manual_seed(D + H)
        kc, vc = W.fp8_codes(kc.shape, g), W.fp8_codes(vc.shape, g)
        ks, vs = ks * 0.01, vs * 0.01
    if mode == 0:
        g = torch.Generator().manual_seed(98)
        ks = torch.rand(H, D, generator=g) * 0.05
        vs = torch.rand(H, D, generator=g) * 0.05
    ks, vs = ks.to(scale_dtype), vs.to(scale_dtype)
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode)
    _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode, with_v=False)


def _small_layout(seed, B=5, NB=40, BS=16, H=4, D=128, max_ctx=100):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_ctx + 1, (B,), generator=g).to(torch.int32)
    ctx[0] = BS  # exactly one full page
    MB = (max_ctx + BS - 1) // BS
    bt = torch.randperm(NB, generator=g)[: B * MB].reshape(B, MB).to(torch.int32) \
        if B * MB <= NB else torch.randint(0, NB, (B, MB), generator=g).to(torch.int32)
    kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    ks = torch.rand(NB, H, BS, generator=g) * 0.1
    vs = torch.rand(NB, H, BS, generator=g) * 0.1
    return W.DequantLayout(f"small{seed}", ctx, bt, NB, BS), (kc, vc, ks, vs)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("D,BS,H", [
    (128, 16, 4), (64, 32, 4),   # page-list kernels (the op passes a workspace)
    (128, 16, 3), (64, 16, 1),   # per-page kernel (heads not a power of two / small pages)
    (80, 16, 4), (128, 12, 4),   # scalar kernel (head size / block size off the vector path)
])
def test_dequant_modes_dtypes_layouts(tmo, ref, dev, out_dtype, mode, D, BS, H):
    layout, (kc, vc, ks, vs) = _small_layout(seed=D + BS + mode + H, D=D, BS=BS, NB=64, H=H)
    if mode == 0:
        g = torch.Generator().manual_seed(99)
        ks = torch.rand(H, D, generator=g) * 0.05
        vs = torch.rand(H, D, generator=g) * 0.05
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode)
    _dequant_both(tmo, ref, dev, layout, caches, out_dtype, mode, with_v=False)


@pytest.mark.parametrize("D,BS,H", [(128, 16, 4), (128, 16, 3), (80, 16, 4)])
def test_dequant_ignores_max_context_len(tmo, ref, dev, D, BS, H):
    """max_context_len understated, 0 and negative: every context_lengths[i] token is still
    dequantised (the reference math reads context_lengths only), on the page-list, per-page
    and scalar kernels."""
    layout, (kc, vc, ks, vs) = _small_layout(seed=7 * D + H, D=D, BS=BS, NB=64, H=H)
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    for mctx in (layout.max_context_len // 3, 1, 0, -1):
        print(f"[dequant] max_context_len={mctx} (true max {layout.max_context_len})", flush=True)
        _dequant_both(tmo, ref, dev, layout, caches, torch.bfloat16, 1, max_ctx=mctx)


def test_dequant_many_sequences(tmo, ref, dev):
    """More sequences than the persistent kernel keeps in LDS (per-page kernel), and a batch
    just below that limit (persistent kernel), with empty and single-token sequences."""
    for B in (4100, 3000):
        g = torch.Generator().manual_seed(B)
        ctx = torch.randint(0, 20, (B,), generator=g).to(torch.int32)
        NB, H, BS, D = 2 * B, 8, 16, 128
        bt = torch.randperm(NB, generator=g)[: 2 * B].reshape(B, 2).to(torch.int32)
        kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
        ks = torch.rand(NB, H, BS, generator=g)
        layout = W.DequantLayout(f"B={B}", ctx, bt, NB, BS)
        caches = (kc.to(dev), kc.to(dev), ks.to(dev), ks.to(dev))
        _dequant_both(tmo, ref, dev, layout, caches, torch.bfloat16, 1)


@pytest.mark.parametrize("B", [64, 65])
def test_dequant_batches_and_truncated_output(tmo, ref, dev, B):
    """Empty and one-token sequences, a missing page, both scale modes, K only, fp32 output,
    and fewer output rows than the context lengths sum (later rows are dropped)."""
    g = torch.Generator().manual_seed(B)
    ctx = torch.randint(0, 90, (B,), generator=g).to(torch.int32)
    ctx[3], ctx[5], ctx[B - 1] = 0, 1, 0
    NB, H, BS, D = 8 * B, 8, 16, 128
    bt = torch.randperm(NB, generator=g)[: 6 * B].reshape(B, 6).to(torch.int32)
    bt[7, 2] = -1                                   # a missing page inside a sequence
    kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    ks = torch.rand(NB, H, BS, generator=g) * 0.1
    vs = torch.rand(NB, H, BS, generator=g) * 0.1
    layout = W.DequantLayout(f"B={B}", ctx, bt, NB, BS)
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    print(f"[dequant] fine/persistent B={B} sum(ctx)={layout.total_tokens}", flush=True)
    _dequant_both(tmo, ref, dev, layout, caches, torch.bfloat16, 1)
    _dequant_both(tmo, ref, dev, layout, caches, torch.float32, 1, with_v=False)
    _dequant_both(tmo, ref, dev, layout, caches, torch.float16, 1, total=layout.total_tokens - 37)
    chan = (torch.rand(H, D, generator=g) * 0.05).to(dev), (torch.rand(H, D, generator=g) * 0.05).to(dev)
    _dequant_both(tmo, ref, dev, layout, (caches[0], caches[1]) + chan, torch.bfloat16, 0)


def _dequant_c_abi(out_k, out_v, caches, layout, mode, seq_offset, max_ctx, workspace):
    """tmo_hip_dequant_from_paged_cache through ctypes, with or without a workspace."""
    import ctypes
    from domesticated_torch_mlu_ops_amd import _loader
    L = _loader.c_abi()
    P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    L.tmo_hip_dequant_from_paged_cache.argtypes = [P, P] + [I64] * 5 + [P] * 7 + [I64] * 7 + \
        [INT] * 5 + [P, I64, P]
    L.tmo_hip_dequant_workspace_bytes.argtypes = [I64] * 4
    L.tmo_hip_dequant_workspace_bytes.restype = I64
    kc, vc, ks, vs = caches
    NB, H, BS, D = kc.shape
    ctx = layout.context_lengths.to(out_k.device)
    bt = layout.block_tables.to(out_k.device)
    off = seq_offset.to(out_k.device) if seq_offset is not None else None
    B, MB = bt.shape
    ws, ws_bytes = None, 0
    if workspace:
        ws_bytes = L.tmo_hip_dequant_workspace_bytes(B, MB, max_ctx, BS)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=out_k.device)
    dt = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[out_k.dtype]
    torch.cuda.synchronize()
    st = L.tmo_hip_dequant_from_paged_cache(
        out_k.data_ptr(), out_v.data_ptr() if out_v is not None else None, out_k.stride(0),
        out_k.stride(1), out_v.stride(0) if out_v is not None else 0,
        out_v.stride(1) if out_v is not None else 0, out_k.shape[0], kc.data_ptr(),
        vc.data_ptr() if out_v is not None else None, ks.data_ptr(),
        vs.data_ptr() if out_v is not None else None, ctx.data_ptr(),
        off.data_ptr() if off is not None else None, bt.data_ptr(), B, MB, max_ctx, NB, H, BS, D,
        mode, 8, dt, 3, 0, ws.data_ptr() if ws is not None else None, ws_bytes, None)
    torch.cuda.synchronize()
    assert st == 0


@pytest.mark.parametrize("B", [5, 70])
@pytest.mark.parametrize("mode", [0, 1])
def test_dequant_workspace_and_single_kernel_paths_agree(tmo, ref, dev, B, mode):
    """The C ABI without a workspace (one kernel: the persistent page-list kernel, or the
    per-page one) and with one (page-list pre-pass + item kernel) write identical bytes, and
    both match the oracle; with and without context_seq_offset."""
    layout, (kc, vc, ks, vs) = _small_layout(seed=40 + B + mode, B=B, NB=8 * B)
    if mode == 0:
        g = torch.Generator().manual_seed(7)
        ks, vs = torch.rand(4, 128, generator=g) * 0.05, torch.rand(4, 128, generator=g) * 0.05
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    total = layout.total_tokens + 5
    for off in (None, (torch.cumsum(layout.context_lengths, 0) - layout.context_lengths
                       + 3).to(torch.int32)):
        want_k = torch.full((total, 4, 128), -3.0).to(torch.bfloat16)
        want_v = want_k.clone()
        ref.dequant_from_paged_cache(want_k, want_v, kc, vc, ks, vs, layout.context_lengths, off,
                                     layout.block_tables, mode)
        for workspace in (False, True):
            got_k = torch.full((total, 4, 128), -3.0, device=dev).to(torch.bfloat16)
            got_v = got_k.clone()
            print(f"[dequant c-abi] B={B} mode={mode} offsets={off is not None} "
                  f"workspace={workspace}", flush=True)
            _dequant_c_abi(got_k, got_v, caches, layout, mode, off, layout.max_context_len,
                           workspace)
            assert_bits_equal(got_k, want_k, f"B={B} ws={workspace} key")
            assert_bits_equal(got_v, want_v, f"B={B} ws={workspace} value")


def test_dequant_seq_offset_invalid_blocks_and_extreme_scales(tmo, ref, dev):
    layout, (kc, vc, ks, vs) = _small_layout(seed=3, B=6, NB=64)
    bt = layout.block_tables.clone()
    bt[2, 1] = 64        # out of range: page skipped, its rows keep the sentinel
    bt[3, 0] = -1
    layout = W.DequantLayout("offsets", layout.context_lengths, bt, 64)
    ks[0, 0, 0] = 3e38   # code * scale overflows bf16 -> inf, like the oracle
    ks[1, 1, 1] = 1e-40  # subnormal scale
    off = torch.cumsum(layout.context_lengths, 0) - layout.context_lengths
    off = (off.flip(0) * 0 + off).to(torch.int32) + 7  # shifted start rows
    caches = tuple(t.to(dev) for t in (kc, vc, ks, vs))
    _dequant_both(tmo, ref, dev, layout, caches, torch.bfloat16, 1, seq_offset=off,
                  total=layout.total_tokens + 20)


# ---------------------------------------------------------------------------- scaled_quantize

def _sq_both(tmo, ref, dev, case: W.SmoothQuantCase, gather_start=None, smooth=True,
             x_dev=None):
    """x_dev: the GPU input when it must keep a layout .to() would not (e.g. a column slice)."""
    x = case.x
    rows = case.rows
    shape_scale = (rows,) + tuple(x.shape[1:-1])
    out_w = torch.full((rows,) + tuple(x.shape[1:]), W.CACHE_SENTINEL, dtype=torch.int8)
    sc_w = torch.full(shape_scale, W.SCALE_SENTINEL)
    sm = case.smooth if smooth else None
    ref.scaled_quantize_per_token(x, out_w, sc_w, sm, case.token_count, case.gather_index,
                                  gather_start)
    out_g = out_w.clone().fill_(W.CACHE_SENTINEL).to(dev)
    sc_g = torch.full_like(sc_w, W.SCALE_SENTINEL).to(dev)
    d = (lambda t: t.to(dev) if t is not None else None)
    xg = x.to(dev) if x_dev is None else x_dev
    if smooth:
        o, s = tmo.moe_quantize(xg, case.smooth.to(dev), None, d(case.token_count),
                                d(case.gather_index), d(gather_start), out_g, sc_g)
        assert o is out_g and s is sc_g
    else:
        torch.ops.torch_mlu_ops.scaled_quantize(
            xg, out_g, sc_g, None, None, d(case.token_count), d(case.gather_index),
            d(gather_start), None, "dynamic_per_token", "none", 1.0, False)
    assert_bits_equal(out_g, out_w, f"{case.name} output")
    assert_bits_equal(sc_g, sc_w, f"{case.name} output_scale")
    return out_g, sc_g


def test_smooth_quant_cfg4(tmo, ref, dev):
    _sq_both(tmo, ref, dev, W.cfg4())


def test_smooth_quant_cfg4_moe(tmo, ref, dev):
    case = W.cfg4_moe()
    _sq_both(tmo, ref, dev, case)
    # gather_index_start_position: rows gather_index[start : start + sum(token_count)]
    tc = case.token_count.clone()
    tc[40:] = 0
    case2 = W.SmoothQuantCase("moe-start", case.x, case.smooth, tc, case.gather_index)
    _sq_both(tmo, ref, dev, case2, gather_start=torch.tensor([37], dtype=torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("C", [4096, 7168, 512, 64, 16384, 100, 8])
def test_smooth_quant_widths(tmo, ref, dev, dtype, C):
    """Register-resident widths (1..16 vectors per lane), the generic path (C not a vector
    multiple, or more than 16 vectors per lane), and every dtype."""
    g = torch.Generator().manual_seed(C)
    x = (torch.randn(37, C, generator=g) * torch.logspace(-3, 3, 37)[:, None]).to(dtype)
    x[3] = 0
    smooth = 0.5 + 1.5 * torch.rand(C, generator=g)
    _sq_both(tmo, ref, dev, W.SmoothQuantCase(f"C={C} {dtype}", x, smooth))


@pytest.mark.parametrize("dtype,C,smooth", [
    (torch.bfloat16, 512, "channel"), (torch.bfloat16, 4096, "channel"),
    (torch.float16, 1024, "scalar"), (torch.float32, 1024, "none"), (torch.bfloat16, 2048, "none"),
])
def test_smooth_quant_many_rows_per_wavefront(tmo, ref, dev, dtype, C, smooth):
    """Large dense row counts that are not a multiple of any launch width (10573 and 4141 rows),
    with zero rows in the middle and at the very end, per-channel, scalar and no smooth."""
    g = torch.Generator().manual_seed(C + 7)
    rows = 2048 * 5 + 333 if C <= 2048 else 2048 * 2 + 45
    x = (torch.randn(rows, C, generator=g) * torch.logspace(-2, 2, rows)[:, None]).to(dtype)
    x[rows - 1] = 0
    x[17] = 0
    sm = {"channel": 0.5 + 1.5 * torch.rand(C, generator=g), "scalar": torch.tensor([0.625]),
          "none": torch.ones(C)}[smooth]
    _sq_both(tmo, ref, dev, W.SmoothQuantCase(f"{rows}x{C} {dtype} {smooth}", x, sm),
             smooth=smooth != "none")


@pytest.mark.parametrize("smooth", ["scalar", "none"])
def test_smooth_quant_dense_layouts(tmo, ref, dev, smooth):
    """The dense kernel (no gather, no groups, no or scalar smooth): 3-D [n0, inner, C] rows,
    and rows that are a column slice of wider rows (row stride C + 64)."""
    g = torch.Generator().manual_seed(77)
    sm = torch.tensor([0.8125]) if smooth == "scalar" else torch.ones(512)
    x3 = (torch.randn(300, 3, 512, generator=g) * 4).to(torch.bfloat16)
    x3[7, 1] = 0
    _sq_both(tmo, ref, dev, W.SmoothQuantCase(f"3d {smooth}", x3, sm), smooth=smooth == "scalar")
    wide = (torch.randn(1000, 512 + 64, generator=g) * 2).to(torch.bfloat16)
    xg = wide.to(dev)[:, :512]
    assert xg.stride(0) == 576
    _sq_both(tmo, ref, dev, W.SmoothQuantCase(f"strided {smooth}", wide[:, :512], sm),
             smooth=smooth == "scalar", x_dev=xg)


def test_smooth_quant_variants(tmo, ref, dev):
    g = torch.Generator().manual_seed(42)
    x = torch.randn(24, 3, 256, generator=g).to(torch.bfloat16)   # [n0, inner, C]
    # scalar smooth, no smooth, 3-D rows
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("3d scalar smooth", x, torch.tensor([1.75])))
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("3d no smooth", x, torch.ones(256)), smooth=False)
    # token_count grouping without gather, sum < rows: trailing rows untouched
    tc = torch.tensor([5, 0, 9, 6], dtype=torch.int32)
    sm = 0.5 + torch.rand(4, 256, generator=g)
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("groups", x, sm, tc))
    # gather with out-of-range entries: those rows untouched
    gi = torch.randint(0, 24, (30,), generator=g).to(torch.int32)
    gi[4] = 24
    gi[9] = -2
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("gather oob", x, torch.rand(256, generator=g) + 0.5,
                                              None, gi))


@pytest.mark.parametrize("dtype,C", [(torch.bfloat16, 512), (torch.bfloat16, 4096),
                                     (torch.float16, 2048), (torch.float32, 1024),
                                     (torch.float32, 2048), (torch.bfloat16, 8192)])
def test_smooth_quant_grouped_rows(tmo, ref, dev, dtype, C):
    """Gathered / grouped rows with per-group smooth rows (the per-workgroup LDS staging path):
    groups of 0-3 rows so that groups start and end inside workgroups of 4 rows, long groups,
    more than 64 groups, token_count summing past and short of the row count,
    gather_index_start_position, out-of-range gather entries, groups without gather, and
    gather without groups (one per-channel smooth vector)."""
    g = torch.Generator().manual_seed(C + 11)
    n0 = 97
    x = (torch.randn(n0, C, generator=g) * torch.logspace(-2, 2, n0)[:, None]).to(dtype)
    x[5] = 0
    counts = [0, 1, 2, 3, 0, 0, 5, 1, 1, 17, 2, 0, 3, 40, 1, 2] * 9  # 144 groups, 702 rows
    tc = torch.tensor(counts, dtype=torch.int32)
    E = tc.numel()
    rows = int(tc.sum())
    gi = torch.randint(0, n0, (rows,), generator=g).to(torch.int32)
    gi[7] = n0          # out of range: row not produced
    gi[300] = -1
    sm = 0.5 + torch.rand(E, C, generator=g)
    _sq_both(tmo, ref, dev, W.SmoothQuantCase(f"groups {dtype} C={C}", x, sm, tc, gi))
    # token_count summing short of the gathered rows (trailing rows untouched) and past them
    tc_short = tc.clone()
    tc_short[100:] = 0
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("short", x, sm, tc_short, gi))
    tc_long = tc.clone()
    tc_long[-1] += 50
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("long", x, sm, tc_long, gi))
    # gather_index_start_position: rows gather_index[start : start + sum(token_count)]
    tc_start = tc.clone()
    tc_start[120:] = 0
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("start", x, sm, tc_start, gi),
             gather_start=torch.tensor([29], dtype=torch.int32))
    # groups without gather (rows of x in order), and gather without groups
    tc_rows = torch.tensor([0, 3, 1, 0, 2, 40, 7, 1, 1, 30], dtype=torch.int32)  # 85 of 97 rows
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("groups, no gather", x,
                                              0.5 + torch.rand(10, C, generator=g), tc_rows))
    _sq_both(tmo, ref, dev, W.SmoothQuantCase("gather, no groups", x,
                                              0.5 + torch.rand(C, generator=g), None, gi))


def test_public_wrappers(tmo, ref, dev):
    """scaled_quantize and the per_token_smooth_quantize alias return what moe_quantize does."""
    case = W.cfg4()
    x = case.x[:512].to(dev)
    sm = case.smooth.to(dev)
    o1, s1 = tmo.moe_quantize(x, sm)
    o2, s2 = tmo.scaled_quantize(x, sm)
    o3, s3 = tmo.per_token_smooth_quantize(x, sm)
    for o, s in ((o2, s2), (o3, s3)):
        assert_bits_equal(o, o1, "output")
        assert_bits_equal(s, s1, "scale")
    with pytest.raises(RuntimeError):
        tmo.scaled_quantize(x, sm, quant_mode="dynamic_per_tensor")
