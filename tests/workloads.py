"""Seeded synthetic inputs of the five benchmark configurations (BASELINE.json ``configs``).

Shared by the parity tests and ``bench.py``.  Everything is drawn on the CPU from
``torch.Generator().manual_seed(1000 + cfg)`` in the order written below (fp32 normals,
rounded to bf16 with torch's round-to-nearest-even), so a GPU run and the CPU oracle see
identical bits after a copy.  Config 5's pages are filled on the device (see ``cfg5_fill``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

H, D, BS = 8, 128, 16
CACHE_SENTINEL = 0x5A          # int8 pattern of never-written cache bytes
SCALE_SENTINEL = -12345.0      # fp32 pattern of never-written scale slots


def _gen(cfg: int) -> torch.Generator:
    return torch.Generator().manual_seed(1000 + cfg)


@dataclass
class PagedQuantCase:
    """Inputs of quant_to_paged_cache / reshape_paged_cache (CPU tensors)."""
    name: str
    k: torch.Tensor
    v: torch.Tensor
    slot_mapping: torch.Tensor
    num_blocks: int
    block_size: int = BS

    @property
    def tokens(self) -> int:
        return self.k.shape[0]

    def empty_caches(self, device="cpu", dtype=torch.int8):
        shape = (self.num_blocks, self.k.shape[1], self.block_size, self.k.shape[2])
        if dtype == torch.int8:
            kc = torch.full(shape, CACHE_SENTINEL, dtype=torch.int8, device=device)
        else:
            kc = torch.full(shape, -7.0, dtype=dtype, device=device)
        vc = kc.clone()
        ks = torch.full(shape[:3], SCALE_SENTINEL, dtype=torch.float32, device=device)
        vs = ks.clone()
        return kc, vc, ks, vs

    def valid_tokens(self) -> int:
        return int((self.slot_mapping >= 0).sum())

    def algorithmic_bytes(self) -> int:
        """Bytes quant_to_paged_cache must touch once: valid K/V rows read, codes and scales
        written, slot_mapping read."""
        t_valid = self.valid_tokens()
        heads, dim = self.k.shape[1], self.k.shape[2]
        es = self.k.element_size()
        return 2 * t_valid * heads * (dim * es + dim + 4) + 4 * self.tokens


def cfg1() -> PagedQuantCase:
    """16 tokens x 8 heads x 128, bf16 ~N(0,1); 64 blocks x 16; slots = randperm(1024)[:16]."""
    g = _gen(1)
    k = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(16, H, D, generator=g).to(torch.bfloat16)
    slot = torch.randperm(64 * BS, generator=g)[:16].to(torch.int32)
    return PagedQuantCase("cfg1", k, v, slot, 64)


def cfg2() -> PagedQuantCase:
    """Decode step: 256 tokens; 16384 blocks; unique random slots, 26 (10%) set to -1."""
    g = _gen(2)
    k = torch.randn(256, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(256, H, D, generator=g).to(torch.bfloat16)
    slot = torch.randperm(16384 * BS, generator=g)[:256].to(torch.int32)
    pad = torch.randperm(256, generator=g)[:26]
    slot[pad] = -1
    return PagedQuantCase("cfg2", k, v, slot, 16384)


def cfg3() -> PagedQuantCase:
    """Prefill chunk: 32768 tokens (8 sequences x 4096 contiguous slots at random block
    offsets); one channel per head scaled x20 in K and V."""
    g = _gen(3)
    k = torch.randn(32768, H, D, generator=g)
    v = torch.randn(32768, H, D, generator=g)
    ch = torch.randint(0, D, (H,), generator=g)
    for h in range(H):
        k[:, h, ch[h]] *= 20.0
        v[:, h, ch[h]] *= 20.0
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    starts = 256 * torch.randperm(256, generator=g)[:8]
    slot = torch.cat([BS * s + torch.arange(4096) for s in starts.tolist()]).to(torch.int32)
    return PagedQuantCase("cfg3", k, v, slot, 65536)


@dataclass
class SmoothQuantCase:
    name: str
    x: torch.Tensor
    smooth: torch.Tensor
    token_count: Optional[torch.Tensor] = None
    gather_index: Optional[torch.Tensor] = None

    @property
    def rows(self) -> int:
        return self.gather_index.numel() if self.gather_index is not None else self.x.shape[0]

    def algorithmic_bytes(self, per_row_reads: bool = False) -> int:
        C = self.x.shape[-1]
        es = self.x.element_size()
        if self.gather_index is None:
            reads = self.x.shape[0] * C * es
        elif per_row_reads:
            reads = self.rows * C * es
        else:
            reads = int(torch.unique(self.gather_index).numel()) * C * es
        idx = 0
        if self.gather_index is not None:
            idx += 4 * self.gather_index.numel()
        if self.token_count is not None:
            idx += 4 * self.token_count.numel()
        return reads + self.rows * (C + 4) + self.smooth.numel() * 4 + idx


def _heavy_tail_x(g: torch.Generator, rows: int, C: int) -> torch.Tensor:
    x = torch.randn(rows, C, generator=g)
    ch = torch.randperm(C, generator=g)[: round(0.01 * C)]
    z = torch.randn(rows, ch.numel(), generator=g)
    chi2 = torch.randn(rows, ch.numel(), 3, generator=g).pow(2).sum(-1)
    x[:, ch] = z / torch.sqrt(chi2 / 3.0)  # Student-t, 3 degrees of freedom
    return x.to(torch.bfloat16)


def cfg4() -> SmoothQuantCase:
    """8192 x 4096 bf16 with 41 Student-t(3) channels; smooth ~ U[0.5, 2)."""
    g = _gen(4)
    x = _heavy_tail_x(g, 8192, 4096)
    smooth = 0.5 + 1.5 * torch.rand(4096, generator=g)
    return SmoothQuantCase("cfg4", x, smooth)


def cfg4_moe() -> SmoothQuantCase:
    """MoE variant: top-2 of 64 experts -> 16384 gathered rows sorted by expert; per-expert
    smooth [64, 4096]."""
    g = _gen(4)
    x = _heavy_tail_x(g, 8192, 4096)
    _ = torch.rand(4096, generator=g)  # the dense variant's smooth, keeps the streams aligned
    logits = torch.randn(8192, 64, generator=g)
    experts = logits.topk(2, dim=-1).indices.reshape(-1)          # token-major [16384]
    order = torch.sort(experts, stable=True).indices
    gather_index = (order // 2).to(torch.int32)                     # source token of each row
    token_count = torch.bincount(experts, minlength=64).to(torch.int32)
    smooth = 0.5 + 1.5 * torch.rand(64, 4096, generator=g)
    return SmoothQuantCase("cfg4_moe", x, smooth, token_count, gather_index)


@dataclass
class DequantLayout:
    """Sequences and block tables of dequant_from_paged_cache (CPU int32 tensors)."""
    name: str
    context_lengths: torch.Tensor
    block_tables: torch.Tensor
    num_blocks: int
    block_size: int = BS

    @property
    def total_tokens(self) -> int:
        return int(self.context_lengths.sum())

    @property
    def max_context_len(self) -> int:
        return int(self.context_lengths.max())

    def algorithmic_bytes(self, heads: int = H, dim: int = D, out_bytes: int = 2) -> int:
        """Per token and head: K+V codes read, K+V scales read, K+V rows written; plus the
        block-table entries and context lengths read."""
        pages = int(((self.context_lengths + self.block_size - 1) // self.block_size).sum())
        per_tok = 2 * heads * (dim + 4 + dim * out_bytes)
        return self.total_tokens * per_tok + 4 * pages + 4 * self.context_lengths.numel()


def cfg5() -> DequantLayout:
    """64 sequences, ctx ~ U[1024, 32768]; block_tables [64, 2048] from randperm(131072)."""
    g = _gen(5)
    ctx = torch.randint(1024, 32769, (64,), generator=g).to(torch.int32)
    bt = torch.randperm(131072, generator=g).to(torch.int32).reshape(64, 2048)
    return DequantLayout("cfg5", ctx, bt, 131072)


def cfg5_fill(layout: DequantLayout, device, seed: int = 1005, heads: int = H, dim: int = D,
              cache_dtype=torch.int8):
    """Int8 (or float8_e4m3fn, ``cache_dtype``) pages + fp32 per-token scales for every page a
    sequence of ``layout`` uses, produced the way a serving engine fills them: config-3-style
    bf16 K/V (N(0,1), one x20 channel per head) quantised with quant_to_paged_cache on
    ``device``.  Generated on the device (a CPU draw of ~2e9 values would dominate the run);
    unused pages keep the sentinel.  Returns (k_cache, v_cache, k_scale, v_scale)."""
    import domesticated_torch_mlu_ops_amd as tmo

    NB, bs = layout.num_blocks, layout.block_size
    kc = torch.full((NB, heads, bs, dim), CACHE_SENTINEL, dtype=torch.uint8,
                    device=device).view(cache_dtype)
    vc = torch.full((NB, heads, bs, dim), CACHE_SENTINEL, dtype=torch.uint8,
                    device=device).view(cache_dtype)
    ks = torch.full((NB, heads, bs), SCALE_SENTINEL, dtype=torch.float32, device=device)
    vs = torch.full_like(ks, SCALE_SENTINEL)
    g = torch.Generator(device=device).manual_seed(seed)
    bt = layout.block_tables.to(device)
    ch = torch.randint(0, dim, (heads,), generator=g, device=device)
    scale = torch.ones(heads, dim, device=device)
    scale[torch.arange(heads, device=device), ch] = 20.0
    for i, n in enumerate(layout.context_lengths.tolist()):
        t = torch.arange(n, device=device)
        slots = (bt[i, t // bs].to(torch.int64) * bs + t % bs).to(torch.int32)
        k = (torch.randn(n, heads, dim, generator=g, device=device) * scale).to(torch.bfloat16)
        v = (torch.randn(n, heads, dim, generator=g, device=device) * scale).to(torch.bfloat16)
        tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, slots)
    return kc, vc, ks, vs


def fused_rope_case(dtype, mode, seed, B=3, S=20, Hq=4, Hk=2, D=128, rope=128, NB=12, BS=16,
                    maxpos=128, positions=(0, 7, 40, 120)):
    """Inputs of a fused_rope / fused_rmsnorm_rope_store_paged_cache call: qkv [B, S, Hq+2Hk, D]
    with magnitudes spread over S, a zero K row, sin/cos tables of `maxpos` rows (a sequence
    starting at 120 runs past the table), gammas ~U[0.5, 1.5), slots with -1 entries, and
    caches / scales for mode "none" (qkv's dtype), "dynamic" or "static" (int8)."""
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(B, S, Hq + 2 * Hk, D, generator=g) * torch.logspace(-2, 1, S)[None, :, None, None]).to(dtype)
    qkv[1, 3, Hq] = 0                                        # a zero K row
    ang = torch.arange(maxpos)[:, None] * (0.5 ** (torch.arange(rope // 2) / 8.0))[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    sin, cos = torch.sin(ang).to(dtype), torch.cos(ang).to(dtype)
    position_id = torch.tensor(list(positions)[:B], dtype=torch.int32)
    k_gamma = (0.5 + torch.rand(D, generator=g)).to(dtype)
    q_gamma = (0.5 + torch.rand(D, generator=g)).to(dtype)
    slot = torch.randperm(NB * BS, generator=g)[:B * S].to(torch.int32)
    slot[::7] = -1
    cdt = dtype if mode == "none" else torch.int8
    kc = torch.zeros(NB, Hk, BS, D, dtype=cdt)
    vc = torch.zeros_like(kc)
    if mode == "dynamic":
        ks, vs = torch.full((NB, Hk, BS), -1.0), torch.full((NB, Hk, BS), -1.0)
    elif mode == "static":
        ks = 0.005 + 0.02 * torch.rand(Hk, D, generator=g)
        vs = 0.005 + 0.02 * torch.rand(Hk, D, generator=g)
    else:
        ks = vs = None
    return qkv, kc, vc, sin, cos, position_id, k_gamma, q_gamma, ks, vs, slot


@dataclass
class LinearCase:
    """Inputs of the linear-cache ops: token-major K/V (packed [T, H, D] or padded
    [B, S, H, D]), sequence lengths and the optional offset / batch-id tensors (CPU)."""
    key: torch.Tensor
    value: torch.Tensor
    lens: torch.Tensor                        # [B] lengths
    packed: bool
    context_seq_offset: Optional[torch.Tensor]
    cache_bs_id: Optional[torch.Tensor]
    cache_seq_offset: Optional[torch.Tensor]
    cache_batch: int
    cache_len: int

    @property
    def context_lengths(self) -> torch.Tensor:
        """The write ops' context_lengths: batch + 1 prefix offsets when packed."""
        if not self.packed:
            return self.lens
        return torch.cat((torch.zeros(1, dtype=torch.int32), self.lens.cumsum(0).to(torch.int32)))

    @property
    def max_context_len(self) -> int:
        return int(self.lens.max()) if self.lens.numel() else 0

    def caches(self, dtype, fill=CACHE_SENTINEL):
        """Sentinel-filled [cache_batch, H, cache_len, D] caches of `dtype`."""
        H, D = self.key.shape[-2], self.key.shape[-1]
        shape = (self.cache_batch, H, self.cache_len, D)
        if dtype in (torch.int8, torch.float8_e4m3fn):
            return tuple(torch.full(shape, fill, dtype=torch.uint8).view(dtype) for _ in range(2))
        return tuple(torch.full(shape, -7.0, dtype=dtype) for _ in range(2))

    def scales(self, groups: int = 0):
        """Sentinel-filled per-token scales [cache_batch, H, cache_len] (or [..., groups])."""
        H = self.key.shape[-2]
        shape = (self.cache_batch, H, self.cache_len) + ((groups,) if groups else ())
        return torch.full(shape, SCALE_SENTINEL), torch.full(shape, SCALE_SENTINEL)


def linear_case(dtype, seed: int, packed: bool = True, offsets: bool = False, B: int = 5,
                H: int = 2, D: int = 64, S: int = 24, cache_batch: int = 7,
                cache_len: int = 40) -> LinearCase:
    """Sequences of random lengths in [0, S] (the first full, the second empty) with
    magnitudes spread over tokens and a zero row.  With `offsets`: non-overlapping shuffled
    token segments with gaps (context_seq_offset), a cache batch permutation with one
    negative id, and cache position offsets of which one runs past cache_len."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, S + 1, (B,), generator=g).to(torch.int32)
    lens[0] = S
    if B > 1:
        lens[1] = 0
    cso = bsi = coff = None
    if packed:
        rows = int(lens.sum())
        if offsets:
            order = torch.randperm(B, generator=g).tolist()
            gaps = torch.randint(0, 4, (B,), generator=g).tolist()
            cso = torch.zeros(B, dtype=torch.int32)
            at = 0
            for i, gap in zip(order, gaps):
                at += gap
                cso[i] = at
                at += int(lens[i])
            rows = at + 2
        scale = torch.logspace(-3, 2, rows)[:, None, None]
        key = (torch.randn(rows, H, D, generator=g) * scale).to(dtype)
        value = (torch.randn(rows, H, D, generator=g) * 3).to(dtype)
        key[min(2, rows - 1)] = 0
    else:
        scale = torch.logspace(-3, 2, S)[None, :, None, None]
        key = (torch.randn(B, S, H, D, generator=g) * scale).to(dtype)
        value = (torch.randn(B, S, H, D, generator=g) * 3).to(dtype)
        key[0, 1] = 0
        if offsets:  # absolute rows of the flattened [B * S] tensor, inside each sequence
            cso = torch.tensor([i * S + int(torch.randint(0, S - int(lens[i]) + 1, (1,),
                                                           generator=g)) for i in range(B)],
                               dtype=torch.int32)
    if offsets:
        bsi = torch.randperm(cache_batch, generator=g)[:B].to(torch.int32)
        bsi[-1] = -1
        coff = torch.tensor([int(torch.randint(0, max(1, cache_len - int(n) + 1), (1,), generator=g))
                             for n in lens], dtype=torch.int32)
        if B > 2:
            coff[2] = cache_len - max(1, int(lens[2]) // 2)     # runs past the cache's end
    return LinearCase(key, value, lens, packed, cso, bsi, coff, cache_batch, cache_len)


@dataclass
class AttnCase:
    """Inputs of single_query_cached_kv_attn for one query token per sequence (CPU)."""
    q: torch.Tensor                  # [B, Hq, D]
    k_cache: torch.Tensor            # [NB, Hkv, BS, D]
    v_cache: torch.Tensor
    k_scale: Optional[torch.Tensor]  # int8: [NB, Hkv, BS] per token, [Hkv, D] per channel, or
                                     # per group K [NB, Hkv, BS, D / 32], V [NB, Hkv, BS / 32, D]
    v_scale: Optional[torch.Tensor]
    block_tables: torch.Tensor       # [B, max_blocks] int32
    context_lens: torch.Tensor       # [B] int32
    alibi: Optional[torch.Tensor] = None
    int4: bool = False               # int8 caches of 4-bit pairs (kv_cache_quant_bit_size 4)

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max()) if self.context_lens.numel() else 0


def fp8_codes(shape, g) -> torch.Tensor:
    """float8_e4m3fn cache values as a quantiser leaves them: N(0, 1) * 96 rounded to e4m3fn
    (torch's RNE cast) and clipped to +-448, with every 97th value replaced by a subnormal
    code (|m| * 2^-9) and every 211th by +-448."""
    x = (torch.randn(shape, generator=g) * 96).clamp(-448, 448)
    flat = x.view(-1)
    sub = torch.randint(1, 8, flat[::97].shape, generator=g).to(torch.float32) * 2.0 ** -9
    flat[::97] = torch.where(flat[::97] < 0, -sub, sub)
    flat[::211] = torch.where(flat[::211] < 0, -448.0, 448.0)
    return x.to(torch.float8_e4m3fn)


def pack_int4(codes: torch.Tensor, dim: int) -> torch.Tensor:
    """Signed 4-bit codes (int8 in [-8, 7]) -> int8 bytes of pairs along `dim`: the even
    element in the high nibble, the odd one in the low nibble."""
    c = codes.movedim(dim, -1).to(torch.int16)
    b = ((c[..., 0::2] & 0xF) << 4) | (c[..., 1::2] & 0xF)
    return b.to(torch.uint8).view(torch.int8).movedim(-1, dim).contiguous()


def unpack_int4(b: torch.Tensor, dim: int) -> torch.Tensor:
    """pack_int4's inverse: int8 bytes of 4-bit pairs along `dim` -> int8 codes in [-8, 7]."""
    u = b.movedim(dim, -1).view(torch.uint8).to(torch.int16)
    hi, lo = (u >> 4) & 0xF, u & 0xF
    c = torch.stack([hi, lo], dim=-1).reshape(u.shape[:-1] + (2 * u.shape[-1],))
    c = torch.where(c >= 8, c - 16, c)
    return c.to(torch.int8).movedim(-1, dim).contiguous()


def attn_case(dtype, seed: int, kv: str = "int8_token", B: int = 5, Hq: int = 8, Hkv: int = 2,
              D: int = 128, BS: int = 16, NB: int = 64, max_ctx: int = 200,
              alibi: bool = False, scale_dtype=torch.float32,
              v_pairs: str = "rows") -> AttnCase:
    """Decode attention inputs: q ~ N(0, 1) in `dtype`; caches int8 (`kv` "int8_token" /
    "int8_channel" / "int8_group", codes uniform in [-127, 127] with scales ~U[0.005, 0.03)),
    float8_e4m3fn (`kv` "fp8_token" / "fp8_channel" / "fp8_group", fp8_codes with scales
    ~U[0.0003, 0.0015)), scales in `scale_dtype` (float32 or bfloat16), or of q's dtype
    (`kv` "plain", N(0, 1)); or int4 pairs (`kv` "int4_token" / "int4_channel" / "int4_group",
    codes uniform in [-8, 7], scales ~U[0.05, 0.3)): K [NB, Hkv, BS, D / 2] pairing channels, V
    [NB, Hkv, BS / 2, D] pairing rows (`v_pairs` "rows") or [NB, Hkv, BS, D / 2] (`v_pairs`
    "channels"); context lengths in [1, max_ctx] (the first max_ctx, one 1); each sequence's
    pages a random choice of distinct blocks."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    lens = torch.randint(1, max_ctx + 1, (B,), generator=g).to(torch.int32)
    lens[0] = max_ctx
    if B > 1:
        lens[1] = 1
    MB = (max_ctx + BS - 1) // BS
    assert B * MB <= NB, "not enough blocks for distinct pages"
    bt = torch.randperm(NB, generator=g)[:B * MB].reshape(B, MB).to(torch.int32)
    ks = vs = None
    if kv.startswith("int8") or kv.startswith("fp8") or kv.startswith("int4"):
        form = kv.split("_")[1]
        if kv.startswith("int4"):
            kc = pack_int4(torch.randint(-8, 8, (NB, Hkv, BS, D), generator=g, dtype=torch.int8), 3)
            vcodes = torch.randint(-8, 8, (NB, Hkv, BS, D), generator=g, dtype=torch.int8)
            vc = pack_int4(vcodes, 2 if v_pairs == "rows" else 3)
            lo, span = 0.05, 0.25
        elif kv.startswith("int8"):
            kc = torch.randint(-127, 128, (NB, Hkv, BS, D), generator=g, dtype=torch.int8)
            vc = torch.randint(-127, 128, (NB, Hkv, BS, D), generator=g, dtype=torch.int8)
            lo, span = 0.005, 0.025
        else:
            kc = fp8_codes((NB, Hkv, BS, D), g)
            vc = fp8_codes((NB, Hkv, BS, D), g)
            lo, span = 0.0003, 0.0012
        shape = {"token": (NB, Hkv, BS), "channel": (Hkv, D), "group": (NB, Hkv, BS, D // 32)}[form]
        ks = (lo + span * torch.rand(shape, generator=g)).to(scale_dtype)
        vshape = (NB, Hkv, BS // 32, D) if form == "group" else shape
        vs = (lo + span * torch.rand(vshape, generator=g)).to(scale_dtype)
    else:
        kc = torch.randn(NB, Hkv, BS, D, generator=g).to(dtype)
        vc = torch.randn(NB, Hkv, BS, D, generator=g).to(dtype)
    al = (0.5 ** torch.arange(1, Hq + 1, dtype=torch.float32)).repeat(B, 1) if alibi else None
    return AttnCase(q, kc, vc, ks, vs, bt, lens, al, int4=kv.startswith("int4"))


def attn_queries(dtype, seed: int, B: int, Hq: int, D: int, S: Optional[int] = None,
                 counts: Optional[list] = None):
    """Query tokens for several per sequence, q ~ N(0, 1) in `dtype`: S each -> q [B, S, Hq,
    D] (the reference's 4-D form); or `counts[i]` for sequence i -> (q [T, Hq, D], cu_seq_q
    [B + 1] int32), T = sum(counts) (the 3-D form with cu_seq_q)."""
    g = torch.Generator().manual_seed(seed)
    if counts is None:
        return torch.randn(B, S, Hq, D, generator=g).to(dtype)
    assert len(counts) == B
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(counts, dtype=torch.int32).cumsum(0)
    return torch.randn(int(cu[-1]), Hq, D, generator=g).to(dtype), cu
