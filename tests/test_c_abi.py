"""The C ABI (include/tmo_hip.h) of libtmo_hip.so, checked on the CPU: the library loads,
exports every declared entry point, and rejects invalid arguments with the documented status
codes before touching any device memory (the pointers below are never dereferenced)."""
import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "tmo_hip.h"

P = ctypes.c_void_p
I64 = ctypes.c_int64
INT = ctypes.c_int
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(tmo_hip_\w+)\s*\(",
                                 text, re.M)))


def header_enum(name):
    m = re.search(rf"\b{name}\s*=\s*(-?\d+)", HEADER.read_text())
    return int(m.group(1))


@pytest.fixture(scope="module")
def lib():
    from domesticated_torch_mlu_ops_amd import _loader
    L = _loader.c_abi()
    L.tmo_hip_status_string.restype = ctypes.c_char_p
    L.tmo_hip_quant_to_paged_cache.argtypes = [P, P] + [I64] * 4 + [P] * 5 + [I64] * 5 + [INT, INT, P]
    L.tmo_hip_reshape_paged_cache.argtypes = [P, P] + [I64] * 4 + [P] * 3 + [I64] * 5 + [INT, INT, P]
    L.tmo_hip_dequant_from_paged_cache.argtypes = [P, P] + [I64] * 5 + [P] * 7 + [I64] * 7 + \
        [INT] * 5 + [P, I64, P]
    L.tmo_hip_dequant_workspace_bytes.argtypes = [I64] * 4
    L.tmo_hip_dequant_workspace_bytes.restype = I64
    L.tmo_hip_scaled_quantize_per_token.argtypes = [P] + [I64] * 4 + [P] * 3 + [I64, P, I64, P, I64, P, I64, INT, P]
    L.tmo_hip_fused_rope_paged.argtypes = [P] + [I64] * 5 + [P, P] + [I64] * 4 + [P, I64, P, P, P] + \
        [ctypes.c_float, INT] + [P] * 4 + [INT, P, I64, I64, INT, P]
    L.tmo_hip_fused_rope_linear.argtypes = [P] + [I64] * 5 + [P, P] + [I64] * 4 + [P, I64, P, P, P] + \
        [ctypes.c_float, INT] + [P] * 4 + [INT, P, P, I64, I64, INT, P]
    L.tmo_hip_offline_quant_to_paged_cache.argtypes = [P, P] + [I64] * 4 + [P] * 4 + \
        [ctypes.c_float] * 2 + [P] + [I64] * 5 + [INT, INT, P]
    L.tmo_hip_reshape_linear_cache.argtypes = [P, P] + [I64] * 5 + [P, P] + [I64] * 4 + \
        [P, I64, I64, INT, I64, P, P, P, INT, P]
    L.tmo_hip_quant_to_linear_cache.argtypes = [P, P] + [I64] * 5 + [P] * 4 + [I64] * 5 + \
        [P, I64, I64, INT, I64, P, P, P, INT, INT, INT, P]
    L.tmo_hip_offline_quant_to_linear_cache.argtypes = [P, P] + [I64] * 5 + [P] * 4 + \
        [ctypes.c_float] * 2 + [INT] + [I64] * 4 + [P, I64, I64, INT, I64, P, P, P, INT, INT, P]
    L.tmo_hip_dequant_from_linear_cache.argtypes = [P, P] + [I64] * 5 + [P] * 4 + [I64] * 4 + \
        [P, I64, I64, P, P, P, INT, INT, INT, P]
    L.tmo_hip_reshape_from_cache.argtypes = [P, P] + [I64] * 5 + [P, P] + [I64] * 4 + \
        [P, I64, I64, P, P, I64, P, INT, P]
    L.tmo_hip_single_query_cached_kv_attn.argtypes = [P, I64, I64, P, P, P, P, INT, P, I64, P, P,
                                                      P, I64, I64, P, I64, I64] + [I64] * 8 + \
        [ctypes.c_float, INT, INT, I64, P, I64, P]
    L.tmo_hip_attn_workspace_bytes.argtypes = [I64] * 6
    L.tmo_hip_attn_workspace_bytes.restype = I64
    L.tmo_hip_cached_kv_attn.argtypes = [P, I64, I64, I64, P, INT, INT, I64, I64, I64, I64,
                                         P, I64, I64, P, P, I64, I64, P, P, INT,
                                         INT, I64, I64, I64, I64, P, I64, I64, P, P, P,
                                         P, INT, I64, I64, I64,
                                         P, I64, I64, I64,
                                         P, I64, I64, I64] + [I64] * 9 + \
        [ctypes.c_float, INT, INT, INT, INT, I64, P, I64, P]
    L.tmo_hip_cached_kv_attn_workspace_bytes.argtypes = [I64] * 6
    L.tmo_hip_cached_kv_attn_workspace_bytes.restype = I64
    return L


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert set(names) == {"tmo_hip_abi_version", "tmo_hip_status_string",
                          "tmo_hip_reshape_paged_cache", "tmo_hip_quant_to_paged_cache",
                          "tmo_hip_dequant_from_paged_cache", "tmo_hip_dequant_workspace_bytes",
                          "tmo_hip_dequant_from_paged_cache_noalloc",
                          "tmo_hip_scaled_quantize_per_token",
                          "tmo_hip_offline_quant_to_paged_cache", "tmo_hip_fused_rope_paged",
                          "tmo_hip_fused_rope_linear", "tmo_hip_reshape_linear_cache", "tmo_hip_quant_to_linear_cache",
                          "tmo_hip_offline_quant_to_linear_cache",
                          "tmo_hip_dequant_from_linear_cache", "tmo_hip_reshape_from_cache",
                          "tmo_hip_single_query_cached_kv_attn", "tmo_hip_attn_workspace_bytes",
                          "tmo_hip_cached_kv_attn", "tmo_hip_cached_kv_attn_workspace_bytes"}
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_and_status_strings(lib):
    m = re.search(r"#define\s+TMO_HIP_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert lib.tmo_hip_abi_version() == int(m.group(1))
    for name in ("TMO_OK", "TMO_ERR_INVALID_ARGUMENT", "TMO_ERR_UNSUPPORTED_DTYPE",
                 "TMO_ERR_UNSUPPORTED_MODE", "TMO_ERR_LAUNCH"):
        s = lib.tmo_hip_status_string(header_enum(name))
        assert s and s != b"unknown status"
    assert lib.tmo_hip_status_string(12345) == b"unknown status"


EINVAL = -1
EDTYPE = -2
EMODE = -3


def quant(lib, k=FAKE, v=None, kc=FAKE, vc=None, ks=FAKE, vs=None, slot=FAKE, T=4, H=8, D=128,
          NB=4, BS=16, dtype=2, st=1024, sh=128, cdt=3):
    return lib.tmo_hip_quant_to_paged_cache(k, v, st, sh, st, sh, kc, vc, ks, vs, slot, T, H, D,
                                            NB, BS, dtype, cdt, None)


def test_quant_validation(lib):
    assert quant(lib, dtype=3) == EDTYPE          # int8 input
    assert quant(lib, cdt=2) == EDTYPE            # bf16 cache
    assert quant(lib, cdt=4, T=0) == 0            # float8_e4m3fn cache
    assert quant(lib, dtype=9) == EDTYPE
    assert quant(lib, k=None) == EINVAL
    assert quant(lib, slot=None) == EINVAL
    assert quant(lib, v=FAKE) == EINVAL           # v without v_cache / v_scale
    assert quant(lib, v=FAKE, vc=FAKE) == EINVAL
    assert quant(lib, H=0) == EINVAL
    assert quant(lib, D=-1) == EINVAL
    assert quant(lib, BS=0) == EINVAL
    assert quant(lib, T=-1) == EINVAL
    assert quant(lib, st=-5) == EINVAL
    assert quant(lib, T=0) == 0                   # nothing to do: success, nothing enqueued
    assert quant(lib, NB=0) == 0


def test_reshape_validation(lib):
    def call(dtype=2, k=FAKE, v=None, vc=None, H=8, BS=16, T=4):
        return lib.tmo_hip_reshape_paged_cache(k, v, 1024, 128, 1024, 128, FAKE, vc, FAKE, T, H,
                                               128, 4, BS, dtype, 0, None)
    assert call(dtype=7) == EDTYPE
    assert call(k=None) == EINVAL
    assert call(v=FAKE) == EINVAL
    assert call(H=-2) == EINVAL
    assert call(BS=0) == EINVAL
    assert call(T=0) == 0


def test_dequant_validation(lib):
    def call(mode=1, bit=8, dtype=2, key=FAKE, value=None, vc=None, vs=None, B=2, H=8, total=10,
             ws=None, ws_bytes=0, cdt=3, sdt=0):
        return lib.tmo_hip_dequant_from_paged_cache(
            key, value, 1024, 128, 1024, 128, total, FAKE, vc, FAKE, vs, FAKE, None, FAKE, B, 4,
            64, 16, H, 16, 128, mode, bit, dtype, cdt, sdt, ws, ws_bytes, None)
    assert call(ws_bytes=-1) == EINVAL
    assert call(ws_bytes=64) == EINVAL          # bytes without a pointer
    assert call(mode=2) == EMODE
    assert call(bit=4) == EMODE
    assert call(dtype=3) == EDTYPE
    assert call(cdt=2) == EDTYPE                # caches: int8 or float8_e4m3fn
    assert call(sdt=1) == EDTYPE                # scales: fp32 or bf16
    assert call(cdt=4, sdt=2, B=0) == 0         # float8_e4m3fn pages, bf16 scales
    assert call(key=None) == EINVAL
    assert call(value=FAKE) == EINVAL
    assert call(H=0) == EINVAL
    assert call(B=-1) == EINVAL
    assert call(B=0) == 0
    assert call(total=0) == 0


def test_dequant_noalloc_validation(lib):
    """The allocation-free dequant refuses, before touching the GPU, a call whose page list
    would not fit the library's static scratch (TMO_HIP_DEQUANT_SCRATCH_BYTES)."""
    fn = lib.tmo_hip_dequant_from_paged_cache_noalloc
    fn.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 5 + [ctypes.c_void_p] * 7 + \
        [ctypes.c_int64] * 7 + [ctypes.c_int] * 5 + [ctypes.c_void_p]
    m = re.search(r"#define\s+TMO_HIP_DEQUANT_SCRATCH_BYTES\s+(\d+)", HEADER.read_text())
    pages = (int(m.group(1)) - 16) // 16 // 8 * 8      # 262136 with 4 MiB
    too_small = header_enum("TMO_ERR_SCRATCH_TOO_SMALL")

    def call(B, MB):
        return fn(FAKE, None, 1024, 128, 0, 0, 10, FAKE, None, FAKE, None, FAKE, None, FAKE, B,
                  MB, 64, 16, 8, 16, 128, 1, 8, 2, 3, 0, None)
    assert pages == 262136
    assert call(1, pages + 1) == too_small
    assert call(pages // 8 + 1, 8) == too_small
    assert call(1 << 40, 1 << 30) == too_small          # no overflow in batch * max_blocks
    assert call(-1, 4) == EINVAL
    assert call(0, 4) == 0
    assert "scratch" in lib.tmo_hip_status_string(too_small).decode()


def test_dequant_workspace_bytes(lib):
    # 16-byte header + 16 bytes per page the call can cover, batch * max_blocks rounded up to
    # a multiple of 8; max_context_len does not limit the pages (the reference math reads
    # context_lengths only)
    assert lib.tmo_hip_dequant_workspace_bytes(64, 2048, 32768, 16) == 16 + 16 * 64 * 2048
    assert lib.tmo_hip_dequant_workspace_bytes(3, 4, 1000, 16) == 16 + 16 * 16
    assert lib.tmo_hip_dequant_workspace_bytes(3, 100, 17, 16) == 16 + 16 * 304
    assert lib.tmo_hip_dequant_workspace_bytes(0, 4, 64, 16) == 0
    assert lib.tmo_hip_dequant_workspace_bytes(2, 4, 0, 16) == 16 + 16 * 8
    assert lib.tmo_hip_dequant_workspace_bytes(2, 4, -1, 16) == 16 + 16 * 8
    assert lib.tmo_hip_dequant_workspace_bytes(2, 0, 64, 16) == 0


def test_scaled_quantize_validation(lib):
    def call(dtype=2, x=FAKE, smooth=None, smooth_len=0, tc=None, groups=0, gi=None, gs=None,
             C=64, stride=64, rows=4):
        return lib.tmo_hip_scaled_quantize_per_token(x, 4, 1, C, stride, FAKE, FAKE, smooth,
                                                     smooth_len, tc, groups, gi, 0, gs, rows,
                                                     dtype, None)
    assert call(dtype=3) == EDTYPE
    assert call(x=None) == EINVAL
    assert call(smooth=FAKE, smooth_len=7) == EINVAL   # neither 1 nor C
    assert call(tc=FAKE, groups=0) == EINVAL
    assert call(gs=FAKE) == EINVAL                     # start position without gather_index
    assert call(stride=10) == EINVAL                   # rows overlap
    assert call(rows=0) == 0


def test_offline_quant_validation(lib):
    def call(dtype=2, cdt=3, k=FAKE, v=None, vc=None, vch=None, slot=FAKE, T=4, H=8, D=128, BS=16):
        return lib.tmo_hip_offline_quant_to_paged_cache(k, v, 1024, 128, 1024, 128, FAKE, vc, None,
                                                        vch, 0.5, 0.5, slot, T, H, D, 4, BS,
                                                        dtype, cdt, None)
    assert call(dtype=3) == EDTYPE          # int8 input
    assert call(cdt=2) == EDTYPE            # bf16 cache
    assert call(cdt=header_enum("TMO_DTYPE_F8E4M3"), T=0) == 0
    assert call(k=None) == EINVAL
    assert call(slot=None) == EINVAL
    assert call(v=FAKE) == EINVAL           # v without v_cache
    assert call(vch=FAKE) == EINVAL         # v scale without v
    assert call(H=0) == EINVAL
    assert call(BS=-1) == EINVAL
    assert call(T=0) == 0


def test_fused_rope_validation(lib):
    def call(dtype=2, mode=0, qkv=FAKE, ks=None, T=8, S=8, D=128, rope=128, off=0, B=1, stride=128,
             rows=64, beta=None, qg=None, norm=0):
        return lib.tmo_hip_fused_rope_paged(qkv, T, S, 4, 2, D, FAKE, FAKE, rows, stride, rope, off,
                                            FAKE, B, FAKE, beta, qg, 1e-5, norm, FAKE, FAKE, ks,
                                            ks, mode, FAKE, 4, 16, dtype, None)
    assert call(dtype=0) == EDTYPE           # fp32 qkv
    assert call(mode=3) == EMODE
    assert call(norm=2) == EMODE             # neither rmsnorm nor layernorm
    assert call(norm=1, qg=FAKE, T=0) == 0   # q_gamma is ignored by layernorm (as the torch op)
    assert call(norm=1, qg=FAKE, mode=1) == EINVAL  # ... the missing scales still fail
    assert call(norm=0, beta=FAKE) == EINVAL  # k_beta belongs to layernorm
    assert call(mode=1) == EINVAL            # quantised without scales
    assert call(qkv=None) == EINVAL
    assert call(D=1024, rope=128) == EINVAL  # head_size > 512
    assert call(rope=127) == EINVAL          # odd rope_dim
    assert call(off=8) == EINVAL             # window past head_size
    assert call(stride=64) == EINVAL         # table rows shorter than rope_dim
    assert call(T=9) == EINVAL               # more tokens than batch * seq_len
    assert call(T=0) == 0


def test_fused_rope_linear_validation(lib):
    def call(mode=0, ks=None, T=8, MB=4, L=64, bs_id=None, off=None, norm=0, qg=None):
        return lib.tmo_hip_fused_rope_linear(FAKE, T, 8, 4, 2, 128, FAKE, FAKE, 64, 128, 128, 0,
                                             FAKE, 1, FAKE, None, qg, 1e-5, norm, FAKE, FAKE, ks,
                                             ks, mode, bs_id, off, MB, L, 2, None)
    assert call(mode=3) == EMODE
    assert call(mode=2) == EINVAL            # quantised without scales
    assert call(norm=1, qg=FAKE, T=0) == 0   # q_gamma is ignored by layernorm
    assert call(L=0) == EINVAL               # cache_len must be positive
    assert call(MB=-1) == EINVAL
    assert call(MB=1 << 20, L=1 << 12) == EINVAL  # slots past int32
    assert call(T=0) == 0
    assert call(T=0, MB=0) == 0              # no cache batches: nothing to store


def lin_write(lib, fn, *, key=FAKE, value=None, kc=FAKE, vc=None, rows=64, MB=4, H=8, L=32,
              D=128, lens=FAKE, B=2, max_len=16, packed=1, seqlen=0, dtype=2, extra=()):
    head = (key, value, 1024, 128, 1024, 128, rows, kc, vc)
    tail = (lens, B, max_len, packed, seqlen, None, None, None)
    if fn == "reshape":
        return lib.tmo_hip_reshape_linear_cache(*head, MB, H, L, D, *tail, dtype, None)
    if fn == "quant":
        ks, vs, groups, bit, cdt = extra or (FAKE, None, 1, 8, 3)
        return lib.tmo_hip_quant_to_linear_cache(*head, ks, vs, MB, H, L, D, groups, *tail, bit,
                                                 dtype, cdt, None)
    ks, vs, mode, cdt = extra or (FAKE, None, 0, 3)
    return lib.tmo_hip_offline_quant_to_linear_cache(*head, ks, vs, 1.0, 1.0, mode, MB, H, L, D,
                                                     *tail, dtype, cdt, None)


def test_linear_write_validation(lib):
    for fn in ("reshape", "quant", "offline"):
        assert lin_write(lib, fn, key=None) == EINVAL, fn
        assert lin_write(lib, fn, lens=None) == EINVAL, fn
        assert lin_write(lib, fn, value=FAKE) == EINVAL, fn     # value without value_cache
        assert lin_write(lib, fn, H=0) == EINVAL, fn
        assert lin_write(lib, fn, B=-1) == EINVAL, fn
        assert lin_write(lib, fn, max_len=-1) == EINVAL, fn
        assert lin_write(lib, fn, dtype=9) == EDTYPE, fn
        assert lin_write(lib, fn, B=0) == 0, fn                  # nothing to do
        assert lin_write(lib, fn, max_len=0) == 0, fn
        assert lin_write(lib, fn, rows=0) == 0, fn
    assert lin_write(lib, "quant", dtype=3) == EDTYPE          # int8 input
    assert lin_write(lib, "quant", extra=(FAKE, None, 1, 5, 3)) == EMODE   # quant_bit 5
    # 4-bit: int8 caches only; head_size a multiple of 8; an even cache_len for V pairs; scale
    # groups over whole aligned lane groups (head_size 80: 10 lanes of 8 channels); valid
    # arguments with nothing to do return 0 before anything is launched
    assert lin_write(lib, "quant", extra=(FAKE, None, 1, 4, 4)) == EDTYPE
    assert lin_write(lib, "quant", D=20, extra=(FAKE, None, 1, 4, 3)) == EMODE
    assert lin_write(lib, "quant", value=FAKE, vc=FAKE, L=33, extra=(FAKE, FAKE, 1, 4, 3)) == EMODE
    assert lin_write(lib, "quant", D=80, extra=(FAKE, None, 2, 4, 3)) == EMODE
    assert lin_write(lib, "quant", D=1024, extra=(FAKE, None, 1, 4, 3)) == EMODE
    assert lin_write(lib, "quant", B=0, extra=(FAKE, None, 1, 4, 3)) == 0
    assert lin_write(lib, "quant", extra=(FAKE, None, 1, 8, 2)) == EDTYPE  # bf16 cache
    assert lin_write(lib, "quant", extra=(FAKE, None, 3, 8, 3)) == EINVAL  # 128 % 3 != 0
    assert lin_write(lib, "quant", extra=(None, None, 1, 8, 3)) == EINVAL  # no scale
    assert lin_write(lib, "offline", extra=(FAKE, None, 4, 3)) == EMODE
    assert lin_write(lib, "offline", extra=(None, None, 0, 3)) == EINVAL   # per channel, no scale
    assert lin_write(lib, "offline", extra=(None, None, 2, 4), B=0) == 0  # per tensor: no tensor


def test_linear_read_validation(lib):
    def deq(mode=1, bit=8, dtype=2, key=FAKE, value=None, vc=None, vs=None, B=2, H=8, rows=10,
            D=128, L=32):
        return lib.tmo_hip_dequant_from_linear_cache(
            key, value, 1024, 128, 1024, 128, rows, FAKE, vc, FAKE, vs, 4, H, L, D, FAKE, B,
            16, None, None, None, mode, bit, dtype, None)
    assert deq(mode=2) == EMODE
    assert deq(bit=5) == EMODE
    assert deq(bit=4, D=20) == EMODE                              # head_size % 8 != 0
    assert deq(bit=4, value=FAKE, vc=FAKE, vs=FAKE, L=33) == EMODE  # odd cache_len with V
    assert deq(bit=4, B=0) == 0
    assert deq(dtype=3) == EDTYPE
    assert deq(key=None) == EINVAL
    assert deq(value=FAKE, vc=FAKE) == EINVAL                    # value without value scale
    assert deq(H=0) == EINVAL
    assert deq(B=0) == 0 and deq(rows=0) == 0

    def rfc(dtype=2, key=FAKE, value=None, vc=None, bt=None, mb=0, B=2, NB=4):
        return lib.tmo_hip_reshape_from_cache(key, value, 1024, 128, 1024, 128, 10, FAKE, vc, NB,
                                              8, 16, 128, FAKE, B, 16, None, bt, mb, None, dtype,
                                              None)
    assert rfc(dtype=8) == EDTYPE
    assert rfc(key=None) == EINVAL
    assert rfc(value=FAKE) == EINVAL
    assert rfc(bt=FAKE, mb=0) == EINVAL                          # a table needs columns
    assert rfc(B=0) == 0 and rfc(NB=0) == 0


def test_attention_validation(lib):
    def call(q=FAKE, kc=FAKE, vc=FAKE, ks=FAKE, vs=FAKE, smode=1, bt=FAKE, lens=FAKE, out=FAKE,
             B=2, Hq=8, Hkv=2, D=128, NB=16, BS=16, qdt=2, cdt=3, splits=1, ws=None, wsb=0,
             mctx=64):
        return lib.tmo_hip_single_query_cached_kv_attn(
            q, 1024, 128, kc, vc, ks, vs, smode, bt, 4, lens, None, out, 1024, 128, None, 0, 0,
            B, Hq, Hkv, D, NB, BS, mctx, -1, 0.1, qdt, cdt, splits, ws, wsb, None)
    assert call(qdt=3) == EDTYPE                   # int8 q
    assert call(cdt=1) == EDTYPE                   # fp16 cache with bf16 q
    assert call(smode=0) == EMODE                  # int8 cache without a scale mode
    assert call(q=None) == EINVAL
    assert call(ks=None) == EINVAL
    assert call(Hq=7) == EINVAL                    # not a multiple of the KV heads
    assert call(D=600) == EINVAL
    assert call(BS=0) == EINVAL
    assert call(splits=0) == EINVAL
    assert call(splits=4) == EINVAL                # splits without a workspace
    need = lib.tmo_hip_attn_workspace_bytes(2, 2, 8, 128, 64, 4)
    assert need == 2 * 2 * 4 * 4 * 130 * 4
    assert lib.tmo_hip_attn_workspace_bytes(2, 2, 8, 128, 64, 1) == 0
    assert call(splits=4, ws=FAKE, wsb=need - 4) == EINVAL
    assert call(B=0) == 0
    assert call(B=0, mctx=-1) == 0                 # negative max_context_len: unknown, like 0
    # an empty cache may come with null cache and per-token scale pointers (nothing reads
    # them); a non-empty one may not
    assert call(kc=None, vc=None, ks=None, vs=None, NB=0, B=0) == 0
    assert call(kc=None, NB=16) == EINVAL
    assert call(vc=None, NB=16) == EINVAL
    assert call(ks=None, NB=0, smode=2) == EINVAL  # per-channel scales are never empty
    assert call(bt=None) == EINVAL


def test_multi_token_attention_validation(lib):
    def call(q=FAKE, cu=None, S=4, T=0, B=2, Hq=8, Hkv=2, D=128, Dv=128, kdim=128, vdim=128,
             vc=FAKE, smode=1, ssb=32, BS=16, splits=1, ws=None, wsb=0, qdt=2, cdt=3,
             qss=128 * 8, oss=128 * 8, sink=None, sdt=0, mask=None, mdt=0, mlen=8, msb=32,
             mss=8, vch=0, NB=16, qs=None, qsm=0, qsdt=0, qsst=8, qsg=0, bth=0, odt=None):
        return lib.tmo_hip_cached_kv_attn(
            q, 4 * 1024, qss, 128, qs, qsm, qsdt, 32, qsst, 1, qsg, cu, S, T, FAKE, vc, kdim, vdim,
            FAKE, FAKE, smode, sdt, ssb, 16, 32, 16, FAKE, 4, bth, FAKE, None, sink, mask, mdt,
            mlen, msb, mss, FAKE, 4 * 1024, oss, 128, None, 0, 0, 0, B, Hq, Hkv, D, Dv, NB, BS, 64,
            -1, 0.1, qdt, cdt, vch, qdt if odt is None else odt, splits, ws, wsb, None)
    assert call(qdt=3) == EDTYPE
    assert call(smode=4) == EMODE and call(smode=0) == EMODE
    assert call(sdt=1) == EDTYPE                   # scales: fp32 or bf16
    assert call(cdt=4, sdt=2, B=0) == 0            # float8_e4m3fn caches, bf16 scales
    assert call(cdt=4, smode=0) == EMODE           # ... which need a scale mode
    assert call(q=None) == EINVAL
    assert call(kdim=64) == EINVAL                 # a K row shorter than the key head size
    assert call(vdim=64) == EINVAL                 # a V row shorter than the value head size
    assert call(vc=None, kdim=128, Dv=192, B=0) == EINVAL   # one cache: row >= both head sizes
    assert call(vc=None, kdim=192, Dv=192, B=0) == 0
    assert call(Dv=600, vdim=600) == EINVAL and call(D=5000, kdim=5000) == EINVAL
    assert call(ssb=-1) == EINVAL                  # negative per-token scale stride
    assert call(smode=3, BS=16) == EINVAL          # per-group scales: 32-row pages
    assert call(smode=3, BS=32, D=48, kdim=48) == EINVAL    # ... and 32-channel groups
    assert call(smode=3, BS=32, B=0) == 0
    assert call(S=-1) == EINVAL
    assert call(qss=-1) == EINVAL and call(oss=-1) == EINVAL
    assert call(cu=FAKE, T=-1) == EINVAL           # cu_seq_q with a negative row count
    assert call(S=2 ** 31 // 8) == EINVAL          # seq_q * heads beyond 32 bits
    assert call(splits=3) == EINVAL                # splits without a workspace
    # workspace [batch, kv_heads, splits, seq_q * group, head_size_v + 2] floats
    need = lib.tmo_hip_cached_kv_attn_workspace_bytes(2, 2, 8, 128, 4, 3)
    assert need == 2 * 2 * 3 * 4 * 4 * 130 * 4
    assert lib.tmo_hip_cached_kv_attn_workspace_bytes(2, 2, 8, 128, 1, 3) == \
        lib.tmo_hip_attn_workspace_bytes(2, 2, 8, 128, 999, 3)
    assert lib.tmo_hip_cached_kv_attn_workspace_bytes(2, 2, 8, 128, 0, 3) == 0
    assert call(splits=3, ws=FAKE, wsb=need - 4) == EINVAL
    assert call(B=0) == 0 and call(S=0) == 0       # nothing to compute
    assert call(S=0, cu=FAKE, T=5, sink=FAKE) == 0
    # mask: float32 / float16 / bfloat16 logit terms, a positive length, non-negative strides
    assert call(mask=FAKE, mdt=2, B=0) == 0 and call(mask=FAKE, mdt=1, B=0) == 0
    assert call(mask=FAKE, mdt=3) == EDTYPE and call(mask=FAKE, mdt=4) == EDTYPE
    assert call(mask=FAKE, mlen=0) == EINVAL and call(mask=FAKE, msb=-1) == EINVAL
    assert call(mask=FAKE, mss=-1) == EINVAL
    assert call(mask=None, mdt=9, mlen=-5, B=0) == 0            # ignored without a mask
    # int4 pairs (cdt 5): K rows of head_size / 2 bytes; V rows pairs (block_size / 2 rows of
    # head_size_v bytes, block_size even) or channel pairs (head_size_v / 2 bytes)
    assert call(cdt=5, kdim=64, vdim=128, B=0) == 0
    assert call(cdt=5, kdim=64, vdim=64, vch=1, B=0) == 0
    assert call(cdt=5, kdim=63, vdim=128) == EINVAL             # K row under head_size / 2
    assert call(cdt=5, kdim=64, vdim=64) == EINVAL              # row pairs need head_size_v bytes
    assert call(cdt=5, kdim=64, vdim=63, vch=1) == EINVAL
    assert call(cdt=5, kdim=64, vdim=128, BS=15) == EINVAL      # odd block_size: no row pairs
    assert call(cdt=5, kdim=64, vdim=128, vc=None) == EINVAL    # int4 needs its own V cache
    assert call(cdt=5, kdim=64, vdim=128, vc=None, NB=0, B=0) == 0
    assert call(cdt=5, kdim=64, vdim=128, smode=0) == EMODE     # int4 codes need scales
    # int8 / float8_e4m3fn q: codes with q scales (modes 1-3, fp32 or bf16), an output dtype of
    # its own, quantised caches only
    assert call(qdt=3, qs=FAKE, qsm=2, odt=1, B=0) == 0
    assert call(qdt=4, qs=FAKE, qsm=1, qsdt=2, odt=1, B=0) == 0
    assert call(qdt=3, qs=FAKE, qsm=3, qsg=4, odt=2, B=0) == 0
    assert call(qdt=3, qs=FAKE, qsm=3, qsg=3, odt=2) == EINVAL   # groups must divide head_size
    assert call(qdt=3, qs=None, qsm=2, odt=1) == EINVAL
    assert call(qdt=3, qs=FAKE, qsm=0, odt=1) == EMODE and call(qdt=3, qs=FAKE, qsm=4, odt=1) == EMODE
    assert call(qdt=3, qs=FAKE, qsm=2, qsdt=1, odt=1) == EDTYPE   # q scales: fp32 or bf16
    assert call(qdt=3, qs=FAKE, qsm=2, odt=3) == EDTYPE             # output: a float type
    assert call(qdt=3, qs=FAKE, qsm=2, qsst=-1, odt=1) == EINVAL
    assert call(qdt=3, qs=FAKE, qsm=2, odt=1, cdt=2, smode=0) == EDTYPE  # plain caches need q's dtype
    assert call(qdt=2, odt=1) == EDTYPE                           # float q: out has q's dtype
    # sparse-KV tables: one row per KV head or per query head
    assert call(bth=2, B=0) == 0 and call(bth=8, B=0) == 0
    assert call(bth=3) == EINVAL

