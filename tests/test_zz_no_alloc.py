"""tmo_hip_dequant_from_paged_cache_noalloc (the allocation-free entry point, page list in the
library's static device scratch) against tmo_hip_dequant_from_paged_cache with a caller
workspace, through the C ABI: two calls in a row on one GPU, the second with a smaller input,
each bit-exact against the allocating entry point's output and the oracle; the bytes past the
smaller call's rows keep their sentinel; two calls enqueued on two streams with no host wait
between them (the entry point orders them on the shared scratch) give the same results as one
after the other, and so do calls from two host threads on their own streams; a call beyond the
scratch is refused."""
import ctypes

import pytest
import torch

from tests import workloads as W

pytestmark = pytest.mark.gpu

P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SCRATCH_TOO_SMALL = -5


def _lib():
    from domesticated_torch_mlu_ops_amd import _loader
    L = _loader.c_abi()
    args = [P, P] + [I64] * 5 + [P] * 7 + [I64] * 7 + [INT] * 5
    L.tmo_hip_dequant_from_paged_cache.argtypes = args + [P, I64, P]
    L.tmo_hip_dequant_from_paged_cache_noalloc.argtypes = args + [P]
    L.tmo_hip_dequant_workspace_bytes.argtypes = [I64] * 4
    L.tmo_hip_dequant_workspace_bytes.restype = I64
    return L


def _layout(seed, B, MB, NB, H=8, BS=16, D=128):
    """B sequences of up to MB pages over NB cache blocks, caches and per-token scales."""
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, MB * BS + 1, (B,), generator=g).to(torch.int32)
    ctx[0] = MB * BS
    bt = torch.randperm(NB, generator=g)[: B * MB].reshape(B, MB).to(torch.int32)
    kc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (NB, H, BS, D), generator=g, dtype=torch.int8)
    ks = torch.rand(NB, H, BS, generator=g) * 0.05
    vs = torch.rand(NB, H, BS, generator=g) * 0.05
    return W.DequantLayout(f"noalloc{seed}", ctx, bt, NB, BS), (kc, vc, ks, vs)


def _args(out_k, out_v, caches, layout):
    """C-ABI arguments (and the device index tensors they point into, to keep alive)."""
    kc, vc, ks, vs = caches
    NB, H, BS, D = kc.shape
    ctx = layout.context_lengths.to(out_k.device)
    bt = layout.block_tables.to(out_k.device)
    B, MB = bt.shape
    args = [out_k.data_ptr(), out_v.data_ptr(), out_k.stride(0), out_k.stride(1), out_v.stride(0),
            out_v.stride(1), out_k.shape[0], kc.data_ptr(), vc.data_ptr(), ks.data_ptr(),
            vs.data_ptr(), ctx.data_ptr(), None, bt.data_ptr(), B, MB,
            layout.max_context_len, NB, H, BS, D, 1, 8, 2, 3, 0]
    return args, (ctx, bt)


def _call(L, fn, out_k, out_v, caches, layout, workspace=None):
    args, keep = _args(out_k, out_v, caches, layout)
    torch.cuda.synchronize()
    if fn == "noalloc":
        st = L.tmo_hip_dequant_from_paged_cache_noalloc(*args, None)
    else:
        st = L.tmo_hip_dequant_from_paged_cache(*args, workspace.data_ptr(), workspace.numel(),
                                                None)
    torch.cuda.synchronize()
    return st


def test_noalloc_matches_workspace_entry_point(ref, dev):
    L = _lib()
    rows_cap = 0
    for seed, B, MB, NB in ((1, 48, 40, 2048), (2, 7, 9, 96)):  # the second call is smaller
        layout, caches_h = _layout(seed, B, MB, NB)
        caches = tuple(t.to(dev) for t in caches_h)
        total = layout.total_tokens
        rows_cap = max(rows_cap, total)
        print(f"[noalloc] B={B} pages/seq={MB} tokens={total}", flush=True)
        want_k = torch.full((rows_cap, 8, 128), -3.0).to(torch.bfloat16)
        want_v = want_k.clone()
        ref.dequant_from_paged_cache(want_k[:total], want_v[:total], *caches_h,
                                     layout.context_lengths, None, layout.block_tables, 1)
        ws = torch.empty(L.tmo_hip_dequant_workspace_bytes(B, MB, layout.max_context_len, 16),
                         dtype=torch.uint8, device=dev)
        outs = {}
        for fn in ("workspace", "noalloc"):
            ok = torch.full((rows_cap, 8, 128), -3.0, device=dev).to(torch.bfloat16)
            ov = ok.clone()
            assert _call(L, fn, ok[:total], ov[:total], caches, layout, ws) == 0
            outs[fn] = (ok.cpu(), ov.cpu())
        for i, name in enumerate(("key", "value")):
            a = outs["noalloc"][i].view(torch.int16)
            assert torch.equal(a, outs["workspace"][i].view(torch.int16)), name
            assert torch.equal(a, (want_k, want_v)[i].view(torch.int16)), name


def test_noalloc_calls_on_two_streams_are_ordered(dev):
    """A large call on one stream and a small one on another, enqueued back to back: the
    second call's page-list pass rewrites the shared scratch, so it must wait for the first
    call's kernels; each output is compared with the allocating entry point's, computed one
    call at a time."""
    L = _lib()
    cases = []
    for seed, B, MB, NB in ((4, 64, 64, 4096), (5, 5, 7, 64)):
        layout, caches_h = _layout(seed, B, MB, NB)
        caches = tuple(t.to(dev) for t in caches_h)
        total = layout.total_tokens
        print(f"[noalloc streams] B={B} pages/seq={MB} tokens={total}", flush=True)
        ws = torch.empty(L.tmo_hip_dequant_workspace_bytes(B, MB, layout.max_context_len, 16),
                         dtype=torch.uint8, device=dev)
        wk = torch.full((total, 8, 128), -3.0, device=dev).to(torch.bfloat16)
        wv = wk.clone()
        assert _call(L, "workspace", wk, wv, caches, layout, ws) == 0
        ok = torch.full((total, 8, 128), -5.0, device=dev).to(torch.bfloat16)
        ov = ok.clone()
        cases.append((layout, caches, (wk.cpu(), wv.cpu()), (ok, ov)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    keep = []
    torch.cuda.synchronize()
    for (layout, caches, _, (ok, ov)), st in zip(cases, streams):
        args, k = _args(ok, ov, caches, layout)
        keep.append(k)
        assert L.tmo_hip_dequant_from_paged_cache_noalloc(*args, ctypes.c_void_p(st.cuda_stream)) == 0
    torch.cuda.synchronize()
    for layout, _, want, got in cases:
        for i, name in enumerate(("key", "value")):
            assert torch.equal(got[i].cpu().view(torch.int16), want[i].view(torch.int16)), \
                (layout.name, name)


def test_noalloc_calls_from_two_host_threads(dev):
    """Two host threads, each enqueueing calls on its own stream with no host wait between
    them (ctypes releases the GIL during the call, so the enqueues interleave): every output
    equals the allocating entry point's."""
    import threading
    L = _lib()
    cases = []
    for seed, B, MB, NB in ((6, 32, 48, 2048), (7, 9, 11, 128)):
        layout, caches_h = _layout(seed, B, MB, NB)
        caches = tuple(t.to(dev) for t in caches_h)
        total = layout.total_tokens
        print(f"[noalloc threads] B={B} pages/seq={MB} tokens={total}", flush=True)
        ws = torch.empty(L.tmo_hip_dequant_workspace_bytes(B, MB, layout.max_context_len, 16),
                         dtype=torch.uint8, device=dev)
        wk = torch.full((total, 8, 128), -3.0, device=dev).to(torch.bfloat16)
        wv = wk.clone()
        assert _call(L, "workspace", wk, wv, caches, layout, ws) == 0
        outs = [(torch.full((total, 8, 128), -5.0, device=dev).to(torch.bfloat16),
                 torch.full((total, 8, 128), -5.0, device=dev).to(torch.bfloat16))
                for _ in range(4)]
        cases.append((layout, caches, (wk.cpu(), wv.cpu()), outs))
    torch.cuda.synchronize()
    status = []

    def worker(case):
        layout, caches, _, outs = case
        st = torch.cuda.Stream()
        keep = []
        for ok, ov in outs:
            args, k = _args(ok, ov, caches, layout)
            keep.append(k)
            status.append(L.tmo_hip_dequant_from_paged_cache_noalloc(
                *args, ctypes.c_void_p(st.cuda_stream)))
        st.synchronize()

    threads = [threading.Thread(target=worker, args=(c,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert status == [0] * 8
    for layout, _, want, outs in cases:
        for ok, ov in outs:
            for got, w, name in ((ok, want[0], "key"), (ov, want[1], "value")):
                assert torch.equal(got.cpu().view(torch.int16), w.view(torch.int16)), \
                    (layout.name, name)


def test_noalloc_refuses_calls_beyond_the_scratch(dev):
    L = _lib()
    layout, caches_h = _layout(3, 2, 4, 16)
    caches = tuple(t.to(dev) for t in caches_h)
    ok = torch.full((layout.total_tokens, 8, 128), -3.0, device=dev).to(torch.bfloat16)
    ov = ok.clone()
    # 65536 sequences x 5 pages = 327680 pages > 262136: refused before anything is enqueued
    big = W.DequantLayout("big", torch.zeros(65536, dtype=torch.int32),
                          torch.zeros(65536, 5, dtype=torch.int32), 16, 16)
    assert _call(L, "noalloc", ok, ov, caches, big) == SCRATCH_TOO_SMALL
    assert torch.all(ok.cpu() == -3.0) and torch.all(ov.cpu() == -3.0)
