"""The drop-in boundary, checked on the CPU: Python signatures and return conventions of the
reference wrappers, the torch_mlu_ops::* schemas (mutation annotations), the fake kernels,
tracing through torch.export, and the absence of any CPU / oracle fallback."""
import inspect
import subprocess
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent

# Parameter lists of the reference wrappers (name, default), cited per function.
REFERENCE_SIGNATURES = {
    # _ops.py:1251-1258
    "reshape_paged_cache": [("k", None), ("v", None), ("k_cache", None), ("v_cache", None),
                            ("slot_mapping", None), ("direction", False)],
    # _ops.py:1511-1519
    "quant_to_paged_cache": [("k", None), ("v", None), ("k_cache", None), ("v_cache", None),
                             ("k_cache_quant_scale", None), ("v_cache_quant_scale", None),
                             ("slot_mapping", None)],
    # _ops.py:1639-1647
    "offline_quant_to_paged_cache": [("k", None), ("v", None), ("k_cache_scale", None),
                                     ("v_cache_scale", None), ("slot_mapping", None),
                                     ("k_cache", None), ("v_cache", None)],
    # _ops.py:3469-3492
    "fused_rope": [("qkv", None), ("k_cache_hp", None), ("v_cache_hp", None), ("sin_cache", None),
                   ("cos_cache", None), ("position_id", None), ("k_gamma", None), ("k_beta", None),
                   ("k_cache_lp", None), ("v_cache_lp", None), ("cache_bs_id_hp", None),
                   ("cache_seq_offsets_hp", None), ("cache_bs_id_lp", None),
                   ("cache_seq_offsets_lp", None), ("k_scale_hp", None), ("v_scale_hp", None),
                   ("k_scale_lp", None), ("v_scale_lp", None), ("slot_mapping_hp", None),
                   ("slot_mapping_lp", None), ("norm_type", "layernorm"), ("rope_dim_offset", 0),
                   ("eps", 1e-5), ("q_gamma", None)],
    # _ops.py:6356-6367
    "fused_rmsnorm_rope_store_paged_cache": [("qkv", None), ("k_cache", None), ("v_cache", None),
                                             ("sin_cache", None), ("cos_cache", None),
                                             ("position_id", None), ("k_gamma", None),
                                             ("q_gamma", None), ("slot_mapping", None),
                                             ("k_scale", None), ("v_scale", None), ("eps", 1e-5)],
    # _ops.py:3734-3745
    "dequant_from_paged_cache": [("key", None), ("value", None), ("key_cache", None),
                                 ("value_cache", None), ("key_cache_quant_scale", None),
                                 ("value_cache_quant_scale", None), ("context_lengths", None),
                                 ("max_context_len", None), ("context_seq_offset", None),
                                 ("block_tables", None), ("quant_mode", 0), ("quant_bit", 8)],
    # _ops.py:3126-3143
    "moe_quantize": [("x", None), ("smooth", None), ("zero", None), ("token_count", None),
                     ("gather_index", None), ("gather_index_start_position", None),
                     ("output", None), ("output_scale", None), ("dynamic_quant", True),
                     ("act_mode", "none"), ("active_coef", 1.0), ("is_gated", False),
                     ("quant_type", torch.int8), ("quant_bit_size", 8),
                     ("scale_type", torch.float32), ("need_output_scale_trans", False),
                     ("output_reduced", None), ("group_size", 1)],
    # _ops.py:4407-4421
    "scaled_quantize": [("x", None), ("scale", None), ("zero", None), ("scale_ub", None),
                        ("quant_type", torch.int8), ("quant_mode", "dynamic_per_token"),
                        ("act_mode", "none"), ("active_coef", 1.0), ("is_gated", False),
                        ("quant_bit_size", 8), ("scale_type", torch.float32),
                        ("need_output_scale_trans", False), ("output_reduced", None),
                        ("group_size", 1)],
    # _ops.py:1189-1200
    "reshape_linear_cache": [("key", None), ("value", None), ("key_cache", None),
                             ("value_cache", None), ("context_lengths", None),
                             ("max_context_len", None), ("packed", None),
                             ("context_seq_offset", None), ("cache_bs_id", None),
                             ("cache_seqlen_offset", None)],
    # _ops.py:1708-1722
    "quant_to_linear_cache": [("key", None), ("value", None), ("key_cache", None),
                              ("value_cache", None), ("key_cache_quant_scale", None),
                              ("value_cache_quant_scale", None), ("context_lengths", None),
                              ("max_context_len", None), ("packed", None),
                              ("context_seq_offset", None), ("cache_bs_id", None),
                              ("cache_seqlen_offset", None), ("quant_bit", 8)],
    # _ops.py:1808-1822
    "offline_quant_to_linear_cache": [("key", None), ("value", None), ("key_cache", None),
                                      ("value_cache", None), ("key_cache_quant_scale", None),
                                      ("value_cache_quant_scale", None),
                                      ("context_lengths", None), ("max_context_len", None),
                                      ("quant_mode", None), ("packed", None),
                                      ("context_seq_offset", None), ("cache_bs_id", None),
                                      ("cache_seqlen_offset", None)],
    # _ops.py:3642-3654
    "dequant_from_linear_cache": [("key", None), ("value", None), ("key_cache", None),
                                  ("value_cache", None), ("key_cache_quant_scale", None),
                                  ("value_cache_quant_scale", None), ("context_lengths", None),
                                  ("max_context_len", None), ("context_seq_offset", None),
                                  ("cache_bs_id", None), ("cache_seq_offset", None),
                                  ("quant_mode", 0), ("quant_bit", 8)],
    # _ops.py:777-801
    "single_query_cached_kv_attn": [("q", None), ("k_cache", None), ("v_cache", None),
                                    ("out", None), ("block_tables", None),
                                    ("context_lens", None), ("k_cache_quant_scale", None),
                                    ("v_cache_quant_scale", None), ("alibi_slopes", None),
                                    ("max_context_len", None), ("windows_size_left", None),
                                    ("windows_size_right", None), ("softmax_scale", None),
                                    ("return_lse", False), ("kv_cache_quant_bit_size", -1),
                                    ("q_quant_scale", None), ("out_quant_scale", None),
                                    ("out_dtype", torch.half), ("compute_dtype", torch.float),
                                    ("head_size_v", -1), ("mask", None), ("cu_seq_q", None),
                                    ("max_seq_q", -1), ("sink", None)],
    # _ops.py:3898-3906
    "reshape_from_cache": [("key", None), ("value", None), ("key_cache", None),
                           ("value_cache", None), ("context_lengths", None),
                           ("max_context_len", None), ("context_seq_offset", None),
                           ("block_tables", None), ("cache_seq_offset", None)],
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_python_signatures_match_reference(tmo, name):
    sig = inspect.signature(getattr(tmo, name))
    got = [(p.name, None if p.default is inspect.Parameter.empty else p.default)
           for p in sig.parameters.values()]
    assert got == REFERENCE_SIGNATURES[name]


def test_alias_signature(tmo):
    names = list(inspect.signature(tmo.per_token_smooth_quantize).parameters)
    assert names == [n for n, _ in REFERENCE_SIGNATURES["moe_quantize"][:9]]


WRITES = {
    "reshape_paged_cache": {"k", "v", "k_cache", "v_cache"},
    "quant_to_paged_cache": {"k_cache", "v_cache", "k_cache_scale", "v_cache_scale"},
    "offline_quant_to_paged_cache": {"k_cache", "v_cache"},
    "dequant_from_paged_cache": {"key", "value"},
    "fused_rope": {"qkv", "key_cache_hp", "value_cache_hp", "key_cache_lp", "value_cache_lp",
                   "key_scale_hp", "value_scale_hp", "key_scale_lp", "value_scale_lp"},
    "scaled_quantize": {"output", "output_scale", "output_reduced"},
    "reshape_linear_cache": {"key_cache", "value_cache"},
    "quant_to_linear_cache": {"key_cache", "value_cache", "key_cache_scale", "value_cache_scale"},
    "offline_quant_to_linear_cache": {"key_cache", "value_cache"},
    "dequant_from_linear_cache": {"key", "value"},
    "reshape_from_cache": {"key", "value"},
    "single_query_cached_kv_attn": {"output", "output_lse"},
}


@pytest.mark.parametrize("op", sorted(WRITES))
def test_schema_mutation_annotations(tmo, op):
    schema = getattr(torch.ops.torch_mlu_ops, op).default._schema
    written = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == WRITES[op]
    assert len(schema.returns) == 0


def _meta_quant_args(device="meta"):
    k = torch.empty(16, 8, 128, dtype=torch.bfloat16, device=device)
    kc = torch.empty(64, 8, 16, 128, dtype=torch.int8, device=device)
    ks = torch.empty(64, 8, 16, dtype=torch.float32, device=device)
    slot = torch.empty(16, dtype=torch.int32, device=device)
    return k, k.clone(), kc, kc.clone(), ks, ks.clone(), slot


def test_fakes_run_on_meta_tensors(tmo):
    k, v, kc, vc, ks, vs, slot = _meta_quant_args()
    out = tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, slot)
    assert out[0] is kc and out[1] is vc and out[2] is ks and out[3] is vs
    assert tmo.quant_to_paged_cache(k, None, kc, None, ks, None, slot) == (kc, ks)
    assert tmo.reshape_paged_cache(k, v, kc.to(torch.bfloat16), vc.to(torch.bfloat16), slot)[0] \
        .dtype == torch.bfloat16
    key = torch.empty(100, 8, 128, dtype=torch.bfloat16, device="meta")
    ctx = torch.empty(4, dtype=torch.int32, device="meta")
    bt = torch.empty(4, 8, dtype=torch.int32, device="meta")
    assert tmo.dequant_from_paged_cache(key, None, kc, None, ks, None, ctx, 100, None, bt, 1, 8) is None
    x = torch.empty(32, 4096, dtype=torch.bfloat16, device="meta")
    sm = torch.empty(4096, dtype=torch.float32, device="meta")
    o, s = tmo.moe_quantize(x, sm)
    assert o.shape == (32, 4096) and o.dtype == torch.int8 and s.shape == (32,)
    gi = torch.empty(48, dtype=torch.int32, device="meta")
    o, s = tmo.moe_quantize(x, sm, gather_index=gi)
    assert o.shape == (48, 4096) and s.shape == (48,)
    o, s = tmo.scaled_quantize(torch.empty(2, 3, 64, device="meta"), torch.empty(64, device="meta"))
    assert o.shape == (2, 3, 64) and s.shape == (2, 3)
    f8 = kc.to(torch.float8_e4m3fn)
    assert tmo.offline_quant_to_paged_cache(k, v, 0.5, 0.25, slot, kc, vc) == (kc, vc)
    chan = torch.empty(8, 128, dtype=torch.float32, device="meta")
    assert tmo.offline_quant_to_paged_cache(k, None, chan, None, slot, f8, None) is f8
    qkv = torch.empty(2, 8, 48, 128, dtype=torch.bfloat16, device="meta")
    kcb = torch.empty(64, 8, 16, 128, dtype=torch.bfloat16, device="meta")
    tab = torch.empty(64, 128, dtype=torch.bfloat16, device="meta")
    pid = torch.empty(2, dtype=torch.int32, device="meta")
    g = torch.empty(128, dtype=torch.bfloat16, device="meta")
    out = tmo.fused_rmsnorm_rope_store_paged_cache(qkv, kcb, kcb.clone(), tab, tab, pid, g, g, slot)
    assert len(out) == 3 and out[0] is qkv
    out = tmo.fused_rmsnorm_rope_store_paged_cache(qkv, kc, vc, tab, tab, pid, g, None, slot, ks, vs)
    assert len(out) == 5 and out[3] is ks


def test_linear_fakes_run_on_meta_tensors(tmo):
    m = dict(device="meta")
    key = torch.empty(40, 8, 128, dtype=torch.bfloat16, **m)
    kc = torch.empty(4, 8, 64, 128, dtype=torch.int8, **m)
    ks = torch.empty(4, 8, 64, dtype=torch.float32, **m)
    cu = torch.empty(5, dtype=torch.int32, **m)
    lens = torch.empty(4, dtype=torch.int32, **m)
    kb = kc.to(torch.bfloat16)
    assert tmo.reshape_linear_cache(key, key, kb, kb, cu, 16, True, None, None, None) == (kb, kb)
    assert tmo.reshape_linear_cache(key, None, kb, None, cu, 16, True, None, None, None) is kb
    assert tmo.quant_to_linear_cache(key, key, kc, kc, ks, ks, cu, 16, True, None, None,
                                     None) == (kc, kc, ks, ks)
    assert tmo.offline_quant_to_linear_cache(key, None, kc, None, 0.5, None, cu, 16, 2, True,
                                             None, None, None) == (kc, 0.5)
    assert tmo.dequant_from_linear_cache(key, None, kc, None, ks, None, lens, 16, None, None,
                                         None, 1, 8) is None
    assert tmo.reshape_from_cache(key, key, kb, kb, lens, 16) is None


def test_attention_fake_returns_the_reference_shapes(tmo):
    m = dict(device="meta")
    q = torch.empty(4, 1, 32, 128, dtype=torch.bfloat16, **m)
    kc = torch.empty(64, 8, 16, 128, dtype=torch.int8, **m)
    ks = torch.empty(64, 8, 16, **m)
    bt = torch.empty(4, 8, dtype=torch.int32, **m)
    lens = torch.empty(4, dtype=torch.int32, **m)
    out, lse = tmo.single_query_cached_kv_attn(q, kc, kc, None, bt, lens, ks, ks, None, 128, -1,
                                               -1, 0.088, True, 8)
    assert out.shape == q.shape and out.dtype == torch.bfloat16 and lse.shape == (4, 32, 1)
    q3 = torch.empty(4, 32, 128, dtype=torch.float16, **m)
    out = tmo.single_query_cached_kv_attn(q3, kc, kc, None, bt, lens, ks, ks, None, 128, -1, -1,
                                          0.088, False, 8)
    assert out.shape == q3.shape and out.dtype == torch.float16


def test_fake_tensor_mode(tmo):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        k, v, kc, vc, ks, vs, slot = _meta_quant_args(device="cpu")
        out = tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, slot)
        assert out[0] is kc


def test_export_keeps_the_in_place_cache_writes(tmo):
    """torch.export functionalises the mutating op; the cache writes must survive as
    mutated-buffer outputs (this is what the Tensor(a!) annotations guarantee)."""

    class Step(torch.nn.Module):
        def forward(self, k, v, kc, vc, ks, vs, slot):
            tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, slot)
            return k.float().sum()

    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode(allow_non_fake_inputs=True):
        args = _meta_quant_args(device="cpu")
    ep = torch.export.export(Step(), args).run_decompositions({})
    code = ep.graph_module.code
    assert "torch_mlu_ops.quant_to_paged_cache" in code and "auto_functionalized" in code
    mutated = set(ep.graph_signature.user_inputs_to_mutate.values())
    assert mutated == {"kc", "vc", "ks", "vs"}  # the caches, and nothing else


def test_cpu_tensors_fail_loudly(tmo):
    k, v, kc, vc, ks, vs, slot = (t.to("cpu") if t.device.type == "meta" else t
                                  for t in _meta_quant_args(device="cpu"))
    with pytest.raises(NotImplementedError):
        tmo.quant_to_paged_cache(k, v, kc, vc, ks, vs, slot)
    with pytest.raises(NotImplementedError):
        tmo.moe_quantize(torch.zeros(4, 64, dtype=torch.bfloat16), torch.ones(64))
    with pytest.raises(NotImplementedError):
        tmo.offline_quant_to_paged_cache(k, v, 0.5, 0.5, slot, kc, vc)


def test_product_package_never_imports_the_oracle():
    code = ("import sys, domesticated_torch_mlu_ops_amd as m; "
            "bad = [n for n in sys.modules if n == 'oracle' or n.startswith('oracle.') "
            "or n.startswith('tests')]; print(bad); assert not bad, bad")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=str(REPO))
    pkg = REPO / "domesticated_torch_mlu_ops_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.cpp")):
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text, f
        assert "libtmo_oracle" not in text, f
