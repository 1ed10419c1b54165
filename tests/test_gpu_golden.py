"""The HIP ops reproduce the golden fixtures of tests/golden bit for bit (through the public
wrappers -> torch_mlu_ops ops -> C ABI), on cuda:0."""
import pytest
import torch

from tests import golden_cases as G

pytestmark = pytest.mark.gpu


def _assert_all(triples):
    torch.cuda.synchronize()
    for name, got, want in triples:
        assert torch.equal(G.bits(got), G.bits(want)), name


@pytest.mark.parametrize("name", G.QUANT_PAGED)
def test_quant_to_paged_cache_fixtures(tmo, dev, name):
    _assert_all(G.run_quant_paged(name, tmo.quant_to_paged_cache, dev))


def test_smooth_quant_fixture(tmo, dev):
    _assert_all(G.run_smooth_quant(
        lambda x, out, osc, sm, tc, gi: tmo.moe_quantize(x, sm, None, tc, gi, None, out, osc), dev))


def test_dequant_fixture(tmo, dev):
    _assert_all(G.run_dequant_paged(
        lambda key, val, kc, vc, ks, vs, ctx, bt: tmo.dequant_from_paged_cache(
            key, val, kc, vc, ks, vs, ctx, int(ctx.max()), None, bt, 1, 8), dev))


def test_linear_int4_fixture(tmo, dev):
    _assert_all(G.run_linear_int4(
        lambda key, val, kc, vc, ks, vs, ctx, mctx, cso, bsi, coff: tmo.quant_to_linear_cache(
            key, val, kc, vc, ks, vs, ctx, mctx, True, cso, bsi, coff, 4), dev))


@pytest.mark.parametrize("name", G.FUSED_ROPE)
def test_fused_rope_fixtures(tmo, dev, name):
    def fn(qkv, kc, vc, sin, cos, pid, kg, qg, kb, ks, vs, slot, norm):
        if norm == "layernorm":
            tmo.fused_rope(qkv, kc, vc, sin, cos, pid, kg, kb, k_scale_hp=ks, v_scale_hp=vs,
                           slot_mapping_hp=slot, norm_type="layernorm", eps=1e-5)
        else:
            tmo.fused_rmsnorm_rope_store_paged_cache(qkv, kc, vc, sin, cos, pid, kg, qg, slot,
                                                     ks, vs, 1e-5)
    _assert_all(G.run_fused_rope(name, fn, dev))


@pytest.mark.parametrize("name", G.OFFLINE)
def test_offline_quant_fixtures(tmo, dev, name):
    _assert_all(G.run_offline(name, tmo.offline_quant_to_paged_cache, dev))


def test_linear_int8_fixture(tmo, dev):
    _assert_all(G.run_linear_int4(
        lambda key, val, kc, vc, ks, vs, ctx, mctx, cso, bsi, coff: tmo.quant_to_linear_cache(
            key, val, kc, vc, ks, vs, ctx, mctx, True, cso, bsi, coff, 8), dev, name="linear_int8"))
