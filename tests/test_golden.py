"""The golden fixtures of tests/golden: their hashes match MANIFEST.sha256, and the CPU oracle
reproduces every stored output bit for bit from the stored inputs (CPU only)."""
import pytest
import torch

import oracle
from tests import golden_cases as G


def _assert_all(triples):
    for name, got, want in triples:
        assert torch.equal(G.bits(got), G.bits(want)), name


def test_manifest_hashes():
    m = G.manifest()
    assert len(m) == 12
    for fname, digest in m.items():
        assert G.sha256(fname) == digest, fname


@pytest.mark.parametrize("name", G.QUANT_PAGED)
def test_oracle_quant_to_paged_cache_fixtures(name):
    _assert_all(G.run_quant_paged(name, oracle.quant_to_paged_cache))


def test_oracle_smooth_quant_fixture():
    _assert_all(G.run_smooth_quant(
        lambda x, out, osc, sm, tc, gi: oracle.scaled_quantize_per_token(x, out, osc, sm, tc, gi)))


def test_oracle_dequant_fixture():
    _assert_all(G.run_dequant_paged(
        lambda key, val, kc, vc, ks, vs, ctx, bt: oracle.dequant_from_paged_cache(
            key, val, kc, vc, ks, vs, ctx, None, bt, 1)))


def test_oracle_linear_int4_fixture():
    _assert_all(G.run_linear_int4(
        lambda key, val, kc, vc, ks, vs, ctx, mctx, cso, bsi, coff: oracle.linear_cache(
            1, key, val, kc, vc, ctx, mctx, packed=True, context_seq_offset=cso,
            cache_bs_id=bsi, cache_seq_offset=coff, key_scale=ks, value_scale=vs, bits=4)))


@pytest.mark.parametrize("name", G.FUSED_ROPE)
def test_oracle_fused_rope_fixtures(name):
    def fn(qkv, kc, vc, sin, cos, pid, kg, qg, kb, ks, vs, slot, norm):
        ln = norm == "layernorm"
        oracle.fused_rope_paged(qkv, kc, vc, sin, cos, pid, kg, ks, vs, slot, 1e-5,
                                None if ln else qg, 0, norm_type=norm, k_beta=kb if ln else None)
    _assert_all(G.run_fused_rope(name, fn))


@pytest.mark.parametrize("name", G.OFFLINE)
def test_oracle_offline_quant_fixtures(name):
    _assert_all(G.run_offline(name, oracle.offline_quant_to_paged_cache))


def test_oracle_linear_int8_fixture():
    _assert_all(G.run_linear_int4(
        lambda key, val, kc, vc, ks, vs, ctx, mctx, cso, bsi, coff: oracle.linear_cache(
            1, key, val, kc, vc, ctx, mctx, packed=True, context_seq_offset=cso,
            cache_bs_id=bsi, cache_seq_offset=coff, key_scale=ks, value_scale=vs, bits=8),
        name="linear_int8"))
