"""The golden fixtures of tests/golden against the torch restatements of the reference math
(the functions of tests/test_oracle_pins.py, which follow the reference's Math blocks and
share no code with the C oracle): torch on the CPU reproduces every stored output of every
fixture bit for bit from the stored inputs.  The fixtures were written by the oracle; this
pins them to the docstring math independently of it (CPU only)."""
from types import SimpleNamespace

import pytest
import torch

from tests import golden_cases as G
from tests import test_oracle_pins as P


def _assert_all(triples):
    for name, got, want in triples:
        assert torch.equal(G.bits(got), G.bits(want)), name


@pytest.mark.parametrize("name", G.QUANT_PAGED)
def test_quant_to_paged_cache_fixtures_match_torch(name):
    # reference _ops.py:1524-1537 with the slot scatter of _ops.py:1262-1268
    _assert_all(G.run_quant_paged(name, P.torch_quant_to_paged))


def test_smooth_quant_fixture_matches_torch():
    # reference _ops.py:3147-3172 (gather, per-expert smooth rows, per-row int8)
    def fn(x, out, osc, smooth, token_count, gather_index):
        codes, scale = P.torch_moe_quantize(x, smooth, token_count, gather_index)
        out.copy_(codes)
        osc.copy_(scale)
    _assert_all(G.run_smooth_quant(fn))


def test_dequant_fixture_matches_torch():
    # reference _ops.py:3749-3774, per-token scales, rows packed by the exclusive prefix of
    # the context lengths
    def fn(key, value, kc, vc, ks, vs, ctx, bt):
        offsets = torch.cumsum(ctx, 0) - ctx
        for out, c, s in ((key, kc, ks), (value, vc, vs)):
            for off, rows in P.torch_dequant(c, s, ctx, bt, 1, out.dtype, offsets).items():
                out[off:off + rows.shape[0]] = rows
    _assert_all(G.run_dequant_paged(fn))


@pytest.mark.parametrize("name", G.OFFLINE)
def test_offline_quant_fixtures_match_torch(name):
    # reference _ops.py:1652-1670 (int8, and the float8_e4m3fn cast of _ops.py:1829-1840)
    _assert_all(G.run_offline(name, P.torch_offline_quant_to_paged))


@pytest.mark.parametrize("name", G.FUSED_ROPE)
def test_fused_rope_fixtures_match_torch(name):
    # reference _ops.py:3493-3520 in the fp32 summation order of D10 / D13
    def fn(qkv, kc, vc, sin, cos, pid, k_gamma, q_gamma, k_beta, ks, vs, slot, norm):
        ln = norm == "layernorm"
        out = P.torch_fused_rope(qkv, kc, vc, sin, cos, pid, k_gamma, ks, vs, slot, 1e-5,
                                 None if ln else q_gamma, 0, exact=True, norm_type=norm,
                                 k_beta=k_beta if ln else None)
        qkv.copy_(out)
    _assert_all(G.run_fused_rope(name, fn))


def _linear_writer(bits):
    """quant_to_linear_cache with quant_bit 8 (_ops.py:1728-1742) or 4 (D15) by torch, on a
    case rebuilt from the fixture's inputs (packed token rows; context_lengths holds the batch + 1
    prefix offsets of the packed form)."""
    def fn(key, value, kc, vc, ks, vs, ctx, max_len, cso, bsi, coff):
        lens = (ctx[1:] - ctx[:-1]).to(torch.int32)
        case = SimpleNamespace(key=key, value=value, lens=lens, max_context_len=max_len,
                               context_seq_offset=cso, cache_bs_id=bsi, cache_seq_offset=coff,
                               packed=True, cache_batch=kc.shape[0], cache_len=kc.shape[2])
        if bits == 4:
            P.torch_linear_write4(case, kc, vc, ks, vs)
        else:
            P.torch_linear_write(case, 1, kc, vc, ks, vs)
    return fn


@pytest.mark.parametrize("name,bits", [("linear_int8", 8), ("linear_int4", 4)])
def test_linear_cache_fixtures_match_torch(name, bits):
    _assert_all(G.run_linear_int4(_linear_writer(bits), name=name))
