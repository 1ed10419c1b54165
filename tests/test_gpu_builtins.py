"""gfx950 hardware operations the kernels rely on, checked exhaustively on the GPU against
their definitions (tests/native/gfx950_builtins.hip, built in-tree by __graft_entry__.build()):
the v_rcp_f32 + Newton reciprocal is IEEE 1/s for every scale on the static quantiser's
reciprocal path; the v_cvt_pk_fp8_f32 conversion is the round-to-nearest-even e4m3fn encoding
for every fp32 value in [-448, 448]; the fp8 readers (v_cvt_f32_fp8, v_cvt_pk_f32_fp8 and
its f16 packing) decode every e4m3fn code to its value; the dynamic scales' fp64 reciprocal is within 2^-52 of
1/s for every scale, and the encoders' fp64-product quotient is the IEEE fp32 quotient on every
bf16 and fp16 (amax, x) pair; the fused rope's square root is
correctly rounded for every positive finite fp32 value; the MFMA lane layouts the
decode-attention kernel assumes; and the DPP wavefront prefix sum of the grouped smooth
quantiser."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BINARY = Path(__file__).resolve().parent / "native" / "_build" / "gfx950_builtins"


@pytest.mark.parametrize("mode", ["rcp", "fp8", "fp8dec", "recip64", "div64", "sqrt", "mfma",
                                  "scan"])
def test_gfx950_builtin_exhaustive(dev, mode):
    assert BINARY.exists(), f"{BINARY} not built (run __graft_entry__.build())"
    print(f"[gfx950_builtins] {mode}", flush=True)
    res = subprocess.run([str(BINARY), mode], capture_output=True, text=True, timeout=100)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches=0" in res.stdout
