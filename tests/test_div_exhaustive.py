"""The kernels' int8 encoder divides through a reciprocal plus two FMA correction steps
(tmo_device.h: div_by_recip) and computes the row scale amax / 127 with a constant-reciprocal
correction (scale_of).  This CPU test compiles that same source for the host and checks both
against IEEE fp32 division: the quotient on every bf16 and every fp16 (amax, x) pair and on
random and near-tie fp32 pairs, the scale on every fp32 amax it is used for, the static-scale
quotient (offline quantisation, int8 and fp8 codes) on random scales and near-ties, the
fp8 e4m3 encoder on every fp32 value in [-448, 448], and the fused rope's square-root
correction on every fp32 value in [2^-96, FLT_MAX] (tests/native/div_exhaustive.hip)."""
import os
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
SRC = REPO / "tests" / "native" / "div_exhaustive.hip"
HIPCC = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"


@pytest.fixture(scope="module")
def binary(tmp_path_factory):
    if not HIPCC.exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("div") / "div_exhaustive"
    cmd = [str(HIPCC), "-x", "hip", "--offload-host-only", "-O2", "-ffp-contract=off",
           "-std=c++17", f"-I{REPO / 'include'}",
           f"-I{REPO / 'domesticated_torch_mlu_ops_amd' / 'csrc'}", str(SRC), "-o", str(out),
           "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True)
    return out


@pytest.mark.parametrize("mode,extra", [("bf16", []), ("f16", []), ("f32", ["20000000"]),
                                        ("scale", []), ("static", ["4000000"]), ("fp8", []),
                                        ("sqrt", [])])
def test_reciprocal_quotient_matches_ieee(binary, mode, extra):
    threads = str(max(1, min(8, len(os.sched_getaffinity(0)))))
    res = subprocess.run([str(binary), mode, threads, *extra], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches=0" in res.stdout
