"""bench.py's host-side contract, checked on the CPU: a request for more than one GPU exits
with a message, the fused rope workloads' algorithmic bytes follow their per-token formula
(summed by hand below, term by term), and the CPU baseline of the 80-head fused rope workload
runs the oracle on a bounded sample and reports the fields the bench line carries."""
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    res = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


@pytest.mark.parametrize("hq,expected", [
    # 32768 tokens, D = 128, 8 KV heads, 128-wide rope window, 8 sequences:
    # qkv read T*(hq+16)*256, Q written back T*hq*256, codes + scales 2*T*8*132,
    # slots 4*T, sin + cos rows 2*T*256, two gammas 2*256, positions 4*8
    (32, 32768 * 48 * 256 + 32768 * 32 * 256 + 2 * 32768 * 8 * 132 + 4 * 32768
     + 2 * 32768 * 256 + 512 + 32),
    (64, 671_088_640 + 536_870_912 + 69_206_016 + 131_072 + 16_777_216 + 512 + 32),
])
def test_fused_rope_bytes(hq, expected):
    assert bench.fused_rope_bytes(bench.FR_B * bench.FR_S, hq=hq) == expected


def test_fused_rope_bytes_match_the_committed_figures():
    # the per-config algorithmic bytes of the committed bench runs
    assert bench.fused_rope_bytes(32768) == 757_203_488
    assert bench.fused_rope_bytes(32768, hq=bench.fr_q_heads("fused_rope_70b")) == 1_294_074_400


def test_every_workload_has_a_kernel_label():
    assert set(bench.WORKLOADS) == set(bench.KERNELS)


def test_cpu_baseline_fused_rope_70b():
    import torch
    from tests import workloads as W
    cpu = bench.cpu_baseline(torch, W, "fused_rope_70b", 0.2)
    assert cpu["unit"] == "GB/s" and cpu["kind"] == "port"
    assert cpu["value"] > 0 and cpu["cores"] >= 1
    assert "fused rope" in cpu["sample"]
