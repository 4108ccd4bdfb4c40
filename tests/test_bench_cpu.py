"""CPU checks of bench.py's contract: the algorithmic byte counts behind `roofline`, the
one-GPU rule for --gpus, and the per-kernel time statistics."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_config1_algorithmic_bytes():
    """B16 L512 D512 N16 fp32 with gate and skip: fwd 68,716,544 B and bwd 119,607,296 B (every
    tensor read or written once: x, delta, B, C, z in, y out, A, D, last; the backward re-reads
    the inputs, reads dy and writes dx, ddelta, dz, dB, dC, dA, dD)."""
    fwd, bwd = bench.alg_bytes(16, 512, 512, 16)
    BL, D, N = 16 * 512, 512, 16
    assert fwd == 4 * BL * (2 * D + 2 * N) + 4 * BL * D + 4 * BL * D + 4 * D * N + 4 * D + 4 * 16 * D * N
    assert (fwd, bwd) == (68_716_544, 119_607_296)
    fwd0, _ = bench.alg_bytes(1, 512, 512, 16, gate=False)
    assert fwd0 == 3_278_848                                 # config 0 (D skip, no gate)
    fwd2, _ = bench.alg_bytes(1, 131072, 512, 16, gate=False)
    assert fwd2 == 822_151_168                               # config 2 at L = 131072
    fwd2b, _ = bench.alg_bytes(1, 131072, 512, 16, s=2, gate=False)
    # bf16 streams; A, D skip and last stay float32
    assert fwd2b == 2 * 131072 * (2 * 512 + 2 * 16) + 2 * 131072 * 512 + 4 * 512 * 16 + 4 * 512 + 4 * 512 * 16


def test_time_stats_quartiles():
    st = bench.time_stats([5.0, 1.0, 3.0, 2.0, 4.0])
    assert st["median"] == 3.0 and st["n"] == 5 and st["q1"] <= 2.0 <= st["q3"] and st["q3"] >= 4.0
    assert bench.time_stats([7.0]) == {"median": 7.0, "q1": None, "q3": None, "n": 1}


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


@pytest.mark.skipif(os.environ.get("HIP_VISIBLE_DEVICES") is None and os.path.exists("/dev/kfd"),
                    reason="a GPU may be present")
def test_no_gpu_is_an_error():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 1
    assert "needs a ROCm GPU" in r.stderr
