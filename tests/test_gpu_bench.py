"""bench.py's workloads run in this process with a few steps: the JSON line of each carries
the fields of the driver's contract (metric, value, unit, step counts, dtype, config) and, for
config 1, a `roofline` whose achieved bandwidth is the algorithmic bytes over the measured
kernel time; config 4's decode is timed and its graph replay matches its eager step."""

import json
import math
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

pytestmark = pytest.mark.gpu

CONTRACT = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data", "config")


def args(**kw):
    ns = bench.parser().parse_args([])   # bench.py's own defaults, then the small test sizes
    base = dict(steps=3, warmup=1, decode_steps=8, seqlen=4096, no_cpu_baseline=True)
    base.update(kw)
    for k, v in base.items():
        setattr(ns, k, v)
    return ns


def check_line(rec):
    json.dumps(rec)                                    # serializable as one JSON line
    for k in CONTRACT:
        assert k in rec, k
    assert rec["n_gpus"] == 1 and rec["vs_baseline"] is None
    assert math.isfinite(rec["value"]) and rec["value"] > 0
    assert "workload" in rec["config"]


def test_config1_line(dev):
    rec = bench.bench_c1(args(), dev)
    check_line(rec)
    assert rec["unit"] == "Mtok/s" and rec["dtype"] == "f32"
    roof = rec["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == 8000.0 and roof["unit"] == "GB/s"
    expect = roof["alg_bytes_per_launch"] / (rec["kernels_ms"]["ssm_bwd"] * 1e-3) / 1e9
    assert roof["achieved"] == pytest.approx(expect) and roof["frac"] == pytest.approx(expect / 8000.0)
    assert rec["graph_matches_eager"] is True


def test_config2_short_line(dev):
    rec = bench.bench_fwd(args(workload="c2"), dev, 1, 4096, torch.float32, "config 2: fwd B1 L4096 D512 N16")
    check_line(rec)
    assert rec["roofline"]["frac"] > 0


def test_config4_line(dev):
    rec = bench.bench_decode(args(workload="c4"), dev)
    check_line(rec)
    assert rec["unit"] == "us/layer" and rec["higher_is_better"] is False
