"""MI355X (gfx950) selective-scan engine.

Drop-in counterpart of the reference's scan path:
  ssm_scan.scan      <-> models/scan.py        (selective_scan, discretize, SCANS, ...)
  ssm_scan.hip_scan  <-> kernels/triton_scan.py (fused forward/backward)
  ssm_scan.step      <-> the recurrent decode step of models/mamba.py:113-118
  ssm_scan.conv      <-> the causal depthwise conv + SiLU of models/mamba.py:101-107
  ssm_scan.norm      <-> RMSNorm of models/common.py:8-16
  ssm_scan.block     <-> the Mamba mixer, block and Mamba-only LM of models/mamba.py, models/lm.py
  ssm_scan.decode    <-> a fused per-layer decode step for benchmarks/bench_decode.py's loop
All compute runs in libssmscan.so (hand-written HIP kernels behind a C ABI, see
include/ssm_scan.h); the package only prepares views, allocates outputs with torch and
launches on torch's current stream.  There is no CPU fallback.
"""

from . import _abi, plan, scan
from .conv import causal_conv1d
from .hip_scan import (METHODS, FusedSelectiveScanFn, selective_scan_fn, selective_scan_hip,
                       selective_scan_triton)
from .norm import rms_norm
from .profiling import KernelTimer
from .scan import (DISCRETIZATIONS, SCANS, SelectiveScanFn, default_chunk, discretize,
                   scan_blelloch, scan_chunked, scan_hillis_steele, scan_sequential,
                   selective_scan, selective_scan_reference)
from .step import ssm_step

__all__ = ["METHODS", "FusedSelectiveScanFn", "selective_scan_fn", "selective_scan_hip",
           "selective_scan_triton", "ssm_step", "KernelTimer", "plan", "scan", "DISCRETIZATIONS",
           "SCANS", "SelectiveScanFn", "default_chunk", "discretize", "scan_blelloch", "scan_chunked",
           "scan_hillis_steele", "scan_sequential", "selective_scan", "selective_scan_reference",
           "causal_conv1d", "rms_norm"]


def library_path():
    """Path of the engine library this package loads (libssmscan.so)."""
    return _abi.LIB_PATH
