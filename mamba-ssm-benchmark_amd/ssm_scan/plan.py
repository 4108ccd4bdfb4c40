"""The reference's integer planning functions, computed by the engine library (exact integers).

  default_chunk   models/scan.py:138-139
  blocks          models/scan.py:185-190 (channel tiles of SelectiveScanFn)
  block_d         kernels/triton_scan.py:245-250
  bwd_tile        kernels/triton_scan.py:305
  resolve_scan    models/scan.py:286-287 with _triton_ok :305-314 (the selected algorithm)
"""

import ctypes

from . import _abi

SCAN_ELEMENT_BUDGET = 1 << 24      # models/scan.py:182
HBUF_BUDGET = 1 << 27              # kernels/triton_scan.py:242
BLOCK_D = 16                       # kernels/triton_scan.py:231


def default_chunk(L):
    return int(_abi.lib().ssm_default_chunk(int(L)))


def blocks(shape_bld, N, d_block=None):
    Bsz, L, D = (int(v) for v in shape_bld)
    lib = _abi.lib()
    n = lib.ssm_scan_blocks(Bsz, L, D, int(N), int(d_block or 0), None, 0)
    if n < 0:
        raise ValueError(f"invalid scan shape {shape_bld} with N={N}")
    buf = (ctypes.c_int64 * (2 * n))()
    lib.ssm_scan_blocks(Bsz, L, D, int(N), int(d_block or 0), buf, n)
    return [(buf[2 * i], buf[2 * i + 1]) for i in range(n)]


def block_d(Bsz, D):
    return int(_abi.lib().ssm_block_d(int(Bsz), int(D)))


def bwd_tile(Bsz, L, N, bd):
    return int(_abi.lib().ssm_bwd_tile(int(Bsz), int(L), int(N), int(bd)))


def resolve_scan(scan, on_gpu, method, N, engine_available=True):
    """Name of the algorithm `scan` selects; KeyError for an unknown name."""
    if scan not in _abi.SCAN_IDS:
        raise KeyError(scan)
    m = {"zoh": 0, "euler": 1, "bilinear": 2}.get(method, -1)
    sid = _abi.lib().ssm_resolve_scan(_abi.SCAN_IDS[scan], int(bool(on_gpu)), m, int(N),
                                      int(bool(engine_available)))
    if sid < 0:
        raise KeyError(scan)
    return _abi.SCAN_NAMES[sid]
