"""ctypes binding of oracle/ssm_oracle.c (float64 sequential scan + adjoint).

Test infrastructure only.  build() compiles it with the Makefile beside this file.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libssm_oracle.so")
_lib = None
METHODS = {"zoh": 0, "euler": 1, "bilinear": 2}


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        _lib.ssm_oracle_fwd.argtypes = [I64, I64, I64, I64, ctypes.c_int] + [P] * 11 + [ctypes.c_int]
        _lib.ssm_oracle_bwd.argtypes = [I64, I64, I64, I64, ctypes.c_int] + [P] * 22 + [ctypes.c_int]
        _lib.ssm_oracle_fwd.restype = ctypes.c_int
        _lib.ssm_oracle_bwd.restype = ctypes.c_int
    return _lib


def _c(a):
    return None if a is None else np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def fwd(x, delta, A, Bm, Cm, h0=None, method="zoh", D=None, z=None, nthreads=0):
    """Returns (out, y, last) in float64; same contract as scan_ref.selective_scan_fwd."""
    lib = _load()
    x, delta, A, Bm, Cm, h0, D, z = (_c(v) for v in (x, delta, A, Bm, Cm, h0, D, z))
    Bsz, L, Dm = x.shape
    N = A.shape[1]
    out = np.empty((Bsz, L, Dm))
    y = np.empty((Bsz, L, Dm))
    last = np.empty((Bsz, Dm, N))
    rc = lib.ssm_oracle_fwd(Bsz, L, Dm, N, METHODS[method], _p(x), _p(delta), _p(A), _p(Bm),
                            _p(Cm), _p(h0), _p(D), _p(z), _p(out), _p(y), _p(last), nthreads)
    if rc:
        raise RuntimeError(f"ssm_oracle_fwd failed: {rc}")
    return out, y, last


def bwd(x, delta, A, Bm, Cm, dout, h0=None, method="zoh", D=None, z=None, dlast=None,
        nthreads=0, mag=False):
    """Returns the gradient dict of scan_ref.selective_scan_bwd, in float64.  With mag=True it
    also holds "ddelta_mag", "dA_mag", "dB_mag" and "dC_mag": per element the sum of the |terms|
    it adds (over the states for ddelta, over batch and time for dA, over the channels for dB and
    dC), as
    scan_ref.selective_scan_bwd(mag=True)."""
    lib = _load()
    x, delta, A, Bm, Cm, dout, h0, D, z, dlast = (
        _c(v) for v in (x, delta, A, Bm, Cm, dout, h0, D, z, dlast))
    Bsz, L, Dm = x.shape
    N = A.shape[1]
    g = {k: np.empty_like(v) for k, v in
         (("dx", x), ("ddelta", delta), ("dA", A), ("dB", Bm), ("dC", Cm))}
    g_dD = np.empty_like(D) if D is not None else None
    g_dz = np.empty_like(z) if z is not None else None
    g_dh0 = np.empty_like(h0) if h0 is not None else None
    g_mag = np.empty_like(delta) if mag else None
    g_amag = np.empty_like(A) if mag else None
    g_bmag = np.empty_like(Bm) if mag else None
    g_cmag = np.empty_like(Cm) if mag else None
    rc = lib.ssm_oracle_bwd(Bsz, L, Dm, N, METHODS[method], _p(x), _p(delta), _p(A), _p(Bm),
                            _p(Cm), _p(h0), _p(D), _p(z), _p(dout), _p(dlast), _p(g["dx"]),
                            _p(g["ddelta"]), _p(g["dA"]), _p(g["dB"]), _p(g["dC"]), _p(g_dD),
                            _p(g_dz), _p(g_dh0), _p(g_mag), _p(g_amag), _p(g_bmag), _p(g_cmag), nthreads)
    if rc:
        raise RuntimeError(f"ssm_oracle_bwd failed: {rc}")
    if g_dD is not None:
        g["dD"] = g_dD
    if g_dz is not None:
        g["dz"] = g_dz
    if g_dh0 is not None:
        g["dh0"] = g_dh0
    if g_mag is not None:
        g["ddelta_mag"] = g_mag
        g["dA_mag"] = g_amag
        g["dB_mag"] = g_bmag
        g["dC_mag"] = g_cmag
    return g
