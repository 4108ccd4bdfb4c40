"""Writes tests/golden/vectors.npz: small seeded inputs (float32 values) and the float64 oracle's
outputs for them, per function on the path:

  scan/<method>/<variant>  the fused selective scan forward and every gradient
                           (oracle/scan_ref.py:selective_scan_fwd / _bwd; models/scan.py:264-274,
                           kernels/triton_scan.py:56-67,187-223), with and without gate, D skip,
                           h0 and dlast;
  lscan                    the linear scan h_t = a_t h_{t-1} + b_t and its VJP (models/scan.py:70-76);
  disc/<method>            discretize and its VJP (models/scan.py:39-55);
  conv                     the depthwise causal conv + SiLU with a carried state
                           (models/mamba.py:101-107);
  step/<method>            the recurrent decode step (models/mamba.py:113-118,122-124).

Inputs are stored as float32 (the values the GPU path reads), outputs as float64.  The CPU
tests recompute every output from the stored inputs with the oracle; the GPU tests run the HIP
path on the same inputs.  Run from the repository root:  python tests/golden/make_vectors.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import scan_ref as R  # noqa: E402

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vectors.npz")


def _f32(g, *shape, scale=1.0, shift=0.0):
    return (g.standard_normal(shape) * scale + shift).astype(np.float32)


def _uniform(g, lo, hi, *shape):
    return g.uniform(lo, hi, shape).astype(np.float32)


def make_inputs():
    """{case name: {input name: float32 array}}, seeded."""
    g = np.random.default_rng(20240)
    cases = {}
    for method in R.DISCRETIZATIONS:
        for variant, (B, L, D, N, full) in {"plain": (2, 37, 6, 4, False), "full": (2, 37, 6, 4, True),
                                            "n16": (1, 70, 8, 16, True)}.items():
            c = dict(x=_f32(g, B, L, D), delta=_uniform(g, 1e-3, 0.3, B, L, D),
                     A=-_uniform(g, 0.05, 4.0, D, N), Bm=_f32(g, B, L, N), Cm=_f32(g, B, L, N),
                     dout=_f32(g, B, L, D))
            if full:
                c.update(D=_f32(g, D), z=_f32(g, B, L, D), h0=_f32(g, B, D, N), dlast=_f32(g, B, D, N))
            cases[f"scan/{method}/{variant}"] = c
    cases["lscan"] = dict(a=_uniform(g, 0.5, 1.0, 2, 45, 7), b=_f32(g, 2, 45, 7), h0=_f32(g, 2, 7),
                          dh=_f32(g, 2, 45, 7))
    for method in R.DISCRETIZATIONS:
        cases[f"disc/{method}"] = dict(delta=_uniform(g, 1e-3, 0.3, 2, 9, 5), A=-_uniform(g, 0.05, 4.0, 5, 4),
                                       Bm=_f32(g, 2, 9, 4), x=_f32(g, 2, 9, 5), ga=_f32(g, 2, 9, 5, 4),
                                       gb=_f32(g, 2, 9, 5, 4))
    cases["conv"] = dict(x=_f32(g, 2, 13, 6), w=_f32(g, 6, 4, scale=0.5), bias=_f32(g, 6), state=_f32(g, 2, 6, 3))
    for method in R.DISCRETIZATIONS:
        cases[f"step/{method}"] = dict(h=_f32(g, 3, 6, 4), x=_f32(g, 3, 6), delta=_uniform(g, 1e-3, 0.3, 3, 6),
                                       A=-_uniform(g, 0.05, 4.0, 6, 4), Bm=_f32(g, 3, 4), Cm=_f32(g, 3, 4),
                                       D=_f32(g, 6), z=_f32(g, 3, 6))
    return cases


def compute(name, c):
    """The float64 oracle's outputs for case `name` from its inputs `c`."""
    c = {k: v.astype(np.float64) for k, v in c.items()}
    kind = name.split("/")[0]
    if kind == "scan":
        method = name.split("/")[1]
        opt = {k: c.get(k) for k in ("h0", "D", "z")}
        out, _, last = R.selective_scan_fwd(c["x"], c["delta"], c["A"], c["Bm"], c["Cm"], opt["h0"], method,
                                            opt["D"], opt["z"])
        gr = R.selective_scan_bwd(c["x"], c["delta"], c["A"], c["Bm"], c["Cm"], c["dout"], opt["h0"], method,
                                  opt["D"], opt["z"], c.get("dlast"))
        return dict(out=out, last=last, **gr)
    if kind == "lscan":
        h = R.scan_sequential(c["a"], c["b"], c["h0"])
        da, db, dh0 = R.scan_vjp(c["a"], c["h0"], h, c["dh"])
        return dict(h=h, da=da, db=db, dh0=dh0)
    if kind == "disc":
        method = name.split("/")[1]
        a, b = R.discretize(c["delta"], c["A"], c["Bm"], c["x"], method)
        dd, dA, dB, dx = R.discretize_vjp(c["delta"], c["A"], c["Bm"], c["x"], c["ga"], c["gb"], method)
        return dict(a=a, b=b, ddelta=dd, dA=dA, dBm=dB, dx=dx)
    if kind == "conv":
        y, st = R.conv1d_causal(c["x"].transpose(0, 2, 1), c["w"], c["bias"], c["state"])
        return dict(y=y.transpose(0, 2, 1), state=st)
    if kind == "step":
        method = name.split("/")[1]
        y, h = R.ssm_step(c["h"], c["x"], c["delta"], c["A"], c["Bm"], c["Cm"], method, c["D"], c["z"])
        return dict(y=y, h=h)
    raise KeyError(name)


def load():
    """{case name: (inputs, outputs)} from vectors.npz."""
    data = np.load(PATH)
    cases = {}
    for key in data.files:
        io, name, field = key.split(":")
        cases.setdefault(name, ({}, {}))[0 if io == "in" else 1][field] = data[key]
    return cases


if __name__ == "__main__":
    arrays = {}
    for name, c in make_inputs().items():
        for k, v in c.items():
            arrays[f"in:{name}:{k}"] = v
        for k, v in compute(name, c).items():
            arrays[f"out:{name}:{k}"] = v
    np.savez_compressed(PATH, **arrays)
    print("wrote", PATH, len(arrays), "arrays")
