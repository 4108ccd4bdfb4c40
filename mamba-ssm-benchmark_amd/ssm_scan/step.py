"""Single-token recurrent step on the HIP engine (decode).

Counterpart of the inline decode of models/mamba.py:113-118 and the state write-back of
:122-123, with the D skip and gate of :124 fused: ``h`` is updated in place.
"""

import ctypes

import torch

from . import _abi
from .hip_scan import METHODS, _require_gpu


def ssm_step(h, x, delta, A, Bm, Cm, D=None, z=None, delta_bias=None, delta_softplus=False,
             method="zoh"):
    """h (B, D, N) state (float32, or float64 for float64 inputs), updated in place;
    x, delta, z (B, D); Bm, Cm (B, N); A (D, N).  Returns out (B, D) in x's dtype:
    (sum_n C h' + D x) * silu(z) with h' = a h + b."""
    if method not in METHODS:
        raise ValueError(f"unknown discretization {method!r}")
    _require_gpu(h, x, delta, A, Bm, Cm, D, z, delta_bias)
    ct = torch.promote_types(x.dtype, torch.float32)
    if h.dtype != ct:
        raise ValueError(f"state h must be {ct}, got {h.dtype}")
    Bsz, Dm = x.shape
    N = A.shape[1]
    if tuple(h.shape) != (Bsz, Dm, N):
        raise ValueError(f"h must be {(Bsz, Dm, N)}, got {tuple(h.shape)}")
    # the kernel indexes every operand by (batch, dim, dstate): their shapes are checked here
    want = dict(delta=(Bsz, Dm), A=(Dm, N), Bm=(Bsz, N), Cm=(Bsz, N), D=(Dm,), z=(Bsz, Dm), delta_bias=(Dm,))
    for name, t in dict(delta=delta, A=A, Bm=Bm, Cm=Cm, D=D, z=z, delta_bias=delta_bias).items():
        if t is not None and tuple(t.shape) != want[name]:
            raise ValueError(f"{name} must be {want[name]}, got {tuple(t.shape)}")
    io = x.dtype if all(t is None or t.dtype == x.dtype for t in (delta, Bm, Cm, z)) else ct
    if io not in _abi.DTYPE_CODE:
        io = ct
    xs, ds, Bs, Cs, zs = (None if t is None else t.to(io) for t in (x, delta, Bm, Cm, z))
    As, Dv, bv = (None if t is None else t.to(ct) for t in (A, D, delta_bias))
    out = torch.empty((Bsz, Dm), dtype=io, device=x.device)
    args = _abi.StepArgs()
    args.batch, args.dim, args.dstate = Bsz, Dm, N
    args.method, args.dtype = METHODS[method], _abi.DTYPE_CODE[io]
    args.x, args.delta, args.A = _abi.view(xs), _abi.view(ds), _abi.view(As)
    args.Bm, args.Cm, args.Dskip = _abi.view(Bs), _abi.view(Cs), _abi.view(Dv)
    args.z, args.delta_bias = _abi.view(zs), _abi.view(bv)
    args.delta_softplus = 1 if delta_softplus else 0
    args.h, args.out = _abi.view(h), _abi.view(out)
    lib = _abi.lib()
    with _abi.on_device(x.device):
        rc = lib.ssm_step(ctypes.byref(args), _abi.stream_handle(x.device))
    _abi.check(rc, "ssm_step")
    return out if out.dtype == x.dtype else out.to(x.dtype)
