"""Fused selective scan on the HIP engine: the counterpart of kernels/triton_scan.py.

``selective_scan_hip`` keeps the contract of ``selective_scan_triton``
(kernels/triton_scan.py:322-329): x, delta (B, L, D); A (D, N); Bm, Cm (B, L, N);
h0 (B, D, N) -> (y, last).  ``selective_scan_fn`` is the fused extension with the D skip,
SiLU(z) gate and optional delta bias/softplus of models/mamba.py:76,124.

Every tensor may have arbitrary strides (no .contiguous() copies, unlike
kernels/triton_scan.py:278).  Arithmetic is float32 (float64 for float64 inputs), as the
reference computes in promote(dtype, float32) (models/scan.py:289); bf16/fp16 inputs are read
directly when x, delta, B, C (and z) share one dtype, otherwise they are upcast first, which
gives the same values the reference's casts give.  Reductions are fixed-order, so the
backward is bitwise deterministic in every mode (the reference only is in
torch's deterministic mode, kernels/triton_scan.py:298).
"""

import ctypes

import torch

from . import _abi
from .linear import rocblas, weight_grad
from .profiling import timed_launch

ZOH, EULER, BILINEAR = 0, 1, 2
METHODS = {"zoh": ZOH, "euler": EULER, "bilinear": BILINEAR}     # kernels/triton_scan.py:23-24
_IO_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float64)


def _require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("ssm_scan runs on ROCm GPU tensors only; got a tensor on "
                               f"{t.device} (there is no CPU path)")


def _dtypes(x, streams):
    """(io dtype of the big streams, compute/state dtype)."""
    ct = torch.promote_types(x.dtype, torch.float32)
    if ct == torch.float64:
        return torch.float64, torch.float64
    if x.dtype in _IO_DTYPES and all(t is None or t.dtype == x.dtype for t in streams):
        return x.dtype, torch.float32
    return torch.float32, torch.float32


def is_dense(t):
    """True when t's elements tile its storage exactly (a permutation of a contiguous layout),
    so torch.empty_like keeps its strides."""
    expected = 1
    for size, stride in sorted(zip(t.shape, t.stride()), key=lambda p: p[1]):
        if size == 1:
            continue
        if stride != expected:
            return False
        expected *= size
    return True


def empty_like_layout(t, dtype):
    """Output buffer with t's layout when t is dense (e.g. channel-major views), else contiguous."""
    if is_dense(t):
        return torch.empty_like(t, dtype=dtype, memory_format=torch.preserve_format)
    return torch.empty(t.shape, dtype=dtype, device=t.device)


def _cast_keep(t, dt):
    return t if t is None or t.dtype == dt else t.to(dt)


def _fill_common(args, x, delta, A, Bm, Cm, D, z, bias, softplus, h0, method, io):
    Bsz, L, Dm = x.shape
    args.batch, args.seqlen, args.dim, args.dstate = Bsz, L, Dm, A.shape[1]
    args.method = method
    args.dtype = _abi.DTYPE_CODE[io]
    args.x, args.delta, args.A = _abi.view(x), _abi.view(delta), _abi.view(A)
    args.Bm, args.Cm = _abi.view(Bm), _abi.view(Cm)
    args.Dskip, args.z, args.delta_bias = _abi.view(D), _abi.view(z), _abi.view(bias)
    args.delta_softplus = 1 if softplus else 0
    args.h0 = _abi.view(h0)


def _check_shapes(x, delta, A, Bm, Cm, D, z, bias, h0, delta_proj=None):
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got {tuple(x.shape)}")
    Bsz, L, Dm = x.shape
    if A.dim() != 2 or A.shape[0] != Dm:
        raise ValueError(f"A must be (D, N) = ({Dm}, N), got {tuple(A.shape)}")
    N = A.shape[1]
    dshape = (Bsz, L, Dm)
    if delta_proj is not None:
        if delta_proj.dim() != 2 or delta_proj.shape[0] != Dm:
            raise ValueError(f"delta_proj must be (D, R) = ({Dm}, R), got {tuple(delta_proj.shape)}")
        dshape = (Bsz, L, delta_proj.shape[1])
    for name, t, shp in (("delta", delta, dshape), ("Bm", Bm, (Bsz, L, N)), ("Cm", Cm, (Bsz, L, N)),
                         ("D", D, (Dm,)), ("z", z, (Bsz, L, Dm)), ("delta_bias", bias, (Dm,)),
                         ("h0", h0, (Bsz, Dm, N))):
        if t is not None and tuple(t.shape) != shp:
            raise ValueError(f"{name} must have shape {shp}, got {tuple(t.shape)}")


def scan_forward(x, delta, A, Bm, Cm, D, z, delta_bias, h0, method, delta_softplus, segments=0,
                 delta_proj=None, A_is_log=False, need_saved=True):
    """One ssm_fwd launch.  Returns (out in the io dtype, last, state) where `state` holds what
    scan_backward needs: the tensors as the kernels read them, the saved chunk states and the
    launch settings."""
    io, ct = _dtypes(x, (delta, Bm, Cm, z))
    xs, ds, Bs, Cs, zs = (_cast_keep(t, io) for t in (x, delta, Bm, Cm, z))
    As, Dv, bv, h0v, Wv = (_cast_keep(t, ct) for t in (A, D, delta_bias, h0, delta_proj))
    Bsz, L, Dm = x.shape
    N = A.shape[1]
    dev = x.device
    out = empty_like_layout(xs, io)
    last = torch.empty((Bsz, Dm, N), dtype=ct, device=dev)
    args = _abi.FwdArgs()
    _fill_common(args, xs, ds, As, Bs, Cs, Dv, zs, bv, delta_softplus, h0v, method, io)
    args.out, args.last = _abi.view(out), _abi.view(last)
    args.segments = int(segments or 0)
    if Wv is not None:
        args.delta_proj, args.delta_rank = _abi.view(Wv), Wv.shape[1]
    args.A_is_log = 1 if A_is_log else 0
    lib = _abi.lib()
    wbytes = lib.ssm_fwd_workspace_bytes(ctypes.byref(args))
    if wbytes < 0:
        _abi.check(lib.ssm_fwd_check(ctypes.byref(args)), "ssm_fwd")
    ws = torch.empty(wbytes, dtype=torch.uint8, device=dev) if wbytes else None
    if ws is not None:
        args.workspace, args.workspace_bytes = ws.data_ptr(), wbytes
    saved = None
    if need_saved:
        nbytes = lib.ssm_fwd_saved_bytes(ctypes.byref(args))
        _abi.check(0 if nbytes >= 0 else 1, "ssm_fwd_saved_bytes")
        saved = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        args.saved = saved.data_ptr()
    with _abi.on_device(dev):
        stream = _abi.stream_handle(dev)
        rc = timed_launch("ssm_fwd", stream, lambda: lib.ssm_fwd(ctypes.byref(args), stream))
    _abi.check(rc, "ssm_fwd")
    state = ((xs, ds, As, Bs, Cs, Dv, zs, bv, h0v, Wv, saved),
             (method, bool(delta_softplus), io, ct, bool(A_is_log), int(segments or 0)))
    return out, last, state


def scan_backward(tensors, settings, dout, dlast, dz=None, dB=None, dC=None):
    """One ssm_bwd launch from scan_forward's state.  dz, dB, dC may be given (views into a
    caller's buffer, e.g. the in_proj / x_proj output gradients); the others are allocated.
    Returns (dx, ddelta, dA, dB, dC, dD, dz, ddelta_bias, dh0); with a delta projection,
    ddelta is the gradient of the projected (B, L, D) delta."""
    xs, ds, As, Bs, Cs, Dv, zs, bv, h0v, Wv, saved = tensors
    method, softplus, io, ct, a_log, segments = settings
    if dout is None:
        dout = torch.zeros(xs.shape, dtype=io, device=xs.device)
    dout = _cast_keep(dout, io)
    dlast = _cast_keep(dlast, ct)
    Bsz, L, Dm = xs.shape
    N = As.shape[1]
    dev = xs.device
    like = empty_like_layout
    dx, dd = like(xs, io), like(ds if Wv is None else xs, io)
    dA = torch.empty((Dm, N), dtype=ct, device=dev)
    dB = like(Bs, io) if dB is None else dB
    dC = like(Cs, io) if dC is None else dC
    dD = torch.empty((Dm,), dtype=ct, device=dev) if Dv is not None else None
    if zs is not None and dz is None:
        dz = like(zs, io)
    db = torch.empty((Dm,), dtype=ct, device=dev) if bv is not None else None
    dh0 = torch.empty((Bsz, Dm, N), dtype=ct, device=dev) if h0v is not None else None
    args = _abi.BwdArgs()
    _fill_common(args, xs, ds, As, Bs, Cs, Dv, zs, bv, softplus, h0v, method, io)
    args.saved = saved.data_ptr()
    args.segments = segments
    args.dout, args.dlast = _abi.view(dout), _abi.view(dlast)
    args.dx, args.ddelta, args.dA = _abi.view(dx), _abi.view(dd), _abi.view(dA)
    args.dBm, args.dCm, args.dD = _abi.view(dB), _abi.view(dC), _abi.view(dD)
    args.dz, args.ddelta_bias, args.dh0 = _abi.view(dz), _abi.view(db), _abi.view(dh0)
    if Wv is not None:
        args.delta_proj, args.delta_rank = _abi.view(Wv), Wv.shape[1]
    args.A_is_log = 1 if a_log else 0
    lib = _abi.lib()
    nbytes = lib.ssm_bwd_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        _abi.check(lib.ssm_bwd_check(ctypes.byref(args)), "ssm_bwd")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    with _abi.on_device(dev):
        stream = _abi.stream_handle(dev)
        rc = timed_launch("ssm_bwd", stream, lambda: lib.ssm_bwd(ctypes.byref(args), stream))
    _abi.check(rc, "ssm_bwd")
    return dx, dd, dA, dB, dC, dD, dz, db, dh0


class FusedSelectiveScanFn(torch.autograd.Function):
    """out, last = fused scan; gradients for x, delta, A, Bm, Cm, D, z, delta_bias, h0."""

    @staticmethod
    def forward(ctx, x, delta, A, Bm, Cm, D, z, delta_bias, h0, method, delta_softplus, segments=0,
                delta_proj=None, A_is_log=False):
        need_bwd = any(ctx.needs_input_grad[:9]) or (delta_proj is not None and ctx.needs_input_grad[12])
        out, last, (tensors, settings) = scan_forward(x, delta, A, Bm, Cm, D, z, delta_bias, h0, method,
                                                      delta_softplus, segments, delta_proj, A_is_log, need_bwd)
        if need_bwd:
            ctx.save_for_backward(*tensors)
        ctx.set_materialize_grads(False)   # an unused `last` passes dlast = None (no zero fill)
        ctx.settings = settings
        ctx.in_dtypes = [None if t is None else t.dtype for t in (x, delta, A, Bm, Cm, D, z, delta_bias, h0)]
        ctx.proj_dtype = None if delta_proj is None else delta_proj.dtype
        if out.dtype != x.dtype:
            out = out.to(x.dtype)
        return out, last

    @staticmethod
    def backward(ctx, dout, dlast):
        tensors = ctx.saved_tensors
        dx, dd, dA, dB, dC, dD, dz, db, dh0 = scan_backward(tensors, ctx.settings, dout, dlast)
        ds, Wv = tensors[1], tensors[9]
        dW = None
        if Wv is not None:
            # the projection's gradients: the two small GEMMs of F.linear's backward, in torch
            ct = ctx.settings[3]
            ddc = dd.to(ct)
            with rocblas():
                dW = weight_grad(ddc.reshape(-1, ddc.shape[-1]), ds.to(ct).reshape(-1, Wv.shape[1]))
                dd = torch.matmul(ddc, Wv)
        grads = [dx, dd, dA, dB, dC, dD, dz, db, dh0]
        out = []
        for g, dt in zip(grads, ctx.in_dtypes):
            out.append(None if g is None or dt is None else _cast_keep(g, dt))
        return (*out, None, None, None, None if dW is None else _cast_keep(dW, ctx.proj_dtype), None)


LOWRANK_MAX = 16  # rank of a delta projection the kernels apply while staging delta


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      h0=None, method="zoh", return_last_state=False, segments=None, delta_proj=None,
                      A_is_log=False):
    """out = (scan(u, delta', A, B, C) + D u) * silu(z), delta' = softplus(delta + bias).

    Logical layouts as the reference: u, delta, z (B, L, D); A (D, N); B, C (B, L, N);
    h0 (B, D, N).  Pass ``x.transpose(1, 2)`` for channel-major (B, D, L) storage.
    ``segments`` forces the number of time segments the forward and the backward scan in
    parallel (default: chosen by the engine; more than one only when B x D is too small to fill
    the GPU).
    ``delta_proj`` (D, R): ``delta`` is then the low-rank (B, L, R) input and the scan uses
    delta @ delta_proj^T -- the dt_proj GEMM of models/mamba.py:76, done by the kernels while
    they stage delta for R <= 16 and dstate <= 16 with 16/32-bit inputs (no (B, L, D) delta in
    memory), by a torch GEMM otherwise.  Gradients flow to both.
    ``A_is_log``: ``A`` holds A_log (the parameter of models/mamba.py:61,81) and the kernels
    use A = -exp(A_log); its gradient is that of A_log."""
    if method not in METHODS:
        raise ValueError(f"unknown discretization {method!r}")
    _require_gpu(u, delta, A, B, C, D, z, delta_bias, h0, delta_proj)
    _check_shapes(u, delta, A, B, C, D, z, delta_bias, h0, delta_proj)
    if delta_proj is not None and (delta_proj.shape[1] > LOWRANK_MAX or A.shape[1] > 16
                                   or torch.promote_types(u.dtype, torch.float32) == torch.float64):
        delta, delta_proj = torch.nn.functional.linear(delta, delta_proj), None
    out, last = FusedSelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, h0, METHODS[method],
                                           bool(delta_softplus), segments or 0, delta_proj, bool(A_is_log))
    return (out, last) if return_last_state else out


def selective_scan_hip(x, delta, A, Bm, Cm, h0=None, method="zoh", d_block=None):
    """Same contract as kernels/triton_scan.py:322-329 (selective_scan_triton): returns (y, last).

    Raises ValueError for an unknown method and, as the reference does, for a dstate that
    is not a power of two (use selective_scan_fn for other dstate <= 64)."""
    if method not in METHODS:
        raise ValueError(f"fused scan supports {list(METHODS)}, got {method!r}")
    N = A.shape[1]
    if N & (N - 1):
        raise ValueError("d_state must be a power of two for the fused kernel")
    _require_gpu(x, delta, A, Bm, Cm, h0)
    _check_shapes(x, delta, A, Bm, Cm, None, None, None, h0)
    return FusedSelectiveScanFn.apply(x, delta, A, Bm, Cm, None, None, None, h0, METHODS[method], False)


# The reference's module exposes the fused path under this name (kernels/triton_scan.py:322);
# it is kept so callers written against it keep working.  It runs the HIP engine.
selective_scan_triton = selective_scan_hip
