"""The reference's scan module (models/scan.py) on the HIP engine.

Same names, signatures, dispatch strings and error classes as models/scan.py, so callers such
as models/mamba.py:120-121 switch by changing the import:

  discretize        models/scan.py:39-55     materialized (a, b) from the ssm_disc kernels
  zoh_matrix        models/scan.py:58-62     dense test helper (torch.linalg on the device)
  scan_sequential   models/scan.py:70-76     \
  scan_hillis_steele models/scan.py:87-98     | ssm_lscan kernels, one per algorithm, each
  scan_blelloch     models/scan.py:101-135    | differentiable through ssm_lscan_bwd
  scan_chunked      models/scan.py:142-165   /
  SCANS, default_chunk, SCAN_ELEMENT_BUDGET, _blocks   models/scan.py:138-190
  SelectiveScanFn   models/scan.py:193-255   per channel tile: discretize -> scan -> contract,
                                             backward by recompute + reverse scan
  selective_scan_reference  models/scan.py:264-274   the time loop; runs on the fused engine,
                                             which walks the same recurrence step by step
  selective_scan    models/scan.py:277-299   dispatcher ('triton' and 'auto' select the fused
                                             engine, ssm_scan.hip_scan)

Everything runs on ROCm tensors; a CPU tensor raises RuntimeError (there is no CPU path).
"""

import ctypes

import torch

from . import _abi, plan
from .hip_scan import METHODS, FusedSelectiveScanFn, _check_shapes, _require_gpu
from .profiling import timed_launch

DISCRETIZATIONS = ("zoh", "euler", "bilinear")      # models/scan.py:36
SCAN_ELEMENT_BUDGET = plan.SCAN_ELEMENT_BUDGET       # models/scan.py:182
_SCAN_ALGO = {"sequential": 1, "hillis_steele": 2, "blelloch": 3, "chunked": 4}


def default_chunk(L):
    """max(4, 2^ceil(log2 sqrt(L))) (models/scan.py:138-139), computed in exact integers."""
    return plan.default_chunk(L)


def _blocks(shape_bld, N, d_block):
    """Channel tiles of SelectiveScanFn (models/scan.py:185-190)."""
    return plan.blocks(shape_bld, N, d_block)


def _ct(*ts):
    dt = torch.float32
    for t in ts:
        if t is not None:
            dt = torch.promote_types(dt, t.dtype)
    return dt


def _launch(name, fn, args, dev):
    with _abi.on_device(dev):
        stream = _abi.stream_handle(dev)
        rc = timed_launch(name, stream, lambda: fn(ctypes.byref(args), stream))
    _abi.check(rc, name)


# ------------------------------------------------------------------ discretization
class DiscretizeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, delta, A, Bm, x, method):
        ct = delta.dtype
        Bsz, L, D = x.shape
        N = A.shape[1]
        a = torch.empty((Bsz, L, D, N), dtype=ct, device=x.device)
        b = torch.empty_like(a)
        args = _disc_args(delta, A, Bm, x, method)
        args.a, args.b = a.data_ptr(), b.data_ptr()
        _launch("ssm_disc_fwd", _abi.lib().ssm_disc_fwd, args, x.device)
        ctx.save_for_backward(delta, A, Bm, x)
        ctx.method = method
        return a, b

    @staticmethod
    def backward(ctx, da, db):
        delta, A, Bm, x = ctx.saved_tensors
        dev = x.device
        shape = (*x.shape, A.shape[1])
        if da is None:
            da = torch.zeros(shape, dtype=delta.dtype, device=dev)
        if db is None:
            db = torch.zeros(shape, dtype=delta.dtype, device=dev)
        da, db = da.contiguous(), db.contiguous()
        ddelta, dx = torch.empty_like(delta), torch.empty_like(x)
        dA, dB = torch.empty_like(A), torch.empty_like(Bm)
        args = _disc_args(delta, A, Bm, x, ctx.method)
        args.da, args.db = da.data_ptr(), db.data_ptr()
        args.ddelta, args.dx, args.dA, args.dBm = (_abi.view(t) for t in (ddelta, dx, dA, dB))
        lib = _abi.lib()
        nbytes = lib.ssm_disc_workspace_bytes(ctypes.byref(args))
        if nbytes < 0:
            _abi.check(lib.ssm_disc_check(ctypes.byref(args)), "ssm_disc_bwd")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        _launch("ssm_disc_bwd", lib.ssm_disc_bwd, args, dev)
        return ddelta, dA, dB, dx, None


def _disc_args(delta, A, Bm, x, method):
    Bsz, L, D = x.shape
    args = _abi.DiscArgs()
    args.batch, args.seqlen, args.dim, args.dstate = Bsz, L, D, A.shape[1]
    args.method = METHODS[method]
    args.dtype = _abi.DTYPE_CODE[delta.dtype]
    args.delta, args.x, args.A, args.Bm = (_abi.view(t) for t in (delta, x, A, Bm))
    return args


def discretize(delta, A, Bm, x, method="zoh"):
    """delta, x: (B, L, D); A: (D, N) with A < 0; Bm: (B, L, N) -> a, b: (B, L, D, N).

    zoh a = exp(dA), b = expm1(dA)/A * B x; euler b = delta B x; bilinear (Tustin)
    a = (1 + dA/2)/(1 - dA/2), b = delta/(1 - dA/2) B x (models/scan.py:39-55).
    Differentiable in all four tensors."""
    if method not in DISCRETIZATIONS:
        raise ValueError(f"unknown discretization {method!r}")
    _require_gpu(delta, A, Bm, x)
    _check_shapes(x, delta, A, Bm, Bm, None, None, None, None)  # the kernels index by (B, L, D, N)
    ct = _ct(delta, A, Bm, x)
    return DiscretizeFn.apply(delta.to(ct), A.to(ct), Bm.to(ct), x.to(ct), method)


def zoh_matrix(A, B, delta):
    """Dense ZOH (models/scan.py:58-62): Ad = expm(A delta), Bd = A^{-1}(Ad - I) B.
    A test helper for general (non-diagonal) A; uses the device's linear-algebra library."""
    Ad = torch.matrix_exp(A * delta)
    eye = torch.eye(A.shape[0], dtype=A.dtype, device=A.device)
    return Ad, torch.linalg.solve(A, (Ad - eye) @ B)


# ------------------------------------------------------------------ linear scans
class LinearScanFn(torch.autograd.Function):
    """h = scan(a, b, h0) on (B, L, M) with a chosen algorithm; backward via ssm_lscan_bwd."""

    @staticmethod
    def forward(ctx, a, b, h0, algo, chunk, reverse):
        Bsz, L, M = a.shape
        h = torch.empty((Bsz, L, M), dtype=a.dtype, device=a.device)
        args = _abi.LscanArgs()
        _lscan_common(args, a, algo, chunk, reverse)
        args.a, args.b, args.h0, args.h = (_abi.view(t) for t in (a, b, h0, h))
        lib = _abi.lib()
        nbytes = lib.ssm_lscan_workspace_bytes(ctypes.byref(args))
        if nbytes < 0:
            _abi.check(lib.ssm_lscan_check(ctypes.byref(args)), "ssm_lscan")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=a.device) if nbytes else None
        if ws is not None:
            args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        _launch("ssm_lscan", lib.ssm_lscan, args, a.device)
        ctx.save_for_backward(a, h0, h)
        ctx.cfg = (algo, chunk, reverse)
        return h

    @staticmethod
    def backward(ctx, dh):
        a, h0, h = ctx.saved_tensors
        algo, chunk, reverse = ctx.cfg
        da, db = torch.empty_like(h), torch.empty_like(h)
        dh0 = torch.empty_like(h0) if h0 is not None and ctx.needs_input_grad[2] else None
        lscan_bwd(a, h0, h, dh, da, db, dh0, algo, chunk, reverse)
        return da, db, dh0, None, None, None


def _lscan_common(args, a, algo, chunk, reverse):
    Bsz, L, M = a.shape
    args.batch, args.seqlen, args.width = Bsz, L, M
    args.algo, args.dtype, args.reverse = algo, _abi.DTYPE_CODE[a.dtype], int(bool(reverse))
    args.chunk = int(chunk or 0)


def lscan_bwd(a, h0, h, dh, da, db, dh0, algo, chunk=None, reverse=False):
    """Adjoint of a linear scan into preallocated (B, L, M) da, db (= lambda) and (B, M) dh0."""
    args = _abi.LscanBwdArgs()
    _lscan_common(args, a, algo, chunk, reverse)
    args.a, args.h0, args.h, args.dh = (_abi.view(t) for t in (a, h0, h, dh))
    args.da, args.db, args.dh0 = (_abi.view(t) for t in (da, db, dh0))
    lib = _abi.lib()
    nbytes = lib.ssm_lscan_bwd_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        _abi.check(lib.ssm_lscan_bwd_check(ctypes.byref(args)), "ssm_lscan_bwd")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=a.device) if nbytes else None
    if ws is not None:
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    _launch("ssm_lscan_bwd", lib.ssm_lscan_bwd, args, a.device)


def _scan(name, a, b, h0=None, chunk_size=None, reverse=False):
    """a, b (B, L, *rest), h0 (B, *rest) -> h (B, L, *rest) by the named algorithm."""
    _require_gpu(a, b, h0)
    if a.shape != b.shape or a.dim() < 2:
        raise ValueError(f"a and b must share a (B, L, ...) shape, got {tuple(a.shape)} and {tuple(b.shape)}")
    if h0 is not None and (tuple(h0.shape) != (a.shape[0],) + tuple(a.shape[2:])):
        raise ValueError(f"h0 must have shape {(a.shape[0],) + tuple(a.shape[2:])}, got {tuple(h0.shape)}")
    shape = a.shape
    Bsz, L = shape[:2]
    M = 1
    for s in shape[2:]:
        M *= s
    ct = _ct(a, b, h0)
    a3 = a.to(ct).reshape(Bsz, L, M)
    b3 = b.to(ct).reshape(Bsz, L, M)
    h03 = None if h0 is None else h0.to(ct).reshape(Bsz, M)
    h = LinearScanFn.apply(a3, b3, h03, _SCAN_ALGO[name], chunk_size, reverse)
    return h.reshape(shape).to(b.dtype)


def scan_sequential(a, b, h0=None):
    """h_t = a_t h_{t-1} + b_t, one lane per recurrence (models/scan.py:70-76)."""
    return _scan("sequential", a, b, h0)


def scan_hillis_steele(a, b, h0=None):
    """Recursive-doubling inclusive scan (models/scan.py:87-98)."""
    return _scan("hillis_steele", a, b, h0)


def scan_blelloch(a, b, h0=None):
    """Work-efficient up-sweep / down-sweep scan (models/scan.py:101-135)."""
    return _scan("blelloch", a, b, h0)


def scan_chunked(a, b, h0=None, chunk_size=None):
    """Two-level scan with chunk size C = chunk_size or default_chunk(L) (models/scan.py:142-165)."""
    return _scan("chunked", a, b, h0, chunk_size)


SCANS = {
    "sequential": scan_sequential,
    "hillis_steele": scan_hillis_steele,
    "blelloch": scan_blelloch,
    "chunked": scan_chunked,
}


def _scan_algo(name):
    """Algorithm id for a SCANS name; KeyError otherwise (models/scan.py:258-261)."""
    SCANS[name]
    return _SCAN_ALGO[name]


# ------------------------------------------------------------------ composed selective scan
def _scan_into(algo, chunk, a, b, h0):
    """Forward scan of (B, L, d, N) tensors into a new (B, L, d, N) h."""
    Bsz, L, d, N = a.shape
    h = torch.empty_like(a)
    args = _abi.LscanArgs()
    _lscan_common(args, a.view(Bsz, L, d * N), algo, chunk, False)
    args.a = _abi.view(a.view(Bsz, L, d * N))
    args.b = _abi.view(b.view(Bsz, L, d * N))
    args.h0 = _abi.view(None if h0 is None else h0.reshape(Bsz, d * N))
    args.h = _abi.view(h.view(Bsz, L, d * N))
    lib = _abi.lib()
    nbytes = lib.ssm_lscan_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        _abi.check(lib.ssm_lscan_check(ctypes.byref(args)), "ssm_lscan")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=a.device) if nbytes else None
    if ws is not None:
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    _launch("ssm_lscan", lib.ssm_lscan, args, a.device)
    return h


def _disc_fwd(delta, A, Bm, x, method):
    Bsz, L, d = x.shape
    N = A.shape[1]
    a = torch.empty((Bsz, L, d, N), dtype=delta.dtype, device=x.device)
    b = torch.empty_like(a)
    args = _disc_args(delta, A, Bm, x, method)
    args.a, args.b = a.data_ptr(), b.data_ptr()
    _launch("ssm_disc_fwd", _abi.lib().ssm_disc_fwd, args, x.device)
    return a, b


class SelectiveScanFn(torch.autograd.Function):
    """y, last = selective scan with recomputation (models/scan.py:193-255).

    Saves only x, delta, A, Bm, Cm, h0.  Channels run in tiles of d_block (default sized to
    SCAN_ELEMENT_BUDGET); per tile the forward discretizes into (B, L, d, N), scans with the
    chosen algorithm and contracts with C; the backward recomputes the states, runs the
    adjoint scan lambda_t = g_t + a_{t+1} lambda_{t+1} with the same algorithm and maps
    (da, db) = (lambda h_{t-1}, lambda) back through the discretization."""

    @staticmethod
    def forward(ctx, x, delta, A, Bm, Cm, h0, method, scan_name, d_block, chunk_size):
        algo = _scan_algo(scan_name)
        if method not in DISCRETIZATIONS:
            raise ValueError(f"unknown discretization {method!r}")
        Bsz, L, D = x.shape
        N = A.shape[1]
        y = torch.empty_like(x)
        last = torch.empty(Bsz, D, N, dtype=x.dtype, device=x.device)
        Cc = Cm.unsqueeze(-1)
        for i, j in _blocks(x.shape, N, d_block):
            a, b = _disc_fwd(delta[..., i:j], A[i:j], Bm, x[..., i:j], method)
            h = _scan_into(algo, chunk_size, a, b, None if h0 is None else h0[:, i:j])
            del a, b
            y[..., i:j] = torch.matmul(h, Cc).squeeze(-1)
            last[:, i:j] = h[:, -1]
            del h
        ctx.save_for_backward(x, delta, A, Bm, Cm, h0)
        ctx.cfg = (method, algo, d_block, chunk_size)
        return y, last

    @staticmethod
    def backward(ctx, dy, dlast):
        x, delta, A, Bm, Cm, h0 = ctx.saved_tensors
        method, algo, d_block, chunk_size = ctx.cfg
        Bsz, L, D = x.shape
        N = A.shape[1]
        dev = x.device
        if dy is None:
            dy = torch.zeros_like(x)
        dx, ddelta, dA = torch.empty_like(x), torch.empty_like(delta), torch.empty_like(A)
        dBm, dCm = torch.zeros_like(Bm), torch.zeros_like(Cm)
        dh0 = None if h0 is None else torch.empty_like(h0)
        lib = _abi.lib()
        for i, j in _blocks(x.shape, N, d_block):
            d = j - i
            h0_blk = None if h0 is None else h0[:, i:j]
            a, b = _disc_fwd(delta[..., i:j], A[i:j], Bm, x[..., i:j], method)
            h = _scan_into(algo, chunk_size, a, b, h0_blk)                 # recompute
            del b
            dy_blk = dy[..., i:j]
            dCm += torch.matmul(dy_blk.unsqueeze(2), h).squeeze(2)
            g = dy_blk.unsqueeze(-1) * Cm.unsqueeze(2)                       # dL/dh_t (direct)
            if dlast is not None:
                g[:, -1] += dlast[:, i:j]
            da, lam = torch.empty_like(h), torch.empty_like(h)
            dh0_blk = None if h0 is None else torch.empty((Bsz, d, N), dtype=h.dtype, device=dev)
            M = d * N
            lscan_bwd(a.view(Bsz, L, M), None if h0_blk is None else h0_blk.reshape(Bsz, M),
                      h.view(Bsz, L, M), g.view(Bsz, L, M), da.view(Bsz, L, M), lam.view(Bsz, L, M),
                      None if dh0_blk is None else dh0_blk.view(Bsz, M), algo, chunk_size, False)
            del g, h, a
            if dh0 is not None:
                dh0[:, i:j] = dh0_blk
            gB = torch.empty_like(Bm)
            args = _disc_args(delta[..., i:j], A[i:j], Bm, x[..., i:j], method)
            args.da, args.db = da.data_ptr(), lam.data_ptr()
            args.ddelta, args.dx = _abi.view(ddelta[..., i:j]), _abi.view(dx[..., i:j])
            args.dA, args.dBm = _abi.view(dA[i:j]), _abi.view(gB)
            nbytes = lib.ssm_disc_workspace_bytes(ctypes.byref(args))
            if nbytes < 0:
                _abi.check(lib.ssm_disc_check(ctypes.byref(args)), "ssm_disc_bwd")
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
            args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
            _launch("ssm_disc_bwd", lib.ssm_disc_bwd, args, dev)
            dBm += gB
            del da, lam, ws
        return dx, ddelta, dA, dBm, dCm, dh0, None, None, None, None


def selective_scan_reference(x, delta, A, Bm, Cm, h0=None, method="zoh"):
    """The step-by-step recurrence of models/scan.py:264-274, returning (y, h_last).

    Runs on the fused engine, which walks h_t = a_t h_{t-1} + b_t one time step at a time
    in every lane -- the same recurrence as the reference's loop, without storing the states."""
    if method not in DISCRETIZATIONS:
        raise ValueError(f"unknown discretization {method!r}")
    _require_gpu(x, delta, A, Bm, Cm, h0)
    _check_shapes(x, delta, A, Bm, Cm, None, None, None, h0)
    return FusedSelectiveScanFn.apply(x, delta, A, Bm, Cm, None, None, None, h0, METHODS[method], False)


def selective_scan(x, delta, A, Bm, Cm, h0=None, method="zoh", scan="chunked",
                   d_block=None, chunk_size=None):
    """Returns (y, h_last) (models/scan.py:277-299).

    scan = 'reference' | 'sequential' | 'hillis_steele' | 'blelloch' | 'chunked'
           | 'triton' (the fused engine) | 'auto' (fused when N is a power of two, else chunked)
    Computes in promote(dtype, float32); y is returned in x's dtype, h_last in the compute
    dtype.  KeyError for an unknown scan, ValueError for an unknown method."""
    _require_gpu(x, delta, A, Bm, Cm, h0)
    if scan == "auto":
        scan = plan.resolve_scan("auto", x.is_cuda, method, A.shape[1])
    elif scan not in _abi.SCAN_IDS:
        raise KeyError(scan)
    dtype = x.dtype
    ct = torch.promote_types(dtype, torch.float32)
    with torch.autocast(device_type=x.device.type, enabled=False):
        if scan == "triton":
            from .hip_scan import selective_scan_hip
            # the engine reads low-precision inputs directly and computes in ct
            y, last = selective_scan_hip(x, delta, A.to(ct), Bm, Cm, None if h0 is None else h0.to(ct),
                                         method=method, d_block=d_block)
            return y.to(dtype), last
        args = [t.to(ct) if t is not None else None for t in (x, delta, A, Bm, Cm, h0)]
        if scan == "reference":
            y, last = selective_scan_reference(*args, method=method)
        else:
            _check_shapes(*args[:5], None, None, None, args[5])
            y, last = SelectiveScanFn.apply(*args, method, scan, d_block, chunk_size)
    return y.to(dtype), last
