"""RMSNorm on the HIP engine: the LM's pre-norms (models/common.py:8-16).

``rms_norm(x, weight, eps)`` computes ``(x * rsqrt(mean(x^2, -1) + eps)) * weight`` in one
launch forward and two backward (the row kernel and the weight-gradient sum), in place of the
six forward and about ten backward torch kernels of the composed expression.  float32 rows of
up to 1024 elements with a float32 weight run on the kernels.  Other inputs keep the
reference's torch expression on the GPU, which gives what the reference gives: a bf16
residual stream under autocast (its product with the float32 weight promotes), float64 rows
(the reference normalizes them in float32, `x.float()`), wider rows.  The C ABI also takes
float64 rows, computed in float64 throughout.
"""

import ctypes

import torch

from . import _abi
from .hip_scan import _require_gpu

MAX_DIM = 1024


def _args(x2, weight, eps):
    args = _abi.NormArgs()
    args.rows, args.dim = x2.shape
    args.dtype = _abi.DTYPE_CODE[x2.dtype]
    args.eps = float(eps)
    args.x, args.weight = _abi.view(x2), _abi.view(weight)
    return args


def _launch(name, fn, args, dev):
    with _abi.on_device(dev):
        rc = fn(ctypes.byref(args), _abi.stream_handle(dev))
    _abi.check(rc, name)


class RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
        rstd = torch.empty(x2.shape[0], dtype=x.dtype, device=x.device)
        w = weight.contiguous()
        args = _args(x2, w, eps)
        args.out, args.rstd = _abi.view(out), rstd.data_ptr()
        _launch("ssm_norm_fwd", _abi.lib().ssm_norm_fwd, args, x.device)
        ctx.save_for_backward(x2, w, rstd)
        ctx.eps, ctx.shape = eps, shape
        return out.view(shape)

    @staticmethod
    def backward(ctx, dout):
        x2, w, rstd = ctx.saved_tensors
        dev = x2.device
        dy = dout.reshape(x2.shape)
        if dy.dtype != x2.dtype:
            dy = dy.to(x2.dtype)
        if dy.stride(-1) != 1:
            dy = dy.contiguous()
        dx = torch.empty(x2.shape, dtype=x2.dtype, device=dev)
        dw = torch.empty(w.shape, dtype=w.dtype, device=dev)
        args = _args(x2, w, ctx.eps)
        args.rstd = rstd.data_ptr()
        args.dout, args.dx, args.dweight = _abi.view(dy), _abi.view(dx), dw.data_ptr()
        lib = _abi.lib()
        nbytes = lib.ssm_norm_workspace_bytes(ctypes.byref(args))
        if nbytes < 0:
            _abi.check(lib.ssm_norm_check(ctypes.byref(args)), "ssm_norm_bwd")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        _launch("ssm_norm_bwd", lib.ssm_norm_bwd, args, dev)
        return dx.view(ctx.shape), dw, None


def rms_norm_reference(x, weight, eps):
    """models/common.py:14-16 as torch ops (any dtype)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * weight


def rms_norm(x, weight, eps=1e-5):
    """models/common.py:14-16.  The kernels run for float32 x and weight and a last dimension
    <= 1024; otherwise the reference's torch expression runs on the GPU."""
    _require_gpu(x, weight)
    if tuple(weight.shape) != (x.shape[-1],):  # the kernels read dim weights
        raise ValueError(f"weight must be ({x.shape[-1]},), got {tuple(weight.shape)}")
    if (x.dtype == torch.float32 and weight.dtype == torch.float32 and 0 < x.shape[-1] <= MAX_DIM
            and x.numel() > 0):
        return RMSNormFn.apply(x, weight, eps)
    return rms_norm_reference(x, weight, eps)
