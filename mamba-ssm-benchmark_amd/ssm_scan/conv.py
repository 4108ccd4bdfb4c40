"""Causal depthwise conv1d + SiLU on the HIP engine: the producer of the scan's input.

Counterpart of models/mamba.py:101-107 (F.pad / state concat, F.conv1d with groups=D, SiLU,
and the conv-state update of :104-106).  ``x`` is the (B, L, D) view the in_proj split gives
(no transposes or copies are needed); the output is (B, L, D) contiguous, which the fused scan
reads directly.  Training uses ``causal_conv1d`` (differentiable in x, weight and bias); the
recurrent decode step passes a ``state`` (B, D, W-1) that is read and then updated in place.
"""

import ctypes

import torch

from . import _abi
from .hip_scan import _require_gpu


def _weight2d(weight):
    """nn.Conv1d's (D, 1, W) weight, or a (D, W) tensor, as (D, W)."""
    return weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight


def _args(x, weight, bias, activation):
    Bsz, L, D = x.shape
    args = _abi.ConvArgs()
    args.batch, args.seqlen, args.dim, args.width = Bsz, L, D, weight.shape[1]
    args.dtype = _abi.DTYPE_CODE[x.dtype]
    args.silu = 1 if activation else 0
    args.x, args.weight, args.bias = _abi.view(x), _abi.view(weight), _abi.view(bias)
    return args


def _launch(name, fn, args, dev):
    with _abi.on_device(dev):
        rc = fn(ctypes.byref(args), _abi.stream_handle(dev))
    _abi.check(rc, name)


def conv_forward(x, w2, bias, activation):
    """One ssm_conv_fwd launch: (B, L, D) out for x, weight (D, W) and bias in the state type."""
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    args = _args(x, w2, bias, activation)
    args.out = _abi.view(out)
    _launch("ssm_conv_fwd", _abi.lib().ssm_conv_fwd, args, x.device)
    return out


def conv_backward(x, w2, bias, dout, activation, dx=None):
    """One ssm_conv_bwd launch: (dx, dweight, dbias).  dx may be given (a (B, L, D) view into a
    caller's buffer); it is allocated otherwise."""
    dev = x.device
    dout = dout.to(x.dtype)
    dx = torch.empty(x.shape, dtype=x.dtype, device=dev) if dx is None else dx
    dw = torch.empty_like(w2)
    db = None if bias is None else torch.empty_like(bias)
    args = _args(x, w2, bias, activation)
    args.dout, args.dx = _abi.view(dout), _abi.view(dx)
    args.dweight, args.dbias = _abi.view(dw), _abi.view(db)
    lib = _abi.lib()
    nbytes = lib.ssm_conv_workspace_bytes(ctypes.byref(args))
    if nbytes < 0:
        _abi.check(lib.ssm_conv_check(ctypes.byref(args)), "ssm_conv_bwd")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    _launch("ssm_conv_bwd", lib.ssm_conv_bwd, args, dev)
    return dx, dw, db


class CausalConv1dFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, activation):
        ct = torch.promote_types(x.dtype, torch.float32)
        w2, bv = weight.to(ct), None if bias is None else bias.to(ct)
        out = conv_forward(x, w2, bv, activation)
        ctx.save_for_backward(x, w2, bv)
        ctx.activation = activation
        ctx.wdtype = weight.dtype
        ctx.bdtype = None if bias is None else bias.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        x, w2, bv = ctx.saved_tensors
        dx, dw, db = conv_backward(x, w2, bv, dout, ctx.activation)
        return dx, dw.to(ctx.wdtype), None if db is None else db.to(ctx.bdtype), None


def causal_conv1d(x, weight, bias=None, state=None, activation=True):
    """out = silu(conv1d(pad_left(x), weight, bias, groups=D)) over time, as (B, L, D).

    x (B, L, D); weight (D, W) or nn.Conv1d's (D, 1, W); bias (D,) or None.  With ``state``
    (B, D, W-1) the previous inputs replace the zero padding and ``state`` is overwritten with
    the last W-1 inputs (models/mamba.py:104-106); that path is not differentiable."""
    _require_gpu(x, weight, bias, state)
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got {tuple(x.shape)}")
    w2 = _weight2d(weight)
    Bsz, L, D = x.shape
    if w2.shape[0] != D:
        raise ValueError(f"weight must have {D} channels, got {tuple(weight.shape)}")
    if bias is not None and tuple(bias.shape) != (D,):
        raise ValueError(f"bias must be ({D},), got {tuple(bias.shape)}")
    if state is None:
        return CausalConv1dFn.apply(x, w2, bias, bool(activation))
    W = w2.shape[1]
    if tuple(state.shape) != (Bsz, D, W - 1) or state.dtype != x.dtype:
        raise ValueError(f"state must be ({Bsz}, {D}, {W - 1}) of {x.dtype}, got {tuple(state.shape)} {state.dtype}")
    ct = torch.promote_types(x.dtype, torch.float32)
    w2c, bv = w2.detach().to(ct), None if bias is None else bias.detach().to(ct)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    args = _args(x, w2c, bv, activation)
    args.state_in, args.state_out, args.out = _abi.view(state), _abi.view(state), _abi.view(out)
    _launch("ssm_conv_fwd", _abi.lib().ssm_conv_fwd, args, x.device)
    return out
