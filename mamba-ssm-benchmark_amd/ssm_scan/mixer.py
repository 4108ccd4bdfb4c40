"""One Mamba layer's path from the in_proj output to the scan output as a single autograd
node (models/mamba.py:100-124 between in_proj and out_proj): conv1d + SiLU, x_proj, and the
fused scan with dt_proj, its bias and softplus, A = -exp(A_log), the D skip and the SiLU(z)
gate.

The forward is the same launches as the module-by-module path (conv kernel, x_proj GEMM, one
ssm_fwd).  The backward writes the gradients of the conv input and of the gate into one
(B, L, 2 d_inner) buffer -- the gradient of the in_proj output -- and those of the low-rank dt,
B and C into one (B, L, dt_rank + 2 N) buffer -- the gradient of the x_proj output -- so the
concatenations that autograd of `chunk` / `split` adds disappear, and the layer's backward is
one Python call instead of a chain of autograd nodes.
"""

import torch
import torch.nn.functional as F

from .conv import conv_backward, conv_forward
from .hip_scan import LOWRANK_MAX, METHODS, scan_backward, scan_forward
from .linear import rocblas, weight_grad


class MixerFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xz, conv_w, conv_b, xproj_w, dtproj_w, dt_bias, A_log, Dv, method):
        Dm = xz.shape[-1] // 2
        R = dtproj_w.shape[1]
        N = A_log.shape[1]
        x, z = xz[..., :Dm], xz[..., Dm:]
        w2 = conv_w.reshape(conv_w.shape[0], conv_w.shape[-1])
        xc = conv_forward(x, w2, conv_b, True)
        with rocblas():
            proj = F.linear(xc, xproj_w)
        dt, Bm, Cm = proj[..., :R], proj[..., R:R + N], proj[..., R + N:]
        need = any(ctx.needs_input_grad)
        y, _, (tensors, settings) = scan_forward(xc, dt, A_log, Bm, Cm, Dv, z, dt_bias, None, method, True, 0,
                                                 dtproj_w, True, need_saved=need)
        if need:
            ctx.save_for_backward(xz, xc, proj, w2, conv_b, xproj_w, *tensors)
        ctx.settings = settings
        ctx.conv_shape = conv_w.shape
        return y

    @staticmethod
    def backward(ctx, dy):
        xz, xc, proj, w2, conv_b, xproj_w, *tensors = ctx.saved_tensors
        Dm = xz.shape[-1] // 2
        Wdt = tensors[9]
        R = Wdt.shape[1]
        P = proj.shape[-1]
        N = (P - R) // 2
        dxz = torch.empty_like(xz)
        dproj = torch.empty_like(proj)
        dxc, dd, dA, _, _, dD, _, db, _ = scan_backward(tensors, ctx.settings, dy, None, dz=dxz[..., Dm:],
                                                        dB=dproj[..., R:R + N], dC=dproj[..., R + N:])
        dd2 = dd.reshape(-1, Dm)
        dt2 = proj.reshape(-1, P)[:, :R]
        with rocblas():
            dW_dt = weight_grad(dd2, dt2)                       # dt_proj weight (D, R)
            dproj[..., :R] = (dd2 @ Wdt).view(dd.shape[:-1] + (R,))
            dproj2 = dproj.view(-1, P)
            dxc2 = torch.addmm(dxc.reshape(-1, Dm), dproj2, xproj_w).view(xc.shape)
            dW_x = weight_grad(dproj2, xc.reshape(-1, Dm))      # x_proj weight (P, D)
        _, dwc, dbc = conv_backward(xz[..., :Dm], w2, conv_b, dxc2, True, dx=dxz[..., :Dm])
        return dxz, dwc.view(ctx.conv_shape), dbc, dW_x, dW_dt, db, dA, dD, None


def mixer_applies(m, u, state, return_delta):
    """The single-node path serves the training / prefill-without-state forward of a selective
    S4D-A layer in float32 with a fused scan, a low-rank dt_proj the kernels apply (rank and
    dstate <= 16) and no autocast."""
    return (state is None and not return_delta and not getattr(m, "record_delta", False)
            and m.selective and m.a_mode == "s4d" and m.scan in ("auto", "triton")
            and u.dtype == torch.float32 and m.dt_rank <= LOWRANK_MAX and m.d_state <= 16
            and m.A_log.dtype == torch.float32 and not torch.is_autocast_enabled(u.device.type))


def mixer(m, xz):
    """y of the Mamba layer `m` for its in_proj output xz (B, L, 2 d_inner)."""
    return MixerFn.apply(xz, m.conv.weight, m.conv.bias, m.x_proj.weight, m.dt_proj.weight, m.dt_proj.bias,
                         m.A_log, m.D, METHODS[m.discretization])
