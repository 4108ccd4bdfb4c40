"""torch-CPU float64 restatement of the reference's Mamba LM (test infrastructure only).

Restates models/mamba.py:93-126 (Mamba.forward: in_proj, causal depthwise conv + SiLU,
x_proj / dt_proj / softplus, selective scan, D skip, SiLU(z) gate, out_proj; the recurrent
decode step of :113-118 and the state updates of :104-106, :122-123) and models/lm.py
(pre-norm residual blocks, RMSNorm of models/common.py:8-16, tied head), with the scan as the
textbook time loop of models/scan.py:264-274, so autograd gives every gradient.  It reads the
parameters of a model's state_dict by the reference's names.  Used by tests only.

For sizes where autograd through the time loop would hold (B, D, N) tensors per step (BASELINE
config 3: 10 layers at B16 x L512), `scan="c"` runs each layer's scan + D skip + SiLU(z) gate
as one autograd node over oracle/ssm_oracle.c's float64 forward and hand-written adjoint
(kernels/triton_scan.py:171-226).  It is pinned against the loop by
tests/test_lm_host.py (forward and every parameter gradient, float64).
"""

import torch
import torch.nn.functional as F

from . import c_oracle


def rmsnorm(x, w, eps=1e-5):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def discretize(delta, A, Bm, x, method):
    """models/scan.py:39-55 on (B, D) inputs -> (B, D, N)."""
    dA = delta.unsqueeze(-1) * A
    Bx = x.unsqueeze(-1) * Bm.unsqueeze(1)
    if method == "zoh":
        return torch.exp(dA), torch.expm1(dA) / A * Bx
    if method == "euler":
        return torch.exp(dA), delta.unsqueeze(-1) * Bx
    inv = 1.0 / (1.0 - 0.5 * dA)
    return (1.0 + 0.5 * dA) * inv, delta.unsqueeze(-1) * inv * Bx


class _CScan(torch.autograd.Function):
    """out = (scan(x, delta, A, B, C) + D x) * silu(z) in float64 on the C oracle, h0 = 0."""

    @staticmethod
    def forward(ctx, x, delta, A, Bm, Cm, Dv, z, method):
        ctx.method = method
        ctx.save_for_backward(x, delta, A, Bm, Cm, Dv, z)
        out, _, _ = c_oracle.fwd(*(t.detach().numpy() for t in (x, delta, A, Bm, Cm)), None, method,
                                 Dv.detach().numpy(), z.detach().numpy())
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, dout):
        x, delta, A, Bm, Cm, Dv, z = ctx.saved_tensors
        g = c_oracle.bwd(*(t.detach().numpy() for t in (x, delta, A, Bm, Cm)), dout.numpy(), None,
                         ctx.method, Dv.detach().numpy(), z.detach().numpy())
        return tuple(torch.from_numpy(g[k]) for k in ("dx", "ddelta", "dA", "dB", "dC", "dD", "dz")) + (None,)


def mamba_layer(p, pre, u, d_state, dt_rank, d_conv, state=None, method="zoh", scan="loop"):
    """One Mamba mixer on u (B, L, d_model); p maps parameter names (prefix `pre`) to tensors.
    With `state` (dict conv (B, D, W-1), ssm (B, D, N)) it continues a sequence and updates it.
    scan="c" (no state): the scan, skip and gate as one node on the C oracle."""
    Bsz, L, _ = u.shape
    x, z = F.linear(u, p[pre + "in_proj.weight"]).chunk(2, dim=-1)
    D = x.shape[-1]
    xc = x.transpose(1, 2)
    if state is None:
        xc = F.pad(xc, (d_conv - 1, 0))
    else:
        xc = torch.cat([state["conv"], xc], dim=-1)
        state["conv"] = xc[..., xc.shape[-1] - (d_conv - 1):].clone()  # (B, D, 0) at width 1
    x = F.silu(F.conv1d(xc, p[pre + "conv.weight"], p[pre + "conv.bias"], groups=D)).transpose(1, 2)
    dt, Bm, Cm = F.linear(x, p[pre + "x_proj.weight"]).split([dt_rank, d_state, d_state], dim=-1)
    delta = F.softplus(F.linear(dt, p[pre + "dt_proj.weight"], p[pre + "dt_proj.bias"]))
    A = -torch.exp(p[pre + "A_log"])
    if scan == "c":
        if state is not None:
            raise ValueError("scan='c' runs whole sequences from a zero state")
        return F.linear(_CScan.apply(x, delta, A, Bm, Cm, p[pre + "D"], z, method), p[pre + "out_proj.weight"])
    h = torch.zeros(Bsz, D, d_state, dtype=u.dtype) if state is None else state["ssm"]
    ys = []
    for t in range(L):
        a, b = discretize(delta[:, t], A, Bm[:, t], x[:, t], method)
        h = a * h + b
        ys.append((h * Cm[:, t].unsqueeze(1)).sum(-1))
    if state is not None:
        state["ssm"] = h
    y = torch.stack(ys, 1)
    y = (y + x * p[pre + "D"]) * F.silu(z)
    return F.linear(y, p[pre + "out_proj.weight"])


def lm_forward(p, idx, n_layers, d_state=16, dt_rank=16, d_conv=4, states=None, method="zoh", scan="loop"):
    """Logits (B, L, V) of the Mamba LM (models/lm.py:LM.forward with kind-"M" blocks)."""
    x = F.embedding(idx, p["embed.weight"])
    for i in range(n_layers):
        pre = f"blocks.{i}."
        h = rmsnorm(x, p[pre + "norm1.weight"])
        x = x + mamba_layer(p, pre + "mixer.", h, d_state, dt_rank, d_conv,
                            None if states is None else states[i], method, scan)
    return F.linear(rmsnorm(x, p["norm_f.weight"]), p["embed.weight"])
