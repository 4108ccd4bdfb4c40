"""The dt_proj projection fused into the scan kernels (selective_scan_fn(..., delta_proj=W)):
delta is the low-rank (B, L, R) input dt and the scan uses dt @ W^T + bias, softplus
(models/mamba.py:75-76).  Checked against the float64 oracle on delta = dt @ W^T computed in
float64, including the gradients of dt and W (the GEMM backward of F.linear), and against the
engine's own path with the projection done by a torch GEMM first.

Tolerances as the fused tests: float32 rtol 1e-4 / atol 1e-5 (tests/parity.py) on every output and
gradient; bf16 inputs rtol 2e-2.
"""

import numpy as np
import pytest
import torch

import ssm_scan
from oracle import scan_ref as R
from ssm_inputs import np64

from parity import ATOL, RTOL, close, close_or_cancelled  # noqa: F401  (the north_star bar)

pytestmark = pytest.mark.gpu


def make(B, L, D, N, Rk, seed, channel_major=False, dtype=torch.float32):
    """x (optionally channel-major storage), dt as the split view of an x_proj-like output
    (B, L, R + 2N) with B, C beside it, W (D, R), gate, skip, bias, A = S4D-real."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, L, D, generator=g)
    if channel_major:
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    proj = torch.randn(B, L, Rk + 2 * N, generator=g)
    W = torch.randn(D, Rk, generator=g) * (0.5 / Rk ** 0.5)
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1)
    Dv = torch.randn(D, generator=g)
    z = torch.randn(B, L, D, generator=g)
    bias = torch.rand(D, generator=g) * 2.0 - 4.0
    dout = torch.randn(B, L, D, generator=g)
    if dtype != torch.float32:
        x, proj, z = x.to(dtype), proj.to(dtype), z.to(dtype)
    return x, proj, W, A, Dv, z, bias, dout


def run(dev, x, proj, W, A, Dv, z, bias, dout, Rk, N, method, lowrank=True, segments=None):
    leaves = [t.to(dev).requires_grad_() for t in (x, proj, W, A, Dv, z, bias)]
    xg, pg, Wg, Ag, Dg, zg, bg = leaves
    dt, Bm, Cm = pg[..., :Rk], pg[..., Rk:Rk + N], pg[..., Rk + N:]
    if lowrank:
        out, last = ssm_scan.selective_scan_fn(xg, dt, Ag, Bm, Cm, D=Dg, z=zg, delta_bias=bg, delta_softplus=True,
                                               method=method, return_last_state=True, segments=segments,
                                               delta_proj=Wg)
    else:
        out, last = ssm_scan.selective_scan_fn(xg, torch.nn.functional.linear(dt, Wg), Ag, Bm, Cm, D=Dg, z=zg,
                                               delta_bias=bg, delta_softplus=True, method=method,
                                               return_last_state=True, segments=segments)
    (out.float() * dout.to(dev)).sum().backward()
    grads = {n: t.grad for n, t in zip(("dx", "dproj", "dW", "dA", "dD", "dz", "dbias"), leaves)}
    return out.detach(), last.detach(), grads


def oracle(x, proj, W, A, Dv, z, bias, dout, Rk, N, method):
    x, proj, W, A, Dv, z, bias, dout = (np64(t) for t in (x, proj, W, A, Dv, z, bias, dout))
    dt, Bm, Cm = proj[..., :Rk], proj[..., Rk:Rk + N], proj[..., Rk + N:]
    raw = dt @ W.T + bias
    delta = np.log1p(np.exp(raw))
    out, _, last = R.selective_scan_fwd(x, delta, A, Bm, Cm, None, method, Dv, z)
    g = R.selective_scan_bwd(x, delta, A, Bm, Cm, dout, None, method, Dv, z, None)
    draw = g["ddelta"] / (1.0 + np.exp(-raw))
    dproj = np.concatenate([draw @ W, g["dB"], g["dC"]], -1)
    dW = draw.reshape(-1, W.shape[0]).T @ dt.reshape(-1, Rk)
    dW_mag = np.abs(draw).reshape(-1, W.shape[0]).T @ np.abs(dt).reshape(-1, Rk)   # sum of |terms|
    return out, last, {"dx": g["dx"], "dproj": dproj, "dW": dW, "dA": g["dA"], "dD": g["dD"], "dz": g["dz"],
                       "dbias": draw.sum(axis=(0, 1)), "dW_mag": dW_mag}


@pytest.mark.parametrize("method", ["zoh", "euler", "bilinear"])
@pytest.mark.parametrize("Rk,N,channel_major", [(16, 16, True), (5, 16, False), (1, 8, True), (12, 32, False)])
def test_lowrank_delta_matches_oracle(dev, method, Rk, N, channel_major):
    B, L, D = 2, 83, 40
    ins = make(B, L, D, N, Rk, seed=Rk * 7 + N, channel_major=channel_major)
    out, last, grads = run(dev, *ins, Rk, N, method)
    rout, rlast, rg = oracle(*ins, Rk, N, method)
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        close(v, rg[k], name=k)


def test_lowrank_equals_projected_delta_at_config1_shape(dev):
    """B16 L512 D512 N16 R16 (the config-3 layer's scan shape): the fused projection and a
    torch GEMM before the scan give the same outputs and gradients (to float32 rounding)."""
    B, L, D, N, Rk = 16, 512, 512, 16, 16
    ins = make(B, L, D, N, Rk, seed=3, channel_major=True)
    a = run(dev, *ins, Rk, N, "zoh", lowrank=True)
    b = run(dev, *ins, Rk, N, "zoh", lowrank=False)
    for u, v, name in ((a[0], b[0], "out"), (a[1], b[1], "last")):
        close(u, np64(v), name=name)
    for k in a[2]:
        # dW is a float32 GEMM over the 8192 tokens in both paths, summed in different orders
        # (torch's F.linear backward vs the engine's token-sliced GEMMs): its absolute error
        # scales with the largest element; every scan output keeps the literal bar.
        atol = 1e-5 * max(1.0, float(b[2][k].abs().max())) if k == "dW" else 1e-5
        close(a[2][k], np64(b[2][k]), rtol=1e-4, atol=atol, name=k)


def test_lowrank_long_sequence_segments(dev):
    """The segmented long-sequence forward (summary, carry and main passes all stage delta
    through the projection) equals the unsegmented one."""
    B, L, D, N, Rk = 1, 4096, 64, 16, 16
    x, proj, W, A, Dv, z, bias, dout = (t.to(dev) for t in make(B, L, D, N, Rk, seed=5))
    dt, Bm, Cm = proj[..., :Rk], proj[..., Rk:Rk + N], proj[..., Rk + N:]
    with torch.no_grad():
        res = [ssm_scan.selective_scan_fn(x, dt, A, Bm, Cm, D=Dv, z=z, delta_bias=bias, delta_softplus=True,
                                          return_last_state=True, segments=s, delta_proj=W) for s in (1, 8)]
        ref = ssm_scan.selective_scan_fn(x, torch.nn.functional.linear(dt, W), A, Bm, Cm, D=Dv, z=z,
                                         delta_bias=bias, delta_softplus=True, return_last_state=True, segments=1)
    for y, last in res:
        close(y, np64(ref[0]), name="y")
        close(last, np64(ref[1]), name="last")


def test_lowrank_rank_above_capacity_uses_a_gemm(dev):
    """R = 24 (> 16) takes a torch GEMM first; results and gradients still match the oracle."""
    B, L, D, N, Rk = 2, 40, 32, 16, 24
    ins = make(B, L, D, N, Rk, seed=9)
    out, last, grads = run(dev, *ins, Rk, N, "zoh")
    rout, rlast, rg = oracle(*ins, Rk, N, "zoh")
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        close(v, rg[k], name=k)


def test_lowrank_mixed_layouts(dev):
    """x a split view (row stride 2D, as in_proj's output) while the outputs it allocates are
    contiguous: not a uniform layout, so forward and backward take the strided-address path;
    the projection is staged the same way."""
    B, L, D, N, Rk = 2, 50, 48, 16, 16
    x, proj, W, A, Dv, z, bias, dout = make(B, L, D, N, Rk, seed=13)
    xz = torch.cat([x, z], -1).to(dev).requires_grad_()          # split on the device: views
    leaves = [t.to(dev).requires_grad_() for t in (proj, W, A, Dv, bias)]
    pg, Wg, Ag, Dg, bg = leaves
    xg, zg = xz[..., :D], xz[..., D:]
    assert xg.stride() == (L * 2 * D, 2 * D, 1)
    dt, Bm, Cm = pg[..., :Rk], pg[..., Rk:Rk + N], pg[..., Rk + N:]
    out = ssm_scan.selective_scan_fn(xg, dt, Ag, Bm, Cm, D=Dg, z=zg, delta_bias=bg, delta_softplus=True,
                                     delta_proj=Wg)
    (out * dout.to(dev)).sum().backward()
    rout, _, rg = oracle(x, proj, W, A, Dv, z, bias, dout, Rk, N, "zoh")
    close(out, rout, name="out")
    close(xz.grad[..., :D], rg["dx"], name="dx")
    close(xz.grad[..., D:], rg["dz"], name="dz")
    for name, t in zip(("dproj", "dW", "dA", "dD", "dbias"), leaves):
        close(t.grad, rg[name], name=name)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 4e-3)])
def test_lowrank_half_precision_inputs(dev, dtype, tol):
    """16-bit x, dt, B, C, z (state float32): the output and last state against the oracle on
    the rounded inputs at rtol 2e-2 (bf16) or 4e-3 (fp16) with atol 1e-5, as the 16-bit tests
    of the materialized-delta path.  dW is the GEMM of the scan's 16-bit ddelta output with dt
    over the B x L tokens (the weight gradient of dt_proj): each of its terms carries the
    16-bit rounding of ddelta, so an element outside the bar must be within two units of that
    rounding (2^-7 bf16, 2^-10 fp16) of the sum of its terms' magnitudes; the count outside
    the bar is printed."""
    B, L, D, N, Rk = 2, 64, 32, 16, 16
    ins = make(B, L, D, N, Rk, seed=17, dtype=dtype)
    out, last, grads = run(dev, *ins, Rk, N, "zoh")
    assert out.dtype == dtype
    rout, rlast, rg = oracle(*ins, Rk, N, "zoh")
    close(out, rout, tol, 1e-5, "out")
    close(last, rlast, tol, 1e-5, "last")
    unit = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    close_or_cancelled(grads["dW"], rg["dW"], rg["dW_mag"], "dW", allow=rg["dW"].size, rtol=tol, atol=1e-5,
                       unit=unit)


def test_lowrank_with_initial_state_and_last_gradient(dev):
    """h0 and a gradient on the final state through the projected-delta path equal the same
    computation with the projection done by a torch GEMM first."""
    B, L, D, N, Rk = 2, 45, 24, 16, 8
    x, proj, W, A, Dv, z, bias, dout = make(B, L, D, N, Rk, seed=31)
    g = torch.Generator().manual_seed(32)
    h0 = torch.randn(B, D, N, generator=g)
    dlast = torch.randn(B, D, N, generator=g)
    res = []
    for lowrank in (True, False):
        leaves = [t.to(dev).requires_grad_() for t in (x, proj, W, A, Dv, z, bias, h0)]
        xg, pg, Wg, Ag, Dg, zg, bg, hg = leaves
        dt, Bm, Cm = pg[..., :Rk], pg[..., Rk:Rk + N], pg[..., Rk + N:]
        kw = dict(D=Dg, z=zg, delta_bias=bg, delta_softplus=True, h0=hg, return_last_state=True)
        if lowrank:
            out, last = ssm_scan.selective_scan_fn(xg, dt, Ag, Bm, Cm, delta_proj=Wg, **kw)
        else:
            out, last = ssm_scan.selective_scan_fn(xg, torch.nn.functional.linear(dt, Wg), Ag, Bm, Cm, **kw)
        ((out * dout.to(dev)).sum() + (last * dlast.to(dev)).sum()).backward()
        res.append([out.detach(), last.detach()] + [t.grad for t in leaves])
    for i, (a, b_) in enumerate(zip(*res)):
        close(a, np64(b_), name=str(i))


def test_lowrank_backward_in_segments(dev):
    """The projected-delta path with both passes in 5 time segments: outputs and every gradient
    (incl. dW through the fused projection) against the float64 oracle."""
    B, L, D, N, Rk = 2, 200, 32, 16, 16
    ins = make(B, L, D, N, Rk, seed=51)
    out, last, grads = run(dev, *ins, Rk, N, "zoh", segments=5)
    rout, rlast, rg = oracle(*ins, Rk, N, "zoh")
    close(out, rout, name="out")
    close(last, rlast, name="last")
    for k, v in grads.items():
        close(v, rg[k], name=k)
